"""Row-wise softmax (reference kernel/triton/softmax.py ``softmax`` :73-102):
``softmax(x) -> y`` over the last dimension (dim 1 of the reference's 2-D input),
y with x's dtype and shape.  One pass over HBM: each row is held in registers
for the max, exp and sum (icpp_softmax).  The reference's ``naive_softmax``
(:10-28) is a torch composition used as a baseline; the CPU oracle restates it
for the tests."""

from __future__ import annotations

import torch

from .. import runtime


def softmax(x: torch.Tensor) -> torch.Tensor:
    return runtime.softmax(x)


__all__ = ["softmax"]
