"""Standalone LayerNorm with backward (reference kernel/triton/layernorm.py).

``LayerNorm`` is a torch.autograd.Function like the reference's (:214-275):
``forward(ctx, x, normalized_shape, weight, bias, eps)`` normalises over the
last dimension and saves (x, weight, bias, mean, rstd); ``backward`` returns
(dx, None, dw, db, None).  ``layer_norm = LayerNorm.apply`` (:278).  Both
directions run the gfx950 row kernels of libicpp_hip.so (icpp_layernorm_fwd /
icpp_layernorm_bwd); torch only provides memory, streams and autograd.

Differences from the reference: rows of any length up to 32768 (f16/bf16
forward; 16384 backward) instead of a 64 KB cap with a power-of-two block; dw /
db are summed in fp32 in a fixed order (the reference accumulates fp16 partial
buffers under spin locks, :164-181), so the backward is deterministic.
"""

from __future__ import annotations

import torch

from .. import runtime


class LayerNorm(torch.autograd.Function):

    @staticmethod
    def forward(ctx, x, normalized_shape, weight, bias, eps):
        if tuple(normalized_shape) != (x.shape[-1],):
            raise ValueError("normalized_shape must be the last dimension of x")
        y, mean, rstd = runtime.layernorm_fwd(x.contiguous(), weight, bias, eps)
        ctx.save_for_backward(x, weight, bias, mean, rstd)
        ctx.eps = eps
        return y

    @staticmethod
    def backward(ctx, dy):
        x, w, b, mean, rstd = ctx.saved_tensors
        dx, dw, db = runtime.layernorm_bwd(dy, x, w, mean, rstd)
        return dx, None, dw, db, None


layer_norm = LayerNorm.apply

__all__ = ["LayerNorm", "layer_norm"]
