"""Plain GEMM C = A @ B (fp16 in, fp32 accumulate, fp16 out).

Mirrors kernel/tilelang/gemm/gemm.py: ``get_configs`` (:24-48), ``build_kernel``
(:84-89, out-allocating ``kernel(a, b) -> C``) and ``DESCRIPTOR`` (:97-114,
name "gemm_splitk", split-K aware op spec and score adjustment).  Split-K
partials go to an fp32 workspace and are reduced deterministically instead of
the reference's ``T.atomic_add`` into an uninitialised output (gemm.py:78).
"""

from __future__ import annotations

from typing import Any, Dict, Optional

import torch

from ..autotuner.cost_model import make_matmul_spec
from ..autotuner.perfdb import select_config
from .. import inputs as _inputs
from .. import runtime
from ._base import InstanceDescriptor


class GemmDescriptor(InstanceDescriptor):
    family = "gemm"
    dtype = "f16"
    split_k_values = (1, 2, 4)

    @property
    def name(self) -> str:
        return "gemm_splitk"

    def make_op_spec(self, raw_config=None, M=0, N=0, K=0, **kw):
        sk = raw_config.get("split_k", 1) if raw_config else 1
        return make_matmul_spec(M=M, N=N, K=K // sk, dtype=self.dtype)

    def make_inputs(self, M, N, K, **kw):
        d = _inputs.config1(M, N, K, device="cuda")
        d["C"] = torch.empty((M, N), dtype=torch.float16, device="cuda")
        return d

    def make_runner(self, raw, inputs, M, N, K, **kw):
        k = build_kernel(M, N, K, config=raw)
        return lambda: k(inputs["A"], inputs["B"], out=inputs["C"])


DESCRIPTOR = GemmDescriptor()


def get_configs(M, K, split_k_values=(1, 2, 4), N: int = 0):
    """Compiled candidates valid for this K (each K slice a multiple of block_K)."""
    d = GemmDescriptor()
    d.split_k_values = tuple(split_k_values)
    return d.get_raw_configs(M=M, N=N, K=K)


class CompiledGemm:
    """A resolved instance bound to a shape: ``kernel(a, b) -> C`` (out_idx=[-1] convention)."""

    def __init__(self, descriptor: InstanceDescriptor, M: int, N: int, K: int, config: Dict[str, Any],
                 act: str = "none"):
        self.descriptor, self.M, self.N, self.K, self.config, self.act = descriptor, M, N, K, config, act
        self.inst = descriptor.instance_index(config)
        self.split_k = config.get("split_k", 1)
        self._ws: Optional[torch.Tensor] = None

    def _workspace(self, device):
        need = runtime.workspace_bytes(self.descriptor.family, self.inst, self.M, self.N, self.K, self.split_k)
        if need and (self._ws is None or self._ws.device != device):
            self._ws = runtime.alloc_workspace(need, device)
        return self._ws

    def __call__(self, a, b, bias=None, out=None, scale_a: float = 1.0, scale_b: float = 1.0):
        return runtime.gemm(self.inst, self.descriptor.dtype, a, b, bias=bias, out=out, act=self.act,
                            scale_a=scale_a, scale_b=scale_b, split_k=self.split_k,
                            workspace=self._workspace(a.device))


def build_kernel(M, N, K, config=None):
    """Resolve a config to its compiled instance; None selects one (the shipped
    measured table for profiled shape ranges, else the cost model's top-1)."""
    if config is None:
        config = select_config(DESCRIPTOR, M=M, N=N, K=K)
    return CompiledGemm(DESCRIPTOR, M, N, K, config)


def flops(M, N, K) -> float:
    return 2.0 * M * N * K


__all__ = ["DESCRIPTOR", "CompiledGemm", "GemmDescriptor", "build_kernel", "flops", "get_configs"]
