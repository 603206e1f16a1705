"""Fused GEMM + bias + activation, epilogue in registers (bf16 / f16).

Mirrors kernel/tilelang/gemm/gemm_bias_act.py: ``get_configs`` (:20-41),
``build_kernel`` (:91-96, ``kernel(a, b, bias) -> C``) and ``DESCRIPTOR``
(:104-116).  The reference fuses ReLU only (:80-82); the activation here is a
launch argument: "relu", "gelu_tanh" (evaluation/end2end.py:37-38) or "silu".
Output dtype follows the inputs (bf16 -> bf16), fp32 accumulation.
"""

from __future__ import annotations

import math

import torch

from ..autotuner.cost_model import ACT_PRIMITIVE, make_matmul_spec
from ..autotuner.perfdb import select_config
from .. import inputs as _inputs
from ._base import InstanceDescriptor
from .gemm import CompiledGemm

ACTIVATIONS = ("relu", "gelu_tanh", "silu", "gelu_erf")   # gelu_erf: torch's default F.gelu (end2end.py:83)


class GemmBiasActDescriptor(InstanceDescriptor):
    family = "gemm"
    split_k_values = (1,)

    def __init__(self, act: str = "relu", dtype: str = "bf16"):
        super().__init__(dtype)
        if act not in ACTIVATIONS:
            raise ValueError(f"act must be one of {ACTIVATIONS}")
        self.act = act

    @property
    def name(self) -> str:
        return f"gemm_bias_{self.act}"

    def make_op_spec(self, raw_config=None, M=0, N=0, K=0, **kw):
        return make_matmul_spec(M=M, N=N, K=K, primitives=["bias_add", ACT_PRIMITIVE[self.act]], dtype=self.dtype)

    def make_inputs(self, M, N, K, **kw):
        d = _inputs.config2(M, N, K, dtype=torch.bfloat16 if self.dtype == "bf16" else torch.float16, device="cuda")
        d["C"] = torch.empty((M, N), dtype=d["A"].dtype, device="cuda")
        return d

    def make_runner(self, raw, inputs, M, N, K, **kw):
        k = CompiledGemm(self, M, N, K, raw, act=self.act)
        return lambda: k(inputs["A"], inputs["B"], inputs["bias"], out=inputs["C"])


DESCRIPTOR = GemmBiasActDescriptor("relu", "bf16")
_DESCRIPTORS = {}


def descriptor(act: str = "relu", dtype: str = "bf16") -> GemmBiasActDescriptor:
    key = (act, dtype)
    if key not in _DESCRIPTORS:
        _DESCRIPTORS[key] = GemmBiasActDescriptor(act, dtype)
    return _DESCRIPTORS[key]


def get_configs(M, K, dtype: str = "bf16", N: int = 0):
    return descriptor("relu", dtype).get_raw_configs(M=M, N=N, K=K)


def build_kernel(M, N, K, config=None, act: str = "relu", dtype: str = "bf16"):
    """``kernel(a, b, bias) -> act(a @ b + bias)``; config=None selects one (the shipped
    measured table for profiled shape ranges, else the cost model's top-1)."""
    d = descriptor(act, dtype)
    if config is None:
        config = select_config(d, M=M, N=N, K=K)
    return CompiledGemm(d, M, N, K, config, act=act)


__all__ = ["ACTIVATIONS", "DESCRIPTOR", "GemmBiasActDescriptor", "build_kernel", "descriptor", "get_configs"]
