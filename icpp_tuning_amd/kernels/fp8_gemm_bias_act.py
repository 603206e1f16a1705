"""fp8 (OCP e4m3fn) GEMM + bias + SiLU with per-tensor scales, bf16 out.

No reference kernel exists for this op; it follows the GEMM+bias+act module's
API (gemm_bias_act.py) with the quantised-inference contract of the benchmark:
``kernel(a_q, b_q, scale_a, scale_b, bias) -> act(scale_a*scale_b * a_q @ b_q + bias)``
with fp32 bias and fp32 accumulation; scales are applied once in the epilogue.
Small M is HBM-bound, so split-K candidates put >= 256 workgroups on B.
"""

from __future__ import annotations

import torch

from ..autotuner.cost_model import ACT_PRIMITIVE, make_matmul_spec
from ..autotuner.perfdb import select_config
from .. import inputs as _inputs
from ._base import InstanceDescriptor
from .gemm import CompiledGemm


class Fp8GemmBiasActDescriptor(InstanceDescriptor):
    family = "gemm"
    dtype = "fp8"
    split_k_values = (1, 2, 4, 8, 16)

    def __init__(self, act: str = "silu"):
        super().__init__("fp8")
        self.act = act

    @property
    def name(self) -> str:
        return f"fp8_gemm_bias_{self.act}"

    def make_op_spec(self, raw_config=None, M=0, N=0, K=0, **kw):
        sk = raw_config.get("split_k", 1) if raw_config else 1
        return make_matmul_spec(M=M, N=N, K=K // sk, primitives=["bias_add", ACT_PRIMITIVE[self.act]],
                                dtype="fp8", output_element_bytes=2)

    def make_inputs(self, M, N, K, **kw):
        d = _inputs.config5(M, N, K, device="cuda")
        d["C"] = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        return d

    def make_runner(self, raw, inputs, M, N, K, **kw):
        k = CompiledGemm(self, M, N, K, raw, act=self.act)
        return lambda: k(inputs["A"], inputs["B"], inputs["bias"], out=inputs["C"],
                         scale_a=inputs["scale_a"], scale_b=inputs["scale_b"])


DESCRIPTOR = Fp8GemmBiasActDescriptor("silu")


def get_configs(M, K, N: int = 0):
    return DESCRIPTOR.get_raw_configs(M=M, N=N, K=K)


class CompiledFp8Gemm(CompiledGemm):
    def __call__(self, a_q, b_q, scale_a, scale_b, bias=None, out=None):
        return super().__call__(a_q, b_q, bias=bias, out=out, scale_a=float(scale_a), scale_b=float(scale_b))


def build_kernel(M, N, K, config=None, act: str = "silu"):
    d = DESCRIPTOR if act == "silu" else Fp8GemmBiasActDescriptor(act)
    if config is None:
        config = select_config(d, M=M, N=N, K=K)
    return CompiledFp8Gemm(d, M, N, K, config, act=act)


class PackedFp8Decode:
    """``kernel(a_q, scale_a, scale_b, bias) -> act(scale_a*scale_b * a_q @ b_q + bias)`` for
    M <= 32 rows per call, with b_q [K, N] packed once at construction (icpp_fp8_pack_b)
    and every call one launch of icpp_fp8_gemm_packed: for weights that stay fixed across
    calls (decode), where the tiled path needs split-K plus a reduce launch."""

    def __init__(self, b_q: torch.Tensor, act: str = "silu"):
        from .. import runtime

        self.K, self.N = b_q.shape
        self.act = act
        self.packed = runtime.fp8_pack_b(b_q)

    def __call__(self, a_q, scale_a, scale_b, bias=None, out=None):
        from .. import runtime

        return runtime.fp8_gemm_packed(a_q, self.packed, self.N, bias=bias, out=out, act=self.act,
                                       scale_a=float(scale_a), scale_b=float(scale_b))


def build_packed_kernel(b_q: torch.Tensor, act: str = "silu") -> PackedFp8Decode:
    """The decode kernel over pre-packed weights (see PackedFp8Decode); needs K % 128 == 0
    and N % 16 == 0."""
    return PackedFp8Decode(b_q, act=act)


__all__ = ["DESCRIPTOR", "Fp8GemmBiasActDescriptor", "PackedFp8Decode", "build_kernel", "build_packed_kernel",
           "get_configs"]
