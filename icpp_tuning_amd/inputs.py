"""Seeded synthetic inputs for the benchmark configurations.

Every tensor is drawn on the CPU from ``torch.Generator().manual_seed(
1000 * config_index + tensor_index)`` and then copied to the device, so the CPU
oracle and the GPU see bit-identical inputs.  Distributions follow the
benchmark configurations:

  config 1  GEMM 1024^3 fp16            A, B ~ N(0, 1)
  config 2  GEMM+bias+act 4096^3 bf16   A ~ N(0,1), B ~ N(0, 1/sqrt(K)), bias ~ N(0, 0.02)
  config 3  GEMM+bias+LN fp16           + gamma ~ N(1, 0.1), beta ~ N(0, 0.1)
  config 4  conv2d NHWC fp16            X ~ N(0,1), W ~ N(0, 1/sqrt(9 C))
  config 5  fp8 GEMM+bias+SiLU          A ~ N(0,1), B ~ N(0, 1/sqrt(K)) quantised per tensor
                                        (scale = amax / 448), bias fp32 ~ N(0, 0.02)
"""

from __future__ import annotations

import math
from typing import Dict, Optional

import torch

FP8_MAX = 448.0


def normal(shape, std: float, seed: int, mean: float = 0.0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float32) * std + mean


def quantize_e4m3(x: torch.Tensor):
    """Per-tensor e4m3fn quantisation, scale = amax / 448."""
    amax = float(x.abs().max().clamp_min(1e-12))
    scale = amax / FP8_MAX
    return (x / scale).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn), scale


def gemm_inputs(M: int, N: int, K: int, dtype: torch.dtype, cfg: int, *, b_std: Optional[float] = None,
                bias: bool = False, device="cpu") -> Dict[str, torch.Tensor]:
    base = 1000 * cfg
    out = {
        "A": normal((M, K), 1.0, base + 0).to(dtype),
        "B": normal((K, N), 1.0 if b_std is None else b_std, base + 1).to(dtype),
    }
    if bias:
        out["bias"] = normal((N,), 0.02, base + 2).to(dtype)
    return {k: v.to(device) for k, v in out.items()}


def config1(M=1024, N=1024, K=1024, device="cpu"):
    return gemm_inputs(M, N, K, torch.float16, 1, device=device)


def config2(M=4096, N=4096, K=4096, dtype=torch.bfloat16, device="cpu"):
    return gemm_inputs(M, N, K, dtype, 2, b_std=1.0 / math.sqrt(K), bias=True, device=device)


def config3(M=8192, N=1024, K=4096, device="cpu"):
    d = gemm_inputs(M, N, K, torch.float16, 3, b_std=1.0 / math.sqrt(K), bias=True)
    d["gamma"] = normal((N,), 0.1, 3000 + 3, mean=1.0).to(torch.float16)
    d["beta"] = normal((N,), 0.1, 3000 + 4).to(torch.float16)
    return {k: v.to(device) for k, v in d.items()}


C3_OFFSETS = ("bias+64", "bias+256", "row_mean")


def config3_offset(M=8192, N=1024, K=4096, kind="bias+256", device="cpu"):
    """Config-3 inputs whose pre-LayerNorm X = A.B + bias sits far from zero relative
    to its spread (row std ~1): "bias+64" / "bias+256" add a column offset common to
    every row; "row_mean" gives each row its own mean in [100, 400] (A[:, 0] ~
    U(100, 400), B[0, :] = 1).  This is the regime where the reference's fp32 X
    (gemm_bias_layernorm.py:59, :66, :103) differs from a 16-bit copy of X."""
    d = config3(M, N, K)
    if kind == "bias+64":
        d["bias"] = (d["bias"].float() + 64.0).to(torch.float16)
    elif kind == "bias+256":
        d["bias"] = (d["bias"].float() + 256.0).to(torch.float16)
    elif kind == "row_mean":
        g = torch.Generator().manual_seed(3100)
        d["A"][:, 0] = (torch.rand(M, generator=g) * 300.0 + 100.0).to(torch.float16)
        d["B"][0, :] = 1.0
    else:
        raise ValueError(f"unknown offset kind {kind!r} (one of {C3_OFFSETS})")
    return {k: v.to(device) for k, v in d.items()}


def config4(N=32, H=56, W=56, C=64, F=64, KH=3, KW=3, device="cpu"):
    X = normal((N, H, W, C), 1.0, 4000 + 0).to(torch.float16)
    Wt = normal((KH, KW, C, F), 1.0 / math.sqrt(KH * KW * C), 4000 + 1).to(torch.float16)
    return {"X": X.to(device), "W": Wt.to(device)}


def bn_params(F: int, seed: int = 4100, device="cpu"):
    """Inference BatchNorm parameters [F] f16 as the reference's fused-conv checks draw
    them (conv_bn_add_relu.py:195-198): gamma, beta, mean ~ N(0, 1), var ~ U(0.5, 1.5)."""
    g = torch.Generator().manual_seed(seed)
    out = {k: torch.randn(F, generator=g).to(torch.float16) for k in ("gamma", "beta", "mean")}
    out["var"] = (torch.rand(F, generator=g) + 0.5).to(torch.float16)
    return {k: v.to(device) for k, v in out.items()}


def residual(shape, seed: int = 4200, device="cpu"):
    """Residual input [N, OH, OW, F] f16 ~ N(0, 1) (conv_bn_add_relu.py:194)."""
    return normal(shape, 1.0, seed).to(torch.float16).to(device)


def config5(M=256, N=4096, K=4096, device="cpu"):
    a = normal((M, K), 1.0, 5000 + 0)
    b = normal((K, N), 1.0 / math.sqrt(K), 5000 + 1)
    aq, sa = quantize_e4m3(a)
    bq, sb = quantize_e4m3(b)
    bias = normal((N,), 0.02, 5000 + 2)
    return {"A": aq.to(device), "B": bq.to(device), "scale_a": sa, "scale_b": sb, "bias": bias.to(device)}


__all__ = ["C3_OFFSETS", "config1", "config2", "config3", "config3_offset", "config4", "config5", "gemm_inputs",
           "normal", "quantize_e4m3"]
