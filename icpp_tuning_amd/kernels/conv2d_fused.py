"""NHWC conv2d with fused epilogues: ReLU, inference BatchNorm, BN+ReLU, BN+residual+ReLU.

One implementation behind the four reference modules (kernel/tilelang/conv/
conv2d_relu.py, conv2d_bn.py, conv2d_bn_relu.py, conv_bn_add_relu.py), each of
which repeats the conv mainloop of conv2d.py with its own epilogue.  Here the
conv instances of ``conv2d`` run them all: the epilogue is chosen per call
(icpp_conv2d_nhwc_fused).  Semantics per variant, from the reference:

  conv2d_relu       relu(conv)                                    conv2d_relu.py:128-139
  conv2d_bn         BN(conv), eps 1e-3                            conv2d_bn.py:140-152
  conv2d_bn_relu    relu(BN(conv)), eps 1e-5                      conv2d_bn_relu.py:254-265
  conv_bn_add_relu  relu(BN(conv) + residual), var >= 0, eps 1e-5 conv_bn_add_relu.py:147-162

BN(x) = (x - mean) * rsqrt(var + eps) * gamma + beta per output channel, on the
conv value rounded to f16 (the reference epilogues read it from an f16 tile).
"""

from __future__ import annotations

from dataclasses import replace
from typing import Any, Dict, Optional

import torch

from ..autotuner.cost_model import make_conv2d_spec
from ..autotuner.perfdb import select_config
from .. import inputs as _inputs
from .. import runtime
from .conv2d import DESCRIPTOR as CONV_DESCRIPTOR
from .conv2d import Conv2dDescriptor, calc_conv_flops, calc_oh_ow

# name -> (BN, residual, var clamp, act, default eps, cost-model primitives, epilogue flops per output)
VARIANTS = {
    "conv2d_relu": (False, False, False, "relu", 1e-5, ("relu",), 1),          # conv2d_relu.py:158-163, :371
    "conv2d_bn": (True, False, False, "none", 1e-3, ("batchnorm",), 6),        # conv2d_bn.py:67, :169-174, :395
    "conv2d_bn_relu": (True, False, False, "relu", 1e-5, ("batchnorm", "relu"), 7),      # conv2d_bn_relu.py:282-290
    "conv_bn_add_relu": (True, True, True, "relu", 1e-5, ("batchnorm", "relu"), 8),      # conv_bn_add_relu.py:179-184
}


class FusedConv2dDescriptor(Conv2dDescriptor):
    """Descriptor of one fused variant (reference names and primitives,
    e.g. conv2d_bn_relu.py:462-477); shares the conv instance set."""

    def __init__(self, variant: str):
        super().__init__()
        if variant not in VARIANTS:
            raise ValueError(f"variant must be one of {sorted(VARIANTS)}")
        self.variant = variant
        self.bn, self.residual, self.var_clamp, self.act, self.eps, self.primitives, self.epi_flops = VARIANTS[variant]

    @property
    def name(self) -> str:
        return self.variant

    def make_op_spec(self, raw_config=None, N=0, C=0, H=0, W=0, OC=0, KH=3, KW=3, stride=1, padding=0, **kw):
        sk = raw_config.get("split_k", 1) if raw_config else 1
        spec = make_conv2d_spec(N, C, H, W, OC, KH, KW, stride=stride, padding=padding, primitives=self.primitives,
                                name=self.variant)
        if sk == 1:
            return spec
        return replace(spec, mainloop=replace(spec.mainloop, K=spec.mainloop.K // sk))

    def flops(self, N=0, C=0, H=0, W=0, OC=0, KH=3, KW=3, stride=1, padding=0, **kw):
        OH, OW = calc_oh_ow(H, W, KH, KW, stride, padding, 1)
        return float(calc_conv_flops(N, C, OH, OW, OC, KH, KW) + self.epi_flops * N * OH * OW * OC)

    def make_inputs(self, N, C, H, W, OC, KH=3, KW=3, stride=1, padding=1, **kw):
        d = super().make_inputs(N, C, H, W, OC, KH, KW, stride, padding)
        d.update(_inputs.bn_params(OC, device="cuda"))
        if self.residual:
            d["R"] = _inputs.residual(tuple(d["Y"].shape), device="cuda")
        return d

    def make_runner(self, raw, inputs, N, C, H, W, OC, KH=3, KW=3, stride=1, padding=1, **kw):
        k = build_fused_conv2d_kernel(self.variant, N, C, H, W, OC, KH, KW, stride, padding, 1, config=raw)
        bn = [inputs[x] for x in ("gamma", "beta", "mean", "var")] if self.bn else []
        res = [inputs["R"]] if self.residual else []
        return lambda: k(inputs["X"], inputs["W"], *res, *bn, inputs["Y"])


DESCRIPTORS = {v: FusedConv2dDescriptor(v) for v in VARIANTS}


class CompiledFusedConv2d:
    """``kernel(X, W, [residual,] [gamma, beta, mean, var,] Y)``: the argument
    order of the reference prim_funcs (conv_bn_add_relu.py:87-96)."""

    def __init__(self, variant: str, N, C, H, W, F_out, KH, KW, S, P, D, config: Dict[str, Any],
                 eps: Optional[float] = None):
        self.desc = DESCRIPTORS[variant]
        self.geom = (N, C, H, W, F_out, KH, KW, S, P, D)
        self.config = config
        self.inst = CONV_DESCRIPTOR.instance_index(config)
        self.split_k = config.get("split_k", 1)
        self.eps = self.desc.eps if eps is None else float(eps)
        self._ws: Optional[torch.Tensor] = None

    def __call__(self, X, W_weight, *args):
        d = self.desc
        nargs = 1 + (1 if d.residual else 0) + (4 if d.bn else 0)
        if len(args) != nargs:
            raise TypeError(f"{d.variant} kernel takes X, W{', residual' if d.residual else ''}"
                            f"{', gamma, beta, mean, var' if d.bn else ''}, Y ({2 + nargs} tensors)")
        Y = args[-1]
        res = args[0] if d.residual else None
        bn = tuple(args[(1 if d.residual else 0):(1 if d.residual else 0) + 4]) if d.bn else None
        N, C, H, W, F_out, KH, KW, S, P, D = self.geom
        OH, OW = calc_oh_ow(H, W, KH, KW, S, P, D)
        need = runtime.workspace_bytes("conv2d", self.inst, N * OH * OW, F_out, KH * KW * C, self.split_k)
        if need and (self._ws is None or self._ws.device != X.device):
            self._ws = runtime.alloc_workspace(need, X.device)
        runtime.conv2d_nhwc(self.inst, X, W_weight, Y, S, P, D, self.split_k, self._ws, act=d.act, bn=bn,
                            eps=self.eps, var_clamp=d.var_clamp, residual=res)


def build_fused_conv2d_kernel(variant: str, N, C, H, W, F_out, KH, KW, S=1, P=1, D=1, config=None, eps=None):
    if config is None:
        config = select_config(DESCRIPTORS[variant], N=N, C=C, H=H, W=W, OC=F_out, KH=KH, KW=KW, stride=S, padding=P)
    return CompiledFusedConv2d(variant, N, C, H, W, F_out, KH, KW, S, P, D, config, eps)


def estimate_total_flops(variant: str, N, OH, OW, F_out, C, KH, KW):
    """Conv flops plus the reference's per-output epilogue estimate (1 ReLU,
    6 BN, 7 BN+ReLU, 8 BN+add+ReLU)."""
    return calc_conv_flops(N, C, OH, OW, F_out, KH, KW) + VARIANTS[variant][6] * N * OH * OW * F_out


__all__ = ["CompiledFusedConv2d", "DESCRIPTORS", "FusedConv2dDescriptor", "VARIANTS", "build_fused_conv2d_kernel",
           "estimate_total_flops"]
