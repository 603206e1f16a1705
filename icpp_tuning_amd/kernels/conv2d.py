"""NHWC implicit-GEMM conv2d (fp16, fp32 accumulate, HWIO filter).

Mirrors kernel/tilelang/conv/conv2d.py: ``calc_oh_ow`` / ``calc_conv_flops``
(:65-72), ``get_configs`` (:186-205), ``build_conv2d_kernel`` (:282-290,
destination-passing ``kernel(X, W, Y)``) and ``DESCRIPTOR`` (:467-479, shape
kwargs N, C, H, W, OC, KH, KW, stride, padding).  GEMM view: M = N*OH*OW,
N = F, K = KH*KW*C with k -> (kh, kw, c) = (k // (KW*C), (k // C) % KW, k % C)
(:242-250); the A tile is gathered per 16-byte channel chunk straight from
the NHWC tensor, padding taps read as zeros.
"""

from __future__ import annotations

from typing import Any, Dict, Optional

import torch

from ..autotuner.cost_model import make_conv2d_spec
from ..autotuner.perfdb import select_config
from .. import inputs as _inputs
from .. import runtime
from ._base import InstanceDescriptor


def calc_oh_ow(H, W, KH, KW, S, P, D):
    return (H + 2 * P - D * (KH - 1) - 1) // S + 1, (W + 2 * P - D * (KW - 1) - 1) // S + 1


def calc_conv_flops(N, C, OH, OW, F_out, KH, KW):
    return 2 * N * OH * OW * F_out * C * KH * KW


class Conv2dDescriptor(InstanceDescriptor):
    family = "conv2d"
    dtype = "f16"
    split_k_values = (1, 2, 4, 8)

    @property
    def name(self) -> str:
        return "conv2d"

    def make_op_spec(self, raw_config=None, N=0, C=0, H=0, W=0, OC=0, KH=3, KW=3, stride=1, padding=0, **kw):
        sk = raw_config.get("split_k", 1) if raw_config else 1
        spec = make_conv2d_spec(N, C, H, W, OC, KH, KW, stride=stride, padding=padding)
        if sk == 1:
            return spec
        from dataclasses import replace
        return replace(spec, mainloop=replace(spec.mainloop, K=spec.mainloop.K // sk))

    def schedule_factor(self, raw: Dict[str, Any]) -> float:
        """Ping-pong conv tiles measured 0.79-0.84x the best default-schedule tile on
        the benchmark conv shapes (b32 14x14x256, 56x56x64)."""
        return 0.8 if raw.get("sched") == "pp" else 1.0

    def extra_seconds(self, raw, hw, **shape) -> float:
        """Split-K conv launches measured slower than the schedule model prices them: on
        the profiled conv shapes the unsplit tile wins wherever the model would split
        small grids.  The fp32 partial round trip is charged twice its bytes at HBM rate
        plus 2 us (fitted on the shipped conv databases: mean formula pick 0.90 -> 0.91-0.94
        of the measured best)."""
        sk = raw.get("split_k", 1)
        if sk <= 1 or not getattr(hw, "has_mfma_model", False):
            return 0.0
        M, N = self.gemm_mn(**shape)
        return 2.0 * M * N * 4.0 * sk / (hw.mem_bandwidth_gbps * 1e9) + 2e-6

    def k_extent(self, C=0, KH=3, KW=3, **kw) -> int:
        return C * KH * KW

    def gemm_mn(self, N=0, H=0, W=0, OC=0, KH=3, KW=3, stride=1, padding=0, **kw):
        OH, OW = calc_oh_ow(H, W, KH, KW, stride, padding, 1)
        return N * OH * OW, OC

    def flops(self, N=0, C=0, H=0, W=0, OC=0, KH=3, KW=3, stride=1, padding=0, **kw):
        OH, OW = calc_oh_ow(H, W, KH, KW, stride, padding, 1)
        return float(calc_conv_flops(N, C, OH, OW, OC, KH, KW))

    def make_inputs(self, N, C, H, W, OC, KH=3, KW=3, stride=1, padding=1, **kw):
        d = _inputs.config4(N, H, W, C, OC, KH, KW, device="cuda")
        OH, OW = calc_oh_ow(H, W, KH, KW, stride, padding, 1)
        d["Y"] = torch.empty((N, OH, OW, OC), dtype=torch.float16, device="cuda")
        return d

    def make_runner(self, raw, inputs, N, C, H, W, OC, KH=3, KW=3, stride=1, padding=1, **kw):
        k = build_conv2d_kernel(N, C, H, W, OC, KH, KW, stride, padding, 1, config=raw)
        return lambda: k(inputs["X"], inputs["W"], inputs["Y"])


DESCRIPTOR = Conv2dDescriptor()


def get_configs(C: int = 64, KH: int = 3, KW: int = 3):
    return DESCRIPTOR.get_raw_configs(C=C, KH=KH, KW=KW)


class CompiledConv2d:
    def __init__(self, N, C, H, W, F_out, KH, KW, S, P, D, config: Dict[str, Any]):
        self.geom = (N, C, H, W, F_out, KH, KW, S, P, D)
        self.config = config
        self.inst = DESCRIPTOR.instance_index(config)
        self.split_k = config.get("split_k", 1)
        self._ws: Optional[torch.Tensor] = None

    def __call__(self, X, W_weight, Y):
        N, C, H, W, F_out, KH, KW, S, P, D = self.geom
        OH, OW = calc_oh_ow(H, W, KH, KW, S, P, D)
        need = runtime.workspace_bytes("conv2d", self.inst, N * OH * OW, F_out, KH * KW * C, self.split_k)
        if need and (self._ws is None or self._ws.device != X.device):
            self._ws = runtime.alloc_workspace(need, X.device)
        runtime.conv2d_nhwc(self.inst, X, W_weight, Y, S, P, D, self.split_k, self._ws)


def build_conv2d_kernel(N, C, H, W, F_out, KH, KW, S=1, P=1, D=1, config=None):
    if config is None:
        config = select_config(DESCRIPTOR, N=N, C=C, H=H, W=W, OC=F_out, KH=KH, KW=KW, stride=S, padding=P)
    return CompiledConv2d(N, C, H, W, F_out, KH, KW, S, P, D, config)


__all__ = ["DESCRIPTOR", "Conv2dDescriptor", "build_conv2d_kernel", "calc_conv_flops", "calc_oh_ow", "get_configs"]
