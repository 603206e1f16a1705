"""Conv2d + ReLU (reference kernel/tilelang/conv/conv2d_relu.py): ``get_configs``,
``build_conv2d_relu_kernel`` (:146-155, ``kernel(X, W, Y)``),
``estimate_total_flops`` (:158-163) and ``DESCRIPTOR`` (:363-378)."""

from .conv2d import get_configs  # noqa: F401  (same candidate set as conv2d)
from .conv2d_fused import DESCRIPTORS, build_fused_conv2d_kernel
from .conv2d_fused import estimate_total_flops as _flops

DESCRIPTOR = DESCRIPTORS["conv2d_relu"]


def build_conv2d_relu_kernel(N, C, H, W, F_out, KH, KW, S=1, P=1, D=1, config=None):
    return build_fused_conv2d_kernel("conv2d_relu", N, C, H, W, F_out, KH, KW, S, P, D, config)


def estimate_total_flops(N, OH, OW, F_out, C, KH, KW):
    return _flops("conv2d_relu", N, OH, OW, F_out, C, KH, KW)


__all__ = ["DESCRIPTOR", "build_conv2d_relu_kernel", "estimate_total_flops", "get_configs"]
