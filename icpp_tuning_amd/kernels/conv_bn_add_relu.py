"""Conv2d + BatchNorm (inference) + residual add + ReLU (reference
kernel/tilelang/conv/conv_bn_add_relu.py): ``get_configs``,
``build_conv2d_bn_add_relu_kernel`` (:169-175, ``kernel(x, w, residual, gamma,
beta, mean, var, y)``, eps 1e-5, negative variances clamped to 0 :158),
``estimate_total_flops`` (:179-184) and ``DESCRIPTOR`` (:219-234)."""

from .conv2d import get_configs  # noqa: F401
from .conv2d_fused import DESCRIPTORS, build_fused_conv2d_kernel
from .conv2d_fused import estimate_total_flops as _flops

DESCRIPTOR = DESCRIPTORS["conv_bn_add_relu"]


def build_conv2d_bn_add_relu_kernel(n, c, h, w, f_out, kh, kw, s=1, p=1, d=1, config=None):
    return build_fused_conv2d_kernel("conv_bn_add_relu", n, c, h, w, f_out, kh, kw, s, p, d, config)


def estimate_total_flops(n, oh, ow, f_out, c, kh, kw):
    return _flops("conv_bn_add_relu", n, oh, ow, f_out, c, kh, kw)


__all__ = ["DESCRIPTOR", "build_conv2d_bn_add_relu_kernel", "estimate_total_flops", "get_configs"]
