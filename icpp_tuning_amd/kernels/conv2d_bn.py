"""Conv2d + BatchNorm (inference statistics; reference kernel/tilelang/conv/
conv2d_bn.py): ``get_configs``, ``build_conv2d_bn_kernel`` (:159-166,
``kernel(X, W, gamma, beta, mean, var, Y)``, eps 1e-3 as the reference's
factory default :67), ``estimate_total_flops`` (:169-174) and ``DESCRIPTOR``
(:387-402)."""

from .conv2d import get_configs  # noqa: F401
from .conv2d_fused import DESCRIPTORS, build_fused_conv2d_kernel
from .conv2d_fused import estimate_total_flops as _flops

DESCRIPTOR = DESCRIPTORS["conv2d_bn"]


def build_conv2d_bn_kernel(N, C, H, W, F_out, KH, KW, S=1, P=1, D=1, config=None, eps=1e-3):
    return build_fused_conv2d_kernel("conv2d_bn", N, C, H, W, F_out, KH, KW, S, P, D, config, eps)


def estimate_total_flops(N, OH, OW, F_out, C, KH, KW):
    return _flops("conv2d_bn", N, OH, OW, F_out, C, KH, KW)


__all__ = ["DESCRIPTOR", "build_conv2d_bn_kernel", "estimate_total_flops", "get_configs"]
