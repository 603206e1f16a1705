"""GPU parity of the fused conv epilogues (ReLU, BN, BN+ReLU, BN+residual+ReLU)
against the CPU oracle, through icpp_conv2d_nhwc_fused.

Tolerance |y - y_ref| <= 1e-2 + 1e-2 |y_ref| elementwise (the reference's
verify_correctness, e.g. conv_bn_add_relu.py:207).  Inputs are drawn as the
reference draws BN parameters (gamma, beta, mean ~ N(0,1), var ~ U(0.5, 1.5));
the filter is scaled by 1/sqrt(KH*KW*C) so conv values are O(1) and the f16
rounding both sides apply before BN stays below the tolerance after the BN
scale.
"""

import pytest
import torch

from icpp_tuning_amd import inputs as I
from icpp_tuning_amd.kernels import conv2d_fused as CF
from icpp_tuning_amd.kernels._base import family_instances, raw_from_inst
from oracle import ops as O

pytestmark = pytest.mark.gpu

VARIANTS = list(CF.VARIANTS)


def _close(y, ref, what):
    y = y.float().cpu()
    assert torch.isfinite(y).all(), f"{what}: non-finite output"
    err = (y - ref).abs()
    bad = err > 1e-2 + 1e-2 * ref.abs()
    if bad.any():
        idx = bad.nonzero()[0].tolist()
        raise AssertionError(f"{what}: {int(bad.sum())} / {y.numel()} outside tol; max err {err.max().item():.4g}; "
                             f"first at {idx}: got {y[tuple(idx)].item():.5g} want {ref[tuple(idx)].item():.5g}")


def _case(variant, Nb, H, W, C, Fo, KH=3, KW=3, S=1, P=1, D=1, seed=0):
    desc = CF.DESCRIPTORS[variant]
    d = I.config4(Nb, H, W, C, Fo, KH, KW)
    bn = I.bn_params(Fo, seed=4100 + seed)
    OH, OW = O.conv_out_hw(H, W, KH, KW, S, P, D)
    R = I.residual((Nb, OH, OW, Fo), seed=4200 + seed) if desc.residual else None
    params = tuple(bn[k] for k in ("gamma", "beta", "mean", "var")) if desc.bn else None
    ref = O.conv2d_bn_act_ref(d["X"], d["W"], S, P, D, bn=params, eps=desc.eps, var_clamp=desc.var_clamp,
                              residual=R, act=desc.act)
    dev = [d["X"].cuda(), d["W"].cuda()] + ([R.cuda()] if R is not None else []) + \
          ([t.cuda() for t in params] if params else [])
    return ref, dev


@pytest.mark.parametrize("variant", VARIANTS)
def test_every_conv_instance_fused(gpu, variant):
    """Every conv tile, split-K 1 and 3 (the split-K reduce runs the epilogue)."""
    Nb, H, W, C, Fo = 2, 9, 7, 64, 64
    ref, dev = _case(variant, Nb, H, W, C, Fo)
    for inst in family_instances("conv2d"):
        for sk in (1, 3):
            if (9 * C) % inst.bk or sk > 9 * C // inst.bk:
                continue
            raw = raw_from_inst(inst, sk)
            print(f"[parity] {variant} {inst.name} sk={sk}", flush=True)
            k = CF.build_fused_conv2d_kernel(variant, Nb, C, H, W, Fo, 3, 3, 1, 1, 1, config=raw)
            Y = torch.full((Nb, H, W, Fo), float("nan"), dtype=torch.float16, device="cuda")
            k(*dev, Y)
            torch.cuda.synchronize()
            _close(Y, ref, f"{variant} {inst.name} sk={sk}")


@pytest.mark.parametrize("variant", VARIANTS)
@pytest.mark.parametrize("shape", [(32, 56, 56, 64, 64), (32, 14, 14, 256, 256), (32, 7, 7, 512, 512)])
def test_config4_fused(gpu, variant, shape):
    """The C4 ResNet shapes with the default (adaptive) config choice."""
    Nb, H, W, C, Fo = shape
    ref, dev = _case(variant, Nb, H, W, C, Fo, seed=1)
    k = CF.build_fused_conv2d_kernel(variant, Nb, C, H, W, Fo, 3, 3)
    print(f"[parity] {variant} {shape} {k.config}", flush=True)
    Y = torch.empty((Nb, H, W, Fo), dtype=torch.float16, device="cuda")
    k(*dev, Y)
    torch.cuda.synchronize()
    _close(Y, ref, f"{variant} {shape} {k.config}")


@pytest.mark.parametrize("geom", [
    # (N, H, W, C, F, KH, KW, stride, pad, dilation): 3x3 with C = 2 x 64, general gather,
    # stride 2, 1x1 with a partial N tile
    (2, 9, 7, 128, 64, 3, 3, 1, 1, 1),
    (2, 7, 6, 16, 64, 2, 2, 1, 0, 1),
    (2, 9, 9, 64, 64, 3, 3, 2, 1, 1),
    (1, 5, 5, 128, 72, 1, 1, 1, 0, 1),
])
def test_fused_geometries(gpu, geom):
    Nb, H, W, C, Fo, KH, KW, S, P, D = geom
    for variant in VARIANTS:
        ref, dev = _case(variant, Nb, H, W, C, Fo, KH, KW, S, P, D, seed=2)
        for inst in family_instances("conv2d"):
            if (KH * KW * C) % inst.bk:
                continue
            raw = raw_from_inst(inst, 1)
            print(f"[parity] {variant} {geom} {inst.name}", flush=True)
            k = CF.build_fused_conv2d_kernel(variant, Nb, C, H, W, Fo, KH, KW, S, P, D, config=raw)
            Y = torch.full(tuple(ref.shape), float("nan"), dtype=torch.float16, device="cuda")
            k(*dev, Y)
            torch.cuda.synchronize()
            _close(Y, ref, f"{variant} {geom} {inst.name}")


def test_negative_variance_clamped(gpu):
    """conv_bn_add_relu clamps var at 0 (conv_bn_add_relu.py:158): with half the
    variances negative the output stays finite and matches the oracle."""
    Nb, H, W, C, Fo = 2, 8, 8, 64, 64
    d = I.config4(Nb, H, W, C, Fo)
    bn = I.bn_params(Fo, seed=4300)
    var = bn["var"].clone()
    var[::2] = -0.5
    var[1::4] = 0.0
    params = (bn["gamma"], bn["beta"], bn["mean"], var)
    R = I.residual((Nb, H, W, Fo), seed=4301)
    ref = O.conv2d_bn_act_ref(d["X"], d["W"], bn=params, eps=1e-5, var_clamp=True, residual=R, act="relu")
    k = CF.build_fused_conv2d_kernel("conv_bn_add_relu", Nb, C, H, W, Fo, 3, 3)
    Y = torch.empty((Nb, H, W, Fo), dtype=torch.float16, device="cuda")
    k(d["X"].cuda(), d["W"].cuda(), R.cuda(), *[t.cuda() for t in params], Y)
    torch.cuda.synchronize()
    y = Y.float().cpu()
    assert torch.isfinite(y).all()
    # per-channel BN scale |gamma| * rsqrt(var + eps); beyond 4 (the largest the standard draw gives),
    # one f16 rounding step of the conv value moves the output by more: widen the tolerance by scale / 4
    scale = bn["gamma"].float().abs() * torch.rsqrt(torch.clamp(var.float(), min=0) + 1e-5)
    widen = (scale / 4.0).clamp_min(1.0)
    err = (y - ref).abs()
    assert bool((err <= (1e-2 + 1e-2 * ref.abs()) * widen).all()), float(err.max())
