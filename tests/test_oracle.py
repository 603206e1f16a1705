"""Pins for the CPU oracle (oracle/ops.py) -- each against something independent
of the oracle's own formula: fp64 brute-force loops, library routines, exact
special cases."""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from icpp_tuning_amd import inputs as I
from oracle import ops as O


def _np64(t):
    return t.float().double().numpy()


def test_gemm_ref_matches_fp64_triple_loop():
    g = torch.Generator().manual_seed(7)
    A = torch.randn(17, 65, generator=g).half()
    B = torch.randn(65, 33, generator=g).half()
    a, b = _np64(A), _np64(B)
    ref = np.zeros((17, 33))
    for i in range(17):
        for j in range(33):
            s = 0.0
            for k in range(65):
                s += a[i, k] * b[k, j]
            ref[i, j] = s
    np.testing.assert_allclose(O.gemm_ref(A, B).double().numpy(), ref, rtol=1e-5, atol=1e-4)


def test_gemm_identity_and_zero():
    A = torch.randn(8, 16).half()
    eye = torch.eye(16).half()
    assert torch.equal(O.gemm_ref(A, eye), A.float())
    bias = torch.randn(16).half()
    z = torch.zeros(8, 16).half()
    for act, fn in (("relu", F.relu), ("silu", F.silu), ("gelu_tanh", lambda x: F.gelu(x, approximate="tanh"))):
        y = O.gemm_bias_act_ref(z, eye, bias, act)
        torch.testing.assert_close(y, fn(bias.float()).expand(8, 16), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("act,lib", [("relu", F.relu), ("silu", F.silu),
                                     ("gelu_tanh", lambda x: F.gelu(x, approximate="tanh"))])
def test_activations_match_library(act, lib):
    x = torch.linspace(-8, 8, 4001)
    torch.testing.assert_close(O.apply_act(x, act), lib(x), rtol=1e-6, atol=1e-6)


def test_gelu_tanh_special_values():
    # gelu(0) = 0, odd part: gelu(x) - gelu(-x) = x exactly for the tanh form
    x = torch.tensor([0.0, 0.5, 1.0, 3.0], dtype=torch.float64)
    g = O.gelu_tanh(x)
    assert g[0].item() == 0.0
    torch.testing.assert_close(g - O.gelu_tanh(-x), x, rtol=1e-12, atol=1e-12)


def test_layernorm_ref_fp64_and_library():
    g = torch.Generator().manual_seed(3)
    A = torch.randn(9, 40, generator=g).half()
    B = (torch.randn(40, 24, generator=g) / 6).half()
    bias, gamma, beta = (torch.randn(24, generator=g).half() for _ in range(3))
    y = O.gemm_bias_layernorm_ref(A, B, bias, gamma, beta, 1e-5).double().numpy()
    x = _np64(A) @ _np64(B) + _np64(bias)[None]
    mu = x.mean(1, keepdims=True)
    var = ((x - mu) ** 2).mean(1, keepdims=True)
    ref = (x - mu) / np.sqrt(var + 1e-5) * _np64(gamma)[None] + _np64(beta)[None]
    np.testing.assert_allclose(y, ref, rtol=1e-4, atol=1e-4)
    lib = F.layer_norm(torch.from_numpy(x).float(), (24,), gamma.float(), beta.float(), 1e-5)
    np.testing.assert_allclose(y, lib.double().numpy(), rtol=1e-4, atol=1e-4)


def test_layernorm_constant_rows_give_beta():
    A = torch.ones(4, 8).half()
    B = torch.ones(8, 16).half()      # every row of A@B is the constant 8
    bias = torch.zeros(16).half()
    gamma = torch.randn(16).half()
    beta = torch.randn(16).half()
    y = O.gemm_bias_layernorm_ref(A, B, bias, gamma, beta)
    torch.testing.assert_close(y, beta.float().expand(4, 16), rtol=0, atol=1e-6)


def test_conv_ref_matches_direct_7_loop_sum():
    g = torch.Generator().manual_seed(11)
    N, H, W, C, Fo, KH, KW, S, P = 2, 5, 6, 3, 4, 3, 3, 1, 1
    X = torch.randn(N, H, W, C, generator=g).half()
    Wt = torch.randn(KH, KW, C, Fo, generator=g).half()
    x, w = _np64(X), _np64(Wt)
    OH, OW = O.conv_out_hw(H, W, KH, KW, S, P)
    ref = np.zeros((N, OH, OW, Fo))
    for n in range(N):
        for oh in range(OH):
            for ow in range(OW):
                for f in range(Fo):
                    s = 0.0
                    for kh in range(KH):
                        for kw in range(KW):
                            for c in range(C):
                                ih, iw = oh * S - P + kh, ow * S - P + kw
                                if 0 <= ih < H and 0 <= iw < W:
                                    s += x[n, ih, iw, c] * w[kh, kw, c, f]
                    ref[n, oh, ow, f] = s
    np.testing.assert_allclose(O.conv2d_nhwc_ref(X, Wt, S, P).double().numpy(), ref, rtol=1e-5, atol=1e-5)


def test_conv_ref_is_gemm_under_im2col_map():
    """k -> (kh, kw, c) = (k // (KW*C), (k // C) % KW, k % C) (reference conv2d.py:242-250)."""
    g = torch.Generator().manual_seed(5)
    N, H, W, C, Fo = 1, 4, 4, 2, 3
    X = torch.randn(N, H, W, C, generator=g).half()
    Wt = torch.randn(3, 3, C, Fo, generator=g).half()
    x = _np64(X)
    OH, OW = O.conv_out_hw(H, W, 3, 3, 1, 1)
    Kg = 9 * C
    A = np.zeros((N * OH * OW, Kg))
    for m in range(N * OH * OW):
        n, oh, ow = m // (OH * OW), (m % (OH * OW)) // OW, m % OW
        for k in range(Kg):
            kh, kw, c = k // (3 * C), (k // C) % 3, k % C
            ih, iw = oh - 1 + kh, ow - 1 + kw
            if 0 <= ih < H and 0 <= iw < W:
                A[m, k] = x[n, ih, iw, c]
    ref = A @ _np64(Wt).reshape(Kg, Fo)
    np.testing.assert_allclose(O.conv2d_nhwc_ref(X, Wt, 1, 1).double().numpy().reshape(-1, Fo), ref,
                               rtol=1e-5, atol=1e-5)


def _e4m3_decode(byte: int) -> float:
    """OCP e4m3fn from its bits: bias 7, no infinities, S.1111.111 = NaN."""
    s = -1.0 if byte & 0x80 else 1.0
    e = (byte >> 3) & 0xF
    m = byte & 0x7
    if e == 0xF and m == 0x7:
        return float("nan")
    if e == 0:
        return s * (m / 8.0) * 2.0 ** -6
    return s * (1.0 + m / 8.0) * 2.0 ** (e - 7)


def test_fp8_dequant_matches_bit_decode():
    codes = torch.arange(256, dtype=torch.uint8)
    vals = codes.view(torch.float8_e4m3fn).float()
    for c in range(256):
        want = _e4m3_decode(c)
        got = vals[c].item()
        assert (math.isnan(want) and math.isnan(got)) or want == got, (c, want, got)
    assert _e4m3_decode(0x7E) == O.FP8_MAX


def test_fp8_ref_matches_fp64_with_scales():
    d = I.config5(M=8, N=16, K=32)
    a = np.array([[_e4m3_decode(int(b)) for b in row] for row in d["A"].view(torch.uint8).tolist()])
    b = np.array([[_e4m3_decode(int(v)) for v in row] for row in d["B"].view(torch.uint8).tolist()])
    x = a @ b * (d["scale_a"] * d["scale_b"]) + d["bias"].double().numpy()[None]
    ref = x / (1 + np.exp(-x))
    got = O.fp8_gemm_bias_act_ref(d["A"], d["B"], d["scale_a"], d["scale_b"], d["bias"], "silu")
    np.testing.assert_allclose(got.double().numpy(), ref, rtol=1e-5, atol=1e-6)
    # quantisation: scale = amax/448 maps the largest magnitude to exactly +-448
    assert abs(d["A"].float().abs().max().item() - 448.0) < 1e-6


def test_seeded_inputs_are_deterministic():
    a = I.config2(64, 64, 64)
    b = I.config2(64, 64, 64)
    for k in a:
        assert torch.equal(a[k], b[k])
    assert abs(I.config2(64, 64, 4096)["B"].float().std().item() - 1 / 64) < 2e-3
