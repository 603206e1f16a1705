"""fp8 decode over pre-packed weights (icpp_fp8_pack_b, icpp_fp8_gemm_packed) on the GPU:
the pack kernel's bytes against the layout's tensor permutation (pinned on the CPU in
test_fp8_pack_layout.py), and the one-launch decode GEMM against the dequantised fp32
oracle at the tolerance of the other fp8 parity tests, with the split-K path beside it."""

import sys
from pathlib import Path

import pytest
import torch

from icpp_tuning_amd import inputs as I
from icpp_tuning_amd import runtime
from icpp_tuning_amd.kernels import fp8_gemm_bias_act as fp8_mod
from oracle import ops as O

sys.path.insert(0, str(Path(__file__).resolve().parent))
from test_fp8_pack_layout import pack_ref  # noqa: E402

pytestmark = pytest.mark.gpu


def _close(got, ref, atol, rtol, what):
    got = got.float().cpu()
    err = (got - ref).abs()
    bad = err > atol + rtol * ref.abs()
    assert not bad.any(), f"{what}: {int(bad.sum())} of {bad.numel()} outside tolerance, max err {float(err.max()):.4g}"


@pytest.mark.parametrize("K,N", [(128, 16), (384, 48), (4096, 4096), (11008, 4096), (4096, 11008)])
def test_pack_kernel_matches_the_layout(gpu, K, N):
    g = torch.Generator().manual_seed(K + N)
    b = torch.randint(0, 256, (K, N), generator=g, dtype=torch.uint8)
    print(f"[decode] pack K={K} N={N}", flush=True)
    bp = runtime.fp8_pack_b(b.cuda().view(torch.float8_e4m3fn))
    torch.cuda.synchronize()
    assert torch.equal(bp.cpu(), pack_ref(b))


@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (5, 4096, 4096), (16, 4096, 4096), (16, 11008, 4096),
                                   (16, 4096, 11008), (3, 48, 384), (16, 16, 128), (17, 4096, 4096),
                                   (32, 4096, 11008), (23, 48, 384)])
@pytest.mark.parametrize("act,with_bias", [("silu", True), ("none", False)])
def test_decode_matches_oracle(gpu, M, N, K, act, with_bias):
    d = I.config5(M, N, K)
    bias = d["bias"] if with_bias else None
    ref = O.fp8_gemm_bias_act_ref(d["A"], d["B"], d["scale_a"], d["scale_b"], bias, act)
    print(f"[decode] M={M} N={N} K={K} act={act} bias={with_bias}", flush=True)
    bp = runtime.fp8_pack_b(d["B"].cuda())
    y = runtime.fp8_gemm_packed(d["A"].cuda(), bp, N, bias=bias.cuda() if bias is not None else None, act=act,
                                scale_a=d["scale_a"], scale_b=d["scale_b"])
    torch.cuda.synchronize()
    _close(y, ref, 1e-2, 1e-2, f"decode M={M} N={N} K={K} {act}")


def test_decode_beside_the_split_k_path(gpu):
    """The same call through icpp_gemm's tuned fp8 instance (split-K + reduce): both within
    the oracle's tolerance of each other (different summation orders, not bitwise)."""
    M, N, K = 16, 4096, 4096
    d = I.config5(M, N, K)
    k = fp8_mod.build_kernel(M, N, K)
    A, B, bias = d["A"].cuda(), d["B"].cuda(), d["bias"].cuda()
    y_split = k(A, B, d["scale_a"], d["scale_b"], bias)
    y_dec = runtime.fp8_gemm_packed(A, runtime.fp8_pack_b(B), N, bias=bias, act="silu", scale_a=d["scale_a"],
                                    scale_b=d["scale_b"])
    torch.cuda.synchronize()
    _close(y_dec, y_split.float().cpu(), 1e-2, 1e-2, "decode vs split-K")


@pytest.mark.parametrize("M", [7, 23])
def test_decode_rows_past_m_and_repeated_calls(gpu, M):
    """Rows m >= M are never written (the output past them keeps its contents), and two
    calls in a row on one output give identical results (one and two row tiles)."""
    N, K = 256, 1024
    d = I.config5(M, N, K)
    bp = runtime.fp8_pack_b(d["B"].cuda())
    buf = torch.full((32, N), 3.0, dtype=torch.bfloat16, device="cuda")
    out = buf[:M]
    a = d["A"].cuda()
    runtime.fp8_gemm_packed(a, bp, N, bias=d["bias"].cuda(), out=out, scale_a=d["scale_a"], scale_b=d["scale_b"])
    first = out.clone()
    runtime.fp8_gemm_packed(a, bp, N, bias=d["bias"].cuda(), out=out, scale_a=d["scale_a"], scale_b=d["scale_b"])
    torch.cuda.synchronize()
    assert torch.equal(first, out)
    assert bool((buf[M:] == 3.0).all())


def test_decode_in_a_graph(gpu):
    """The decode call has no workspace and allocates nothing: captured in a HIP graph and
    replayed three times, with eager work and a synchronize between replays, every replay
    equals the eager result bit for bit."""
    M, N, K = 16, 1024, 2048
    d = I.config5(M, N, K)
    a, bias = d["A"].cuda(), d["bias"].cuda()
    bp = runtime.fp8_pack_b(d["B"].cuda())
    eager = runtime.fp8_gemm_packed(a, bp, N, bias=bias, scale_a=d["scale_a"], scale_b=d["scale_b"])
    out = torch.empty_like(eager)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        runtime.fp8_gemm_packed(a, bp, N, bias=bias, out=out, scale_a=d["scale_a"], scale_b=d["scale_b"])
    for rep in range(3):
        out.fill_(0.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {rep}"
        _ = (a.float() * 2).sum().item()  # eager work between replays


def test_build_packed_kernel(gpu):
    """The module-level wrapper: weights packed once at build time, then calls like the
    tiled kernel's (a_q, scale_a, scale_b, bias)."""
    M, N, K = 9, 512, 1024
    d = I.config5(M, N, K)
    ref = O.fp8_gemm_bias_act_ref(d["A"], d["B"], d["scale_a"], d["scale_b"], d["bias"], "silu")
    k = fp8_mod.build_packed_kernel(d["B"].cuda())
    y = k(d["A"].cuda(), d["scale_a"], d["scale_b"], d["bias"].cuda())
    torch.cuda.synchronize()
    _close(y, ref, 1e-2, 1e-2, "build_packed_kernel")
