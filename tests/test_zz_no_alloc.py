"""icpp_gemm_noalloc (through the C ABI) against icpp_gemm with a caller workspace.

Both run the same kernels in the same order, so the outputs must be bit-identical.
Two calls in a row, the second smaller, so a stale partial left in the shared
static scratch by the first call would show up in the second; plus a split-K-free
call and a rejected oversize call (refused on the host, before any launch).
"""

import ctypes
import math

import pytest
import torch

from icpp_tuning_amd import inputs as I
from icpp_tuning_amd import runtime
from icpp_tuning_amd._lib import ACT, lib
from icpp_tuning_amd.kernels._base import family_instances
from oracle import ops as O

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20  # ICPP_NOALLOC_SCRATCH_BYTES in include/icpp_hip.h


def _inst(name):
    fam = family_instances("gemm")
    return next(i for i, t in enumerate(fam) if t.name == name), next(t for t in fam if t.name == name)


def _noalloc(idx, dtype, A, B, bias, act, split_k, scale_a=1.0, scale_b=1.0):
    M, K = A.shape
    N = B.shape[1]
    out = torch.full((M, N), float("nan"), dtype=runtime.OUT_DTYPE[dtype], device=A.device)
    lib().call("icpp_gemm_noalloc", idx, A.data_ptr(), B.data_ptr(), bias.data_ptr() if bias is not None else None,
               out.data_ptr(), M, N, K, K, N, N, ACT[act], float(scale_a), float(scale_b), split_k,
               torch.cuda.current_stream().cuda_stream)
    return out


def _with_workspace(idx, dtype, A, B, bias, act, split_k, scale_a=1.0, scale_b=1.0):
    return runtime.gemm(idx, dtype, A, B, bias=bias, act=act, scale_a=scale_a, scale_b=scale_b, split_k=split_k)


CASES = [
    # (instance, dtype, M, N, K, split_k, act): the first fills most of the scratch, the second is smaller
    ("gemm_fp8_64x128x128_w1x4_m16_s4", "fp8", 64, 4096, 4096, 8, "silu"),
    ("gemm_fp8_64x128x128_w1x4_m16_s4", "fp8", 16, 1024, 2048, 4, "silu"),
    ("gemm_bf16_128x128x64_w2x2_m16_s2", "bf16", 200, 1032, 1024, 4, "gelu_tanh"),
    ("gemm_bf16_128x128x64_w2x2_m16_s2", "bf16", 72, 264, 512, 3, "relu"),
]


@pytest.mark.parametrize("order", ["as_listed"])
def test_noalloc_matches_workspace_entry_point(gpu, order):
    for (name, dtype, M, N, K, sk, act) in CASES:
        idx, inst = _inst(name)
        assert sk * M * N * 4 <= SCRATCH_BYTES
        print(f"[noalloc] {name} M={M} N={N} K={K} split_k={sk} act={act}", flush=True)
        if dtype == "fp8":
            d = I.config5(M, N, K, device="cuda")
            args = (d["A"], d["B"], d["bias"], act, sk, d["scale_a"], d["scale_b"])
        else:
            d = I.gemm_inputs(M, N, K, runtime.TORCH_DTYPE[dtype], 91, b_std=1 / math.sqrt(K), bias=True,
                              device="cuda")
            args = (d["A"], d["B"], d["bias"], act, sk)
        y0 = _noalloc(idx, dtype, *args)
        y1 = _with_workspace(idx, dtype, *args)
        torch.cuda.synchronize()
        assert torch.equal(y0.view(torch.int16), y1.view(torch.int16)), f"{name}: outputs differ"
        # and to the oracle's tolerance (bf16 out: rtol 1e-2 / atol 1e-2)
        if dtype == "fp8":
            ref = O.fp8_gemm_bias_act_ref(d["A"], d["B"], d["scale_a"], d["scale_b"], d["bias"], act)
        else:
            ref = O.gemm_bias_act_ref(d["A"], d["B"], d["bias"], act)
        err = (y0.float().cpu() - ref).abs()
        assert bool((err <= 1e-2 + 1e-2 * ref.abs()).all()), f"{name}: max err {err.max().item():.4g}"


def test_noalloc_without_split_k(gpu):
    idx, _ = _inst("gemm_bf16_128x128x64_w2x2_m16_s2")
    d = I.gemm_inputs(136, 264, 256, torch.bfloat16, 92, b_std=1 / 16, bias=True, device="cuda")
    y0 = _noalloc(idx, "bf16", d["A"], d["B"], d["bias"], "silu", 1)
    y1 = _with_workspace(idx, "bf16", d["A"], d["B"], d["bias"], "silu", 1)
    torch.cuda.synchronize()
    assert torch.equal(y0.view(torch.int16), y1.view(torch.int16))


def test_noalloc_rejects_partials_beyond_the_scratch(gpu):
    idx, _ = _inst("gemm_fp8_64x128x128_w1x4_m16_s4")
    M, N, K, sk = 256, 11008, 4096, 4  # 45 MB of partials
    assert sk * M * N * 4 > SCRATCH_BYTES
    d = I.config5(M, N, K, device="cuda")
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    rc = lib()._dll.icpp_gemm_noalloc(idx, d["A"].data_ptr(), d["B"].data_ptr(), d["bias"].data_ptr(),
                                      out.data_ptr(), M, N, K, K, N, N, ACT["silu"], ctypes.c_float(d["scale_a"]),
                                      ctypes.c_float(d["scale_b"]), sk, torch.cuda.current_stream().cuda_stream)
    assert rc == -3, rc  # ICPP_E_WORKSPACE
    assert "static scratch" in lib().last_error()


def test_noalloc_captured_in_a_graph(gpu):
    """After a first eager call on the device (the one that resolves the scratch array's
    address), a split-K icpp_gemm_noalloc call is captured in a HIP graph; every replay,
    with eager work in between, matches icpp_gemm with a caller workspace bitwise."""
    name, dtype, M, N, K, sk, act = "gemm_bf16_128x128x64_w2x2_m16_s2", "bf16", 200, 1032, 1024, 4, "gelu_tanh"
    idx, _ = _inst(name)
    d = I.gemm_inputs(M, N, K, runtime.TORCH_DTYPE[dtype], 93, b_std=1 / math.sqrt(K), bias=True, device="cuda")
    ref = _with_workspace(idx, dtype, d["A"], d["B"], d["bias"], act, sk)
    out = torch.empty((M, N), dtype=runtime.OUT_DTYPE[dtype], device="cuda")

    def run():
        lib().call("icpp_gemm_noalloc", idx, d["A"].data_ptr(), d["B"].data_ptr(), d["bias"].data_ptr(),
                   out.data_ptr(), M, N, K, K, N, N, ACT[act], 1.0, 1.0, sk,
                   torch.cuda.current_stream().cuda_stream)

    run()
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        run()
    torch.cuda.synchronize()
    for r in range(4):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {r} differs"
