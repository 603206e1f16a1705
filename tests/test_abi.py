"""The C ABI library: loads without a GPU, exports every declared symbol, its
instance table matches instances.py, and argument validation rejects bad
calls before anything is launched (no device work happens in these tests)."""

import ctypes
import re
from pathlib import Path

import pytest

from icpp_tuning_amd import _lib, runtime
from icpp_tuning_amd.instances import INSTANCES
from icpp_tuning_amd.kernels._base import family_instances

HEADER = Path(__file__).resolve().parents[1] / "include" / "icpp_hip.h"


@pytest.fixture(scope="module")
def L():
    return _lib.lib()


def test_header_symbols_are_exported(L):
    declared = set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(icpp_\w+)\s*\(", HEADER.read_text(), re.M))
    assert declared == set(_lib.EXPORTED_SYMBOLS)
    for name in declared:
        assert L.has_symbol(name), name


def test_abi_version(L):
    assert L._dll.icpp_abi_version() == _lib.ABI_VERSION


def test_instance_table_matches_python_list(L):
    for fam, fid in _lib.FAMILY.items():
        rows = L.instances(fid)
        expect = family_instances(fam)
        assert [r["name"] for r in rows] == [i.name for i in expect]
        for r, i in zip(rows, expect):
            assert (r["block_m"], r["block_n"], r["block_k"], r["waves_m"], r["waves_n"], r["stages"], r["mfma_m"]) == (
                i.bm, i.bn, i.bk, i.wm, i.wn, i.stages, i.mf)
            assert r["lds_bytes"] == i.lds_bytes and r["threads"] == i.threads
    assert sum(len(L.instances(f)) for f in _lib.FAMILY.values()) == len(INSTANCES)


def test_resources_recorded_for_every_instance():
    res = _lib.resources()
    for i in INSTANCES:
        r = res[i.name]
        # pipeline stages plus the 16-byte placeholders of unused stage arrays
        assert i.lds_bytes <= r["lds"] <= i.lds_bytes + 64, (i.name, r["lds"])
        assert r["vgprs"] + r["agprs"] <= 512
        assert r["scratch"] == 0, i.name


def test_workspace_bytes(L):
    gemm0 = 0
    assert L.workspace_bytes(_lib.FAMILY["gemm"], gemm0, 128, 256, 512, 1) == 0
    assert L.workspace_bytes(_lib.FAMILY["gemm"], gemm0, 128, 256, 512, 4) == 4 * 128 * 256 * 4
    st = family_instances("gemm_ln_stats")[0]
    cols = -(-1000 // (st.bn // st.wn))
    assert L.workspace_bytes(_lib.FAMILY["gemm_ln_stats"], 0, 64, 1000, 512, 1) == 64 * cols * 2 * 4


def _gemm_call(L, inst=0, A=16, B=16, C=16, M=64, N=64, K=64, ldc=None, split=1, ws=None, wsb=0, act=0):
    f = L._dll.icpp_gemm
    return f(inst, A, B, None, C, M, N, K, K, N, N if ldc is None else ldc, act, 1.0, 1.0, split, ws, wsb, None)


def test_validation_errors_before_launch(L):
    # null tensors, bad instance, bad shapes, missing workspace: all rejected on the host
    assert _gemm_call(L, A=None) == -4
    assert _gemm_call(L, inst=10 ** 6) == -1
    assert _gemm_call(L, N=60) == -2           # N % 8
    assert _gemm_call(L, K=40) == -2           # K not a multiple of block_k
    assert _gemm_call(L, act=9) == -4
    assert _gemm_call(L, split=2, K=256) == -3  # split-K without workspace
    assert _gemm_call(L, split=64, K=256) == -2  # more slices than K tiles
    assert _gemm_call(L, A=17) == -4           # misaligned pointer
    assert "aligned" in L.last_error()
    f = L._dll.icpp_gemm_bias_layernorm
    assert f(7, 0, 16, 16, None, 16, 16, 16, 64, 64, 64, 1e-5, None, 0, None) == -1
    row = _lib.FAMILY["gemm_ln_row"]
    assert f(row, 0, 16, 16, None, 16, 16, 16, 64, 2048, 64, 1e-5, None, 0, None) == -2  # N > block_n
    # GEMM-then-LN: f16 GEMM instances only, and the residual may not overlap Y
    fr = L._dll.icpp_gemm_bias_residual_layernorm
    gem = _lib.FAMILY["gemm"]
    gems = family_instances("gemm")
    i16 = next(i for i, t in enumerate(gems) if t.dtype == "f16")
    ibf = next(i for i, t in enumerate(gems) if t.dtype == "bf16")
    assert fr(gem, ibf, 16, 16, None, None, 16, 16, 4096, 64, 64, 64, 1e-5, None, 0, None) == -1
    assert fr(gem, i16, 16, 16, None, 4096 + 64, 16, 16, 4096, 64, 64, 64, 1e-5, None, 0, None) == -4
    assert "overlap" in L.last_error()
    # co-resident LayerNorm: f16 GEMM tiles only (every one carries its kernel; bf16 and
    # fp8 tiles do not), checked before any device query
    cr = _lib.LN_CORESIDENT
    i8 = next(i for i, t in enumerate(gems) if t.dtype == "fp8")
    for bad in (ibf, i8):
        assert fr(cr, bad, 16, 16, None, None, 16, 16, 4096, 64, 64, 64, 1e-5, None, 0, None) == -1
        assert "co-resident" in L.last_error()
    assert fr(cr, i16, 16, 16, None, None, 16, 16, 4096, 64, 64, 64, -1.0, None, 0, None) == -4  # eps
    c = L._dll.icpp_conv2d_nhwc
    assert c(0, 16, 16, 16, 1, 8, 8, 3, 64, 3, 3, 1, 1, 1, 1, None, 0, None) == -2  # C % 8


def test_coresident_workspace_layout(L):
    """ICPP_LN_CORESIDENT workspace: M x ceil(N / block_n) (mean, M2) fp32 pairs, 16-byte
    aligned, then a 16-byte error block, then two int counters per block_m rows; none
    for tiles without the co-resident kernel."""
    from icpp_tuning_amd.kernels import gemm_bias_layernorm as ln_mod

    gems = family_instances("gemm")
    n_cr = 0
    for i, t in enumerate(gems):
        for M, N in ((333, 776), (8192, 4096), (1, 8)):
            got = L.ln_workspace_bytes(_lib.LN_CORESIDENT, i, M, N, 512)
            if not ln_mod.coresident_fits(t, 0):
                assert got == 0, t.name
                continue
            pairs = M * -(-N // t.bn) * 8
            assert got == -(-pairs // 16) * 16 + 16 + -(-M // t.bm) * 8, (t.name, M, N)
            # the runtime's int32 view of it (error word, counters) ends where the library's does
            err, ctr, n = runtime.coresident_layout(i, M, N)
            assert err * 4 == -(-pairs // 16) * 16 and ctr == err + 4 and (ctr + n) * 4 == got, (t.name, M, N)
        n_cr += ln_mod.coresident_fits(t, 0)
    assert n_cr >= 20
    assert L.ln_workspace_bytes(_lib.LN_CORESIDENT, len(gems), 64, 64, 64) == 0


def test_fused_conv_validation_errors_before_launch(L):
    """icpp_conv2d_nhwc_fused rejects inconsistent epilogue arguments before any
    device work (pointers are never dereferenced on these paths)."""
    f = L._dll.icpp_conv2d_nhwc_fused
    geo = (2, 8, 8, 64, 64, 3, 3, 1, 1, 1, 1, None, 0, None)   # N H W C F KH KW s p d split ws wsb stream

    def call(res=None, g=None, b=None, m=None, v=None, eps=1e-5, flags=0, act=0, X=16, Y=16):
        return f(0, X, 16, Y, res, g, b, m, v, ctypes.c_float(eps), flags, act, *geo)

    BN, RES, CLAMP = _lib.CONV_EPI["bn"], _lib.CONV_EPI["residual"], _lib.CONV_EPI["var_clamp"]
    assert call(flags=8) == -4                                  # unknown flag
    assert call(act=_lib.ACT["silu"]) == -4                     # only none / relu
    assert call(flags=BN) == -4                                 # BN without its parameters
    assert call(flags=BN, g=16, b=16, m=16) == -4               # ... var missing
    assert call(flags=CLAMP) == -4                              # clamp without BN
    assert call(flags=RES) == -4                                # residual flag, no residual
    assert call(flags=BN, g=16, b=16, m=16, v=16, eps=-1.0) == -4
    assert call(flags=BN, g=24, b=16, m=16, v=16) == -4         # misaligned gamma
    assert call(flags=RES, res=40) == -4                        # misaligned residual
    assert call(X=None) == -4
    assert "icpp_conv2d_nhwc" in L.last_error()


def test_rowops_validation_errors_before_launch(L):
    """icpp_layernorm_fwd / _bwd and icpp_softmax reject bad arguments before any
    device work; the backward's workspace size follows one fp32 [dw | db] row per
    workgroup (at most 256)."""
    f16, f32 = _lib.DTYPE["f16"], _lib.DTYPE["f32"]
    fwd, bwd, sm = L._dll.icpp_layernorm_fwd, L._dll.icpp_layernorm_bwd, L._dll.icpp_softmax
    eps = ctypes.c_float(1e-5)
    assert fwd(f16, None, 16, 16, 16, None, None, 4, 64, 64, 64, eps, None) == -4       # null x
    assert fwd(9, 16, 16, 16, 16, None, None, 4, 64, 64, 64, eps, None) == -4          # bad dtype
    assert fwd(f16, 16, 16, 16, 16, None, None, 4, 64, 32, 64, eps, None) == -2        # ld < N
    assert fwd(f16, 16, 16, 16, 16, None, None, 0, 64, 64, 64, eps, None) == -2        # empty
    assert fwd(f16, 16, 16, 16, 16, None, None, 4, 64, 64, 64, ctypes.c_float(-1.0), None) == -4
    assert fwd(f16, 16, 16, 16, 16, None, None, 4, 1 << 17, 1 << 17, 1 << 17, eps, None) == -2  # row too long
    assert sm(f32, None, 16, 4, 64, 64, 64, None) == -4
    assert sm(f32, 16, 16, 4, 20000, 20001, 20001, None) == -2                        # scalar path limit 16384
    smm = L._dll.icpp_softmax_scaled_masked
    assert smm(f32, None, 16, None, 1.0, 4, 64, 64, 64, 1, None) == -4                  # null x
    assert smm(f32, 16, 16, 16, 1.0, 4, 64, 64, 64, 0, None) == -2                      # mask without rows
    assert smm(f32, 16, 16, None, float("inf"), 4, 64, 64, 64, 1, None) == -4          # non-finite scale
    assert smm(f32, 16, 16, None, float("nan"), 4, 64, 64, 64, 1, None) == -4
    qs, mh = L._dll.icpp_qkv_split_heads, L._dll.icpp_merge_heads
    assert qs(f16, None, None, 16, 16, 16, 2, 128, 12, 64, 0, None) == -4              # null qkv
    assert qs(f16, 16, None, 16, 16, 16, 2, 128, 12, 32, 0, None) == -2                # head_dim 64 only
    assert qs(f32, 16, None, 16, 16, 16, 2, 128, 12, 64, 0, None) == -4                # f16 / bf16 only
    assert qs(f16, 24, None, 16, 16, 16, 2, 128, 12, 64, 0, None) == -4                # misaligned
    assert qs(f16, 16, None, 16, 16, 16, 0, 128, 12, 64, 0, None) == -2                # empty
    assert qs(f16, 16, None, 16, 16, 16, 2, 128, 12, 64, 2, None) == -4                # layout 0 or 1
    att = L._dll.icpp_attention_fwd
    assert att(f16, 16, 16, 16, None, 0.125, 16, 2, 100, 12, 64, None) == -2           # seq % 32
    assert att(f16, 16, 16, 16, None, 0.125, 16, 2, 544, 12, 64, None) == -2           # seq <= 512
    assert att(f16, 16, 16, 16, None, float("inf"), 16, 2, 128, 12, 64, None) == -4
    assert att(f16, None, 16, 16, None, 0.125, 16, 2, 128, 12, 64, None) == -4
    assert att(f16, 16, 16, 16, 24, 0.125, 16, 2, 128, 12, 64, None) == -4             # misaligned mask
    assert "icpp_attention_fwd" in L.last_error()
    assert mh(f16, 16, 16, 2, 128, 12, 48, None) == -2
    assert mh(f16, 16, None, 2, 128, 12, 64, None) == -4
    assert "icpp_merge_heads" in L.last_error()
    ws = L.layernorm_bwd_workspace_bytes
    # N = 8192 f16: one 16-byte chunk per thread, 1024 threads = one row per workgroup
    assert ws(f16, 4096, 8192, 8192) == 256 * 2 * 8192 * 4
    assert ws(f16, 100, 8192, 8192) == 100 * 2 * 8192 * 4
    # N = 1024 f16: the larger of the vector geometry (128 threads per row, 8 rows per
    # workgroup: 13 groups) and the scalar one (256 threads per row, 4 rows: 25 groups)
    assert ws(f16, 100, 1024, 1024) == 25 * 2 * 1024 * 4
    assert ws(f16, 4096, 32768, 32768) == 0                                           # beyond the backward's limit
    args = (f16, 16, 16, 16, 16, 16, 16, 16, 16, 4096, 8192, 8192)
    assert bwd(*args, None, 0, None) == -3                                             # no workspace
    assert bwd(*args, 16, 1024, None) == -3                                            # too small
    assert bwd(f16, None, *args[2:], 16, 1 << 30, None) == -4                          # null dy
    assert "icpp_layernorm_bwd" in L.last_error()


def test_fp8_packed_decode_rejections_before_launch(L):
    """icpp_fp8_pack_b / icpp_fp8_gemm_packed check every argument before any device work
    (the pointers here are never dereferenced)."""
    pk = L._dll.icpp_fp8_pack_b
    assert pk(None, 32, 256, 64, None) == -4
    assert pk(16, 32, 200, 64, None) == -2          # K % 128
    assert pk(16, 32, 256, 40, None) == -2          # N % 16
    assert pk(16, 33, 256, 64, None) == -4          # Bp misaligned
    g = L._dll.icpp_fp8_gemm_packed
    ok = dict(A=16, Bp=32, bias=None, C=48, M=4, N=64, K=256, act=3)

    def call(**kw):
        a = dict(ok, **kw)
        return g(a["A"], a["Bp"], a["bias"], a["C"], a["M"], a["N"], a["K"], a["act"], 1.0, 1.0, None)

    assert call(M=0) == -2 and call(M=33) == -2
    assert call(K=200) == -2 and call(N=40) == -2 and call(K=0) == -2
    assert call(A=None) == -4 and call(C=None) == -4
    assert call(act=9) == -4
    assert call(A=24) == -4 and call(bias=8) == -4
    assert "aligned" in L.last_error()
