"""Search space: the reference's documented pruning counts (A100), sampling
invariants, and the CDNA4 pruning rules (LDS, VGPR, occupancy, CU fill)."""

import math
from collections import Counter

import pytest

from icpp_tuning_amd.autotuner import search_space as ss
from icpp_tuning_amd.autotuner.cost_model import TuneConfig
from icpp_tuning_amd.autotuner.gpu_spec import A100, MI355X


def test_a100_tilelang_matmul_prune_counts():
    """Known answer from the reference design doc (docs/autotuner_design.md:240-245, 396):
    TileLang matmul 252 -> 229 after L1+L2 -> 86 after L3."""
    full = ss.generate_exhaustive_configs("matmul", "tilelang")
    assert len(full) == 252
    l1 = ss.prune_shared_memory(full, A100)
    l2 = ss.prune_register_pressure(l1, A100)
    l3 = ss.prune_minimum_occupancy(l2, A100)
    assert (len(l1), len(l2), len(l3)) == (244, 229, 86)
    # 21 four-warp + 65 eight-warp survivors
    assert Counter(c.num_warps for c in l3) == {4: 21, 8: 65}


def test_exhaustive_generation_does_not_crash_for_every_backend():
    for op in ("matmul", "conv2d"):
        for be in ("tilelang", "triton", "hip"):
            assert ss.generate_exhaustive_configs(op, be)


def test_lcm_marginal_uniformity():
    pools = {"a": [1, 2, 3], "b": [10, 20], "c": [5, 6, 7, 8]}
    out = ss.lcm_marginal_sample(pools, seed=1)
    assert len(out) == 12
    for name, pool in pools.items():
        cnt = Counter(d[name] for d in out)
        assert set(cnt) == set(pool) and len(set(cnt.values())) == 1
    assert out == ss.lcm_marginal_sample(pools, seed=1)


def test_stratified_sample_properties():
    valid = ss.prune_configs(ss.generate_exhaustive_configs("matmul", "tilelang"), A100)
    s = ss._stratified_sample_from_valid(valid, seed=3)
    keys = [ss._key(c) for c in s]
    assert len(keys) == len(set(keys))
    assert set(keys) <= {ss._key(c) for c in valid}
    # default size min(max(2*LCM, 30), |valid|)
    pools = [len({getattr(c, f) for c in valid}) for f in ("block_M", "block_N", "block_K", "num_stages", "num_warps")]
    lcm = math.lcm(*pools)
    assert len(s) == min(max(2 * lcm, 30), len(valid))
    small = ss._stratified_sample_from_valid(valid, n_samples=14, seed=3)
    per_bm = Counter(c.block_M for c in small)
    assert max(per_bm.values()) - min(per_bm.values()) <= 1


def _cfg(bm, bn, bk, st=2, waves=4, mf=32, esz=2, vgprs=0, sk=1):
    kf = {(2, 16): 32, (2, 32): 16, (1, 16): 128, (1, 32): 64}[(esz, mf)]
    return TuneConfig(bm, bn, bk, st, waves, warp_size=64, a_bytes=esz, b_bytes=esz, mfma=f"{mf}x{mf}x{kf}",
                      vgprs=vgprs, split_k=sk)


def test_cdna4_l1_rejects_lds_overflow():
    ok = _cfg(256, 256, 64, st=2)          # 128 KiB
    too_big = _cfg(256, 256, 128, st=2)    # 256 KiB
    assert ss.prune_shared_memory([ok, too_big], MI355X) == [ok]


def test_cdna4_l2_rejects_vgpr_overflow():
    fits = _cfg(128, 128, 64, waves=4)                 # 64 acc regs / lane
    spills = _cfg(256, 256, 64, waves=4, vgprs=600)    # compiler-reported overflow
    eight_waves = _cfg(256, 256, 64, waves=8, vgprs=300)  # 2 waves / SIMD -> 256 budget
    assert ss.prune_register_pressure([fits, spills, eight_waves], MI355X) == [fits]


def test_cdna4_l4_rejects_cu_underfill():
    big = _cfg(256, 256, 64)
    small = _cfg(64, 64, 64)
    # 1024 x 1024: 256-tiles give 16 workgroups (6% of 256 CUs), 64-tiles give 256
    assert ss.prune_cu_underfill([big, small], MI355X, 1024, 1024) == [small]
    # 8192 x 8192: both fill the machine
    assert len(ss.prune_cu_underfill([big, small], MI355X, 8192, 8192)) == 2
    # split-K counts toward the grid
    assert len(ss.prune_cu_underfill([_cfg(256, 256, 64, sk=8), small], MI355X, 1024, 1024)) == 2


def test_cdna4_summary_runs():
    s = ss.search_space_summary("matmul", MI355X, backend="hip", dtype="bf16")
    assert s["exhaustive_full"] >= s["after_smem_prune"] >= s["after_reg_prune"] >= s["after_occupancy_prune"] > 0


def test_sample_shapes():
    shapes = ss.generate_matmul_sample_shapes()
    ms = sorted({s["M"] for s in shapes})
    assert ms[:16] == list(range(1, 17)) and ms[-1] == 4096
    assert len(ss.generate_conv2d_sample_shapes()) == 6 * 6 * 4 * 4


def test_tiles_of_8x_the_rows_are_not_offered():
    """A tile of 8x or more the problem's rows (rounded to 16) is not offered while a
    shorter one is: at M = 16 no 128- or 256-row tile, at M = 40 (48 rows) none of 384+."""
    from icpp_tuning_amd.kernels import fp8_gemm_bias_act as F

    d = F.DESCRIPTOR
    rows16 = {c["block_M"] for c in d.get_raw_configs(M=16, N=4096, K=4096)}
    assert rows16 and max(rows16) < 128 and 16 in rows16
    rows40 = {c["block_M"] for c in d.get_raw_configs(M=40, N=4096, K=4096)}
    assert 256 in rows40
    rows4k = {c["block_M"] for c in d.get_raw_configs(M=4096, N=4096, K=4096)}
    assert rows4k == {i.bm for i in d.instances()}
