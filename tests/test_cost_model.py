"""Cost model: A100 reference-mode parity against the reference's published
scores, then CDNA4-mode properties."""

import json
import math
from dataclasses import replace
from pathlib import Path

import pytest

from icpp_tuning_amd.autotuner import cost_model as cm
from icpp_tuning_amd.autotuner.gpu_spec import A100, MI355X
from oracle import reference_configs as rc

GOLD = json.loads((Path(__file__).parent / "golden" / "formula_scores.json").read_text())
# CSV scores are printed with 6 decimals
SCORE_TOL = 5.1e-7


def _argmax(op, M, N, K):
    best, best_s = None, -1.0
    for raw in rc.configs_for(op, M, K):
        s = rc.adjust(op, raw, cm.score_formula(rc.op_spec(op, raw, M, N, K), rc.to_tune_config(raw), A100))
        if s > best_s:
            best, best_s = raw, s
    return best, best_s


@pytest.mark.parametrize("row", GOLD["gemm"], ids=lambda r: f"{r['op']}-M{r['M']}")
def test_a100_gemm_top1_and_score(row):
    best, score = _argmax(row["op"], row["M"], row["N"], row["K"])
    assert rc.format_config(best) == row["config"]
    assert abs(score - row["score"]) <= SCORE_TOL


@pytest.mark.parametrize("row", GOLD["conv2d"], ids=lambda r: f"conv-N{r['N']}-C{r['C']}-H{r['H']}-F{r['F']}")
def test_a100_conv_top1_and_score(row):
    spec = rc.conv_spec(row["N"], row["C"], row["H"], row["W"], row["F"], row["KH"], row["KW"], row["stride"], row["pad"])
    best, best_s = None, -1.0
    for raw in rc.conv_configs():
        s = cm.score_formula(spec, rc.to_tune_config(raw), A100)
        if s > best_s:
            best, best_s = raw, s
    assert rc.format_config(best) == row["config"]
    assert abs(best_s - row["score"]) <= SCORE_TOL


def test_a100_specific_score_of_named_config():
    """Score of a fixed (not argmax) config: gemm_bias_act M=1 BM16_BN128_BK64_S2_T128 = 0.001136."""
    raw = rc.parse_config("BM16_BN128_BK64_S2_T128")
    s = cm.score_formula(rc.op_spec("gemm_bias_act", raw, 1, 2304, 768), rc.to_tune_config(raw), A100)
    assert abs(s - 0.001136) <= SCORE_TOL


def test_reference_mode_is_the_factor_product():
    op = cm.make_matmul_spec(256, 256, 256)
    cfg = cm.TuneConfig(64, 128, 32, 2, 4)
    d = cm.score_formula_detailed(op, cfg, A100)
    factors = [v for k, v in d.items() if k.startswith("eff_")]
    assert len(factors) == 7
    assert d["score"] == pytest.approx(math.prod(factors))
    assert "schedule" not in d
    assert cfg.threads == 128


def test_cdna4_threads_lds_and_dtype():
    cfg = cm.TuneConfig(256, 256, 128, 2, 4, warp_size=64, a_bytes=1, b_bytes=1, mfma="32x32x64", waves_m=2, waves_n=2)
    assert cfg.threads == 256
    assert cfg.shared_mem_bytes == (256 * 128 + 128 * 256) * 2
    fp8 = cm.make_matmul_spec(4096, 4096, 4096, dtype="fp8")
    assert fp8.mainloop.input_element_bytes == 1
    assert MI355X.ridge_point("fp8") == pytest.approx(5033.2e3 / 8000.0)


def test_cdna4_prefers_large_tiles_for_large_gemm():
    op = cm.make_matmul_spec(4096, 4096, 4096, dtype="bf16")
    big = cm.TuneConfig(256, 256, 64, 2, 4, warp_size=64, mfma="32x32x16", waves_m=2, waves_n=2)
    small = cm.TuneConfig(64, 64, 64, 2, 4, warp_size=64, mfma="16x16x32", waves_m=2, waves_n=2)
    assert cm.score_formula(op, big, MI355X) > cm.score_formula(op, small, MI355X)


# Constants that remove every cost but MFMA issue: no latency, no per-step or
# per-tile cost, unbounded L2 / store / epilogue rates, LDS made free below.
_MFMA_ONLY = cm.ModelConstants(
    mfma_rate=cm.CDNA4_CONSTANTS.mfma_rate, l2_bytes_per_clk_per_cu=1e12, mem_latency_clk=0.0,
    step_overhead_clk=0.0, tile_overhead_clk=0.0, store_bytes_per_clk_per_cu=1e12,
    epilogue_flops_per_clk_per_cu=1e12, hbm_efficiency=1.0, launch_overhead_s=0.0)


def _cfg(bm, bn, bk, waves, wm, wn, mfma, stages=2, sk=1, a_bytes=2):
    return cm.TuneConfig(bm, bn, bk, stages, waves, warp_size=64, mfma=mfma, waves_m=wm, waves_n=wn,
                         split_k=sk, a_bytes=a_bytes, b_bytes=a_bytes)


def test_cdna4_ideal_seconds_closed_form():
    op = cm.make_matmul_spec(4096, 4096, 4096, dtype="bf16")
    assert cm.ideal_seconds(op, _cfg(256, 256, 64, 4, 2, 2, "32x32x16"), MI355X) == pytest.approx(
        2 * 4096 ** 3 / 2516.6e12)
    fp8 = cm.make_matmul_spec(4096, 4096, 4096 // 4, dtype="fp8")   # a split-K spec carries K / split_k
    assert cm.ideal_seconds(fp8, _cfg(128, 128, 128, 4, 2, 2, "16x16x128", sk=4, a_bytes=1), MI355X) == \
        pytest.approx(2 * 4096 ** 3 / 5033.2e12)


@pytest.mark.parametrize("mfma,rate", [("32x32x16", 1.0), ("16x16x32", 0.87)])
def test_cdna4_mfma_bound_tile_reaches_the_shape_rate(mfma, rate):
    """One 256x256 tile per CU (4096^2 outputs = 256 tiles), four waves on four
    SIMDs: with every other cost removed the launch runs at the MFMA shape's
    sustained rate, i.e. the dense peak times the rate, whatever the shape."""
    op = cm.make_matmul_spec(4096, 4096, 4096, dtype="bf16")
    cfg = _cfg(256, 256, 64, 4, 2, 2, mfma)
    hw = replace(MI355X, lds_bytes_per_clk=1 << 30)
    t = cm.predict_schedule(op, cfg, hw, _MFMA_ONLY)
    assert t["n_cu"] == 1 and t["rounds"] == 1
    # the quoted peak (2516.6 TFLOP/s) is 256 CUs x 2.4 GHz x 4096 FLOP/clk to 5 digits
    assert cm.ideal_seconds(op, cfg, hw) / t["seconds"] == pytest.approx(rate, rel=1e-4)


def test_cdna4_waves_queue_on_the_busiest_simd():
    """Three 2-wave workgroups on one CU put 6 waves on 4 SIMDs: two SIMDs
    hold two waves, so the CU takes 2 wave-issue times per round, not 1.5."""
    op = cm.make_matmul_spec(128 * 256 * 3, 64, 4096, dtype="f16")   # 768 tiles: 3 per CU
    cfg = _cfg(128, 64, 64, 2, 2, 1, "32x32x16")
    hw = replace(MI355X, lds_bytes_per_clk=1 << 30)
    t = cm.predict_schedule(op, cfg, hw, _MFMA_ONLY)
    assert t["n_cu"] == 3 and t["concurrent"] == 3
    wave_issue = (64 // 32) * (64 // 32) * (64 // 16) * 32          # one wave's 64x64 tile, one K step
    steps = 4096 // 64
    assert t["mainloop_s"] == pytest.approx(2 * wave_issue * steps / (MI355X.clock_ghz * 1e9))


def test_cdna4_latency_bound_scales_with_prefetch_depth():
    """A latency-bound tile: per K step it waits memory latency / (stages - 1),
    so going from 2 to 4 stages divides the mainloop by 3."""
    c = replace(_MFMA_ONLY, mem_latency_clk=1e6)
    op = cm.make_matmul_spec(256, 256, 4096, dtype="f16")
    t2 = cm.predict_schedule(op, _cfg(64, 64, 64, 4, 2, 2, "16x16x32", stages=2), MI355X, c)
    t4 = cm.predict_schedule(op, _cfg(64, 64, 64, 4, 2, 2, "16x16x32", stages=4), MI355X, c)
    assert not t2["throughput_bound"]
    assert t2["mainloop_s"] == pytest.approx(1e6 * 64 / (MI355X.clock_ghz * 1e9))
    assert t2["mainloop_s"] / t4["mainloop_s"] == pytest.approx(3.0)


def test_cdna4_split_k_pays_its_reduction():
    """Split-K: the reduction reads every fp32 partial and writes the output once,
    plus a launch; no reduction without a split."""
    c = replace(_MFMA_ONLY, launch_overhead_s=2e-6, reduce_efficiency=0.5)
    M = N = 1024
    full = cm.make_matmul_spec(M, N, 4096)
    split = cm.make_matmul_spec(M, N, 4096 // 4)
    assert cm.predict_schedule(full, _cfg(128, 128, 64, 4, 2, 2, "16x16x32"), MI355X, c)["reduce_s"] == 0.0
    r = cm.predict_schedule(split, _cfg(128, 128, 64, 4, 2, 2, "16x16x32", sk=4), MI355X, c)["reduce_s"]
    assert r == pytest.approx((4 * M * N * 4 + M * N * 2) / (8000e9 * 0.5) + 2e-6)


def test_cdna4_hbm_floor():
    """A skinny launch cannot beat reading its operands at HBM rate."""
    op = cm.make_matmul_spec(16, 16384, 16384, dtype="f16")
    t = cm.predict_schedule(op, _cfg(32, 128, 64, 4, 1, 4, "16x16x32"), MI355X, _MFMA_ONLY)
    assert t["hbm_s"] == pytest.approx((16 * 16384 * 2 + 16384 * 16384 * 2 + 16 * 16384 * 2) / 8000e9)
    assert t["kernel_s"] >= t["hbm_s"]


def test_cdna4_detailed_score_is_ideal_over_predicted():
    op = cm.make_matmul_spec(1024, 768, 4096, ["bias_add", "row_layernorm"])
    cfg = cm.TuneConfig(128, 128, 64, 2, 4, warp_size=64, mfma="32x32x16", waves_m=2, waves_n=2)
    d = cm.score_formula_detailed(op, cfg, MI355X)
    assert d["score"] == pytest.approx(d["ideal_s"] / d["schedule"]["seconds"])
    assert d["score"] == pytest.approx(cm.score_formula(op, cfg, MI355X))
    assert not any(k.startswith("eff_") for k in d)
