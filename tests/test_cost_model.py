"""Cost model: A100 reference-mode parity against the reference's published
scores, then CDNA4-mode properties."""

import json
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


def test_reference_mode_ignores_cdna_terms():
    op = cm.make_matmul_spec(256, 256, 256)
    cfg = cm.TuneConfig(64, 128, 32, 2, 4)
    proj = cm.project_config(op, cfg, A100)
    assert cm.eff_mfma(op, cfg, proj, A100) == 1.0
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


def test_cdna4_mfma_factor_prefers_32x32_issue_rate():
    op = cm.make_matmul_spec(4096, 4096, 4096, dtype="bf16")
    a = cm.TuneConfig(256, 256, 64, 2, 4, warp_size=64, mfma="32x32x16", waves_m=2, waves_n=2)
    b = cm.TuneConfig(256, 256, 64, 2, 4, warp_size=64, mfma="16x16x32", waves_m=2, waves_n=2)
    pa, pb = cm.project_config(op, a, MI355X), cm.project_config(op, b, MI355X)
    assert cm.eff_mfma(op, a, pa, MI355X) > cm.eff_mfma(op, b, pb, MI355X)


def test_detailed_score_is_product_of_factors():
    op = cm.make_matmul_spec(1024, 768, 4096, ["bias_add", "row_layernorm"])
    cfg = cm.TuneConfig(128, 128, 64, 2, 4, warp_size=64, mfma="32x32x16", waves_m=2, waves_n=2)
    d = cm.score_formula_detailed(op, cfg, MI355X)
    prod = 1.0
    for k, v in d.items():
        if k.startswith("eff_"):
            prod *= v
    assert d["score"] == pytest.approx(prod)
    assert d["score"] == pytest.approx(cm.score_formula(op, cfg, MI355X))
