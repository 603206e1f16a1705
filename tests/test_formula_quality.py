"""Cold-start quality of the CDNA4 schedule model on measured data.

The shipped offline databases hold the time of every compiled config at every
profiled shape, measured on MI355X.  At each such shape the formula's top-1
(what ``build_kernel(config=None)`` falls back to outside the databases'
ranges) is scored as fastest_ms / pick_ms.  The model's fitted constants came
from these same shapes, so this is an in-sample floor that catches regressions
of the model; the held-out shapes are scored by ``perfdb --rescore``.
"""

import json
import statistics

import pytest

from icpp_tuning_amd.autotuner import MI355X, select_best
from icpp_tuning_amd.autotuner.perfdb import PerformanceDB, _descriptors, op_key, shipped_path

DESCS = {op_key(d): d for d in _descriptors().values()}


@pytest.mark.parametrize("key", sorted(DESCS))
def test_formula_top1_close_to_measured_best(key):
    desc = DESCS[key]
    db = PerformanceDB.load(shipped_path(key, MI355X))
    by_shape = {}
    for r in db.records:
        by_shape.setdefault(json.dumps(r.shape, sort_keys=True), {})[desc.format_config(r.config)] = r.ms
    ratios = []
    for shape_key, ms in by_shape.items():
        pick = desc.format_config(select_best(desc, MI355X, **json.loads(shape_key))[0])
        ratios.append(min(ms.values()) / ms[pick])
    assert statistics.mean(ratios) >= 0.9, (key, statistics.mean(ratios))
    assert min(ratios) >= 0.6, (key, min(ratios))


def test_rescore_repicks_the_formula_against_stored_times():
    """`perfdb --rescore`: the formula column is re-picked with the current model
    and priced from the row's own measurements; table picks stay, a table miss
    takes the new formula pick."""
    from icpp_tuning_amd.autotuner.perfdb import rescore

    desc = DESCS["gemm_bias_gelu_tanh_bf16"]
    shape = {"M": 1000, "N": 4096, "K": 4096}
    names = [desc.format_config(r) for r in desc.get_raw_configs(**shape)]
    ms = {n: 1.0 + i for i, n in enumerate(names)}
    best = desc.format_config(select_best(desc, MI355X, **shape)[0])
    rows = [{"shape": shape, "oracle": names[0], "oracle_ms": 1.0, "level": level, "pick": names[1],
             "pick_ms": 2.0, "formula": names[2], "formula_ms": 3.0, "pruned_best_ms": 1.0, "ms": ms}
            for level in ("table", "formula")]
    rep = rescore(desc, {"rows": rows}, MI355X)
    t, f = rep["rows"]
    assert t["formula"] == f["formula"] == best and t["formula_ms"] == ms[best]
    assert t["pick"] == names[1] and f["pick"] == best and f["pick_ms"] == ms[best]
    assert rep["formula"]["perf_ratio_mean"] == pytest.approx(1.0 / ms[best])


def test_layernorm_second_pass_is_priced():
    """Two-pass and GEMM-then-LN launch a pass that reads and writes Y once more;
    the one-launch row strategy does not; the co-resident one pays ~4 us of statistics
    exchange per launch, one launch per chunk of row blocks the CUs hold (256 // tiles_n
    row blocks per launch)."""
    from icpp_tuning_amd.autotuner import rank_all
    from icpp_tuning_amd.autotuner.cost_model import CDNA4_CONSTANTS as C

    desc = DESCS["gemm_bias_layernorm_f16"]
    M, N, K = 4096, 768, 768
    ranked = rank_all(desc, MI355X, detailed=True, M=M, N=N, K=K)
    seen = set()
    for e in ranked:
        strategy = e["raw_config"]["strategy"]
        seen.add(strategy)
        want = 0.0 if strategy == "row" else 2 * M * N * 2 / (8000e9 * C.hbm_efficiency) + C.launch_overhead_s
        if strategy == "coresident":
            raw = e["raw_config"]
            per_launch = 256 // -(-N // raw["block_N"])
            want = 4e-6 * -(-(-(-M // raw["block_M"])) // per_launch)
        assert e["detail"]["extra_s"] == pytest.approx(want), e["formatted"]
        if strategy == "gemm_ln":      # a plain GEMM + bias launch: no statistics epilogue
            assert [p.name for p in desc.make_op_spec(e["raw_config"], M=M, N=N, K=K).epilogue] == ["bias_add"]
    assert seen == {"row", "two_pass", "gemm_ln", "coresident"}


def test_report_topk_is_the_best_measured_of_the_ranking():
    """`formula_topk[k]`: the fastest measured config among the formula's first k
    against the oracle, i.e. what tune(top_k=k) without seeds finds."""
    from icpp_tuning_amd.autotuner import rank_all
    from icpp_tuning_amd.autotuner.perfdb import TOPK, rescore

    desc = DESCS["gemm_splitk_f16"]
    shape = {"M": 500, "N": 2304, "K": 768}
    ranked = [e["formatted"] for e in rank_all(desc, MI355X, **shape)]
    ms = {n: 10.0 for n in (desc.format_config(r) for r in desc.get_raw_configs(**shape))}
    ms[ranked[0]], ms[ranked[2]], ms[ranked[7]] = 4.0, 2.0, 1.0      # oracle 1.0 at rank 8
    row = {"shape": shape, "oracle": ranked[7], "oracle_ms": 1.0, "level": "table", "pick": ranked[7],
           "pick_ms": 1.0, "pruned_best_ms": 1.0, "ms": ms}
    rep = rescore(desc, {"rows": [row]}, MI355X)
    assert rep["rows"][0]["formula_ranking"] == ranked[:max(TOPK)]
    got = {k: v["perf_ratio_mean"] for k, v in rep["formula_topk"].items()}
    assert got == {"1": 0.25, "2": 0.25, "4": 0.5, "8": 1.0}
