"""The residual level of the online select (autotuner/residual.py), on the CPU.

The boosted trees are pinned by cases whose answer is fixed by the
construction (a one-split tree reproduces two group means exactly; boosting
drives the training error of a step + linear target towards zero; the JSON
form predicts what the fitted model predicts).  The level order of
`AdaptiveTuner` and the shipped databases' stored models are checked against
the shipped measurements.
"""

import json

import numpy as np
import pytest

from icpp_tuning_amd.autotuner import MI355X
from icpp_tuning_amd.autotuner.perfdb import (AdaptiveTuner, PerformanceDB, _descriptors, _group_key, op_key,
                                              shipped_path)
from icpp_tuning_amd.autotuner.residual import (FEATURES, BoostedTrees, ResidualModel, cross_validate,
                                                fit_boosted_trees, fit_residual, schedule_features)

DESCS = {op_key(d): d for d in _descriptors().values()}


def test_one_split_tree_is_the_two_group_means():
    rng = np.random.default_rng(0)
    x0 = np.repeat([0.0, 1.0], 40)
    X = np.stack([x0, rng.normal(size=80)], axis=1)           # feature 1 is noise
    y = np.where(x0 > 0.5, 3.0, -1.0) + rng.normal(scale=0.1, size=80)
    m = fit_boosted_trees(X, y, n_trees=1, depth=1, learning_rate=1.0, min_leaf=1, l2=0.0)
    root = m.trees[0][0]
    assert int(root[0]) == 0 and root[1] == pytest.approx(0.5)
    pred = m.predict(X)
    assert pred[:40] == pytest.approx(np.full(40, y[:40].mean()))
    assert pred[40:] == pytest.approx(np.full(40, y[40:].mean()))


def test_boosting_fits_step_plus_linear():
    """x0 takes 20 values, so every midpoint between them is a split candidate
    and the step is representable exactly; the linear part is resolved to the
    32-bin histogram of x1 (error ~ (0.5 / 31)^2 / 12)."""
    rng = np.random.default_rng(1)
    X = rng.uniform(size=(2000, 3))
    X[:, 0] = rng.integers(0, 20, size=2000) / 20.0
    y = 2.0 * (X[:, 0] > 0.32) + 0.5 * X[:, 1]                # X[:, 2] is irrelevant
    m = fit_boosted_trees(X, y, n_trees=100, depth=3, learning_rate=0.2, min_leaf=10)
    err = np.mean((m.predict(X) - y) ** 2)
    assert err < 0.01 * np.var(y)
    root = m.trees[0][0]                                       # the largest effect is split first, at the step
    assert int(root[0]) == 0 and 0.30 < root[1] < 0.35
    shuffled = X.copy()
    shuffled[:, 2] = rng.permutation(shuffled[:, 2])
    assert np.sqrt(np.mean((m.predict(shuffled) - m.predict(X)) ** 2)) < 0.05


def test_json_form_predicts_the_same():
    rng = np.random.default_rng(2)
    X = rng.normal(size=(500, 4))
    y = np.sin(X[:, 0]) + X[:, 1] * X[:, 2]
    m = fit_boosted_trees(X, y, n_trees=30, depth=4)
    m2 = BoostedTrees.from_dict(json.loads(json.dumps(m.as_dict())))
    Xt = rng.normal(size=(200, 4))
    assert m2.predict(Xt) == pytest.approx(m.predict(Xt), abs=1e-5)


def test_model_with_other_features_is_ignored():
    m = ResidualModel(BoostedTrees(trees=[[[-1.0, 0.0, -1.0, -1.0, 0.5]]]))
    d = m.as_dict()
    assert ResidualModel.from_dict(d) is not None
    assert ResidualModel.from_dict(dict(d, features=list(FEATURES[:-1]))) is None


def test_feature_row_matches_the_schedule_model():
    from icpp_tuning_amd.autotuner import cost_model as cm

    desc = DESCS["gemm_bias_layernorm_f16"]
    shape = {"M": 4096, "N": 768, "K": 768}
    for raw in desc.get_raw_configs(**shape)[:6]:
        row, t = schedule_features(desc, raw, MI355X, shape)
        sc = cm.predict_schedule(desc.make_op_spec(raw_config=raw, **shape), desc.raw_config_to_tune_config(raw),
                                 MI355X)
        assert len(row) == len(FEATURES)
        assert t == pytest.approx(sc["seconds"] + desc.extra_seconds(raw, MI355X, **shape))
        assert row[0] == pytest.approx(np.log(t))


def test_levels_table_then_residual_then_formula():
    desc = DESCS["gemm_bias_gelu_tanh_bf16"]
    t = AdaptiveTuner(desc, hw=MI355X)
    assert t.residual is not None
    assert t.select(M=3000, N=4096, K=4096).level == "table"
    unseen = {"M": 3000, "N": 2048, "K": 2560}                # an (N, K) group the database never saw
    r = t.select(**unseen)
    assert r.level == "residual" and r.score > 0
    pruned = desc.prune(desc.get_raw_configs(**unseen), MI355X, **unseen)
    assert r.config in pruned
    lt = t.residual.log_time(desc, pruned, MI355X, unseen)
    assert r.config == pruned[int(lt.argmin())]
    assert AdaptiveTuner(desc, None, MI355X).select(**unseen).level == "formula"


@pytest.mark.parametrize("key", ["gemm_bias_gelu_erf_f16", "conv2d_f16"])
def test_shipped_residual_is_the_fit_of_its_records(key):
    """The stored model is what fitting the database's own records gives
    (the fit is deterministic), so it can be rebuilt from the JSON alone."""
    db = PerformanceDB.load(shipped_path(key, MI355X))
    assert db.residual is not None
    assert fit_residual(DESCS[key], db.records, MI355X).as_dict() == db.residual


def test_cross_validate_reports_every_group():
    key = "gemm_bias_gelu_erf_f16"
    db = PerformanceDB.load(shipped_path(key, MI355X))
    rows = cross_validate(DESCS[key], db.records, MI355X, lambda s: _group_key(s, db.table.axis), n_trees=20)
    groups = {_group_key(r.shape, db.table.axis) for r in db.records}
    assert {r["group"] for r in rows} == groups
    assert sum(r["shapes"] for r in rows) == len({json.dumps(r.shape, sort_keys=True) for r in db.records})
    for r in rows:
        for k in ("formula_mean", "formula_min", "residual_mean", "residual_min"):
            assert 0.0 < r[k] <= 1.0


@pytest.mark.parametrize("key", sorted(DESCS))
def test_unseen_plan_misses_the_table(key):
    """`perfdb --eval-unseen` measures the residual level: every shape of its
    plan lies in a group the shipped database never profiled."""
    from icpp_tuning_amd.autotuner.perfdb import unseen_plan

    desc = DESCS[key]
    db = PerformanceDB.load(shipped_path(key, MI355X))
    profiled = {_group_key(r.shape, db.table.axis) for r in db.records}
    t = AdaptiveTuner(desc, db, MI355X)
    for shape in unseen_plan(desc.name):
        assert _group_key(shape, db.table.axis) not in profiled
        assert desc.get_raw_configs(**shape)
        assert t.select(**shape).level == "residual"


def test_select_is_memoised_per_shape():
    desc = DESCS["gemm_bias_gelu_tanh_bf16"]
    t = AdaptiveTuner(desc, hw=MI355X)
    unseen = {"M": 3000, "N": 2048, "K": 2560}
    a = t.select(**unseen)
    a.config["block_M"] = -1                      # a caller's change does not reach the memo
    b = t.select(**unseen)
    assert b.level == "residual" and b.config["block_M"] > 0
    assert b.seconds < 1e-3
    t.MEMO_MAX = 1
    t.select(M=3001, N=2048, K=2560)
    assert len(t._memo) == 1


def test_cli_fit_and_cross_validate(tmp_path):
    """`perfdb --fit-residual` stores the fit in the database at --out;
    `--cv-residual` writes one report row per group."""
    from icpp_tuning_amd.autotuner.perfdb import main

    key = "gemm_bias_gelu_erf_f16"
    path = tmp_path / "db.json"
    db = PerformanceDB.load(shipped_path(key, MI355X))
    db.residual = None
    db.save(path)
    assert main(["--op", "gemm_bias_gelu_erf", "--out", str(path), "--fit-residual"]) == 0
    fitted = PerformanceDB.load(path)
    assert fitted.residual == PerformanceDB.load(shipped_path(key, MI355X)).residual
    assert [r.as_dict() for r in fitted.records] == [r.as_dict() for r in db.records]
    report = tmp_path / "cv.json"
    assert main(["--op", "gemm_bias_gelu_erf", "--out", str(path), "--cv-residual", str(report)]) == 0
    rep = json.loads(report.read_text())
    assert rep["op"] == key and len(rep["groups"]) == len({_group_key(r.shape, db.table.axis) for r in db.records})
