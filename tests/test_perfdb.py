"""PerformanceDB / DecisionTable / AdaptiveTuner on the CPU (no device work).

The reference designs this stage without shipping code for it
(docs/autotuner_design.md:457-525), so the checks here pin what the design
fixes: a profiled shape returns its measured-best config, an unprofiled axis
value inside a group's range returns the config of the profiled point nearest
to it on a log scale (checked by brute force, not by the interval arithmetic),
shapes outside every profiled range fall back to the formula, and the database
survives a JSON round trip unchanged.
"""

import json
import math

import pytest

from icpp_tuning_amd.autotuner import MI355X, select_best
from icpp_tuning_amd.autotuner.perfdb import (AdaptiveTuner, DecisionTable, PerformanceDB, ProfileRecord,
                                              build_decision_table, build_sampling_plan, op_key)
from icpp_tuning_amd.kernels import conv2d, gemm_bias_act

DESC = gemm_bias_act.descriptor("gelu_tanh", "bf16")


def _cfgs(n):
    return [{"block_M": 64 * (i + 1), "block_N": 128, "block_K": 64, "num_stages": 2, "thread_num": 256}
            for i in range(n)]


def _records(points, group=(4096, 4096), extra_slower=True):
    """points: {M: best config}; every shape also gets a slower record of another config."""
    A = _cfgs(8)
    recs = []
    for m, cfg in points.items():
        recs.append(ProfileRecord({"M": m, "N": group[0], "K": group[1]}, cfg, 1.0))
        if extra_slower:
            other = A[(A.index(cfg) + 1) % len(A)]
            recs.append(ProfileRecord({"M": m, "N": group[0], "K": group[1]}, other, 2.0))
    return recs


def test_profiled_points_return_measured_best():
    A = _cfgs(8)
    pts = {64: A[0], 256: A[0], 1024: A[1], 4096: A[2], 8192: A[1]}
    t = build_decision_table(_records(pts))
    for m, cfg in pts.items():
        assert t.lookup({"M": m, "N": 4096, "K": 4096}) == cfg


def test_slowest_record_never_wins_whatever_order():
    A = _cfgs(3)
    shape = {"M": 512, "N": 1024, "K": 1024}
    recs = [ProfileRecord(shape, A[0], 3.0), ProfileRecord(shape, A[1], 1.5), ProfileRecord(shape, A[2], 2.0)]
    for order in (recs, recs[::-1], [recs[1], recs[0], recs[2]]):
        assert build_decision_table(order).lookup(shape) == A[1]


def test_between_points_is_log_nearest_neighbour():
    A = _cfgs(8)
    pts = {16: A[3], 96: A[0], 256: A[4], 1000: A[1], 3000: A[2], 8192: A[5]}
    t = build_decision_table(_records(pts))
    ms = sorted(pts)
    for m in range(16, 8193, 7):
        # brute force: the profiled M with the smallest |log m - log p| (ties go to the larger point)
        nearest = min(ms, key=lambda p: (abs(math.log(m) - math.log(p)), -p))
        assert t.lookup({"M": m, "N": 4096, "K": 4096}) == pts[nearest], m


def test_misses_outside_range_and_unknown_groups():
    A = _cfgs(2)
    t = build_decision_table(_records({128: A[0], 2048: A[1]}))
    assert t.lookup({"M": 127, "N": 4096, "K": 4096}) is None
    assert t.lookup({"M": 2049, "N": 4096, "K": 4096}) is None
    assert t.lookup({"M": 2048, "N": 4096, "K": 4096}) == A[1]      # closed at the top
    assert t.lookup({"M": 512, "N": 4096, "K": 1024}) is None        # group never profiled
    assert t.lookup({"N": 4096, "K": 4096}) is None                   # no axis value


def test_equal_neighbours_merge_into_one_interval():
    A = _cfgs(2)
    t = build_decision_table(_records({64: A[0], 128: A[0], 256: A[0], 512: A[1]}))
    (intervals,) = t.groups.values()
    assert [c for _, _, c in intervals] == [A[0], A[1]]
    assert intervals[0][0] == 64 and intervals[-1][1] == 512


def test_groups_are_independent():
    A = _cfgs(4)
    recs = _records({256: A[0], 4096: A[1]}, group=(4096, 4096)) + _records({256: A[2], 4096: A[3]}, group=(768, 4096))
    t = build_decision_table(recs)
    assert t.lookup({"M": 256, "N": 4096, "K": 4096}) == A[0]
    assert t.lookup({"M": 256, "N": 768, "K": 4096}) == A[2]
    assert t.lookup({"M": 4096, "N": 768, "K": 4096}) == A[3]


def test_conv_axis_is_batch():
    geo = dict(C=64, H=56, W=56, OC=64, KH=3, KW=3, stride=1, padding=1)
    A = _cfgs(2)
    recs = [ProfileRecord(dict(geo, N=8), A[0], 1.0), ProfileRecord(dict(geo, N=64), A[1], 1.0)]
    t = build_decision_table(recs)
    assert t.axis == "N"
    assert t.lookup(dict(geo, N=9)) == A[0] and t.lookup(dict(geo, N=60)) == A[1]
    assert t.lookup(dict(geo, N=32, C=128)) is None


def test_json_round_trip(tmp_path):
    A = _cfgs(8)
    db = PerformanceDB(op=op_key(DESC), hw=MI355X.name, records=_records({64: A[0], 1024: A[1], 8192: A[2]}),
                       created=1.5)
    db.rebuild()
    path = tmp_path / "db.json"
    db.save(path)
    json.loads(path.read_text())                     # plain JSON
    db2 = PerformanceDB.load(path)
    assert db2.op == db.op and db2.hw == db.hw and db2.created == db.created
    assert [r.as_dict() for r in db2.records] == [r.as_dict() for r in db.records]
    assert db2.table.as_dict() == db.table.as_dict()
    for m in (64, 100, 500, 1024, 3000, 8192, 9000):
        s = {"M": m, "N": 4096, "K": 4096}
        assert db2.table.lookup(s) == db.table.lookup(s)


def test_empty_db_is_all_misses():
    t = build_decision_table([])
    assert t.lookup({"M": 64, "N": 64, "K": 64}) is None
    assert DecisionTable.from_dict(t.as_dict()).groups == {}


def test_adaptive_tuner_levels():
    shape = {"M": 512, "N": 4096, "K": 4096}
    pool = DESC.get_raw_configs(**shape)
    formula, score = select_best(DESC, MI355X, **shape)
    # a table entry that is not the formula's choice, so that the level is visible in the config
    pick = next(c for c in pool if c != formula)
    db = PerformanceDB(op=op_key(DESC), hw=MI355X.name,
                       records=[ProfileRecord(shape, pick, 0.1), ProfileRecord(shape, formula, 0.2)])
    db.rebuild()
    tuner = AdaptiveTuner(DESC, db, MI355X)
    r = tuner.select(**shape)
    assert (r.level, r.config) == ("table", pick)
    miss = tuner.select(M=1 << 15, N=4096, K=4096)
    assert miss.level == "formula"
    assert miss.config == select_best(DESC, MI355X, M=1 << 15, N=4096, K=4096)[0]
    # no DB, a DB of another op or GPU: formula only
    for t in (AdaptiveTuner(DESC, None, MI355X),
              AdaptiveTuner(DESC, PerformanceDB(op_key(DESC), MI355X.name), MI355X),
              AdaptiveTuner(DESC, PerformanceDB("other_op", MI355X.name, db.records, db.table), MI355X),
              AdaptiveTuner(DESC, PerformanceDB(op_key(DESC), "other GPU", db.records, db.table), MI355X)):
        r = t.select(**shape)
        assert (r.level, r.config, r.score) == ("formula", formula, score)


def test_adaptive_tuner_rejects_config_outside_compiled_set():
    shape = {"M": 512, "N": 4096, "K": 4096}
    bogus = {"block_M": 48, "block_N": 48, "block_K": 48, "num_stages": 7, "thread_num": 192}
    db = PerformanceDB(op=op_key(DESC), hw=MI355X.name, records=[ProfileRecord(shape, bogus, 0.01)])
    db.rebuild()
    r = AdaptiveTuner(DESC, db, MI355X).select(**shape)
    assert r.level == "formula" and r.config != bogus
    with pytest.raises(KeyError):
        AdaptiveTuner(DESC, db, MI355X).precompile()


def test_precompile_resolves_instances():
    shape = {"M": 512, "N": 4096, "K": 4096}
    pool = DESC.get_raw_configs(**shape)
    db = PerformanceDB(op=op_key(DESC), hw=MI355X.name,
                       records=[ProfileRecord(dict(shape, M=m), pool[i], 1.0) for i, m in enumerate((64, 512, 4096))])
    db.rebuild()
    idx = AdaptiveTuner(DESC, db, MI355X).precompile()
    assert len(idx) == len({DESC.format_config(pool[i]) for i in range(3)})
    assert all(DESC.instance_index(pool[i]) == idx[DESC.format_config(pool[i])] for i in range(3))


def test_sampling_plan_wave_strata():
    nk = [(4096, 4096), (768, 4096)]
    plan = build_sampling_plan("gemm", MI355X, m_range=(16, 16384), nk=nk)
    for N, K in nk:
        ms = [s["M"] for s in plan if (s["N"], s["K"]) == (N, K)]
        assert ms == sorted(set(ms)) and ms[0] == 16 and ms[-1] == 16384
        tiles_n = -(-N // 128)
        small = [m for m in ms[:-1] if m < 128 * max(1, round(MI355X.num_sm / 8 / tiles_n))]
        # below the 1/8-wave stratum: the powers of two from 16
        assert small == [2 ** e for e in range(4, 20) if 2 ** e in small] and (not small or small[0] == 16)
        waves = {(-(-m // 128)) * tiles_n / MI355X.num_sm for m in ms[1:-1] if m not in small}
        # every other interior point sits within one 128-row tile of a power-of-two wave count
        for w in waves:
            assert abs(math.log2(w) - round(math.log2(w))) < 0.5
        # and every power-of-two wave count that fits the range is present
        lo_w = (-(-16 // 128)) * tiles_n / MI355X.num_sm
        hi_w = (-(-16384 // 128)) * tiles_n / MI355X.num_sm
        want = {2.0 ** e for e in range(-3, 12) if lo_w <= 2.0 ** e <= hi_w}
        got = {2.0 ** round(math.log2((-(-m // 128)) * tiles_n / MI355X.num_sm)) for m in ms}
        assert want <= got, (N, want - got)


def test_sampling_plan_conv():
    geos = [dict(C=64, H=56, W=56, OC=64, KH=3, KW=3, stride=1, padding=1),
            dict(C=512, H=7, W=7, OC=512, KH=3, KW=3, stride=1, padding=1)]
    plan = build_sampling_plan("conv2d", MI355X, conv=geos, batches=(1, 8, 32))
    assert len(plan) == 6 and {p["N"] for p in plan} == {1, 8, 32}
    assert all(conv2d.DESCRIPTOR.get_raw_configs(**p) for p in plan)


SHIPPED = ["gemm_splitk_f16", "gemm_bias_gelu_tanh_bf16", "gemm_bias_relu_bf16", "gemm_bias_silu_bf16", "gemm_bias_relu_f16",
           "gemm_bias_layernorm_f16", "fp8_gemm_bias_silu_fp8",
           "conv2d_f16", "conv2d_relu_f16", "conv2d_bn_f16", "conv2d_bn_relu_f16", "conv_bn_add_relu_f16",
           "gemm_bias_gelu_erf_f16"]


def _shipped_descriptors():
    from icpp_tuning_amd.autotuner.perfdb import _descriptors

    return {op_key(d): d for d in _descriptors().values()}


@pytest.mark.parametrize("key", SHIPPED)
def test_shipped_database(key):
    """The databases measured on MI355X that ship with the package: they load,
    belong to their op and GPU, cover the offline plan exhaustively (every
    compiled config at every planned shape), and their table returns, for
    every profiled shape, the fastest record measured for it."""
    from icpp_tuning_amd.autotuner.perfdb import default_plan, shipped_path

    desc = _shipped_descriptors()[key]
    path = shipped_path(key, MI355X)
    db = PerformanceDB.load(path)
    assert db.op == key and db.hw == MI355X.name
    plan = default_plan(desc.name, MI355X)
    by_shape = {}
    for r in db.records:
        by_shape.setdefault(json.dumps(r.shape, sort_keys=True), []).append(r)
    assert set(by_shape) == {json.dumps(s, sort_keys=True) for s in plan}
    for s in plan:
        recs = by_shape[json.dumps(s, sort_keys=True)]
        # every config offered for the shape is measured (a database profiled before a
        # config stopped being offered may hold more), and the table's pick is offered
        offered = {json.dumps(c, sort_keys=True) for c in desc.get_raw_configs(**s)}
        recorded = {json.dumps(r.config, sort_keys=True) for r in recs}
        assert offered <= recorded, s
        assert all(r.ms > 0 and math.isfinite(r.ms) for r in recs)
        assert db.table.lookup(s) == min(recs, key=lambda r: r.ms).config, s
        assert json.dumps(db.table.lookup(s), sort_keys=True) in offered, s
    # the stored table is what the records rebuild to, and names compiled instances only
    stored = db.table.as_dict()
    db.rebuild()
    assert db.table.as_dict() == stored
    assert AdaptiveTuner(desc, db, MI355X).precompile()


def test_shipped_database_is_the_default():
    desc = _shipped_descriptors()["gemm_bias_gelu_tanh_bf16"]
    t = AdaptiveTuner(desc, hw=MI355X)
    assert t.db is not None and t.select(M=4096, N=4096, K=4096).level == "table"
    # another dtype of the same op name has no database: formula
    f16 = gemm_bias_act.descriptor("gelu_tanh", "f16")
    assert AdaptiveTuner(f16, hw=MI355X).select(M=4096, N=4096, K=4096).level == "formula"
