"""tune()'s candidate order on the CPU, with the device timing replaced by a
function of the config: seeds (the measured database's pick) are measured
first, never twice, and a seed the descriptor does not offer for the shape is
skipped; the formula's top-1 is reported as such whatever the seeds are, and
the fastest measured candidate wins."""

import pytest

from icpp_tuning_amd.autotuner import MI355X, interface
from icpp_tuning_amd.autotuner.interface import rank_all, tune
from icpp_tuning_amd.kernels import gemm

SHAPE = dict(M=2048, N=1024, K=1024)


@pytest.fixture
def fake_device(monkeypatch):
    d = gemm.DESCRIPTOR
    monkeypatch.setattr(d, "make_inputs", lambda **shape: {})
    monkeypatch.setattr(d, "make_runner", lambda raw, inp, **shape: raw)
    # "time" of a config: the tile area decides, so the fastest config is known in advance
    monkeypatch.setattr(interface, "benchmark_ms",
                        lambda run, **kw: 1.0 / (run["block_M"] * run["block_N"]) + 1e-6 * run["num_stages"])
    return d


def test_seed_measured_first_and_can_win(fake_device):
    d = fake_device
    ranked = rank_all(d, MI355X, **SHAPE)
    offered = d.get_raw_configs(**SHAPE)
    # a seed far down the ranking with the largest tile, so it is the fastest
    seed = max(offered, key=lambda c: (c["block_M"] * c["block_N"], -c["num_stages"]))
    r = tune(d, MI355X, top_k=2, seed_configs=[seed], **SHAPE)
    assert r.candidates[0]["config"] == seed and r.candidates[0]["seed"]
    assert [c["config"] for c in r.candidates[1:]] == [e["raw_config"] for e in ranked
                                                      if e["raw_config"] != seed][:2]
    assert r.formula_top1 == ranked[0]["raw_config"]
    assert r.best_config == seed
    assert r.best_ms == min(c["ms"] for c in r.candidates)


def test_seed_equal_to_formula_top1_is_measured_once(fake_device):
    d = fake_device
    top1 = rank_all(d, MI355X, **SHAPE)[0]["raw_config"]
    r = tune(d, MI355X, top_k=3, seed_configs=[top1], **SHAPE)
    cfgs = [c["config"] for c in r.candidates]
    assert cfgs.count(top1) == 1 and len(cfgs) == 3
    assert r.formula_top1 == top1 and r.formula_top1_ms == r.candidates[0]["ms"]


def test_seed_not_offered_for_the_shape_is_skipped(fake_device):
    d = fake_device
    bad = dict(rank_all(d, MI355X, **SHAPE)[0]["raw_config"], block_K=48)  # no compiled instance
    r = tune(d, MI355X, top_k=2, seed_configs=[bad], **SHAPE)
    assert all(not c["seed"] for c in r.candidates) and len(r.candidates) == 2


def test_first_timing_discarded_and_two_fastest_retimed(monkeypatch, fake_device):
    """Timings drift down over the search (a clock ramping up): the first
    timing is thrown away, and the winner is decided on the mean of two
    timings of the two fastest, not on one lucky timing."""
    d = fake_device
    calls = []

    def drifting(run, **kw):
        calls.append(run)
        base = 1.0 / (run["block_M"] * run["block_N"])
        return base * (1.0 + 0.5 / len(calls))  # later calls read faster

    monkeypatch.setattr(interface, "benchmark_ms", drifting)
    r = tune(d, MI355X, top_k=4, **SHAPE)
    n = len(r.candidates)
    assert len(calls) == 1 + n + 2
    assert calls[0] == calls[1] == r.candidates[0]["config"]       # warm-up timing, then the real one
    retimed = [c for c in r.candidates if "ms_again" in c]
    assert len(retimed) == 2
    fastest_two = sorted(r.candidates, key=lambda c: c["ms"])[:2]
    assert {c["formatted"] for c in retimed} == {c["formatted"] for c in fastest_two}
    win = min(retimed, key=lambda c: c["ms"] + c["ms_again"])
    assert r.best_config == win["config"]
    assert r.best_ms == pytest.approx((win["ms"] + win["ms_again"]) / 2)


def test_failing_candidate_is_dropped_with_its_reason(monkeypatch, fake_device):
    """A candidate the library rejects (here: the runner raises the library's call
    error) is dropped from the ranking with the reason recorded, and the search
    goes on; when every candidate fails the search raises."""
    from icpp_tuning_amd._lib import IcppCallError

    d = fake_device
    ranked = rank_all(d, MI355X, **SHAPE)
    bad = ranked[1]["raw_config"]

    def runner(raw, inp, **shape):
        if raw == bad:
            raise IcppCallError("icpp_gemm", -3, "injected: LDS overflow")
        return raw

    monkeypatch.setattr(d, "make_runner", runner)
    r = tune(d, MI355X, top_k=4, **SHAPE)
    assert [f["config"] for f in r.failed] == [bad]
    assert "injected" in r.failed[0]["error"]
    assert bad not in [c["config"] for c in r.candidates] and len(r.candidates) == 3

    monkeypatch.setattr(d, "make_runner",
                        lambda raw, inp, **shape: (_ for _ in ()).throw(IcppCallError("icpp_gemm", -3, "no")))
    with pytest.raises(RuntimeError, match="every measured candidate failed"):
        tune(d, MI355X, top_k=2, **SHAPE)


def test_operand_error_is_not_taken_for_a_rejected_candidate(monkeypatch, fake_device):
    """An argument-check error (ValueError: wrong device, shape, contiguity) is a bug of
    the caller, not a property of one tile: it propagates from the first candidate
    instead of being recorded as a failed configuration."""
    d = fake_device
    calls = []

    def runner(raw, inp, **shape):
        calls.append(raw)
        raise ValueError("A must be contiguous")

    monkeypatch.setattr(d, "make_runner", runner)
    with pytest.raises(ValueError, match="contiguous"):
        tune(d, MI355X, top_k=4, **SHAPE)
    assert len(calls) == 1


def test_given_ranking_replaces_the_formula(fake_device):
    """tune(ranked=...) measures down the given order (e.g. AdaptiveTuner.rank)."""
    from icpp_tuning_amd.autotuner.perfdb import AdaptiveTuner

    d = fake_device
    order = AdaptiveTuner(d, hw=MI355X).rank(**SHAPE)
    assert {e["formatted"] for e in order} == {e["formatted"] for e in rank_all(d, MI355X, **SHAPE)}
    reverse = order[::-1]
    r = tune(d, MI355X, top_k=3, ranked=reverse, **SHAPE)
    assert [c["config"] for c in r.candidates] == [e["raw_config"] for e in reverse[:3]]
    assert r.formula_top1 == reverse[0]["raw_config"]
