"""Kernel descriptor API and the select / rank / tune loop.

Mirrors the reference's plugin interface (kernel/autotuner/interface.py):
``TileLangKernelBase`` with ``name``, ``make_op_spec``, ``get_raw_configs``,
``raw_config_to_tune_config``, ``score_adjustment``, ``format_config``, and the
generic ``select_best`` (:136-178) / ``rank_all`` (:181-241).  Descriptors
written for the reference run unchanged.

Additions for the gfx950 build:
  * ``prune(configs, hw, **shape)`` hook, applied before scoring.  The default
    keeps every config (reference behaviour); the MI355X descriptors reject
    tiles that overflow LDS or VGPRs or under-fill the CUs for the shape.
  * ``tune(...)``: prune + rank, resolve ("compile") the top-k, benchmark them
    on the device and return the measured best, with the wall-clock split the
    reference reports as time-to-best.
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple, Union

from .._lib import IcppCallError
from .cost_model import OpSpec, TuneConfig, ideal_seconds, score_formula, score_formula_detailed
from .gpu_spec import GPUSpec, get_gpu_spec


class TileLangKernelBase:
    """Descriptor base class (reference interface.py:50-128).

    Subclasses must override ``name``, ``make_op_spec`` and ``get_raw_configs``.
    """

    @property
    def name(self) -> str:
        raise NotImplementedError

    def make_op_spec(self, raw_config: Optional[Dict[str, Any]] = None, **shape_kwargs: Any) -> OpSpec:
        raise NotImplementedError

    def get_raw_configs(self, **shape_kwargs: Any) -> List[Dict[str, Any]]:
        raise NotImplementedError

    # -- defaults ---------------------------------------------------------------
    def raw_config_to_tune_config(self, raw: Dict[str, Any]) -> TuneConfig:
        """``thread_num`` -> warps of 32 lanes (reference :92-103)."""
        return TuneConfig(
            block_M=raw["block_M"], block_N=raw["block_N"], block_K=raw["block_K"],
            num_stages=raw["num_stages"], num_warps=raw["thread_num"] // 32,
        )

    def score_adjustment(self, raw: Dict[str, Any], base_score: float, **shape_kwargs: Any) -> float:
        return base_score

    def schedule_factor(self, raw: Dict[str, Any]) -> float:
        """Relative mainloop efficiency of the config's schedule (1 for the default one)."""
        return 1.0

    def extra_seconds(self, raw: Dict[str, Any], hw: GPUSpec, **shape_kwargs: Any) -> float:
        """Time of launches the config adds beside the scored kernel (e.g. a
        separate normalisation pass over the output).  Used by the CDNA4
        schedule model only, whose score is a time ratio; 0 by default."""
        return 0.0

    def format_config(self, raw: Dict[str, Any]) -> str:
        """``BM{}_BN{}_BK{}[_SK{}]_S{}_T{}`` (reference :117-128), plus the MFMA
        wave grid / shape suffix when the config carries one."""
        parts = [f"BM{raw['block_M']}", f"BN{raw['block_N']}", f"BK{raw['block_K']}"]
        if "split_k" in raw:
            parts.append(f"SK{raw['split_k']}")
        parts.append(f"S{raw['num_stages']}")
        parts.append(f"T{raw['thread_num']}")
        if "waves_m" in raw and "waves_n" in raw:
            parts.append(f"W{raw['waves_m']}x{raw['waves_n']}")
        if "mfma" in raw:
            parts.append(f"M{raw['mfma'].split('x')[0]}")
        if raw.get("sched"):
            parts.append(str(raw["sched"]).upper())
        return "_".join(parts)

    def prune(self, raw_configs: List[Dict[str, Any]], hw: GPUSpec, **shape_kwargs: Any) -> List[Dict[str, Any]]:
        return raw_configs

    # -- tune() hooks (device descriptors implement these) ---------------------
    def make_inputs(self, **shape_kwargs: Any) -> Dict[str, Any]:
        raise NotImplementedError(f"{self.name} cannot be benchmarked")

    def make_runner(self, raw: Dict[str, Any], inputs: Dict[str, Any], **shape_kwargs: Any) -> Callable[[], Any]:
        raise NotImplementedError(f"{self.name} cannot be benchmarked")

    def flops(self, **shape_kwargs: Any) -> float:
        op = self.make_op_spec(**shape_kwargs)
        return float(op.mainloop.mainloop_flops)


def _score(descriptor: TileLangKernelBase, raw, hw, detailed: bool, shape):
    op = descriptor.make_op_spec(raw_config=raw, **shape)
    cfg = descriptor.raw_config_to_tune_config(raw)
    if detailed:
        detail = score_formula_detailed(op, cfg, hw)
        base = detail["score"]
    else:
        base, detail = score_formula(op, cfg, hw), None
    if hw.has_mfma_model:
        extra = descriptor.extra_seconds(raw, hw, **shape)
        if extra > 0.0 and base > 0.0:
            ideal = ideal_seconds(op, cfg, hw)
            base = ideal / (ideal / base + extra)
        if detail is not None:
            detail["extra_s"] = extra
    return descriptor.score_adjustment(raw, base * descriptor.schedule_factor(raw), **shape), detail


def select_best(descriptor: TileLangKernelBase, hw: Optional[GPUSpec] = None,
                **shape_kwargs: Any) -> Tuple[Dict[str, Any], float]:
    """Highest-scoring raw config (strict ``>``: the first of equal scores wins)."""
    if hw is None:
        hw = get_gpu_spec()
    configs = descriptor.prune(descriptor.get_raw_configs(**shape_kwargs), hw, **shape_kwargs)
    best, best_score = None, -1.0
    for raw in configs:
        s, _ = _score(descriptor, raw, hw, False, shape_kwargs)
        if s > best_score:
            best, best_score = raw, s
    if best is None:
        raise RuntimeError(f"No configs generated for {descriptor.name} with {shape_kwargs}")
    return best, best_score


def rank_all(descriptor: TileLangKernelBase, hw: Optional[GPUSpec] = None, detailed: bool = False,
             prune: bool = True, **shape_kwargs: Any) -> List[Dict[str, Any]]:
    """Every (pruned, unless prune=False) config with its score, best first (stable sort)."""
    if hw is None:
        hw = get_gpu_spec()
    configs = descriptor.get_raw_configs(**shape_kwargs)
    if prune:
        configs = descriptor.prune(configs, hw, **shape_kwargs)
    out = []
    for raw in configs:
        s, detail = _score(descriptor, raw, hw, detailed, shape_kwargs)
        e = {"raw_config": raw, "score": s, "formatted": descriptor.format_config(raw)}
        if detailed:
            e["detail"] = detail
        out.append(e)
    out.sort(key=lambda e: e["score"], reverse=True)
    return out


@dataclass
class TuneResult:
    best_config: Dict[str, Any]
    best_ms: float
    best_tflops: float
    formula_top1: Dict[str, Any]        # the ranking's first config: the formula's, unless `ranked` was given
    formula_top1_ms: float
    candidates: List[Dict[str, Any]] = field(default_factory=list)
    prune_rank_s: float = 0.0
    compile_s: float = 0.0
    bench_s: float = 0.0
    time_to_best_s: float = 0.0
    n_configs: int = 0
    n_pruned: int = 0
    inputs_s: float = 0.0   # synthetic input generation (excluded from time_to_best)
    failed: List[Dict[str, Any]] = field(default_factory=list)  # candidates dropped, with the reason

    def as_dict(self) -> Dict[str, Any]:
        return dict(self.__dict__)


def benchmark_ms(fn, warmup: int = 3, reps: int = 10, batches: int = 3, graph: bool = True) -> float:
    """Per-launch device time in ms: HIP events around ``reps`` back-to-back
    launches (the way the reference times conv2d, conv2d.py:171-183), median
    over ``batches``.

    With ``graph`` the ``reps`` launches are captured once into a HIP graph and
    the graph is replayed between the events, so the figure is the device time
    of the kernels themselves: issuing a launch from Python (argument checks +
    the ctypes call) costs ~10 us, more than a small kernel runs, and an eager
    loop would time the host instead.  Capture failures fall back to the eager
    loop.

    ``fn`` is a callable, or a list of callables used round-robin (distinct
    input copies, so that a working set larger than the caches stays cold)."""
    import torch

    fns = list(fn) if isinstance(fn, (list, tuple)) else [fn]
    for i in range(max(warmup, len(fns))):
        fns[i % len(fns)]()
    torch.cuda.synchronize()

    def launch_all():
        for i in range(reps):
            fns[i % len(fns)]()

    run = launch_all
    if graph:
        try:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                launch_all()
            g.replay()
            torch.cuda.synchronize()
            run = g.replay
        except Exception:  # noqa: BLE001 - capture unsupported here: time the eager loop
            torch.cuda.synchronize()
            run = launch_all
    times = []
    for _ in range(batches):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        run()
        e.record()
        e.synchronize()
        times.append(s.elapsed_time(e) / reps)
    times.sort()
    return times[len(times) // 2]


def input_bytes(inputs: Any) -> int:
    """Bytes of the device tensors in one input set (a dict / sequence of tensors)."""
    vals = inputs.values() if isinstance(inputs, dict) else inputs
    return sum(int(v.numel()) * int(v.element_size()) for v in vals if hasattr(v, "element_size"))


def tune(descriptor: TileLangKernelBase, hw: Optional[GPUSpec] = None, top_k: int = 4, warmup: int = 2,
         reps: int = 5, budget_ms: float = 0.0, prune: bool = True, input_copies: Union[int, str] = 1,
         seed_configs: Sequence[Dict[str, Any]] = (), ranked: Optional[Sequence[Dict[str, Any]]] = None,
         **shape_kwargs: Any) -> TuneResult:
    """Formula-rank, then measure candidates on the device and keep the fastest.

    The formula's top_k are always measured.  With ``budget_ms`` the search goes
    on down the ranking while the device time spent measuring stays within the
    budget, so cheap (small) problems get a wider search than large ones.
    ``seed_configs`` (e.g. the measured database's pick for the shape, the
    design's warm start) are measured first, in addition to the ranking; a seed
    the descriptor does not offer for the shape is skipped.  The first timing
    of a search is discarded (it absorbs the clock ramp-up of an idle device),
    and the two fastest candidates are timed again and ranked on the mean.
    ``prune=False`` ranks (and, with a large top_k, measures) the whole compiled
    set for the shape, as offline profiling does.  ``ranked`` replaces the
    formula's ranking with another one in `rank_all`'s form (e.g.
    `AdaptiveTuner.rank`, which corrects the formula with a database's
    learned residual).  ``input_copies`` > 1 times
    every candidate round-robin over that many input sets, so an operand set
    that would otherwise stay resident in the 256 MiB MALL is read from HBM on
    every launch -- the condition a memory-bound op is judged in; "auto" picks
    enough sets (at most 16) to exceed 600 MiB.

    time_to_best = prune+rank (host) + compile (instance lookup: kernels are AOT)
    + device benchmarks.  Generating the synthetic inputs is reported
    separately (inputs_s) and not counted.
    """
    t0 = time.perf_counter()
    if hw is None:
        hw = get_gpu_spec()
    all_cfgs = descriptor.get_raw_configs(**shape_kwargs)
    ranked = list(ranked) if ranked is not None else rank_all(descriptor, hw, prune=prune, **shape_kwargs)
    if not ranked:
        raise RuntimeError(f"No configs survive pruning for {descriptor.name} with {shape_kwargs}")
    t1 = time.perf_counter()
    inputs = [descriptor.make_inputs(**shape_kwargs)]  # benchmark harness, not tuner work
    if input_copies == "auto":
        copies = max(1, min(16, -(-(600 << 20) // max(1, input_bytes(inputs[0])))))
    else:
        copies = max(1, int(input_copies))
    inputs += [descriptor.make_inputs(**shape_kwargs) for _ in range(copies - 1)]
    t_in = time.perf_counter()
    if copies > 1:
        warmup, reps = max(warmup, copies), max(reps, 2 * copies)
    compile_s = 0.0
    flops = descriptor.flops(**shape_kwargs)
    cands = []
    spent_ms = 0.0
    launches = max(warmup, 1) + 3 * reps + reps       # warmup + 3 timed batches + graph capture

    runners = {}
    failed = []

    def measure(raw, formatted, score, seed):
        nonlocal compile_s, spent_ms
        try:
            tc = time.perf_counter()
            runs = [descriptor.make_runner(raw, inp, **shape_kwargs) for inp in inputs]
            compile_s += time.perf_counter() - tc
            if not cands:
                # the first timing after an idle device absorbs the clock ramp-up: discard it
                benchmark_ms(runs if copies > 1 else runs[0], warmup=warmup, reps=reps)
            ms = benchmark_ms(runs if copies > 1 else runs[0], warmup=warmup, reps=reps)
        except IcppCallError as e:
            # a candidate the library rejects is dropped with its reason (the reference's
            # harness records "ERROR" rows and goes on, conv2d.py:453-460); operand errors
            # (ValueError from the argument checks) are bugs of the caller and propagate
            failed.append({"config": raw, "formatted": formatted, "error": f"{type(e).__name__}: {e}"})
            return
        runners[formatted] = runs
        spent_ms += ms * launches
        cands.append({"config": raw, "formatted": formatted, "score": score, "ms": ms,
                      "tflops": flops / ms / 1e9, "seed": seed})
        # only the two fastest are timed again: release the other runners (each holds its
        # split-K workspace; a whole-set search kept them all and ran the device out of memory)
        keep = {c["formatted"] for c in sorted(cands, key=lambda c: c["ms"])[:2]}
        for f in [f for f in runners if f not in keep]:
            del runners[f]

    seeds = [c for c in seed_configs if c in all_cfgs]
    for c in seeds:
        measure(c, descriptor.format_config(c), None, True)
    for rank, e in enumerate(ranked):
        if rank >= max(1, top_k) and spent_ms >= budget_ms:
            break
        if e["raw_config"] in seeds:
            continue
        measure(e["raw_config"], e["formatted"], e["score"], False)
    # the two fastest are timed once more, in reverse order, and ranked on the mean of
    # both timings: the clock drifts over a search, and near-equal tiles swap places
    for c in sorted(cands, key=lambda c: c["ms"])[:2][::-1] if len(cands) > 1 else ():
        runs = runners[c["formatted"]]
        c["ms_again"] = benchmark_ms(runs if copies > 1 else runs[0], warmup=warmup, reps=reps)
    if not cands:
        raise RuntimeError(f"{descriptor.name}: every measured candidate failed for {shape_kwargs}: "
                           + "; ".join(f"{f['formatted']}: {f['error']}" for f in failed[:4]))
    t2 = t_in + compile_s
    t3 = time.perf_counter()
    best = min(cands, key=lambda c: (c["ms"] + c.get("ms_again", c["ms"])) / 2 if "ms_again" in c else float("inf"))
    if "ms_again" in best:
        best = dict(best, ms=(best["ms"] + best["ms_again"]) / 2)
        best["tflops"] = flops / best["ms"] / 1e9
    top1 = ranked[0]["raw_config"]
    top1_ms = next((c["ms"] for c in cands if c["config"] == top1), float("nan"))
    return TuneResult(
        best_config=best["config"], best_ms=best["ms"], best_tflops=best["tflops"],
        formula_top1=top1, formula_top1_ms=top1_ms, candidates=cands, failed=failed,
        prune_rank_s=t1 - t0, compile_s=t2 - t_in, bench_s=t3 - t2, time_to_best_s=(t3 - t0) - (t_in - t1),
        n_configs=len(all_cfgs), n_pruned=len(all_cfgs) - len(ranked), inputs_s=t_in - t1)


def configure_autotuner_cache(cache_dir: str = ".icpp_cache") -> None:
    """Reference :249-261 configures TileLang's JIT cache.  Kernels here are
    compiled ahead of time into libicpp_hip.so, so there is no cache to set up;
    kept so callers of the reference API keep working."""
    return None


__all__ = ["TileLangKernelBase", "TuneResult", "benchmark_ms", "configure_autotuner_cache", "rank_all",
           "select_best", "tune"]
