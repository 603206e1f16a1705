"""Offline performance database, decision table and the three-level online select.

The reference designs this stage but ships no code for it
(docs/autotuner_design.md:234-268 offline / online split; :457-465
`build_sampling_plan`, :475-477 `build_decision_table`, :482-484
`precompile_top_configs`, :488-525 `AdaptiveTuner.select`; the package
docstring kernel/autotuner/__init__.py:1-11 names the levels):

  offline  profile a stratified set of shapes on the device  -> PerformanceDB
           group the measurements by every shape dimension but one axis
           (M for GEMM-family ops, the batch N for conv) and split that axis
           into intervals, each owning the measured-best config -> DecisionTable
           fit a residual on the schedule model from every record (residual.py)
  online   Level 1: decision-table lookup (profiled shape ranges)
           Level 2: schedule model + learned residual for shapes the table misses
           Level 3: formula argmax (select_best) without a database

Here "measured best" comes from `tune()` on the device, every candidate it
measured is kept as a record, and the database is plain JSON (no pickle), keyed
by the descriptor name and the GPU it was measured on.  Databases profiled on
MI355X ship in the package (perf_db/mi355x/<name>_<dtype>.json) and are what
`AdaptiveTuner(descriptor)` loads by default.  `evaluate` measures, on shapes
that were not profiled, how close each level's pick comes to the exhaustively
measured best (the reference's accuracy table, docs :529-535); `cross_validate`
(residual.py) checks the residual level on groups of shapes it was not fitted
on.  The reference's residual is a LightGBM model; LightGBM is not in this
image, and the residual here is numpy gradient-boosted trees stored as JSON.
"""

from __future__ import annotations

import json
import math
import time
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any, Dict, Iterable, List, Optional, Sequence, Tuple

from .cost_model import ideal_seconds
from .gpu_spec import GPUSpec, get_gpu_spec
from .interface import TileLangKernelBase, rank_all, select_best, tune
from .residual import ResidualModel, cross_validate, fit_residual

SHIPPED_DIR = Path(__file__).resolve().parents[1] / "perf_db"


def op_key(descriptor: TileLangKernelBase) -> str:
    """Database key of a descriptor: its name and, when it has one, its dtype
    (one name covers several dtypes whose timings differ)."""
    dt = getattr(descriptor, "dtype", None)
    return f"{descriptor.name}_{dt}" if dt else descriptor.name


def shipped_path(op: str, hw: GPUSpec) -> Path:
    """Where the package keeps the offline database of `op` for this GPU."""
    slug = "mi355x" if "MI355X" in hw.name else "".join(c for c in hw.name.lower() if c.isalnum())
    return SHIPPED_DIR / slug / f"{op}.json"


def default_axis(shape: Dict[str, Any]) -> str:
    """The interval axis: the batch N for conv shapes, M for GEMM-family shapes."""
    return "N" if "OC" in shape else "M"


def _group_key(shape: Dict[str, Any], axis: str) -> str:
    return json.dumps({k: v for k, v in sorted(shape.items()) if k != axis}, sort_keys=True)


@dataclass
class ProfileRecord:
    shape: Dict[str, int]
    config: Dict[str, Any]
    ms: float

    def as_dict(self) -> Dict[str, Any]:
        return {"shape": self.shape, "config": self.config, "ms": self.ms}


@dataclass
class DecisionTable:
    """Per group (all shape dimensions but `axis`), sorted intervals
    [lo, hi) on the axis -> config; the last interval of a group is closed.

    Interval boundaries sit at the geometric midpoint of neighbouring profiled
    axis values (problem sizes are spread on a log scale); a lookup outside the
    profiled range of its group, or in a group never profiled, misses.
    """

    axis: str = "M"
    groups: Dict[str, List[Tuple[float, float, Dict[str, Any]]]] = field(default_factory=dict)

    def lookup(self, shape: Dict[str, Any]) -> Optional[Dict[str, Any]]:
        intervals = self.groups.get(_group_key(shape, self.axis))
        if not intervals or self.axis not in shape:
            return None
        v = float(shape[self.axis])
        for i, (lo, hi, cfg) in enumerate(intervals):
            last = i == len(intervals) - 1
            if lo <= v < hi or (last and v == hi):
                return cfg
        return None

    def as_dict(self) -> Dict[str, Any]:
        return {"axis": self.axis, "groups": {k: [[lo, hi, c] for lo, hi, c in v] for k, v in self.groups.items()}}

    @classmethod
    def from_dict(cls, d: Dict[str, Any]) -> "DecisionTable":
        return cls(axis=d["axis"], groups={k: [(float(lo), float(hi), c) for lo, hi, c in v]
                                           for k, v in d["groups"].items()})


def build_decision_table(records: Iterable[ProfileRecord], axis: Optional[str] = None) -> DecisionTable:
    """Measured-best config per profiled shape, then per group the axis split
    into intervals around the profiled points; neighbours with the same best
    config merge (reference design: group by (N, K), split M, docs :475-477)."""
    records = list(records)
    if not records:
        return DecisionTable(axis=axis or "M")
    axis = axis or default_axis(records[0].shape)
    best: Dict[str, Dict[float, Tuple[float, Dict[str, Any]]]] = {}
    for r in records:
        g = best.setdefault(_group_key(r.shape, axis), {})
        v = float(r.shape[axis])
        if v not in g or r.ms < g[v][0]:
            g[v] = (r.ms, r.config)
    groups: Dict[str, List[Tuple[float, float, Dict[str, Any]]]] = {}
    for key, pts in best.items():
        vs = sorted(pts)
        bounds = [vs[0]] + [math.sqrt(a * b) for a, b in zip(vs, vs[1:])] + [vs[-1]]
        out: List[Tuple[float, float, Dict[str, Any]]] = []
        for i, v in enumerate(vs):
            lo, hi, cfg = bounds[i], bounds[i + 1], pts[v][1]
            if out and out[-1][2] == cfg:
                out[-1] = (out[-1][0], hi, cfg)
            else:
                out.append((lo, hi, cfg))
        groups[key] = out
    return DecisionTable(axis=axis, groups=groups)


@dataclass
class PerformanceDB:
    op: str
    hw: str
    records: List[ProfileRecord] = field(default_factory=list)
    table: DecisionTable = field(default_factory=DecisionTable)
    created: float = 0.0
    residual: Optional[Dict[str, Any]] = None    # ResidualModel.as_dict() fitted on `records`

    def rebuild(self, axis: Optional[str] = None) -> None:
        self.table = build_decision_table(self.records, axis)

    def fit_residual(self, descriptor: TileLangKernelBase, hw: GPUSpec) -> None:
        """Fit the second online level's residual model on this database's records
        (none without records)."""
        self.residual = fit_residual(descriptor, self.records, hw).as_dict() if self.records else None

    def residual_model(self) -> Optional[ResidualModel]:
        return ResidualModel.from_dict(self.residual) if self.residual else None

    def to_json(self) -> str:
        """Shapes and configs are pooled once; a record is [shape index, config index, ms]."""
        shapes: Dict[str, int] = {}
        configs: Dict[str, int] = {}
        rows = []
        for r in self.records:
            sk = json.dumps(r.shape, sort_keys=True)
            ck = json.dumps(r.config, sort_keys=True)
            rows.append([shapes.setdefault(sk, len(shapes)), configs.setdefault(ck, len(configs)), r.ms])
        d = {"op": self.op, "hw": self.hw, "created": self.created,
             "shapes": [json.loads(k) for k in shapes], "configs": [json.loads(k) for k in configs],
             "records": rows, "table": self.table.as_dict()}
        if self.residual is not None:
            d["residual"] = self.residual
        return json.dumps(d, sort_keys=True, separators=(",", ":"))

    @classmethod
    def from_json(cls, text: str) -> "PerformanceDB":
        d = json.loads(text)
        shapes, configs = d["shapes"], d["configs"]
        return cls(op=d["op"], hw=d["hw"], created=d.get("created", 0.0),
                   records=[ProfileRecord(dict(shapes[si]), dict(configs[ci]), float(ms)) for si, ci, ms in d["records"]],
                   table=DecisionTable.from_dict(d["table"]), residual=d.get("residual"))

    def save(self, path) -> None:
        Path(path).write_text(self.to_json())

    @classmethod
    def load(cls, path) -> "PerformanceDB":
        return cls.from_json(Path(path).read_text())


def build_sampling_plan(op_type: str, hw: Optional[GPUSpec] = None, *, m_range=(16, 16384),
                        nk: Sequence[Tuple[int, int]] = ((4096, 4096),), conv: Sequence[Dict[str, int]] = (),
                        batches: Sequence[int] = (1, 4, 16, 32, 64, 128), ref_tile: Tuple[int, int] = (128, 128),
                        points_per_wave: int = 1) -> List[Dict[str, int]]:
    """Shapes to profile, stratified by wave count (reference docs :457-461).

    GEMM-family ops: for each (N, K), M values at which a reference tile grid
    (ref_tile) crosses 1/8, 1/4, 1/2, 1, 2, 4, ... waves of the device's CUs
    (with points_per_wave > 1, also evenly between them), the powers of two
    from 16 below the first of those (small M, where split-K decides), and the
    range ends, all clipped to m_range.  Conv: every given base geometry
    (without N) at each batch size in `batches`."""
    hw = hw or get_gpu_spec()
    if op_type.startswith("conv"):
        return [dict(g, N=b) for g in conv for b in batches]
    lo, hi = m_range
    shapes = []
    for (N, K) in nk:
        tiles_n = -(-N // ref_tile[1])
        ms = {lo, hi}
        w, first = 1.0 / 8, None
        while True:
            m = max(1, int(round(w * hw.num_sm / tiles_n))) * ref_tile[0]
            if m > hi:
                break
            if m >= lo:
                first = m if first is None else first
                for j in range(points_per_wave):
                    ms.add(max(lo, min(hi, int(m * (1 + j / max(1, points_per_wave))))))
            w *= 2
        p2 = 16
        while p2 < min(hi, first or hi):
            if p2 >= lo:
                ms.add(p2)
            p2 *= 2
        shapes += [dict(M=m, N=N, K=K) for m in sorted(ms)]
    return shapes


def profile(descriptor: TileLangKernelBase, shapes: Sequence[Dict[str, int]], hw: Optional[GPUSpec] = None,
            top_k: int = 0, budget_ms: float = 0.0, reps: int = 10, log=None) -> List[ProfileRecord]:
    """Measure candidates for every shape with `tune()` (the device); every
    measured candidate becomes a record.  top_k=0 (the default) measures the
    whole compiled set for the shape, unpruned: the offline stage is exhaustive
    (reference docs :440-451), so the table is not limited by the formula.
    Candidates are timed round-robin over input copies larger than the MALL
    (`tune(input_copies="auto")`), the condition the kernels run in when their
    operands are not cache-resident: ranked on one resident input set, configs
    that win cache-hot lost up to 1.5x on HBM-resident operands."""
    hw = hw or get_gpu_spec()
    records: List[ProfileRecord] = []
    for shape in shapes:
        if top_k <= 0:
            res = tune(descriptor, hw, top_k=1 << 30, reps=reps, prune=False, input_copies="auto", **shape)
        else:
            res = tune(descriptor, hw, top_k=top_k, reps=reps, budget_ms=budget_ms, input_copies="auto", **shape)
        for c in res.candidates:
            records.append(ProfileRecord(dict(shape), c["config"], float(c["ms"])))
        if log:
            log(f"[perfdb] {descriptor.name} {shape}: {len(res.candidates)} measured, best "
                f"{descriptor.format_config(res.best_config)} {res.best_ms * 1e3:.1f} us")
    return records


def build_db(descriptor: TileLangKernelBase, shapes: Sequence[Dict[str, int]], hw: Optional[GPUSpec] = None,
             **kw) -> PerformanceDB:
    hw = hw or get_gpu_spec()
    db = PerformanceDB(op=op_key(descriptor), hw=hw.name, records=profile(descriptor, shapes, hw, **kw),
                       created=time.time())
    db.rebuild()
    return db


@dataclass
class SelectResult:
    config: Dict[str, Any]
    level: str            # "table", "residual" or "formula"
    score: Optional[float] = None
    seconds: float = 0.0


class AdaptiveTuner:
    """Three-level online select (reference docs :491-525, levels named in
    kernel/autotuner/__init__.py:8-11): the decision table for profiled shape
    ranges; the schedule model corrected by the database's learned residual for
    shapes the table misses; the formula argmax when there is no database (or it
    carries no residual).  A table entry is used only when the descriptor still
    offers that config for the shape (same compiled set, K / split constraints
    hold).  The residual level ranks the same pruned configs as the formula."""

    def __init__(self, descriptor: TileLangKernelBase, db: Any = "auto", hw: Optional[GPUSpec] = None):
        """db: a PerformanceDB, a path to one, "auto" (the database shipped for
        this op and GPU, if any) or None (cold start: formula only).  A
        database measured for another op or GPU is ignored."""
        self.descriptor = descriptor
        self.hw = hw or get_gpu_spec()
        if isinstance(db, str) and db == "auto":
            path = shipped_path(op_key(descriptor), self.hw)
            db = PerformanceDB.load(path) if path.exists() else None
        elif isinstance(db, (str, Path)):
            db = PerformanceDB.load(db)
        self.db = db if (db is None or (db.op == op_key(descriptor) and db.hw == self.hw.name)) else None
        self.residual = self.db.residual_model() if self.db is not None and self.hw.has_mfma_model else None
        self._memo: Dict[str, SelectResult] = {}

    MEMO_MAX = 4096

    def select(self, **shape) -> SelectResult:
        """The answers are memoised per shape (at most MEMO_MAX shapes), so a
        process that meets the same shapes again pays the residual level once."""
        t0 = time.perf_counter()
        key = json.dumps(shape, sort_keys=True)
        hit = self._memo.get(key)
        if hit is None:
            hit = self._select(shape)
            if len(self._memo) >= self.MEMO_MAX:
                self._memo.clear()
            self._memo[key] = hit
        return SelectResult(dict(hit.config), hit.level, hit.score, time.perf_counter() - t0)

    def _select(self, shape: Dict[str, Any]) -> SelectResult:
        t0 = time.perf_counter()
        if self.db is not None:
            cfg = self.db.table.lookup(shape)
            if cfg is not None and cfg in self.descriptor.get_raw_configs(**shape):
                return SelectResult(cfg, "table", None, time.perf_counter() - t0)
        if self.residual is not None:
            ranked = self.rank(**shape)
            if ranked:
                return SelectResult(ranked[0]["raw_config"], "residual", ranked[0]["score"], time.perf_counter() - t0)
        cfg, score = select_best(self.descriptor, self.hw, **shape)
        return SelectResult(cfg, "formula", score, time.perf_counter() - t0)

    def rank(self, **shape) -> List[Dict[str, Any]]:
        """The pruned configs best first, in `rank_all`'s form, by the formula
        corrected with the database's residual when there is one (the order the
        residual level picks from), else by the formula.  For `tune(ranked=...)`."""
        if self.residual is None:
            return rank_all(self.descriptor, self.hw, **shape)
        raws = self.descriptor.prune(self.descriptor.get_raw_configs(**shape), self.hw, **shape)
        lt = self.residual.log_time(self.descriptor, raws, self.hw, shape)
        out = []
        for i in sorted(range(len(raws)), key=lambda i: lt[i]):
            op = self.descriptor.make_op_spec(raw_config=raws[i], **shape)
            ideal = ideal_seconds(op, self.descriptor.raw_config_to_tune_config(raws[i]), self.hw)
            out.append({"raw_config": raws[i], "score": ideal / math.exp(lt[i]),
                        "formatted": self.descriptor.format_config(raws[i])})
        return out

    def precompile(self) -> Dict[str, int]:
        """Reference `precompile_top_configs` (docs :482-484).  Kernels here are
        compiled ahead of time, so this resolves every config the table names to
        its instance and raises if one is not in the compiled set."""
        out: Dict[str, int] = {}
        if self.db is None:
            return out
        for intervals in self.db.table.groups.values():
            for _, _, cfg in intervals:
                out[self.descriptor.format_config(cfg)] = self.descriptor.instance_index(cfg)
        return out


_TUNERS: Dict[int, AdaptiveTuner] = {}


def select_config(descriptor: TileLangKernelBase, **shape) -> Dict[str, Any]:
    """The config `build_kernel(config=None)` uses: the shipped database's
    table for profiled shape ranges, else the formula (one AdaptiveTuner per
    descriptor, created on first use)."""
    t = _TUNERS.get(id(descriptor))
    if t is None or t.descriptor is not descriptor:
        t = _TUNERS[id(descriptor)] = AdaptiveTuner(descriptor)
    return t.select(**shape).config


def evaluate(descriptor: TileLangKernelBase, db: Optional[PerformanceDB], shapes: Sequence[Dict[str, int]],
             hw: Optional[GPUSpec] = None, reps: int = 10, log=None) -> Dict[str, Any]:
    """Measure every compiled candidate of each shape, unpruned (the oracle),
    and score the picks of the table and of the formula against it: top-1 hit
    rate and oracle_ms / pick_ms (1.0 = the pick is the fastest).  `pruned_best`
    is the fastest config that survives the L1-L4 prune, i.e. what the online
    `tune()` search could find at best."""
    hw = hw or get_gpu_spec()
    tuner = AdaptiveTuner(descriptor, db, hw)
    rows = []
    for shape in shapes:
        res = tune(descriptor, hw, top_k=1 << 30, reps=reps, prune=False, input_copies="auto", **shape)
        ms = {descriptor.format_config(c["config"]): c["ms"] for c in res.candidates}
        kept = {descriptor.format_config(c) for c in descriptor.prune(descriptor.get_raw_configs(**shape), hw, **shape)}
        sel = tuner.select(**shape)
        ranked = _formula_ranking(descriptor, hw, shape)
        formula = ranked[0]
        pick = descriptor.format_config(sel.config)
        oracle = min(ms, key=ms.get)       # from the same single timings as every pick it is compared with
        row = {"shape": dict(shape), "oracle": oracle, "oracle_ms": ms[oracle],
               "level": sel.level, "pick": pick, "pick_ms": ms.get(pick), "formula": formula,
               "formula_ms": ms[formula], "formula_ranking": ranked,
               "pruned_best_ms": min(v for k, v in ms.items() if k in kept),
               "n_measured": len(ms), "n_pruned_set": len(kept), "ms": ms}
        rows.append(row)
        if log:
            log(f"[perfdb-eval] {descriptor.name} {shape}: oracle {oracle} {ms[oracle] * 1e3:.1f} us, "
                f"{sel.level} {pick} {(row['pick_ms'] or float('nan')) * 1e3:.1f} us, formula {formula} "
                f"{row['formula_ms'] * 1e3:.1f} us")
    return _report(descriptor, rows)


def rescore(descriptor: TileLangKernelBase, report: Dict[str, Any], hw: Optional[GPUSpec] = None) -> Dict[str, Any]:
    """Re-pick the formula's top-1 of every row of an `evaluate` report with the
    current cost model and score it against the times the row already holds
    (every compiled config was measured there): no device work.  The oracle is
    the fastest of those times (reports written before that rule took the
    tuner's re-timed best)."""
    hw = hw or get_gpu_spec()
    rows = []
    for r in report["rows"]:
        ranked = _formula_ranking(descriptor, hw, r["shape"])
        formula = ranked[0]
        oracle = min(r["ms"], key=r["ms"].get)
        row = dict(r, oracle=oracle, oracle_ms=r["ms"][oracle], formula=formula, formula_ms=r["ms"][formula],
                   formula_ranking=ranked)
        if r["level"] == "formula":      # a table miss falls back to the formula's pick
            row.update(pick=formula, pick_ms=r["ms"][formula])
        rows.append(row)
    return _report(descriptor, rows)


TOPK = (1, 2, 4, 8)


def _formula_ranking(descriptor: TileLangKernelBase, hw: GPUSpec, shape: Dict[str, Any]) -> List[str]:
    """The formula's first max(TOPK) configs for the shape (pruned, best first;
    the first is `select_best`'s pick)."""
    return [e["formatted"] for e in rank_all(descriptor, hw, **shape)[:max(TOPK)]]


def _report(descriptor: TileLangKernelBase, rows: List[Dict[str, Any]]) -> Dict[str, Any]:
    def topk(k):
        """A measured search of the formula's top k (tune() without seeds, top_k=k):
        the fastest of those k against the oracle."""
        ratios = [r["oracle_ms"] / min(r["ms"][c] for c in r["formula_ranking"][:k])
                  for r in rows if r.get("formula_ranking")]
        return {"n": len(ratios), "perf_ratio_mean": sum(ratios) / max(1, len(ratios)),
                "perf_ratio_min": min(ratios, default=0.0)}

    def summary(key, sel_rows):
        sel_rows = [r for r in sel_rows if r[key + "_ms"] is not None]
        if not sel_rows:
            return {"n": 0}
        ratios = [r["oracle_ms"] / r[key + "_ms"] for r in sel_rows]
        return {"n": len(sel_rows), "top1": sum(r[key] == r["oracle"] for r in sel_rows) / len(sel_rows),
                "perf_ratio_mean": sum(ratios) / len(ratios), "perf_ratio_min": min(ratios)}

    table_rows = [r for r in rows if r["level"] == "table"]
    pr = [r["oracle_ms"] / r["pruned_best_ms"] for r in rows]
    return {"op": op_key(descriptor), "rows": rows, "table": summary("pick", table_rows),
            "formula": summary("formula", rows), "formula_topk": {str(k): topk(k) for k in TOPK},
            "combined": summary("pick", rows),
            "pruned_set": {"n": len(rows), "perf_ratio_mean": sum(pr) / max(1, len(pr)), "perf_ratio_min": min(pr, default=0)}}


def held_out(shapes: Sequence[Dict[str, int]], axis: Optional[str] = None) -> List[Dict[str, int]]:
    """Shapes between the profiled ones: per group, the geometric midpoint of
    each neighbouring pair on the axis, moved off the tile grid (+3 for M)."""
    groups: Dict[str, List[Dict[str, int]]] = {}
    for s in shapes:
        groups.setdefault(_group_key(s, axis or default_axis(s)), []).append(s)
    out = []
    for g in groups.values():
        ax = axis or default_axis(g[0])
        vs = sorted({s[ax] for s in g})
        for a, b in zip(vs, vs[1:]):
            v = int(round(math.sqrt(a * b))) + (3 if ax == "M" else 0)
            if a < v < b:
                out.append(dict(g[0], **{ax: v}))
    return out


def default_plan(op: str, hw: Optional[GPUSpec] = None) -> List[Dict[str, int]]:
    """The shapes the shipped databases were profiled on."""
    hw = hw or get_gpu_spec()
    if op == "conv2d" or op.startswith("conv2d_") or op == "conv_bn_add_relu":
        # the three C4 geometries, then ResNet-50's other kinds of layer: the 28^2 stage's
        # 3x3, a stride-2 3x3, and two 1x1 bottleneck projections
        geos = [dict(C=64, H=56, W=56, OC=64, KH=3, KW=3, stride=1, padding=1),
                dict(C=256, H=14, W=14, OC=256, KH=3, KW=3, stride=1, padding=1),
                dict(C=512, H=7, W=7, OC=512, KH=3, KW=3, stride=1, padding=1),
                dict(C=128, H=28, W=28, OC=128, KH=3, KW=3, stride=1, padding=1),
                dict(C=128, H=56, W=56, OC=128, KH=3, KW=3, stride=2, padding=1),
                dict(C=256, H=56, W=56, OC=64, KH=1, KW=1, stride=1, padding=0),
                dict(C=1024, H=14, W=14, OC=256, KH=1, KW=1, stride=1, padding=0)]
        return build_sampling_plan("conv2d", hw, conv=geos, batches=(1, 2, 4, 8, 16, 32, 48, 64, 128))
    if op == "gemm_splitk":   # the reference's offline-builder example (docs :543-549)
        nk = [(n, k) for n in (768, 2304, 4096) for k in (768, 2304, 4096)]
        return build_sampling_plan(op, hw, m_range=(1, 4096), nk=nk, points_per_wave=2)
    if op == "fp8_gemm_bias_silu":
        return build_sampling_plan(op, hw, m_range=(16, 4096), nk=[(4096, 4096), (11008, 4096), (4096, 11008)],
                                   points_per_wave=2)
    if op == "gemm_bias_layernorm":   # C3 shapes, BERT-base's attention-output and FFN-output blocks, and the
        # reference's evaluation shape (N = 2304, K = 768: gemm_three_ops_formula_summary.csv,
        # M = 1 ... 126), from decode-sized M up.  Below 128 rows every 16 rows: the one-launch
        # strategy's time steps with the row-block count, which a power-of-two grid misses
        nk = [(768, 4096), (1024, 4096), (4096, 4096), (768, 768), (768, 3072), (2304, 768)]
        plan = build_sampling_plan(op, hw, m_range=(16, 8192), nk=nk, points_per_wave=2)
        have = {(s["M"], s["N"], s["K"]) for s in plan}
        plan += [dict(M=m, N=n, K=k) for n, k in nk for m in range(16, 128, 16) if (m, n, k) not in have]
        return plan
    if op == "gemm_bias_gelu_erf":     # BERT-base's FFN-in block (end2end.py:82-83)
        return build_sampling_plan(op, hw, m_range=(128, 16384), nk=[(3072, 768), (4096, 1024)], points_per_wave=2)
    # GEMM + bias + activation: C2's 4096-class shapes and the reference's evaluation shape
    return build_sampling_plan(op, hw, m_range=(16, 8192), nk=[(4096, 4096), (1024, 4096), (4096, 1024), (2304, 768)],
                               points_per_wave=2)


def unseen_plan(op: str) -> List[Dict[str, int]]:
    """Shapes in groups the shipped databases never profiled -- other (N, K)
    pairs, other conv geometries -- where the table always misses: what the
    residual level is for."""
    if op == "conv2d" or op.startswith("conv2d_") or op == "conv_bn_add_relu":
        geos = [dict(C=192, H=28, W=28, OC=192, KH=3, KW=3, stride=1, padding=1),
                dict(C=256, H=28, W=28, OC=256, KH=3, KW=3, stride=1, padding=1),
                dict(C=512, H=28, W=28, OC=128, KH=1, KW=1, stride=1, padding=0)]
        return [dict(g, N=b) for g in geos for b in (4, 16, 48)]
    grid = {
        "gemm_splitk": ([(1536, 3072), (3072, 1536), (6144, 2048)], (48, 700, 2500)),
        "fp8_gemm_bias_silu": ([(8192, 8192), (14336, 4096), (4096, 14336)], (32, 512, 2048)),
        "gemm_bias_layernorm": ([(512, 1024), (2048, 2048)], (1000, 4000)),
        "gemm_bias_gelu_erf": ([(2048, 512), (5120, 1280)], (512, 4000)),
    }
    nk, ms = grid.get(op, ([(3072, 768), (8192, 2048), (2048, 8192)], (256, 1500, 6000)))
    return [dict(M=m, N=n, K=k) for n, k in nk for m in ms]


def _descriptors():
    from ..kernels import conv2d, conv2d_fused, fp8_gemm_bias_act, gemm, gemm_bias_act, gemm_bias_layernorm

    ds = [gemm.DESCRIPTOR, gemm_bias_act.descriptor("gelu_tanh", "bf16"), gemm_bias_act.descriptor("relu", "bf16"),
          gemm_bias_act.descriptor("silu", "bf16"), gemm_bias_act.descriptor("gelu_erf", "f16"),
          gemm_bias_layernorm.DESCRIPTOR, fp8_gemm_bias_act.DESCRIPTOR, conv2d.DESCRIPTOR] + \
        list(conv2d_fused.DESCRIPTORS.values())
    out = {d.name: d for d in ds}
    # a second dtype of a name is keyed name_dtype: ReLU in fp16, the reference's own gemm_bias_act
    out["gemm_bias_relu_f16"] = gemm_bias_act.descriptor("relu", "f16")
    return out


def main(argv=None) -> int:  # pragma: no cover - device tool
    """Offline builder (reference docs :539-553): profile, build the table, fit
    the residual, write the JSON, and optionally evaluate the levels on held-out
    shapes."""
    import argparse

    ops = _descriptors()
    ap = argparse.ArgumentParser(description="profile shapes on the device and write a PerformanceDB (JSON)")
    ap.add_argument("--op", choices=sorted(ops), required=True)
    ap.add_argument("--out", default="", help="default: the package's shipped location for this GPU")
    ap.add_argument("--top-k", type=int, default=0, help="0: measure the whole compiled set per shape")
    ap.add_argument("--budget-ms", type=float, default=0.0)
    ap.add_argument("--eval-out", default="", help="also evaluate on held-out shapes and write the report here")
    ap.add_argument("--eval-only", action="store_true", help="evaluate the database at --out (or the shipped one)")
    ap.add_argument("--rescore", default="", help="an --eval-out report: re-pick its formula column with the "
                    "current cost model against the times it holds (no device work), write to --eval-out")
    ap.add_argument("--eval-unseen", default="", help="evaluate the database at --out (or the shipped one) on "
                    "shapes of groups it never profiled (unseen_plan); write the report to this path")
    ap.add_argument("--fit-residual", action="store_true",
                    help="fit the residual level on the database at --out (or the shipped one) and save it there")
    ap.add_argument("--cv-residual", default="", help="leave-one-group-out check of the residual level on the "
                    "database at --out (or the shipped one); write the report to this path")
    a = ap.parse_args(argv)
    desc = ops[a.op]
    hw = get_gpu_spec()
    if a.fit_residual or a.cv_residual:
        path = Path(a.out) if a.out else shipped_path(op_key(desc), hw)
        db = PerformanceDB.load(path)
        if a.cv_residual:
            axis = db.table.axis
            rows = cross_validate(desc, db.records, hw, lambda s: _group_key(s, axis))
            Path(a.cv_residual).write_text(json.dumps({"op": op_key(desc), "groups": rows}, indent=1))
            for r in rows:
                print(json.dumps(r), flush=True)
        if a.fit_residual:
            db.fit_residual(desc, hw)
            db.save(path)
            print(f"[perfdb] residual fitted on {len(db.records)} records -> {path}", flush=True)
        return 0
    if a.rescore:
        rep = rescore(desc, json.loads(Path(a.rescore).read_text()), hw)
        if a.eval_out:
            Path(a.eval_out).write_text(json.dumps(rep, indent=1))
        print(json.dumps({k: rep[k] for k in ("op", "table", "formula", "formula_topk", "combined", "pruned_set")}),
              flush=True)
        return 0
    shapes = default_plan(a.op, hw)
    out = Path(a.out) if a.out else shipped_path(op_key(desc), hw)
    if a.eval_unseen:
        rep = evaluate(desc, PerformanceDB.load(out), unseen_plan(a.op), hw, log=lambda m: print(m, flush=True))
        Path(a.eval_unseen).write_text(json.dumps(rep, indent=1))
        print(json.dumps({k: rep[k] for k in ("op", "formula", "formula_topk", "combined", "pruned_set")}), flush=True)
        return 0
    if a.eval_only:
        db = PerformanceDB.load(out)
    else:
        print(f"[perfdb] {a.op}: {len(shapes)} shapes", flush=True)
        db = build_db(desc, shapes, hw, top_k=a.top_k, budget_ms=a.budget_ms, log=lambda m: print(m, flush=True))
        db.fit_residual(desc, hw)
        out.parent.mkdir(parents=True, exist_ok=True)
        db.save(out)
        print(f"[perfdb] {len(db.records)} records, {sum(len(v) for v in db.table.groups.values())} intervals -> "
              f"{out}", flush=True)
    if a.eval_out:
        rep = evaluate(desc, db, held_out(shapes), hw, log=lambda m: print(m, flush=True))
        Path(a.eval_out).write_text(json.dumps(rep, indent=1))
        print(json.dumps({k: rep[k] for k in ("op", "table", "formula", "combined", "pruned_set")}), flush=True)
    return 0


if __name__ == "__main__":  # pragma: no cover
    raise SystemExit(main())


__all__ = ["AdaptiveTuner", "DecisionTable", "PerformanceDB", "ProfileRecord", "SelectResult", "build_db",
           "build_decision_table", "build_sampling_plan", "default_axis", "default_plan", "evaluate", "held_out",
           "op_key", "profile", "rescore", "select_config", "shipped_path", "unseen_plan"]
