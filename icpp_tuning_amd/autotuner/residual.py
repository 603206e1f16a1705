"""Learned residual on the CDNA4 schedule model (the second online level).

The reference's package docstring names three online levels
(kernel/autotuner/__init__.py:4-11): a decision table for profiled shapes, the
formula plus an ML residual (LightGBM) for unseen shapes, and the pure formula
as the cold-start fallback.  LightGBM is not in this image; this module fits
the same kind of model -- gradient-boosted regression trees over
histogram-binned features, squared loss -- in numpy, deterministically, and
stores it as JSON inside the PerformanceDB it was fitted on.

Target.  For every profiled shape of the database and every config measured
there: log(measured ms / predicted s), minus its mean over that shape's
configs.  The select only compares configs of one shape, so only relative
times matter; centring removes what the model cannot know (the device's clock
on the day, launch overheads common to all configs).

Features (`FEATURES`): the schedule model's breakdown of the launch (log times
of its parts, rounds, residency), the config's template parameters, and the
problem size.  They are computed by the same descriptor and cost model that
rank the configs, so the residual corrects exactly the model it was fitted on.
"""

from __future__ import annotations

import json
import math
from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import cost_model as cm
from .gpu_spec import GPUSpec
from .interface import select_best

FEATURES = (
    "log_predicted_s", "log_mainloop_s", "log_epilogue_s", "log_hbm_s", "log_reduce_s", "log_extra_s",
    "throughput_bound", "tiles_per_cu", "concurrent", "rounds",
    "block_M", "block_N", "block_K", "num_stages", "waves", "mfma_m", "split_k", "vgprs", "pingpong",
    "log_M", "log_N", "log_K",
)


def schedule_features(descriptor, raw: Dict[str, Any], hw: GPUSpec, shape: Dict[str, Any]) -> Tuple[List[float], float]:
    """(feature row, predicted seconds incl. the descriptor's extra launches) of one config."""
    op = descriptor.make_op_spec(raw_config=raw, **shape)
    cfg = descriptor.raw_config_to_tune_config(raw)
    sc = cm.predict_schedule(op, cfg, hw)
    extra = descriptor.extra_seconds(raw, hw, **shape)
    t = sc["seconds"] + extra
    mf = int(cfg.mfma.split("x")[0]) if cfg.mfma else 0
    row = [math.log(t), math.log(sc["mainloop_s"] + 1e-9), math.log(sc["epilogue_s"] + 1e-9),
           math.log(sc["hbm_s"] + 1e-9), math.log(sc["reduce_s"] + 1e-7), math.log(extra + 1e-7),
           float(sc["throughput_bound"]), float(sc["n_cu"]), float(sc["concurrent"]), float(sc["rounds"]),
           float(cfg.block_M), float(cfg.block_N), float(cfg.block_K), float(cfg.num_stages), float(cfg.num_warps),
           float(mf), float(cfg.split_k), float(cfg.vgprs), float(raw.get("sched") == "pp"),
           math.log(op.M), math.log(op.N), math.log(op.K * max(1, cfg.split_k))]
    return row, t


# ---------------------------------------------------------------------------
# Gradient-boosted regression trees (squared loss, histogram splits)
# ---------------------------------------------------------------------------


@dataclass
class BoostedTrees:
    """Trees are flat node lists [feature, threshold, left, right, value]; a
    leaf has feature -1.  A sample goes left when x[feature] <= threshold."""

    learning_rate: float = 0.1
    trees: List[List[List[float]]] = field(default_factory=list)

    def predict(self, X: np.ndarray) -> np.ndarray:
        X = np.asarray(X, dtype=np.float64)
        out = np.zeros(len(X))
        rows = np.arange(len(X))
        for tree in self.trees:
            nodes = np.asarray(tree, dtype=np.float64)
            at = np.zeros(len(X), dtype=np.int64)
            while True:
                feat = nodes[at, 0].astype(np.int64)
                inner = feat >= 0
                if not inner.any():
                    break
                go_left = X[rows[inner], feat[inner]] <= nodes[at[inner], 1]
                at[inner] = np.where(go_left, nodes[at[inner], 2], nodes[at[inner], 3]).astype(np.int64)
            out += nodes[at, 4]
        return out

    def as_dict(self) -> Dict[str, Any]:
        """JSON form: an inner node is [feature, threshold, left, right], a leaf [value]."""
        def node(n):
            if n[0] < 0:
                return [float(f"{n[4]:.7g}")]
            return [int(n[0]), float(f"{n[1]:.9g}"), int(n[2]), int(n[3])]
        return {"learning_rate": self.learning_rate, "trees": [[node(n) for n in t] for t in self.trees]}

    @classmethod
    def from_dict(cls, d: Dict[str, Any]) -> "BoostedTrees":
        def node(n):
            return [-1.0, 0.0, -1.0, -1.0, float(n[0])] if len(n) == 1 else [float(v) for v in n] + [0.0]
        return cls(learning_rate=float(d["learning_rate"]), trees=[[node(n) for n in t] for t in d["trees"]])


def _bin_edges(col: np.ndarray, n_bins: int) -> np.ndarray:
    """Split candidates of one feature: midpoints between its distinct values,
    thinned to at most n_bins - 1 by quantile when there are more."""
    u = np.unique(col)
    if len(u) <= 1:
        return np.empty(0)
    mids = (u[:-1] + u[1:]) / 2.0
    if len(mids) > n_bins - 1:
        mids = np.unique(np.quantile(mids, np.linspace(0.0, 1.0, n_bins - 1)))
    return mids


def fit_boosted_trees(X: np.ndarray, y: np.ndarray, n_trees: int = 100, depth: int = 4, learning_rate: float = 0.2,
                      min_leaf: int = 20, n_bins: int = 32, l2: float = 1.0) -> BoostedTrees:
    """Least-squares boosting: each tree fits the current residual with
    depth-wise greedy splits on binned features (gain = G_L^2/(n_L+l2) +
    G_R^2/(n_R+l2) - G^2/(n+l2)); leaves hold G/(n+l2), shrunk by the rate."""
    X = np.asarray(X, dtype=np.float64)
    y = np.asarray(y, dtype=np.float64)
    n, nf = X.shape
    edges = [_bin_edges(X[:, f], n_bins) for f in range(nf)]
    binned = np.stack([np.searchsorted(edges[f], X[:, f], side="left") for f in range(nf)], axis=1)
    pred = np.zeros(n)
    model = BoostedTrees(learning_rate=learning_rate)
    for _ in range(n_trees):
        g = y - pred
        nodes: List[List[float]] = []
        frontier = [(np.arange(n), 0, -1, 0)]     # (sample indices, depth, parent node, side)
        while frontier:
            idx, d, parent, side = frontier.pop(0)
            me = len(nodes)
            gs = g[idx].sum()
            nodes.append([-1.0, 0.0, -1.0, -1.0, 0.0])
            if parent >= 0:
                nodes[parent][2 + side] = float(me)
            split = _best_split(binned, edges, idx, g, gs, min_leaf, l2) if d < depth else None
            if split is None:      # a leaf: its samples move by the shrunk mean step
                value = learning_rate * gs / (len(idx) + l2)
                nodes[me][4] = value
                pred[idx] += value
                continue
            f, k = split
            nodes[me][0], nodes[me][1] = float(f), float(edges[f][k])
            left = binned[idx, f] <= k
            frontier.append((idx[left], d + 1, me, 0))
            frontier.append((idx[~left], d + 1, me, 1))
        model.trees.append(nodes)
    return model


def _best_split(binned: np.ndarray, edges: List[np.ndarray], idx: np.ndarray, g: np.ndarray, gs: float,
                min_leaf: int, l2: float) -> Optional[Tuple[int, int]]:
    """(feature, bin) of the largest positive gain with >= min_leaf samples on each side."""
    n = len(idx)
    if n < 2 * min_leaf:
        return None
    best, out = 0.0, None
    base = gs * gs / (n + l2)
    for f in range(binned.shape[1]):
        nb = len(edges[f]) + 1
        if nb < 2:
            continue
        b = binned[idx, f]
        cnt = np.bincount(b, minlength=nb)[:-1].cumsum()
        sm = np.bincount(b, weights=g[idx], minlength=nb)[:-1].cumsum()
        ok = (cnt >= min_leaf) & (n - cnt >= min_leaf)
        if not ok.any():
            continue
        gain = np.where(ok, sm ** 2 / (cnt + l2) + (gs - sm) ** 2 / (n - cnt + l2) - base, -np.inf)
        k = int(np.argmax(gain))
        if gain[k] > best:
            best, out = float(gain[k]), (f, k)
    return out


# ---------------------------------------------------------------------------
# The residual model of one database
# ---------------------------------------------------------------------------


@dataclass
class ResidualModel:
    trees: BoostedTrees
    features: Sequence[str] = FEATURES

    def log_time(self, descriptor, raws: Sequence[Dict[str, Any]], hw: GPUSpec,
                 shape: Dict[str, Any]) -> np.ndarray:
        """Corrected log predicted time of each config (lower is faster)."""
        rows, base = [], []
        for raw in raws:
            r, t = schedule_features(descriptor, raw, hw, shape)
            rows.append(r)
            base.append(math.log(t))
        if not rows:
            return np.empty(0)
        return np.asarray(base) + self.trees.predict(np.asarray(rows))

    def as_dict(self) -> Dict[str, Any]:
        return {"features": list(self.features), **self.trees.as_dict()}

    @classmethod
    def from_dict(cls, d: Dict[str, Any]) -> Optional["ResidualModel"]:
        """None when the stored model was fitted on other features."""
        if tuple(d.get("features", ())) != FEATURES:
            return None
        return cls(BoostedTrees.from_dict(d))


def training_set(descriptor, records, hw: GPUSpec) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(X, centred target, shape id) from PerformanceDB records."""
    by: Dict[str, list] = {}
    for r in records:
        by.setdefault(json.dumps(r.shape, sort_keys=True), []).append(r)
    X, y, gid = [], [], []
    for i, (key, recs) in enumerate(by.items()):
        shape = json.loads(key)
        res = []
        for r in recs:
            row, t = schedule_features(descriptor, r.config, hw, shape)
            X.append(row)
            res.append(math.log(r.ms * 1e-3 / t))
        mean = sum(res) / len(res)
        y.extend(v - mean for v in res)
        gid.extend([i] * len(res))
    return np.asarray(X), np.asarray(y), np.asarray(gid)


def fit_residual(descriptor, records, hw: GPUSpec, **kw) -> ResidualModel:
    X, y, _ = training_set(descriptor, records, hw)
    return ResidualModel(fit_boosted_trees(X, y, **kw))


def cross_validate(descriptor, records, hw: GPUSpec, group_of, **kw) -> List[Dict[str, Any]]:
    """Leave one group of shapes out (e.g. one (N, K) pair): fit on the other
    groups' records, then at each shape of the left-out group pick the
    fastest-predicted pruned config with and without the residual and score it
    as fastest measured / pick measured.  `group_of(shape)` names the group."""
    X, y, gid = training_set(descriptor, records, hw)
    by: Dict[str, list] = {}
    for r in records:
        by.setdefault(json.dumps(r.shape, sort_keys=True), []).append(r)
    keys = list(by)                      # the shape order of training_set's ids
    groups = [group_of(json.loads(k)) for k in keys]
    out = []
    for g in sorted(set(groups)):
        train = np.array([groups[i] != g for i in gid])
        model = fit_boosted_trees(X[train], y[train], **kw)
        ratios: Dict[str, List[float]] = {"formula": [], "residual": []}
        for i, key in enumerate(keys):
            if groups[i] != g:
                continue
            shape, recs, rows = json.loads(key), by[key], gid == i
            ms = np.array([r.ms for r in recs])
            names = [descriptor.format_config(r.config) for r in recs]
            kept = {descriptor.format_config(c)
                    for c in descriptor.prune(descriptor.get_raw_configs(**shape), hw, **shape)}
            ok = np.array([n in kept for n in names])
            formula = names.index(descriptor.format_config(select_best(descriptor, hw, **shape)[0]))
            corrected = np.where(ok, X[rows, 0] + model.predict(X[rows]), np.inf)
            ratios["formula"].append(float(ms.min() / ms[formula]))
            ratios["residual"].append(float(ms.min() / ms[int(np.argmin(corrected))]))
        out.append({"group": g, "shapes": len(ratios["formula"]),
                    **{f"{k}_mean": sum(v) / len(v) for k, v in ratios.items()},
                    **{f"{k}_min": min(v) for k, v in ratios.items()}})
    return out


__all__ = ["FEATURES", "BoostedTrees", "ResidualModel", "cross_validate", "fit_boosted_trees", "fit_residual",
           "schedule_features", "training_set"]
