"""Descriptor base for the AOT-compiled gfx950 instances.

A raw config is the reference's dict layout (``block_M, block_N, block_K,
num_stages, thread_num`` [+ ``split_k``], gemm.py:40-47) plus the gfx950
template parameters ``waves_m, waves_n, mfma``.  Each raw config maps to
exactly one compiled instance of libicpp_hip.so (plus a split-K factor), so
"compile" is an index lookup.
"""

from __future__ import annotations

import functools
from typing import Any, Dict, List, Optional, Sequence, Tuple

from ..autotuner.cost_model import TuneConfig
from ..autotuner.gpu_spec import GPUSpec
from ..autotuner.interface import TileLangKernelBase
from ..autotuner.search_space import prune_for_shape
from ..instances import ESZ, FAMILY_ID, INSTANCES, MFMA_K, Inst


@functools.lru_cache(maxsize=None)
def family_instances(family: str) -> Tuple[Inst, ...]:
    """Instances of a family in library index order (the ABI sorts by name)."""
    return tuple(sorted((i for i in INSTANCES if i.family == family), key=lambda i: i.name))


def raw_from_inst(inst: Inst, split_k: Optional[int] = None) -> Dict[str, Any]:
    raw = {
        "block_M": inst.bm, "block_N": inst.bn, "block_K": inst.bk,
        "num_stages": inst.stages, "thread_num": inst.threads,
        "waves_m": inst.wm, "waves_n": inst.wn,
        "mfma": f"{inst.mf}x{inst.mf}x{MFMA_K[(inst.dtype, inst.mf)]}",
    }
    if split_k is not None:
        raw["split_k"] = split_k
    if inst.sched:
        raw["sched"] = inst.sched
    return raw


class InstanceDescriptor(TileLangKernelBase):
    """Descriptor whose candidate space is the compiled instance set of one family/dtype."""

    family: str = "gemm"
    dtype: str = "f16"
    split_k_values: Sequence[int] = (1,)

    def __init__(self, dtype: Optional[str] = None):
        if dtype is not None:
            self.dtype = dtype

    # ---- instance mapping --------------------------------------------------
    def instances(self) -> List[Inst]:
        return [i for i in family_instances(self.family) if i.dtype == self.dtype]

    def instance_index(self, raw: Dict[str, Any]) -> int:
        mf = int(str(raw["mfma"]).split("x")[0]) if "mfma" in raw else None
        for idx, inst in enumerate(family_instances(self.family)):
            if inst.dtype != self.dtype:
                continue
            if (inst.bm, inst.bn, inst.bk, inst.stages, inst.threads) != (
                    raw["block_M"], raw["block_N"], raw["block_K"], raw["num_stages"], raw["thread_num"]):
                continue
            if "waves_m" in raw and (inst.wm, inst.wn) != (raw["waves_m"], raw["waves_n"]):
                continue
            if mf is not None and inst.mf != mf:
                continue
            if inst.sched != raw.get("sched", ""):
                continue
            return idx
        raise KeyError(f"{self.name}: no compiled {self.family}/{self.dtype} instance for {self.format_config(raw)}")

    def instance_of(self, raw: Dict[str, Any]) -> Inst:
        return family_instances(self.family)[self.instance_index(raw)]

    # ---- descriptor API ----------------------------------------------------
    def k_extent(self, **shape) -> int:
        return shape["K"]

    def shape_ok(self, inst: Inst, split_k: int, **shape) -> bool:
        """K a whole number of tiles, and split_k slices of ceil(tiles / split_k)
        tiles each are all non-empty (the launcher's split plan uses exactly
        split_k slices), so distinct split_k values are distinct launches."""
        k = self.k_extent(**shape)
        if k % inst.bk:
            return False
        nkt = k // inst.bk
        if split_k > nkt:
            return False
        per = -(-nkt // split_k)
        return -(-nkt // per) == split_k

    def get_raw_configs(self, **shape_kwargs: Any) -> List[Dict[str, Any]]:
        out = []
        for inst in self.instances():
            for sk in self.split_k_values:
                if self.shape_ok(inst, sk, **shape_kwargs):
                    out.append(raw_from_inst(inst, sk if len(self.split_k_values) > 1 or sk != 1 else None))
        return self._drop_row_waste(out, **shape_kwargs)

    def _drop_row_waste(self, configs: List[Dict[str, Any]], **shape_kwargs: Any) -> List[Dict[str, Any]]:
        """Tiles of 8x or more the problem's rows (rounded up to 16) are not offered
        while a shorter tile is: 7/8 of their MFMA rows are padding.  At fp8 M = 16 the
        128-row tile tied or trailed the 16-row tiles with 3-4 stages (4096^2: 10.48 vs
        9.43 us; K = 11008: 15.88 vs 15.76; N = 11008: 21.9 vs 15.1 for 64 rows); on every
        profiled database shape the best tile is under this bound."""
        try:
            M, _ = self.gemm_mn(**shape_kwargs)
        except (KeyError, TypeError):
            return configs
        if not M or M <= 0:
            return configs
        limit = 8 * (-(-M // 16) * 16)
        kept = [c for c in configs if c["block_M"] < limit]
        return kept if kept else configs

    def raw_config_to_tune_config(self, raw: Dict[str, Any]) -> TuneConfig:
        e = ESZ[self.dtype]
        try:
            vgprs = instance_vgprs(self.instance_of(raw))
        except KeyError:
            vgprs = 0
        return TuneConfig(
            block_M=raw["block_M"], block_N=raw["block_N"], block_K=raw["block_K"],
            num_stages=raw["num_stages"], num_warps=raw["thread_num"] // 64, warp_size=64,
            a_bytes=e, b_bytes=e, mfma=raw.get("mfma", ""), waves_m=raw.get("waves_m", 0),
            waves_n=raw.get("waves_n", 0), split_k=raw.get("split_k", 1), vgprs=vgprs)

    def schedule_factor(self, raw: Dict[str, Any]) -> float:
        """The ping-pong mainloop measured 2-8% faster than its default-schedule twin
        on 4096^3 - 8192^3 bf16 (same tile, bit-identical results)."""
        return 1.03 if raw.get("sched") == "pp" else 1.0

    def gemm_mn(self, **shape) -> tuple:
        return shape["M"], shape["N"]

    def prune(self, raw_configs: List[Dict[str, Any]], hw: GPUSpec, **shape_kwargs: Any) -> List[Dict[str, Any]]:
        """CDNA4 L1-L4 pruning (LDS, VGPR, occupancy, CU fill) on the compiled set."""
        if not hw.has_mfma_model:
            return raw_configs
        M, N = self.gemm_mn(**shape_kwargs)
        cfgs = [self.raw_config_to_tune_config(r) for r in raw_configs]
        keep = set(id(c) for c in prune_for_shape(cfgs, hw, M, N))
        return [r for r, c in zip(raw_configs, cfgs) if id(c) in keep]


__all__ = ["InstanceDescriptor", "family_instances", "raw_from_inst"]


def compiled_resources(inst: Inst) -> Dict[str, int]:
    """Compiler-reported registers of an instance (empty when the library is not built)."""
    from .._lib import resources

    return resources().get(inst.name, {})


def instance_vgprs(inst: Inst) -> int:
    """Registers per lane (VGPRs rounded to the allocation granule + AGPRs).  An
    instance that spilled to scratch needed more than the register file held:
    it reports the whole file plus one, so the L2 register prune rejects it."""
    r = compiled_resources(inst)
    if not r:
        return 0
    if r.get("scratch", 0) > 0:
        return 513
    return -(-(r.get("vgprs", 0)) // 8) * 8 + r.get("agprs", 0)
