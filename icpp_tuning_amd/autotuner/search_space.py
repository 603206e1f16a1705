"""Search-space initialisation and hardware pruning.

Restates the reference's search_space.py (parameter pools, LCM marginal
sampling, three-level pruning, cold / structure / warm initialisation, shape
samplers) with its defects fixed -- ``generate_exhaustive_configs`` called a
``TuneConfig.is_valid_for_backend`` that does not exist (reference :194), and
nothing on the select path used the module -- and adds the CDNA4 pruning the
gfx950 descriptors apply before ranking:

  L1  LDS:       (BM*BK*a_bytes + BK*BN*b_bytes) * stages <= 160 KiB
  L2  VGPRs:     accumulators + fragments + staging <= 512 / waves-per-SIMD
                 (or the compiler-reported VGPR+AGPR count of an AOT instance)
  L3  occupancy: at least one wave per SIMD
  L4  CU fill:   for a given shape, reject tiles whose grid reaches less than
                 half of the best achievable fraction of the 256 CUs
"""

from __future__ import annotations

import math
import random
from collections import defaultdict
from dataclasses import replace
from typing import Dict, Iterable, List, Optional

from .cost_model import TuneConfig, _estimate_occupancy, _resident_blocks_per_sm
from .gpu_spec import GPUSpec

# ---------------------------------------------------------------------------
# Parameter pools
# ---------------------------------------------------------------------------

# reference pools (search_space.py:32-66)
_TRITON_MATMUL_PARAMS = {"block_M": [32, 64, 128], "block_N": [32, 64, 128, 256], "block_K": [32, 64],
                         "num_stages": [2, 3, 4, 5], "num_warps": [2, 4, 8]}
_TILELANG_MATMUL_PARAMS = {"block_M": [32, 48, 64, 80, 96, 112, 128], "block_N": [64, 128, 256],
                           "block_K": [32, 64], "num_stages": [2, 3, 4], "num_warps": [4, 8]}
_TRITON_CONV2D_PARAMS = {"block_M": [32, 64, 128], "block_N": [32, 64, 128], "block_K": [16, 32, 64],
                         "num_stages": [2, 3, 4, 5], "num_warps": [2, 4, 8]}
_TILELANG_CONV2D_PARAMS = {"block_M": [32, 48, 64, 96, 128], "block_N": [32, 64, 128], "block_K": [16, 32, 64],
                           "num_stages": [2, 3, 4], "num_warps": [4, 8]}
# gfx950 MFMA templates (csrc/icpp_kernels.hpp): power-of-two tiles, 1-2 LDS
# stages, 4 or 8 waves, 16x16 or 32x32 MFMA.
_HIP_MATMUL_PARAMS = {"block_M": [16, 32, 64, 128, 256], "block_N": [64, 128, 256], "block_K": [32, 64, 128],
                      "num_stages": [1, 2], "num_warps": [4, 8], "mfma": [16, 32]}
_HIP_CONV2D_PARAMS = {"block_M": [64, 128, 256], "block_N": [64, 128, 256], "block_K": [32, 64],
                      "num_stages": [1, 2], "num_warps": [4, 8], "mfma": [16, 32]}

MIN_OCCUPANCY_THRESHOLD = 0.2
CDNA4_MIN_WAVES_PER_SIMD = 1
CU_FILL_RELATIVE = 0.5


def _get_param_pools(op_type: str, backend: str) -> Dict[str, List[int]]:
    table = {
        ("matmul", "triton"): _TRITON_MATMUL_PARAMS, ("matmul", "tilelang"): _TILELANG_MATMUL_PARAMS,
        ("conv2d", "triton"): _TRITON_CONV2D_PARAMS, ("conv2d", "tilelang"): _TILELANG_CONV2D_PARAMS,
        ("matmul", "hip"): _HIP_MATMUL_PARAMS, ("conv2d", "hip"): _HIP_CONV2D_PARAMS,
    }
    if (op_type, backend) not in table:
        raise ValueError(f"Unsupported op_type/backend: {op_type}/{backend}")
    return {k: list(v) for k, v in table[(op_type, backend)].items()}


# ---------------------------------------------------------------------------
# LCM marginal-stratified sampling (reference :86-156)
# ---------------------------------------------------------------------------


def _lcm(a: int, b: int) -> int:
    return abs(a * b) // math.gcd(a, b)


def _multi_lcm(values: List[int]) -> int:
    out = values[0]
    for v in values[1:]:
        out = _lcm(out, v)
    return out


def lcm_marginal_sample(param_pools: Dict[str, List[int]], n_samples: Optional[int] = None,
                        seed: Optional[int] = None) -> List[Dict[str, int]]:
    """Each pool is repeated to a common length (a multiple of every pool size),
    shuffled independently and zipped, so every value of every parameter occurs
    equally often when ``n_samples`` is the LCM of the pool sizes."""
    rng = random.Random(seed)
    names = list(param_pools)
    L = _multi_lcm([len(param_pools[n]) for n in names])
    n = L if n_samples is None else n_samples
    length = max(L, n)
    columns = {}
    for name in names:
        pool = param_pools[name]
        col = (pool * math.ceil(length / len(pool)))[:length]
        rng.shuffle(col)
        columns[name] = col
    return [{name: columns[name][i] for name in names} for i in range(n)]


def _dict_to_tuneconfig(d: Dict[str, int]) -> TuneConfig:
    return TuneConfig(block_M=d["block_M"], block_N=d["block_N"], block_K=d["block_K"],
                      num_stages=d["num_stages"], num_warps=d["num_warps"])


# ---------------------------------------------------------------------------
# Exhaustive enumeration
# ---------------------------------------------------------------------------


def is_valid_for_backend(cfg: TuneConfig, backend: str) -> bool:
    """Structural validity of a tile for a code generator.

    tilelang: tile dims multiples of 16; triton: powers of two >= 16; hip: the
    gfx950 template constraints (wave grid divides the tile, MFMA tile divides
    the wave tile, BK a multiple of the MFMA K, B rows >= 128 bytes)."""
    dims = (cfg.block_M, cfg.block_N, cfg.block_K)
    if backend == "tilelang":
        return all(d % 16 == 0 for d in dims)
    if backend == "triton":
        return all(d >= 16 and d & (d - 1) == 0 for d in dims)
    if backend == "hip":
        wm, wn = cfg.wave_grid()
        mf, kf = cfg.mfma_dims()
        if cfg.block_M % wm or cfg.block_N % wn:
            return False
        if (cfg.block_M // wm) % mf or (cfg.block_N // wn) % mf:
            return False
        if cfg.block_K % kf or cfg.block_N * cfg.b_bytes < 128 or cfg.block_K * cfg.a_bytes < 32:
            return False
        return True
    raise ValueError(f"unknown backend {backend}")


def _hip_wave_grid(bm: int, bn: int, waves: int, mf: int):
    """Wave grid the gfx950 templates use for a tile: as square as the tile allows."""
    best = None
    wm = 1
    while wm <= waves:
        wn = waves // wm
        if wm * wn == waves and bm % (wm * mf) == 0 and bn % (wn * mf) == 0:
            cand = (abs(math.log2((bm / wm) / (bn / wn))), wm, wn)
            if best is None or cand < best:
                best = cand
        wm *= 2
    return (best[1], best[2]) if best else (0, 0)


def generate_exhaustive_configs(op_type: str = "matmul", backend: str = "tilelang",
                                dtype: str = "f16") -> List[TuneConfig]:
    pools = _get_param_pools(op_type, backend)
    esz = 1 if dtype == "fp8" else 2
    out = []
    for bm in pools["block_M"]:
        for bn in pools["block_N"]:
            for bk in pools["block_K"]:
                for ns in pools["num_stages"]:
                    for nw in pools["num_warps"]:
                        if backend != "hip":
                            cfg = TuneConfig(block_M=bm, block_N=bn, block_K=bk, num_stages=ns, num_warps=nw)
                            if is_valid_for_backend(cfg, backend):
                                out.append(cfg)
                            continue
                        for mf in pools["mfma"]:
                            wm, wn = _hip_wave_grid(bm, bn, nw, mf)
                            if not wm:
                                continue
                            kf = {2: {16: 32, 32: 16}, 1: {16: 128, 32: 64}}[esz][mf]
                            cfg = TuneConfig(block_M=bm, block_N=bn, block_K=bk, num_stages=ns, num_warps=nw,
                                             warp_size=64, a_bytes=esz, b_bytes=esz, mfma=f"{mf}x{mf}x{kf}",
                                             waves_m=wm, waves_n=wn)
                            if is_valid_for_backend(cfg, backend):
                                out.append(cfg)
    return out


# ---------------------------------------------------------------------------
# Pruning
# ---------------------------------------------------------------------------


def estimate_occupancy(config: TuneConfig, hw: GPUSpec) -> float:
    """Fraction of a CU's wave slots held by resident workgroups (reference :208-232)."""
    return _estimate_occupancy(config, hw)


def prune_shared_memory(configs: List[TuneConfig], hw: GPUSpec) -> List[TuneConfig]:
    """L1: tile footprint must fit the per-workgroup LDS / shared-memory limit."""
    return [c for c in configs if c.shared_mem_bytes <= hw.shared_mem_per_block]


def _vgpr_budget(c: TuneConfig, hw: GPUSpec) -> int:
    waves_per_simd = max(1, -(-c.num_warps // hw.simds_per_cu))
    return hw.vgprs_per_lane_max // waves_per_simd


def prune_register_pressure(configs: List[TuneConfig], hw: GPUSpec) -> List[TuneConfig]:
    """L2: register demand within the per-block (NVIDIA) or per-lane (CDNA4) budget."""
    if hw.has_mfma_model:
        return [c for c in configs if c.vgpr_estimate() <= _vgpr_budget(c, hw)]
    return [c for c in configs if c.regs_per_thread_estimate * c.threads <= hw.max_regs_per_block]


def prune_minimum_occupancy(configs: List[TuneConfig], hw: GPUSpec,
                            min_occupancy: Optional[float] = None) -> List[TuneConfig]:
    """L3: thread limits, then a minimum theoretical occupancy (0.2 of the SM for
    the reference; one wave per SIMD on CDNA4)."""
    if min_occupancy is None:
        min_occupancy = (CDNA4_MIN_WAVES_PER_SIMD * hw.simds_per_cu / hw.max_warps_per_sm
                         if hw.has_mfma_model else MIN_OCCUPANCY_THRESHOLD)
    out = []
    for c in configs:
        if c.threads > hw.max_threads_per_block or c.threads > hw.max_threads_per_sm:
            continue
        if c.shared_mem_bytes > hw.shared_mem_per_sm:
            continue
        if estimate_occupancy(c, hw) < min_occupancy - 1e-12:
            continue
        out.append(c)
    return out


def grid_size(c: TuneConfig, M: int, N: int) -> int:
    return -(-M // c.block_M) * -(-N // c.block_N) * max(1, c.split_k)


def prune_cu_underfill(configs: List[TuneConfig], hw: GPUSpec, M: int, N: int,
                       relative: float = CU_FILL_RELATIVE) -> List[TuneConfig]:
    """L4 (shape-aware): drop tiles whose launch fills less than ``relative`` of the
    best CU fill any candidate reaches for this (M, N)."""
    if not configs:
        return configs
    fill = [min(1.0, grid_size(c, M, N) / hw.num_sm) for c in configs]
    best = max(fill)
    return [c for c, f in zip(configs, fill) if f >= relative * best - 1e-12]


def prune_configs(configs: List[TuneConfig], hw: GPUSpec) -> List[TuneConfig]:
    """L1 -> L2 -> L3 (reference :281-286)."""
    return prune_minimum_occupancy(prune_register_pressure(prune_shared_memory(configs, hw), hw), hw)


def prune_for_shape(configs: List[TuneConfig], hw: GPUSpec, M: int, N: int) -> List[TuneConfig]:
    """L1 -> L2 -> L3 -> L4 for one GEMM-shaped problem."""
    return prune_cu_underfill(prune_configs(configs, hw), hw, M, N)


# ---------------------------------------------------------------------------
# Initialisation modes (reference :293-596)
# ---------------------------------------------------------------------------


def _key(c: TuneConfig):
    return (c.block_M, c.block_N, c.block_K, c.num_stages, c.num_warps, c.mfma, c.waves_m, c.waves_n)


def _stratified_sample_from_valid(valid_configs: List[TuneConfig], n_samples: Optional[int] = None,
                                  seed: int = 42) -> List[TuneConfig]:
    """Round-robin over block_M strata (shuffled within each), then fill from the rest.

    Target size defaults to min(max(2 * LCM(pool sizes), 30), |valid|)."""
    if not valid_configs:
        return []
    rng = random.Random(seed)
    pools = [sorted({getattr(c, f) for c in valid_configs})
             for f in ("block_M", "block_N", "block_K", "num_stages", "num_warps")]
    lcm_size = _multi_lcm([len(p) for p in pools])
    target = max(2 * lcm_size, 30)
    n = min(target if n_samples is None else n_samples, len(valid_configs))
    if n >= len(valid_configs):
        out = list(valid_configs)
        rng.shuffle(out)
        return out
    strata: Dict[int, List[TuneConfig]] = defaultdict(list)
    for c in valid_configs:
        strata[c.block_M].append(c)
    for k in strata:
        rng.shuffle(strata[k])
    order = sorted(strata)
    cursor = {k: 0 for k in order}
    picked: List[TuneConfig] = []
    seen = set()
    while len(picked) < n:
        progress = False
        for k in order:
            if len(picked) >= n:
                break
            bucket = strata[k]
            while cursor[k] < len(bucket):
                c = bucket[cursor[k]]
                cursor[k] += 1
                if _key(c) not in seen:
                    picked.append(c)
                    seen.add(_key(c))
                    progress = True
                    break
        if not progress:
            break
    if len(picked) < n:
        rest = [c for c in valid_configs if _key(c) not in seen]
        rng.shuffle(rest)
        picked.extend(rest[: n - len(picked)])
    return picked


def cold_start_configs(op_type: str, backend: str, hw: GPUSpec, n_samples: Optional[int] = None,
                       seed: int = 42, dtype: str = "f16") -> List[TuneConfig]:
    valid = prune_configs(generate_exhaustive_configs(op_type, backend, dtype), hw)
    return _stratified_sample_from_valid(valid, n_samples, seed) if valid else []


def structure_aware_cold_start_configs(valid_configs: List[TuneConfig], hw: GPUSpec,
                                       n_samples: Optional[int] = None, seed: int = 42) -> List[TuneConfig]:
    pruned = prune_configs(list(valid_configs), hw) if valid_configs else []
    return _stratified_sample_from_valid(pruned, n_samples, seed) if pruned else []


def warm_start_configs(top_k_configs: List[TuneConfig], op_type: str, backend: str, hw: GPUSpec,
                       n_explore: Optional[int] = None, seed: int = 42, dtype: str = "f16") -> List[TuneConfig]:
    if n_explore is None:
        n_explore = max(len(top_k_configs), 10)
    exploit = prune_configs(list(top_k_configs), hw)
    explore = cold_start_configs(op_type, backend, hw, n_samples=n_explore * 2, seed=seed, dtype=dtype)
    seen = {_key(c) for c in exploit}
    merged = list(exploit)
    for c in explore:
        if _key(c) in seen:
            continue
        seen.add(_key(c))
        merged.append(c)
        if len(merged) >= len(exploit) + n_explore:
            break
    return merged


def generate_search_space(op_type: str, hw: GPUSpec, backend: str = "tilelang", mode: str = "exhaustive",
                          n_samples: Optional[int] = None, valid_configs: Optional[List[TuneConfig]] = None,
                          top_k_configs: Optional[List[TuneConfig]] = None, seed: int = 42,
                          dtype: str = "f16") -> List[TuneConfig]:
    if mode == "exhaustive":
        return prune_configs(generate_exhaustive_configs(op_type, backend, dtype), hw)
    if mode == "cold":
        return cold_start_configs(op_type, backend, hw, n_samples, seed, dtype)
    if mode == "structure":
        if valid_configs is None:
            raise ValueError("mode='structure' requires valid_configs")
        return structure_aware_cold_start_configs(valid_configs, hw, n_samples, seed)
    if mode == "warm":
        if top_k_configs is None:
            raise ValueError("mode='warm' requires top_k_configs")
        return warm_start_configs(top_k_configs, op_type, backend, hw, n_samples, seed, dtype)
    raise ValueError(f"Unsupported mode: {mode}")


# ---------------------------------------------------------------------------
# Shape samplers for offline profiling (reference :603-664)
# ---------------------------------------------------------------------------


def generate_matmul_sample_shapes(M_range=(1, 4096), N_values: Optional[Iterable[int]] = None,
                                  K_values: Optional[Iterable[int]] = None) -> List[dict]:
    """Dense small-M sampling (1..16, step 16 to 128, 64 to 1024, 256 to 4096)."""
    N_values = [768, 2304, 4096] if N_values is None else list(N_values)
    K_values = [768, 2304, 4096] if K_values is None else list(K_values)
    ms = set(range(1, 17)) | set(range(16, 129, 16)) | set(range(128, 1025, 64))
    ms |= set(range(1024, min(M_range[1] + 1, 4097), 256))
    ms = sorted(m for m in ms if M_range[0] <= m <= M_range[1])
    return [{"M": m, "N": n, "K": k} for m in ms for n in N_values for k in K_values]


def generate_conv2d_sample_shapes(N_values=None, HW_values=None, C_values=None, OC_values=None) -> List[dict]:
    N_values = [1, 2, 4, 8, 16, 32] if N_values is None else N_values
    HW_values = [7, 14, 28, 56, 112, 224] if HW_values is None else HW_values
    C_values = [64, 128, 256, 512] if C_values is None else C_values
    OC_values = [64, 128, 256, 512] if OC_values is None else OC_values
    return [{"N": n, "C": c, "H": s, "W": s, "OC": oc, "KH": 3, "KW": 3, "stride": 1, "padding": 1}
            for n in N_values for s in HW_values for c in C_values for oc in OC_values]


def search_space_summary(op_type: str, hw: GPUSpec, backend: str = "tilelang", mode: str = "exhaustive",
                         dtype: str = "f16", **kwargs) -> dict:
    full = generate_exhaustive_configs(op_type, backend, dtype)
    l1 = prune_shared_memory(full, hw)
    l2 = prune_register_pressure(l1, hw)
    l3 = prune_minimum_occupancy(l2, hw)
    mode_cfgs = generate_search_space(op_type, hw, backend, mode=mode, dtype=dtype, **kwargs)
    occ = [estimate_occupancy(c, hw) for c in l3]
    return {
        "op_type": op_type, "backend": backend, "mode": mode,
        "exhaustive_full": len(full), "after_smem_prune": len(l1), "after_reg_prune": len(l2),
        "after_occupancy_prune": len(l3),
        "min_occupancy_threshold": (CDNA4_MIN_WAVES_PER_SIMD * hw.simds_per_cu / hw.max_warps_per_sm
                                    if hw.has_mfma_model else MIN_OCCUPANCY_THRESHOLD),
        "avg_occupancy": round(sum(occ) / len(occ), 3) if occ else 0,
        "mode_output_size": len(mode_cfgs),
        "pruning_ratio": round(1 - len(l3) / len(full), 3) if full else 0,
    }


__all__ = [
    "CU_FILL_RELATIVE", "MIN_OCCUPANCY_THRESHOLD", "cold_start_configs", "estimate_occupancy",
    "generate_conv2d_sample_shapes", "generate_exhaustive_configs", "generate_matmul_sample_shapes",
    "generate_search_space", "grid_size", "is_valid_for_backend", "lcm_marginal_sample", "prune_configs",
    "prune_cu_underfill", "prune_for_shape", "prune_minimum_occupancy", "prune_register_pressure",
    "prune_shared_memory", "search_space_summary", "structure_aware_cold_start_configs", "warm_start_configs",
]
