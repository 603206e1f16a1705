"""Trait-driven analytical cost model, re-targeted to CDNA4.

The reference scores a candidate tile configuration with a closed-form product
of efficiency factors (kernel/autotuner/cost_model.py:765-775).  This module
keeps that contract -- same dataclasses, same builder functions, same factor
functions, same ``score_formula`` -- so that descriptors written for the
reference work unchanged, and so the published A100 scores can be reproduced
(reference mode, ``GPUSpec.has_mfma_model == False``: every formula below
reduces exactly to the reference's).

On a spec that carries an MFMA model (MI355X) ``score_formula`` is instead
the predicted fraction of dense MFMA peak of one launch, from a per-CU
schedule model (``predict_schedule``): rounds of co-resident workgroups, per
K step the largest of MFMA issue, LDS traffic and L2 feed, or the memory
latency over the prefetch depth; the epilogue's stores and FLOPs; the HBM
floor; and the split-K reduction launch.  Threads are waves x 64, LDS bytes
use each operand's element size (fp8 = 1), residency is limited per SIMD (8
waves, 512 registers per lane) with the compiler's register counts.  The
descriptors' split-K adjustments of the reference are part of that model.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Any, Dict, Iterable, List, Literal, Optional, Sequence, Tuple

from .gpu_spec import GPUSpec

ReductionAxis = Literal["none", "m", "n", "k", "spatial", "channel"]
MainloopKind = Literal["gemm", "implicit_gemm_conv"]


# ---------------------------------------------------------------------------
# Operator description (reference cost_model.py:52-152)
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class FusionPrimitive:
    """Epilogue / side-reduction primitive described by execution traits."""

    name: str
    flops_per_output: float
    bytes_per_output: float = 0.0
    reduction_axis: ReductionAxis = "none"
    extra_passes: int = 0
    sync_penalty: float = 0.0
    preferred_outputs_per_thread: float = 16.0
    preferred_tile_m: Optional[float] = None
    preferred_tile_n: Optional[float] = None
    smem_bytes_per_output: float = 0.0

    @property
    def has_reduction(self) -> bool:
        return self.reduction_axis != "none"

    @property
    def work_units(self) -> float:
        return max(1.0, self.flops_per_output + self.bytes_per_output)


@dataclass(frozen=True)
class MainloopSpec:
    """Dominant tiled compute structure (GEMM or implicit-GEMM conv)."""

    kind: MainloopKind
    M: int
    N: int
    K: int
    input_elements: int
    weight_elements: int
    output_elements: int
    input_element_bytes: int = 2
    weight_element_bytes: int = 2
    output_element_bytes: int = 2
    accum_element_bytes: int = 4
    flops_per_fma: int = 2
    input_reuse_hint: float = 1.0
    weight_reuse_hint: float = 1.0
    spatial_reuse_hint: float = 1.0
    preferred_group_m: int = 8
    dtype: str = "f16"

    @property
    def mainloop_flops(self) -> int:
        return self.flops_per_fma * self.M * self.N * self.K

    @property
    def min_global_bytes(self) -> int:
        return (self.input_elements * self.input_element_bytes
                + self.weight_elements * self.weight_element_bytes
                + self.output_elements * self.output_element_bytes)


@dataclass(frozen=True)
class OpSpec:
    name: str
    mainloop: MainloopSpec
    epilogue: Tuple[FusionPrimitive, ...] = field(default_factory=tuple)

    @property
    def M(self) -> int:
        return self.mainloop.M

    @property
    def N(self) -> int:
        return self.mainloop.N

    @property
    def K(self) -> int:
        return self.mainloop.K

    @property
    def flops(self) -> float:
        per_out = sum(p.flops_per_output for p in self.epilogue)
        return float(self.mainloop.mainloop_flops + self.M * self.N * per_out)

    @property
    def bytes_accessed(self) -> float:
        per_out = sum(p.bytes_per_output for p in self.epilogue)
        return float(self.mainloop.min_global_bytes + self.M * self.N * per_out)

    @property
    def arithmetic_intensity(self) -> float:
        b = self.bytes_accessed
        return self.flops / b if b > 0 else 0.0

    @property
    def has_reduction_epilogue(self) -> bool:
        return any(p.has_reduction for p in self.epilogue)


@dataclass(frozen=True)
class TuneConfig:
    """Candidate tile configuration.

    Reference fields first (cost_model.py:154-178); the trailing fields default
    to the reference's implicit assumptions (32-lane warps, 2-byte operands) and
    carry the CDNA4 specifics when a descriptor targets gfx950.
    """

    block_M: int
    block_N: int
    block_K: int
    num_stages: int
    num_warps: int
    group_size_m: int = 8
    warp_size: int = 32
    a_bytes: int = 2
    b_bytes: int = 2
    mfma: str = ""          # "16x16x32", "32x32x16", "16x16x128", "32x32x64"
    waves_m: int = 0        # wave grid inside the workgroup (0: unspecified)
    waves_n: int = 0
    split_k: int = 1
    vgprs: int = 0          # compiler-reported VGPR+AGPR count of an AOT instance (0: estimate)

    @property
    def threads(self) -> int:
        return self.num_warps * self.warp_size

    @property
    def shared_mem_bytes(self) -> int:
        a_tile = self.block_M * self.block_K * self.a_bytes
        b_tile = self.block_K * self.block_N * self.b_bytes
        return (a_tile + b_tile) * self.num_stages

    @property
    def regs_per_thread_estimate(self) -> int:
        acc_elements = (self.block_M * self.block_N) // max(1, self.threads)
        return acc_elements * 2 + 40

    # ---- CDNA4 register model -------------------------------------------------
    def mfma_dims(self) -> Tuple[int, int]:
        if not self.mfma:
            return (16, 32 if self.a_bytes == 2 else 128)
        m, _, k = (int(x) for x in self.mfma.split("x"))
        return m, k

    def wave_grid(self) -> Tuple[int, int]:
        if self.waves_m and self.waves_n:
            return self.waves_m, self.waves_n
        wm = 1
        while wm * wm < self.num_warps:
            wm *= 2
        wm = min(wm, self.num_warps)
        return wm, self.num_warps // wm

    def vgpr_estimate(self) -> int:
        """32-bit registers per lane for the MFMA templates in csrc/.

        accumulators (fp32, BM*BN spread over the workgroup's lanes)
        + A/B fragments for one MFMA k-step (16 B per lane per tile, 32 B for fp8)
        + global->LDS staging (the tile's bytes spread over the lanes)
        + ~24 registers of addressing / loop state.
        An AOT instance carries the count its compiler reported instead.
        """
        if self.vgprs:
            return self.vgprs
        lanes = max(1, self.threads)
        acc = (self.block_M * self.block_N) // lanes
        mf, _ = self.mfma_dims()
        wm, wn = self.wave_grid()
        tm = max(1, self.block_M // max(1, wm) // mf)
        tn = max(1, self.block_N // max(1, wn) // mf)
        frag_dw = 4 if self.a_bytes == 2 else 8
        frags = (tm + tn) * frag_dw
        staging = (self.block_M * self.block_K * self.a_bytes
                   + self.block_K * self.block_N * self.b_bytes) // (4 * lanes)
        return acc + frags + staging + 24


@dataclass(frozen=True)
class ConfigProjection:
    tiles_M: int
    tiles_N: int
    tiles_K: int
    grid_size: int
    tile_outputs: int
    outputs_per_thread: float
    mainloop_iterations: int
    mainloop_flops_per_tile: float
    epilogue_flops_per_tile: float
    total_flops_per_tile: float
    input_bytes_per_tile: float
    weight_bytes_per_tile: float
    output_bytes_per_tile: float
    epilogue_bytes_per_tile: float
    total_global_bytes_per_tile: float
    shared_mem_bytes_per_tile: float
    tile_arithmetic_intensity: float
    occupancy: float
    resident_blocks_per_sm: int
    wave_fill: float
    preferred_num_stages: int
    reduction_work: float
    reduction_passes: int
    epilogue_preferred_outputs: float


# ---------------------------------------------------------------------------
# Primitive library (reference cost_model.py:220-273; same trait values)
# ---------------------------------------------------------------------------

BIAS_ADD = FusionPrimitive("bias_add", 1.0, 0.0, preferred_outputs_per_thread=16.0)
RELU = FusionPrimitive("relu", 1.0, 0.0, preferred_outputs_per_thread=16.0)
SILU = FusionPrimitive("silu", 4.0, 0.0, preferred_outputs_per_thread=12.0)
GELU = FusionPrimitive("gelu", 8.0, 0.0, preferred_outputs_per_thread=8.0)
ROW_LAYERNORM = FusionPrimitive(
    "row_layernorm", 10.0, 4.0, reduction_axis="n", extra_passes=1, sync_penalty=0.35,
    preferred_outputs_per_thread=8.0, preferred_tile_n=128.0)
BATCHNORM = FusionPrimitive(
    "batchnorm", 6.0, 2.0, reduction_axis="channel", extra_passes=1, sync_penalty=0.25,
    preferred_outputs_per_thread=12.0, preferred_tile_n=128.0)

PRIMITIVE_LIBRARY: Dict[str, FusionPrimitive] = {
    p.name: p for p in (BIAS_ADD, RELU, SILU, GELU, ROW_LAYERNORM, BATCHNORM)
}
# activation name used by the kernel ABI -> primitive name used by the scorer
ACT_PRIMITIVE = {"none": None, "relu": "relu", "gelu_tanh": "gelu", "gelu": "gelu", "silu": "silu",
                 "gelu_erf": "gelu"}


def resolve_primitives(primitives: Iterable) -> Tuple[FusionPrimitive, ...]:
    out: List[FusionPrimitive] = []
    for p in primitives:
        if isinstance(p, FusionPrimitive):
            out.append(p)
        elif p in PRIMITIVE_LIBRARY:
            out.append(PRIMITIVE_LIBRARY[p])
        else:
            raise KeyError(f"Unknown fusion primitive: {p}")
    return tuple(out)


# ---------------------------------------------------------------------------
# Builders (reference cost_model.py:293-364)
# ---------------------------------------------------------------------------

_DTYPE_BYTES = {"f16": 2, "bf16": 2, "fp8": 1, "f32": 4}


def make_matmul_spec(M: int, N: int, K: int, primitives: Sequence = (), *,
                     input_element_bytes: Optional[int] = None,
                     weight_element_bytes: Optional[int] = None,
                     output_element_bytes: int = 2, name: Optional[str] = None,
                     dtype: str = "f16") -> OpSpec:
    ib = _DTYPE_BYTES[dtype] if input_element_bytes is None else input_element_bytes
    wb = _DTYPE_BYTES[dtype] if weight_element_bytes is None else weight_element_bytes
    main = MainloopSpec(
        kind="gemm", M=M, N=N, K=K,
        input_elements=M * K, weight_elements=K * N, output_elements=M * N,
        input_element_bytes=ib, weight_element_bytes=wb, output_element_bytes=output_element_bytes,
        dtype=dtype)
    return OpSpec(name=name or "matmul", mainloop=main, epilogue=resolve_primitives(primitives))


def conv_output_hw(H: int, W: int, KH: int, KW: int, stride: int, padding: int, dilation: int = 1):
    """Output spatial size (reference conv2d.py:65-68)."""
    OH = (H + 2 * padding - dilation * (KH - 1) - 1) // stride + 1
    OW = (W + 2 * padding - dilation * (KW - 1) - 1) // stride + 1
    return OH, OW


def make_conv2d_spec(N: int, C: int, H: int, W: int, OC: int, KH: int, KW: int, *,
                     stride: int = 1, padding: int = 0, primitives: Sequence = (),
                     input_element_bytes: int = 2, weight_element_bytes: int = 2,
                     output_element_bytes: int = 2, name: Optional[str] = None,
                     dtype: str = "f16") -> OpSpec:
    # The reference sizes OH/OW without dilation (cost_model.py:340-341).
    OH = (H + 2 * padding - KH) // stride + 1
    OW = (W + 2 * padding - KW) // stride + 1
    overlap = max(1.0, (KH * KW) / max(1.0, float(stride * stride)))
    main = MainloopSpec(
        kind="implicit_gemm_conv", M=N * OH * OW, N=OC, K=C * KH * KW,
        input_elements=N * C * H * W, weight_elements=OC * C * KH * KW,
        output_elements=N * OC * OH * OW,
        input_element_bytes=input_element_bytes, weight_element_bytes=weight_element_bytes,
        output_element_bytes=output_element_bytes,
        input_reuse_hint=math.sqrt(overlap), weight_reuse_hint=math.sqrt(overlap),
        spatial_reuse_hint=overlap, dtype=dtype)
    return OpSpec(name=name or "conv2d", mainloop=main, epilogue=resolve_primitives(primitives))


# ---------------------------------------------------------------------------
# Model constants: reference values (cost_model.py:372-389) and CDNA4 values
# ---------------------------------------------------------------------------


@dataclass(frozen=True)
class ModelConstants:
    preferred_occupancy: float = 0.5
    occupancy_saturation_exponent: float = 0.15
    wave_fill_exponent: float = 0.35
    high_warp_count_penalty: float = 0.9
    high_warp_free_count: int = 4
    memory_efficiency_exponent: float = 0.75
    pipeline_fill_exponent: float = 0.5
    stage_mismatch_penalty: float = 0.5
    mainloop_target_outputs_per_thread: float = 32.0
    mainloop_min_outputs_per_thread: float = 2.0
    mainloop_output_distance_penalty: float = 0.4
    epilogue_distance_penalty: float = 0.5
    reduction_distance_penalty: float = 0.3
    conv_block_m_distance_penalty: float = 0.45
    conv_block_n_distance_penalty: float = 0.6
    conv_high_warp_penalty: float = 0.94
    conv_plain_spatial_work_penalty: float = 0.18
    conv_plain_block_k_oversize_penalty: float = 0.45
    conv_plain_high_warp_penalty: float = 0.55
    conv_preferred_block_m: Tuple[float, float] = (32.0, 64.0)
    conv_preferred_block_n: Tuple[float, float] = (64.0, 128.0)
    conv_block_k_free: int = 32
    # CDNA4 schedule model (unused in reference mode)
    mfma_rate: Tuple[Tuple[str, float], ...] = ()
    l2_bytes_per_clk_per_cu: float = 0.0
    mem_latency_clk: float = 0.0
    step_overhead_clk: float = 0.0
    tile_overhead_clk: float = 0.0
    store_bytes_per_clk_per_cu: float = 0.0
    epilogue_flops_per_clk_per_cu: float = 0.0
    hbm_efficiency: float = 1.0
    reduce_efficiency: float = 1.0
    launch_overhead_s: float = 0.0


REFERENCE_CONSTANTS = ModelConstants()

# CDNA4 schedule-model constants.  The MFMA rates are relative sustained issue
# rates measured on MI355X with a dependency-free MFMA stream (32x32x16 bf16:
# 1970 TFLOP/s, 16x16x32 bf16: 1711 TFLOP/s; fp8 16x16x128: 4579 TFLOP/s).  The
# other values are effective rates and latencies fitted to the shipped offline
# databases (every compiled config timed at every profiled shape): they are
# what ranks the compiled configs best on those shapes, checked on shapes the
# fit never saw, not independent hardware measurements.
CDNA4_CONSTANTS = ModelConstants(
    mfma_rate=(("16x16x32", 0.87), ("32x32x16", 1.0), ("16x16x128", 1.0), ("32x32x64", 1.0)),
    l2_bytes_per_clk_per_cu=22.5,
    mem_latency_clk=2400.0,
    step_overhead_clk=7.5,
    tile_overhead_clk=3000.0,
    store_bytes_per_clk_per_cu=4.75,
    epilogue_flops_per_clk_per_cu=256.0,
    hbm_efficiency=0.81,
    reduce_efficiency=0.7,
    launch_overhead_s=0.6e-6,
)


def constants_for(hw: GPUSpec) -> ModelConstants:
    return CDNA4_CONSTANTS if hw.has_mfma_model else REFERENCE_CONSTANTS


# ---------------------------------------------------------------------------
# Projection helpers
# ---------------------------------------------------------------------------


def _ceildiv(a: int, b: int) -> int:
    return -(-a // b)


def _resident_blocks_per_sm(config: TuneConfig, hw: GPUSpec) -> int:
    """Workgroups that fit on one CU/SM at once."""
    waves = max(1, config.num_warps)
    by_threads = hw.max_warps_per_sm // waves
    smem = config.shared_mem_bytes
    by_smem = hw.shared_mem_per_sm // smem if smem > 0 else hw.max_blocks_per_sm
    if hw.has_mfma_model:
        # Registers are allocated per SIMD: a wave holding V registers per lane
        # leaves floor(512 / V) wave slots on its SIMD.
        v = config.vgpr_estimate()
        v = -(-v // 8) * 8
        waves_per_simd = min(hw.max_waves_per_simd, hw.vgprs_per_lane_max // max(1, v))
        by_regs = (waves_per_simd * hw.simds_per_cu) // waves
    else:
        regs = config.regs_per_thread_estimate * config.threads
        by_regs = hw.max_regs_per_sm // regs if regs > 0 else hw.max_blocks_per_sm
    return max(0, min(by_threads, by_smem, by_regs, hw.max_blocks_per_sm))


def _estimate_occupancy(config: TuneConfig, hw: GPUSpec) -> float:
    if hw.max_warps_per_sm <= 0:
        return 0.0
    return min(1.0, _resident_blocks_per_sm(config, hw) * config.num_warps / hw.max_warps_per_sm)


def _preferred_block_k(op: OpSpec) -> int:
    K = op.K
    if K >= 64:
        return 64
    if K >= 32:
        return 32
    return 16


def _warp_count_efficiency(config: TuneConfig, c: ModelConstants) -> float:
    if config.num_warps <= c.high_warp_free_count:
        return 1.0
    return c.high_warp_count_penalty ** math.log2(config.num_warps / c.high_warp_free_count)


def _weighted_preferred_outputs(op: OpSpec) -> float:
    if not op.epilogue:
        return 16.0
    total = sum(p.work_units for p in op.epilogue)
    return sum(p.preferred_outputs_per_thread * p.work_units for p in op.epilogue) / total


def _estimate_operand_reuse(op: OpSpec, config: TuneConfig, tiles_M: int) -> Tuple[float, float]:
    group_m = max(1, min(config.group_size_m, max(1, tiles_M)))
    if op.mainloop.kind == "gemm":
        return 1.0, max(1.0, group_m ** 0.5)
    return (max(1.0, op.mainloop.input_reuse_hint),
            max(1.0, (group_m * op.mainloop.weight_reuse_hint) ** 0.5))


def _preferred_num_stages(op: OpSpec, config: TuneConfig, tile_ai: float, hw: GPUSpec) -> int:
    ridge = hw.ridge_point_fp16
    mem_eff = 1.0 if ridge <= 0 else min(1.0, tile_ai / ridge)
    k_iters = max(1, _ceildiv(op.K, config.block_K))
    pref = 2
    if op.mainloop.kind == "implicit_gemm_conv":
        pref += 1
    if mem_eff < 0.9:
        pref += 1
    if mem_eff < 0.5:
        pref += 1
    if op.has_reduction_epilogue:
        pref += 1
    return min(max(2, pref), max(2, min(6, k_iters)))


def project_config(op: OpSpec, config: TuneConfig, hw: GPUSpec) -> ConfigProjection:
    tiles_M = _ceildiv(op.M, config.block_M)
    tiles_N = _ceildiv(op.N, config.block_N)
    tiles_K = _ceildiv(op.K, config.block_K)
    grid = tiles_M * tiles_N * (config.split_k if hw.has_mfma_model else 1)
    tile_outputs = config.block_M * config.block_N
    opt = tile_outputs / max(1, config.threads)

    in_reuse, w_reuse = _estimate_operand_reuse(op, config, tiles_M)
    main_flops = op.mainloop.flops_per_fma * config.block_M * config.block_N * op.K
    epi_flops = tile_outputs * sum(p.flops_per_output for p in op.epilogue)
    tot_flops = main_flops + epi_flops
    in_bytes = op.K * config.block_M * op.mainloop.input_element_bytes / in_reuse
    w_bytes = op.K * config.block_N * op.mainloop.weight_element_bytes / w_reuse
    out_bytes = tile_outputs * op.mainloop.output_element_bytes
    epi_bytes = tile_outputs * sum(p.bytes_per_output for p in op.epilogue)
    gbytes = in_bytes + w_bytes + out_bytes + epi_bytes
    smem = config.shared_mem_bytes + tile_outputs * sum(p.smem_bytes_per_output for p in op.epilogue)
    tile_ai = tot_flops / gbytes if gbytes > 0 else 0.0

    resident = max(1, _resident_blocks_per_sm(config, hw))
    slots = max(1, hw.num_sm * resident)
    waves = max(1, _ceildiv(grid, slots))
    return ConfigProjection(
        tiles_M=tiles_M, tiles_N=tiles_N, tiles_K=tiles_K, grid_size=grid,
        tile_outputs=tile_outputs, outputs_per_thread=opt, mainloop_iterations=max(1, tiles_K),
        mainloop_flops_per_tile=main_flops, epilogue_flops_per_tile=epi_flops,
        total_flops_per_tile=tot_flops, input_bytes_per_tile=in_bytes,
        weight_bytes_per_tile=w_bytes, output_bytes_per_tile=out_bytes,
        epilogue_bytes_per_tile=epi_bytes, total_global_bytes_per_tile=gbytes,
        shared_mem_bytes_per_tile=smem, tile_arithmetic_intensity=tile_ai,
        occupancy=_estimate_occupancy(config, hw), resident_blocks_per_sm=resident,
        wave_fill=grid / (waves * slots),
        preferred_num_stages=_preferred_num_stages(op, config, tile_ai, hw),
        reduction_work=sum(p.work_units for p in op.epilogue if p.has_reduction),
        reduction_passes=sum(p.extra_passes for p in op.epilogue if p.has_reduction),
        epilogue_preferred_outputs=_weighted_preferred_outputs(op),
    )


# ---------------------------------------------------------------------------
# Score factors (reference cost_model.py:544-757)
# ---------------------------------------------------------------------------


def _log2_distance(x: float, target: float) -> float:
    return abs(math.log2(max(1e-6, x / target)))


def eff_mainloop(op: OpSpec, config: TuneConfig, proj: ConfigProjection,
                 hw: Optional[GPUSpec] = None) -> float:
    """Tile padding waste x outputs-per-thread fit x block_K adequacy."""
    c = constants_for(hw) if hw is not None else REFERENCE_CONSTANTS
    padded = (proj.tiles_M * config.block_M) * (proj.tiles_N * config.block_N) * (proj.tiles_K * config.block_K)
    padding_eff = 1.0 if padded == 0 else (op.M * op.N * op.K) / padded
    # Launches that cannot fill the machine want smaller per-thread tiles.
    launch_fill = min(1.0, proj.wave_fill * max(1, proj.resident_blocks_per_sm))
    occ_fill = min(1.0, proj.occupancy / max(c.preferred_occupancy, 1e-6))
    signal = math.sqrt(max(1e-6, launch_fill * occ_fill))
    target = c.mainloop_min_outputs_per_thread + (
        c.mainloop_target_outputs_per_thread - c.mainloop_min_outputs_per_thread) * signal
    thread_eff = 1.0 / (1.0 + c.mainloop_output_distance_penalty * _log2_distance(proj.outputs_per_thread, target))
    k_eff = math.sqrt(min(1.0, config.block_K / _preferred_block_k(op)))
    return padding_eff * thread_eff * k_eff


def eff_memory(op: OpSpec, config: TuneConfig, proj: ConfigProjection, hw: GPUSpec) -> float:
    """Tile arithmetic intensity against the roofline ridge, x LDS footprint."""
    c = constants_for(hw)
    ridge = hw.ridge_point_fp16
    if ridge <= 0:
        return 1.0
    roof = min(1.0, proj.tile_arithmetic_intensity / ridge)
    pressure = min(1.0, proj.shared_mem_bytes_per_tile / max(1.0, float(hw.shared_mem_per_sm)))
    return (roof ** c.memory_efficiency_exponent) / (1.0 + 0.25 * pressure)


def eff_parallel(op: OpSpec, config: TuneConfig, proj: ConfigProjection, hw: GPUSpec) -> float:
    """Occupancy saturation x last-wave fill x wave-count cost."""
    if proj.grid_size == 0 or hw.num_sm == 0:
        return 1.0
    c = constants_for(hw)
    occ = min(1.0, proj.occupancy / c.preferred_occupancy) ** c.occupancy_saturation_exponent
    return occ * (proj.wave_fill ** c.wave_fill_exponent) * _warp_count_efficiency(config, c)


def eff_pipeline(op: OpSpec, config: TuneConfig, proj: ConfigProjection, hw: GPUSpec) -> float:
    """Pipeline prologue cost x distance from the preferred stage count."""
    if config.num_stages <= 0 or proj.mainloop_iterations <= 0:
        return 1.0
    c = constants_for(hw)
    it = proj.mainloop_iterations
    fill = (it / (it + config.num_stages - 1)) ** c.pipeline_fill_exponent
    match = 1.0 / (1.0 + c.stage_mismatch_penalty * abs(config.num_stages - proj.preferred_num_stages))
    return fill * match


def eff_implicit_conv(op: OpSpec, config: TuneConfig, proj: ConfigProjection, hw: GPUSpec) -> float:
    """Gather / address-generation cost of implicit-GEMM convolution."""
    if op.mainloop.kind != "implicit_gemm_conv":
        return 1.0
    overlap = max(1.0, op.mainloop.spatial_reuse_hint)
    if overlap <= 1.0:
        return 1.0
    c = constants_for(hw)
    sig = min(1.5, math.log2(overlap) / math.log2(9.0))
    slots = max(1, hw.num_sm * max(1, proj.resident_blocks_per_sm))
    util = min(1.0, proj.grid_size / slots)
    underfill = 1.0 - util

    spatial_eff = bk_eff = plain_warp_eff = 1.0
    plain = not op.epilogue
    in_channels = op.K / overlap
    if plain and overlap >= 8.5 and (op.N >= 512 or in_channels <= 96.0):
        work = min(1.0, op.mainloop.mainloop_flops / 1.0e10)
        launch = max(0.35, util)
        spatial_eff = 1.0 / (1.0 + c.conv_plain_spatial_work_penalty * sig * work * launch)
        if config.block_K > c.conv_block_k_free:
            bk_eff = 1.0 / (1.0 + c.conv_plain_block_k_oversize_penalty * sig * work
                            * math.log2(config.block_K / float(c.conv_block_k_free)))
        if config.num_warps > c.high_warp_free_count:
            plain_warp_eff = c.conv_plain_high_warp_penalty ** (
                work * math.log2(config.num_warps / float(c.high_warp_free_count)))
    base = spatial_eff * bk_eff * plain_warp_eff
    if underfill <= 0.0:
        return base

    pref_n = c.conv_preferred_block_n[0] if overlap >= 4.0 and underfill >= 0.2 else c.conv_preferred_block_n[1]
    pref_m = c.conv_preferred_block_m[0] if overlap >= 4.0 and underfill >= 0.5 else c.conv_preferred_block_m[1]
    m_eff = 1.0 / (1.0 + c.conv_block_m_distance_penalty * sig * underfill * abs(math.log2(config.block_M / pref_m)))
    n_eff = 1.0 / (1.0 + c.conv_block_n_distance_penalty * sig * underfill * abs(math.log2(config.block_N / pref_n)))
    if overlap >= 4.0 and underfill >= 0.2 and config.num_warps > c.high_warp_free_count:
        warp_eff = c.conv_high_warp_penalty ** math.log2(config.num_warps / float(c.high_warp_free_count))
    else:
        warp_eff = 1.0
    stage_eff = 1.0
    if config.num_stages > 1:
        ridge = hw.ridge_point_fp16
        pressure = 1.0 - min(1.0, proj.tile_arithmetic_intensity / ridge) if ridge > 0 else 0.0
        stage_eff = 1.0 / (1.0 + 0.25 * (config.num_stages - 1) * sig * pressure)
    return m_eff * n_eff * warp_eff * stage_eff * base


def _primitive_efficiency(p: FusionPrimitive, config: TuneConfig, proj: ConfigProjection,
                          c: ModelConstants) -> float:
    eff = 1.0 / (1.0 + c.epilogue_distance_penalty * _log2_distance(proj.outputs_per_thread, p.preferred_outputs_per_thread))
    if p.preferred_tile_m:
        eff /= 1.0 + 0.2 * abs(math.log2(config.block_M / p.preferred_tile_m))
    if p.preferred_tile_n:
        eff /= 1.0 + 0.2 * abs(math.log2(config.block_N / p.preferred_tile_n))
    return eff


def eff_epilogue(op: OpSpec, config: TuneConfig, proj: ConfigProjection,
                 hw: Optional[GPUSpec] = None) -> float:
    """Work-weighted geometric mean of per-primitive fit, scaled by epilogue share."""
    if not op.epilogue:
        return 1.0
    c = constants_for(hw) if hw is not None else REFERENCE_CONSTANTS
    total = sum(p.work_units for p in op.epilogue)
    log_sum = sum((p.work_units / total) * math.log(max(1e-9, _primitive_efficiency(p, config, proj, c)))
                  for p in op.epilogue)
    share = proj.epilogue_flops_per_tile / max(1.0, proj.total_flops_per_tile)
    strength = min(1.0, 0.25 + 4.0 * share)
    if any(p.has_reduction or p.bytes_per_output > 0.0 or p.sync_penalty > 0.0 for p in op.epilogue):
        strength = max(strength, 0.65)
    return math.exp(log_sum * strength)


def eff_reduction(op: OpSpec, config: TuneConfig, proj: ConfigProjection,
                  hw: Optional[GPUSpec] = None) -> float:
    """Geometric mean over reduction primitives of axis-extent x pass x sync costs."""
    reds = [p for p in op.epilogue if p.has_reduction]
    if not reds:
        return 1.0
    c = constants_for(hw) if hw is not None else REFERENCE_CONSTANTS
    prod = 1.0
    for p in reds:
        along_n = p.reduction_axis in ("n", "channel")
        extent = config.block_N if along_n else config.block_M
        pref = p.preferred_tile_n if along_n else p.preferred_tile_m
        if pref is None:
            pref = 128.0 if along_n else 64.0
        prod *= (1.0 / (1.0 + 0.2 * p.extra_passes)) * (1.0 / (1.0 + p.sync_penalty)) * (
            1.0 / (1.0 + c.reduction_distance_penalty * abs(math.log2(extent / pref))))
    return prod ** (1.0 / len(reds))


# ---------------------------------------------------------------------------
# CDNA4 schedule model
# ---------------------------------------------------------------------------


def _operand_bytes(op: OpSpec, split_k: int) -> float:
    """A and B bytes of the whole launch (a split-K spec carries K / split_k)."""
    m = op.mainloop
    if m.kind == "gemm":
        k = m.K * split_k
        return float(m.M * k * m.input_element_bytes + k * m.N * m.weight_element_bytes)
    return float(m.input_elements * m.input_element_bytes + m.weight_elements * m.weight_element_bytes)


def ideal_seconds(op: OpSpec, config: TuneConfig, hw: GPUSpec) -> float:
    """Mainloop FLOPs of the whole launch at the dtype's dense MFMA peak."""
    flops = op.mainloop.flops_per_fma * op.M * op.N * op.K * max(1, config.split_k)
    return flops / (hw.peak_tflops(op.mainloop.dtype) * 1e12)


def predict_schedule(op: OpSpec, config: TuneConfig, hw: GPUSpec,
                     c: Optional[ModelConstants] = None) -> Dict[str, Any]:
    """Predicted time of one launch on a CDNA4 device, in seconds.

    Workgroups are spread evenly over the CUs: the busiest CU runs
    ``n_cu = ceil(grid / CUs)`` tiles, ``conc`` of them at once (residency
    from registers, LDS and wave slots), in ``rounds = ceil(n_cu / conc)``.
    One K step of one workgroup needs

      MFMA   (BM/m)(BN/n)(BK/k) issue cycles / sustained rate, spread over
             the waves, which sit on the 4 SIMDs round-robin: the busiest
             SIMD issues for ceil(waves on the CU / 4) of them,
      LDS    every wave reads its A rows and B columns, and the tile is
             written once: (waves (WTM + WTN) + BM + BN) BK bytes at
             ``hw.lds_bytes_per_clk``,
      L2     (BM + BN) BK bytes at the per-CU L2 feed rate.

    The mainloop is the larger of the throughput bound (all n_cu tiles share
    the CU's SIMDs, LDS and L2 port) and the latency bound (each round walks
    its K steps one after another; a step cannot beat the memory latency
    divided by the prefetch depth ``num_stages - 1``, plus a fixed per-step
    cost).  Each round then stores its tiles (fp32 partials under split-K)
    and runs the epilogue primitives' FLOPs, plus a fixed per-tile cost.  The
    launch cannot beat its operands and outputs at HBM rate; split-K adds the
    reduction launch (read every partial, write the output).
    """
    c = c or constants_for(hw)
    proj = project_config(op, config, hw)
    sk = max(1, config.split_k)
    waves = max(1, config.num_warps)
    simds = max(1, hw.simds_per_cu)
    clk = hw.clock_ghz * 1e9
    n_cu = _ceildiv(proj.grid_size, hw.num_sm)
    conc = max(1, min(proj.resident_blocks_per_sm, n_cu))
    rounds = _ceildiv(n_cu, conc)

    shape = hw.mfma(op.mainloop.dtype, config.mfma) if config.mfma else None
    if shape is not None:
        rate = dict(c.mfma_rate).get(config.mfma, 1.0)
        issue = (max(1, config.block_M // shape.m) * max(1, config.block_N // shape.n)
                 * max(1, config.block_K // shape.k) * shape.cycles / rate)
    else:   # no MFMA shape: the dtype's dense peak per SIMD
        per_simd = hw.peak_tflops(op.mainloop.dtype) * 1e12 / (hw.num_sm * simds * clk)
        issue = op.mainloop.flops_per_fma * config.block_M * config.block_N * config.block_K / per_simd
    mfma_shared = _ceildiv(conc * waves, simds) * issue / (waves * conc)
    mfma_alone = _ceildiv(waves, simds) * issue / waves
    wm, wn = config.wave_grid()
    wtm, wtn = config.block_M // max(1, wm), config.block_N // max(1, wn)
    ab, bb = op.mainloop.input_element_bytes, op.mainloop.weight_element_bytes
    steps = proj.tiles_K
    step_bytes = (config.block_M * ab + config.block_N * bb) * config.block_K
    lds = (waves * (wtm * ab + wtn * bb) * config.block_K + step_bytes) / max(1, hw.lds_bytes_per_clk)
    l2 = step_bytes / c.l2_bytes_per_clk_per_cu
    latency = c.mem_latency_clk / max(1, config.num_stages - 1)
    t_thru = n_cu * steps * max(mfma_shared, lds, l2)
    t_lat = rounds * steps * (max(mfma_alone, lds, l2, latency) + c.step_overhead_clk)
    mainloop_clk = max(t_thru, t_lat)

    outs = proj.tile_outputs
    out_b = 4 if sk > 1 else op.mainloop.output_element_bytes
    store = outs * (out_b + sum(p.bytes_per_output for p in op.epilogue)) / c.store_bytes_per_clk_per_cu
    epi = outs * sum(p.flops_per_output for p in op.epilogue) / c.epilogue_flops_per_clk_per_cu
    epilogue_clk = rounds * (store + epi + c.tile_overhead_clk)

    bw = hw.mem_bandwidth_gbps * 1e9 * c.hbm_efficiency
    mn = float(op.M * op.N)
    hbm_s = (_operand_bytes(op, sk) + mn * out_b * sk
             + mn * sum(p.bytes_per_output for p in op.epilogue)) / bw
    kernel_s = max((mainloop_clk + epilogue_clk) / clk, hbm_s)
    reduce_s = ((mn * 4 * sk + mn * op.mainloop.output_element_bytes) / (bw * c.reduce_efficiency)
                + c.launch_overhead_s if sk > 1 else 0.0)
    return {"seconds": kernel_s + reduce_s, "kernel_s": kernel_s, "reduce_s": reduce_s, "hbm_s": hbm_s,
            "mainloop_s": mainloop_clk / clk, "epilogue_s": epilogue_clk / clk,
            "throughput_bound": t_thru >= t_lat, "n_cu": n_cu, "concurrent": conc, "rounds": rounds}


def extra_pass_seconds(op: OpSpec, hw: GPUSpec, bytes_moved: float) -> float:
    """A separate memory-bound launch (e.g. a normalisation pass over the output)."""
    c = constants_for(hw)
    return bytes_moved / (hw.mem_bandwidth_gbps * 1e9 * c.hbm_efficiency) + c.launch_overhead_s


# ---------------------------------------------------------------------------
# Combined score (reference cost_model.py:765-829)
# ---------------------------------------------------------------------------


def _factors(op: OpSpec, config: TuneConfig, hw: GPUSpec):
    proj = project_config(op, config, hw)
    f = {
        "eff_mainloop": eff_mainloop(op, config, proj, hw),
        "eff_memory": eff_memory(op, config, proj, hw),
        "eff_parallel": eff_parallel(op, config, proj, hw),
        "eff_pipeline": eff_pipeline(op, config, proj, hw),
        "eff_implicit_conv": eff_implicit_conv(op, config, proj, hw),
        "eff_epilogue": eff_epilogue(op, config, proj, hw),
        "eff_reduction": eff_reduction(op, config, proj, hw),
    }
    return proj, f


def score_formula(op: OpSpec, config: TuneConfig, hw: GPUSpec) -> float:
    """Reference mode: the product of the seven factors.  CDNA4 mode: the
    predicted fraction of dense MFMA peak, ideal_seconds / predicted seconds."""
    if hw.has_mfma_model:
        return ideal_seconds(op, config, hw) / predict_schedule(op, config, hw)["seconds"]
    _, f = _factors(op, config, hw)
    s = 1.0
    for name in ("eff_mainloop", "eff_memory", "eff_parallel", "eff_pipeline",
                 "eff_implicit_conv", "eff_epilogue", "eff_reduction"):
        s *= f[name]
    return s


def score_formula_detailed(op: OpSpec, config: TuneConfig, hw: GPUSpec) -> dict:
    if hw.has_mfma_model:
        sched = predict_schedule(op, config, hw)
        ideal = ideal_seconds(op, config, hw)
        out = {"score": ideal / sched["seconds"], "ideal_s": ideal, "schedule": sched}
        proj = project_config(op, config, hw)
    else:
        proj, f = _factors(op, config, hw)
        score = 1.0
        for v in f.values():
            score *= v
        out = {"score": score}
        out.update(f)
    out["projection"] = {k: getattr(proj, k) for k in (
        "tiles_M", "tiles_N", "tiles_K", "grid_size", "tile_outputs", "outputs_per_thread",
        "mainloop_iterations", "tile_arithmetic_intensity", "occupancy", "resident_blocks_per_sm",
        "wave_fill", "preferred_num_stages", "input_bytes_per_tile", "weight_bytes_per_tile",
        "output_bytes_per_tile", "epilogue_bytes_per_tile", "shared_mem_bytes_per_tile",
        "reduction_passes", "epilogue_preferred_outputs")}
    return out


def score_configs(op: OpSpec, configs: Sequence[TuneConfig], hw: GPUSpec) -> List[float]:
    return [score_formula(op, c, hw) for c in configs]


def select_best_config(op: OpSpec, configs: Sequence[TuneConfig], hw: GPUSpec):
    scores = score_configs(op, configs, hw)
    best = max(range(len(scores)), key=lambda i: scores[i])
    return best, configs[best], scores[best]


__all__ = [
    "ACT_PRIMITIVE", "BATCHNORM", "BIAS_ADD", "CDNA4_CONSTANTS", "ConfigProjection", "FusionPrimitive",
    "GELU", "MainloopSpec", "ModelConstants", "OpSpec", "PRIMITIVE_LIBRARY", "REFERENCE_CONSTANTS",
    "RELU", "ROW_LAYERNORM", "SILU", "TuneConfig", "conv_output_hw", "constants_for", "eff_epilogue",
    "eff_implicit_conv", "eff_mainloop", "eff_memory", "eff_parallel", "eff_pipeline",
    "eff_reduction", "extra_pass_seconds", "ideal_seconds", "make_conv2d_spec", "make_matmul_spec",
    "predict_schedule", "project_config", "resolve_primitives",
    "score_configs", "score_formula", "score_formula_detailed", "select_best_config",
]
