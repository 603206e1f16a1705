"""Hardware description consumed by the cost model and the search-space pruner.

Mirrors the reference's ``GPUSpec`` (kernel/autotuner/gpu_spec.py:14-69): the
same field names, so that descriptors and cost-model code written against the
reference keep working, plus the CDNA4 facts the reference cannot express
(wave64, unified VGPR/AGPR file, MFMA shapes and rates, XCD count, fp8 peak).

Two specs matter here:

* ``A100`` -- restated from the reference's known-GPU table
  (kernel/autotuner/gpu_spec.py:73-90).  It exists so the restated scorer can be
  checked against the scores the reference published for A100
  (evaluation/gemm_three_ops_formula_summary.csv), i.e. to prove the formula
  was carried over faithfully before it is re-targeted.
* ``MI355X`` -- the target.  256 CUs in 8 XCDs, 64-lane waves, 160 KiB LDS per
  CU, 512 VGPRs per lane per wave (256 arch + 256 acc), 8 waves per SIMD,
  8 TB/s HBM3E, dense MFMA peaks 2516.6 TFLOP/s (fp16/bf16) and 5033.2 (fp8).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, Optional, Tuple


@dataclass(frozen=True)
class MfmaShape:
    """One MFMA instruction family usable by the kernel templates."""

    m: int
    n: int
    k: int
    dtype: str              # "f16" / "bf16" / "fp8"
    cycles: int             # issue-to-issue cycles on one SIMD at full rate

    @property
    def flops(self) -> int:
        return 2 * self.m * self.n * self.k

    @property
    def tag(self) -> str:
        return f"{self.m}x{self.n}x{self.k}"


@dataclass(frozen=True)
class GPUSpec:
    """Hardware specification (reference field names; CDNA4 extensions below)."""

    # Identity
    name: str
    compute_capability: tuple

    # Compute resources (reference semantics: "sm" = CU, "warp" = wavefront)
    num_sm: int
    max_threads_per_sm: int
    max_warps_per_sm: int
    warp_size: int
    max_threads_per_block: int
    max_regs_per_block: int
    max_regs_per_sm: int

    # Memory hierarchy
    shared_mem_per_block: int
    shared_mem_per_sm: int
    l2_cache_size: int
    global_mem_size: int

    # Bandwidth & throughput
    mem_bandwidth_gbps: float
    peak_fp16_tflops: float
    peak_fp32_tflops: float

    # ---- CDNA extensions (defaults describe "no MFMA model": reference mode)
    arch: str = ""
    peak_fp8_tflops: float = 0.0
    num_xcd: int = 1
    simds_per_cu: int = 4
    max_waves_per_simd: int = 0
    vgprs_per_lane_max: int = 0          # arch + acc registers addressable per lane
    lds_bytes_per_clk: int = 0
    clock_ghz: float = 0.0
    mall_bytes: int = 0
    mfma_shapes: Tuple[MfmaShape, ...] = field(default_factory=tuple)
    max_blocks_per_cu: int = 0

    # Derived ---------------------------------------------------------------
    @property
    def ridge_point_fp16(self) -> float:
        """FLOP/byte needed to saturate the fp16/bf16 matrix peak (reference :47-51)."""
        if self.mem_bandwidth_gbps <= 0:
            return float("inf")
        return (self.peak_fp16_tflops * 1e3) / self.mem_bandwidth_gbps

    @property
    def ridge_point_fp32(self) -> float:
        if self.mem_bandwidth_gbps <= 0:
            return float("inf")
        return (self.peak_fp32_tflops * 1e3) / self.mem_bandwidth_gbps

    def ridge_point(self, dtype: str) -> float:
        """Ridge point for the matrix datatype of the mainloop."""
        if dtype == "fp8" and self.peak_fp8_tflops > 0:
            return (self.peak_fp8_tflops * 1e3) / self.mem_bandwidth_gbps
        return self.ridge_point_fp16

    def peak_tflops(self, dtype: str) -> float:
        if dtype == "fp8" and self.peak_fp8_tflops > 0:
            return self.peak_fp8_tflops
        if dtype == "f32":
            return self.peak_fp32_tflops
        return self.peak_fp16_tflops

    @property
    def max_blocks_per_sm(self) -> int:
        """Concurrent workgroups per CU/SM (reference :60-69 for NVIDIA)."""
        if self.max_blocks_per_cu:
            return self.max_blocks_per_cu
        major = self.compute_capability[0]
        if major >= 7:
            return 32
        return 16

    @property
    def has_mfma_model(self) -> bool:
        return bool(self.mfma_shapes)

    def mfma(self, dtype: str, tag: str) -> Optional[MfmaShape]:
        for s in self.mfma_shapes:
            if s.dtype == dtype and s.tag == tag:
                return s
        return None


A100 = GPUSpec(
    name="NVIDIA A100",
    compute_capability=(8, 0),
    num_sm=108,
    max_threads_per_sm=2048,
    max_warps_per_sm=64,
    warp_size=32,
    max_threads_per_block=1024,
    max_regs_per_block=65536,
    max_regs_per_sm=65536,
    shared_mem_per_block=163840,
    shared_mem_per_sm=167936,
    l2_cache_size=40 * 1024 * 1024,
    global_mem_size=80 * 1024 ** 3,
    mem_bandwidth_gbps=2039.0,
    peak_fp16_tflops=312.0,
    peak_fp32_tflops=19.5,
)

# MFMA issue cycles per SIMD: one CU retires 4096 dense fp16 FLOP/clk
# (2516.6e12 / (256 CU * 2.4e9)), i.e. 1024 per SIMD; fp8 doubles that.
_MI355X_MFMA = (
    MfmaShape(16, 16, 32, "f16", 16),
    MfmaShape(32, 32, 16, "f16", 32),
    MfmaShape(16, 16, 32, "bf16", 16),
    MfmaShape(32, 32, 16, "bf16", 32),
    MfmaShape(16, 16, 128, "fp8", 32),
    MfmaShape(32, 32, 64, "fp8", 64),
)

MI355X = GPUSpec(
    name="AMD Instinct MI355X",
    compute_capability=(9, 5),
    num_sm=256,
    max_threads_per_sm=2048,
    max_warps_per_sm=32,
    warp_size=64,
    max_threads_per_block=1024,
    max_regs_per_block=131072,       # 512 KiB register file per CU, 32-bit regs
    max_regs_per_sm=131072,
    shared_mem_per_block=163840,
    shared_mem_per_sm=163840,
    l2_cache_size=4 * 1024 * 1024,   # per XCD
    global_mem_size=288 * 1024 ** 3,
    mem_bandwidth_gbps=8000.0,
    peak_fp16_tflops=2516.6,
    peak_fp32_tflops=157.3,
    arch="gfx950",
    peak_fp8_tflops=5033.2,
    num_xcd=8,
    simds_per_cu=4,
    max_waves_per_simd=8,
    vgprs_per_lane_max=512,
    lds_bytes_per_clk=128,
    clock_ghz=2.4,
    mall_bytes=256 * 1024 * 1024,
    mfma_shapes=_MI355X_MFMA,
    max_blocks_per_cu=32,
)

KNOWN_GPUS: Dict[str, GPUSpec] = {"A100": A100, "MI355X": MI355X}


def detect_gpu(device_id: int = 0) -> GPUSpec:
    """Return the spec of the visible device.

    The kernels in this package are built for gfx950 only, so a visible device
    that is not gfx950 is an error; with no visible device the build target
    (MI355X) is returned so ranking and pruning work on a CPU-only host.
    """
    import torch

    if not torch.cuda.is_available():
        return MI355X
    props = torch.cuda.get_device_properties(device_id)
    arch = getattr(props, "gcnArchName", "")
    if not arch.startswith("gfx950"):
        raise RuntimeError(f"icpp_tuning_amd targets gfx950 (MI355X); device {device_id} is {arch or props.name}")
    cus = props.multi_processor_count
    if cus == MI355X.num_sm:
        return MI355X
    # Partitioned device (e.g. CPX mode): scale the per-device totals.
    frac = cus / MI355X.num_sm
    from dataclasses import replace
    return replace(
        MI355X,
        num_sm=cus,
        num_xcd=max(1, round(MI355X.num_xcd * frac)),
        mem_bandwidth_gbps=MI355X.mem_bandwidth_gbps * frac,
        peak_fp16_tflops=MI355X.peak_fp16_tflops * frac,
        peak_fp32_tflops=MI355X.peak_fp32_tflops * frac,
        peak_fp8_tflops=MI355X.peak_fp8_tflops * frac,
        global_mem_size=props.total_memory,
    )


_cached_spec: Optional[GPUSpec] = None


def get_gpu_spec(device_id: int = 0, force_refresh: bool = False) -> GPUSpec:
    """Cached device spec (reference :280-285)."""
    global _cached_spec
    if _cached_spec is None or force_refresh:
        _cached_spec = detect_gpu(device_id)
    return _cached_spec


__all__ = ["A100", "MI355X", "GPUSpec", "KNOWN_GPUS", "MfmaShape", "detect_gpu", "get_gpu_spec"]
