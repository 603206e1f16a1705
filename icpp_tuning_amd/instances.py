"""The ahead-of-time instance set compiled into libicpp_hip.so.

Each entry is one template instantiation of ``gemm_kernel`` in
csrc/icpp_kernels.hpp.  This list is the tuner's compiled candidate space: the
descriptors rank it, the pruner filters it, and ``build.py`` generates one
translation unit per entry.  The reference instead enumerates a config grid in
each kernel file and JIT-compiles the winner with TileLang
(gemm.py:24-48 + :84-89); on gfx950 every candidate is compiled once at build
time, so "compile" in the tuning loop costs nothing.

Families
  gemm          dense A, epilogue bias+act or split-K fp32 partials
  gemm_ln_stats GEMM+bias writing X plus per-(row, wave column block) LN stats
  gemm_ln_row   GEMM+bias+LayerNorm, one workgroup owns whole rows (N <= BN)
  conv2d        NHWC implicit GEMM (A gathered per 16-byte channel chunk)

Mainloop schedules (``sched``)
  ""            every wave streams MFMAs and its fragment reads together; one
                workgroup barrier per K tile
  "pp"          ping-pong (8 waves, gemm and conv2d families): each group of four
                waves (one per SIMD) alternates between an MFMA-only phase and a
                memory phase (fragment reads + tile loads), offset by one phase from
                the other group, so the two waves of a SIMD never split its matrix
                core and one issues memory instructions while the other's MFMAs run
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List

FAMILY_ID = {"gemm": 0, "gemm_ln_stats": 1, "gemm_ln_row": 2, "conv2d": 3}
DTYPE_ID = {"f16": 0, "bf16": 1, "fp8": 2}
EPI_ID = {"gemm": 0, "gemm_ln_stats": 1, "gemm_ln_row": 2, "conv2d": 0}
ALOAD_ID = {"gemm": 0, "gemm_ln_stats": 0, "gemm_ln_row": 0, "conv2d": 1}
ESZ = {"f16": 2, "bf16": 2, "fp8": 1}
MFMA_K = {("f16", 16): 32, ("f16", 32): 16, ("bf16", 16): 32, ("bf16", 32): 16, ("fp8", 16): 128, ("fp8", 32): 64}


@dataclass(frozen=True)
class Inst:
    family: str
    dtype: str
    bm: int
    bn: int
    bk: int
    wm: int
    wn: int
    mf: int
    stages: int
    sched: str = ""

    @property
    def name(self) -> str:
        return (f"{self.family}_{self.dtype}_{self.bm}x{self.bn}x{self.bk}"
                f"_w{self.wm}x{self.wn}_m{self.mf}_s{self.stages}" + (f"_{self.sched}" if self.sched else ""))

    @property
    def threads(self) -> int:
        return 64 * self.wm * self.wn

    @property
    def acc_regs(self) -> int:
        """fp32 accumulator registers per lane."""
        return self.bm * self.bn // self.threads

    @property
    def compile_flags(self) -> List[str]:
        """Per-instance code-generation flags.  When the accumulators fit the
        architectural VGPRs alongside the fragments, the MFMAs are told to read
        and write VGPRs: otherwise the backend may keep the loop-carried
        accumulators in VGPRs and copy them into AGPRs every iteration."""
        if self.acc_regs <= 160:
            return ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
        return []

    @property
    def lds_bytes(self) -> int:
        e = ESZ[self.dtype]
        return (self.bm * self.bk + self.bk * self.bn) * e * self.stages

    def validate(self) -> None:
        e = ESZ[self.dtype]
        kf = MFMA_K[(self.dtype, self.mf)]
        wtm, wtn = self.bm // self.wm, self.bn // self.wn
        problems = []
        if self.bm % self.wm or self.bn % self.wn:
            problems.append("block not divisible by wave grid")
        if wtm % self.mf or wtn % self.mf:
            problems.append("wave tile not a multiple of the MFMA tile")
        if self.bk % kf:
            problems.append("block_k not a multiple of MFMA K")
        if self.bn * e < 128:
            problems.append("B rows shorter than 128 bytes")
        if self.bk * e < 32:
            problems.append("A rows shorter than 32 bytes")
        if self.lds_bytes > 160 * 1024:
            problems.append("LDS overflow")
        if not 2 <= self.stages <= 8:
            problems.append("stages must be 2 to 8")
        if (self.stages * (self.bk // kf)) % 2:
            problems.append("stages x MFMA K-steps per tile must be even (fragment double buffer)")
        loads = -(-(self.bm * self.bk * e // 16) // self.threads) - (-(self.bk * self.bn * e // 16) // self.threads)
        if loads * (self.stages - 1) >= 64:
            problems.append("too many loads in flight for vmcnt")
        if self.sched not in ("", "pp"):
            problems.append("unknown mainloop schedule")
        if self.sched == "pp" and (self.family not in ("gemm", "conv2d") or self.wm * self.wn != 8):
            problems.append("ping-pong needs the gemm or conv2d family and 8 waves")
        if problems:
            raise ValueError(f"{self.name}: " + "; ".join(problems))


def _g(dtype, bm, bn, bk, wm, wn, mf, st=2, fam="gemm"):
    return Inst(fam, dtype, bm, bn, bk, wm, wn, mf, st)


def _with_pp(tiles: List[Inst]) -> List[Inst]:
    """Each 2 x 4-wave tile plus its ping-pong twin."""
    out = []
    for t in tiles:
        out.append(t)
        if (t.wm, t.wn) == (2, 4):
            out.append(Inst(t.family, t.dtype, t.bm, t.bn, t.bk, t.wm, t.wn, t.mf, t.stages, "pp"))
    return out


# 4-wave 256x256 tiles (128x128 per wave) are left out: 256 accumulator
# registers per lane plus double-buffered fragments spill to scratch.
def _gemm_tiles(dtype: str) -> List[Inst]:
    return [
        _g(dtype, 256, 256, 64, 2, 4, 32),
        _g(dtype, 256, 256, 64, 2, 4, 16),
        _g(dtype, 256, 256, 32, 2, 4, 32, st=4),
        _g(dtype, 256, 128, 64, 2, 2, 32, st=3),
        _g(dtype, 128, 256, 64, 2, 2, 32, st=3),
        _g(dtype, 256, 128, 64, 2, 2, 32),
        _g(dtype, 128, 256, 64, 2, 2, 32),
        _g(dtype, 128, 128, 64, 2, 2, 32),
        _g(dtype, 128, 128, 64, 2, 2, 16),
        _g(dtype, 128, 128, 32, 2, 2, 32),
        _g(dtype, 64, 128, 64, 1, 4, 16),
        _g(dtype, 64, 64, 64, 2, 2, 16),
        _g(dtype, 32, 128, 64, 1, 4, 16),
        _g(dtype, 16, 128, 64, 1, 4, 16),
        _g(dtype, 16, 64, 128, 1, 4, 16),
        # deeper rings and 8-wave mid-size tiles
        _g(dtype, 256, 128, 64, 2, 4, 16),
        _g(dtype, 128, 256, 64, 2, 4, 16),
        _g(dtype, 128, 128, 64, 2, 2, 16, st=3),
        _g(dtype, 128, 128, 32, 2, 2, 16, st=4),
        _g(dtype, 64, 128, 64, 1, 4, 16, st=4),
        _g(dtype, 64, 64, 64, 2, 2, 16, st=4),
        _g(dtype, 32, 128, 64, 1, 4, 16, st=4),
        _g(dtype, 16, 128, 64, 1, 4, 16, st=4),
        # 192-column tiles: 8192 x 768 outputs in exactly 256 tiles (one per CU)
        _g(dtype, 128, 192, 64, 2, 2, 16),
        _g(dtype, 128, 192, 64, 2, 2, 16, st=3),
        _g(dtype, 128, 192, 64, 2, 4, 16),
        # 8-wave half-size tiles with three stages (144 KiB, one workgroup per CU): two
        # K tiles in flight cover the HBM latency of an A panel that no other
        # workgroup has pulled into L2 yet (8192 x 1024 outputs: 16% faster cold)
        _g(dtype, 128, 256, 64, 2, 4, 16, st=3),
        _g(dtype, 256, 128, 64, 2, 4, 16, st=3),
    ]


def _fp8_tiles() -> List[Inst]:
    d = "fp8"
    return [
        _g(d, 256, 256, 128, 2, 4, 32),
        _g(d, 256, 256, 64, 2, 4, 32, st=4),
        _g(d, 256, 128, 128, 2, 2, 32),
        _g(d, 128, 128, 128, 2, 2, 32),
        _g(d, 128, 128, 128, 2, 2, 16),
        _g(d, 64, 128, 128, 1, 4, 16),
        _g(d, 32, 128, 128, 1, 4, 16),
        _g(d, 16, 128, 256, 1, 4, 16),
        _g(d, 16, 256, 128, 1, 4, 16),
        # deeper rings / one-shot K for skinny (decode) shapes
        _g(d, 128, 128, 128, 2, 2, 16, st=4),
        _g(d, 64, 128, 128, 1, 4, 16, st=4),
        _g(d, 32, 128, 256, 1, 4, 16, st=3),
        _g(d, 16, 256, 128, 1, 4, 16, st=4),
        _g(d, 16, 128, 512, 1, 4, 16),
        _g(d, 16, 128, 128, 1, 4, 16, st=4),
        _g(d, 16, 128, 256, 1, 4, 16, st=3),
        # 32-row tiles with 4- and 6-stage rings (no split-K needed from M = 32 to 64;
        # the profiled table picks them at 4 of 41 shapes, 0-3% ahead)
        _g(d, 32, 128, 128, 1, 4, 16, st=4),
        _g(d, 32, 128, 128, 2, 2, 16, st=6),
    ]


def _ln_tiles() -> List[Inst]:
    st = "gemm_ln_stats"
    row = "gemm_ln_row"
    return [
        _g("f16", 256, 128, 64, 2, 2, 32, fam=st),
        _g("f16", 128, 256, 64, 2, 2, 32, fam=st),
        _g("f16", 128, 128, 64, 2, 2, 32, fam=st),
        _g("f16", 128, 128, 64, 2, 2, 16, fam=st),
        _g("f16", 256, 256, 64, 2, 4, 16, fam=st),
        _g("f16", 256, 256, 64, 2, 4, 32, fam=st),
        _g("f16", 128, 256, 64, 2, 4, 16, fam=st),
        _g("f16", 128, 128, 64, 2, 2, 16, st=3, fam=st),
        _g("f16", 128, 128, 32, 2, 2, 16, st=4, fam=st),
        # small tiles: short activations (BERT's M = batch x seq from 128) still fill the CUs
        _g("f16", 64, 64, 64, 2, 2, 16, fam=st),
        _g("f16", 64, 64, 64, 2, 2, 16, st=4, fam=st),
        _g("f16", 64, 128, 64, 1, 4, 16, fam=st),
        _g("f16", 32, 128, 64, 1, 4, 16, fam=st),
        _g("f16", 32, 768, 32, 1, 8, 16, fam=row),
        _g("f16", 64, 768, 32, 1, 8, 16, fam=row),
        _g("f16", 32, 1024, 32, 1, 8, 16, fam=row),
        _g("f16", 64, 1024, 32, 1, 8, 16, fam=row),
    ]


def _conv_tiles() -> List[Inst]:
    c = "conv2d"
    return [
        _g("f16", 256, 64, 64, 4, 1, 32, fam=c),
        _g("f16", 128, 64, 64, 2, 1, 32, fam=c),
        _g("f16", 128, 64, 64, 2, 2, 16, fam=c),
        _g("f16", 256, 128, 64, 2, 2, 32, fam=c),
        _g("f16", 128, 128, 64, 2, 2, 32, fam=c),
        _g("f16", 128, 128, 64, 2, 2, 16, fam=c),
        _g("f16", 64, 128, 64, 1, 4, 16, fam=c),
        _g("f16", 64, 64, 64, 2, 2, 16, fam=c),
        _g("f16", 128, 64, 64, 2, 2, 16, st=4, fam=c),
        _g("f16", 64, 64, 64, 2, 2, 16, st=4, fam=c),
        _g("f16", 128, 128, 64, 2, 2, 16, st=3, fam=c),
        _g("f16", 128, 128, 32, 2, 2, 16, st=4, fam=c),
        _g("f16", 64, 128, 64, 1, 4, 16, st=4, fam=c),
        _g("f16", 256, 128, 64, 2, 4, 16, fam=c),
        # row-aligned / deeper tiles for wide images under the input-halo loader
        # (224 = 4 rows of 56; 8 waves on 256 rows)
        _g("f16", 256, 64, 64, 4, 2, 16, fam=c),
        _g("f16", 224, 64, 64, 2, 2, 16, fam=c),
        _g("f16", 224, 64, 64, 7, 1, 32, fam=c),
        # ping-pong conv tiles (the tap gather and the input halo under the 8-wave
        # ping-pong loop): measured 16-25% slower than the best default-schedule tile at
        # every benchmark conv shape, kept so that both loader paths stay compiled and tested
        Inst(c, "f16", 64, 128, 64, 2, 4, 16, 4, "pp"),
        Inst(c, "f16", 256, 64, 64, 4, 2, 16, 2, "pp"),
    ]


INSTANCES: List[Inst] = (_with_pp(_gemm_tiles("f16")) + _with_pp(_gemm_tiles("bf16")) + _with_pp(_fp8_tiles())
                         + _ln_tiles() + _conv_tiles())

for _i in INSTANCES:
    _i.validate()
assert len({i.name for i in INSTANCES}) == len(INSTANCES), "duplicate instance names"


def instances(family: str | None = None, dtype: str | None = None) -> List[Inst]:
    return [i for i in INSTANCES if (family is None or i.family == family) and (dtype is None or i.dtype == dtype)]


__all__ = ["ALOAD_ID", "DTYPE_ID", "EPI_ID", "FAMILY_ID", "INSTANCES", "Inst", "MFMA_K", "instances"]
