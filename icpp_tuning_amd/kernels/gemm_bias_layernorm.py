"""Fused GEMM + bias + LayerNorm over N (fp16 in/out, fp32 statistics).

Mirrors kernel/tilelang/gemm/gemm_bias_layernorm.py: ``get_gemm_configs``
(:19-40), ``build_fused_kernel`` (:167-188, ``fused(A, B, bias, gamma, beta) ->
Y``) and ``DESCRIPTOR`` (:196-208).  The reference launches a GEMM+bias kernel
that writes X in fp32 and then a separate two-pass row LayerNorm kernel that
reads X twice and computes var = E[x^2] - mean^2 (:143).  Four strategies here,
chosen per shape by the tuner:

  "row"       (gemm_ln_row)    one workgroup owns whole rows (N <= block_N):
              mean and centred variance reduced in registers + LDS, no
              intermediate in HBM, one launch.
  "two_pass"  (gemm_ln_stats)  GEMM tiles write X into Y and a per-(row,
              wave column block) (mean, M2) pair into the workspace; a finalize
              pass merges the pairs (Chan et al.) and normalises Y in place.
  "gemm_ln"   (gemm, f16)      a GEMM + bias into Y (any GEMM tile, staged
              stores) plus per-(row, wave column block) means in the workspace,
              then the row LayerNorm kernel in place: the same HBM traffic as
              two-pass, with only a mean in the epilogue.
  "coresident" (gemm, f16)     one launch per chunk of row blocks the device keeps
              resident at once: the tiles of a row block exchange their rows'
              (mean, M2) through the workspace, wait for each other, and normalise
              from registers -- no X in memory, no second pass (the reference's
              fp32 X never leaves the accumulators).

Both two-launch strategies keep X in Y as f16 values centred on their block's
mean (the mean itself in fp32 in the workspace), where the reference keeps X in
fp32 (:59, :66, :103): the 16-bit copy rounds only the spread around the block
mean, so rows with a large common offset keep the fp32 precision.
"""

from __future__ import annotations

from typing import Any, Dict, List, Optional

import torch

from ..autotuner.cost_model import extra_pass_seconds, make_matmul_spec
from ..autotuner.perfdb import select_config
from .. import inputs as _inputs
from .. import runtime
from ._base import InstanceDescriptor, family_instances, raw_from_inst

STRATEGY_FAMILY = {"row": "gemm_ln_row", "two_pass": "gemm_ln_stats", "gemm_ln": "gemm", "coresident": "gemm"}
# the strategy code passed to the C ABI (runtime.ln_workspace_bytes / gemm_bias_layernorm)
STRATEGY_CALL = {"row": "gemm_ln_row", "two_pass": "gemm_ln_stats", "gemm_ln": "gemm", "coresident": "gemm_ln_cr"}
SUFFIX = {"row": "_ROW", "two_pass": "_2P", "gemm_ln": "_GL", "coresident": "_CR"}


def coresident_fits(inst, N: int) -> bool:
    """The f16 GEMM tiles built with the co-resident LayerNorm kernel (every f16 GEMM
    tile with 2+ stages), for row widths whose block_m x ceil(N / block_n) (mean, M2)
    pairs fit two LDS stage arrays (an even number of rows in the first, the rest in
    the second, as the kernel splits them); the library also checks that one row
    block's ceil(N / block_n) workgroups fit the device at once."""
    if inst.family != "gemm" or inst.dtype != "f16" or inst.stages < 2:
        return False
    if N <= 0:
        return True
    per = (inst.bm + inst.bn) * inst.bk * 2 // (-(-N // inst.bn) * 8)
    return inst.bm <= (per & ~1) + per


class GemmBiasLayerNormDescriptor(InstanceDescriptor):
    dtype = "f16"
    family = "gemm_ln_stats"

    @property
    def name(self) -> str:
        return "gemm_bias_layernorm"

    def make_op_spec(self, raw_config=None, M=0, N=0, K=0, **kw):
        """The GEMM launch of the strategy: "gemm_ln" is a plain GEMM + bias (the
        LayerNorm runs in a pass of its own); the other two carry the row
        statistics in their epilogue."""
        if raw_config is not None and raw_config.get("strategy") == "gemm_ln":
            return make_matmul_spec(M=M, N=N, K=K, primitives=["bias_add"], dtype=self.dtype)
        return make_matmul_spec(M=M, N=N, K=K, primitives=["bias_add", "row_layernorm"], dtype=self.dtype)

    def _family(self, raw) -> str:
        return STRATEGY_FAMILY[raw.get("strategy", "two_pass")]

    def instance_index(self, raw: Dict[str, Any]) -> int:
        fam = self._family(raw)
        mf = int(str(raw["mfma"]).split("x")[0])
        for idx, inst in enumerate(family_instances(fam)):
            if inst.dtype != self.dtype or inst.sched != raw.get("sched", ""):
                continue
            if (inst.bm, inst.bn, inst.bk, inst.stages, inst.threads, inst.wm, inst.wn, inst.mf) == (
                    raw["block_M"], raw["block_N"], raw["block_K"], raw["num_stages"], raw["thread_num"],
                    raw["waves_m"], raw["waves_n"], mf):
                return idx
        raise KeyError(f"no compiled {fam} instance for {self.format_config(raw)}")

    def instance_of(self, raw):
        return family_instances(self._family(raw))[self.instance_index(raw)]

    def get_raw_configs(self, **shape) -> List[Dict[str, Any]]:
        K, N = shape["K"], shape.get("N", 0)
        out = []
        for strategy, fam in STRATEGY_FAMILY.items():
            for inst in family_instances(fam):
                if K % inst.bk or inst.dtype != self.dtype:
                    continue
                if strategy == "row" and N and (N > inst.bn or inst.bn >= 2 * N):
                    continue  # whole row must fit one tile without wasting half of it
                if strategy == "coresident" and not coresident_fits(inst, N):
                    continue
                raw = raw_from_inst(inst)
                raw["strategy"] = strategy
                out.append(raw)
        return out

    def format_config(self, raw):
        return super().format_config(raw) + SUFFIX[raw.get("strategy", "two_pass")]

    def extra_seconds(self, raw, hw, M=0, N=0, K=0, **kw):
        """Two-pass and GEMM-then-LN run a second launch that reads and writes Y; the
        co-resident strategy waits once per launch for its row blocks' statistics
        (about one device-memory round trip each way, ~4 us), one launch per chunk of
        row blocks one workgroup per CU holds."""
        strategy = raw.get("strategy")
        if strategy == "row":
            return 0.0
        if strategy == "coresident":
            tiles_n = -(-N // raw["block_N"]) if N else 1
            tiles_m = -(-M // raw["block_M"]) if M else 1
            per_launch = max(1, hw.num_sm // max(1, tiles_n))
            return 4e-6 * -(-tiles_m // per_launch)
        op = self.make_op_spec(raw, M=M, N=N, K=K)
        return extra_pass_seconds(op, hw, 2.0 * M * N * op.mainloop.output_element_bytes)

    def make_inputs(self, M, N, K, **kw):
        d = _inputs.config3(M, N, K, device="cuda")
        d["Y"] = torch.empty((M, N), dtype=torch.float16, device="cuda")
        return d

    def make_runner(self, raw, inputs, M, N, K, **kw):
        k = build_fused_kernel(M, N, K, gemm_config=raw)
        return lambda: k(inputs["A"], inputs["B"], inputs["bias"], inputs["gamma"], inputs["beta"], out=inputs["Y"])


DESCRIPTOR = GemmBiasLayerNormDescriptor()


def get_gemm_configs(K, N: int = 0):
    return DESCRIPTOR.get_raw_configs(K=K, N=N)


def _overlap(a: torch.Tensor, b: torch.Tensor) -> bool:
    a0, b0 = a.data_ptr(), b.data_ptr()
    return a0 < b0 + b.numel() * b.element_size() and b0 < a0 + a.numel() * a.element_size()


class CompiledGemmLayerNorm:
    def __init__(self, M, N, K, config, eps=1e-5):
        self.M, self.N, self.K, self.config, self.eps = M, N, K, config, eps
        self.family = STRATEGY_CALL[config.get("strategy", "two_pass")]
        self.inst = DESCRIPTOR.instance_index(config)
        self._ws: Optional[torch.Tensor] = None

    def __call__(self, A, B, bias, gamma, beta, out=None, residual=None):
        """``LayerNorm(A @ B + bias [+ residual]) * gamma + beta``; the residual ([M, N] f16, may be
        ``out``) is the add of the BERT attention-output / FFN-output blocks (end2end.py:76-79)."""
        need = runtime.ln_workspace_bytes(self.family, self.inst, self.M, self.N, self.K)
        if need and (self._ws is None or self._ws.device != A.device):
            self._ws = runtime.alloc_workspace(need, A.device, zeroed=self.family == "gemm_ln_cr")
        if self.family == "gemm" and residual is not None and out is not None and _overlap(out, residual):
            # GEMM-then-LN writes Y before reading the residual: go through a fresh output
            y = runtime.gemm_bias_layernorm(self.family, self.inst, A, B, bias, gamma, beta, eps=self.eps,
                                            workspace=self._ws, residual=residual)
            return out.copy_(y)
        return runtime.gemm_bias_layernorm(self.family, self.inst, A, B, bias, gamma, beta, out=out,
                                           eps=self.eps, workspace=self._ws, residual=residual)

    def wait_failed(self, clear: bool = False) -> bool:
        """Co-resident strategy: whether a call since the flag was last cleared ran out of its
        bounded wait (its output is then invalid; see runtime.coresident_wait_failed).  False
        for the other strategies.  Synchronises."""
        if self.family != "gemm_ln_cr" or self._ws is None:
            return False
        return runtime.coresident_wait_failed(self._ws, self.inst, self.M, self.N, clear=clear)


def build_fused_kernel(M, N, K, gemm_config=None, block_M_ln=16, block_N_ln=128, thread_num_ln=128, eps=1e-5):
    """``fused(A, B, bias, gamma, beta) -> Y``.  The ``*_ln`` tile arguments of the
    reference's standalone LN kernel are accepted for call compatibility; the
    LayerNorm here is either fused into the GEMM epilogue or a fixed-geometry
    finalize pass (one wave per row)."""
    if gemm_config is None:
        gemm_config = select_config(DESCRIPTOR, M=M, N=N, K=K)
    return CompiledGemmLayerNorm(M, N, K, gemm_config, eps=eps)


__all__ = ["DESCRIPTOR", "GemmBiasLayerNormDescriptor", "STRATEGY_CALL", "STRATEGY_FAMILY", "coresident_fits", "build_fused_kernel", "get_gemm_configs"]
