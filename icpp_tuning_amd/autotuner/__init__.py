"""Autotuner for the gfx950 fused-kernel set: hardware spec, CDNA4 cost model,
search-space pruning and the select / rank / tune loop (reference
kernel/autotuner/)."""

from .interface import TileLangKernelBase, TuneResult, configure_autotuner_cache, rank_all, select_best, tune  # noqa: F401
from .gpu_spec import A100, MI355X, GPUSpec, get_gpu_spec  # noqa: F401
