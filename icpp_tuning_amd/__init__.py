"""icpp_tuning_amd -- MI355X (gfx950) fused-kernel library and autotuner.

Hand-written HIP MFMA kernels (csrc/, built into libicpp_hip.so) behind the
reference project's kernel / autotuner API (op spec, candidate configs,
compile, benchmark, select best)."""

__version__ = "0.1.0"
