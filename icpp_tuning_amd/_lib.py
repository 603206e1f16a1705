"""ctypes binding of libicpp_hip.so (C ABI declared in include/icpp_hip.h).

The library is the only compute path of this package: there is no CPU or
PyTorch fallback.  If it is missing or fails to load, every entry point raises
``IcppLibraryError``; rebuild with ``python -m icpp_tuning_amd.build``.
"""

from __future__ import annotations

import ctypes
import json
import threading
from pathlib import Path
from typing import Dict, List, Optional

PKG = Path(__file__).resolve().parent
LIB_PATH = PKG / "libicpp_hip.so"
RESOURCES_PATH = PKG / "libicpp_hip.resources.json"

ABI_VERSION = 2
FAMILY = {"gemm": 0, "gemm_ln_stats": 1, "gemm_ln_row": 2, "conv2d": 3}
FAMILY_NAME = {v: k for k, v in FAMILY.items()}
# strategy codes of the LayerNorm entry points: the instance families above plus
# ICPP_LN_CORESIDENT (f16 GEMM instances run with the co-resident row-block epilogue)
LN_CORESIDENT = 16
LN_STRATEGY = dict(FAMILY, gemm_ln_cr=LN_CORESIDENT)
DTYPE = {"f16": 0, "bf16": 1, "fp8": 2, "f32": 3}
DTYPE_NAME = {v: k for k, v in DTYPE.items()}
ACT = {"none": 0, "relu": 1, "gelu_tanh": 2, "gelu": 2, "silu": 3, "gelu_erf": 4}

# every symbol declared in include/icpp_hip.h
EXPORTED_SYMBOLS = (
    "icpp_abi_version", "icpp_last_error", "icpp_num_instances", "icpp_instance_info",
    "icpp_workspace_bytes", "icpp_gemm", "icpp_gemm_bias_layernorm", "icpp_conv2d_nhwc", "icpp_conv2d_nhwc_fused",
    "icpp_layernorm_fwd", "icpp_layernorm_bwd_workspace_bytes", "icpp_layernorm_bwd", "icpp_softmax",
    "icpp_softmax_scaled_masked",
    "icpp_gemm_bias_residual_layernorm", "icpp_qkv_split_heads", "icpp_merge_heads", "icpp_attention_fwd",
    "icpp_clock_probe", "icpp_gemm_noalloc", "icpp_gemm_bias_layernorm_workspace_bytes",
    "icpp_fp8_pack_b", "icpp_fp8_gemm_packed",
)
CONV_EPI = {"bn": 1, "residual": 2, "var_clamp": 4}


class IcppLibraryError(RuntimeError):
    pass


class IcppCallError(RuntimeError):
    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} returned {code}: {msg}")
        self.code = code


class IcppTile(ctypes.Structure):
    _fields_ = [
        ("family", ctypes.c_int), ("dtype", ctypes.c_int),
        ("block_m", ctypes.c_int), ("block_n", ctypes.c_int), ("block_k", ctypes.c_int),
        ("waves_m", ctypes.c_int), ("waves_n", ctypes.c_int), ("stages", ctypes.c_int),
        ("mfma_m", ctypes.c_int), ("mfma_n", ctypes.c_int), ("mfma_k", ctypes.c_int),
        ("lds_bytes", ctypes.c_int), ("threads", ctypes.c_int), ("name", ctypes.c_char * 96),
    ]


_vp, _i, _f, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
_SIGNATURES = {
    "icpp_abi_version": (_i, []),
    "icpp_last_error": (ctypes.c_char_p, []),
    "icpp_num_instances": (_i, [_i]),
    "icpp_instance_info": (_i, [_i, _i, ctypes.POINTER(IcppTile)]),
    "icpp_workspace_bytes": (_sz, [_i, _i, _i, _i, _i, _i]),
    "icpp_gemm_bias_layernorm_workspace_bytes": (_sz, [_i, _i, _i, _i, _i]),
    "icpp_gemm": (_i, [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _f, _f, _i, _vp, _sz, _vp]),
    "icpp_gemm_bias_layernorm": (_i, [_i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _vp, _sz, _vp]),
    "icpp_gemm_bias_residual_layernorm": (_i, [_i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _vp, _sz,
                                               _vp]),
    "icpp_conv2d_nhwc": (_i, [_i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _sz, _vp]),
    "icpp_conv2d_nhwc_fused": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _f, _i, _i,
                                    _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _i, _vp, _sz, _vp]),
    "icpp_layernorm_fwd": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _vp]),
    "icpp_layernorm_bwd_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "icpp_layernorm_bwd": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp, _sz, _vp]),
    "icpp_softmax": (_i, [_i, _vp, _vp, _i, _i, _i, _i, _vp]),
    "icpp_softmax_scaled_masked": (_i, [_i, _vp, _vp, _vp, _f, _i, _i, _i, _i, _i, _vp]),
    "icpp_qkv_split_heads": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "icpp_attention_fwd": (_i, [_i, _vp, _vp, _vp, _vp, _f, _vp, _i, _i, _i, _i, _vp]),
    "icpp_merge_heads": (_i, [_i, _vp, _vp, _i, _i, _i, _i, _vp]),
    "icpp_clock_probe": (_i, [_vp, ctypes.c_double, _vp]),
    "icpp_gemm_noalloc": (_i, [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _f, _f, _i, _vp]),
    "icpp_fp8_pack_b": (_i, [_vp, _vp, _i, _i, _vp]),
    "icpp_fp8_gemm_packed": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _f, _vp]),
}


class Lib:
    def __init__(self, path: Path = LIB_PATH):
        if not path.exists():
            raise IcppLibraryError(f"{path} not built; run `python -m icpp_tuning_amd.build`")
        try:
            self._dll = ctypes.CDLL(str(path))
        except OSError as e:
            raise IcppLibraryError(f"cannot load {path}: {e}") from e
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(self._dll, name)
            fn.restype = res
            fn.argtypes = args
        v = self._dll.icpp_abi_version()
        if v != ABI_VERSION:
            raise IcppLibraryError(f"{path}: ABI version {v}, expected {ABI_VERSION}")
        self.path = path
        self._tables: Dict[int, List[dict]] = {}

    # ---- raw calls -------------------------------------------------------
    def call(self, name: str, *args) -> None:
        rc = getattr(self._dll, name)(*args)
        if rc != 0:
            raise IcppCallError(name, rc, self.last_error())

    def last_error(self) -> str:
        s = self._dll.icpp_last_error()
        return s.decode() if s else ""

    def has_symbol(self, name: str) -> bool:
        return hasattr(self._dll, name)

    def workspace_bytes(self, family: int, inst: int, M: int, N: int, K: int, split_k: int) -> int:
        return int(self._dll.icpp_workspace_bytes(family, inst, M, N, K, split_k))

    def ln_workspace_bytes(self, family: int, inst: int, M: int, N: int, K: int) -> int:
        return int(self._dll.icpp_gemm_bias_layernorm_workspace_bytes(family, inst, M, N, K))

    def layernorm_bwd_workspace_bytes(self, dtype: int, M: int, N: int, ld: int) -> int:
        return int(self._dll.icpp_layernorm_bwd_workspace_bytes(dtype, M, N, ld))

    # ---- instance table --------------------------------------------------
    def instances(self, family: int) -> List[dict]:
        if family not in self._tables:
            n = self._dll.icpp_num_instances(family)
            if n < 0:
                raise IcppCallError("icpp_num_instances", n, self.last_error())
            rows = []
            for idx in range(n):
                t = IcppTile()
                self.call("icpp_instance_info", family, idx, ctypes.byref(t))
                rows.append({
                    "index": idx, "family": FAMILY_NAME[t.family], "dtype": DTYPE_NAME[t.dtype],
                    "block_m": t.block_m, "block_n": t.block_n, "block_k": t.block_k,
                    "waves_m": t.waves_m, "waves_n": t.waves_n, "stages": t.stages,
                    "mfma_m": t.mfma_m, "mfma_n": t.mfma_n, "mfma_k": t.mfma_k,
                    "lds_bytes": t.lds_bytes, "threads": t.threads, "name": t.name.decode(),
                })
            self._tables[family] = rows
        return self._tables[family]


_lib: Optional[Lib] = None
_lock = threading.Lock()


def lib() -> Lib:
    global _lib
    with _lock:
        if _lib is None:
            _lib = Lib()
        return _lib


def reload() -> Lib:
    global _lib
    with _lock:
        _lib = Lib()
        return _lib


_resources_cache: Dict[str, object] = {}


def resources() -> Dict[str, dict]:
    """Compiler-reported resources per instance name (VGPRs, AGPRs, scratch, occupancy, LDS)."""
    if not RESOURCES_PATH.exists():
        return {}
    mtime = RESOURCES_PATH.stat().st_mtime
    if _resources_cache.get("mtime") != mtime:
        _resources_cache["data"] = json.loads(RESOURCES_PATH.read_text()).get("instances", {})
        _resources_cache["mtime"] = mtime
    return _resources_cache["data"]


__all__ = ["ACT", "DTYPE", "EXPORTED_SYMBOLS", "FAMILY", "LN_CORESIDENT", "LN_STRATEGY", "IcppCallError", "IcppLibraryError", "Lib", "lib", "resources"]
