"""Host-side AddressSanitizer build of the C ABI (CPU-only tool).

Compiles the hand-written translation units and two instance TUs (one GEMM,
one conv) with AddressSanitizer on the host pass only (`-Xarch_host`); the
gfx950 device code is compiled as usual and never runs here.  The result,
`_build/asan/libicpp_hip_asan.so`, is loaded by tests/test_host_asan.py in a
child process that preloads the compiler's ASan runtime, and every entry point
is driven through its argument checks and error paths: the host code that sits
between a caller's pointers and a launch (instance table, workspace sizing,
last-error formatting, the no-alloc scratch sizing).

This file is for the CPU container only; nothing on a GPU run builds or loads
the sanitized library.
"""

from __future__ import annotations

import concurrent.futures as cf
import subprocess
import sys
from pathlib import Path
from typing import List

from .build import ARCH, BUILD, CSRC, FIXED_SOURCES, HIP_FLAGS, HIPCC, INCLUDE, INSTANCES, _tu_source

ASAN_DIR = BUILD / "asan"
ASAN_LIB = ASAN_DIR / "libicpp_hip_asan.so"
CLANG = Path(HIPCC).resolve().parent.parent / "lib" / "llvm" / "bin" / "clang++"
# one GEMM and one conv instance: enough to exercise the instance table and both
# launcher families' checks
INSTANCE_NAMES = ("gemm_f16_64x64x64_w2x2_m16_s2", "conv2d_f16_64x64x64_w2x2_m16_s2")
HOST_ASAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]


def asan_runtime() -> Path:
    """The shared ASan runtime of the compiler that built the library."""
    clang = CLANG if CLANG.exists() else Path("/opt/rocm/lib/llvm/bin/clang++")
    out = subprocess.run([str(clang), "-print-file-name=libclang_rt.asan-x86_64.so"], capture_output=True, text=True)
    p = Path(out.stdout.strip())
    if not p.is_file():
        raise RuntimeError(f"ASan runtime not found (clang printed {out.stdout.strip()!r})")
    return p


def _compile(src: Path, obj: Path) -> None:
    if obj.exists() and obj.stat().st_mtime > max(src.stat().st_mtime, _newest_header()):
        return
    cmd = [HIPCC, *HIP_FLAGS, *HOST_ASAN, f"-I{CSRC}", f"-I{INCLUDE}", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr[-4000:]}")


def _newest_header() -> float:
    return max(p.stat().st_mtime for p in list(CSRC.glob("*.hpp")) + list(INCLUDE.glob("*.h")))


def build_asan(jobs: int = 8) -> Path:
    ASAN_DIR.mkdir(parents=True, exist_ok=True)
    srcs: List[Path] = [CSRC / f"{stem}.hip" for stem, _ in FIXED_SOURCES]
    for inst in INSTANCES:
        if inst.name in INSTANCE_NAMES:
            tu = ASAN_DIR / f"{inst.name}.hip"
            text = _tu_source(inst)
            if not tu.exists() or tu.read_text() != text:
                tu.write_text(text)
            srcs.append(tu)
    if len(srcs) != len(FIXED_SOURCES) + len(INSTANCE_NAMES):
        raise RuntimeError("build_asan: an instance named in INSTANCE_NAMES is not in the instance set")
    objs = [ASAN_DIR / (s.stem + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        list(ex.map(_compile, srcs, objs))
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *HOST_ASAN[:2], "-shared-libasan",
           "-o", str(ASAN_LIB), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr[-4000:]}")
    return ASAN_LIB


if __name__ == "__main__":
    print(build_asan())
    print(asan_runtime())
    sys.exit(0)
