"""Build ``libseoulkv4_hip.so`` in-tree for gfx950 with hipcc.

Used by ``__graft_entry__.build()``; also runnable as
``python -m seoulkv_amd.build``.  The library is the only native artefact of
the package; ``seoulkv_amd._hip`` loads it from this directory.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libseoulkv4_hip.so"
SOURCES = ["skv_runtime.hip", "skv_kernels.hip", "skv_dense.hip"]
ARCH = os.environ.get("SKV_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    # packed FP32 VALU forms are kept out of every device code object
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # leading scalar / pointer kernel arguments arrive in scalar registers at
    # dispatch (kernel argument preloading), so a kernel's first loads need
    # not wait for its argument block to be read from memory
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the SeoulKV4 HIP library cannot be built")


# host code only: AddressSanitizer + UndefinedBehaviorSanitizer on the CPU
# side of the library (descriptor validation, mate and page tables, staging);
# the device code objects are built exactly as in the product library
SANITIZE_FLAGS = [
    "-Xarch_host", "-fsanitize=address",
    "-Xarch_host", "-fsanitize=undefined",
    "-Xarch_host", "-fno-sanitize-recover=all",
    "-Xarch_host", "-fno-omit-frame-pointer",
    "-g",
]


def build(verbose: bool = False, trace: bool = False, sanitize_dir: Path | None = None) -> Path:
    """Compile the library; ``trace`` builds the phase-timestamp variant
    ``libseoulkv4_hip_trace.so`` (development only) instead; ``sanitize_dir``
    builds ``libseoulkv4_hip_asan.so`` there, its host code instrumented with
    the address and undefined-behaviour sanitizers (tests only: a program
    that loads it must itself be linked with ``-fsanitize=address,undefined``
    by clang, which provides the runtime)."""
    if sanitize_dir is not None:
        lib = Path(sanitize_dir) / "libseoulkv4_hip_asan.so"
    else:
        lib = LIB.with_name("libseoulkv4_hip_trace.so") if trace else LIB
    tmp = lib.with_suffix(".so.tmp")
    extra = ["-DSKV_TRACE"] if trace else []
    if sanitize_dir is not None:
        extra += SANITIZE_FLAGS
    cmd = [hipcc(), *FLAGS, *extra, "-o", str(tmp), *[str(CSRC / s) for s in SOURCES]]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with exit code {res.returncode}")
    if verbose and res.stderr.strip():
        # hipcc's host pass reports the device-only target feature; harmless
        lines = [l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l]
        if lines:
            print("\n".join(lines))
    os.replace(tmp, lib)
    return lib


if __name__ == "__main__":
    print(build(verbose=True, trace="--trace" in sys.argv[1:]))
