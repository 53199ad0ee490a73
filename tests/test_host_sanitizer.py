"""The library's host code under AddressSanitizer and UndefinedBehaviorSanitizer.

``seoulkv_amd.build`` builds ``libseoulkv4_hip_asan.so``: the same sources
with the host code instrumented (``-Xarch_host -fsanitize=address`` and
``undefined``; device code objects unchanged).  ``tests/sanitizer_driver.c``,
linked by clang with the sanitizer runtime, loads a seeded config-0 index
from a case file and drives the host paths of the C ABI: descriptor
validation and every rejection, the spill-2 mate table of a valid index, the
page-table checks of ``skv_create_paged``, the size checks of the
allocation-free dense entry point and the NULL-handle calls.  Without a GPU
(CPU suite) ``skv_create`` then stops at the absent device; on a GPU box it
succeeds and the driver also runs the query staging ring, host appends
across staging chunks, the dense decode and destroy.  A sanitizer report
fails the run."""

from __future__ import annotations

import os
import subprocess
import struct
from pathlib import Path

import numpy as np
import pytest
import torch

from seoulkv_amd import _hip
from seoulkv_amd.build import CSRC, LIB, build
from tests.helpers import case

ROOT = Path(__file__).resolve().parents[1]
DRIVER = Path(__file__).resolve().with_name("sanitizer_driver.c")
CLANG = Path("/opt/rocm/llvm/bin/clang")
IN_TREE = LIB.with_name("libseoulkv4_hip_asan.so")
APPEND = 1100  # tokens the driver appends on a GPU (more than one staging chunk)


def _sanitized_library(tmp: Path) -> Path:
    """The in-tree sanitized library when it is newer than every source, else
    a fresh build under ``tmp``."""
    newest = max(p.stat().st_mtime for p in [*CSRC.iterdir(), ROOT / "include" / "seoulkv4_hip.h"])
    if IN_TREE.exists() and IN_TREE.stat().st_mtime >= newest:
        return IN_TREE
    return build(sanitize_dir=tmp)


def _write_case(path: Path) -> None:
    index, k, v, qs = case()
    desc, keep = _hip.index_desc(index, pool_min=0, pool_capacity=None, debug=True)
    with open(path, "wb") as f:
        f.write(struct.pack("<5i", desc.context, desc.sink, desc.local, desc.n_centroids,
                            APPEND))
        for g, arrays in enumerate(keep):
            cell = desc.cells[g]
            f.write(struct.pack("<ifi", cell.nprobe, cell.lam, arrays["values"].size))
            for name in ("upper", "lower", "scale", "resid_f16", "gfs_f16", "offsets", "values"):
                f.write(np.ascontiguousarray(arrays[name]).tobytes())
        for t in (k, v, qs[0]):
            f.write(t.contiguous().view(torch.int16).numpy().tobytes())


def _run_driver(tmp: Path, lib: Path, *, detect_leaks: bool) -> str:
    exe = tmp / "sanitizer_driver"
    subprocess.run([str(CLANG), "-std=c99", "-O1", "-g", "-fsanitize=address,undefined",
                    "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-Wall", "-Werror",
                    "-I", str(ROOT / "include"), str(DRIVER), "-o", str(exe),
                    "-L", str(lib.parent), f"-l:{lib.name}", f"-Wl,-rpath,{lib.parent}"],
                   check=True)
    data = tmp / "case.bin"
    _write_case(data)
    env = dict(os.environ)
    # leak checking on the CPU only: the HIP runtime keeps allocations of its
    # own until exit on a GPU box
    env["ASAN_OPTIONS"] = f"halt_on_error=1:detect_leaks={int(detect_leaks)}:exitcode=23"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    res = subprocess.run([str(exe), str(data)], capture_output=True, text=True, timeout=300,
                         env=env)
    assert res.returncode == 0, (res.returncode, res.stdout[-2000:], res.stderr[-6000:])
    assert "ERROR: AddressSanitizer" not in res.stderr
    assert "runtime error" not in res.stderr  # UBSan
    return res.stdout


@pytest.mark.skipif(not CLANG.exists(), reason="ROCm clang not installed")
def test_host_paths_under_sanitizers(tmp_path):
    if torch.cuda.is_available():
        pytest.skip("the GPU variant below runs on a GPU box")
    out = _run_driver(tmp_path, _sanitized_library(tmp_path), detect_leaks=True)
    assert "sanitizer driver ok (host paths" in out


@pytest.mark.gpu
@pytest.mark.skipif(not CLANG.exists(), reason="ROCm clang not installed")
def test_device_lifecycle_under_host_sanitizers(tmp_path):
    if not IN_TREE.exists():
        pytest.fail(f"sanitized library not built at {IN_TREE} (run __graft_entry__.build())")
    print("[gpu] sanitized host code: ring, appends, dense, destroy", flush=True)
    out = _run_driver(tmp_path, IN_TREE, detect_leaks=False)  # built beforehand
    assert "sanitizer driver ok (device lifecycle)" in out
