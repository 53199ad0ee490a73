"""The boundary from plain C, without a GPU: include/seoulkv4_hip.h compiles as
C99 and a C program linked against libseoulkv4_hip.so reaches its entry points
(the calls here fail their argument checks before any device work, as a
cgo / JNI / N-API binding would see them)."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

from seoulkv_amd import _hip

ROOT = Path(__file__).resolve().parents[1]
PROGRAM = r"""
#include <stdio.h>
#include <string.h>
#include "seoulkv4_hip.h"

int main(void) {
  void *h = (void *)1;
  skv_index_desc ix;
  skv_kv_pages pages;
  int code;
  memset(&ix, 0, sizeof ix);
  memset(&pages, 0, sizeof pages);
  if (strncmp(skv_version(), "seoulkv4-hip", 12) != 0) return 10;
  if (skv_kernel_count() != 7) return 11;
  /* NULL index: rejected before any device work, handle cleared */
  code = skv_create(NULL, NULL, NULL, 0, NULL, &h);
  if (code != SKV_EINVAL || h != NULL) return 12;
  /* a page descriptor without a pool */
  ix.context = 8192; ix.sink = 128; ix.local = 256; ix.n_centroids = 512;
  code = skv_create_paged(&ix, (const uint16_t *)&ix, (const uint16_t *)&ix, NULL, 0, NULL, &h);
  if (code != SKV_EINVAL || strstr(skv_last_error(NULL), "page") == NULL) return 13;
  /* a closed (NULL) handle */
  if (skv_enqueue(NULL) != SKV_ESTATE) return 14;
  printf("c caller ok: %s\n", skv_version());
  return 0;
}
"""


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not installed")
def test_header_compiles_as_c99():
    subprocess.run(["gcc", "-fsyntax-only", "-std=c99", "-Wall", "-Wextra", "-pedantic",
                    "-Werror", "-x", "c", str(ROOT / "include" / "seoulkv4_hip.h")], check=True)


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not installed")
def test_c_program_calls_the_library(tmp_path):
    lib = _hip.LIB_PATH
    if not lib.exists():
        pytest.fail(f"library not built at {lib}")
    src = tmp_path / "caller.c"
    src.write_text(PROGRAM)
    exe = tmp_path / "caller"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", str(ROOT / "include"), str(src),
                    "-o", str(exe), "-L", str(lib.parent), "-lseoulkv4_hip",
                    f"-Wl,-rpath,{lib.parent}"], check=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, (res.returncode, res.stdout, res.stderr)
    assert "c caller ok" in res.stdout
