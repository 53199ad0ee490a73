"""An index archive written by the reference's own writer, loaded here.

``tests/golden/ref_index_v4.npz.xz`` holds the bytes of a four-cell v4 NPZ
that the reference's ``SeoulKV4Index.dump`` wrote (``index.py:74-76`` ->
``dump_index``, ``_codecs/index.py:220-230``; generator:
``tests/golden/make_index_golden.py``), xz-compressed.  The archive is data:
it is decompressed and read with ``numpy.load(allow_pickle=False)`` through
this package's loader.  Checks: it loads (format compatibility with the
reference's writer); its cells equal this package's builder on the same
seeded keys, array for array and bit for bit; this package's writer emits the
same array names, dtypes and metadata fields, and its archive reloads to
equal cells; the ``nprobe`` override applies.  CPU only."""

from __future__ import annotations

import json
import lzma
from pathlib import Path

import numpy as np
import pytest
import torch

from seoulkv_amd import SeoulKV4Index
from seoulkv_amd.index import build_cell, centroid_count
from seoulkv_amd.synthetic import make_cache

ARCHIVE = Path(__file__).resolve().parent / "golden" / "ref_index_v4.npz.xz"
# the generator's case: (context, components, sink, local, p, seed)
CASE = (1024, 32, 64, 128, 32, 0)


@pytest.fixture(scope="module")
def ref_path(tmp_path_factory):
    path = tmp_path_factory.mktemp("ref") / "ref_index_v4.npz"
    path.write_bytes(lzma.decompress(ARCHIVE.read_bytes()))
    return path


@pytest.fixture(scope="module")
def own_cells():
    context, comps, sink, local, p, seed = CASE
    k, _, _ = make_cache(context, comps, clustered=True, sink=sink, local=local)
    r0, r1 = sink, context - local
    return [build_cell(k[h], p=p, lam=0.0625, seed=seed, r0=r0, r1=r1,
                       nc=centroid_count(r1 - r0)) for h in range(4)]


def _same(a, b) -> bool:
    if isinstance(a, torch.Tensor):
        return (isinstance(b, torch.Tensor) and a.dtype == b.dtype and a.shape == b.shape
                and torch.equal(a.view(torch.uint8) if a.dtype == torch.bfloat16 else a,
                                b.view(torch.uint8) if b.dtype == torch.bfloat16 else b))
    return a == b


def test_reference_archive_loads_and_equals_own_build(ref_path, own_cells):
    index = SeoulKV4Index.load(ref_path)
    loaded = index._cells
    assert len(loaded) == 4
    for h, (got, want) in enumerate(zip(loaded, own_cells)):
        want = {k: v for k, v in want.items() if k in got}
        assert set(got) == set(want), f"cell {h} fields"
        for name in got:
            assert _same(got[name], want[name]), f"cell {h} field {name}"
    meta = index.metadata()
    assert meta["nprobe"] == [CASE[4]] * 4
    assert meta["nprobe_source"] == "explicit (build)"


def test_own_writer_matches_reference_layout(ref_path, tmp_path):
    index = SeoulKV4Index.load(ref_path)
    mine = tmp_path / "own.npz"
    index.dump(mine)
    with np.load(ref_path, allow_pickle=False) as zr, np.load(mine, allow_pickle=False) as zo:
        assert set(zr.files) == set(zo.files)
        for name in zr.files:
            if name == "metadata":
                continue
            assert zr[name].dtype == zo[name].dtype and zr[name].shape == zo[name].shape, name
            assert np.array_equal(zr[name], zo[name]), name
        mr, mo = json.loads(str(zr["metadata"])), json.loads(str(zo["metadata"]))
    assert mr == mo
    again = SeoulKV4Index.load(mine)
    for a, b in zip(again._cells, index._cells):
        assert set(a) == set(b)
        assert all(_same(a[n], b[n]) for n in a)


def test_reference_archive_nprobe_override(ref_path):
    index = SeoulKV4Index.load(ref_path, nprobe=16)
    assert index.metadata()["nprobe"] == [16] * 4
    assert index.metadata()["nprobe_source"] == "load override"
    with pytest.raises(ValueError):
        SeoulKV4Index.load(ref_path, nprobe=24)  # not a multiple of 16
