"""Legacy grouped fixtures (NPZ versions 1-3) load as indexes.

The reference wrote replay fixtures before its query-free version-4 index
(``_codecs/index.py:184-211``, ``save_fixture`` ``:214-220``): per-cell arrays
``"{i}_{name}"`` with BF16 tensors widened to float32, the cell's replay query
(``q``, ``query_hash``, ``coarse_ids``, ``head_mask``) and JSON metadata with
the version.  Version 1 files may lack the coarse operands, which the loader
derives (``ensure_coarse_metadata`` ``:52-63``).  These tests write such
files from an index built here, in that layout, and check what
``SeoulKV4Index.load`` returns (``_load_archive`` ``:130-177``): the replay
query is discarded and every static array survives bit for bit.
"""

from __future__ import annotations

import json

import numpy as np
import pytest
import torch

from seoulkv_amd import SeoulKV4Index
from seoulkv_amd._codecs import QUERY_FIELDS
from tests.helpers import case

COARSE = ("coarse2", "coarse_odd", "coarse_residual_norm")


def _legacy_arrays(cells, version, drop=()):
    """The reference's pre-version-4 archive layout (float32 for BF16)."""
    data, rows = {}, []
    for i, cell in enumerate(cells):
        scalars = {}
        for name, value in cell.items():
            if name in drop:
                continue
            if isinstance(value, torch.Tensor):
                if value.dtype == torch.bfloat16:
                    value = value.float()
                data[f"{i}_{name}"] = value.contiguous().numpy()
            else:
                scalars[name] = value
        rows.append(scalars)
    data["metadata"] = np.array(json.dumps({"version": version, "cells": rows}))
    return data


def _with_replay_query(cells, seed=5):
    """Add a valid replay query to every cell: a BF16 query, ascending coarse
    IDs and head masks that admit at least p centroids per head."""
    g = torch.Generator().manual_seed(seed)
    out = []
    for cell in cells:
        nc = len(cell["centroids"])
        ids = torch.arange(0, nc, 2, dtype=torch.int32)
        mask = torch.full((len(ids),), 15, dtype=torch.int32)
        q = torch.randn(4, 256, generator=g).bfloat16()
        out.append(dict(cell, q=q, query_hash="replay", coarse_ids=ids, head_mask=mask))
    return out


@pytest.fixture(scope="module")
def built():
    return case(context=8192, components=64, nc=256, nprobe=16, sink=0, local=64)[0]


@pytest.mark.parametrize("version", [1, 2, 3])
def test_legacy_fixture_loads_as_index(tmp_path, built, version):
    cells = _with_replay_query(built.cells)
    drop = COARSE if version == 1 else ()
    path = tmp_path / f"fixture_v{version}.npz"
    np.savez(path, **_legacy_arrays(cells, version, drop))
    loaded = SeoulKV4Index.load(path)
    for orig, got in zip(built.cells, loaded.cells):
        assert not QUERY_FIELDS.intersection(got)  # the replay query is discarded
        for name, value in orig.items():
            if not isinstance(value, torch.Tensor) or name in drop:
                continue
            want = value.float() if value.dtype == torch.bfloat16 else value
            assert torch.equal(got[name], want), name
        for name in COARSE:  # present (kept or derived) and well formed
            assert got[name].shape[0] == len(orig["centroids"])
    if version == 1:  # derived from the stored centroids and planes
        for orig, got in zip(built.cells, loaded.cells):
            assert torch.equal(got["coarse_odd"].float(), orig["coarse_odd"].float())


def test_legacy_fixture_with_bad_replay_query_is_rejected(tmp_path, built):
    cells = _with_replay_query(built.cells)
    cells[2] = dict(cells[2], head_mask=torch.zeros_like(cells[2]["head_mask"]))
    path = tmp_path / "bad.npz"
    np.savez(path, **_legacy_arrays(cells, 3))
    with pytest.raises(AssertionError):
        SeoulKV4Index.load(path)


def test_unsupported_and_incomplete_archives_are_rejected(tmp_path, built):
    path = tmp_path / "v5.npz"
    data = _legacy_arrays(_with_replay_query(built.cells), 3)
    data["metadata"] = np.array(json.dumps({"version": 5, "cells": []}))
    np.savez(path, **data)
    with pytest.raises(ValueError, match="version"):
        SeoulKV4Index.load(path)
    # a version-4 index must hold every BF16 array its manifest declares
    good = tmp_path / "v4.npz"
    built.dump(good)
    with np.load(good, allow_pickle=False) as z:
        arrays = {name: z[name] for name in z.files}
    meta = json.loads(str(arrays["metadata"]))
    missing = meta["bf16_arrays"][0]
    del arrays[missing]
    bad = tmp_path / "v4_missing.npz"
    np.savez(bad, **arrays)
    with pytest.raises(ValueError, match="BF16"):
        SeoulKV4Index.load(bad)
