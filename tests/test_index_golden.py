"""Index builder against golden vectors written by the reference's own builder
(``tests/golden/make_index_golden.py``: ``build_stage1_cell``,
``_index_build.py:23-59``, and ``_refined_hierarchical_ivf``,
``_clustering.py:73-236``), plus the NPZ dump/load round trip and the cell
invariants (``_codecs/index.py:97-116``).  CPU only."""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from seoulkv_amd import SeoulKV4Index
from seoulkv_amd._clustering import hierarchical_ivf
from seoulkv_amd._codecs import validate_static_cell
from seoulkv_amd.index import build_cell, centroid_count
from seoulkv_amd.synthetic import make_cache

GOLDEN = Path(__file__).resolve().parent / "golden" / "index_cells.npz"
FULL = ("upper", "lower", "scale", "group_fine_scale", "coarse_residual_norm", "offsets", "values")


@pytest.fixture(scope="module")
def golden():
    z = np.load(GOLDEN)  # allow_pickle stays False: plain arrays + JSON text
    return z, json.loads(str(z["meta"])), json.loads(str(z["ivf_meta"]))


def digest(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def _raw(t: torch.Tensor) -> np.ndarray:
    return (t.view(torch.int16) if t.dtype == torch.float16 else t).numpy()


@pytest.mark.parametrize("i", range(3))
def test_build_cell_matches_reference_builder(golden, i):
    z, meta, _ = golden
    m = meta[i]
    k, _, _ = make_cache(m["context"], max(m["components"], 1), clustered=m["clustered"],
                         sink=m["sink"], local=m["local"])
    r0, r1 = m["sink"], m["context"] - m["local"]
    cell = build_cell(k[m["head"]], p=m["p"], lam=0.0625, seed=m["seed"], r0=r0, r1=r1,
                      nc=centroid_count(r1 - r0))
    assert cell["key_hash"] == m["key_hash"]
    assert cell["builder"] == m["builder"]
    for f in FULL:
        assert np.array_equal(_raw(cell[f]), z[f"{m['name']}/{f}"]), f
    for f, want in m["digests"].items():
        assert digest(cell[f]) == want, f
    assert cell["max_codec_error"] == pytest.approx(m["max_codec_error"], abs=0)
    validate_static_cell(cell)


def _ivf_keys(n: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, 256, generator=g)
    return x / x.norm(dim=-1, keepdim=True)


@pytest.mark.parametrize("i", range(3))
def test_hierarchical_ivf_matches_reference(golden, i):
    z, _, ivf = golden
    m = ivf[i]
    cen, vals, off, _, labs, stats = hierarchical_ivf(
        _ivf_keys(m["n"], m["seed"]), m["n_leaves"], 2, m["seed"], coarse_clusters=m["coarse"]
    )
    out = dict(centroids=cen, values=vals, offsets=off, labels=labs)
    for field, value in out.items():
        key = f"{m['name']}/{field}"
        if key in z.files:
            assert np.array_equal(value.numpy(), z[key]), field
        else:
            assert digest(value) == m["digests"][field], field
    assert stats == m["stats"]


def test_index_dump_load_round_trip(tmp_path):
    k, v, _ = make_cache(8192, 256, clustered=True)
    index = SeoulKV4Index.build(k, v, nprobe=64, n_centroids=512)
    path = tmp_path / "cache.npz"
    index.dump(path)
    loaded = SeoulKV4Index.load(path)
    assert loaded.metadata() == index.metadata()
    for a, b in zip(index.cells, loaded.cells):
        for f in FULL + ("centroids",):
            assert torch.equal(a[f].view(torch.uint8) if a[f].dtype.is_floating_point else a[f],
                               b[f].view(torch.uint8) if b[f].dtype.is_floating_point else b[f]), f
    reprobed = SeoulKV4Index.load(path, nprobe=32)
    assert [c["p"] for c in reprobed.cells] == [32] * 4
    loaded._check_keys(k)
    with pytest.raises(ValueError):
        loaded._check_keys(v)  # a different cache does not match the key fingerprint


def test_cell_invariants_reject_broken_csr():
    k, _, _ = make_cache(8192, 256, clustered=True)
    cell = build_cell(k[0], p=64, lam=0.0625, seed=0, r0=128, r1=8192 - 256, nc=512)
    validate_static_cell(cell)
    bad = dict(cell, values=cell["values"].clone())
    bad["values"][0] = 0  # a sink token posted in a list
    with pytest.raises(AssertionError):
        validate_static_cell(bad)
    bad = dict(cell, offsets=cell["offsets"].clone())
    bad["offsets"][5] = bad["offsets"][6] + 1  # non-monotone CSR
    with pytest.raises(AssertionError):
        validate_static_cell(bad)
