"""Query-independent IVF index over four KV heads (host prefill).

Mirrors ``SeoulKV4Index`` (reference ``index.py:38-189``): ``build`` clusters
the retrieval range of each KV head into spill-2 posting lists with 4-bit
group-scale centroid codes, ``dump``/``load`` persist it as NPZ version 4, and
``load(nprobe=...)`` overrides the probe budget without rebuilding.

Extensions (both are needed by the MI355X benchmark profiles and keep the
reference behaviour when left at their defaults):

* ``n_centroids=`` sets the centroid count per head; the default is the
  reference's ``ceil(R / 128) * 32`` for R retrieval tokens.
* contexts up to 2**20 tokens are accepted (the reference stops at 524288);
  device selection keys carry 20-bit token IDs.
"""

from __future__ import annotations

import math
from collections.abc import Sequence
from numbers import Real
from pathlib import Path

import numpy as np
import torch

from seoulkv_amd._clustering import hierarchical_ivf, midrise
from seoulkv_amd._codecs import (
    GROUP,
    QUERY_FIELDS,
    dump_index,
    encode_group_scale_cell,
    fingerprint,
    load_index,
    require_group_scale_cell,
    validate_static_cell,
)
from seoulkv_amd._zones import AttentionZones
from seoulkv_amd.config import DEFAULT_NPROBE, MAX_CENTROIDS, MAX_CONTEXT, STAGE15_M

MIN_CONTEXT = 6400


def centroid_count(retrieval_tokens: int) -> int:
    """About four keys per centroid before spill, padded to whole 32-centroid
    scale groups (reference ``_index_build.py:16-19``)."""
    return math.ceil(retrieval_tokens / (4 * GROUP)) * GROUP


def probe_counts(nprobe, nc: int) -> tuple[int, ...]:
    """One probe budget per KV head: a multiple of 16 in [16, min(512, nc)]
    (reference ``index.py:24-35``)."""
    if type(nprobe) is int:
        probes = (nprobe,) * 4
    elif isinstance(nprobe, Sequence) and not isinstance(nprobe, (str, bytes)):
        probes = tuple(nprobe)
    else:
        raise ValueError("nprobe must be an integer or four per-head integers")
    if len(probes) != 4 or any(
        type(p) is not int or not 16 <= p <= min(512, nc) or p % 16 for p in probes
    ):
        raise ValueError(f"each nprobe must be a multiple of 16 in [16, {min(512, nc)}]")
    return probes


@torch.no_grad()
def build_cell(k, *, p, lam, seed, r0, r1, nc, device=None, coarse_clusters=128, iters=10):
    """Index one KV head: normalise its retrieval keys, cluster, encode
    (reference ``build_stage1_cell`` ``_index_build.py:23-59``)."""
    if not 0 <= r0 < r1 <= len(k) or r1 - r0 < nc or not 0 < p <= nc:
        raise ValueError("not enough retrieval keys for spill2 / requested nprobe")
    x = k[r0:r1].to(device=device or k.device, dtype=torch.float32)
    if not torch.isfinite(x).all():
        raise ValueError("retrieval keys must be finite")
    x = x / x.norm(dim=-1, keepdim=True).clamp_min(1e-9)
    cen, values, offsets, _, _, stats = hierarchical_ivf(
        x,
        nc,
        2,
        seed,
        coarse_clusters=min(coarse_clusters, max(2, nc // 2)),
        local_iters=iters,
    )
    cell, _ = encode_group_scale_cell(
        dict(
            centroids=midrise(cen, 4).half().cpu(),
            offsets=offsets.cpu().int(),
            values=values.cpu().int() + r0,
            context=len(k),
            r0=r0,
            r1=r1,
            spill=2,
            p=p,
            lam=lam,
            seed=seed,
            key_hash=fingerprint(k.cpu().bfloat16()),
            builder=stats,
        )
    )
    validate_static_cell(cell)
    return cell


def posting_pairs(cell) -> np.ndarray:
    """[tokens][2]: the two posting lists (ascending) of each listed token of
    a spill-2 cell, rows in token order, from its CSR (``offsets``,
    ``values``).  Two builds of the same keys agree on a token when its row
    matches."""
    off = cell["offsets"].numpy().astype(np.int64)
    vals = cell["values"].numpy().astype(np.int64)
    lists = np.repeat(np.arange(len(off) - 1), np.diff(off))
    order = np.lexsort((lists, vals))
    return lists[order].reshape(-1, 2)



def list_agreement(a, b) -> float:
    """How far two builds of the same keys put tokens in the same posting
    lists, whatever the lists' numbering: each list of ``b`` is matched to the
    list of ``a`` holding most of its tokens, and the result is the fraction
    of ``b``'s (token, list) memberships whose token is in the matched list
    (1.0: the same partition).  A leaf allocation that differs by one leaf
    renumbers every later list, which a per-ID comparison would count as a
    total mismatch."""
    pa, pb = posting_pairs(a), posting_pairs(b)
    if pa.shape != pb.shape:
        raise ValueError("the cells list different token sets")
    na = int(pa.max()) + 1
    # every token joins its 2 lists in b with its 2 lists in a: 4 (b, a) pairs
    pairs = (pb[:, :, None].astype(np.int64) * na + pa[:, None, :]).reshape(-1)
    keys, counts = np.unique(pairs, return_counts=True)
    best = np.zeros(int(pb.max()) + 1, dtype=np.int64)
    np.maximum.at(best, keys // na, counts)
    return float(best.sum()) / pb.size



def posting_cosine(cell, k) -> float:
    """Clustering quality of a cell over its KV head's keys ``k`` [T][256]:
    the mean, over the retrieval tokens, of the cosine between a token's
    normalised key and the nearer of its two lists' centroids (the stored
    BF16 centroids).  Two builds of the same keys that differ only in which
    near-tied assignments they took score the same to ~1e-3."""
    r0, r1 = int(cell["r0"]), int(cell["r1"])
    x = k[r0:r1].float()
    x = x / x.norm(dim=-1, keepdim=True).clamp_min(1e-9)
    c = cell["centroids"].float()
    c = c / c.norm(dim=-1, keepdim=True).clamp_min(1e-9)
    pairs = torch.from_numpy(posting_pairs(cell))
    cos = torch.stack([(x * c[pairs[:, j]]).sum(-1) for j in range(2)]).amax(0)
    return float(cos.mean())


class SeoulKV4Index:
    """Query-independent CPU index for four ordered KV heads."""

    def __init__(self, cells, metadata):
        if len(cells) != 4:
            raise ValueError("SeoulKV4 requires four ordered index cells")
        self._zones = AttentionZones.from_cells(cells, context=int(cells[0]["context"]))
        self._zones.count()
        self._cells = tuple(
            {
                name: value
                for name, value in require_group_scale_cell(cell).items()
                if name not in QUERY_FIELDS
            }
            for cell in cells
        )
        if len({len(cell["centroids"]) for cell in self._cells}) != 1:
            raise ValueError("all index cells must have the same centroid count")
        self._nprobe_source = metadata.get("nprobe_source")

    @classmethod
    def load(cls, path: str | Path, *, nprobe=None) -> "SeoulKV4Index":
        """Read an index; legacy replay queries are discarded and ``nprobe``
        optionally overrides the saved probe budget."""
        cells, metadata = load_index(path)
        if nprobe is not None:
            if len(cells) != 4:
                raise ValueError("SeoulKV4 requires four ordered index cells")
            probes = probe_counts(nprobe, min(len(cell["centroids"]) for cell in cells))
            cells = [dict(cell, p=p) for cell, p in zip(cells, probes, strict=True)]
            metadata = dict(metadata, nprobe_source="load override")
        return cls(cells, metadata)

    def dump(self, path: str | Path) -> None:
        """Save the static index as an NPZ that ``load()`` can reopen."""
        dump_index(path, self._cells, {"nprobe_source": self._nprobe_source})

    @classmethod
    def build(
        cls,
        k: torch.Tensor,
        v: torch.Tensor | None = None,
        *,
        sink: int = 128,
        local: int = 256,
        nprobe=DEFAULT_NPROBE,
        lam: float = 0.0625,
        seed: int = 0,
        build_device="cpu",
        n_centroids: int | None = None,
    ) -> "SeoulKV4Index":
        """Index CPU BF16 post-RoPE K [4, T, 256]; V is only shape-checked.

        PyTorch may cluster on the CPU or on a GPU (``build_device``); the
        returned index is always CPU-resident and holds no query or V data.
        """
        if not (
            isinstance(k, torch.Tensor)
            and k.device.type == "cpu"
            and k.dtype == torch.bfloat16
            and k.ndim == 3
            and k.shape[0] == 4
            and k.shape[2] == 256
        ):
            raise ValueError("expected CPU BF16 post-RoPE K [4,T,256]")
        if v is not None and not (
            isinstance(v, torch.Tensor)
            and v.device == k.device
            and v.dtype == k.dtype
            and v.shape == k.shape
        ):
            raise ValueError("V must match K's shape, dtype, and CPU device")
        context = k.shape[1]
        if not MIN_CONTEXT <= context <= MAX_CONTEXT or context % 4:
            raise ValueError("unsupported context for the fixed SeoulKV4 profile")
        if type(sink) is not int or type(local) is not int:
            raise ValueError("sink and local must be integer token counts")
        zones = AttentionZones(context, sink, local)
        retrieval = zones.local_begin - sink
        if retrieval < STAGE15_M:
            raise ValueError(
                f"retrieval zone needs at least {STAGE15_M} keys "
                "for the fixed Stage-1.5 profile"
            )
        if n_centroids is None:
            nc = centroid_count(retrieval)
        else:
            if type(n_centroids) is not int or n_centroids <= 0 or n_centroids % GROUP:
                raise ValueError("n_centroids must be a positive multiple of 32")
            if n_centroids > retrieval:
                raise ValueError("n_centroids exceeds the retrieval token count")
            nc = n_centroids
        if nc > MAX_CENTROIDS:
            raise ValueError("centroid count exceeds the Fine selector's 16-bit positions")
        probes = probe_counts(nprobe, nc)
        if isinstance(lam, bool) or not isinstance(lam, Real) or not (
            math.isfinite(lam) and lam >= 0
        ):
            raise ValueError("lam must be finite and nonnegative")
        if type(seed) is not int or not 0 <= seed <= 2**63 - 1:
            raise ValueError("seed must be a nonnegative signed 64-bit integer")
        device = torch.device(build_device)
        if device.type not in ("cpu", "cuda"):
            raise ValueError("build_device must be a PyTorch CPU or CUDA device")
        if device.type == "cuda" and not torch.cuda.is_available():
            raise ValueError("build_device requests CUDA, but PyTorch CUDA is unavailable")
        cells = [
            build_cell(
                k[head],
                p=p,
                lam=float(lam),
                seed=seed,
                r0=sink,
                r1=zones.local_begin,
                nc=nc,
                device=device,
            )
            for head, p in enumerate(probes)
        ]
        return cls(cells, {"nprobe_source": "explicit (build)"})

    @property
    def cells(self) -> tuple:
        return self._cells

    @property
    def zones(self) -> AttentionZones:
        return self._zones

    @property
    def n_centroids(self) -> int:
        return len(self._cells[0]["centroids"])

    def _check_keys(self, k) -> None:
        for i, cell in enumerate(self._cells):
            if fingerprint(k[i]) != cell["key_hash"]:
                raise ValueError(f"Stage-I index K fingerprint mismatch at cell {i}")

    def metadata(self) -> dict:
        return {
            **self._zones.metadata(),
            "summary_codec": "group-scale-32-v1",
            "nprobe": [int(cell["p"]) for cell in self._cells],
            "lambda": [float(cell["lam"]) for cell in self._cells],
            "key_hashes": [cell["key_hash"] for cell in self._cells],
            "nprobe_source": self._nprobe_source,
            "n_centroids": self.n_centroids,
        }
