"""Write golden index cells from the reference's own index builder.

The IVF clustering (torch RNG stream + op order) is the one part of the index
that no closed form pins, so its expected outputs come from running the
reference builder ``build_stage1_cell`` (``_index_build.py:23-59``) on small,
seeded keys.  Run once in a container that has the reference checkout:

    python tests/golden/make_index_golden.py /root/reference/src

It writes ``tests/golden/index_cells.npz``: per case the generator parameters,
the full small arrays of the encoded cell and SHA-256 digests of the large
ones.  Tests regenerate the same keys and compare ``seoulkv_amd``'s builder
against these vectors; they never import the reference.

It also writes ``tests/golden/ref_index_v4.npz.xz``: the bytes of a whole
four-cell index archive written by the reference's own ``SeoulKV4Index.dump``
(``index.py:74-76`` -> ``_codecs/index.py:220-230``), xz-compressed for the
repository, so that loading an archive the reference wrote is tested, not
only this package's own writer.  ``--archive-only`` rewrites just that file.
"""

from __future__ import annotations

import hashlib
import json
import lzma
import sys
import tempfile
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from seoulkv_amd.synthetic import make_cache  # noqa: E402

# (name, context, components, clustered, sink, local, p, seed, head)
CASES = [
    ("clustered_t2048", 2048, 64, True, 64, 128, 64, 0, 0),
    ("iid_t2048_seed7", 2048, 0, False, 64, 128, 32, 7, 1),
    ("clustered_t4096_h3", 4096, 16, True, 128, 256, 128, 3, 3),
]
# Direct clustering cases small enough to take the "bucket solved alone"
# branch (more leaves than keys in a batch): (name, n, n_leaves, coarse, seed)
IVF_CASES = [
    ("ivf_n8_l32", 8, 32, 8, 5),
    ("ivf_n64_l48", 64, 48, 8, 11),
    ("ivf_n20000_l2048", 20000, 2048, 2, 2),  # one padded slab > 16 Mi scores
]
FULL = ("upper", "lower", "scale", "group_fine_scale", "coarse_residual_norm", "offsets", "values")
DIGEST = ("centroids", "coarse_centroids", "coarse2", "coarse_odd", "levels", "decoded")


def digest(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def ivf_keys(n: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, 256, generator=g)
    return x / x.norm(dim=-1, keepdim=True)


# the archive case: (context, components, sink, local, p, seed); four heads
ARCHIVE = (1024, 32, 64, 128, 32, 0)


def write_archive(build_stage1_cell, ref_index_cls) -> None:
    """Four cells built by the reference builder exactly as its
    ``SeoulKV4Index.build`` does (``index.py:146-157``; its 6400-token
    minimum context is a build-time profile check, not an archive property),
    dumped by the reference's own writer."""
    context, comps, sink, local, p, seed = ARCHIVE
    k, _, _ = make_cache(context, comps, clustered=True, sink=sink, local=local)
    cells = [
        build_stage1_cell(k[head], p=p, lam=0.0625, seed=seed, r0=sink, r1=context - local)
        for head in range(4)
    ]
    with tempfile.TemporaryDirectory() as tmp:
        raw = Path(tmp) / "ref_index_v4.npz"
        ref_index_cls(cells, {"nprobe_source": "explicit (build)"}).dump(raw)
        data = raw.read_bytes()
    path = HERE / "ref_index_v4.npz.xz"
    path.write_bytes(lzma.compress(data, preset=9))
    print("wrote", path, len(data), "archive bytes,", path.stat().st_size, "compressed")


def main(reference_src: str, archive_only: bool = False) -> None:
    # the reference checkout is read-only input: no bytecode caches there
    sys.dont_write_bytecode = True
    sys.path.insert(0, reference_src)
    from seoulkv4._clustering import _refined_hierarchical_ivf  # reference IVF
    from seoulkv4._index_build import build_stage1_cell  # the reference builder
    from seoulkv4.index import SeoulKV4Index as RefIndex  # the reference writer

    write_archive(build_stage1_cell, RefIndex)
    if archive_only:
        return

    arrays, meta = {}, []
    for name, context, comps, clustered, sink, local, p, seed, head in CASES:
        k, _, _ = make_cache(context, max(comps, 1), clustered=clustered, sink=sink, local=local)
        cell = build_stage1_cell(
            k[head], p=p, lam=0.0625, seed=seed, r0=sink, r1=context - local
        )
        entry = dict(
            name=name, context=context, components=comps, clustered=clustered,
            sink=sink, local=local, p=p, seed=seed, head=head,
            key_hash=cell["key_hash"], builder=cell["builder"],
            max_codec_error=cell["max_codec_error"],
            digests={f: digest(cell[f]) for f in DIGEST},
        )
        for f in FULL:
            value = cell[f]
            if value.dtype == torch.float16:
                value = value.view(torch.int16)
            arrays[f"{name}/{f}"] = value.numpy()
        meta.append(entry)
    ivf_meta = []
    for name, n, n_leaves, coarse, seed in IVF_CASES:
        cen, vals, off, counts, labs, stats = _refined_hierarchical_ivf(
            ivf_keys(n, seed), n_leaves, 2, seed, coarse_clusters=coarse
        )
        out = dict(centroids=cen, values=vals, offsets=off, labels=labs)
        digests = {}
        for field, value in out.items():
            if value.numel() <= 65536:
                arrays[f"{name}/{field}"] = value.numpy()
            else:
                digests[field] = digest(value)
        ivf_meta.append(dict(name=name, n=n, n_leaves=n_leaves, coarse=coarse,
                             seed=seed, stats=stats, digests=digests))
    arrays["ivf_meta"] = np.array(json.dumps(ivf_meta))
    arrays["meta"] = np.array(json.dumps(meta))
    np.savez_compressed(HERE / "index_cells.npz", **arrays)
    print("wrote", HERE / "index_cells.npz", [m["name"] for m in meta])


if __name__ == "__main__":
    args = [a for a in sys.argv[1:] if not a.startswith("--")]
    main(args[0] if args else "/root/reference/src", archive_only="--archive-only" in sys.argv)
