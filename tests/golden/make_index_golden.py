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
"""

from __future__ import annotations

import hashlib
import json
import sys
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


def main(reference_src: str) -> None:
    # the reference checkout is read-only input: no bytecode caches there
    sys.dont_write_bytecode = True
    sys.path.insert(0, reference_src)
    from seoulkv4._clustering import _refined_hierarchical_ivf  # reference IVF
    from seoulkv4._index_build import build_stage1_cell  # the reference builder

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
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")
