"""Dense FP8 decode (the comparison path) against the oracle's float64
softmax over all T keys of the same FP8 [V || K] records.

Tolerance: the north-star bound (max-abs <= 2e-2, cosine >= 0.999 per query
head) and, tighter, |out - ref| <= 2^-8 |ref| + 1e-4: the output is BF16 (RNE,
half an ulp <= 2^-8 relative) of an FP32 result, so a dropped query term
(2^-4 relative), a lost key or a wrong softmax scale fails it.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from oracle import arith
from oracle import decode as od
from seoulkv_amd import _hip
from tests.helpers import bits, case, cosine, oracle_inputs

pytestmark = pytest.mark.gpu

CASES = {
    # one tile per wave, 64 blocks per group
    "t8192": dict(context=8192, components=256, nc=512, nprobe=64),
    # a partial last tile and a last block with one busy wave
    "t8200_odd": dict(context=8200, components=64, nc=160, nprobe=32, sink=40, local=200,
                      seed_shift=3),
    # three tiles per wave, partial last tile and block
    "t40008": dict(context=40008, components=512, nc=1280, nprobe=128, seed_shift=5),
}


def dense_reference(params, q):
    _, _, _, k8, v8 = oracle_inputs(**params)
    qf = arith.bf16_to_f32(bits(q).reshape(16, 256))
    ids = np.arange(params["context"])
    return np.stack([od.sdpa(qf[j], k8[j // 4], v8[j // 4], ids) for j in range(16)])


def paged_records(context: int, page_tokens: int, seed: int):
    """(pool, page table): pages for the context, handed out in a seeded
    random order by a pool with spare pages."""
    from seoulkv_amd import KVPagePool

    need = -(-context // page_tokens)
    pool = KVPagePool(need + 3, page_tokens=page_tokens, device="cuda:0")
    pages = pool.allocate(pool.n_pages)
    random.Random(seed).shuffle(pages)
    return pool, pages[:need]


@pytest.mark.parametrize("name,page_tokens", [(n, None) for n in CASES] +
                         [("t8200_odd", 16), ("t40008", 64)])
def test_dense_decode_matches_oracle(name, page_tokens):
    """page_tokens: the FP8 records in pages of that size (16: every tile is a
    page; the odd contexts end in a partial tile of a partial page)."""
    p = CASES[name]
    index, k, v, qs = case(**p)
    print(f"[gpu] dense {name} pages {page_tokens}", flush=True)
    kv_pages = paged_records(p["context"], page_tokens, 7) if page_tokens else None
    rt = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=False,
                      kv_pages=kv_pages)
    try:
        for qi, q in enumerate(qs):
            rt.bind_query(q)
            rt.dense_decode()
            out = rt.read_dense_output().float().reshape(16, 256).numpy().astype(np.float64)
            ref = dense_reference(p, q)
            err = np.abs(out - ref)
            assert err.max() <= 2e-2, (name, qi, err.max())
            for j in range(16):
                assert cosine(out[j], ref[j]) >= 0.999, (name, qi, j)
            bad = err > np.abs(ref) * 2.0**-8 + 1e-4
            assert not bad.any(), (name, qi, int(bad.sum()), float(err.max()))
        # repeated decodes of one query are bit-identical (fixed merge order)
        rt.dense_decode()
        again = rt.read_dense_output()
        rt.dense_decode()
        assert torch.equal(rt.read_dense_output(), again)
    finally:
        rt.close()


def test_dense_decode_with_the_step_interleaved():
    """The dense decode and the sparse step share the handle's stream and
    the FP8 records; neither disturbs the other's output."""
    p = CASES["t8192"]
    index, k, v, qs = case(**p)
    rt = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=False)
    try:
        rt.bind_query(qs[0])
        rt.enqueue()
        step = rt.read_output()
        rt.dense_decode()
        dense = rt.read_dense_output()
        rt.enqueue()
        assert torch.equal(rt.read_output(), step)
        assert torch.equal(rt.read_dense_output(), dense)
        ms = rt.time_dense(reps=3)
        assert all(t > 0 for t in ms)
        assert torch.equal(rt.read_dense_output(), dense)
    finally:
        rt.close()
