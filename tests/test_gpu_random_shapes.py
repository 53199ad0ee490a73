"""Seeded random shapes through the whole decode step against the CPU oracle.

Each case draws a context that is a multiple of 4 (the index takes no
other) but not of 64, a centroid count that is a multiple of 32 but not of
128, a probe budget per KV head (four different multiples of 16, up to
every cluster), sink and local windows of any size, and clustered or
i.i.d. keys.  It checks the status words, the selected clusters, the pool
(encounter order), U1, U2 and the top-100 IDs bit for bit, and the
attention output within max-abs 2e-2 / cosine 0.999 per query head.  The
fixed shapes of ``test_gpu_parity.py`` check every intermediate score;
these check that shapes nobody picked by hand reach the same results, on
every selection path (forced full, forced-miss and radix selections give
the oracle's IDs and the default path's output bits).  The
odd seeds keep the FP8 records in pages of a random power-of-two size
(16 .. 1024 tokens) handed out in a random order.  ``SKV_RANDOM_SHAPES=N``
runs N seeds instead of the default 10; the long caches of
``test_wide_random_shape_matches_the_oracle`` (1 by default,
``SKV_RANDOM_WIDE=N``) take the paths of long centroid lists and pools.
"""

from __future__ import annotations

import os
import random

import numpy as np
import pytest
import torch

from seoulkv_amd import KVPagePool, _hip
from seoulkv_amd.index import MIN_CONTEXT
from tests.helpers import case, cosine, oracle_step

pytestmark = pytest.mark.gpu


def _shape(seed: int) -> dict:
    rng = np.random.default_rng(seed)
    nc = int(rng.choice([96, 160, 224, 352, 480, 608, 736, 864]))
    # the index takes multiples of 4 from MIN_CONTEXT on
    context = max(4 * int(rng.integers(1500, 6000)), MIN_CONTEXT)
    context += 4 if context % 64 == 0 else 0
    sink = int(rng.integers(0, 200))
    local = int(rng.integers(16, 400))
    top = max(16, min(512, nc) // 16 * 16)
    nprobe = tuple(int(x) for x in rng.choice(np.arange(16, top + 1, 16), size=4))
    clustered = bool(rng.integers(0, 2))
    return dict(context=context, components=int(rng.integers(8, 400)), nc=nc, nprobe=nprobe,
                clustered=clustered, sink=sink, local=local, seed_shift=1000 + seed)


def _wide_shape(seed: int) -> dict:
    """Long caches past the register-resident selections: more than 8192
    centroids per head (the tile-maxima threshold path), pools of tens of
    thousands of keys (the sampled-cut top-1600)."""
    rng = np.random.default_rng(10_000 + seed)
    nc = 32 * int(rng.integers(257, 513))  # 8224 .. 16384
    context = 4 * int(rng.integers(10000, 40000))  # 40K .. 160K
    context += 4 if context % 64 == 0 else 0
    sink = int(rng.integers(0, 200))
    local = int(rng.integers(16, 400))
    nprobe = tuple(int(x) for x in rng.choice(np.arange(16, 513, 16), size=4))
    return dict(context=context, components=int(rng.integers(512, 8192)), nc=nc, nprobe=nprobe,
                clustered=bool(rng.integers(0, 2)), sink=sink, local=local,
                seed_shift=5000 + seed)


# 10 seeds by default; SKV_RANDOM_SHAPES=N runs seeds 0 .. N-1 (a wider sweep)
SEEDS = list(range(int(os.environ.get("SKV_RANDOM_SHAPES", "10"))))
# 1 long cache by default; SKV_RANDOM_WIDE=N runs N
WIDE_SEEDS = list(range(int(os.environ.get("SKV_RANDOM_WIDE", "1"))))


@pytest.mark.parametrize("seed", SEEDS)
def test_random_shape_matches_the_oracle(seed):
    _check(_shape(seed), seed, f"random shape {seed}")


@pytest.mark.parametrize("seed", WIDE_SEEDS)
def test_wide_random_shape_matches_the_oracle(seed):
    _check(_wide_shape(seed), seed, f"wide random shape {seed}")


def _check(p: dict, seed: int, label: str) -> None:
    index, k, v, qs = case(**p)
    print(f"[gpu] {label}: {p}", flush=True)
    kv_pages = None
    if seed % 2:
        page_tokens = 16 << (seed % 7)
        need = -(-p["context"] // page_tokens)
        pool = KVPagePool(need + 9, page_tokens=page_tokens, device="cuda:0")
        pages = pool.allocate(pool.n_pages)
        random.Random(seed).shuffle(pages)
        kv_pages = (pool, pages[:need])
        print(f"[gpu]   paged records, {page_tokens}-token pages", flush=True)
    rt = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=True,
                      kv_pages=kv_pages)
    try:
        rt.bind_query(qs[0])
        rt.enqueue()
        status = rt.synchronize()
        traces, out = oracle_step(p, qs[0])
        assert status["err"] == [0, 0, 0, 0]
        for g, tr in enumerate(traces):
            assert status["pool"][g] == len(tr.pool), f"g{g} pool size"
            np.testing.assert_array_equal(rt.read_stage("selected", g), tr.selected,
                                          err_msg=f"g{g} selected")
            np.testing.assert_array_equal(rt.read_stage("pool", g), tr.pool, err_msg=f"g{g} pool")
            np.testing.assert_array_equal(rt.read_stage("u1", g), tr.u1, err_msg=f"g{g} u1")
            np.testing.assert_array_equal(rt.read_stage("u2", g), tr.u2, err_msg=f"g{g} u2")
            np.testing.assert_array_equal(rt.read_stage("top", g), tr.top100,
                                          err_msg=f"g{g} top100")
        got = rt.read_output().float().numpy().reshape(16, 256)
        for j in range(16):
            assert np.abs(got[j] - out[j]).max() <= 2e-2, f"head {j} max-abs"
            assert cosine(got[j], out[j]) >= 0.999, f"head {j} cosine"
        # every other selection path: full selections (1), sampled cuts
        # forced to miss (2), in-memory radix passes (3) give the same IDs
        # and the same output bits
        want = rt.read_output().view(torch.int16).clone()
        for mode in (1, 2, 3):
            rt.select_mode(mode)
            try:
                rt.bind_query(qs[0])
                rt.enqueue()
                assert rt.synchronize()["err"] == [0, 0, 0, 0], mode
            finally:
                rt.select_mode(0)
            for g, tr in enumerate(traces):
                np.testing.assert_array_equal(rt.read_stage("top", g), tr.top100,
                                              err_msg=f"mode {mode} g{g} top100")
            assert torch.equal(rt.read_output().view(torch.int16), want), f"mode {mode} output"
    finally:
        rt.close()
