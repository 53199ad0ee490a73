"""Paged FP8 K/V records on the GPU (``skv_create_paged``, ``KVPagePool``).

A paged instance keeps its FP8 [V || K] records in pages of a shared device
pool, in whatever physical order the pool's free list hands out, and reads
them through its page table.  Every result must be bit-identical to the
contiguous layout's on the same inputs (top-100 IDs, the attention output
bits, the dense decode's output bits, the records read back in token order),
the top-100 IDs must equal the oracle's, and the output must stay within the
north-star bound of the oracle (max-abs <= 2e-2, cosine >= 0.999).  Pages of
16 tokens put every 16-key tile and every sink/local slice across page
boundaries; pages of 4096 hold the whole sink and local window in two pages,
and one page of 65536 tokens holds the whole cache.
"""

from __future__ import annotations

import random

import numpy as np
import pytest
import torch

from seoulkv_amd import KVPagePool, SeoulKV4, SeoulKV4Config, _hip
from tests.helpers import bits, case, cosine, oracle_step
from tests.test_gpu_append import CAPACITY, P, fp8_bytes, new_tokens, oracle_grown

pytestmark = pytest.mark.gpu


def scrambled_pool(n_pages: int, page_tokens: int, seed: int) -> KVPagePool:
    """A pool whose free list hands out its pages in a seeded random order."""
    pool = KVPagePool(n_pages, page_tokens=page_tokens, device="cuda:0")
    pages = pool.allocate(n_pages)
    random.Random(seed).shuffle(pages)
    pool.release(pages)
    return pool


def step(rt, q):
    rt.bind_query(q)
    rt.enqueue()
    status = rt.synchronize()
    assert status["err"] == [0, 0, 0, 0]
    return rt.debug_ids().clone(), rt.read_output().view(torch.int16).clone(), status


def dense(rt):
    rt.dense_decode()
    return rt.read_dense_output().view(torch.int16).clone()


def runtimes(page_tokens: int, seed: int, append_capacity: int = 0):
    index, k, v, qs = case(**P)
    kw = dict(pool_min=0, pool_capacity=None, debug=True, append_capacity=append_capacity)
    flat = _hip.Runtime(0, k, v, index, **kw)
    need = -(-(P["context"] + append_capacity) // page_tokens)
    pool = scrambled_pool(need + 5, page_tokens, seed)
    table = pool.allocate(need)
    if table == sorted(table):  # few pages: make sure they are out of order
        table = table[::-1]
    paged = _hip.Runtime(0, k, v, index, kv_pages=(pool, table), **kw)
    return flat, paged, pool, table, qs


@pytest.mark.parametrize("page_tokens", [16, 32, 256, 4096, 65536])
def test_paged_step_matches_contiguous(page_tokens):
    print(f"[gpu] paged step, {page_tokens}-token pages", flush=True)
    flat, paged, pool, table, qs = runtimes(page_tokens, seed=page_tokens)
    try:
        assert paged.metadata()["kv_page_tokens"] == page_tokens
        assert flat.metadata()["kv_page_tokens"] == 0
        for qi, q in enumerate(qs):
            ids_f, out_f, st_f = step(flat, q)
            ids_p, out_p, st_p = step(paged, q)
            assert st_p == st_f, qi
            assert torch.equal(ids_p, ids_f), qi
            assert torch.equal(out_p, out_f), qi  # same records, same sums
            traces, ref = oracle_step(P, q)
            for g, tr in enumerate(traces):
                np.testing.assert_array_equal(paged.read_stage("top", g), tr.top100)
            got = paged.read_output().float().numpy().reshape(16, 256)
            for j in range(16):
                assert np.abs(got[j] - ref[j]).max() <= 2e-2, f"q{qi} head {j} max-abs"
                assert cosine(got[j], ref[j]) >= 0.999, f"q{qi} head {j} cosine"
            assert torch.equal(dense(paged), dense(flat)), qi
        for g in range(4):
            rec = paged.read_stage("kv8", g)
            np.testing.assert_array_equal(rec, flat.read_stage("kv8", g))
            np.testing.assert_array_equal(
                pool.gather(table, g, P["context"]).cpu().numpy().ravel(), rec)
    finally:
        paged.close()
        flat.close()


def test_paged_graph_replay_and_selection_paths():
    """16-token pages under graph replay (replayed several times, eager
    steps between) and with every selection path forced (full selection only,
    sampled cuts forced to miss): each step equals the contiguous instance's
    eager step bit for bit."""
    flat, paged, _, _, qs = runtimes(16, seed=5)
    try:
        want = [step(flat, q)[:2] for q in qs]
        paged.graph_mode(True)
        for rep in range(3):
            for qi, q in enumerate(qs):
                print(f"[gpu] paged graph replay {rep}, q{qi}", flush=True)
                ids, out, _ = step(paged, q)
                assert torch.equal(ids, want[qi][0]) and torch.equal(out, want[qi][1]), (rep, qi)
            paged.graph_mode(False)
            ids, out, _ = step(paged, qs[0])  # an eager step between replays
            assert torch.equal(out, want[0][1]), rep
            paged.graph_mode(True)
        paged.graph_mode(False)
        for mode in (1, 2, 0):
            paged.select_mode(mode)
            for qi, q in enumerate(qs):
                print(f"[gpu] paged select mode {mode}, q{qi}", flush=True)
                ids, out, _ = step(paged, q)
                assert torch.equal(ids, want[qi][0]) and torch.equal(out, want[qi][1]), (mode, qi)
    finally:
        paged.close()
        flat.close()


def test_paged_append_matches_contiguous():
    """Host and device appends into 16-token pages (the 700-token capacity
    spans 44 pages, every append crosses page boundaries): records, steps and
    dense decodes equal the contiguous instance's, top-100 IDs the oracle's
    over the grown cache."""
    flat, paged, pool, table, qs = runtimes(16, seed=3, append_capacity=CAPACITY)
    q = qs[0]
    try:
        ks, vs = [], []
        for n_i, (n, where) in enumerate([(1, "cpu"), (300, "cpu"), (257, "cuda")]):
            kn, vn = new_tokens(q, n, seed=200 + n_i)
            print(f"[gpu] paged append {n} tokens from {where}", flush=True)
            flat.append(kn.to(where), vn.to(where))
            paged.append(kn.to(where), vn.to(where))
            ks.append(kn)
            vs.append(vn)
            ids_f, out_f, _ = step(flat, q)
            ids_p, out_p, _ = step(paged, q)
            assert torch.equal(ids_p, ids_f) and torch.equal(out_p, out_f), n_i
            traces, ref, _, _ = oracle_grown(q, ks, vs)
            for g, tr in enumerate(traces):
                np.testing.assert_array_equal(paged.read_stage("top", g), tr.top100)
            got = paged.read_output().float().numpy().reshape(16, 256)
            for j in range(16):
                assert np.abs(got[j] - ref[j]).max() <= 2e-2, f"append {n_i} head {j}"
                assert cosine(got[j], ref[j]) >= 0.999, f"append {n_i} head {j}"
            assert torch.equal(dense(paged), dense(flat)), n_i
        kall, vall = bits(torch.cat(ks, 1)), bits(torch.cat(vs, 1))
        for g in range(4):
            rec = paged.read_stage("kv8", g).reshape(-1, 512)
            np.testing.assert_array_equal(rec, flat.read_stage("kv8", g).reshape(-1, 512))
            np.testing.assert_array_equal(rec[P["context"]:, 256:], fp8_bytes(kall[g]))
            np.testing.assert_array_equal(rec[P["context"]:, :256], fp8_bytes(vall[g]))
    finally:
        paged.close()
        flat.close()


def test_instances_share_one_pool():
    """Two caches in one scrambled pool (their pages interleaved), through the
    public API: each equals its contiguous instance bit for bit, closing one
    returns its pages without disturbing the other, and an instance the pool
    cannot hold fails at its first run without taking pages."""
    cfg = SeoulKV4Config(stage15_capacity=None, debug=True)
    inputs = [case(**P), case(**P, seed_shift=1)]
    page_tokens = 256
    need = -(-P["context"] // page_tokens)
    pool = scrambled_pool(2 * need + 3, page_tokens, seed=9)
    flat = [SeoulKV4(device="cuda:0", k=k, v=v, index=ix, config=cfg) for ix, k, v, _ in inputs]
    paged = [SeoulKV4(device="cuda:0", k=k, v=v, index=ix, config=cfg, kv_pool=pool)
             for ix, k, v, _ in inputs]
    try:
        want = []
        for i, (_, _, _, qs) in enumerate(inputs):
            print(f"[gpu] shared pool, cache {i}", flush=True)
            ref = flat[i].run(qs[0]).to_torch().view(torch.int16).clone()
            got = paged[i].run(qs[0]).to_torch().view(torch.int16).clone()
            assert torch.equal(got, ref), i
            assert torch.equal(paged[i].debug_snapshot()["selected_ids"],
                               flat[i].debug_snapshot()["selected_ids"]), i
            want.append(ref)
        t0, t1 = paged[0].page_table, paged[1].page_table
        assert len(t0) == len(t1) == need and not set(t0) & set(t1)
        assert paged[0].metadata()["cache_layout"] == "paged"
        assert pool.free_pages == 3
        paged[0].close()
        assert pool.free_pages == 3 + need
        got = paged[1].run(inputs[1][3][0]).to_torch().view(torch.int16)
        assert torch.equal(got, want[1])
        # an instance whose pool is too small is refused at its first run
        # and takes no pages
        small = KVPagePool(need - 1, page_tokens=page_tokens, device="cuda:0")
        ix, k, v, qs = inputs[0]
        big = SeoulKV4(device="cuda:0", k=k, v=v, index=ix, config=cfg, kv_pool=small)
        with pytest.raises(RuntimeError, match="exhausted"):
            big.run(qs[0])
        assert small.free_pages == need - 1
    finally:
        for inst in paged + flat:
            inst.close()
    assert pool.free_pages == pool.n_pages


def test_create_paged_rejects_memory_that_is_not_a_device_pool():
    """A page descriptor whose pool is host memory is refused at creation
    (SKV_EINVAL), before any record is written."""
    import ctypes

    index, k, v, _ = case(**P)
    desc, keep = _hip.index_desc(index, pool_min=0, pool_capacity=0, debug=False)
    host = torch.empty(1 << 20, dtype=torch.uint8, pin_memory=True)
    need = -(-P["context"] // 256)
    table = np.arange(need, dtype=np.int32)
    pd = _hip.KVPagesDesc(pool=host.data_ptr(), n_pages=need, page_tokens=256,
                          page_table=table.ctypes.data, table_len=need)
    kb = bits(k)
    vb = bits(v)
    handle = ctypes.c_void_p()
    lib = _hip.load_library()
    code = lib.skv_create_paged(ctypes.byref(desc), kb.ctypes.data, vb.ctypes.data,
                                ctypes.byref(pd), 0, None, ctypes.byref(handle))
    assert code == 1 and handle.value is None  # SKV_EINVAL
    assert "device memory" in lib.skv_last_error(None).decode()


def test_create_paged_rejects_a_pool_smaller_than_its_page_count():
    """A descriptor that declares more pages than the pool's allocation holds
    (2^21 pages of 256 tokens: 1 TiB of records) is refused at creation
    (SKV_EINVAL), before any record is written, and a correct descriptor of
    the same pool is accepted."""
    import ctypes

    index, k, v, _ = case(**P)
    desc, keep = _hip.index_desc(index, pool_min=0, pool_capacity=0, debug=False)
    need = -(-P["context"] // 256)
    pool = KVPagePool(need, page_tokens=256, device="cuda:0")
    table = np.arange(need, dtype=np.int32)[::-1].copy()
    kb, vb = bits(k), bits(v)
    lib = _hip.load_library()
    for n_pages, want in ((1 << 21, 1), (need, 0)):
        pd = _hip.KVPagesDesc(pool=pool.pages.data_ptr(), n_pages=n_pages, page_tokens=256,
                              page_table=table.ctypes.data, table_len=need)
        handle = ctypes.c_void_p()
        print(f"[gpu] paged create with {n_pages} declared pages", flush=True)
        code = lib.skv_create_paged(ctypes.byref(desc), kb.ctypes.data, vb.ctypes.data,
                                    ctypes.byref(pd), 0, None, ctypes.byref(handle))
        assert code == want, lib.skv_last_error(handle).decode()
        if want:
            assert handle.value is None
            assert "past the end of its device allocation" in lib.skv_last_error(None).decode()
        else:
            lib.skv_destroy(handle)


def test_handles_on_concurrent_streams():
    """Two caches (one contiguous, one paged) stepped on two streams of
    their own, 12 steps each enqueued alternately with no host
    synchronisation between them, so their kernels may overlap on the
    device: every step's result equals that cache's step run alone
    (no state is shared between handles)."""
    inputs = [case(**P), case(**P, seed_shift=1)]
    kw = dict(pool_min=0, pool_capacity=None, debug=True)
    streams = [torch.cuda.Stream(device="cuda:0") for _ in range(2)]
    need = -(-P["context"] // 64)
    pool = scrambled_pool(need, 64, seed=11)
    rts = [_hip.Runtime(0, inputs[0][1], inputs[0][2], inputs[0][0], stream=streams[0].cuda_stream,
                        **kw),
           _hip.Runtime(0, inputs[1][1], inputs[1][2], inputs[1][0], stream=streams[1].cuda_stream,
                        kv_pages=(pool, pool.allocate(need)), **kw)]
    try:
        qs = [inputs[0][3], inputs[1][3]]
        want = []
        for i, rt in enumerate(rts):  # each alone, synchronised
            want.append([step(rt, q)[1] for q in qs[i]])
        print("[gpu] two handles on concurrent streams", flush=True)
        for n in range(12):
            for i, rt in enumerate(rts):
                rt.bind_query(qs[i][n % 2])
                rt.enqueue()
            if n % 4 == 3:  # check the last steps of both
                for i, rt in enumerate(rts):
                    assert rt.synchronize()["err"] == [0, 0, 0, 0]
                    got = rt.read_output().view(torch.int16)
                    assert torch.equal(got, want[i][n % 2]), (n, i)
    finally:
        for rt in rts:
            rt.close()
