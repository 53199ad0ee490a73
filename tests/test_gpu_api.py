"""The public API on the GPU: lifecycle, borrowed results, the reference's
error paths (pool below the minimum, pool above capacity: "never truncate"),
the device-resident query binding, and full-pipeline parity at BASELINE
configurations 1 and 2 (T = 32K and 128K) through the same entry points a
caller uses."""

from __future__ import annotations

import functools
import random
import tempfile
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import decode as od
from seoulkv_amd import SeoulKV4, SeoulKV4Config, SeoulKV4Index, _hip
from seoulkv_amd.result import _DeviceArray
from tests.helpers import bits, case, cosine, oracle_step

pytestmark = pytest.mark.gpu

P0 = dict(context=8192, components=256, nc=512, nprobe=64)
P1 = dict(context=32768, components=1024, nc=2048, nprobe=384)


def _check_output(got, ref):
    got = got.float().numpy().reshape(16, 256)
    for j in range(16):
        assert np.abs(got[j] - ref[j]).max() <= 2e-2, f"head {j} max-abs"
        assert cosine(got[j], ref[j]) >= 0.999, f"head {j} cosine"


def _top100(traces):
    return torch.tensor(np.stack([t.top100 for t in traces]), dtype=torch.long)


def test_lifecycle_and_borrowed_results():
    index, k, v, qs = case(**P0)
    print("[gpu] lifecycle cfg0", flush=True)
    with SeoulKV4(device="cuda:0", k=k, v=v, index=index,
                  config=SeoulKV4Config(debug=True)) as skv:
        r0 = skv.run(qs[0])
        assert skv.initialized
        out0 = r0.to_torch()
        assert out0.shape == (1, 1, 16, 256) and out0.dtype == torch.bfloat16
        traces, ref = oracle_step(P0, qs[0])
        _check_output(out0, ref)
        assert torch.equal(skv.debug_snapshot()["selected_ids"], _top100(traces))
        views = r0.device_tensors  # the reference's [1, 32, 4, 256] per KV head
        assert len(views) == 4 and all(t.shape == (1, 32, 4, 256) for t in views)
        diag = torch.cat([torch.stack([t[0, h, h] for h in range(4)]) for t in views])
        assert torch.equal(diag.cpu(), out0.reshape(16, 256))
        for t in views:
            off = t[0].clone()
            for h in range(4):
                off[h, h] = 0
            assert not off.float().abs().sum().item()
        r1 = skv.run(qs[1])
        with pytest.raises(RuntimeError):
            r0.to_torch()  # borrowed output: superseded by the next run
        traces, ref = oracle_step(P0, qs[1])
        _check_output(r1.to_torch(), ref)
        assert torch.equal(skv.debug_snapshot()["selected_ids"], _top100(traces))
        meta = skv.metadata()
        assert meta["initialized"] and meta["runtime"]["kernels_per_step"] == 7
    with pytest.raises(RuntimeError):
        r1.to_torch()  # closed
    with pytest.raises(RuntimeError):
        skv.run(qs[0])


def test_debug_snapshot_requires_debug_config():
    index, k, v, qs = case(**P0)
    skv = SeoulKV4(device=0, k=k, v=v, index=index)
    skv.run(qs[0]).to_torch()
    with pytest.raises(RuntimeError):
        skv.debug_snapshot()
    skv.close()


def test_pool_below_minimum_raises():
    p = dict(context=8192, components=256, nc=1024, nprobe=16)  # pools of ~700 keys
    index, k, v, qs = case(**p)
    print("[gpu] pool underflow", flush=True)
    skv = SeoulKV4(device=0, k=k, v=v, index=index)
    with pytest.raises(ValueError, match="never truncate"):
        skv.run(qs[0])
    assert not skv.initialized
    skv.close()


def test_capacity_error_then_hbm_sized_pool_at_config1():
    index, k, v, qs = case(**P1)
    print("[gpu] capacity cfg1", flush=True)
    skv = SeoulKV4(device=0, k=k, v=v, index=index)  # reference capacity 13056
    with pytest.raises(ValueError, match="never truncate"):
        skv.run(qs[0])
    skv.close()
    print("[gpu] parity cfg1 (HBM-sized pool)", flush=True)
    skv = SeoulKV4(device=0, k=k, v=v, index=index,
                   config=SeoulKV4Config(stage15_capacity=None, debug=True))
    for q in qs:
        out = skv.run(q).to_torch()
        traces, ref = oracle_step(P1, q)
        assert torch.equal(skv.debug_snapshot()["selected_ids"], _top100(traces))
        _check_output(out, ref)
    skv.close()


def test_device_query_binding_matches_host_binding():
    index, k, v, qs = case(**P0)
    rt = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=True)
    try:
        rt.bind_query(qs[0])
        rt.enqueue()
        rt.synchronize()
        host_out, host_ids = rt.read_output(), rt.debug_ids()
        rt.bind_query(qs[1])  # overwrite, then bind the device copy of q0
        rt.enqueue()
        rt.synchronize()
        qd = qs[0].reshape(16, 256).to("cuda:0")
        rt.bind_query_device(qd)
        rt.enqueue()
        rt.synchronize()
        assert torch.equal(rt.read_output(), host_out)
        assert torch.equal(rt.debug_ids(), host_ids)
    finally:
        rt.close()


def test_device_query_produced_on_another_stream():
    """A query written by a PyTorch kernel on a side stream, late: the copy is
    ordered after that kernel (and after the instance's earlier step, which
    still reads the previous query), so both steps see their own query."""
    index, k, v, qs = case(**P0)
    rt = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=True)
    try:
        outs, ids = [], []
        for q in qs:
            rt.bind_query(q)
            rt.enqueue()
            rt.synchronize()
            outs.append(rt.read_output())
            ids.append(rt.debug_ids())
        base = qs[1].reshape(16, 256).to("cuda:0")
        side = torch.cuda.Stream()
        torch.cuda.synchronize()
        print("[gpu] device query from a side stream", flush=True)
        rt.bind_query(qs[0])
        rt.enqueue()  # step on q0, still running while q1 is bound
        with torch.cuda.stream(side):
            torch.cuda._sleep(20_000_000)  # the producer's write lands late
            q1 = base * 1
            rt.bind_query_device(q1)
        del q1  # freed on its stream after the copy
        rt.synchronize()
        assert torch.equal(rt.read_output(), outs[0])
        assert torch.equal(rt.debug_ids(), ids[0])
        rt.enqueue()
        rt.synchronize()
        assert torch.equal(rt.read_output(), outs[1])
        assert torch.equal(rt.debug_ids(), ids[1])
    finally:
        torch.cuda.synchronize()
        rt.close()


def test_host_runs_ahead_through_the_query_ring():
    """Host binds while the device is held back: the host fills the pinned
    staging ring, waits on its completion events and reuses slots; every
    step, read from a copy ordered right after it on the stream, must equal
    the synchronous step on its own query (5 queries in turn, so a reused
    slot holding the wrong query would show)."""
    index, k, v, qs = case(**P0, n_queries=5)
    st = torch.cuda.Stream()
    rt = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=False,
                      stream=st.cuda_stream)
    try:
        want = []
        for q in qs:
            rt.bind_query(q)
            rt.enqueue()
            rt.synchronize()
            want.append(rt.read_output().view(torch.int16).reshape(16, 256))
        out = torch.as_tensor(_DeviceArray(rt.output_device_ptr(), (16, 256), "<i2"),
                              device="cuda:0")
        n = 40
        got = torch.zeros((n, 16, 256), dtype=torch.int16, device="cuda:0")
        torch.cuda.synchronize()  # the fill (default stream) before the copies on st
        print(f"[gpu] {n} host binds ahead of a held-back stream", flush=True)
        with torch.cuda.stream(st):
            torch.cuda._sleep(50_000_000)  # the device starts late
            for i in range(n):
                rt.bind_query(qs[i % 5])
                rt.enqueue()
                got[i].copy_(out)
        st.synchronize()
        got = got.cpu()
        for i in range(n):
            assert torch.equal(got[i], want[i % 5]), f"step {i}"
    finally:
        torch.cuda.synchronize()
        rt.close()


_ARCHIVES = tempfile.TemporaryDirectory(prefix="skv_index_")


@functools.lru_cache(maxsize=2)
def _full_size_inputs(name, clustered, n_queries):
    """(profile, k, v, queries, index at the profile's nprobe, oracle inputs,
    path of the index dumped as NPZ)."""
    from seoulkv_amd.index import SeoulKV4Index
    from seoulkv_amd.synthetic import make_profile

    prof, k, v, qs = make_profile(name, clustered=clustered, n_queries=n_queries)
    index = SeoulKV4Index.build(k, v, sink=prof.sink, local=prof.local, nprobe=prof.nprobe,
                                n_centroids=prof.n_centroids)
    path = Path(_ARCHIVES.name) / f"{name}_{'clustered' if clustered else 'iid'}.npz"
    index.dump(path)
    kb, vb = bits(k), bits(v)
    code8, scales = od.key_codec(kb)
    k8, v8 = od.fp8_records(kb, vb)
    return prof, k, v, qs, index, (code8, scales, k8, v8), path


def _reprobed(path, nprobe):
    """The dumped index re-probed with another nprobe by the reference's own
    route, ``SeoulKV4Index.load(path, nprobe=...)`` (``index.py:58-72``)."""
    index = SeoulKV4Index.load(path, nprobe=nprobe)
    assert index.metadata()["nprobe"] == [nprobe] * 4
    return index


def _full_size_parity(name, *, nprobe=None, clustered=True, pool_min=2048, queries=(0,),
                      n_queries=1, page_tokens=None):
    """Every funnel stage bit-exact against the oracle on a BASELINE-sized
    cache (seeded synthetic inputs), output within the attention tolerance.
    page_tokens: keep the FP8 records in pages of that size, handed out by a
    page pool in a seeded random order."""
    print(f"[gpu] {name} P={nprobe} clustered={clustered}: inputs", flush=True)
    prof, k, v, qs, index, (code8, scales, k8, v8), path = _full_size_inputs(
        name, clustered, n_queries)
    if nprobe is not None and nprobe != prof.nprobe:
        index = _reprobed(path, nprobe)
    cells = [od.GroupCell.from_cell(c) for c in index.cells]
    kv_pages = None
    if page_tokens:
        from seoulkv_amd import KVPagePool

        need = -(-prof.context // page_tokens)
        pool = KVPagePool(need + 64, page_tokens=page_tokens, device="cuda:0")
        pages = pool.allocate(pool.n_pages)
        random.Random(page_tokens).shuffle(pages)
        kv_pages = (pool, pages[:need])
    rt = _hip.Runtime(0, k, v, index, pool_min=pool_min, pool_capacity=None, debug=True,
                      kv_pages=kv_pages)
    try:
        for qi in queries:
            print(f"[gpu] {name}: oracle q{qi}", flush=True)
            traces, ref = od.decode_step(cells, code8, scales, k8, v8,
                                         bits(qs[qi]).reshape(16, 256),
                                         sink=prof.sink, local=prof.local)
            print(f"[gpu] {name}: device step q{qi}", flush=True)
            rt.bind_query(qs[qi])
            rt.enqueue()
            status = rt.synchronize()
            assert status["err"] == [0, 0, 0, 0]
            for g, tr in enumerate(traces):
                assert status["pool"][g] == len(tr.pool)
                np.testing.assert_array_equal(rt.read_stage("thresh", g), tr.thr)
                np.testing.assert_array_equal(rt.read_stage("selected", g), tr.selected)
                np.testing.assert_array_equal(rt.read_stage("pool", g), tr.pool)
                np.testing.assert_array_equal(rt.read_stage("u1", g), tr.u1)
                np.testing.assert_array_equal(rt.read_stage("u2", g), tr.u2)
                np.testing.assert_array_equal(rt.read_stage("top", g), tr.top100)
            _check_output(rt.read_output(), ref)
    finally:
        rt.close()


@pytest.mark.slow
def test_full_size_parity_config2():
    """T = 131072, nc = 8192, P = 384; three queries."""
    _full_size_parity("cfg2", queries=(0, 1, 2), n_queries=3)


@pytest.mark.slow
def test_full_size_parity_config2_paged_records():
    """Configuration 2 with the FP8 records in 16-token pages of a pool, in a
    scrambled order (a page table of 8192 entries): every stage and the
    output as for the contiguous records."""
    _full_size_parity("cfg2", queries=(0, 1), n_queries=3, page_tokens=16)


@pytest.mark.slow
@pytest.mark.parametrize("nprobe,clustered", [(16, True), (64, True), (128, True), (256, True),
                                              (512, True), (16, False), (64, False),
                                              (128, False), (256, False), (384, False),
                                              (512, False)])
def test_full_size_parity_config3_nprobe_sweep(nprobe, clustered):
    """config-2 shapes over the whole nprobe sweep
    (16, 64, 128, 256, 384, 512), clustered and i.i.d. keys (the i.i.d. keys
    give the largest pools; P = 384 clustered is configuration 2).  Each
    nprobe other than the build's comes from the dumped index through
    ``SeoulKV4Index.load(path, nprobe=...)``."""
    _full_size_parity("cfg2", nprobe=nprobe, clustered=clustered, pool_min=0,
                      n_queries=3 if clustered else 1)


@pytest.mark.slow
def test_full_size_parity_config1():
    """T = 32768; every stage for two queries (the
    pool sized in HBM: the reference's capacity rejects this config, see
    test_capacity_error_then_hbm_sized_pool_at_config1)."""
    _full_size_parity("cfg1", queries=(0, 1), n_queries=2)


@pytest.mark.slow
def test_full_size_parity_config4():
    """T = 1048576, nc = 65536, P = 512; two queries."""
    _full_size_parity("cfg4", queries=(0, 1), n_queries=2)


def test_time_kernel_keeps_the_step_consistent():
    """Timing a kernel alone re-runs it on the last step's inputs and then a
    full step: the selection and output stay those of the bound query."""
    index, k, v, qs = case(**P0)
    rt = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=True)
    try:
        rt.bind_query(qs[0])
        rt.enqueue()
        rt.synchronize()
        out, ids = rt.read_output(), rt.debug_ids()
        n = rt.lib.skv_kernel_count()
        times = [rt.time_kernel(i, reps=3) for i in range(n)]
        assert all(t > 0 for t in times)
        assert torch.equal(rt.read_output(), out)
        assert torch.equal(rt.debug_ids(), ids)
        with pytest.raises(RuntimeError):
            rt.time_kernel(n, reps=1)
    finally:
        rt.close()


def test_index_built_on_the_gpu():
    """SeoulKV4Index.build(build_device="cuda") clusters with the same torch
    code on the GPU: the cells pass the index invariants, every token is
    listed exactly twice (spill 2), and the decode step on that index is
    bit-exact against the oracle run on the same cells."""
    from oracle import decode as od
    from seoulkv_amd.synthetic import make_cache
    from tests.helpers import bits, cosine

    k, v, qs = make_cache(8192, 256, clustered=True, seed_k=4321, seed_v=4322, seed_q=4323,
                          n_queries=1)
    print("[gpu] index build on cuda:0", flush=True)
    index = SeoulKV4Index.build(k, v, nprobe=64, n_centroids=512, build_device="cuda:0")
    zones = index.zones
    retrieval = np.arange(zones.sink, zones.local_begin)
    for cell in index.cells:
        values = cell["values"].numpy()
        assert cell["upper"].device.type == "cpu"
        counts = np.bincount(values, minlength=zones.local_begin)
        assert np.all(counts[retrieval] == 2)
        assert counts[: zones.sink].sum() == 0
    rt = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=True)
    try:
        rt.bind_query(qs[0])
        rt.enqueue()
        status = rt.synchronize()
        assert status["err"] == [0, 0, 0, 0]
        cells = [od.GroupCell.from_cell(c) for c in index.cells]
        code8, scales = od.key_codec(bits(k))
        k8, v8 = od.fp8_records(bits(k), bits(v))
        traces, out = od.decode_step(cells, code8, scales, k8, v8,
                                     bits(qs[0]).reshape(16, 256), sink=zones.sink,
                                     local=zones.local)
        for g, tr in enumerate(traces):
            np.testing.assert_array_equal(rt.read_stage("selected", g), tr.selected)
            np.testing.assert_array_equal(rt.read_stage("top", g), tr.top100)
        got = rt.read_output().float().numpy().reshape(16, 256)
        for j in range(16):
            assert cosine(got[j], out[j]) >= 0.999
    finally:
        rt.close()
