"""The reference's own index profile and its archive path on the GPU.

``SeoulKV4Index.build(k, v)`` at its defaults indexes a 128K cache with
ceil(R / 128) * 32 = 32672 centroids per KV head (about 8 postings per list)
and nprobe 256 (reference ``_index_build.py:16-19``, ``config.py:5``), and
``SeoulKV4Config()`` caps the pool at 13056 keys per KV group
(``config.py:10-22``): the profile behind the reference's published 518 µs
per layer (``README.md:7``).  Here it runs through the kernels stage by
stage against the oracle, through the public API and through the
reference's runtime seam, at nprobe 256 and, re-probed by
``SeoulKV4Index.load(path, nprobe=384)`` (``index.py:58-72``), at 384; at
nprobe 512 its pools pass 13056 and the reference's "never truncate" error
is raised.  A config-0 index written by ``dump`` and read by ``load`` (with
and without the nprobe override) decodes bit for bit like the built one."""

from __future__ import annotations

import functools
import types

import numpy as np
import pytest
import torch

from oracle import decode as od
from seoulkv_amd import SeoulKV4, SeoulKV4Config, SeoulKV4Index, _hip, ref_runtime
from seoulkv_amd.synthetic import make_profile
from tests.helpers import bits, case, cosine, oracle_step

pytestmark = pytest.mark.gpu

REF_CAPACITY = 13056  # SeoulKV4Config().stage15_capacity, the reference's default
P0 = dict(context=8192, components=256, nc=512, nprobe=64)


@functools.lru_cache(maxsize=1)
def _ref_profile():
    """(k, v, queries, default-built index, oracle key codes and records)."""
    prof, k, v, qs = make_profile("ref128k", n_queries=2)
    index = SeoulKV4Index.build(k, v)  # every argument at the reference's default
    kb, vb = bits(k), bits(v)
    code8, scales = od.key_codec(kb)
    k8, v8 = od.fp8_records(kb, vb)
    return prof, k, v, qs, index, (code8, scales, k8, v8)


@pytest.fixture(scope="module")
def ref_archive(tmp_path_factory):
    _, _, _, _, index, _ = _ref_profile()
    path = tmp_path_factory.mktemp("ref128k") / "index.npz"
    index.dump(path)
    return path


def _oracle(index, inputs, q):
    code8, scales, k8, v8 = inputs
    cells = [od.GroupCell.from_cell(c) for c in index.cells]
    zones = index.zones
    return od.decode_step(cells, code8, scales, k8, v8, bits(q).reshape(16, 256),
                          sink=zones.sink, local=zones.local)


def _check_output(got, ref):
    got = got.float().numpy().reshape(16, 256)
    for j in range(16):
        assert np.abs(got[j] - ref[j]).max() <= 2e-2, f"head {j} max-abs"
        assert cosine(got[j], ref[j]) >= 0.999, f"head {j} cosine"


def _stages(index, k, v, qs, inputs, label):
    """Every stage bit-exact against the oracle with the reference's pool
    bounds (minimum 2048, capacity 13056)."""
    rt = _hip.Runtime(0, k, v, index, pool_min=2048, pool_capacity=REF_CAPACITY, debug=True)
    try:
        # the first step runs the top-k instance without the two-octet register
        # path; its synchronisation sees pools of 8K-16K keys, so the next
        # step runs the other instance: both are checked below
        assert rt.metadata()["top1600_in_registers_to"] == 8192
        for qi, q in enumerate(qs):
            traces, ref = _oracle(index, inputs, q)
            print(f"[gpu] {label}: device step q{qi}", flush=True)
            rt.bind_query(q)
            rt.enqueue()
            status = rt.synchronize()
            assert status["err"] == [0, 0, 0, 0]
            for g, tr in enumerate(traces):
                assert status["pool"][g] == len(tr.pool) <= REF_CAPACITY
                np.testing.assert_array_equal(rt.read_stage("selected", g), tr.selected)
                np.testing.assert_array_equal(rt.read_stage("pool", g), tr.pool)
                np.testing.assert_array_equal(rt.read_stage("u1", g), tr.u1)
                np.testing.assert_array_equal(rt.read_stage("u2", g), tr.u2)
                np.testing.assert_array_equal(rt.read_stage("top", g), tr.top100)
            _check_output(rt.read_output(), ref)
            if max(status["pool"]) > 8192:
                assert rt.metadata()["top1600_in_registers_to"] == 16384
    finally:
        rt.close()


@pytest.mark.slow
def test_reference_default_profile_every_stage():
    print("[gpu] ref128k: default index build", flush=True)
    prof, k, v, qs, index, inputs = _ref_profile()
    assert index.n_centroids == 32672
    assert index.metadata()["nprobe"] == [256] * 4
    _stages(index, k, v, qs, inputs, "ref128k P=256")


@pytest.mark.slow
def test_reference_default_profile_public_api():
    """SeoulKV4 with SeoulKV4Config() (capacity 13056): top-100 and output."""
    prof, k, v, qs, index, inputs = _ref_profile()
    print("[gpu] ref128k: SeoulKV4 with the default config", flush=True)
    with SeoulKV4(device="cuda:0", k=k, v=v, index=index,
                  config=SeoulKV4Config(debug=True)) as skv:
        for q in qs:
            out = skv.run(q).to_torch()
            traces, ref = _oracle(index, inputs, q)
            want = torch.tensor(np.stack([t.top100 for t in traces]), dtype=torch.long)
            assert torch.equal(skv.debug_snapshot()["selected_ids"], want)
            _check_output(out, ref)


def _ref_options(context, capacity, debug):
    """The fields of the reference's ``_KernelOptions`` (``config.py:25-40``)
    that its runtime reads."""
    return types.SimpleNamespace(
        context_len=context, skv4_stage15_candidates=capacity, skv4_debug_indices=debug,
        n_conc=1, seq_len=1, n_kv_heads=4, n_heads=16, topk=100, skv4_stage15_m=2048,
        skv4_stage15_union_m=1600)


@pytest.mark.slow
def test_reference_default_profile_through_the_reference_seam():
    """The reference's runtime call sequence (``_runtime.py:36,180,189``) on
    its own default profile, with its ``_KernelOptions`` field names."""
    prof, k, v, qs, index, inputs = _ref_profile()
    print("[gpu] ref128k: reference runtime seam", flush=True)
    args = _ref_options(prof.context, REF_CAPACITY, True)
    tt = ref_runtime._ttnn()
    ref_index = types.SimpleNamespace(_cells=index.cells, _zones=index.zones)
    state = ref_runtime.initialize(tt, torch.device("cuda", 0), k, v, qs[0], ref_index, args)
    try:
        for q in qs:
            ref_runtime.bind_query(state, q, args)
            ref_runtime.enqueue(state)
            tt.synchronize_device(0)
            rows = [tt.to_torch(item)[0] for item in state["selector"]["outputs"]]
            out = torch.cat([torch.stack([r[h, h] for h in range(4)]) for r in rows])
            ids = tt.to_torch(state["selector"]["debug_indices"]).reshape(4, 4, -1)[..., :100]
            traces, ref = _oracle(index, inputs, q)
            assert np.array_equal(ids.numpy(), np.stack([t.top100 for t in traces]))
            _check_output(out, ref)
    finally:
        state["runtime"].close()


@pytest.mark.slow
def test_reference_default_profile_reprobed_by_load(ref_archive):
    """``load(path, nprobe=384)`` re-probes the dumped default index: every
    stage against the oracle on the loaded cells, pools still under 13056."""
    prof, k, v, qs, index, inputs = _ref_profile()
    loaded = SeoulKV4Index.load(ref_archive, nprobe=384)
    assert loaded.metadata()["nprobe"] == [384] * 4
    assert loaded.metadata()["nprobe_source"] == "load override"
    _stages(loaded, k, v, qs, inputs, "ref128k P=384 (load)")


@pytest.mark.slow
def test_reference_default_profile_over_capacity_at_nprobe_512(ref_archive):
    """At nprobe 512 the default profile's pools (~15.5K keys) exceed the
    reference's 13056: the first run raises and keeps nothing; an HBM-sized
    pool (``stage15_capacity=None``) then runs it, top-100 against the
    oracle."""
    prof, k, v, qs, index, inputs = _ref_profile()
    loaded = SeoulKV4Index.load(ref_archive, nprobe=512)
    print("[gpu] ref128k P=512: capacity error", flush=True)
    skv = SeoulKV4(device=0, k=k, v=v, index=loaded)
    with pytest.raises(ValueError, match="never truncate"):
        skv.run(qs[0])
    assert not skv.initialized
    skv.close()
    print("[gpu] ref128k P=512: HBM-sized pool", flush=True)
    with SeoulKV4(device=0, k=k, v=v, index=loaded,
                  config=SeoulKV4Config(stage15_capacity=None, debug=True)) as skv:
        out = skv.run(qs[0]).to_torch()
        traces, ref = _oracle(loaded, inputs, qs[0])
        assert max(len(t.pool) for t in traces) > REF_CAPACITY
        want = torch.tensor(np.stack([t.top100 for t in traces]), dtype=torch.long)
        assert torch.equal(skv.debug_snapshot()["selected_ids"], want)
        _check_output(out, ref)


@pytest.mark.parametrize("nprobe", [None, 32, 128])
def test_dumped_and_loaded_index_decodes_like_the_built_one(tmp_path, nprobe):
    """A config-0 index through ``dump`` and ``load`` (``index.py:58-76``):
    the loaded cells decode bit for bit like the built index (top-100 IDs
    and output bits), and ``load(path, nprobe=P)`` decodes like the index
    built with nprobe P, both against the oracle."""
    index, k, v, qs = case(**P0)
    path = tmp_path / "cfg0.npz"
    index.dump(path)
    loaded = SeoulKV4Index.load(path, nprobe=nprobe)
    params = dict(P0, nprobe=nprobe or P0["nprobe"])
    if nprobe is not None:
        assert loaded.metadata()["nprobe"] == [nprobe] * 4
    print(f"[gpu] cfg0 dump/load nprobe={nprobe}", flush=True)
    results = []
    for source in (loaded, case(**params)[0]):
        with SeoulKV4(device="cuda:0", k=k, v=v, index=source,
                      config=SeoulKV4Config(stage15_capacity=None, debug=True)) as skv:
            out = skv.run(qs[0]).to_torch()
            results.append((out.view(torch.int16).clone(),
                            skv.debug_snapshot()["selected_ids"].clone()))
    assert torch.equal(results[0][0], results[1][0])
    assert torch.equal(results[0][1], results[1][1])
    traces, ref = oracle_step(params, qs[0])
    want = torch.tensor(np.stack([t.top100 for t in traces]), dtype=torch.long)
    assert torch.equal(results[0][1], want)
    _check_output(results[0][0].view(torch.bfloat16), ref)
