"""Stage-by-stage parity of the HIP decode step against the CPU oracle.

Bit-exact: key codec records, FP8 records, query operands, coarse intervals,
thresholds, survivor masks, fine scores, selected clusters, the pool (in
encounter order), 2/4/8-bit scores, U1, U2 and the final top-100 IDs.
Attention output: max-abs <= 2e-2 and cosine >= 0.999 per query head against
the oracle's float64 softmax over the same FP8 records.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import arith
from oracle import decode as od
from seoulkv_amd import _hip
from tests.helpers import bits, case, cosine, oracle_inputs, oracle_step, unorder

pytestmark = pytest.mark.gpu

CASES = {
    "t8192_clustered": dict(context=8192, components=256, nc=512, nprobe=64),
    "t8192_iid_p128": dict(context=8192, components=1, nc=512, nprobe=128, clustered=False),
    "t8192_p16_sink0": dict(context=8192, components=64, nc=256, nprobe=16, sink=0, local=64),
    # no sink and no local window: the attention is the top-100 alone (no
    # sink/local slice blocks, nothing to merge)
    "t8192_no_window": dict(context=8192, components=256, nc=512, nprobe=64, sink=0, local=0,
                            seed_shift=11),
    "t16384_nc1024_p256": dict(context=16384, components=512, nc=1024, nprobe=256, seed_shift=7),
    # sizes that are not multiples of 64: context, sink, local, centroids
    "t8200_nc160_odd": dict(context=8200, components=64, nc=160, nprobe=32, sink=40, local=200,
                            seed_shift=3),
}


@pytest.fixture(scope="module")
def runtimes():
    made = {}
    yield made
    for rt in made.values():
        rt.close()


def runtime_for(runtimes, name):
    if name not in runtimes:
        p = CASES[name]
        index, k, v, _ = case(**p)
        print(f"[gpu] create runtime {name}", flush=True)
        runtimes[name] = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=True)
    return runtimes[name]


@pytest.mark.parametrize("name", list(CASES))
def test_prefill_records(runtimes, name):
    p = CASES[name]
    rt = runtime_for(runtimes, name)
    _, code8, scales, _, _ = oracle_inputs(**p)
    index, k, v, _ = case(**p)
    kb, vb = bits(k), bits(v)
    for g in range(4):
        np.testing.assert_array_equal(rt.read_stage("kscale", g), scales[g])
        rec = rt.read_stage("keyrec", g).reshape(-1, 256)
        c = code8[g].astype(np.uint32)
        planes = torch.from_numpy(c.astype(np.uint8))
        from seoulkv_amd._codecs import encode_planes

        ref = encode_planes(planes[None])
        np.testing.assert_array_equal(rec[:, :64], ref["prefix2"][0].numpy())
        np.testing.assert_array_equal(rec[:, 64:128], ref["residual2"][0].numpy())
        np.testing.assert_array_equal(rec[:, 128:], ref["residual4"][0].numpy())
        kv8 = rt.read_stage("kv8", g).reshape(-1, 512)
        kt = torch.from_numpy(kb[g].view(np.int16)).view(torch.bfloat16).float()
        vt = torch.from_numpy(vb[g].view(np.int16)).view(torch.bfloat16).float()
        np.testing.assert_array_equal(
            kv8[:, 256:], kt.to(torch.float8_e4m3fn).view(torch.uint8).numpy())
        np.testing.assert_array_equal(
            kv8[:, :256], vt.to(torch.float8_e4m3fn).view(torch.uint8).numpy())


@pytest.mark.parametrize("qi", [0, 1])
@pytest.mark.parametrize("name", list(CASES))
def test_step_parity(runtimes, name, qi):
    p = CASES[name]
    rt = runtime_for(runtimes, name)
    _, _, _, qs = case(**p)
    q = qs[qi]
    print(f"[gpu] step {name} q{qi}", flush=True)
    rt.bind_query(q)
    rt.enqueue()
    status = rt.synchronize()
    traces, out = oracle_step(p, q)
    index = case(**p)[0]
    # status words: no error (the pool kernel's look-back never gave up) and
    # the stage sizes of the oracle
    assert status["err"] == [0, 0, 0, 0]
    for g, tr in enumerate(traces):
        off = index.cells[g]["offsets"].numpy().astype(np.int64)
        assert status["pool"][g] == len(tr.pool), f"g{g} pool size"
        assert status["selected"][g] == len(tr.selected), f"g{g} selected"
        assert status["survivors"][g] == len(tr.survivors), f"g{g} survivors"
        scanned = int((off[tr.selected + 1] - off[tr.selected]).sum())
        assert status["scanned"][g] == scanned, f"g{g} scanned postings"
    for g, tr in enumerate(traces):
        qp = tr.extra["qprep"]
        dq = rt.read_stage("qprep", g)
        for v, (X, fx) in enumerate([(qp.X0, qp.fx0), (qp.X15, qp.fx15), (qp.Xs, qp.fxs)]):
            np.testing.assert_array_equal(dq[v, :, :256], X, err_msg=f"g{g} X variant {v}")
            np.testing.assert_array_equal(dq[v, :, 256], fx, err_msg=f"g{g} fx variant {v}")
            S = (dq[v, :, 257].astype(np.int64) & 0xFFFFFFFF) | (dq[v, :, 258].astype(np.int64) << 32)
            np.testing.assert_array_equal(S, X.sum(-1), err_msg=f"g{g} S variant {v}")
        np.testing.assert_array_equal(dq[0, :, 259].view(np.float32), qp.norm, err_msg=f"g{g} norm")
        np.testing.assert_array_equal(rt.read_stage("lower", g), tr.lower, err_msg=f"g{g} lower")
        np.testing.assert_array_equal(rt.read_stage("upper", g), tr.upper, err_msg=f"g{g} upper")
        np.testing.assert_array_equal(rt.read_stage("thresh", g), tr.thr, err_msg=f"g{g} thr")
        np.testing.assert_array_equal(rt.read_stage("masks", g), tr.masks, err_msg=f"g{g} masks")
        fine = rt.read_stage("fine", g)[:, tr.survivors]
        elig = ((tr.masks[tr.survivors][None, :] >> np.arange(4)[:, None]) & 1).astype(bool)
        np.testing.assert_array_equal(fine[elig], tr.fine[elig], err_msg=f"g{g} fine")
        assert (fine[~elig] == 0xFFFF).all()
        np.testing.assert_array_equal(rt.read_stage("selected", g), tr.selected,
                                      err_msg=f"g{g} selected")
        np.testing.assert_array_equal(rt.read_stage("pool", g), tr.pool, err_msg=f"g{g} pool")
        assert status["pool"][g] == len(tr.pool)
        np.testing.assert_array_equal(unorder(rt.read_stage("s2", g)), tr.s2, err_msg=f"g{g} s2")
        np.testing.assert_array_equal(rt.read_stage("u1", g), tr.u1, err_msg=f"g{g} u1")
        np.testing.assert_array_equal(unorder(rt.read_stage("s4", g)), tr.s4, err_msg=f"g{g} s4")
        np.testing.assert_array_equal(rt.read_stage("u2", g), tr.u2, err_msg=f"g{g} u2")
        np.testing.assert_array_equal(unorder(rt.read_stage("s8", g)), tr.s8, err_msg=f"g{g} s8")
        np.testing.assert_array_equal(rt.read_stage("top", g), tr.top100, err_msg=f"g{g} top100")
    got = rt.read_output().float().numpy().reshape(16, 256)
    for j in range(16):
        assert np.abs(got[j] - out[j]).max() <= 2e-2, f"head {j} max-abs"
        assert cosine(got[j], out[j]) >= 0.999, f"head {j} cosine"


@pytest.mark.parametrize("mode", [1, 2, 3])
@pytest.mark.parametrize("name", ["t8192_clustered", "t16384_nc1024_p256"])
def test_selection_paths_agree(runtimes, name, mode):
    """Every selection through the full path (mode 1), through a sampled cut
    forced to miss, i.e. the fallback (mode 2), and through the full path
    with the token top-k kernels' in-memory radix passes (mode 3: the path a
    pool beyond the LDS capacity takes) equals the oracle; the status bits
    record which selections fell back.  The attention output bits equal the
    default path's: every path attends the members in the same order."""
    p = CASES[name]
    rt = runtime_for(runtimes, name)
    _, _, _, qs = case(**p)
    print(f"[gpu] select mode {mode} {name}", flush=True)
    rt.bind_query(qs[0])
    rt.enqueue()
    rt.synchronize()
    want = rt.read_output().view(torch.int16).clone()
    rt.select_mode(mode)
    try:
        rt.bind_query(qs[0])
        rt.enqueue()
        status = rt.synchronize()
    finally:
        rt.select_mode(0)
    assert torch.equal(rt.read_output().view(torch.int16), want)
    traces, _ = oracle_step(p, qs[0])
    for g, tr in enumerate(traces):
        np.testing.assert_array_equal(rt.read_stage("thresh", g), tr.thr)
        np.testing.assert_array_equal(rt.read_stage("selected", g), tr.selected)
        np.testing.assert_array_equal(rt.read_stage("u1", g), tr.u1)
        np.testing.assert_array_equal(rt.read_stage("u2", g), tr.u2)
        np.testing.assert_array_equal(rt.read_stage("top", g), tr.top100)
    bits = status["full_select"]
    if mode in (1, 3):
        assert bits == [0, 0, 0, 0]  # the full path ran directly: nothing missed
    else:
        assert all(b == 31 for b in bits), bits  # every stage missed and fell back
    rt.bind_query(qs[0])
    rt.enqueue()
    assert rt.synchronize()["full_select"] == [0, 0, 0, 0]  # default: sampled cuts hit


@pytest.mark.parametrize("name", ["t8192_clustered", "t8192_p16_sink0"])
def test_graph_replay_matches_eager(runtimes, name):
    """The captured step replayed several times, with eager steps
    and host synchronizations between the replays, gives the same top-100
    IDs, status words and output bits as kernel-by-kernel launches, and
    both equal the oracle's IDs."""
    p = CASES[name]
    rt = runtime_for(runtimes, name)
    _, _, _, (q0, q1) = case(**p)
    qs = (q0, q1, (q0.float() - q1.float()).bfloat16(), -q0)
    print(f"[gpu] graph vs eager {name}", flush=True)

    def step(q, graph):
        rt.graph_mode(graph)
        rt.bind_query(q)
        rt.enqueue()
        st = rt.synchronize()
        return st, rt.debug_ids().clone(), rt.read_output().view(torch.int16).clone()

    try:
        for rep in range(3):
            for qi, q in enumerate(qs):
                st_e, ids_e, out_e = step(q, False)
                st_g, ids_g, out_g = step(q, True)
                assert st_g == st_e, (rep, qi)
                assert torch.equal(ids_g, ids_e), (rep, qi)
                assert torch.equal(out_g, out_e), (rep, qi)
                if rep == 0:
                    traces, _ = oracle_step(p, q)
                    for g, tr in enumerate(traces):
                        np.testing.assert_array_equal(rt.read_stage("top", g), tr.top100)
        # consecutive replays with no eager step between them
        rt.graph_mode(True)
        for qi in (3, 0, 2, 1):
            rt.bind_query(qs[qi])
            rt.enqueue()
            rt.synchronize()
            traces, _ = oracle_step(p, qs[qi])
            for g, tr in enumerate(traces):
                np.testing.assert_array_equal(rt.read_stage("top", g), tr.top100)
    finally:
        rt.graph_mode(False)


def degenerate_queries(q: torch.Tensor) -> dict:
    """Queries at the edges of the fixed-point query scaling and of the
    selections' tie handling: all zero (every score of a head ties, so every
    cut is decided by lowest ID), one nonzero coordinate, and a real query
    scaled by 2^-100 and 2^100 (BF16 exponents far from 0; the scores are
    the unscaled query's up to the power of two)."""
    z = torch.zeros(1, 1, 16, 256, dtype=torch.bfloat16)
    one = z.clone()
    one[..., 7] = 1.0
    qf = q.float()
    return {"zero": z, "onehot": one, "tiny": (qf * 2.0**-100).bfloat16(),
            "huge": (qf * 2.0**100).bfloat16()}


@pytest.mark.parametrize("kind", ["zero", "onehot", "tiny", "huge"])
def test_degenerate_queries_match_the_oracle(runtimes, kind):
    p = CASES["t8192_clustered"]
    rt = runtime_for(runtimes, "t8192_clustered")
    _, _, _, qs = case(**p)
    q = degenerate_queries(qs[0])[kind]
    print(f"[gpu] degenerate query {kind}", flush=True)
    rt.bind_query(q)
    rt.enqueue()
    status = rt.synchronize()
    assert status["err"] == [0, 0, 0, 0]
    traces, out = oracle_step(p, q)
    for g, tr in enumerate(traces):
        np.testing.assert_array_equal(rt.read_stage("thresh", g), tr.thr, err_msg=f"g{g}")
        np.testing.assert_array_equal(rt.read_stage("selected", g), tr.selected, err_msg=f"g{g}")
        np.testing.assert_array_equal(rt.read_stage("pool", g), tr.pool, err_msg=f"g{g}")
        np.testing.assert_array_equal(rt.read_stage("u1", g), tr.u1, err_msg=f"g{g}")
        np.testing.assert_array_equal(rt.read_stage("u2", g), tr.u2, err_msg=f"g{g}")
        np.testing.assert_array_equal(rt.read_stage("top", g), tr.top100, err_msg=f"g{g}")
    got = rt.read_output().float().numpy().reshape(16, 256)
    assert np.isfinite(got).all()
    for j in range(16):
        assert np.abs(got[j] - out[j]).max() <= 2e-2, f"head {j} max-abs"
        if np.linalg.norm(out[j]) > 0:
            assert cosine(got[j], out[j]) >= 0.999, f"head {j} cosine"


# Long centroid lists selected in registers (two and four octets per thread,
# about four keys per centroid as in the reference's default index): a real
# query, and the zero query, whose fine scores all tie (far more ties at the
# P-th score than the register ranking holds, so the full selection over LDS
# runs), and the one-hot query.
LONG_NC_CASES = {
    "t40960_nc10240": dict(context=40960, components=1024, nc=10240, nprobe=256, seed_shift=5),
    "t98304_nc24576": dict(context=98304, components=2048, nc=24576, nprobe=256, seed_shift=9),
}


@pytest.mark.parametrize("name", list(LONG_NC_CASES))
def test_long_centroid_lists_in_registers(runtimes, name):
    p = LONG_NC_CASES[name]
    index, k, v, qs = case(**p)
    print(f"[gpu] create runtime {name}", flush=True)
    rt = runtimes[name] = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=True)
    queries = {"real": qs[0], **{k_: q for k_, q in degenerate_queries(qs[0]).items()
                                 if k_ in ("zero", "onehot")}}
    for kind, q in queries.items():
        print(f"[gpu] {name} query {kind}", flush=True)
        rt.bind_query(q)
        rt.enqueue()
        status = rt.synchronize()
        assert status["err"] == [0, 0, 0, 0]
        traces, out = oracle_step(p, q)
        for g, tr in enumerate(traces):
            np.testing.assert_array_equal(rt.read_stage("thresh", g), tr.thr, err_msg=f"{kind} g{g}")
            np.testing.assert_array_equal(rt.read_stage("selected", g), tr.selected,
                                          err_msg=f"{kind} g{g}")
            np.testing.assert_array_equal(rt.read_stage("pool", g), tr.pool, err_msg=f"{kind} g{g}")
            np.testing.assert_array_equal(rt.read_stage("top", g), tr.top100, err_msg=f"{kind} g{g}")
        got = rt.read_output().float().numpy().reshape(16, 256)
        for j in range(16):
            assert np.abs(got[j] - out[j]).max() <= 2e-2, f"{kind} head {j} max-abs"
