"""Cache append on the GPU: appended tokens join the local window.

After n appended tokens the step must equal the oracle's step over the grown
cache (context T0 + n, local window L + n, the prefill's index, codes and
scales): top-100 IDs bit for bit, the attention output within the north-star
bound (max-abs <= 2e-2, cosine >= 0.999 per query head).  The appended FP8
records must equal torch's FP8 e4m3fn cast of the BF16 inputs bit for bit.
The appended keys lean towards the query, so the output moves visibly when
they are attended and a dropped or misplaced token fails the bound.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import arith
from oracle import decode as od
from seoulkv_amd import _hip
from tests.helpers import bits, case, cosine, oracle_inputs

pytestmark = pytest.mark.gpu

P = dict(context=8192, components=256, nc=512, nprobe=64)
SINK, LOCAL = 128, 256
CAPACITY = 700


def new_tokens(q: torch.Tensor, n: int, seed: int):
    """[4, n, 256] BF16 K/V: keys along the group's mean query plus noise."""
    gen = torch.Generator().manual_seed(seed)
    qg = q.reshape(4, 4, 256).float().mean(dim=1)  # [4, 256]
    qg = qg / qg.norm(dim=1, keepdim=True)
    w = torch.rand(4, n, 1, generator=gen) * 8.0
    w[:, 0] = 12.0  # one strong key per call: even a 1-token append shows
    k = w * qg[:, None, :] + torch.randn(4, n, 256, generator=gen)
    v = torch.randn(4, n, 256, generator=gen) * 2.0
    return k.bfloat16(), v.bfloat16()


def fp8_bytes(x_bits: np.ndarray) -> np.ndarray:
    t = torch.from_numpy(np.ascontiguousarray(x_bits).view(np.int16)).view(torch.bfloat16)
    return t.float().to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def oracle_grown(q, ks, vs):
    """The oracle step over the prefill cache plus the appended tokens."""
    cells, code8, scales, k8, v8 = oracle_inputs(**P)
    n = sum(k.shape[1] for k in ks)
    if n:
        k8n, v8n = od.fp8_records(bits(torch.cat(ks, 1)), bits(torch.cat(vs, 1)))
        k8 = np.concatenate([k8, k8n], axis=1)
        v8 = np.concatenate([v8, v8n], axis=1)
    traces, out = od.decode_step(cells, code8, scales, k8, v8, bits(q).reshape(16, 256),
                                 sink=SINK, local=LOCAL + n, context=P["context"] + n)
    return traces, out, k8, v8


def check_step(rt, q, ks, vs, label):
    rt.bind_query(q)
    rt.enqueue()
    status = rt.synchronize()
    assert status["err"] == [0, 0, 0, 0], label
    traces, out, _, _ = oracle_grown(q, ks, vs)
    for g, tr in enumerate(traces):
        np.testing.assert_array_equal(rt.read_stage("top", g), tr.top100, err_msg=f"{label} g{g}")
    got = rt.read_output().float().numpy().reshape(16, 256)
    for j in range(16):
        assert np.abs(got[j] - out[j]).max() <= 2e-2, f"{label} head {j} max-abs"
        assert cosine(got[j], out[j]) >= 0.999, f"{label} head {j} cosine"
    return got


def test_append_host_and_device():
    index, k, v, qs = case(**P)
    q = qs[0]
    print("[gpu] append: create", flush=True)
    rt = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=True,
                      append_capacity=CAPACITY)
    try:
        before = check_step(rt, q, [], [], "prefill")
        ks, vs = [], []
        # 1 token (384 -> 385 dense keys: a second 256-key slice starts),
        # 300 more (a third slice), 257 from device memory (a fourth)
        for step, (n, where) in enumerate([(1, "cpu"), (300, "cpu"), (257, "cuda")]):
            kn, vn = new_tokens(q, n, seed=100 + step)
            print(f"[gpu] append {n} tokens from {where}", flush=True)
            rt.append(kn.to(where), vn.to(where))
            ks.append(kn)
            vs.append(vn)
            got = check_step(rt, q, ks, vs, f"after append {step}")
            assert np.abs(got - before).max() > 5e-2  # the new keys are attended
        assert rt.metadata()["appended"] == 558
        assert rt.metadata()["local"] == LOCAL + 558
        # the appended records, bit for bit
        kall, vall = bits(torch.cat(ks, 1)), bits(torch.cat(vs, 1))
        for g in range(4):
            rec = rt.read_stage("kv8", g).reshape(-1, 512)
            assert rec.shape[0] == P["context"] + 558
            np.testing.assert_array_equal(rec[P["context"]:, 256:], fp8_bytes(kall[g]))
            np.testing.assert_array_equal(rec[P["context"]:, :256], fp8_bytes(vall[g]))
        # beyond the capacity: refused, cache unchanged
        kn, vn = new_tokens(q, CAPACITY - 558 + 1, seed=7)
        with pytest.raises(RuntimeError, match="append"):
            rt.append(kn, vn)
        check_step(rt, q, ks, vs, "after refused append")
        # a device append whose arrays are host memory: refused, cache unchanged
        host = torch.empty(4 * 8 * 256 * 2, dtype=torch.uint8, pin_memory=True)
        code = rt.lib.skv_append_device(rt.handle, host.data_ptr(), host.data_ptr(), 8)
        assert code == 1, code  # SKV_EINVAL
        assert "not device memory" in rt.lib.skv_last_error(rt.handle).decode()
        assert rt.metadata()["appended"] == 558
        check_step(rt, q, ks, vs, "after refused device append")
        # the dense comparison path covers the appended keys too
        rt.dense_decode()
        dense = rt.read_dense_output().float().numpy().reshape(16, 256).astype(np.float64)
        _, _, k8, v8 = oracle_grown(q, ks, vs)
        qf = arith.bf16_to_f32(bits(q).reshape(16, 256))
        ids = np.arange(P["context"] + 558)
        for j in range(16):
            ref = od.sdpa(qf[j], k8[j // 4], v8[j // 4], ids)
            assert np.abs(dense[j] - ref).max() <= 2e-2, f"dense head {j}"
            assert cosine(dense[j], ref) >= 0.999, f"dense head {j}"
    finally:
        rt.close()


def test_append_with_graph_mode():
    """A captured step is dropped by an append and captured again with the
    grown shapes: its output equals the eager step's."""
    index, k, v, qs = case(**P)
    q = qs[1]
    rt = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=True,
                      append_capacity=CAPACITY)
    try:
        rt.bind_query(q)
        rt.graph_mode(True)
        rt.enqueue()
        rt.synchronize()
        kn, vn = new_tokens(q, 200, seed=11)
        print("[gpu] append under graph mode", flush=True)
        rt.append(kn, vn)
        for _ in range(3):
            rt.enqueue()
            rt.synchronize()
            graph_out = rt.read_output()
            rt.graph_mode(False)
            rt.enqueue()
            rt.synchronize()
            assert torch.equal(rt.read_output(), graph_out)
            rt.graph_mode(True)
        check_step(rt, q, [kn], [vn], "graph after append")
    finally:
        rt.close()


def test_host_append_over_several_staging_chunks():
    """A host append of 2100 tokens is staged in 256-token rounds (nine
    rounds here, through two alternating pinned slots): every record lands
    at its row and the step over the grown cache equals the oracle's."""
    index, k, v, qs = case(**P)
    q = qs[0]
    n = 2100
    rt = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=True,
                      append_capacity=2500)
    try:
        kn, vn = new_tokens(q, n, seed=21)
        print(f"[gpu] host append of {n} tokens", flush=True)
        rt.append(kn, vn)
        check_step(rt, q, [kn], [vn], "multi-chunk append")
        kb, vb = bits(kn), bits(vn)
        for g in range(4):
            rec = rt.read_stage("kv8", g).reshape(-1, 512)
            assert rec.shape[0] == P["context"] + n
            np.testing.assert_array_equal(rec[P["context"]:, 256:], fp8_bytes(kb[g]))
            np.testing.assert_array_equal(rec[P["context"]:, :256], fp8_bytes(vb[g]))
    finally:
        rt.close()


def test_host_appends_at_the_staging_slot_boundaries():
    """Host appends of 255, 256, 257, 511, 512 and 513 tokens in a row: one
    slot not quite full, exactly full, a second chunk of one token, both
    slots, and a third chunk that reuses the first slot once the pack kernel
    that read it has finished.  Every record lands at its row (FP8 bytes
    against torch's cast) and the step over the grown cache equals the
    oracle's."""
    index, k, v, qs = case(**P)
    q = qs[1]
    sizes = (255, 256, 257, 511, 512, 513)
    total = sum(sizes)
    rt = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=True,
                      append_capacity=total)
    try:
        ks, vs = [], []
        for i, n in enumerate(sizes):
            kn, vn = new_tokens(q, n, seed=40 + i)
            print(f"[gpu] host append of {n} tokens", flush=True)
            rt.append(kn, vn)
            ks.append(kn)
            vs.append(vn)
        check_step(rt, q, ks, vs, "slot-boundary appends")
        kb, vb = bits(torch.cat(ks, 1)), bits(torch.cat(vs, 1))
        for g in range(4):
            rec = rt.read_stage("kv8", g).reshape(-1, 512)
            assert rec.shape[0] == P["context"] + total
            np.testing.assert_array_equal(rec[P["context"]:, 256:], fp8_bytes(kb[g]))
            np.testing.assert_array_equal(rec[P["context"]:, :256], fp8_bytes(vb[g]))
    finally:
        rt.close()


@pytest.mark.parametrize("paged", [False, True])
def test_decode_loop_folds_small_host_appends_into_the_step(paged):
    """A decoder's loop: append the decoded token from the host, bind the next
    query, enqueue, with no host synchronisation for 12 steps (each step's
    output copied aside on the instance's stream); every step must equal the
    oracle's step over exactly the tokens appended before it.  Then the
    other orders a caller may use: an append followed by a step without a
    new bind, two appends before a step, the largest folded append (16) and
    the smallest unfolded one (17), an append followed by the dense decode,
    by a record readback and by a device-query bind.  FP8 records in pages
    (a scrambled page table) take the same path through the table."""
    from seoulkv_amd import KVPagePool
    from seoulkv_amd.result import _DeviceArray

    index, k, v, qs = case(**P)
    st = torch.cuda.Stream()
    kv_pages = None
    if paged:
        pool = KVPagePool(64, page_tokens=256, device="cuda:0")
        pages = pool.allocate(pool.n_pages)
        import random
        random.Random(3).shuffle(pages)
        kv_pages = (pool, pages[: -(-(P["context"] + CAPACITY) // 256)])
    rt = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=True,
                      append_capacity=CAPACITY, stream=st.cuda_stream, kv_pages=kv_pages)
    try:
        ks, vs = [], []
        n_loop = 12
        toks = [new_tokens(qs[i % 2], 1, seed=300 + i) for i in range(n_loop)]
        out = torch.as_tensor(_DeviceArray(rt.output_device_ptr(), (16, 256), "<i2"),
                              device="cuda:0")
        got = torch.zeros((n_loop, 16, 256), dtype=torch.int16, device="cuda:0")
        torch.cuda.synchronize()
        print(f"[gpu] decode loop of {n_loop} host appends (paged={paged})", flush=True)
        with torch.cuda.stream(st):
            for i, (kn, vn) in enumerate(toks):
                rt.append(kn, vn)
                rt.bind_query(qs[i % 2])
                rt.enqueue()
                got[i].copy_(out)
        st.synchronize()
        got = got.cpu().view(torch.bfloat16).float().numpy()
        for i, (kn, vn) in enumerate(toks):
            ks.append(kn)
            vs.append(vn)
            _, ref, _, _ = oracle_grown(qs[i % 2], ks, vs)
            for j in range(16):
                assert np.abs(got[i][j] - ref[j]).max() <= 2e-2, f"loop step {i} head {j}"
                assert cosine(got[i][j], ref[j]) >= 0.999, f"loop step {i} head {j}"
        q = qs[0]
        rt.bind_query(q)
        # an append, then a step on the bound query (no new bind)
        kn, vn = new_tokens(q, 1, seed=401)
        rt.append(kn, vn)
        ks.append(kn)
        vs.append(vn)
        rt.enqueue()
        rt.synchronize()
        _, ref, _, _ = oracle_grown(q, ks, vs)
        got1 = rt.read_output().float().numpy().reshape(16, 256)
        for j in range(16):
            assert cosine(got1[j], ref[j]) >= 0.999, f"append without bind, head {j}"
        # two appends before a step, the largest folded append, the smallest
        # unfolded one
        for step, sizes in enumerate([(3, 2), (16,), (17,)]):
            for u, n in enumerate(sizes):
                kn, vn = new_tokens(q, n, seed=500 + 10 * step + u)
                rt.append(kn, vn)
                ks.append(kn)
                vs.append(vn)
            check_step(rt, q, ks, vs, f"appends {sizes}")
        # a pending append, then the dense decode over every key
        kn, vn = new_tokens(q, 4, seed=601)
        rt.append(kn, vn)
        ks.append(kn)
        vs.append(vn)
        rt.dense_decode()
        dense = rt.read_dense_output().float().numpy().reshape(16, 256).astype(np.float64)
        _, _, k8, v8 = oracle_grown(q, ks, vs)
        qf = arith.bf16_to_f32(bits(q).reshape(16, 256))
        ids = np.arange(k8.shape[1])
        for j in range(16):
            ref = od.sdpa(qf[j], k8[j // 4], v8[j // 4], ids)
            assert np.abs(dense[j] - ref).max() <= 2e-2, f"dense after append, head {j}"
        # a pending append, then a record readback
        kn, vn = new_tokens(q, 2, seed=602)
        rt.append(kn, vn)
        ks.append(kn)
        vs.append(vn)
        kall, vall = bits(torch.cat(ks, 1)), bits(torch.cat(vs, 1))
        n_app = kall.shape[1]
        for g in range(4):
            rec = rt.read_stage("kv8", g).reshape(-1, 512)
            assert rec.shape[0] == P["context"] + n_app
            np.testing.assert_array_equal(rec[P["context"]:, 256:], fp8_bytes(kall[g]))
            np.testing.assert_array_equal(rec[P["context"]:, :256], fp8_bytes(vall[g]))
        # a pending append, then a device-query bind
        kn, vn = new_tokens(q, 5, seed=603)
        rt.append(kn, vn)
        ks.append(kn)
        vs.append(vn)
        with torch.cuda.stream(st):
            rt.bind_query_device(qs[1].reshape(16, 256).to("cuda:0"))
        rt.enqueue()
        rt.synchronize()
        _, ref, _, _ = oracle_grown(qs[1], ks, vs)
        got2 = rt.read_output().float().numpy().reshape(16, 256)
        for j in range(16):
            assert cosine(got2[j], ref[j]) >= 0.999, f"device bind after append, head {j}"
        assert rt.metadata()["appended"] == n_app + 5
    finally:
        torch.cuda.synchronize()
        rt.close()


def test_appended_records_match_torch_cast_for_every_bf16_pattern():
    """The FP8 e4m3fn records of appended tokens equal torch's cast for all
    65536 BF16 bit patterns (zeros, subnormals, the 448 / 464 rounding edge,
    infinities, every NaN), through the bulk pack kernel and through the
    folded append that the next step's first kernel packs."""
    index, k, v, qs = case(**P)
    rt = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=True,
                      append_capacity=64 + 16)
    try:
        pat = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
        kn = pat.reshape(4, 64, 256)
        vn = pat.flip(0).reshape(4, 64, 256)  # V sees every pattern too
        print("[gpu] every BF16 pattern through the record packers", flush=True)
        rt.append(kn, vn)  # 64 tokens: the bulk pack kernel
        ks, vs = bits(kn), bits(vn)
        for g in range(4):
            rec = rt.read_stage("kv8", g).reshape(-1, 512)[P["context"]:]
            np.testing.assert_array_equal(rec[:, 256:], fp8_bytes(ks[g]))
            np.testing.assert_array_equal(rec[:, :256], fp8_bytes(vs[g]))
        # 16 tokens folded into the next step (their NaN keys make the
        # output NaN; only the records are checked)
        sel = torch.randperm(65536, generator=torch.Generator().manual_seed(5))[:4 * 16 * 256]
        sel[:256] = torch.arange(0x7f80, 0x7f80 + 256)  # +inf and NaNs
        kf = pat[sel].reshape(4, 16, 256)
        vf = pat[sel.flip(0)].reshape(4, 16, 256)
        rt.append(kf, vf)
        rt.bind_query(qs[0])
        rt.enqueue()
        rt.synchronize()
        kb, vb = bits(kf), bits(vf)
        for g in range(4):
            rec = rt.read_stage("kv8", g).reshape(-1, 512)[P["context"] + 64:]
            np.testing.assert_array_equal(rec[:, 256:], fp8_bytes(kb[g]))
            np.testing.assert_array_equal(rec[:, :256], fp8_bytes(vb[g]))
    finally:
        rt.close()
