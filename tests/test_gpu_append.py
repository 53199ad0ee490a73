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
    """A host append of 2100 tokens is staged in 1024-token rounds (three
    rounds here): every record lands at its row and the step over the grown
    cache equals the oracle's."""
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
