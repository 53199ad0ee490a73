"""The allocation-free entry point ``skv_dense_decode_static`` against the
existing ``skv_dense_decode`` through the C ABI: two calls in a row on one
record buffer, the second over fewer keys, each bit-identical to the
existing entry point on a handle over the same keys and within the attention
tolerance of the oracle's float64 softmax."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import arith
from oracle import decode as od
from seoulkv_amd import _hip
from seoulkv_amd.index import SeoulKV4Index
from tests.helpers import bits, case, cosine

pytestmark = pytest.mark.gpu


def _records(k, v):
    """[4, T, 512] uint8 FP8 e4m3fn [V || K] records (torch's cast)."""
    k8 = k.float().to(torch.float8_e4m3fn).view(torch.uint8)
    v8 = v.float().to(torch.float8_e4m3fn).view(torch.uint8)
    return torch.cat([v8, k8], dim=-1).contiguous()


def test_static_dense_decode_matches_handle_dense_decode():
    _, k, v, qs = case(context=8192, components=256, nc=512, nprobe=64)
    q = qs[0]
    dev = torch.device("cuda", 0)
    kv = _records(k, v).to(dev)  # rows = 8192
    qd = q.reshape(16, 256).contiguous().to(dev)
    out = torch.empty(16, 256, dtype=torch.bfloat16, device=dev)
    qf = arith.bf16_to_f32(bits(q).reshape(16, 256))
    for T in (8192, 6400):  # second call: fewer keys, same buffers
        print(f"[gpu] static dense decode T={T}", flush=True)
        _hip.dense_decode_static(kv, T, qd, out)
        torch.cuda.synchronize()
        got = out.cpu()
        kT, vT = k[:, :T].contiguous(), v[:, :T].contiguous()
        index = SeoulKV4Index.build(kT, vT, nprobe=64, n_centroids=256)
        rt = _hip.Runtime(0, kT, vT, index, pool_min=0, pool_capacity=None, debug=False)
        try:
            rt.bind_query(q)
            rt.dense_decode()
            ref_dev = rt.read_dense_output().reshape(16, 256)
        finally:
            rt.close()
        assert torch.equal(got.view(torch.int16), ref_dev.view(torch.int16)), T
        k8, v8 = od.fp8_records(bits(kT), bits(vT))
        g = got.float().numpy()
        for j in range(16):
            ref = od.sdpa(qf[j], k8[j // 4], v8[j // 4], np.arange(T))
            assert np.abs(g[j] - ref).max() <= 2e-2, (T, j)
            assert cosine(g[j], ref) >= 0.999, (T, j)


def test_static_dense_decode_rejects_operands_it_cannot_hold():
    """Records shorter than ``rows`` claims (2 GiB past a small tensor's
    allocation) and a host query are refused with SKV_EINVAL by the runtime
    pointer checks before any launch."""
    lib = _hip.load_library()
    dev = torch.device("cuda", 0)
    kv = torch.zeros(4, 1024, 512, dtype=torch.uint8, device=dev)
    qd = torch.zeros(16, 256, dtype=torch.bfloat16, device=dev)
    out = torch.zeros(16, 256, dtype=torch.bfloat16, device=dev)
    host_q = torch.zeros(16, 256, dtype=torch.bfloat16)
    cases = ((kv.data_ptr(), 1 << 20, qd.data_ptr(), out.data_ptr(), "extends past"),
             (kv.data_ptr(), 1024, host_q.data_ptr(), out.data_ptr(), "not device memory"))
    for kv_ptr, rows, q_ptr, out_ptr, text in cases:
        code = lib.skv_dense_decode_static(kv_ptr, rows, 1024, q_ptr, out_ptr, None)
        assert code == 1, text
        assert text in lib.skv_last_error(None).decode()
    torch.cuda.synchronize()
    assert not out.float().abs().sum().item()  # nothing ran


CAPTURE_SCRIPT = r"""
import sys
import torch
sys.path.insert(0, sys.argv[1])
from seoulkv_amd import _hip

gen = torch.Generator().manual_seed(7)
k = torch.randn(4, 8192, 256, generator=gen).bfloat16()
v = torch.randn(4, 8192, 256, generator=gen).bfloat16()
dev = torch.device("cuda", 0)
k8 = k.float().to(torch.float8_e4m3fn).view(torch.uint8)
v8 = v.float().to(torch.float8_e4m3fn).view(torch.uint8)
kv = torch.cat([v8, k8], dim=-1).contiguous().to(dev)
qs = [torch.randn(16, 256, generator=gen).bfloat16().to(dev) for _ in range(2)]
qbuf = qs[0].clone()
out = torch.zeros(16, 256, dtype=torch.bfloat16, device=dev)
torch.cuda.synchronize()
print("capturing the first call of this process", flush=True)
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph):
    _hip.dense_decode_static(kv, 8192, qbuf, out)
replays = []
for q in (qs[0], qs[1], qs[0]):
    qbuf.copy_(q)
    graph.replay()
    torch.cuda.synchronize()
    replays.append(out.clone())
eager = []
for q in qs:
    qbuf.copy_(q)
    _hip.dense_decode_static(kv, 8192, qbuf, out)
    torch.cuda.synchronize()
    eager.append(out.clone())
same = [torch.equal(replays[0].view(torch.int16), eager[0].view(torch.int16)),
        torch.equal(replays[1].view(torch.int16), eager[1].view(torch.int16)),
        torch.equal(replays[2].view(torch.int16), eager[0].view(torch.int16)),
        not torch.equal(eager[0], eager[1])]
print("replays equal eager:", same, flush=True)
sys.exit(0 if all(same) else 3)
"""


def test_static_dense_decode_captured_on_first_call():
    """A fresh process whose first call of the entry point happens under
    stream capture (so the device-array lookup and the operand checks run
    while capturing): the graph replays with a changed query, then the
    first query again, each bit-identical to an eager call."""
    import subprocess
    import sys
    from pathlib import Path

    root = str(Path(__file__).resolve().parents[1])
    print("[gpu] static dense decode captured in a fresh process", flush=True)
    res = subprocess.run([sys.executable, "-c", CAPTURE_SCRIPT, root], capture_output=True,
                         text=True, timeout=240)
    assert res.returncode == 0, (res.returncode, res.stdout[-2000:], res.stderr[-4000:])
    assert "replays equal eager: [True, True, True, True]" in res.stdout
