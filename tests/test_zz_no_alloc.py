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
