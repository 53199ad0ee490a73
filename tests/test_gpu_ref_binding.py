"""The reference's own call sequence through ``seoulkv_amd.ref_runtime`` on the
GPU, checked against the oracle.

Restated (the reference is not imported): ``SeoulKV4.run`` (``api.py:91-102``)
calls ``_runtime._ttnn()``, ``initialize(tt, device, k, v, q, index, args)``,
``bind_query(state, q, args)`` and ``enqueue(state)``; ``DecodeResult.to_torch``
(``result.py:30-38``) synchronises and stacks ``tt.to_torch(item)[0][g, g]``;
``debug_snapshot`` (``api.py:119-126``) reshapes ``tt.to_torch(debug_indices)``.
The index object exposes only ``_cells`` / ``_zones`` as the reference's does
(``index.py:41-56``) and ``args`` carries the reference's ``_KernelOptions``
field names (``config.py:25-40``)."""

from __future__ import annotations

import types
from dataclasses import dataclass

import numpy as np
import pytest
import torch

from seoulkv_amd import ref_runtime
from tests.helpers import case, cosine, oracle_step

pytestmark = pytest.mark.gpu

P0 = dict(context=8192, components=256, nc=512, nprobe=64)
P1 = dict(context=32768, components=1024, nc=2048, nprobe=384)


@dataclass(frozen=True)
class RefKernelOptions:  # field names of the reference's _KernelOptions
    context_len: int
    skv4_stage15_candidates: int | None
    skv4_debug_indices: bool
    n_conc = seq_len = 1
    n_kv_heads = 4
    n_heads = 16
    topk = 100
    skv4_stage15_m = 2048
    skv4_stage15_union_m = 1600


def _ref_index(index):
    return types.SimpleNamespace(_cells=index.cells, _zones=index.zones)


def _to_torch(tt, device, state):
    tt.synchronize_device(device)
    groups = []
    for item in state["selector"]["outputs"]:
        rows = tt.to_torch(item)[0]
        groups.append(torch.stack([rows[g, g] for g in range(4)]))
    return torch.cat(groups, dim=0).reshape(1, 1, 16, 256).contiguous()


def _check(out, ids, traces, ref):
    want = np.stack([t.top100 for t in traces])
    assert np.array_equal(ids.numpy(), want)
    got = out.float().numpy().reshape(16, 256)
    for j in range(16):
        assert np.abs(got[j] - ref[j]).max() <= 2e-2
        assert cosine(got[j], ref[j]) >= 0.999


def test_reference_call_sequence_matches_the_oracle():
    index, k, v, qs = case(**P0)
    print("[gpu] reference seam cfg0", flush=True)
    args = RefKernelOptions(8192, 13056, True)
    tt = ref_runtime._ttnn()
    device = torch.device("cuda", 0)
    state = ref_runtime.initialize(tt, device, k, v, qs[0], _ref_index(index), args)
    try:
        for q in qs:
            ref_runtime.bind_query(state, q, args)
            ref_runtime.enqueue(state)
            out = _to_torch(tt, device, state)
            ids = tt.to_torch(state["selector"]["debug_indices"]).reshape(4, 4, -1)[..., :100].long()
            traces, ref = oracle_step(P0, q)
            _check(out, ids, traces, ref)
        meta = ref_runtime.metadata(state)
        assert meta["context"] == 8192 and len(meta["programs"]) == meta["kernels_per_step"]
        views = [item.device_view() for item in state["selector"]["outputs"]]
        assert all(t.shape == (1, 32, 4, 256) for t in views)
        diag = torch.cat([torch.stack([t[0, h, h] for h in range(4)]) for t in views])
        assert torch.equal(diag.cpu(), out.reshape(16, 256))
    finally:
        state["runtime"].close()


def test_reference_capacity_check_never_truncates():
    index, k, v, qs = case(**P1)
    print("[gpu] reference seam capacity cfg1", flush=True)
    tt = ref_runtime._ttnn()
    with pytest.raises(ValueError, match="never truncate"):
        ref_runtime.initialize(tt, 0, k, v, qs[0], _ref_index(index),
                               RefKernelOptions(32768, 13056, False))
