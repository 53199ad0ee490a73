"""The reference-side binding (``seoulkv_amd.ref_runtime``), host logic only.

The reference's public classes call five names of ``seoulkv4._runtime`` with
fixed positional parameters (``_runtime.py:21,36,180,189,197``) and read
outputs through ``result.py:30-38``: ``rows = ttnn.to_torch(item)[0]`` then
``rows[g, g]`` for g in 0..3.  These tests pin the seam's signatures and the
output layout without a GPU (a stand-in runtime supplies the output buffer)."""

from __future__ import annotations

import inspect

import pytest
import torch

from seoulkv_amd import ref_runtime


def test_seam_names_and_parameters_match_the_reference():
    expected = {
        "_ttnn": [],
        "initialize": ["ttnn", "device", "k", "v", "q", "index", "args"],
        "bind_query": ["state", "q", "args"],
        "enqueue": ["state"],
        "metadata": ["state"],
    }
    for name, params in expected.items():
        fn = getattr(ref_runtime, name)
        assert list(inspect.signature(fn).parameters) == params, name
    dev = ref_runtime._Device()
    assert callable(dev.synchronize_device) and callable(dev.to_torch)


class _StubHandle:
    """Stand-in output handle: a padded [1, 32, 4, 256] tensor whose row
    [0, h, h] holds 4 * slot + h + 1 (the layout the library writes)."""

    def __init__(self, slot):
        self.t = torch.zeros(1, 32, 4, 256, dtype=torch.bfloat16)
        for h in range(4):
            self.t[0, h, h] = 4 * slot + h + 1

    def to_torch(self):
        return self.t


def test_reference_readback_takes_the_head_diagonal():
    """The reference's DecodeResult.to_torch (result.py:30-38), restated,
    through the shim's device module: row [0, h, h] of KV head g's tensor is
    query head 4 g + h."""
    dev = ref_runtime._Device()
    groups = []
    for item in [_StubHandle(g) for g in range(4)]:
        rows = dev.to_torch(item)[0]
        groups.append(torch.stack([rows[g, g] for g in range(4)]))
    got = torch.cat(groups, dim=0).reshape(16, 256)
    assert torch.equal(got[:, 0].float(), torch.arange(1, 17, dtype=torch.float32))


def test_debug_handle_is_the_runtime_ids():
    class R:
        ids = torch.arange(4 * 4 * 100).reshape(4, 4, 100)

        def debug_ids(self):
            return self.ids

    ids = ref_runtime._Device.to_torch(ref_runtime.DebugIndices(R()))
    assert torch.equal(ids.reshape(4, 4, -1)[..., :100].long(), R.ids)


def test_bind_query_checks_the_reference_shape():
    class Args:
        n_heads = 16

    calls = []

    class R:
        def bind_query(self, q):
            calls.append(tuple(q.shape))

    state = {"n_conc": 1, "head_dim": 256, "runtime": R()}
    with pytest.raises(ValueError, match="unexpected SeoulKV4 query shape"):
        ref_runtime.bind_query(state, torch.zeros(1, 16, 256, dtype=torch.bfloat16), Args)
    ref_runtime.bind_query(state, torch.zeros(1, 1, 16, 256, dtype=torch.bfloat16), Args)
    assert calls == [(1, 1, 16, 256)]


def test_device_argument_is_a_rocm_device():
    assert ref_runtime._ordinal(0) == 0
    assert ref_runtime._ordinal("cuda:1") == 1
    assert ref_runtime._ordinal(torch.device("cuda", 2)) == 2
    with pytest.raises(ValueError):
        ref_runtime._ordinal("cpu")
    with pytest.raises(ValueError):
        ref_runtime._ordinal(None)
