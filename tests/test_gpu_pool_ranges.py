"""Pool ranges whose every cluster is selected, on the GPU.

At n_centroids = 65536 each block of the pool kernel owns a range of 1024
centroids; with nprobe = n_centroids (through the C ABI) all 1024 are
selected in every range, the largest selected count the kernel's range scan
holds.  Every stage is compared with the oracle."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import decode as od
from seoulkv_amd import _hip
from tests.helpers import bits, cosine
from tests.padded_cells import NC_PADDED, padded_index

pytestmark = pytest.mark.gpu


def test_fully_selected_1024_centroid_ranges():
    index, k, v, qs = padded_index()
    code8, scales = od.key_codec(bits(k))
    k8, v8 = od.fp8_records(bits(k), bits(v))
    cells = [od.GroupCell.from_cell(c) for c in index.cells]
    traces, ref = od.decode_step(cells, code8, scales, k8, v8, bits(qs[0]).reshape(16, 256),
                                 sink=index.zones.sink, local=index.zones.local)
    print(f"[gpu] nc={NC_PADDED} nprobe=nc: every range fully selected", flush=True)
    rt = _hip.Runtime(0, k, v, index, pool_min=0, pool_capacity=None, debug=True)
    try:
        rt.bind_query(qs[0])
        rt.enqueue()
        status = rt.synchronize()
        assert status["err"] == [0, 0, 0, 0]
        assert status["selected"] == [NC_PADDED] * 4
        for g, tr in enumerate(traces):
            assert status["pool"][g] == len(tr.pool)
            np.testing.assert_array_equal(rt.read_stage("selected", g), tr.selected)
            np.testing.assert_array_equal(rt.read_stage("pool", g), tr.pool)
            np.testing.assert_array_equal(rt.read_stage("u1", g), tr.u1)
            np.testing.assert_array_equal(rt.read_stage("u2", g), tr.u2)
            np.testing.assert_array_equal(rt.read_stage("top", g), tr.top100)
        got = rt.read_output().float().numpy().reshape(16, 256)
        for j in range(16):
            assert np.abs(got[j] - ref[j]).max() <= 2e-2
            assert cosine(got[j], ref[j]) >= 0.999
    finally:
        rt.close()
