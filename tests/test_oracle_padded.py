"""The oracle on an index whose every centroid is selected (nprobe = nc =
65536): the selection is all clusters ascending, and the pool holds every
retrieval token once, at its first posting in CSR order (the reference's
``expand_lists`` order with duplicates dropped, ``_codecs/index.py:91-94``)."""

from __future__ import annotations

import numpy as np

from oracle import decode as od
from tests.helpers import bits
from tests.padded_cells import NC_PADDED, padded_index


def test_every_centroid_selected_pool_is_first_occurrence_order():
    index, k, v, qs = padded_index()
    code8, scales = od.key_codec(bits(k))
    k8, v8 = od.fp8_records(bits(k), bits(v))
    cells = [od.GroupCell.from_cell(c) for c in index.cells]
    traces, _ = od.decode_step(cells, code8, scales, k8, v8, bits(qs[0]).reshape(16, 256),
                               sink=index.zones.sink, local=index.zones.local)
    for cell, tr in zip(cells, traces):
        assert np.array_equal(tr.selected, np.arange(NC_PADDED))
        _, first = np.unique(cell.values, return_index=True)
        expect = cell.values[np.sort(first)]
        assert np.array_equal(tr.pool, expect)
        z = index.zones
        assert len(tr.pool) == z.context - z.sink - z.local
