"""An index with n_centroids = 65536 built from a small one by appending empty
clusters, with nprobe = n_centroids (accepted by the C ABI, not by
SeoulKV4Index.build): every centroid is then selected, so each 1024-centroid
range of the pool kernel selects all of its 1024 clusters."""

from __future__ import annotations

import types

import torch

from tests.helpers import case

NC_PADDED = 65536
SMALL = dict(context=8192, components=256, nc=512, nprobe=64)


def padded_index(nc_total: int = NC_PADDED):
    index, k, v, qs = case(**SMALL)
    cells = []
    for cell in index.cells:
        nc = int(cell["offsets"].numel()) - 1
        pad = nc_total - nc
        assert pad % 32 == 0
        c = dict(cell)
        zeros = torch.zeros(pad, 64, dtype=torch.uint8)
        c["upper"] = torch.cat([cell["upper"], zeros])
        c["lower"] = torch.cat([cell["lower"], zeros])
        # one shared scale per 32-centroid group (the codec's layout)
        c["scale"] = torch.cat([cell["scale"].float(),
                                torch.full((pad,), float(cell["scale"][-1]))])
        c["coarse_residual_norm"] = torch.cat(
            [cell["coarse_residual_norm"].half(), torch.zeros(pad, dtype=torch.float16)])
        c["group_fine_scale"] = torch.cat(
            [cell["group_fine_scale"].half(),
             torch.full((pad // 32,), float(cell["group_fine_scale"][-1]), dtype=torch.float16)])
        off = cell["offsets"].long()
        c["offsets"] = torch.cat([off, off[-1:].expand(pad)])
        c["p"] = nc_total
        cells.append(c)
    return types.SimpleNamespace(cells=tuple(cells), zones=index.zones), k, v, qs
