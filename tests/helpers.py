"""Shared test helpers: seeded cases and the oracle trace of one decode step."""

from __future__ import annotations

import functools

import numpy as np
import torch

from oracle import arith
from oracle import decode as od
from seoulkv_amd.index import SeoulKV4Index
from seoulkv_amd.synthetic import make_cache


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


@functools.lru_cache(maxsize=8)
def case(context=8192, components=256, nc=512, nprobe=64, clustered=True, n_queries=2,
         sink=128, local=256, seed_shift=0):
    """(index, k, v, queries) for a seeded synthetic cache."""
    k, v, qs = make_cache(
        context, components, clustered=clustered, sink=sink, local=local,
        seed_k=1234 + seed_shift, seed_v=1235 + seed_shift, seed_q=1236 + seed_shift,
        n_queries=n_queries,
    )
    index = SeoulKV4Index.build(k, v, sink=sink, local=local, nprobe=nprobe, n_centroids=nc)
    return index, k, v, tuple(qs)


@functools.lru_cache(maxsize=8)
def oracle_inputs(context=8192, components=256, nc=512, nprobe=64, clustered=True,
                  n_queries=2, sink=128, local=256, seed_shift=0):
    index, k, v, qs = case(context, components, nc, nprobe, clustered, n_queries, sink,
                           local, seed_shift)
    code8, scales = od.key_codec(bits(k))
    k8, v8 = od.fp8_records(bits(k), bits(v))
    cells = [od.GroupCell.from_cell(c) for c in index.cells]
    return cells, code8, scales, k8, v8


def oracle_step(params: dict, q: torch.Tensor):
    cells, code8, scales, k8, v8 = oracle_inputs(**params)
    sink, local = params.get("sink", 128), params.get("local", 256)
    return od.decode_step(cells, code8, scales, k8, v8, bits(q).reshape(16, 256),
                          sink=sink, local=local)


def unorder(o: np.ndarray) -> np.ndarray:
    """Inverse of ordered16: ordered value -> BF16 bits."""
    o = np.asarray(o, dtype=np.uint32)
    return np.where(o & 0x8000, o ^ 0x8000, (~o) & 0xFFFF).astype(np.uint16)


def cosine(a, b) -> float:
    a = np.asarray(a, dtype=np.float64).ravel()
    b = np.asarray(b, dtype=np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


__all__ = ["arith", "bits", "case", "cosine", "oracle_inputs", "oracle_step", "unorder"]
