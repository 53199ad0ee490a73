"""Configuration of the single-cache sparse decode profile.

Mirrors the reference ``config.py:1-40``.  Two extensions:
``stage15_capacity=None``: the reference caps the deduplicated candidate pool
per KV group at 12288..24576 keys because its pool lives in Tensix L1.  On
MI355X the pool lives in HBM and is sized for the worst case (every retrieval
token), so ``None`` lifts the cap; an integer keeps the reference's
"error, never truncate" capacity check bit for bit.
``append_capacity``: tokens per KV head that ``SeoulKV4.append`` may add after
the prefill (0, the default, is the reference's static cache).
"""

from __future__ import annotations

from dataclasses import dataclass

DEFAULT_NPROBE = 256
STAGE16_PER_HEAD = 256
STAGE16_PER_SHARD = STAGE16_PER_HEAD

N_KV_HEADS = 4
N_HEADS = 16
GQA_GROUP = N_HEADS // N_KV_HEADS
HEAD_DIM = 256
TOPK = 100
STAGE15_M = 2048          # Stage-1.5 frontier per head (and the pool minimum)
STAGE15_UNION_M = 1600    # ranks of each head's frontier entering the union
STAGE16_M = STAGE16_PER_HEAD
MAX_CONTEXT = 1 << 20     # token IDs fit 20 bits in the device selection keys
MAX_CENTROIDS = 65536


@dataclass(frozen=True)
class SeoulKV4Config:
    """``stage15_capacity``: pool capacity per KV group (multiple of 768 in
    [12288, 24576], as in the reference) or ``None`` for an HBM-sized pool.
    ``debug``: keep the final top-100 IDs readable via ``debug_snapshot``.
    ``append_capacity``: tokens per KV head ``append`` may add (0: static)."""

    stage15_capacity: int | None = 13056
    debug: bool = False
    append_capacity: int = 0

    def __post_init__(self):
        n = self.stage15_capacity
        if n is not None and (
            type(n) is not int or not 12288 <= n <= 24576 or n % (6 * 4 * 32)
        ):
            raise ValueError(
                "stage15_capacity must be a multiple of 768 in [12288, 24576] "
                "or None for an HBM-sized pool"
            )
        if type(self.debug) is not bool:
            raise TypeError("debug must be a bool")
        if type(self.append_capacity) is not int or not 0 <= self.append_capacity <= MAX_CONTEXT:
            raise ValueError("append_capacity must be an int in [0, 2^20]")


@dataclass(frozen=True)
class _KernelOptions:
    """Fixed budgets of the decode funnel (reference ``config.py:25-40``)."""

    context_len: int
    stage15_capacity: int | None
    debug: bool
    n_conc = seq_len = 1
    n_kv_heads = N_KV_HEADS
    n_heads = N_HEADS
    head_dim = HEAD_DIM
    topk = TOPK
    stage15_m = STAGE15_M
    stage15_union_m = STAGE15_UNION_M
    stage16_m = STAGE16_M
