"""Seeded synthetic caches and queries for the benchmark profiles.

Per KV head g: ``M`` mixture centres ~ N(0, 1)^256, every token draws a
uniform component and ``K_pre = centre + 0.3 * N(0, 1)`` (or i.i.d. N(0, 1)
keys when ``clustered=False``).  RoPE with theta=1e6 in the rotate-half
convention (coordinates i and i+128 form a pair, frequency theta**(-2i/256))
is applied at positions 0..T-1, then K is cast to BF16.  V ~ N(0, 1) BF16.
Query head j (KV head j // 4) is a uniformly drawn retrieval-zone key
``K_pre[g, t*]`` plus N(0, 0.5**2) noise (0.5 is the standard deviation),
rotated at position T.  Seeds: K 1234, V 1235, Q 1236.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

HEAD_DIM = 256
THETA = 1e6


@dataclass(frozen=True)
class Profile:
    name: str
    context: int
    components: int
    n_centroids: int | None  # None: the index builder's default, ceil(R / 128) * 32
    nprobe: int
    sink: int = 128
    local: int = 256


PROFILES = {
    "cfg0": Profile("cfg0", 8192, 256, 512, 64),
    "cfg1": Profile("cfg1", 32768, 1024, 2048, 384),
    "cfg2": Profile("cfg2", 131072, 4096, 8192, 384),
    "cfg4": Profile("cfg4", 1048576, 32768, 65536, 512),
    # the reference's own 128K profile: config 2's cache indexed by
    # SeoulKV4Index.build(k, v) at its defaults (32672 centroids per head,
    # nprobe 256; reference _index_build.py:16-19, config.py:5)
    "ref128k": Profile("ref128k", 131072, 4096, None, 256),
}


def _rope_tables(positions: torch.Tensor):
    half = HEAD_DIM // 2
    inv = THETA ** (-torch.arange(half, dtype=torch.float64) * 2 / HEAD_DIM)
    angle = positions.to(torch.float64)[:, None] * inv[None, :]
    return torch.cos(angle).float(), torch.sin(angle).float()


def rope(x: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE of fp32 rows ``x`` [N, 256] at ``positions`` [N]."""
    cos, sin = _rope_tables(positions)
    a, b = x[..., : HEAD_DIM // 2], x[..., HEAD_DIM // 2 :]
    return torch.cat((a * cos - b * sin, b * cos + a * sin), dim=-1)


def make_cache(
    context: int,
    components: int,
    *,
    clustered: bool = True,
    sink: int = 128,
    local: int = 256,
    seed_k: int = 1234,
    seed_v: int = 1235,
    seed_q: int = 1236,
    n_queries: int = 1,
):
    """Return ``(k, v, qs)``: BF16 K/V [4, T, 256] and a list of BF16 queries
    [1, 1, 16, 256] (``n_queries`` of them, drawn in sequence)."""
    gk = torch.Generator().manual_seed(seed_k)
    gv = torch.Generator().manual_seed(seed_v)
    gq = torch.Generator().manual_seed(seed_q)
    positions = torch.arange(context)
    k = torch.empty(4, context, HEAD_DIM, dtype=torch.bfloat16)
    pre_heads = []
    for g in range(4):
        if clustered:
            centres = torch.randn(components, HEAD_DIM, generator=gk)
            member = torch.randint(0, components, (context,), generator=gk)
            pre = centres[member] + 0.3 * torch.randn(context, HEAD_DIM, generator=gk)
        else:
            pre = torch.randn(context, HEAD_DIM, generator=gk)
        k[g] = rope(pre, positions).bfloat16()
        pre_heads.append(pre)
    v = torch.randn(4, context, HEAD_DIM, generator=gv).bfloat16()
    queries = []
    for _ in range(n_queries):
        rows = []
        for j in range(16):
            g = j // 4
            t = int(torch.randint(sink, context - local, (1,), generator=gq))
            noisy = pre_heads[g][t] + 0.5 * torch.randn(HEAD_DIM, generator=gq)
            rows.append(rope(noisy[None], torch.tensor([context]))[0])
        queries.append(torch.stack(rows).bfloat16().reshape(1, 1, 16, HEAD_DIM))
    return k, v, queries


def make_profile(name: str, *, clustered: bool = True, n_queries: int = 1):
    p = PROFILES[name]
    k, v, qs = make_cache(
        p.context,
        p.components,
        clustered=clustered,
        sink=p.sink,
        local=p.local,
        n_queries=n_queries,
    )
    return p, k, v, qs
