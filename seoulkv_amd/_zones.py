"""Disjoint sink / retrieval / local token ranges of one flat cache.

Mirrors ``AttentionZones`` (reference ``_kernels/common/attention_zones.py:7-75``):
the sink is ``[0, sink)``, the local window is ``[context - local, context)`` and
the retrieval range indexed by the IVF lies between them.  Sparse attention for a
query head reads the sink, the local window and that head's top-``retrieval``
tokens from the retrieval range.
"""

from __future__ import annotations

from dataclasses import dataclass

CHUNK_KEYS = 128  # attention gather granularity reported in metadata


@dataclass(frozen=True)
class AttentionZones:
    context: int
    sink: int
    local: int

    def __post_init__(self):
        if self.context <= 0 or min(self.sink, self.local) < 0:
            raise ValueError("require positive context and nonnegative sink/local")
        if self.sink + self.local > self.context:
            raise ValueError("sink and local must be disjoint and inside context")

    @classmethod
    def from_counts(cls, context, sink, local):
        """Clamp requested windows into the context (reference ``:19-23``)."""
        if context <= 0 or min(sink, local) < 0:
            raise ValueError("require positive context and nonnegative sink/local")
        sink = min(sink, context)
        return cls(context, sink, min(local, context - sink))

    @classmethod
    def from_cells(cls, cells, *, context):
        """Recover the zones an index was built with; all cells must agree
        (reference ``from_fixture`` ``:26-48``)."""
        if not cells:
            raise ValueError("attention requires at least one index cell")
        zones = []
        for cell in cells:
            if int(cell["context"]) != context:
                raise ValueError("index attention context mismatch")
            zones.append(cls(context, int(cell["r0"]), context - int(cell["r1"])))
        if any(zone != zones[0] for zone in zones):
            raise ValueError("all index cells must use the same sink/local zones")
        return zones[0]

    @property
    def local_begin(self) -> int:
        return self.context - self.local

    @property
    def dense_count(self) -> int:
        return self.sink + self.local

    def count(self, retrieval: int = 100) -> int:
        if not 0 <= retrieval <= self.local_begin - self.sink:
            raise ValueError("retrieval count exceeds the indexed range")
        return self.dense_count + retrieval

    def metadata(self, retrieval: int = 100) -> dict:
        total = self.count(retrieval)
        return dict(
            context=self.context,
            sink=self.sink,
            local=self.local,
            retrieval_begin=self.sink,
            retrieval_end=self.local_begin,
            retrieval_tokens=retrieval,
            attention_tokens=total,
            chunk_keys=CHUNK_KEYS,
            chunks=(total + CHUNK_KEYS - 1) // CHUNK_KEYS,
        )
