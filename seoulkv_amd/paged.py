"""Paged FP8 K/V records: a device pool of pages shared by decode instances.

The reference keeps one contiguous static cache per instance and leaves paged
attention out of its proof of concept (reference ``README.md:66-69``).  A
serving engine instead holds the K/V of many sequences in one pool of
fixed-size pages and gives each sequence a page table.  ``KVPagePool`` is that
pool for this path's FP8 ``[V || K]`` records:

    pages = uint8 [n_pages, 4 KV heads, page_tokens, 512] on one device

Logical page ``p`` of a sequence (tokens ``p * page_tokens ..``) is stored in
physical page ``page_table[p]``; a page holds the records of all 4 KV heads
for its tokens.  ``SeoulKV4(..., kv_pool=pool)`` takes the pages its context
and append capacity need from the pool's free list when it initialises,
writes its prefill and appended records into them, reads every record
through its page table (decode step and dense decode) and returns the pages
on ``close()``.  The index's key codes (its retrieval region, fixed at
prefill) stay in the instance's own memory.  Results are bit-identical to
the contiguous layout.
"""

from __future__ import annotations

from collections import deque

import torch

N_KV_HEADS = 4
RECORD_BYTES = 512  # FP8 V (256 B) || FP8 K (256 B)
MAX_POOL_RECORDS = 1 << 31


class PageFreeList:
    """First-in, first-out free list of page indices 0 .. n_pages-1 (the
    bookkeeping of :class:`KVPagePool`, kept apart from device memory)."""

    def __init__(self, n_pages: int):
        if type(n_pages) is not int or n_pages < 1:
            raise ValueError("n_pages must be a positive int")
        self.n_pages = n_pages
        self._free = deque(range(n_pages))
        self._owned: set[int] = set()

    def __len__(self) -> int:
        return len(self._free)

    def allocate(self, n: int) -> list[int]:
        """Take ``n`` pages from the front of the list (raises when fewer are
        free; nothing is taken then)."""
        if type(n) is not int or n < 0:
            raise ValueError("page count must be a non-negative int")
        if n > len(self._free):
            raise RuntimeError(f"page pool exhausted: {n} pages requested, "
                               f"{len(self._free)} of {self.n_pages} free")
        got = [self._free.popleft() for _ in range(n)]
        self._owned.update(got)
        return got

    def release(self, pages) -> None:
        """Return allocated pages to the end of the list (raises, returning
        none, when one is not allocated or appears twice)."""
        pages = [int(p) for p in pages]
        if len(set(pages)) != len(pages):
            raise ValueError("a page appears twice in the release")
        for p in pages:
            if p not in self._owned:
                raise ValueError(f"page {p} is not allocated from this pool")
        for p in pages:
            self._owned.discard(p)
            self._free.append(p)


class KVPagePool:
    """A device pool of ``n_pages`` pages of ``page_tokens`` tokens (a power
    of two in [16, 65536]) for all 4 KV heads; pages are handed out first in,
    first out from a free list."""

    def __init__(self, n_pages: int, *, page_tokens: int = 256, device="cuda"):
        if type(n_pages) is not int or n_pages < 1:
            raise ValueError("n_pages must be a positive int")
        if type(page_tokens) is not int or not 16 <= page_tokens <= 65536 \
                or page_tokens & (page_tokens - 1):
            raise ValueError("page_tokens must be a power of two in [16, 65536]")
        if n_pages * N_KV_HEADS * page_tokens > MAX_POOL_RECORDS:
            raise ValueError("a pool holds at most 2^31 records (pages x 4 x page_tokens)")
        dev = torch.device(device)
        if dev.type != "cuda":
            raise ValueError("the page pool lives on a ROCm GPU device ('cuda' in PyTorch)")
        self.page_tokens = page_tokens
        self.n_pages = n_pages
        self._list = PageFreeList(n_pages)
        self.pages = torch.empty((n_pages, N_KV_HEADS, page_tokens, RECORD_BYTES),
                                 dtype=torch.uint8, device=dev)
        self.device = self.pages.device

    @property
    def free_pages(self) -> int:
        return len(self._list)

    def pages_for(self, tokens: int) -> int:
        """Pages that hold ``tokens`` tokens."""
        return -(-int(tokens) // self.page_tokens)

    def allocate(self, n: int) -> list[int]:
        """Take ``n`` pages from the free list (raises when fewer are free)."""
        return self._list.allocate(n)

    def release(self, pages) -> None:
        """Return pages to the end of the free list."""
        self._list.release(pages)

    def gather(self, page_table, group: int, tokens: int) -> torch.Tensor:
        """The FP8 records of ``tokens`` tokens of KV head ``group`` of the
        sequence with ``page_table``, in token order: uint8 [tokens, 512]
        (a device copy, for inspection and tests)."""
        n = self.pages_for(tokens)
        idx = torch.as_tensor([int(p) for p in page_table[:n]], dtype=torch.long,
                              device=self.device)
        rows = self.pages.index_select(0, idx)[:, group].reshape(-1, RECORD_BYTES)
        return rows[:tokens]
