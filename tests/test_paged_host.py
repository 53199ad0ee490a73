"""Host side of paged K/V records, without a GPU: the page pool's free list
(first in, first out; exhaustion and bad releases leave it unchanged) and the
argument checks of KVPagePool and SeoulKV4(kv_pool=...)."""

from __future__ import annotations

import pytest

from seoulkv_amd import KVPagePool, SeoulKV4, SeoulKV4Config
from seoulkv_amd.paged import PageFreeList
from tests.helpers import case


def test_free_list_is_first_in_first_out():
    fl = PageFreeList(6)
    assert fl.allocate(2) == [0, 1]
    assert fl.allocate(3) == [2, 3, 4]
    fl.release([3, 0])
    assert len(fl) == 3
    assert fl.allocate(3) == [5, 3, 0]  # the free list's order, not the page order
    assert len(fl) == 0
    fl.release([4, 1, 2, 5, 3, 0])
    assert fl.allocate(6) == [4, 1, 2, 5, 3, 0]


def test_free_list_errors_leave_it_unchanged():
    fl = PageFreeList(4)
    a = fl.allocate(3)
    with pytest.raises(RuntimeError, match="exhausted"):
        fl.allocate(2)
    assert len(fl) == 1
    with pytest.raises(ValueError, match="not allocated"):
        fl.release([a[0], 3])  # page 3 was never handed out
    with pytest.raises(ValueError, match="twice"):
        fl.release([a[1], a[1]])
    assert len(fl) == 1
    fl.release(a)
    assert len(fl) == 4
    with pytest.raises(ValueError, match="not allocated"):
        fl.release([a[0]])  # already returned
    for bad in (0, -1, 2.0):
        with pytest.raises(ValueError):
            PageFreeList(bad)
    with pytest.raises(ValueError):
        fl.allocate(-1)


def test_page_pool_argument_checks():
    for kwargs in (dict(page_tokens=8), dict(page_tokens=384), dict(page_tokens=1 << 17)):
        with pytest.raises(ValueError, match="power of two"):
            KVPagePool(4, device="cuda:0", **kwargs)
    with pytest.raises(ValueError, match="2\\^31"):
        KVPagePool((1 << 21) + 1, page_tokens=256, device="cuda:0")
    with pytest.raises(ValueError, match="positive"):
        KVPagePool(0, device="cuda:0")
    with pytest.raises(ValueError, match="ROCm"):
        KVPagePool(4, device="cpu")


def test_seoulkv4_rejects_a_foreign_pool_object():
    index, k, v, _ = case()
    with pytest.raises(TypeError, match="KVPagePool"):
        SeoulKV4(device="cuda:0", k=k, v=v, index=index,
                 config=SeoulKV4Config(stage15_capacity=None), kv_pool=object())
