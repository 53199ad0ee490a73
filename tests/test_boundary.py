"""The drop-in boundary without a GPU: the C-ABI library loads and exports
every function ``include/seoulkv4_hip.h`` declares, ``skv_create`` rejects bad
descriptors before touching a device, and the Python API raises the reference's
error types (``api.py:16-144``, ``result.py:13-23``) on host-side misuse."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from helpers import case
from seoulkv_amd import SeoulKV4, SeoulKV4Config, SeoulKV4Index, _hip

SKV_EINVAL = 1
SKV_ESTATE = 6


@pytest.fixture(scope="module")
def lib():
    return _hip.load_library()


def test_library_exports_every_declared_symbol(lib):
    declared = _hip.declared_symbols()
    assert len(declared) >= 17
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.skv_version().decode().startswith("seoulkv4-hip")
    assert lib.skv_kernel_count() == 7
    names = [lib.skv_kernel_name(i).decode() for i in range(lib.skv_kernel_count())]
    assert names[0] == "front" and names[-1] == "top100_sdpa"
    assert not lib.skv_kernel_name(99)  # out of range: empty name


def _create(lib, desc, k=None, v=None):
    kb = np.zeros(4, dtype=np.uint16) if k is None else k
    vb = np.zeros(4, dtype=np.uint16) if v is None else v
    handle = ctypes.c_void_p()
    code = lib.skv_create(ctypes.byref(desc) if desc is not None else None,
                          kb.ctypes.data, vb.ctypes.data, 0, None, ctypes.byref(handle))
    return code, handle, lib.skv_last_error(None).decode()


def _desc():
    index, k, v, _ = case()
    return _hip.index_desc(index, pool_min=2048, pool_capacity=13056, debug=False)


def _own(desc, keep, g, name):
    """Private copy of one descriptor array (the descriptor arrays share
    memory with the cached index's tensors)."""
    arr = keep[g][name].copy()
    keep[g][name] = arr
    setattr(desc.cells[g], name, arr.ctypes.data)
    return arr


def test_create_rejects_bad_descriptors_on_the_host(lib):
    code, handle, msg = _create(lib, None)
    assert code == SKV_EINVAL and handle.value is None and "NULL" in msg
    for field, value, text in (("context", 0, "context"), ("context", (1 << 20) + 4, "context"),
                               ("n_centroids", 500, "multiple of 32"),
                               ("sink", 8000, "sink/local")):
        desc, keep = _desc()
        setattr(desc, field, value)
        code, handle, msg = _create(lib, desc)
        assert code == SKV_EINVAL and handle.value is None and text in msg, (field, msg)
    desc, keep = _desc()
    desc.cells[2].nprobe = 0
    code, _, msg = _create(lib, desc)
    assert code == SKV_EINVAL and "nprobe" in msg
    desc, keep = _desc()
    desc.cells[1].values = None
    code, _, msg = _create(lib, desc)
    assert code == SKV_EINVAL and "NULL" in msg


def test_create_rejects_spill_violations(lib):
    desc, keep = _desc()
    off, vals = keep[0]["offsets"], _own(desc, keep, 0, "values")
    # a token posted in a third list
    t = int(vals[off[0]])
    vals[off[2]] = t if t not in vals[off[2]:off[3]] else vals[off[2]]
    vals[off[3]] = t
    code, _, msg = _create(lib, desc)
    assert code == SKV_EINVAL and "two memberships" in msg
    desc, keep = _desc()
    off, vals = keep[1]["offsets"], _own(desc, keep, 1, "values")
    vals[off[4] + 1] = vals[off[4]]  # duplicate inside one list
    code, _, msg = _create(lib, desc)
    assert code == SKV_EINVAL and ("duplicate" in msg or "memberships" in msg)
    desc, keep = _desc()
    _own(desc, keep, 3, "values")[7] = desc.context  # token out of range
    code, _, msg = _create(lib, desc)
    assert code == SKV_EINVAL and "token ID" in msg


def test_create_paged_rejects_bad_page_descriptors_on_the_host(lib):
    """``skv_create_paged`` validates the page pool and table before it
    touches a device (no GPU here): alignment, page size, pool size, table
    length, entries in range and distinct."""
    desc, keep = _desc()
    kb = np.zeros(4, dtype=np.uint16)
    need = -(-desc.context // 256)

    def create(pool=1 << 20, n_pages=need, page_tokens=256, table=None, table_len=None):
        tab = np.arange(need, dtype=np.int32) if table is None else np.asarray(table, np.int32)
        pd = _hip.KVPagesDesc(pool=pool, n_pages=n_pages, page_tokens=page_tokens,
                              page_table=tab.ctypes.data,
                              table_len=tab.size if table_len is None else table_len)
        handle = ctypes.c_void_p()
        code = lib.skv_create_paged(ctypes.byref(desc), kb.ctypes.data, kb.ctypes.data,
                                    ctypes.byref(pd), 0, None, ctypes.byref(handle))
        return code, handle.value, lib.skv_last_error(None).decode()

    handle = ctypes.c_void_p()
    assert lib.skv_create_paged(ctypes.byref(desc), kb.ctypes.data, kb.ctypes.data, None, 0,
                                None, ctypes.byref(handle)) == SKV_EINVAL
    for kwargs, text in (
        (dict(pool=0), "NULL"),
        (dict(pool=(1 << 20) + 64), "aligned"),
        (dict(page_tokens=8), "power of two"),
        (dict(page_tokens=384), "power of two"),
        (dict(n_pages=0), "pages"),
        (dict(n_pages=(1 << 21) + 1), "2^31"),
        # products that would wrap a 64-bit record count are refused too
        (dict(n_pages=1 << 58), "2^31"),
        (dict(n_pages=(1 << 63) - 1), "2^31"),
        (dict(table_len=need - 1), "needs %d pages" % need),
        (dict(table=[*range(need - 1), need]), "outside"),
        (dict(table=[*range(need - 1), -1]), "outside"),
        (dict(table=[*range(need - 1), 0]), "twice"),
    ):
        code, h, msg = create(**kwargs)
        assert code == SKV_EINVAL and h is None and text in msg, (kwargs, msg)


def test_handle_entry_points_reject_null(lib):
    # a NULL handle is a closed handle: SKV_ESTATE
    assert lib.skv_enqueue(None) == SKV_ESTATE
    assert lib.skv_sync(None, None) == SKV_ESTATE
    assert lib.skv_bind_query(None, None) == SKV_ESTATE
    assert lib.skv_select_mode(None, 0) == SKV_ESTATE
    lib.skv_destroy(None)  # no-op


# ------------------------------------------------------------------ Python API
def test_api_host_validation():
    index, k, v, qs = case()
    with pytest.raises(ValueError):
        SeoulKV4(device=None, k=k, v=v, index=index)
    with pytest.raises(ValueError):
        SeoulKV4(device="cpu", k=k, v=v, index=index)
    with pytest.raises(TypeError):
        SeoulKV4(device=0, k=k, v=v, index=index, config={"debug": True})
    with pytest.raises(TypeError):
        SeoulKV4(device=0, k=k, v=v, index=object())
    with pytest.raises(ValueError):
        SeoulKV4(device=0, k=k.float(), v=v, index=index)
    with pytest.raises(ValueError):
        SeoulKV4(device=0, k=k, v=v[:, :4096], index=index)
    with pytest.raises(ValueError):
        SeoulKV4(device=0, k=v, v=v, index=index)  # not the indexed cache
    runner = SeoulKV4(device=torch.device("cuda", 0), k=k, v=v, index=index)
    assert not runner.initialized
    with pytest.raises(ValueError):
        runner.run(qs[0].float())
    with pytest.raises(ValueError):
        runner.run(qs[0].reshape(16, 256))
    assert runner.synchronize() is None  # nothing enqueued yet (api.py:104-107)
    with pytest.raises(RuntimeError):
        runner.debug_snapshot()
    assert runner.metadata()["initialized"] is False
    with pytest.raises(RuntimeError):
        runner.append(k[:, :1], v[:, :1])  # append needs an initialised instance
    runner.close()
    runner.close()  # idempotent
    with pytest.raises(RuntimeError):
        runner.run(qs[0])


def test_config_and_index_validation():
    with pytest.raises((TypeError, ValueError)):
        SeoulKV4Config(stage15_capacity=100)
    assert SeoulKV4Config().stage15_capacity == 13056
    assert SeoulKV4Config().append_capacity == 0  # the reference's static cache
    for bad in (-1, 1.5, True, (1 << 20) + 1):
        with pytest.raises(ValueError):
            SeoulKV4Config(append_capacity=bad)
    k, v, _ = __import__("seoulkv_amd.synthetic", fromlist=["make_cache"]).make_cache(8192, 256)
    with pytest.raises(ValueError):
        SeoulKV4Index.build(k[:, :5000], v[:, :5000])  # below the minimum context
    with pytest.raises(ValueError):
        SeoulKV4Index.build(k.float(), v)


def test_static_dense_decode_rejects_sizes_before_any_device_work():
    """``skv_dense_decode_static`` checks its sizes on the host first: a
    context outside [1, 2^20] or fewer rows than keys is SKV_EINVAL with a
    message, before any HIP call (so this runs without a GPU)."""
    import ctypes

    from seoulkv_amd import _hip

    lib = _hip.load_library()
    dummy = ctypes.c_void_p(16)  # never dereferenced: the size checks come first
    for rows, T, what in ((100, 0, "context 0"), (1 << 21, (1 << 20) + 1, "context"),
                          (10, 11, "rows 10 < context 11")):
        code = lib.skv_dense_decode_static(dummy, rows, T, dummy, dummy, None)
        assert code == 1
        assert what in lib.skv_last_error(None).decode()
    assert lib.skv_dense_decode_static(None, 8, 8, dummy, dummy, None) == 1
