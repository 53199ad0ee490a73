"""ctypes binding of ``libseoulkv4_hip.so`` — the runtime seam.

Replaces the reference's ``_runtime`` module (``_runtime.py:36-454``):
``initialize`` -> :meth:`Runtime.__init__` (``skv_create``), ``bind_query``
-> :meth:`Runtime.bind_query`, ``enqueue`` -> :meth:`Runtime.enqueue`,
``metadata`` -> :meth:`Runtime.metadata`.  There is no fallback: if the
library is missing or cannot load, every entry point raises.
"""

from __future__ import annotations

import ctypes
import json
from pathlib import Path

import numpy as np
import torch

LIB_PATH = Path(__file__).resolve().with_name("libseoulkv4_hip.so")
HEADER = Path(__file__).resolve().parents[1] / "include" / "seoulkv4_hip.h"

G, H, D, TOPK = 4, 4, 256, 100

STAGES = {
    "lower": 1, "upper": 2, "thresh": 3, "masks": 4, "fine": 5, "selected": 6,
    "pool": 7, "s2": 8, "u1": 9, "s4": 10, "u2": 11, "s8": 12, "top": 13,
    "qprep": 14, "keyrec": 15, "kv8": 16, "kscale": 17,
}
STATUS_FIELDS = ("pool", "err", "selected", "survivors", "u1", "u2", "scanned", "full_select")
ERRORS = {1: "invalid argument", 2: "HIP runtime error", 3: "out of device memory",
          4: "pool above capacity", 5: "pool below minimum", 6: "invalid state",
          7: "pool kernel wait abandoned"}


class CellDesc(ctypes.Structure):
    _fields_ = [
        ("upper", ctypes.c_void_p),
        ("lower", ctypes.c_void_p),
        ("scale", ctypes.c_void_p),
        ("resid_f16", ctypes.c_void_p),
        ("gfs_f16", ctypes.c_void_p),
        ("offsets", ctypes.c_void_p),
        ("values", ctypes.c_void_p),
        ("nprobe", ctypes.c_int32),
        ("lam", ctypes.c_float),
    ]


class IndexDesc(ctypes.Structure):
    _fields_ = [
        ("context", ctypes.c_int32),
        ("sink", ctypes.c_int32),
        ("local", ctypes.c_int32),
        ("n_centroids", ctypes.c_int32),
        ("pool_min", ctypes.c_int32),
        ("pool_capacity", ctypes.c_int32),
        ("debug", ctypes.c_int32),
        ("cells", CellDesc * G),
        ("append_capacity", ctypes.c_int32),
    ]


class KVPagesDesc(ctypes.Structure):
    _fields_ = [
        ("pool", ctypes.c_void_p),
        ("n_pages", ctypes.c_int64),
        ("page_tokens", ctypes.c_int32),
        ("page_table", ctypes.c_void_p),
        ("table_len", ctypes.c_int32),
    ]


TRACE_LIB_PATH = LIB_PATH.with_name("libseoulkv4_hip_trace.so")

_lib = None
_trace_lib = None


def load_library() -> ctypes.CDLL:
    """Load the HIP library (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"SeoulKV4 HIP library missing at {LIB_PATH}; build it with "
            "`python -m seoulkv_amd.build` (gfx950)"
        )
    _lib = _bind(ctypes.CDLL(str(LIB_PATH)))
    return _lib


def load_trace_library() -> ctypes.CDLL | None:
    """The phase-timestamp build of the same sources (``build(trace=True)``),
    for measurements only, or None when it was not built.  A Runtime opened
    with ``lib=`` this library runs the same kernels and records per-block
    device timestamps, read with :meth:`Runtime.trace_blocks`."""
    global _trace_lib
    if _trace_lib is None and TRACE_LIB_PATH.exists():
        lib = _bind(ctypes.CDLL(str(TRACE_LIB_PATH)))
        lib.skv_trace_blocks.restype = ctypes.c_int32
        lib.skv_trace_blocks.argtypes = [ctypes.c_void_p]
        _trace_lib = lib
    return _trace_lib


def _bind(lib: ctypes.CDLL) -> ctypes.CDLL:
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    sig = {
        "skv_create": (i32, [ctypes.POINTER(IndexDesc), vp, vp, i32, vp, ctypes.POINTER(vp)]),
        "skv_create_paged": (i32, [ctypes.POINTER(IndexDesc), vp, vp, ctypes.POINTER(KVPagesDesc),
                                   i32, vp, ctypes.POINTER(vp)]),
        "skv_bind_query": (i32, [vp, vp]),
        "skv_bind_query_device": (i32, [vp, vp, vp]),
        "skv_enqueue": (i32, [vp]),
        "skv_sync": (i32, [vp, vp]),
        "skv_output_device": (i32, [vp, ctypes.POINTER(vp)]),
        "skv_output_tiles_device": (i32, [vp, ctypes.POINTER(vp)]),
        "skv_read_output": (i32, [vp, vp]),
        "skv_debug_ids": (i32, [vp, vp]),
        "skv_read_stage": (i32, [vp, i32, i32, vp, i64, ctypes.POINTER(i64)]),
        "skv_profile": (i32, [vp, i32]),
        "skv_select_mode": (i32, [vp, i32]),
        "skv_graph_mode": (i32, [vp, i32]),
        "skv_time_kernel": (i32, [vp, i32, i32, vp]),
        "skv_append": (i32, [vp, vp, vp, i32]),
        "skv_append_device": (i32, [vp, vp, vp, i32]),
        "skv_dense_decode": (i32, [vp]),
        "skv_dense_decode_static": (i32, [vp, i32, i32, vp, vp, vp]),
        "skv_dense_output_device": (i32, [vp, ctypes.POINTER(vp)]),
        "skv_read_dense_output": (i32, [vp, vp]),
        "skv_time_dense": (i32, [vp, i32, vp]),
        "skv_profile_read": (i32, [vp, vp, i32, vp]),
        "skv_kernel_count": (i32, []),
        "skv_kernel_name": (ctypes.c_char_p, [i32]),
        "skv_metadata": (ctypes.c_char_p, [vp]),
        "skv_destroy": (None, [vp]),
        "skv_last_error": (ctypes.c_char_p, [vp]),
        "skv_version": (ctypes.c_char_p, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def declared_symbols() -> list[str]:
    """Function names declared by ``include/seoulkv4_hip.h``."""
    import re

    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(skv_[a-z_]+)\s*\(", text)))


def dense_decode_static(kv8: torch.Tensor, context: int, q: torch.Tensor,
                        out: torch.Tensor) -> None:
    """Allocation-free dense FP8 decode (``skv_dense_decode_static``) on
    PyTorch's current stream: ``kv8`` uint8 [4, rows, 512] FP8 [V || K]
    records on the device, rows ``0 .. context-1`` attended; ``q`` BF16
    [16, 256] and ``out`` BF16 [16, 256] on the same device.  Raises on a
    rejected size."""
    if kv8.dtype != torch.uint8 or kv8.dim() != 3 or kv8.shape[0] != G or kv8.shape[2] != 512:
        raise ValueError("expected uint8 records [4, rows, 512]")
    for name, t in (("q", q), ("out", out)):
        if t.dtype != torch.bfloat16 or t.numel() != 16 * D or not t.is_contiguous():
            raise ValueError(f"expected a contiguous BF16 {name} with 16 x 256 elements")
    if not (kv8.is_contiguous() and kv8.device == q.device == out.device):
        raise ValueError("records, query and output must be contiguous on one device")
    lib = load_library()
    with torch.cuda.device(kv8.device):
        stream = torch.cuda.current_stream(kv8.device).cuda_stream
        code = lib.skv_dense_decode_static(kv8.data_ptr(), int(kv8.shape[1]), int(context),
                                           q.data_ptr(), out.data_ptr(),
                                           ctypes.c_void_p(stream or None))
    if code != 0:
        msg = lib.skv_last_error(None).decode()
        raise RuntimeError(f"skv_dense_decode_static failed ({ERRORS.get(code, code)}): {msg}")


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _np(t: torch.Tensor, dtype) -> np.ndarray:
    t = t.contiguous().cpu()
    if t.dtype == torch.bfloat16:
        t = t.view(torch.int16)  # numpy has no BF16; keep the raw bits
    return np.ascontiguousarray(t.numpy()).view(dtype)


def index_desc(index, *, pool_min: int, pool_capacity: int | None, debug: bool,
               append_capacity: int = 0):
    """``skv_index_desc`` of an index: this package's :class:`SeoulKV4Index`
    (``cells`` / ``zones``) or the reference's (``_cells`` / ``_zones``,
    reference ``index.py:41-56``; both hold the same cell dictionaries).
    Returns ``(desc, keep)``; the numpy arrays in ``keep`` back the
    descriptor's pointers and must outlive every call that reads it."""
    cells = index.cells if hasattr(index, "cells") else index._cells
    zones = index.zones if hasattr(index, "zones") else index._zones
    keep = []
    desc = IndexDesc()
    desc.context = int(zones.context)
    desc.sink = int(zones.sink)
    desc.local = int(zones.local)
    desc.n_centroids = int(cells[0]["offsets"].numel()) - 1
    desc.pool_min = int(pool_min)
    desc.pool_capacity = int(pool_capacity or 0)
    desc.debug = int(bool(debug))
    desc.append_capacity = int(append_capacity)
    for g, cell in enumerate(cells):
        arrays = dict(
            upper=_np(cell["upper"], np.uint8),
            lower=_np(cell["lower"], np.uint8),
            scale=_np(cell["scale"].float(), np.float32),
            resid_f16=_np(cell["coarse_residual_norm"].half(), np.uint16),
            gfs_f16=_np(cell["group_fine_scale"].half(), np.uint16),
            offsets=_np(cell["offsets"].int(), np.int32),
            values=_np(cell["values"].int(), np.int32),
        )
        keep.append(arrays)
        c = desc.cells[g]
        for name, arr in arrays.items():
            setattr(c, name, _ptr(arr))
        c.nprobe = int(cell["p"])
        c.lam = float(cell["lam"])
    return desc, keep


class Runtime:
    """One device instance of the decode path (the reference's ``state``)."""

    def __init__(self, device: int, k: torch.Tensor, v: torch.Tensor, index, *,
                 pool_min: int, pool_capacity: int | None, debug: bool, stream=None,
                 append_capacity: int = 0, kv_pages=None, lib: ctypes.CDLL | None = None):
        """``kv_pages``: ``(pool, page_table)`` to keep the FP8 records in
        pages of a :class:`seoulkv_amd.paged.KVPagePool` (``skv_create_paged``);
        ``None`` keeps them contiguous in the instance's own memory.  ``lib``:
        another build of the library (the trace build); default the product."""
        self.lib = lib or load_library()
        desc, keep = index_desc(index, pool_min=pool_min, pool_capacity=pool_capacity,
                                debug=debug, append_capacity=append_capacity)
        kb = _np(k, np.uint16)
        vb = _np(v, np.uint16)
        handle = ctypes.c_void_p()
        self._pool = None
        if kv_pages is None:
            code = self.lib.skv_create(
                ctypes.byref(desc), _ptr(kb), _ptr(vb), int(device),
                ctypes.c_void_p(stream or 0), ctypes.byref(handle),
            )
        else:
            pool, table = kv_pages
            if pool.device.index is not None and pool.device.index != int(device):
                raise ValueError(f"page pool is on {pool.device}, the instance on cuda:{device}")
            tab = np.ascontiguousarray(np.asarray(table, dtype=np.int32))
            pd = KVPagesDesc(pool=pool.pages.data_ptr(), n_pages=pool.n_pages,
                             page_tokens=pool.page_tokens, page_table=_ptr(tab),
                             table_len=int(tab.size))
            # the pool's memory was allocated on torch's stream: order the
            # prefill writes after it
            torch.cuda.synchronize(pool.device)
            code = self.lib.skv_create_paged(
                ctypes.byref(desc), _ptr(kb), _ptr(vb), ctypes.byref(pd), int(device),
                ctypes.c_void_p(stream or 0), ctypes.byref(handle),
            )
            self._pool = pool  # the pages must outlive the handle
            self.page_table = tab.tolist()
        if code != 0:
            msg = self.lib.skv_last_error(None).decode()
            raise RuntimeError(f"skv_create failed ({ERRORS.get(code, code)}): {msg}")
        self.handle = handle
        self.stream = int(stream) if stream else None  # the caller's stream (else the library's)
        self.device = int(device)
        self.nc = desc.n_centroids
        self.context = desc.context  # prefill context: key records, pool bound
        self.T = desc.context  # current context (grows with append)
        self.debug = bool(debug)

    # -------------------------------------------------------------- checks
    def _check(self, code: int, what: str) -> None:
        if code != 0:
            msg = self.lib.skv_last_error(self.handle).decode()
            raise RuntimeError(f"{what} failed ({ERRORS.get(code, code)}): {msg}")

    # ------------------------------------------------------------ the seam
    def bind_query(self, q: torch.Tensor) -> None:
        """Host Q [1, 1, 16, 256] BF16 -> device (async H2D, 8 KiB; the call
        copies the query into a pinned staging slot before it returns)."""
        if q.device.type != "cpu" or q.dtype != torch.bfloat16 or q.numel() != 16 * D:
            raise ValueError("expected a CPU BF16 Q with 16 x 256 elements")
        q = q.contiguous()
        self._check(self.lib.skv_bind_query(self.handle, q.data_ptr()), "bind_query")

    def bind_query_device(self, q_dev: torch.Tensor) -> None:
        """Device-resident Q [16, 256] BF16 on this device, written by work on
        PyTorch's current stream: the library copies it on that stream (after
        the writes and after this instance's earlier steps), and its own
        stream waits for the copy.  A temporary (``.contiguous()``) may be
        freed on return: the copy is ordered on its stream."""
        if q_dev.device.type != "cuda" or q_dev.dtype != torch.bfloat16 or q_dev.numel() != 16 * D:
            raise ValueError("expected a device BF16 Q with 16 x 256 elements")
        if q_dev.device.index is not None and q_dev.device.index != self.device:
            raise ValueError(f"Q is on {q_dev.device}, the instance on cuda:{self.device}")
        q_dev = q_dev.contiguous()
        producer = torch.cuda.current_stream(q_dev.device).cuda_stream
        self._check(self.lib.skv_bind_query_device(self.handle, q_dev.data_ptr(),
                                                   ctypes.c_void_p(producer or None)),
                    "bind_query")

    def trace_blocks(self) -> np.ndarray:
        """Trace builds: the per-block device timestamps of the last step,
        uint64 [12 kernel slots][4096 blocks][4 points] in 10 ns ticks."""
        out = np.zeros((12, 4096, 4), dtype=np.uint64)
        self._check(self.lib.skv_trace_blocks(_ptr(out)), "trace_blocks")
        return out

    def time_kernel(self, kernel: int, reps: int = 50) -> float:
        """Mean milliseconds of step kernel ``kernel`` launched ``reps`` times
        back to back (inputs of the last step)."""
        ms = np.zeros(1, dtype=np.float32)
        self._check(self.lib.skv_time_kernel(self.handle, int(kernel), int(reps), _ptr(ms)),
                    "time_kernel")
        return float(ms[0])

    def graph_mode(self, enable: bool) -> None:
        """True: replay the step as one captured HIP graph (one host call per
        step); False (default): launch the step's kernels one by one."""
        self._check(self.lib.skv_graph_mode(self.handle, int(bool(enable))), "graph_mode")

    def select_mode(self, mode: int) -> None:
        """0: sampled cut with full fallback (default); 1: full selection
        only; 2: every sampled cut forced to miss (exercises the fallback)."""
        self._check(self.lib.skv_select_mode(self.handle, int(mode)), "select_mode")

    def enqueue(self) -> None:
        self._check(self.lib.skv_enqueue(self.handle), "enqueue")

    def synchronize(self) -> dict:
        st = np.zeros((G, 8), dtype=np.int32)
        self._check(self.lib.skv_sync(self.handle, _ptr(st)), "synchronize")
        return {f: st[:, i].tolist() for i, f in enumerate(STATUS_FIELDS)}

    def read_output(self) -> torch.Tensor:
        out = np.zeros((16, D), dtype=np.uint16)
        self._check(self.lib.skv_read_output(self.handle, _ptr(out)), "read_output")
        return torch.from_numpy(out.view(np.int16)).view(torch.bfloat16).reshape(1, 1, 16, D)

    def output_device_ptr(self) -> int:
        p = ctypes.c_void_p()
        self._check(self.lib.skv_output_device(self.handle, ctypes.byref(p)), "output")
        return int(p.value)

    def output_tiles_device_ptr(self) -> int:
        """Device [4][1][32][4][256] BF16 output in the reference's layout."""
        p = ctypes.c_void_p()
        self._check(self.lib.skv_output_tiles_device(self.handle, ctypes.byref(p)), "output")
        return int(p.value)

    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """Append n tokens: ``k``, ``v`` [4, n, 256] BF16, CPU (staged copy;
        up to 16 tokens ride with the next query upload and are packed by the
        next step) or on this device (read in place on the instance's stream,
        ordered after PyTorch's current stream).  The local window grows by n."""
        if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16 or k.shape != v.shape \
                or k.dim() != 3 or k.shape[0] != G or k.shape[2] != D:
            raise ValueError("expected BF16 K/V [4, n, 256] of one shape")
        n = int(k.shape[1])
        if k.device.type == "cpu" and v.device.type == "cpu":
            k, v = k.contiguous(), v.contiguous()  # read by the call itself (staged)
            code = self.lib.skv_append(self.handle, k.data_ptr(), v.data_ptr(), n)
        elif k.device == v.device and k.device.type == "cuda" and k.device.index == self.device:
            k, v = k.contiguous(), v.contiguous()
            cur = torch.cuda.current_stream(k.device)
            if self.stream is not None and cur.cuda_stream == self.stream:
                # one stream: the pack follows k/v's producers, and the
                # caching allocator reuses their memory only after it
                code = self.lib.skv_append_device(self.handle, k.data_ptr(), v.data_ptr(), n)
            elif self.stream is not None:
                ext = torch.cuda.ExternalStream(self.stream, device=k.device)
                ext.wait_stream(cur)
                code = self.lib.skv_append_device(self.handle, k.data_ptr(), v.data_ptr(), n)
                if code == 0:  # keep k/v until the instance's stream has read them
                    k.record_stream(ext)
                    v.record_stream(ext)
            else:  # the library's own stream: order by waiting on the host
                torch.cuda.synchronize(self.device)
                code = self.lib.skv_append_device(self.handle, k.data_ptr(), v.data_ptr(), n)
                if code == 0:
                    self._check(self.lib.skv_sync(self.handle, None), "append sync")
        else:
            raise ValueError("K/V must both be CPU tensors or both on the runtime's device")
        self._check(code, "append")
        self.T += n

    def dense_decode(self) -> None:
        """Enqueue the dense FP8 decode of the bound query over all T keys
        (the comparison path; its output is separate from the step's)."""
        self._check(self.lib.skv_dense_decode(self.handle), "dense_decode")

    def read_dense_output(self) -> torch.Tensor:
        out = np.zeros((16, D), dtype=np.uint16)
        self._check(self.lib.skv_read_dense_output(self.handle, _ptr(out)), "read_dense_output")
        return torch.from_numpy(out.view(np.int16)).view(torch.bfloat16).reshape(1, 1, 16, D)

    def time_dense(self, reps: int = 50) -> tuple[float, float, float]:
        """Mean milliseconds per launch of the dense partial kernel, its merge
        kernel and the pair, each over ``reps`` back-to-back launches."""
        ms = np.zeros(3, dtype=np.float32)
        self._check(self.lib.skv_time_dense(self.handle, int(reps), _ptr(ms)), "time_dense")
        return float(ms[0]), float(ms[1]), float(ms[2])

    def debug_ids(self) -> torch.Tensor:
        out = np.zeros((G, H, TOPK), dtype=np.uint32)
        self._check(self.lib.skv_debug_ids(self.handle, _ptr(out)), "debug_ids")
        return torch.from_numpy(out.view(np.int32).astype(np.int64))

    def read_stage(self, name: str, group: int) -> np.ndarray:
        """Copy one stage output of one KV group (for parity checks)."""
        stage = STAGES[name]
        nc, T = self.nc, self.context
        caps = {
            "lower": (H * nc, np.uint16), "upper": (H * nc, np.uint16),
            "thresh": (H, np.uint32), "masks": (nc, np.uint8), "fine": (H * nc, np.uint16),
            "selected": (nc, np.int32), "pool": (T, np.int32), "s2": (H * T, np.uint16),
            "u1": (6400, np.int32), "s4": (H * 6400, np.uint16), "u2": (1024, np.int32),
            "s8": (H * 1024, np.uint16), "top": (H * TOPK, np.int32),
            "qprep": (3 * H * 260, np.int32), "keyrec": (T * 256, np.uint8),
            "kv8": (self.T * 512, np.uint8), "kscale": (D, np.float32),
        }
        cap, dtype = caps[name]
        buf = np.zeros(cap, dtype=dtype)
        count = ctypes.c_int64()
        self._check(
            self.lib.skv_read_stage(self.handle, stage, group, _ptr(buf), cap, ctypes.byref(count)),
            f"read_stage({name})",
        )
        n = count.value
        if name in ("lower", "upper", "fine", "s2", "s4", "s8"):
            return buf[: H * n].reshape(H, n)
        if name == "top":
            return buf[:n].reshape(H, TOPK)
        if name == "qprep":
            return buf.reshape(3, H, 260)
        return buf[:n]

    def metadata(self) -> dict:
        return json.loads(self.lib.skv_metadata(self.handle).decode())

    def profile(self, enable: bool) -> None:
        """(Re)start per-kernel HIP-event timing of every enqueued step."""
        self._check(self.lib.skv_profile(self.handle, int(enable)), "profile")

    def profile_read(self) -> tuple[dict, int]:
        """Mean milliseconds per kernel over the profiled steps."""
        n = self.lib.skv_kernel_count()
        ms = np.zeros(n, dtype=np.float32)
        steps = ctypes.c_int32()
        self._check(self.lib.skv_profile_read(self.handle, _ptr(ms), n, ctypes.byref(steps)),
                    "profile_read")
        names = [self.lib.skv_kernel_name(i).decode() for i in range(n)]
        return dict(zip(names, ms.tolist())), steps.value

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.lib.skv_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
