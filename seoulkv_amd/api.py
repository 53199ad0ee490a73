"""Public SeoulKV4 lifecycle on an AMD Instinct GPU.

Mirrors ``SeoulKV4`` (reference ``api.py:13-152``): the constructor validates
and retains the CPU K/V, the first ``run(q)`` initialises the device instance
(uploads, prefill kernels, one checked step), later runs bind Q and enqueue
without host synchronisation, ``DecodeResult`` borrows the reusable output.

``device`` is the caller's ROCm device: a ``torch.device("cuda", i)``, the
string ``"cuda:i"`` or the ordinal ``i``.
"""

from __future__ import annotations

import torch

from seoulkv_amd import _hip
from seoulkv_amd.config import MAX_CONTEXT, STAGE15_M, SeoulKV4Config, _KernelOptions
from seoulkv_amd.index import MIN_CONTEXT, SeoulKV4Index
from seoulkv_amd.paged import KVPagePool
from seoulkv_amd.result import DecodeResult


def _device_ordinal(device) -> int:
    if isinstance(device, bool):
        raise ValueError("supply a caller-owned ROCm device")
    if isinstance(device, int):
        return device
    dev = torch.device(device)
    if dev.type != "cuda":
        raise ValueError("SeoulKV4 runs on a ROCm GPU device ('cuda' in PyTorch)")
    return 0 if dev.index is None else dev.index


class SeoulKV4:
    """Static-cache sparse decode.  Call ``run`` with a CPU BF16 post-RoPE query.

    ``kv_pool`` (an extension; the reference cache is contiguous): a
    :class:`~seoulkv_amd.paged.KVPagePool` on the same device.  The instance
    then takes the pages its context and append capacity need from the pool
    when it initialises, keeps its FP8 records there (``page_table``) and
    returns the pages on ``close()``."""

    def __init__(self, *, device, k: torch.Tensor, v: torch.Tensor, index: SeoulKV4Index,
                 config: SeoulKV4Config | None = None, kv_pool: KVPagePool | None = None):
        self._config = SeoulKV4Config() if config is None else config
        if not isinstance(self._config, SeoulKV4Config) or not isinstance(index, SeoulKV4Index):
            raise TypeError("expected SeoulKV4Config and SeoulKV4Index")
        if kv_pool is not None and not isinstance(kv_pool, KVPagePool):
            raise TypeError("kv_pool must be a KVPagePool")
        if device is None:
            raise ValueError("supply a caller-owned ROCm device")
        ordinal = _device_ordinal(device)
        if kv_pool is not None and (kv_pool.device.index or 0) != ordinal:
            raise ValueError(f"kv_pool is on {kv_pool.device}, the instance on cuda:{ordinal}")
        context = index.zones.context
        if not MIN_CONTEXT <= context <= MAX_CONTEXT or context % 4:
            raise ValueError("unsupported context for the fixed SeoulKV4 candidate/tag profile")
        for name, value in (("K", k), ("V", v)):
            if (
                not isinstance(value, torch.Tensor)
                or value.device.type != "cpu"
                or value.dtype != torch.bfloat16
                or tuple(value.shape) != (4, context, 256)
            ):
                raise ValueError(f"expected CPU BF16 {name} [4,{context},256]")
        index._check_keys(k)
        if context + self._config.append_capacity > MAX_CONTEXT:
            raise ValueError("context plus append_capacity exceeds 2^20 tokens")
        self._device = ordinal
        self._kv_pool = kv_pool
        self._pages: list[int] | None = None
        self._index = index
        self._host_kv = (k, v)
        self._args = _KernelOptions(context, self._config.stage15_capacity, self._config.debug)
        self._state: _hip.Runtime | None = None
        self._generation = 0
        self._closed = False
        self._status = None

    @staticmethod
    def _validate_query(q):
        if (
            not isinstance(q, torch.Tensor)
            or q.device.type != "cpu"
            or q.dtype != torch.bfloat16
            or tuple(q.shape) != (1, 1, 16, 256)
        ):
            raise ValueError("expected CPU BF16 Q [1,1,16,256]")

    def _require_open(self):
        if self._closed:
            raise RuntimeError("SeoulKV4 is closed")

    def _require_initialized(self) -> _hip.Runtime:
        self._require_open()
        if self._state is None:
            raise RuntimeError("run(q) must initialize SeoulKV4 first")
        return self._state

    @property
    def initialized(self) -> bool:
        return self._state is not None

    def _initialize(self, q):
        k, v = self._host_kv
        # Steps are enqueued on the caller's current PyTorch stream of the
        # device when it is a created stream; on the legacy default stream
        # the library uses a stream of its own (synchronize() orders both).
        stream = torch.cuda.current_stream(self._device).cuda_stream
        kv_pages = None
        if self._kv_pool is not None:
            pool = self._kv_pool
            self._pages = pool.allocate(
                pool.pages_for(self._index.zones.context + self._config.append_capacity))
            kv_pages = (pool, self._pages)
        try:
            state = _hip.Runtime(
                self._device, k, v, self._index,
                pool_min=self._args.stage15_m,
                pool_capacity=self._args.stage15_capacity,
                debug=self._args.debug,
                stream=stream or None,
                append_capacity=self._config.append_capacity,
                kv_pages=kv_pages,
            )
        except Exception:
            self._release_pages()
            raise
        try:
            # First step is checked like the reference's initialisation
            # handoff (_kernels/stage1_fine/seoulkv4_stage1_live.py:56-81):
            # the live pools must sit in [2048, capacity]; never truncate.
            state.bind_query(q)
            state.enqueue()
            status = state.synchronize()
            pools = status["pool"]
            cap = self._args.stage15_capacity
            if min(pools) < self._args.stage15_m or (cap is not None and max(pools) > cap):
                raise ValueError(
                    f"live Stage-I key counts {pools} outside "
                    f"[{self._args.stage15_m},{cap if cap is not None else 'unbounded'}]; "
                    "change capacity, never truncate"
                )
            # Replay stability (reference verify_initial, seoulkv4_stage1_live.py:200-216).
            first = state.debug_ids()
            state.enqueue()
            state.synchronize()
            if not torch.equal(first, state.debug_ids()):
                raise AssertionError("device selection changed across replay")
        except Exception:
            state.close()
            self._release_pages()
            raise
        return state

    def _release_pages(self):
        if self._pages is not None:
            self._kv_pool.release(self._pages)
            self._pages = None

    @property
    def page_table(self) -> list[int] | None:
        """Physical pool page of each logical page of this cache (paged
        instances after initialisation), else ``None``."""
        return None if self._pages is None else list(self._pages)

    def _bind_query(self, q):
        self._validate_query(q)
        self._require_initialized().bind_query(q)

    def _run_bound(self) -> DecodeResult:
        self._require_initialized().enqueue()
        self._generation += 1
        return DecodeResult(self, self._generation)

    def run(self, q: torch.Tensor) -> DecodeResult:
        """Initialise on the first call, then bind Q and enqueue without readback."""
        self._require_open()
        self._validate_query(q)
        if self._state is None:
            self._state = self._initialize(q)
            self._host_kv = None
        self._bind_query(q)
        return self._run_bound()

    def append(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """Append ``n`` decoded tokens to the cache: ``k``, ``v`` [4, n, 256]
        BF16 post-RoPE keys and values, on the CPU or on this device.  Later
        runs attend them densely with the local window (which grows by n);
        the index, its retrieval region and the key codec stay the prefill's.
        Requires ``SeoulKV4Config(append_capacity=...)`` and an initialised
        instance; raises, the cache unchanged, when the capacity is exceeded."""
        state = self._require_initialized()
        if self._config.append_capacity == 0:
            raise RuntimeError("append requires SeoulKV4Config(append_capacity > 0)")
        state.append(k, v)

    def synchronize(self) -> None:
        """Wait for enqueued work; raise if a step reported a pool error."""
        self._require_open()
        if self._state is None:
            return
        status = self._state.synchronize()
        self._status = status
        bad = [(g, e) for g, e in enumerate(status["err"]) if e]
        if bad:
            g, e = bad[0]
            raise RuntimeError(
                f"SeoulKV4 step failed in KV group {g}: {_hip.ERRORS.get(e, e)} "
                f"(pool sizes {status['pool']})"
            )

    def metadata(self) -> dict:
        """Host-side configuration; never reads device tensors."""
        self._require_open()
        meta = {
            "initialized": self.initialized,
            "cache_layout": "flat" if self._kv_pool is None else "paged",
            "index": self._index.metadata(),
            "implementation": (
                "query prep -> coarse 2-bit interval scan -> P-th lower bound -> survivor "
                "masks -> fine 4-bit top-P union -> spill-2 mate-owned pool -> 2-bit "
                "top-1600 union -> 4-bit top-256 union -> 8-bit top-100 -> sparse FP8 SDPA"
            ),
            "funnel": {
                "stage15_m": self._args.stage15_m,
                "stage15_union_m": self._args.stage15_union_m,
                "stage16_m": self._args.stage16_m,
                "topk": self._args.topk,
                "stage15_capacity": self._args.stage15_capacity,
            },
            "attention_zones": self._index.zones.metadata(),
            "device": f"cuda:{self._device}",
        }
        if self.initialized:
            meta["runtime"] = self._state.metadata()
        return meta

    def debug_snapshot(self) -> dict:
        """Latest final IDs [4, 4, 100] (KV group, query head, rank)."""
        state = self._require_initialized()
        if not self._config.debug:
            raise RuntimeError("debug_snapshot requires SeoulKV4Config(debug=True)")
        self.synchronize()
        return {"selected_ids": state.debug_ids()}

    def close(self) -> None:
        """Wait for pending work and release device buffers; idempotent."""
        if self._closed:
            return
        try:
            if self._state is not None:
                self._state.synchronize()
        finally:
            self._closed = True
            if self._state is not None:
                self._state.close()
            self._release_pages()
            self._state = self._host_kv = self._index = None

    def __enter__(self):
        self._require_open()
        return self

    def __exit__(self, exc_type, exc_value, traceback):
        self.close()
