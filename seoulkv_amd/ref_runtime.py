"""Drop-in replacement of the reference's runtime seam, ``seoulkv4._runtime``.

The reference's public classes reach their device only through five names of
``src/seoulkv4/_runtime.py``: ``_ttnn()`` (``:21``), ``initialize(ttnn,
device, k, v, q, index, args)`` (``:36``), ``bind_query(state, q, args)``
(``:180``), ``enqueue(state)`` (``:189``) and ``metadata(state)`` (``:197``),
plus two calls on the object ``_ttnn()`` returns:
``synchronize_device(device)`` (``api.py:104-107``) and ``to_torch(x)`` on
``state["selector"]["outputs"]`` items (``result.py:25-38``) and on
``state["selector"]["debug_indices"]`` (``api.py:119-126``).  This module
provides all of them over ``libseoulkv4_hip.so``, so the reference's own
``SeoulKV4`` / ``DecodeResult`` run unchanged on an MI355X once its
``_runtime`` name points here (the one-line binding is shown in the
integration notes).  ``device`` is then a ROCm device (``torch.device``,
``"cuda:i"`` or an ordinal) instead of a TT-NN MeshDevice.

The state keeps the reference's output contract: four per-KV-head handles whose
``to_torch`` is a BF16 ``[1, 32, 4, 256]`` tensor with query head ``4 g + h``
at row ``[0, h, h]`` (the Tenstorrent tile-padded layout the reference's
``DecodeResult.to_torch`` takes the diagonal of), and a debug handle whose
``to_torch`` is the ``[4, 4, 100]`` final IDs.
"""

from __future__ import annotations

import torch

from seoulkv_amd import _hip

_N_KV, _GROUP, _D, _TOPK = 4, 4, 256, 100


def _ordinal(device) -> int:
    if isinstance(device, bool) or device is None:
        raise ValueError("supply a caller-owned ROCm device")
    if isinstance(device, int):
        return device
    dev = torch.device(device)
    if dev.type != "cuda":
        raise ValueError("this runtime drives a ROCm GPU ('cuda' in PyTorch)")
    return 0 if dev.index is None else dev.index


class GroupOutput:
    """One KV head's output handle (the reference's native slot tensor)."""

    def __init__(self, runtime: _hip.Runtime, slot: int):
        self._runtime = runtime
        self.slot = slot
        self.shape = (1, 32, _GROUP, _D)

    def to_torch(self) -> torch.Tensor:
        """CPU BF16 [1, 32, 4, 256]: head h of this KV head at [0, h, h]."""
        self._runtime.synchronize()
        return self.device_view().cpu()

    def device_view(self) -> torch.Tensor:
        """Device BF16 [1, 32, 4, 256] view of this KV head's tile of the
        library's padded output buffer (valid until the next enqueue)."""
        from seoulkv_amd.result import _DeviceArray

        raw = torch.as_tensor(
            _DeviceArray(self._runtime.output_tiles_device_ptr(), (4,) + self.shape, "<i2"),
            device=f"cuda:{self._runtime.device}",
        ).view(torch.bfloat16)
        return raw[self.slot]


class DebugIndices:
    """The debug-ID handle (reference ``state["selector"]["debug_indices"]``)."""

    def __init__(self, runtime: _hip.Runtime):
        self._runtime = runtime

    def to_torch(self) -> torch.Tensor:
        """[4, 4, 100] int64 final token IDs (KV head, query head, rank)."""
        return self._runtime.debug_ids()


class _Device:
    """The two TT-NN calls the reference's public classes make."""

    @staticmethod
    def synchronize_device(device) -> None:
        torch.cuda.synchronize(_ordinal(device))

    @staticmethod
    def to_torch(handle) -> torch.Tensor:
        return handle.to_torch()


def _ttnn():
    """The device module handed to ``initialize`` (reference ``_runtime.py:21-28``)."""
    if not torch.cuda.is_available():
        raise RuntimeError("SeoulKV4 requires a ROCm GPU (gfx950)")
    return _Device()


def initialize(ttnn, device, k, v, q, index, args):
    """Build the device instance and run the checked first step
    (reference ``_runtime.py:36-177``).  ``index`` is the reference's
    ``SeoulKV4Index`` (or this package's); ``args`` its ``_KernelOptions``
    (``skv4_stage15_m``, ``skv4_stage15_candidates``, ``skv4_debug_indices``).
    Raises ``ValueError(... never truncate)`` when a live pool falls outside
    [skv4_stage15_m, skv4_stage15_candidates], like the reference's Stage-I
    handoff (``_kernels/stage1_fine/seoulkv4_stage1_live.py:56-81``)."""
    ordinal = _ordinal(device)
    pool_min = int(args.skv4_stage15_m)
    capacity = getattr(args, "skv4_stage15_candidates", None)
    runtime = _hip.Runtime(
        ordinal, k, v, index,
        pool_min=pool_min,
        pool_capacity=capacity,
        debug=bool(args.skv4_debug_indices),
        stream=torch.cuda.current_stream(ordinal).cuda_stream or None,
    )
    try:
        runtime.bind_query(q.reshape(1, 1, 16, _D))
        runtime.enqueue()
        pools = runtime.synchronize()["pool"]
        if min(pools) < pool_min or (capacity is not None and max(pools) > capacity):
            raise ValueError(
                f"live Stage-I key counts {pools} outside "
                f"[{pool_min},{capacity if capacity is not None else 'unbounded'}]; "
                "change capacity, never truncate"
            )
        # replay stability (reference verify_initial, seoulkv4_stage1_live.py:200-216)
        first = runtime.debug_ids()
        runtime.enqueue()
        runtime.synchronize()
        if not torch.equal(first, runtime.debug_ids()):
            raise AssertionError("device selection changed across replay")
    except Exception:
        runtime.close()
        raise
    return {
        "ttnn": ttnn,
        "runtime": runtime,
        "device": device,
        "n_conc": 1,
        "n_kv_heads": _N_KV,
        "group": _GROUP,
        "slots": _N_KV,
        "head_dim": _D,
        "context": int(k.shape[1]),
        "topk": _TOPK,
        "selector": {
            "outputs": [GroupOutput(runtime, g) for g in range(_N_KV)],
            "debug_indices": DebugIndices(runtime),
        },
    }


def bind_query(state, q, args):
    """Reference ``_runtime.py:180-186``: shape check, then the 8 KiB upload."""
    expected = (state["n_conc"], 1, args.n_heads, state["head_dim"])
    if tuple(q.shape) != expected:
        raise ValueError(f"unexpected SeoulKV4 query shape {tuple(q.shape)}, expected {expected}")
    state["runtime"].bind_query(q)


def enqueue(state):
    """Reference ``_runtime.py:189-194``: launch one decode step, no readback."""
    state["runtime"].enqueue()


def metadata(state):
    """Reference ``_runtime.py:197``: host-side description, no device reads."""
    meta = dict(state["runtime"].metadata())
    meta["implementation"] = (
        "MI355X HIP: coarse 2-bit scan -> fine top-P union -> spill-2 pool -> "
        "2/4/8-bit progressive top-k -> sparse FP8 SDPA"
    )
    meta["programs"] = [_hip.load_library().skv_kernel_name(i).decode()
                        for i in range(_hip.load_library().skv_kernel_count())]
    return meta
