"""Borrowed view of the reusable device output.

Mirrors ``DecodeResult`` (reference ``result.py:10-38``): valid until the
owner's next ``run`` or ``close`` (generation check), ``to_torch`` waits and
copies the output to a CPU BF16 [1, 1, 16, 256] tensor.

``device_tensors`` returns one BF16 [1, 32, 4, 256] device tensor per KV
group in the reference's layout (``result.py:25-28``): query head ``4 g + h``
at ``[0, h, h]``, every other row zero.  They alias a library buffer that
each step writes along with the compact output.
"""

from __future__ import annotations

import weakref

import torch


class _DeviceArray:
    """__cuda_array_interface__ wrapper of a raw device pointer."""

    def __init__(self, ptr: int, shape, typestr: str):
        self.__cuda_array_interface__ = {
            "shape": tuple(shape),
            "typestr": typestr,
            "data": (ptr, False),
            "version": 2,
            "strides": None,
        }


class DecodeResult:
    """Output of one ``run``; valid until the next run or close."""

    def __init__(self, owner, generation):
        self._owner_ref = weakref.ref(owner)
        self._generation = generation

    def _owner(self):
        owner = self._owner_ref()
        if owner is None or owner._closed or owner._generation != self._generation:
            raise RuntimeError(
                "SeoulKV4 result is no longer live; read back before the next run or close"
            )
        return owner

    @property
    def device_tensors(self) -> tuple:
        """Per KV group BF16 [1, 32, 4, 256] device views (query head 4g + h
        at [0, h, h]).  Call ``synchronize`` on the owner before reading
        them; do not retain across close."""
        owner = self._owner()
        state = owner._require_initialized()
        ptr = state.output_tiles_device_ptr()
        raw = torch.as_tensor(
            _DeviceArray(ptr, (4, 1, 32, 4, 256), "<i2"), device=f"cuda:{owner._device}"
        ).view(torch.bfloat16)
        return tuple(raw[g] for g in range(4))

    def to_torch(self) -> torch.Tensor:
        """Synchronise and copy into a CPU BF16 [1, 1, 16, 256] tensor."""
        owner = self._owner()
        owner.synchronize()
        return owner._require_initialized().read_output().contiguous()
