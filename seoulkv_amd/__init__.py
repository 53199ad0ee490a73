"""SeoulKV4 static-cache sparse decode attention for AMD Instinct MI355X.

Same public names as the reference package ``seoulkv4`` (``__init__.py:3-8``):
``SeoulKV4``, ``SeoulKV4Config``, ``SeoulKV4Index`` and ``DecodeResult``.
The decode step runs as hand-written gfx950 HIP kernels behind the C ABI in
``include/seoulkv4_hip.h``; there is no CPU fallback.
"""

from seoulkv_amd.api import SeoulKV4
from seoulkv_amd.config import SeoulKV4Config
from seoulkv_amd.index import SeoulKV4Index
from seoulkv_amd.paged import KVPagePool
from seoulkv_amd.result import DecodeResult

__all__ = ["DecodeResult", "KVPagePool", "SeoulKV4", "SeoulKV4Config", "SeoulKV4Index"]
