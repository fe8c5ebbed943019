"""qengine_amd -- MI355X-native compressed KV cache (TQ3 + Q8_0) for gfx950.

The compute lives in libqkv.so (HIP kernels behind the C ABI of include/qkv.h);
this package is the Python host binding used by tests and benchmarks.
"""
from ._lib import QKVError, lib  # noqa: F401
from . import kvcache  # noqa: F401
