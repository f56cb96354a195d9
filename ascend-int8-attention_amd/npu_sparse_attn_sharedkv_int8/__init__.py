"""INT8 shared-KV (C8) attention and INT8 KV cache writer for MI355X (gfx950).

Drop-in for the reference package of the same name (its __init__.py:1-23):
the same lazily resolved exports, with HIP kernels behind a C ABI
(libsharedkv_hip.so) in place of the AscendC ones.  Importing this module
loads neither torch's GPU runtime nor the native library.
"""
from importlib import import_module

__version__ = "0.1.0+mi355x"
__stage__ = "c8-gfx950"

__all__ = ["CacheQuantization", "SharedKVCase", "PreparedAttention", "PreparedCacheWrite"]

_EXPORTS = {
    "CacheQuantization": ("contract", "CacheQuantization"),
    "SharedKVCase": ("contract", "SharedKVCase"),
    "PreparedAttention": ("attention", "PreparedAttention"),
    "PreparedCacheWrite": ("cache", "PreparedCacheWrite"),
}


def __getattr__(name):
    if name not in _EXPORTS:
        raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
    module, attribute = _EXPORTS[name]
    value = getattr(import_module(f".{module}", __name__), attribute)
    globals()[name] = value
    return value
