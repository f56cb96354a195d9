"""Native launcher for libsharedkv_hip.so (reference runtime.py:1-42 and the
pybind host bridges csrc/host/launch.cpp:98-115, c8_launch.cpp:20-43).

The reference launches through a torch_npu pybind module that reads the
caller's current stream and releases the GIL.  Here launches go through
_sharedkv_host, a CPython extension over the C ABI (csrc/host_bridge.cpp) that
releases the GIL around each launch, with torch's current raw HIP stream
passed in; SHAREDKV_USE_CTYPES=1 binds the same C ABI with ctypes instead
(the reference's switch of the same name).  Every launch returns a
hipError_t that is raised as RuntimeError.  There is no host-side fallback:
a missing library or bridge raises at load time.
"""
import ctypes
from functools import lru_cache
import importlib.machinery
import importlib.util
import os
from types import SimpleNamespace

from ._paths import native_path

VARIANT_SPARSE, VARIANT_DENSE, VARIANT_SPARSE_SMALL = 20, 21, 22
VARIANT_DENSE_PAIRED = 23          # grouped plans, 256-key tiles: groups of two (launch_sharedkv_c8_dense_paired)
VARIANT_DENSE_PACKED = 24          # groups of four (launch_sharedkv_c8_dense_packed)
VARIANT_PAIRED_NARROW = 25         # grouped plans, 128-key tiles (launch_sharedkv_c8_dense_paired_narrow)
VARIANT_PACKED_NARROW = 26         # (launch_sharedkv_c8_dense_packed_narrow)
ATTENTION_VARIANT_COUNT = 27


class SharedKVArgs(ctypes.Structure):
    """csrc/kernels/c8/args.h:7-14 (200 bytes); include/sharedkv_hip.h."""
    _fields_ = [(name, ctypes.c_uint64) for name in (
        "q ori cmp oriScale cmpScale oriTable cmpTable indices cuQ seqLens sinks "
        "out workspace lse oriStride cmpStride partial oriIndices").split()] + [
        (name, ctypes.c_uint32) for name in (
            "tokens heads batch oriBlock cmpBlock oriTableWidth cmpTableWidth ratio window topk splits "
            "oriTopk oriPages").split()
    ] + [("softmaxScale", ctypes.c_float)]


class CacheWriteArgs(ctypes.Structure):
    """csrc/kernels/cache_write.h:4-8; include/sharedkv_hip.h."""
    _fields_ = [(name, ctypes.c_uint64) for name in (
        "cache updates slots inverseScale pageStride updateStride slotStride slotColumnStride").split()] + [
        (name, ctypes.c_uint32) for name in "tokens pages pageSize int64Slots pairedSlots".split()]


class SharedKVDebug(ctypes.Structure):
    """Integer dumps for parity tests; include/sharedkv_hip.h."""
    _fields_ = [(name, ctypes.c_uint64) for name in "qcodes alpha scores probs values".split()] + [
        ("cmpCapacity", ctypes.c_uint32), ("tileCapacity", ctypes.c_uint32)]


EXPORTS = ("launch_sharedkv_c8_sparse", "launch_sharedkv_c8_dense", "launch_sharedkv_c8_sparse_small",
           "launch_sharedkv_c8_dense_paired", "launch_sharedkv_c8_dense_packed",
           "launch_sharedkv_c8_dense_paired_narrow", "launch_sharedkv_c8_dense_packed_narrow",
           "launch_sharedkv_c8_noalloc", "sharedkv_c8_attention_debug", "launch_cache_write",
           "sharedkv_c8_workspace_bytes", "sharedkv_c8_partial_bytes", "sharedkv_c8_noalloc_scratch_bytes",
           "sharedkv_c8_noalloc_layout", "sharedkv_c8_set_merge_mode", "sharedkv_c8_set_xcd_local",
           "sharedkv_c8_xcd_local", "sharedkv_attention_args_size", "sharedkv_cache_args_size",
           "sharedkv_abi_version")


@lru_cache(maxsize=1)
def library():
    """Load the C-ABI library and declare every exported signature.

    torch is imported first so that its HIP runtime (libamdhip64.so.7, loaded
    by libtorch_hip) is the one this library binds to: the library's
    dependency is resolved by that SONAME, and a process that loaded the
    system copy first would end up with two HIP runtimes and stream handles
    that do not belong to the runtime launching the kernels.
    """
    import torch  # noqa: F401  (binds the library to torch's HIP runtime)
    lib = ctypes.CDLL(str(native_path()))
    for name in ("launch_sharedkv_c8_sparse", "launch_sharedkv_c8_dense", "launch_sharedkv_c8_sparse_small",
                 "launch_sharedkv_c8_dense_paired", "launch_sharedkv_c8_dense_packed",
                 "launch_sharedkv_c8_dense_paired_narrow", "launch_sharedkv_c8_dense_packed_narrow",
                 "launch_sharedkv_c8_noalloc"):
        fn = getattr(lib, name)
        fn.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p]
        fn.restype = ctypes.c_int
    lib.launch_cache_write.argtypes = [ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p]
    lib.launch_cache_write.restype = ctypes.c_int
    lib.sharedkv_c8_attention_debug.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.sharedkv_c8_attention_debug.restype = ctypes.c_int
    for name in ("sharedkv_c8_workspace_bytes", "sharedkv_c8_partial_bytes"):
        getattr(lib, name).argtypes = [ctypes.c_uint32, ctypes.c_uint32]
        getattr(lib, name).restype = ctypes.c_uint64
    lib.sharedkv_c8_noalloc_scratch_bytes.argtypes = []
    lib.sharedkv_c8_noalloc_scratch_bytes.restype = ctypes.c_uint64
    lib.sharedkv_c8_noalloc_layout.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint64),
                                               ctypes.POINTER(ctypes.c_uint64)]
    lib.sharedkv_c8_noalloc_layout.restype = ctypes.c_int
    lib.sharedkv_c8_set_merge_mode.argtypes = [ctypes.c_int]
    lib.sharedkv_c8_set_merge_mode.restype = ctypes.c_int
    lib.sharedkv_c8_set_xcd_local.argtypes = [ctypes.c_int]
    lib.sharedkv_c8_set_xcd_local.restype = ctypes.c_int
    lib.sharedkv_c8_xcd_local.argtypes = []
    lib.sharedkv_c8_xcd_local.restype = ctypes.c_int
    for name in ("sharedkv_attention_args_size", "sharedkv_cache_args_size", "sharedkv_abi_version"):
        getattr(lib, name).argtypes = []
        getattr(lib, name).restype = ctypes.c_uint32
    if lib.sharedkv_attention_args_size() != ctypes.sizeof(SharedKVArgs):
        raise RuntimeError("Native SharedKVArgs ABI changed; rebuild the library")
    if lib.sharedkv_cache_args_size() != ctypes.sizeof(CacheWriteArgs):
        raise RuntimeError("Native CacheWriteArgs ABI changed; rebuild the library")
    # SHAREDKV_XCD_LOCAL=0 turns the fused merge's XCD-local state exchange
    # off for the process (device-coherent exchange everywhere; same results).
    xcd = os.environ.get("SHAREDKV_XCD_LOCAL", "1")
    if xcd not in ("0", "1"):
        raise ValueError("SHAREDKV_XCD_LOCAL must be 0 or 1")
    if lib.sharedkv_c8_set_xcd_local(int(xcd)) != 0:
        raise RuntimeError("sharedkv_c8_set_xcd_local failed")
    return lib


def _stream(device):
    """Raw handle of torch's current HIP stream on `device` (an index, or
    None for the current device).  torch._C._cuda_getCurrentRawStream skips
    building a Stream object; builds without it use the public call."""
    import torch
    index = torch.cuda.current_device() if device is None else device
    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    return raw(index) if raw is not None else torch.cuda.current_stream(index).cuda_stream


@lru_cache(maxsize=1)
def bridge():
    """The compiled launch bridge (_sharedkv_host), loaded after library() so
    that it binds the same libsharedkv_hip.so."""
    library()
    path = native_path("_sharedkv_host.so")
    loader = importlib.machinery.ExtensionFileLoader("_sharedkv_host", str(path))
    spec = importlib.util.spec_from_file_location("_sharedkv_host", str(path), loader=loader)
    module = importlib.util.module_from_spec(spec)
    loader.exec_module(module)
    return module


def _check(code, what):
    if code:
        raise RuntimeError(f"{what} failed with hipError_t {code}")


class _Host:
    """Counterpart of the reference's pybind host module (launch.cpp:105-115):
    the compiled bridge, or ctypes over the same C ABI."""

    def __init__(self, lib, use_ctypes=False):
        self.lib = lib
        self.attention_args_size = lib.sharedkv_attention_args_size()
        self.cache_args_size = lib.sharedkv_cache_args_size()
        self.attention_variant_count = ATTENTION_VARIANT_COUNT
        self.bridge = None if use_ctypes else bridge()
        self._launchers = {VARIANT_SPARSE: lib.launch_sharedkv_c8_sparse,
                           VARIANT_DENSE: lib.launch_sharedkv_c8_dense,
                           VARIANT_SPARSE_SMALL: lib.launch_sharedkv_c8_sparse_small,
                           VARIANT_DENSE_PAIRED: lib.launch_sharedkv_c8_dense_paired,
                           VARIANT_DENSE_PACKED: lib.launch_sharedkv_c8_dense_packed,
                           VARIANT_PAIRED_NARROW: lib.launch_sharedkv_c8_dense_paired_narrow,
                           VARIANT_PACKED_NARROW: lib.launch_sharedkv_c8_dense_packed_narrow}

    def attention(self, address, blocks, variant, device):
        """Launch on the current stream of `device` (c8_launch.cpp:20-25)."""
        if self.bridge is not None:
            self.bridge.attention(address, blocks, variant, _stream(device))
            return
        fn = self._launchers.get(variant)
        if fn is None:
            raise ValueError("Invalid C8 variant")   # c8_launch.cpp:17
        _check(fn(blocks, _stream(device), address), "sharedkv C8 attention")

    def attention_queued(self, address, blocks, variant, device):
        """The reference copies the argument block by value before enqueueing
        (c8_launch.cpp:27-36).  A HIP launch captures kernel arguments by value
        at launch time, so the direct launch has the same semantics."""
        self.attention(address, blocks, variant, device)

    def cache_write(self, address, blocks, device):
        if self.bridge is not None:
            self.bridge.cache_write(address, blocks, _stream(device))
            return
        _check(self.lib.launch_cache_write(blocks, _stream(device), address), "sharedkv cache write")

    def cache_write_queued(self, address, blocks, device):
        self.cache_write(address, blocks, device)

    def stream_id(self, device):
        """Identity of the current stream (launch.cpp:98-103)."""
        return _stream(device if device is not None and device >= 0 else None)


@lru_cache(maxsize=1)
def native_launcher():
    """reference runtime.py:12-31.  SHAREDKV_USE_CTYPES=1 launches through
    ctypes instead of the compiled bridge; SHAREDKV_HOST_QUEUE=1 selects the
    queued entry points, which equal the direct ones here (a HIP launch
    copies its arguments)."""
    for name in ("SHAREDKV_USE_CTYPES", "SHAREDKV_HOST_QUEUE"):
        if os.environ.get(name, "0") not in ("0", "1"):
            raise ValueError(f"{name} must be 0 or 1")
    host = _Host(library(), use_ctypes=os.environ.get("SHAREDKV_USE_CTYPES") == "1")
    if os.environ.get("SHAREDKV_HOST_QUEUE") == "1":
        return SimpleNamespace(attention=host.attention_queued, cache_write=host.cache_write_queued,
                               attention_args_size=host.attention_args_size,
                               cache_args_size=host.cache_args_size,
                               attention_variant_count=host.attention_variant_count,
                               stream_id=host.stream_id, _owner=host)
    return host


class Kernels:
    """Shared library handle (reference runtime.py:39-42)."""

    def __init__(self):
        self.lib = library()
