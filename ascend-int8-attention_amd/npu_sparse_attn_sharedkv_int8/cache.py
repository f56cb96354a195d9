"""PreparedCacheWrite: fused INT8 quantise + slot scatter into paged caches.

Interface counterpart: npu_sparse_attn_sharedkv_int8/cache.py:16-69 of the
reference checkout (same constructor, validation, _rebind_same_geometry and
run() returning the cache).  The kernel is launch_cache_write in
libsharedkv_hip.so, on the caller's current HIP stream:

  code = clamp(round_half_even(fp32(bf16 update) * inverse_scale[c]), -127, 127)

written to cache[page, offset] where a flat slot s gives page = s // page_size,
offset = s % page_size and a paired slot is (page, offset).  Rows whose slot
is negative or outside the pool are skipped.  Valid slots must be unique in
one call (parallel writes to one row have no defined order).
"""
import ctypes

import torch

from .runtime import CacheWriteArgs, native_launcher

_Args = CacheWriteArgs
ROWS_PER_GROUP = 4   # one wave per update row, four waves per work-group


class PreparedCacheWrite:
    """No host reads, allocations or scale changes happen in run()."""

    def __init__(self, cache, updates, slots, inverse_scale):
        device = cache.device
        if (device.type != "cuda" or cache.dtype != torch.int8 or cache.ndim != 4
                or tuple(cache.shape[-2:]) != (1, 512)):
            raise ValueError("Expected INT8 GPU cache[pages,page_size,1,512]")
        if (not cache.shape[0] or not cache.shape[1] or cache.stride(1) != 512 or cache.stride(-1) != 1
                or cache.stride(0) < cache.shape[1] * 512):
            raise ValueError("Invalid cache strides or empty page storage")
        if (updates.dtype != torch.bfloat16 or updates.ndim not in (2, 3) or updates.shape[-1] != 512
                or (updates.ndim == 3 and updates.shape[1] != 1) or updates.stride(-1) != 1
                or updates.stride(0) < 512):
            raise ValueError("Expected BF16 updates[T,512] or [T,1,512] with contiguous rows")
        if (slots.dtype not in (torch.int32, torch.int64) or slots.ndim not in (1, 2)
                or (slots.ndim == 2 and slots.shape[1] != 2) or slots.shape[0] != updates.shape[0]):
            raise ValueError("Expected INT32/INT64 slots[T] or slots[T,2]")
        if (inverse_scale.dtype != torch.float32 or tuple(inverse_scale.shape) != (512,)
                or not inverse_scale.is_contiguous()):
            raise ValueError("Expected frozen contiguous FP32 inverse_scale[512]")
        if any(t.device != device for t in (updates, slots, inverse_scale)):
            raise ValueError("Cache, updates, slots and scale must be on the same GPU")
        # 16-byte row loads and 8-byte code stores.
        if (updates.stride(0) % 8 or updates.data_ptr() % 16 or cache.stride(0) % 8 or cache.data_ptr() % 8
                or inverse_scale.data_ptr() % 16):
            raise ValueError("Updates rows must be 16-byte aligned and cache pages 8-byte aligned")
        self.cache, self.updates, self.slots, self.inverse_scale = cache, updates, slots, inverse_scale
        self.blocks = (updates.shape[0] + ROWS_PER_GROUP - 1) // ROWS_PER_GROUP
        self.args = _Args(
            cache=cache.data_ptr(), updates=updates.data_ptr(), slots=slots.data_ptr(),
            inverseScale=inverse_scale.data_ptr(), pageStride=cache.stride(0), updateStride=updates.stride(0),
            slotStride=slots.stride(0), slotColumnStride=slots.stride(1) if slots.ndim == 2 else 0,
            tokens=updates.shape[0], pages=cache.shape[0], pageSize=cache.shape[1],
            int64Slots=int(slots.dtype == torch.int64), pairedSlots=int(slots.ndim == 2))
        self.native = native_launcher()
        self.argument_address = ctypes.addressof(self.args)
        self.device_index = device.index if device.index is not None else torch.cuda.current_device()
        if self.native.cache_args_size != ctypes.sizeof(_Args):
            raise RuntimeError("Native host ABI changed; rebuild the library")

    def _rebind_same_geometry(self, cache, updates, slots):
        """Serving fast path; the token count may change, the row layout may not."""
        self.cache, self.updates, self.slots = cache, updates, slots
        self.args.cache, self.args.updates, self.args.slots = cache.data_ptr(), updates.data_ptr(), slots.data_ptr()
        self.args.tokens = updates.shape[0]
        self.blocks = (updates.shape[0] + ROWS_PER_GROUP - 1) // ROWS_PER_GROUP

    def run(self):
        if self.blocks:
            self.native.cache_write(self.argument_address, self.blocks, self.device_index)
        return self.cache
