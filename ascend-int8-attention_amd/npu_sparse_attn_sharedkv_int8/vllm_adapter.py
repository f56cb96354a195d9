"""Serving integration: one LayerRuntime per attention layer of a vLLM-ROCm
deployment, routing its cache writes and sparse attention calls to the HIP
kernels with frozen C8 scales.

Interface counterpart: npu_sparse_attn_sharedkv_int8/vllm_adapter.py:1-277 of
the reference checkout.  Kept: stream_key, geometry, scratch_allocator,
load_scales, check_device, LayerRuntime (scale / write / attention with the
same keyword contract and the same (out, lse[T,H,1] | empty FP32) result),
runtime(impl) and install().  The device check is for MI355X (gfx950)
instead of Ascend910_9382, graph capture is torch.cuda's, and install()
patches the attention classes it is given (vLLM-ROCm's DeepSeek-V4 sparse
attention classes are passed in by the plugin; see vllm_plugin.py) instead of
importing vllm_ascend.

Cached state per layer, as in the reference:
  writers        PreparedCacheWrite per (kind, cache geometry, update/slot
                 geometry, stream); rebound to new tensors on every call
  attention_ops  PreparedAttention per (case geometry, length bound, LSE,
                 adaptive, stream); least recently used of more than 8 dropped
  scratch        workspace / partial buffers per (device, stream, name,
                 dtype), grown by powers of two and never freed (a captured
                 graph keeps using the buffers it was captured with)
"""
from collections import OrderedDict
from dataclasses import replace
from functools import lru_cache
import logging
import math
import os

import torch

from .attention import PreparedAttention
from .c8_attention import enabled as c8_enabled
from .cache import PreparedCacheWrite
from .calibration import load_scale_file
from .contract import SharedKVCase
from .runtime import native_launcher

ARCH = "gfx950"
MAX_CACHED_OPS = 8

_scratch = {}
_reported_c8_routes = set()


def stream_key(device):
    """Identity of the device's current HIP stream (a dictionary key)."""
    return native_launcher().stream_id(device.index if device.index is not None else -1)


def geometry(tensor):
    if tensor is None:
        return None
    return tensor.shape, tensor.stride(), tensor.dtype, tensor.device


def scratch_allocator(name, shape, dtype, device):
    """Scratch shared by the layers that run one after another on a stream;
    another stream gets its own.  Capacity grows to the next power of two and
    older buffers are retained for graphs captured with them."""
    key = device, stream_key(device), name, dtype
    buffers = _scratch.setdefault(key, [])
    count = math.prod(shape)
    if not buffers or buffers[-1].numel() < count:
        buffers.append(torch.empty(1 << max(0, count - 1).bit_length(), dtype=dtype, device=device))
    return buffers[-1][:count].view(shape)


@lru_cache(maxsize=1)
def load_scales():
    """The frozen scale file named by SHAREDKV_SCALES, validated once."""
    path = os.environ.get("SHAREDKV_SCALES")
    if not path:
        raise ValueError("INT8 mode requires SHAREDKV_SCALES containing frozen calibrated scales")
    return load_scale_file(path)


@lru_cache(maxsize=16)
def check_device(device):
    name = torch.cuda.get_device_properties(device).gcnArchName.split(":")[0]
    if name != ARCH:
        raise ValueError(f"This adapter is built and verified for MI355X ({ARCH}); found {name}")
    if native_launcher() is None:
        raise RuntimeError("Build libsharedkv_hip.so before serving")


class LayerRuntime:
    """Cache writes and attention of one layer (`impl` is the engine's
    attention implementation object: swa_cache_layer.prefix, head_dim,
    turboquant, vllm_config.parallel_config)."""

    def __init__(self, impl):
        self.impl = impl
        self.prefix = impl.swa_cache_layer.prefix.removesuffix(".swa_cache")
        if impl.head_dim != 512 or getattr(impl, "turboquant", None) is not None:
            raise ValueError("INT8 shared-KV requires ordinary D=512 DSA")
        parallel = impl.vllm_config.parallel_config
        if (getattr(parallel, "decode_context_parallel_size", 1) != 1
                or getattr(parallel, "prefill_context_parallel_size", 1) != 1):
            raise ValueError("Context-parallel cache writers have not been integrated")
        self.scales = {}
        self.writers = {}
        self.attention_ops = OrderedDict()
        self.captured_ops = []
        self.captured_ids = set()
        self.empty_lse = None
        self.plan = None
        self.reported_caches = set()
        self.adaptive_graph_splits = os.environ.get("SHAREDKV_ADAPTIVE_KV_SPLITS") == "1"
        self.clean_c8_decode = c8_enabled()

    def scale(self, kind, device):
        """(scale, fp32(1 / fp64(scale))) of this layer's `kind` on `device`."""
        if kind not in self.scales:
            check_device(device)
            key = f"{self.prefix}.{kind}"
            cpu = load_scales().get(key)
            if cpu is None:
                raise ValueError(f"Missing real-model calibration for {key}")
            self.scales[kind] = (cpu.to(device), cpu.double().reciprocal().float().to(device))
        return self.scales[kind]

    def write(self, cache, updates, slots, kind):
        if updates is None or updates.shape[0] == 0:
            return
        if slots.shape[0] != updates.shape[0]:
            raise ValueError("Cache-write slot/update lengths differ")
        key = (kind, geometry(cache), updates.shape[1:], updates.stride(), updates.dtype,
               slots.shape[1:], slots.stride(), slots.dtype, updates.device, slots.device,
               stream_key(cache.device))
        writer = self.writers.get(key)
        if writer is None:
            writer = PreparedCacheWrite(cache, updates, slots, self.scale(kind, cache.device)[1])
            self.writers[key] = writer
        else:
            writer._rebind_same_geometry(cache, updates, slots)
        writer.run()
        if kind not in self.reported_caches:
            if not torch.distributed.is_initialized() or torch.distributed.get_rank() == 0:
                logging.getLogger("vllm.sharedkv_c8").info(
                    "INT8 sharedKV cache %s.%s: shape=%s dtype=%s page_stride=%d bytes",
                    self.prefix, kind, tuple(cache.shape), cache.dtype, cache.stride(0))
            self.reported_caches.add(kind)
        # The launch has captured the pointers; holding the activations would
        # keep every layer's last update batch resident.
        writer.updates = writer.slots = None

    def attention(self, q, **kw):
        if kw.get("layout_q") != "TND" or kw.get("layout_kv") != "PA_ND":
            raise ValueError("Expected TND / PA_ND shared-KV layout")
        original_indices = kw.get("ori_sparse_indices")
        if kw.get("ori_mask_mode", 4) != 4 or (kw.get("ori_win_right", 0) != 0 and original_indices is None):
            raise ValueError("Unsupported original window mask")
        ratio = max(1, kw.get("cmp_ratio", 1))
        if ratio > 1 and kw.get("cmp_mask_mode", 3) != 3:
            raise ValueError("Compressed cache must use causal masking")
        case = SharedKVCase(q=q, ori=kw["ori_kv"], ori_block_table=kw["ori_block_table"],
                            cu_q=kw["cu_seqlens_q"], seq_lens=kw["seqused_kv"], sink=kw["sinks"],
                            cmp=kw.get("cmp_kv"), cmp_block_table=kw.get("cmp_block_table"),
                            cmp_indices=kw.get("cmp_sparse_indices"), ratio=ratio,
                            window=kw["ori_win_left"] + 1, softmax_scale=kw["softmax_scale"],
                            ori_indices=original_indices)
        capturing = torch.cuda.is_current_stream_capturing()
        # An eager launch may use the batch's known length bound; a captured
        # one is replayed while lengths grow, so it plans for any length.
        bound = None if capturing else getattr(kw.get("metadata"), "_sharedkv_max_seq_len", None)
        if bound is not None and 0 < bound <= 1024:
            bound = 1024
        elif bound is not None and ratio == 128 and bound > 32768:
            bound = 1 << (int(bound) - 1).bit_length()    # bucketed: no new plan per decode step
        else:
            bound = None
        adaptive = (self.adaptive_graph_splits and capturing and ratio == 4 and original_indices is None
                    and q.shape[1] <= 8 and 24 <= q.shape[0] <= 48 and case.cmp_indices.shape[-1] <= 1024)
        return_lse = kw.get("return_softmax_lse", False)
        output = torch.empty_like(q)
        lse = torch.empty(q.shape[:2], dtype=torch.float32, device=q.device) if return_lse else None
        key = (tuple(geometry(t) if isinstance(t, torch.Tensor) else t for t in vars(case).values()),
               bound, return_lse, adaptive, stream_key(q.device))
        op = self.attention_ops.get(key)
        if op is None:
            op = PreparedAttention(case, self.scale("ori", q.device)[0],
                                   self.scale("cmp", q.device)[0] if ratio > 1 else None,
                                   max_seq_len=bound, return_lse=return_lse, output=output, lse_output=lse,
                                   adaptive_splits=adaptive, scratch_allocator=scratch_allocator)
            if self.clean_c8_decode:
                route = (getattr(op, "c8_dynamic", False), ratio, q.shape[0], getattr(op, "variant", -1))
                if route not in _reported_c8_routes:
                    rank = torch.distributed.get_rank() if torch.distributed.is_initialized() else 0
                    if rank % 16 == 0:
                        logging.getLogger("vllm.sharedkv_c8").info(
                            "C8 route rank=%d c8=%s ratio=%d capacity=%d variant=%s splits=%d",
                            rank, *route, op.splits)
                    _reported_c8_routes.add(route)
            self.attention_ops[key] = op
            if len(self.attention_ops) > MAX_CACHED_OPS:
                self.attention_ops.popitem(last=False)
        else:
            self.attention_ops.move_to_end(key)
            op._rebind_same_geometry(case, output=output, lse_output=lse)
        if capturing and id(op) not in self.captured_ids:
            self.captured_ids.add(id(op))
            self.captured_ops.append(op)
        result = op.run()
        # Outputs allocated during capture belong to the graph's pool like any
        # operator output; the op keeps only geometry and scratch.
        op.case = op.out = op.lse = None
        if lse is not None:
            return result, lse.unsqueeze(-1)
        if self.empty_lse is None:
            self.empty_lse = torch.empty(0, dtype=torch.float32, device=q.device)
        return result, self.empty_lse


def runtime(impl):
    obj = getattr(impl, "_sharedkv_int8_runtime", None)
    if obj is None:
        obj = LayerRuntime(impl)
        impl._sharedkv_int8_runtime = obj
    return obj


def install(impl_cls, cache_spec_classes=(), metadata_builder_cls=None, metadata_method="_build_sas_metadata",
            compact_pages=None):
    """Route an engine's attention classes through LayerRuntime (reference
    vllm_adapter.py:225-277).

    impl_cls              attention implementation: get_kv_plan() returns a
                          dataclass with a `sparse_attn_op` field, and
                          _write_kv_cache(cache, kv, slot_mapping, *, quantize)
                          writes one cache kind
    cache_spec_classes    classes whose get_kv_cache_spec(config) returns the
                          BF16 D=512 cache spec; it becomes INT8
    metadata_builder_cls  builder whose `metadata_method` receives the batch's
                          max_seqlen_kv (6th positional or keyword); its result
                          carries it as _sharedkv_max_seq_len
    """
    load_scales()  # fail before weight loading if the calibration file is absent
    if compact_pages is None:
        compact_pages = os.environ.get("SHAREDKV_COMPACT_PAGES") == "1"
    original_plan = impl_cls.get_kv_plan

    def get_plan(self):
        state = runtime(self)
        if state.plan is None:
            state.plan = replace(original_plan(self), sparse_attn_op=state.attention)
        return state.plan

    def write(self, cache, kv, slot_mapping, *, quantize):
        return runtime(self).write(cache, kv, slot_mapping, "cmp" if quantize else "ori")

    impl_cls.get_kv_plan = get_plan
    impl_cls._write_kv_cache = write

    for cls in cache_spec_classes:
        original_spec = cls.get_kv_cache_spec

        def spec(self, config, _original=original_spec):
            old = _original(self, config)
            if old is None:
                return None
            if old.head_size != 512 or old.dtype != torch.bfloat16:
                raise ValueError("INT8 plugin expects the ordinary BF16 D=512 cache specification")
            # Compact pages get an explicit common stride from the planner;
            # otherwise the BF16 pool's page buckets are kept.
            return replace(old, dtype=torch.int8, page_size_padded=None if compact_pages else old.page_size_bytes,
                           indexes_kv_by_block_stride=True)

        cls.get_kv_cache_spec = spec

    if metadata_builder_cls is not None:
        original_metadata = getattr(metadata_builder_cls, metadata_method)

        def metadata(self, *args, **kwargs):
            result = original_metadata(self, *args, **kwargs)
            bound = kwargs.get("max_seqlen_kv", args[5] if len(args) > 5 else None)
            result._sharedkv_max_seq_len = int(bound) if isinstance(bound, int) else None
            return result

        setattr(metadata_builder_cls, metadata_method, metadata)
