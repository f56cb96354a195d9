"""Serving integration: routes a vLLM-ROCm deployment's D=512 shared-KV cache
writes and sparse attention calls to the HIP kernels with frozen C8 scales.

What is interface (the role of npu_sparse_attn_sharedkv_int8/vllm_adapter.py
in the reference checkout): the keyword contract of the sparse attention call
(ori_kv, cmp_kv, *_block_table, cmp_sparse_indices, cu_seqlens_q, seqused_kv,
sinks, softmax_scale, cmp_ratio, ori_win_left/right, mask modes, TND / PA_ND
layouts, return_softmax_lse; reference vllm_adapter.py:140-160) and its result
(out, lse[T, H, 1]) or (out, empty FP32) (vllm_adapter.py:208-214); the
frozen scale file named by SHAREDKV_SCALES; runtime(impl) and install().

This build's structure:
  SharedKVLayer      one per attention layer: the layer's scales on the
                     device, its cache writers and its attention operators
  OperatorCache      least-recently-used PreparedAttention per launch shape
                     (the non-pointer fields of the C argument block); a hit
                     only rebinds pointers
  StreamScratch      merge scratch per (device, stream), grown to powers of
                     two and never freed, so a captured graph keeps the
                     buffers it was captured with and two streams never
                     share merge tickets
  parse_attention_call   the keyword contract -> SharedKVCase + LSE flag
  install(binding)   hooks the classes an EngineBinding names
The host plan needs no sequence-length bound (the partition count follows the
launch's row count), so eager and captured calls share operators.
"""
from collections import OrderedDict
from dataclasses import dataclass, field, replace
from functools import lru_cache
import logging
import os

import torch

from .attention import PreparedAttention
from .cache import PreparedCacheWrite
from .calibration import load_scale_file
from .contract import SharedKVCase
from .runtime import native_launcher

ARCH = "gfx950"
OPERATORS_PER_LAYER = 8
LOG = logging.getLogger("vllm.sharedkv_c8")


# ------------------------------------------------------------ streams, scratch

def stream_key(device):
    """Identity of `device`'s current HIP stream (usable as a dictionary key)."""
    return native_launcher().stream_id(device.index if device.index is not None else -1)


class StreamScratch:
    """Grow-only named buffers of one (device, stream).  take() returns a view
    of the newest buffer of at least the requested size; older buffers stay
    referenced, because a graph captured with them launches into them."""

    _pools = {}

    def __init__(self, device):
        self.device = device
        self.buffers = {}          # (name, dtype) -> [tensor, ...], newest last

    @classmethod
    def current(cls, device):
        key = (device, stream_key(device))
        pool = cls._pools.get(key)
        if pool is None:
            pool = cls._pools[key] = cls(device)
        return pool

    @classmethod
    def pools(cls):
        return dict(cls._pools)

    def take(self, name, shape, dtype):
        count = 1
        for extent in shape:
            count *= int(extent)
        held = self.buffers.setdefault((name, dtype), [])
        if not held or held[-1].numel() < count:
            capacity = 1
            while capacity < count:
                capacity *= 2
            held.append(torch.empty(capacity, dtype=dtype, device=self.device))
        return held[-1][:count].view(shape)


def scratch_allocator(name, shape, dtype, device):
    """PreparedAttention's scratch_allocator: the current stream's pool."""
    return StreamScratch.current(device).take(name, shape, dtype)


# ------------------------------------------------------------ scales, device

@lru_cache(maxsize=1)
def load_scales():
    """The frozen scale file named by SHAREDKV_SCALES, validated once."""
    path = os.environ.get("SHAREDKV_SCALES")
    if not path:
        raise ValueError("INT8 mode requires SHAREDKV_SCALES containing frozen calibrated scales")
    return load_scale_file(path)


@lru_cache(maxsize=16)
def check_device(device):
    arch = torch.cuda.get_device_properties(device).gcnArchName.split(":")[0]
    if arch != ARCH:
        raise ValueError(f"This adapter is built and verified for MI355X ({ARCH}); found {arch}")
    native_launcher()     # raises if libsharedkv_hip.so is missing


# ------------------------------------------------------------ the call contract

def parse_attention_call(q, kw):
    """(SharedKVCase, return_lse) for one sparse attention call, after the
    contract checks of the reference's adapter (vllm_adapter.py:140-151):
    TND queries over PA_ND pages, the causal band window mask (mode 4, no
    right extent unless explicit original slots are given), causal masking of
    the compressed kind (mode 3)."""
    if kw.get("layout_q") != "TND" or kw.get("layout_kv") != "PA_ND":
        raise ValueError("Expected TND / PA_ND shared-KV layout")
    slots = kw.get("ori_sparse_indices")
    if kw.get("ori_mask_mode", 4) != 4 or (slots is None and kw.get("ori_win_right", 0) != 0):
        raise ValueError("Unsupported original window mask")
    ratio = max(1, int(kw.get("cmp_ratio", 1)))
    if ratio > 1 and kw.get("cmp_mask_mode", 3) != 3:
        raise ValueError("Compressed cache must use causal masking")
    case = SharedKVCase(q=q, ori=kw["ori_kv"], ori_block_table=kw["ori_block_table"], cu_q=kw["cu_seqlens_q"],
                        seq_lens=kw["seqused_kv"], sink=kw["sinks"], cmp=kw.get("cmp_kv"),
                        cmp_block_table=kw.get("cmp_block_table"), cmp_indices=kw.get("cmp_sparse_indices"),
                        ratio=ratio, window=kw["ori_win_left"] + 1, softmax_scale=kw["softmax_scale"],
                        ori_indices=slots)
    return case, bool(kw.get("return_softmax_lse", False))


def launch_shape(case, return_lse):
    """Everything a PreparedAttention bakes into its argument block besides
    device pointers: two calls with equal shapes share one operator, which
    is rebound to the second call's tensors."""
    def pages(cache):
        return None if cache is None else (tuple(cache.shape), cache.stride(0), cache.dtype)

    def extent(t):
        return None if t is None else (tuple(t.shape), t.dtype)

    cmp = case.cmp if case.ratio != 1 else None
    return (case.ratio, case.window, float(case.softmax_scale), extent(case.q), pages(case.ori), pages(cmp),
            extent(case.ori_block_table), extent(case.cmp_block_table if cmp is not None else None),
            extent(case.cmp_indices if case.ratio == 4 else None), extent(case.ori_indices),
            case.seq_lens.numel(), return_lse)


class OperatorCache:
    """At most `capacity` prepared operators, least recently used dropped."""

    def __init__(self, capacity=OPERATORS_PER_LAYER):
        self.capacity = capacity
        self.entries = OrderedDict()

    def get(self, key):
        op = self.entries.get(key)
        if op is not None:
            self.entries.move_to_end(key)
        return op

    def put(self, key, op):
        self.entries[key] = op
        while len(self.entries) > self.capacity:
            self.entries.popitem(last=False)

    def values(self):
        return self.entries.values()


def _rank_zero():
    return not torch.distributed.is_initialized() or torch.distributed.get_rank() == 0


# ------------------------------------------------------------ one layer

@dataclass
class LayerDescription:
    """What the adapter needs to know about an engine's attention layer."""
    prefix: str                      # scale-file key prefix, e.g. "model.layers.0.self_attn"
    head_dim: int = 512
    quantized_elsewhere: bool = False     # the engine already quantizes this cache (e.g. turboquant)
    context_parallel: int = 1             # decode/prefill context-parallel degree


def describe_dsa_impl(impl):
    """LayerDescription of a DeepSeek-V4 sparse attention implementation
    object (the attributes the reference reads, vllm_adapter.py:76-86)."""
    parallel = getattr(getattr(impl, "vllm_config", None), "parallel_config", None)
    cp = max(getattr(parallel, "decode_context_parallel_size", 1) or 1,
             getattr(parallel, "prefill_context_parallel_size", 1) or 1)
    return LayerDescription(prefix=impl.swa_cache_layer.prefix.removesuffix(".swa_cache"),
                            head_dim=impl.head_dim, quantized_elsewhere=getattr(impl, "turboquant", None) is not None,
                            context_parallel=cp)


class SharedKVLayer:
    """Cache writes and sparse attention of one layer on the HIP kernels."""

    def __init__(self, description):
        if description.head_dim != 512 or description.quantized_elsewhere:
            raise ValueError("INT8 shared-KV requires ordinary D=512 DSA")
        if description.context_parallel != 1:
            raise ValueError("Context-parallel cache writers have not been integrated")
        self.prefix = description.prefix
        self.device_scales = {}          # (kind, device) -> (scale, inverse scale)
        self.writers = {}                # writer shape -> PreparedCacheWrite
        self.operators = OperatorCache()
        self.captured = []               # operators launched under graph capture (introspection)
        self.plan = None                 # the engine's attention plan with this layer's attention
        self.reported = set()
        self._empty_lse = {}

    # -- scales
    def scale(self, kind, device):
        """(scale, fp32(1 / fp64(scale))) of this layer's `kind` on `device`."""
        entry = self.device_scales.get((kind, device))
        if entry is None:
            check_device(device)
            key = f"{self.prefix}.{kind}"
            host = load_scales().get(key)
            if host is None:
                raise ValueError(f"Missing real-model calibration for {key}")
            entry = (host.to(device), host.double().reciprocal().float().to(device))
            self.device_scales[(kind, device)] = entry
        return entry

    # -- cache writes
    def write(self, cache, updates, slots, kind):
        """Quantise `updates` with the frozen scale of `kind` ("ori" or "cmp")
        and store them at `slots` of `cache` (PreparedCacheWrite rules)."""
        if updates is None or updates.shape[0] == 0:
            return
        if slots.shape[0] != updates.shape[0]:
            raise ValueError("Cache-write slot/update lengths differ")
        shape = (kind, tuple(cache.shape), cache.stride(), updates.shape[1:], updates.stride(), updates.dtype,
                 slots.shape[1:], slots.stride(), slots.dtype, cache.device, stream_key(cache.device))
        writer = self.writers.get(shape)
        if writer is None:
            writer = self.writers[shape] = PreparedCacheWrite(cache, updates, slots, self.scale(kind, cache.device)[1])
        else:
            writer._rebind_same_geometry(cache, updates, slots)
        writer.run()
        writer.updates = writer.slots = None      # the launch holds the pointers; do not pin the batch
        if kind not in self.reported and _rank_zero():
            LOG.info("INT8 sharedKV cache %s.%s: %s, page stride %d bytes", self.prefix, kind,
                     tuple(cache.shape), cache.stride(0))
        self.reported.add(kind)

    # -- attention
    def attention(self, q, **kw):
        """The sparse attention call (keyword contract above); returns
        (out BF16 [T, H, 512], lse FP32 [T, H, 1]) or (out, empty FP32)."""
        case, return_lse = parse_attention_call(q, kw)
        out = torch.empty_like(q)
        lse = torch.empty(q.shape[:2], dtype=torch.float32, device=q.device) if return_lse else None
        key = (launch_shape(case, return_lse), stream_key(q.device))
        op = self.operators.get(key)
        if op is None:
            op = PreparedAttention(case, self.scale("ori", q.device)[0],
                                   self.scale("cmp", q.device)[0] if case.ratio > 1 else None,
                                   return_lse=return_lse, output=out, lse_output=lse,
                                   scratch_allocator=scratch_allocator)
            self.operators.put(key, op)
            if _rank_zero():
                LOG.info("sharedKV attention %s: ratio %d, %d tokens x %d heads, %d KV partitions", self.prefix,
                         case.ratio, q.shape[0], q.shape[1], op.splits)
        else:
            op._rebind_same_geometry(case, output=out, lse_output=lse)
        if torch.cuda.is_current_stream_capturing() and all(op is not c for c in self.captured):
            self.captured.append(op)
        op.run()
        # The caller owns the outputs (under capture: the graph's pool);
        # the operator keeps only its argument block and scratch.
        op.case = op.out = op.lse = None
        if lse is not None:
            return out, lse.unsqueeze(-1)
        empty = self._empty_lse.get(q.device)
        if empty is None:
            empty = self._empty_lse[q.device] = torch.empty(0, dtype=torch.float32, device=q.device)
        return out, empty


def runtime(impl, describe=describe_dsa_impl):
    """The SharedKVLayer attached to an engine attention object."""
    layer = getattr(impl, "_sharedkv_int8_layer", None)
    if layer is None:
        layer = SharedKVLayer(describe(impl))
        impl._sharedkv_int8_layer = layer
    return layer


# ------------------------------------------------------------ engine hooks

@dataclass
class EngineBinding:
    """The engine classes install() patches, and how.

    impl           attention implementation class.  Its `plan_method()`
                   returns a dataclass whose `plan_field` is the sparse
                   attention callable, and its `write_method(cache, kv,
                   slot_mapping, *, quantize)` writes one cache kind
                   (quantize=True: the compressed cache)
    cache_specs    classes whose `spec_method(config)` returns the BF16 D=512
                   cache spec; it becomes INT8, indexed by block stride
    compact_pages  keep the spec's page bucket (False) or let the compact
                   page planner set a common stride (True)
    describe       impl object -> LayerDescription
    """
    impl: type
    cache_specs: tuple = ()
    plan_method: str = "get_kv_plan"
    plan_field: str = "sparse_attn_op"
    write_method: str = "_write_kv_cache"
    spec_method: str = "get_kv_cache_spec"
    compact_pages: bool = False
    describe: object = field(default=describe_dsa_impl)


def install(binding):
    """Route the binding's classes through SharedKVLayer."""
    load_scales()       # fail before weight loading if the calibration file is absent
    impl_cls, describe = binding.impl, binding.describe
    make_plan = getattr(impl_cls, binding.plan_method)

    def plan(self):
        layer = runtime(self, describe)
        if layer.plan is None:
            layer.plan = replace(make_plan(self), **{binding.plan_field: layer.attention})
        return layer.plan

    def write(self, cache, kv, slot_mapping, *, quantize):
        return runtime(self, describe).write(cache, kv, slot_mapping, "cmp" if quantize else "ori")

    setattr(impl_cls, binding.plan_method, plan)
    setattr(impl_cls, binding.write_method, write)
    for cls in binding.cache_specs:
        setattr(cls, binding.spec_method, _int8_spec(getattr(cls, binding.spec_method), binding.compact_pages))


def _int8_spec(bf16_spec, compact_pages):
    def spec(self, config):
        old = bf16_spec(self, config)
        if old is None:
            return None
        if old.head_size != 512 or old.dtype != torch.bfloat16:
            raise ValueError("INT8 plugin expects the ordinary BF16 D=512 cache specification")
        return replace(old, dtype=torch.int8, indexes_kv_by_block_stride=True,
                       page_size_padded=None if compact_pages else old.page_size_bytes)
    return spec
