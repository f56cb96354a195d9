"""Compact page planner: every cache of every layer in one HBM backing, with
one common physical block stride, so a block ID addresses the same place in
all of them and no page is padded to a bucket size.

Interface counterpart: npu_sparse_attn_sharedkv_int8/cache_layout.py:1-206 of
the reference checkout (uses_compact, group_specs, packed_layout,
pool_bytes_per_block, max_memory_usage, cache_config, allocate, reshape).
The planning rules are the reference's:
  * groups: the C4 and C128 groups are kept whole; other (window / state)
    groups are cut into chunks whose page bytes fit the budget
    round_up(max(C4 page, C128 page), largest page); FP32 state specs drop
    their padded page size (cache_layout.py:32-61)
  * offsets: inside each group, layers by descending page size, each at the
    next multiple of its alignment (element size; lcm with the scale
    element size when it has scales; lcm with 512 for INT8 D=512 caches, so
    a row offset is a whole number of 512-byte rows) (cache_layout.py:64-85)
  * stride: the largest group's bytes, rounded up to 512
  * blocks: available memory // stride, unless the engine overrides it
The engine-specific glue (vLLM's spec/group/tensor classes and the runner
hooks) is injected: `types` defaults to vLLM's classes when vLLM is
importable and to the small stand-ins below otherwise, and the allocator
and the views are plain torch (allocate_backing, page_views) instead of
hooks into vllm_ascend's NPU runner.
"""
from dataclasses import dataclass, field, replace
import logging
import math

import torch

ROW_BYTES = 512
BACKING_ALIGNMENT = 2 * 1024 * 1024


def round_up(value, alignment):
    return (value + alignment - 1) // alignment * alignment


def dtype_size(dtype):
    return torch.empty((), dtype=dtype).element_size()


# ----------------------------------------------------------- engine types

@dataclass
class UniformSpecs:
    """Stand-in for vLLM's UniformTypeKVCacheSpecs: specs sharing a block size."""
    kv_cache_specs: dict

    @property
    def page_size_bytes(self):
        return sum(spec.page_size_bytes for spec in self.kv_cache_specs.values())

    @property
    def block_size(self):
        return next(iter(self.kv_cache_specs.values())).block_size

    def max_memory_usage_pages(self, config):
        return max(spec.max_memory_usage_pages(config) for spec in self.kv_cache_specs.values())

    @classmethod
    def from_specs(cls, specs):
        sizes = {getattr(spec, "block_size", None) for spec in specs.values()}
        return cls(dict(specs)) if len(sizes) == 1 else None


@dataclass
class CacheGroup:
    """Stand-in for vLLM's KVCacheGroupSpec."""
    layer_names: list
    kv_cache_spec: UniformSpecs


@dataclass
class CacheTensor:
    """Stand-in for the engine's KV cache tensor descriptor."""
    size: int
    layers: list = field(default_factory=list)
    offset: int = 0
    layer_stride: int = 0
    block_stride: int = 0


@dataclass(frozen=True)
class EngineTypes:
    group: type
    uniform: type
    tensor: type


def default_types():
    try:
        from vllm.v1.kv_cache_interface import KVCacheGroupSpec, KVCacheTensor, UniformTypeKVCacheSpecs
    except ImportError:
        return EngineTypes(CacheGroup, UniformSpecs, CacheTensor)
    return EngineTypes(KVCacheGroupSpec, UniformTypeKVCacheSpecs, KVCacheTensor)


def _specs_of(group_spec):
    specs = getattr(group_spec, "kv_cache_specs", None)
    return specs.values() if specs is not None else (group_spec,)


# --------------------------------------------------------------- planning

def uses_compact(groups):
    """True when some group holds an INT8 D=512 DeepSeek-V4 cache."""
    return any(spec.dtype == torch.int8 and getattr(spec, "head_size", None) == 512
               and getattr(spec, "model_version", None) == "deepseek_v4"
               for group in groups if group is not None and getattr(group, "kv_cache_spec", None) is not None
               for spec in _specs_of(group.kv_cache_spec))


def group_specs(grouped_specs, types=None):
    """Cut the engine's uniform-type spec groups (C4 first, C128 second, then
    window/state groups) into groups whose page bytes fit the common budget."""
    types = types or default_types()
    if len(grouped_specs) < 2:
        raise ValueError("Expected the C4 and C128 groups first")
    largest_page = max(spec.page_size_bytes for group in grouped_specs for spec in group.kv_cache_specs.values())
    budget = round_up(max(grouped_specs[0].page_size_bytes, grouped_specs[1].page_size_bytes), largest_page)
    groups = []

    def close(chunk):
        merged = types.uniform.from_specs(chunk)
        if merged is None:
            raise ValueError("Incompatible cache specifications in a compact group")
        groups.append(types.group(list(chunk), merged))

    for original in grouped_specs:
        chunk, used = {}, 0
        for name, spec in original.kv_cache_specs.items():
            # FP32 compressor states keep their values and shapes; only the
            # padding a bucketed allocator added to their pages is dropped.
            if spec.dtype == torch.float32 and getattr(spec, "page_size_padded", None) is not None:
                spec = replace(spec, page_size_padded=None)
            if chunk and used + spec.page_size_bytes > budget:
                close(chunk)
                chunk, used = {}, 0
            chunk[name] = spec
            used += spec.page_size_bytes
        if chunk:
            close(chunk)
    return groups


def alignment_of(spec):
    alignment = dtype_size(spec.dtype)
    if getattr(spec, "scale_dim", 0):
        alignment = math.lcm(alignment, dtype_size(spec.scale_dtype))
    if spec.dtype == torch.int8 and getattr(spec, "head_size", None) == 512:
        alignment = math.lcm(alignment, ROW_BYTES)
    return alignment


def packed_layout(groups):
    """(common block stride in bytes, {layer name: byte offset in a block})."""
    offsets, maximum = {}, 0
    for group in groups:
        specs = group.kv_cache_spec.kv_cache_specs
        used = 0
        for name in sorted(group.layer_names, key=lambda n: -specs[n].page_size_bytes):
            spec = specs[name]
            if name in offsets:
                raise ValueError(f"Cache layer appears in multiple groups: {name}")
            offset = round_up(used, alignment_of(spec))
            offsets[name] = offset
            used = offset + spec.page_size_bytes
        maximum = max(maximum, used)
    # The attention kernel addresses a row as page * stride + slot * 512, so
    # the stride is a whole number of 512-byte rows (FP32 states stay aligned).
    return round_up(maximum, ROW_BYTES), offsets


def pool_bytes_per_block(groups):
    return packed_layout(groups)[0]


def max_memory_usage(config, groups):
    return pool_bytes_per_block(groups) * sum(group.kv_cache_spec.max_memory_usage_pages(config) for group in groups)


def _check_single_stage(config):
    parallel = config.parallel_config
    if any(getattr(parallel, name, 1) != 1 for name in (
            "pipeline_parallel_size", "decode_context_parallel_size", "prefill_context_parallel_size")):
        raise ValueError("Compact C8 pages are integrated for single-stage, non-context-parallel serving")
    if getattr(config, "kv_transfer_config", None) is not None:
        raise ValueError("KV transfer is not part of this build; compact pages serve local caches only")


def cache_config(config, groups, available_memory, types=None):
    """(number of blocks, one descriptor per layer over one shared backing)."""
    types = types or default_types()
    _check_single_stage(config)
    stride, offsets = packed_layout(groups)
    blocks = available_memory // stride
    override = getattr(getattr(config, "cache_config", None), "num_gpu_blocks_override", None)
    if override is not None:
        blocks = int(override)
    size = blocks * stride
    return blocks, [types.tensor(size=size, layers=[name], offset=offset, layer_stride=0, block_stride=stride)
                    for name, offset in offsets.items()]


def allocate_backing(groups, descriptors, num_blocks, layer_names, device):
    """One INT8 backing for every layer (2 MiB aligned); returns
    {layer: backing[offset:]} after checking that the descriptors are exactly
    the planner's (cache_layout.py:114-134)."""
    stride, offsets = packed_layout(groups)
    size = stride * num_blocks
    actual = {}
    for descriptor in descriptors:
        if (len(descriptor.layers) != 1 or descriptor.layer_stride != 0 or descriptor.block_stride != stride
                or descriptor.size != size):
            raise ValueError("Invalid compact C8 backing descriptor")
        name = descriptor.layers[0]
        if name in actual or descriptor.offset != offsets.get(name):
            raise ValueError("Invalid compact C8 layer offset")
        actual[name] = descriptor.offset
    if set(actual) != set(layer_names):
        raise ValueError("Compact C8 descriptor/spec coverage differs")
    raw = torch.empty(size + BACKING_ALIGNMENT, dtype=torch.int8, device=device)
    start = (-raw.data_ptr()) % BACKING_ALIGNMENT
    backing = raw[start:start + size]
    logging.getLogger(__name__).info("Compact INT8 sharedKV: %d blocks, %d bytes/block, %d groups, one %d-byte backing",
                                     num_blocks, stride, len(groups), size)
    return {name: backing[offset:] for name, offset in actual.items()}


def page_views(raw, shapes, dtypes, stride):
    """Views of one layer's tensors over its slice of the backing: tensor i
    has shape [blocks, ...] and occupies, in every block, the bytes after
    tensor i-1's; block b starts at b * stride.  INT8 [blocks, 32, 1, 512]
    caches come out with strides (stride, 512, 512, 1), the layout the
    attention kernel and the cache writer read."""
    if raw.dtype != torch.int8 or raw.ndim != 1:
        raise ValueError("Expected the flat INT8 backing slice of one layer")
    views, used = [], 0
    for shape, dtype in zip(shapes, dtypes):
        size = dtype_size(dtype)
        inner = math.prod(shape[1:])
        used = round_up(used, size)
        if stride % size or (used + inner * size) > stride:
            raise ValueError("Tensor does not fit the common block stride")
        blocks = shape[0]
        need = (blocks - 1) * stride + used + inner * size if blocks else 0
        if raw.numel() < need:
            raise ValueError("Backing slice too small for the view")
        whole = (raw.numel() - used) // size * size
        typed = raw[used:used + whole].view(dtype)
        strides, running = [], 1
        for extent in reversed(shape[1:]):
            strides.append(running)
            running *= extent
        views.append(typed.as_strided(tuple(shape), (stride // size, *reversed(strides))))
        used += inner * size
    return views
