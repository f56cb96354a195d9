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

Attribution: the rules above are an allocation format, kept identical so
that a block ID and a layer offset mean the same thing to both builds.  The
reference took the common-stride scheme from vllm-ascend's TurboQuant
planner (vllm_ascend/quantization/methods/kv_cache/turboquant/cache.py,
SPDX-License-Identifier: Apache-2.0, Copyright contributors to the vLLM
project); this module restates the format in its own code and messages.
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

def _is_c8_cache(spec):
    """An INT8 D=512 DeepSeek-V4 attention cache: the kind this path reads."""
    return (spec.dtype == torch.int8 and getattr(spec, "head_size", None) == 512
            and getattr(spec, "model_version", None) == "deepseek_v4")


def _leaf_specs(groups):
    """Every per-layer spec of the engine's groups (skipping empty slots)."""
    for group in groups:
        spec = None if group is None else getattr(group, "kv_cache_spec", None)
        if spec is not None:
            yield from _specs_of(spec)


def uses_compact(groups):
    """True when some group holds an INT8 D=512 DeepSeek-V4 cache."""
    return any(map(_is_c8_cache, _leaf_specs(groups)))


def _without_bucket_padding(spec):
    """FP32 compressor states keep their values and shapes; the padding that a
    bucketed allocator added to their page size is dropped."""
    if spec.dtype == torch.float32 and getattr(spec, "page_size_padded", None) is not None:
        return replace(spec, page_size_padded=None)
    return spec


def _runs_within(items, budget):
    """Consecutive runs of (name, spec) whose page bytes sum to at most
    `budget`; a run always takes at least one item."""
    run, total = [], 0
    for name, spec in items:
        size = spec.page_size_bytes
        if run and total + size > budget:
            yield run
            run, total = [], 0
        run.append((name, spec))
        total += size
    if run:
        yield run


def group_specs(grouped_specs, types=None):
    """Cut the engine's uniform-type spec groups (C4 first, C128 second, then
    window/state groups) into groups whose page bytes fit the common budget.
    The budget is the larger of the C4 and C128 group pages rounded up to the
    largest single page, so those two groups are never cut."""
    types = types or default_types()
    if len(grouped_specs) < 2:
        raise ValueError("Expected the C4 and C128 groups first")
    largest = max(spec.page_size_bytes for source in grouped_specs for spec in source.kv_cache_specs.values())
    budget = round_up(max(source.page_size_bytes for source in grouped_specs[:2]), largest)
    planned = []
    for source in grouped_specs:
        items = [(name, _without_bucket_padding(spec)) for name, spec in source.kv_cache_specs.items()]
        for run in _runs_within(items, budget):
            members = dict(run)
            merged = types.uniform.from_specs(members)
            if merged is None:
                raise ValueError("Specs cut into one compact group must share one block size")
            planned.append(types.group(list(members), merged))
    return planned


def alignment_of(spec):
    """Byte alignment of a layer inside a block: its element size, joined
    (lcm) with the scale element size when it carries scales, and with the
    512-byte row for INT8 D=512 caches (the kernels address a row as
    page * stride + slot * 512)."""
    parts = [dtype_size(spec.dtype)]
    if getattr(spec, "scale_dim", 0):
        parts.append(dtype_size(spec.scale_dtype))
    if spec.dtype == torch.int8 and getattr(spec, "head_size", None) == 512:
        parts.append(ROW_BYTES)
    return math.lcm(*parts)


def _place_group(group):
    """({layer: offset inside a block}, bytes the group uses): layers in
    descending page size (ties keep the group's order), each at the next
    multiple of its alignment."""
    specs = group.kv_cache_spec.kv_cache_specs
    placed, cursor = {}, 0
    for name in sorted(group.layer_names, key=lambda n: specs[n].page_size_bytes, reverse=True):
        if name in placed:
            raise ValueError(f"Layer {name!r} is listed twice in one compact group")
        placed[name] = round_up(cursor, alignment_of(specs[name]))
        cursor = placed[name] + specs[name].page_size_bytes
    return placed, cursor


def packed_layout(groups):
    """(common block stride in bytes, {layer name: byte offset in a block}).
    Every group starts at byte 0 of a block; the stride is the largest
    group's bytes rounded up to whole 512-byte rows."""
    offsets, widest = {}, 0
    for group in groups:
        placed, used = _place_group(group)
        repeated = offsets.keys() & placed.keys()
        if repeated:
            raise ValueError(f"Layer {min(repeated)!r} belongs to more than one compact group")
        offsets.update(placed)
        widest = max(widest, used)
    return round_up(widest, ROW_BYTES), offsets


def pool_bytes_per_block(groups):
    return packed_layout(groups)[0]


def max_memory_usage(config, groups):
    pages = sum(group.kv_cache_spec.max_memory_usage_pages(config) for group in groups)
    return pool_bytes_per_block(groups) * pages


_UNSUPPORTED_PARALLELISM = ("pipeline_parallel_size", "decode_context_parallel_size",
                            "prefill_context_parallel_size")


def _check_single_stage(config):
    """Compact pages serve one local cache per GPU: no pipeline stages, no
    context parallelism, no KV transfer."""
    parallel = config.parallel_config
    wider = [name for name in _UNSUPPORTED_PARALLELISM if getattr(parallel, name, 1) != 1]
    if wider:
        raise ValueError(f"Compact C8 pages need single-stage serving without context parallelism ({wider[0]} != 1)")
    if getattr(config, "kv_transfer_config", None) is not None:
        raise ValueError("Compact C8 pages serve local caches only; KV transfer is not part of this build")


def cache_config(config, groups, available_memory, types=None):
    """(number of blocks, one descriptor per layer over one shared backing)."""
    types = types or default_types()
    _check_single_stage(config)
    stride, offsets = packed_layout(groups)
    override = getattr(getattr(config, "cache_config", None), "num_gpu_blocks_override", None)
    blocks = int(override) if override is not None else available_memory // stride
    return blocks, [types.tensor(size=blocks * stride, layers=[name], offset=offset, layer_stride=0,
                                 block_stride=stride) for name, offset in offsets.items()]


def _descriptor_layer(descriptor, stride, size):
    """(layer, offset) of a descriptor that covers one layer of the backing."""
    one_layer = len(descriptor.layers) == 1 and descriptor.layer_stride == 0
    if not one_layer or descriptor.block_stride != stride or descriptor.size != size:
        raise ValueError(f"Descriptor {descriptor!r} is not one layer of a {size}-byte backing "
                         f"with block stride {stride}")
    return descriptor.layers[0], descriptor.offset


def allocate_backing(groups, descriptors, num_blocks, layer_names, device):
    """One INT8 backing for every layer (2 MiB aligned); returns
    {layer: backing[offset:]}.  The descriptors must be exactly the
    planner's: one per layer, at the planned offset, stride and size."""
    stride, planned = packed_layout(groups)
    size = stride * num_blocks
    bound = {}
    for descriptor in descriptors:
        name, offset = _descriptor_layer(descriptor, stride, size)
        if name in bound or planned.get(name) != offset:
            raise ValueError(f"Layer {name!r}: descriptor offset {offset} is not the planned one")
        bound[name] = offset
    if bound.keys() != set(layer_names):
        raise ValueError("The descriptors do not cover exactly the cache layers")
    raw = torch.empty(size + BACKING_ALIGNMENT, dtype=torch.int8, device=device)
    start = (-raw.data_ptr()) % BACKING_ALIGNMENT
    backing = raw[start:start + size]
    logging.getLogger(__name__).info("compact C8 backing of %d bytes: %d layers in %d groups, %d blocks of %d bytes",
                                     size, len(bound), len(groups), num_blocks, stride)
    return {name: backing[offset:] for name, offset in bound.items()}


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
