"""Host-side logic and the C ABI, without a GPU.

- libsharedkv_hip.so loads and exports every function include/sharedkv_hip.h
  declares; the argument blocks have the reference's sizes and field offsets
  (SharedKVArgs 200 bytes, csrc/kernels/c8/args.h:7-14 of the reference).
- The Python boundary rejects contract violations with ValueError before any
  device work (attention.py:31-83, cache.py:25-41 of the reference).
- The host plan (tile 128, KV partitions) is the documented pure function.
"""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from npu_sparse_attn_sharedkv_int8 import (CacheQuantization, PreparedAttention, PreparedCacheWrite,
                                           SharedKVCase)
from npu_sparse_attn_sharedkv_int8 import c8_attention, runtime
from npu_sparse_attn_sharedkv_int8._paths import native_path

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "sharedkv_hip.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|uint32_t|uint64_t|void)\s+\**\s*(\w+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_function():
    lib = ctypes.CDLL(str(native_path()))
    names = declared_functions()
    assert "launch_sharedkv_c8_sparse" in names and "launch_cache_write" in names
    for name in names:
        assert hasattr(lib, name), name
    assert set(runtime.EXPORTS) <= set(names)


def _noalloc_layout(lib, rows, splits):
    tickets, states = ctypes.c_uint64(), ctypes.c_uint64()
    rc = lib.sharedkv_c8_noalloc_layout(rows, splits, ctypes.byref(tickets), ctypes.byref(states))
    return rc, tickets.value, states.value


def test_noalloc_ticket_and_state_regions_never_overlap():
    """For any two launches of the allocation-free entry, in either order, no
    byte holds one launch's merge tickets and the other's partition states
    (a ticket left non-zero by a state float would never fold its row)."""
    lib = runtime.library()
    limit = lib.sharedkv_c8_noalloc_scratch_bytes()
    per_row = 8 * 520 * 4
    fits = []
    for splits in (1, 2, 3, 5, 8, 16):
        for rows in (1, 4, 20, 63, 64, 65, 100, 255, 256, 257, 300, 503, 504, 505, 1024, 1025, 4096, 1 << 20):
            rc, tickets, states = _noalloc_layout(lib, rows, splits)
            if splits == 1:
                assert rc == 0, (rows, splits)        # one partition: no tickets, no states
                continue
            need = rows * splits * per_row
            assert (rc == 0) == (states + need <= limit), (rows, splits)
            if rc == 0:
                assert tickets + 4 * rows <= states, (rows, splits)
                fits.append((tickets, tickets + 4 * rows, states, states + need))
    assert _noalloc_layout(lib, 504, 2)[0] == 0 and _noalloc_layout(lib, 505, 2)[0] == 1
    for t0, t1, _, _ in fits:
        for _, _, s0, s1 in fits:
            assert t1 <= s0 or s1 <= t0
    assert lib.sharedkv_c8_noalloc_layout(4, 0, ctypes.byref(ctypes.c_uint64()), ctypes.byref(ctypes.c_uint64())) == 1


def test_argument_blocks_match_reference_layout():
    lib = runtime.library()
    assert lib.sharedkv_attention_args_size() == 200 == ctypes.sizeof(runtime.SharedKVArgs)
    assert lib.sharedkv_cache_args_size() == ctypes.sizeof(runtime.CacheWriteArgs) == 88
    a = runtime.SharedKVArgs
    assert a.q.offset == 0 and a.oriIndices.offset == 136 and a.tokens.offset == 144
    assert a.oriPages.offset == 192 and a.softmaxScale.offset == 196
    c = runtime.CacheWriteArgs
    assert c.slotColumnStride.offset == 56 and c.tokens.offset == 64 and c.pairedSlots.offset == 80


def test_module_helpers_match_reference_names():
    """c8_attention exposes the reference module's helper names
    (c8_attention.py:27-46,123-138 there) over the C ABI."""
    lib = runtime.library()
    assert c8_attention.argument_type() is runtime.SharedKVArgs
    assert c8_attention.library() is lib
    assert c8_attention.WORKSPACE_BYTES >= lib.sharedkv_c8_workspace_bytes(c8_attention.WORKSPACE_ROWS, 16)
    for queued in (False, True):
        host = c8_attention.native_host(queued)
        assert host.attention_args_size == ctypes.sizeof(runtime.SharedKVArgs)
        assert host._owner is c8_attention.host_module() and callable(host.attention)


def test_scratch_sizes():
    lib = runtime.library()
    # One partition: the device re-plan's room, at most 256 row partitions
    # (the host's partial_shape); nothing for a single row.
    assert lib.sharedkv_c8_partial_bytes(64, 1) == 64 * 8 * 520 * 4
    assert lib.sharedkv_c8_partial_bytes(4096, 1) == 256 * 8 * 520 * 4
    assert lib.sharedkv_c8_partial_bytes(1, 1) == 0
    for rows in (2, 64, 300, 4096):
        assert lib.sharedkv_c8_partial_bytes(rows, 1) == 4 * int(np.prod(c8_attention.partial_shape(rows, 1)))
    assert lib.sharedkv_c8_partial_bytes(64, 8) == 64 * 8 * 8 * 520 * 4
    assert lib.sharedkv_c8_workspace_bytes(64, 8) >= 64 * 4
    assert lib.sharedkv_c8_workspace_bytes(1, 1) % 256 == 0


def test_launchers_reject_bad_blocks_without_a_device():
    """Argument checks run before any HIP call, so they are testable here."""
    lib = runtime.library()
    args = runtime.SharedKVArgs()
    assert lib.launch_sharedkv_c8_sparse(0, None, ctypes.byref(args)) == 0   # 0 blocks: no launch
    assert lib.launch_sharedkv_c8_sparse(1, None, ctypes.byref(args)) == 1   # ratio 0 rejected
    args.ratio = 128
    assert lib.launch_sharedkv_c8_dense(1, None, ctypes.byref(args)) == 1    # null pointers rejected
    cw = runtime.CacheWriteArgs()
    assert lib.launch_cache_write(1, None, ctypes.byref(cw)) == 1
    assert lib.sharedkv_c8_set_merge_mode(2) == 1
    assert lib.sharedkv_c8_set_merge_mode(1) == 0
    assert lib.sharedkv_c8_set_merge_mode(0) == 0
    # The grouped entries (both tile sizes) check the block the same way.
    for name in ("launch_sharedkv_c8_dense_paired", "launch_sharedkv_c8_dense_packed",
                 "launch_sharedkv_c8_dense_paired_narrow", "launch_sharedkv_c8_dense_packed_narrow"):
        fn = getattr(lib, name)
        assert fn(0, None, ctypes.byref(args)) == 0, name
        assert fn(1, None, None) == 1, name
        assert fn(1, None, ctypes.byref(args)) == 1, name   # null pointers rejected
    # The XCD-local exchange switch takes 0 or 1; no probe runs without a launch.
    assert lib.sharedkv_c8_set_xcd_local(2) == 1
    assert lib.sharedkv_c8_set_xcd_local(0) == 0
    assert lib.sharedkv_c8_set_xcd_local(1) == 0
    if not torch.cuda.is_available():
        assert lib.sharedkv_c8_xcd_local() == -1


@pytest.mark.skipif(torch.cuda.is_available(), reason="placeholder addresses: host-side check only")
def test_launch_rejects_grids_past_the_limit():
    """tokens x ceil(heads / 8) x splits work-groups must fit one grid; a
    launch past it is rejected before any HIP call."""
    lib = runtime.library()
    a = runtime.SharedKVArgs()
    for name in ("q", "ori", "oriScale", "oriTable", "cuQ", "seqLens", "sinks", "out", "cmp", "cmpScale",
                 "cmpTable", "indices", "partial", "workspace"):
        setattr(a, name, 0x10000)
    a.heads, a.ratio, a.window, a.oriBlock, a.cmpBlock, a.batch, a.oriPages = 128, 4, 128, 32, 32, 1, 1
    a.topk, a.oriStride, a.cmpStride, a.tokens, a.splits = 1024, 16384, 16384, 1 << 23, 16
    assert lib.launch_sharedkv_c8_sparse(1, None, ctypes.byref(a)) == 1
    # The writer passes slot strides as 32-bit kernel arguments.
    w = runtime.CacheWriteArgs(cache=0x10000, updates=0x10000, slots=0x10000, inverseScale=0x10000,
                               pageStride=16384, updateStride=512, slotStride=1 << 32, slotColumnStride=1,
                               tokens=4, pages=1, pageSize=32)
    assert lib.launch_cache_write(1, None, ctypes.byref(w)) == 1


def test_compiled_bridge_loads_and_rejects_bad_calls_without_a_device():
    """The CPython launch bridge (csrc/host_bridge.cpp) binds the same
    library; malformed calls raise before any HIP call."""
    bridge = runtime.bridge()
    assert callable(bridge.attention) and callable(bridge.cache_write)
    with pytest.raises(ValueError, match="variant"):
        bridge.attention(0x1000, 1, 99, 0)
    with pytest.raises(ValueError):
        bridge.attention(0, 1, runtime.VARIANT_SPARSE, 0)           # no argument block
    with pytest.raises(ValueError):
        bridge.cache_write(0x1000, 1 << 33, 0)                       # more work-groups than a launch takes
    with pytest.raises(TypeError):
        bridge.attention(0x1000, 1, runtime.VARIANT_SPARSE)
    with pytest.raises(OverflowError):
        bridge.attention(-1, 1, runtime.VARIANT_SPARSE, 0)


def test_host_plan():
    assert c8_attention.max_tiles(4, 1024) == 9
    assert c8_attention.max_tiles(128, 0, 4096) == 2
    assert c8_attention.max_tiles(1, 0) == 1
    assert c8_attention.choose_splits(64, 4, 1024) == 3
    assert c8_attention.choose_splits(32, 4, 1024) == 5       # 160 work-groups: one wave
    assert c8_attention.choose_splits(51, 4, 1024) == 5 and c8_attention.choose_splits(52, 4, 1024) == 3
    # Up to 112 work items: one partition per tile (12 C4 rows of 9 tiles).
    assert c8_attention.choose_splits(1, 4, 1024) == 9
    assert c8_attention.choose_splits(12, 4, 1024) == 9 and c8_attention.choose_splits(13, 4, 1024) == 5
    assert c8_attention.choose_splits(16, 128, 0, 20000) == 3       # 1 + 2 tiles
    assert c8_attention.plan_splits(2, 9, one_tile=False) == 5
    assert c8_attention.plan_splits(8, 9, room=8) == 5                # no room for 9
    assert c8_attention.choose_splits(100, 4, 1024) == 2       # one wave of work-groups
    assert c8_attention.choose_splits(4096, 4, 1024) == 1
    assert c8_attention.choose_splits(1, 128, 0, 4096) == 2
    assert c8_attention.choose_splits(2, 128, 0) == 16       # tile count unknown: its bound
    # Grouped 128-key plans: one partition per tile for few work-groups of a
    # known tile count (16 pairs x 6 tiles at 64 K), else five.
    assert c8_attention.choose_paired_splits(32, 128, 65536) == 6
    assert c8_attention.choose_paired_splits(32, 128) == 5 and c8_attention.choose_paired_splits(64, 128, 65536) == 5
    assert c8_attention.choose_paired_splits(32, 4) == 5 and c8_attention.choose_paired_splits(32, 4, 1024) == 4
    assert c8_attention.choose_splits(1, 1, 0) == 1


def test_device_plan_of_padded_launches():
    """The kernel's re-plan of a graph-padded launch (its host mirror):
    capacity 64 C4 rows at 3 partitions (192 work-groups) replayed with
    8/16/32/64 live requests of 9-tile rows runs what an eager launch of the
    live rows would choose; separate-merge launches keep their plan, and a
    one-partition launch re-plans within its rows (its work-groups)."""
    plan = c8_attention.device_splits
    cap = 64
    assert c8_attention.choose_splits(cap, 4, 1024) == 3
    for live, want, one in ((8, 9, 5), (16, 5, 4), (32, 5, 2), (51, 3, 1), (64, 3, 1)):
        cu = list(range(live + 1)) + [cap] * (cap - live)
        lens = [20000] * live + [0] * (cap - live)
        assert plan(3, cap, 8, 4, 1024, cu, lens) == want, live
        assert plan(3, cap, 8, 4, 1024, cu, lens, fused=False) == 3
        assert plan(1, cap, 8, 4, 1024, cu, lens) == one, live
        assert plan(1, cap, 8, 4, 1024, cu, lens, fused=False) == 1
        # Eager's choice where the work-groups allow it (51 x 5 > 192).
        assert want == c8_attention.choose_splits(live, 4, 1024) or live == 51
    # A one-partition C4 launch of 512 rows (c8_rows) replayed with 16 or 64
    # live sequences of two tokens: the eager plan of the live rows.
    for live, want in ((16, 5), (64, 2)):
        cu = [2 * i for i in range(live + 1)] + [2 * live] * (256 - live)
        lens = [30000] * live + [0] * (256 - live)
        assert plan(1, 512, 8, 4, 1024, cu, lens) == want == c8_attention.choose_splits(2 * live, 4, 1024)
    assert c8_attention.partial_shape(512, 1) == (256, 8, 520) and c8_attention.partial_shape(1, 1) == (0,)
    # Work-groups cap the plan: capacity 6 at 2 partitions, 5 live rows -> 2.
    assert plan(2, 6, 8, 4, 1024, [0, 5, 6], [9000, 0]) == 2
    # The longest live row bounds the plan by its tile count: C4 top-k rows
    # of a 600-key sequence have 1 + ceil(150 / 128) = 3 tiles, C128 rows of
    # 4096 keys 1 + 1, window-only rows 1 (explicit slots: ceil(K / 128)).
    assert plan(2, 64, 8, 4, 1024, [0, 1, 64], [600, 0]) == 3
    assert plan(2, 64, 8, 128, 0, [0, 1, 64], [20000, 0]) == 3      # 1 + ceil(156 / 128) tiles
    assert plan(2, 64, 8, 1, 0, [0, 1, 64], [4096, 0]) == 2
    assert plan(2, 64, 8, 1, 0, [0, 1, 64], [4096, 0], ori_topk=384) == 3
    # Head groups count as rows: 16 heads, 4 live tokens of 32 -> 8 rows of
    # 9 tiles, one partition per tile; 8 live tokens -> 16 rows, 5.
    assert plan(3, 32, 16, 4, 1024, [0, 4, 32], [30000, 0]) == 9
    assert plan(3, 32, 16, 4, 1024, [0, 8, 32], [30000, 0]) == 5
    # The live shape: a cu_q sentinel (-1) or seq_len 0 ends the live batch.
    assert c8_attention.live_shape([0, 2, 4, -1], [5000, 2600, 9000], 6) == (4, 5000)
    assert c8_attention.live_shape([0, 2, 4, 6], [5000, 0, 0], 6) == (2, 5000)
    assert c8_attention.live_shape([0, 2, 9], [1, 8], 6) == (6, 8)
    assert c8_attention.live_shape([0, 0], [0], 4) == (0, 0)
    assert plan(3, 6, 8, 4, 1024, [0, 0, 0], [0, 0]) == 3     # nothing live


def test_device_plan_of_joint_launches():
    """C128 and C4 launches whose live rows all fit one window and one
    compressed tile (longest live sequence // ratio <= 128; C4 also needs a
    compressed block table of at most 128 rows per sequence) run one
    partition per row with joint rows; not above eight heads, with explicit
    slots, for window-only launches, or (for more than one partition) with a
    separate merge launch."""
    plan = c8_attention.device_splits
    short = [0, 1, 2, 3, 4]
    assert plan(5, 4, 8, 128, 0, short, [4096] * 4) == 1
    assert plan(1, 4, 8, 128, 0, short, [4096] * 4, fused=False) == 1
    assert plan(5, 4, 8, 128, 0, short, [4096] * 4, fused=False) == 5
    assert plan(5, 4, 8, 128, 0, short, [16511] * 4) == 1 and plan(5, 4, 8, 128, 0, short, [16512] * 4) == 5
    assert plan(5, 4, 16, 128, 0, short, [4096] * 4) == 5                      # no residual codes
    assert plan(5, 4, 8, 128, 0, short, [4096] * 4, ori_topk=128) == 5         # explicit slots
    # C4: a launch through the small-launch entry (fewer than 24 tokens, the
    # package's routing) follows live lengths whatever the table width, like
    # the reference's c4_small.cpp:10-19; other launches also need a
    # compressed block table of at most 128 rows per sequence.
    assert plan(5, 4, 8, 4, 1024, short, [4096] * 4, cmp_rows=1024) == 5      # long C4 rows keep the plan
    assert plan(5, 4, 8, 4, 1024, short, [515] * 4, cmp_rows=128) == 1
    assert plan(5, 4, 8, 4, 1024, short, [516] * 4, cmp_rows=160) == 5
    assert plan(5, 4, 8, 4, 1024, short, [515] * 4, cmp_rows=160) == 1        # small entry: live lengths
    assert plan(5, 4, 8, 4, 1024, short, [515] * 4, cmp_rows=33760) == 1      # a serving-width table (1055 pages)
    assert plan(5, 4, 8, 4, 1024, short, [515] * 4, cmp_rows=160, small=False) == 5   # sparse entry, wide table
    assert plan(5, 4, 8, 4, 1024, short, [515] * 4, small=False) == 5         # table unknown
    wide_cu = list(range(25)) + [24] * 8
    assert plan(2, 32, 8, 4, 1024, wide_cu, [515] * 24 + [0] * 8, cmp_rows=33760) == 2   # 32 tokens: sparse entry
    assert plan(2, 32, 8, 4, 1024, wide_cu, [515] * 24 + [0] * 8, cmp_rows=128) == 1
    assert plan(5, 4, 8, 4, 1024, short, [515] * 4, ori_topk=128, cmp_rows=128) == 5   # explicit slots
    assert plan(5, 4, 8, 1, 0, short, [100] * 4) == 5                          # window only: no joint rows
    assert plan(3, 64, 8, 128, 0, list(range(9)) + [8] * 56, [4096] * 8 + [0] * 56) == 1   # padded
    assert plan(3, 64, 8, 4, 1024, list(range(9)) + [8] * 56, [300] * 8 + [0] * 56, cmp_rows=96) == 1
    joint = c8_attention.joint_plan
    assert joint(128, 8, False) and joint(128, 4, False) and joint(4, 8, False) and joint(4, 1, False)
    assert not joint(128, 9, False) and not joint(4, 16, False) and not joint(1, 8, False)
    assert not joint(4, 8, True) and not joint(128, 8, True)


def test_device_plan_constants_match_the_host_rule():
    """The kernel's re-plan uses the host's partition rule: its constants
    (csrc/sharedkv_c8.hip) equal c8_attention's."""
    src = (ROOT / "ascend-int8-attention_amd" / "csrc" / "sharedkv_c8.hip").read_text()
    found = re.search(r"constexpr int32_t PLAN_CUS = (\d+), PLAN_FEW = (\d+), PLAN_MANY = (\d+), "
                      r"PLAN_ONE_TILE = (\d+);", src)
    assert found, "plan constants not found in the kernel source"
    assert tuple(int(x) for x in found.groups()) == (c8_attention.CORES, c8_attention.SPLITS_FEW_ROWS,
                                                      c8_attention.SPLITS_MANY_ROWS, c8_attention.ONE_TILE_ITEMS)
    assert re.search(r"constexpr uint32_t MAX_SPLITS = (\d+);", src).group(1) == str(c8_attention.MAX_SPLITS)


def test_keyless_tokens_rule():
    """Tokens the kernel zero-fills: past the live end, outside every live
    request, or at a negative position; the checker (like the reference,
    reference.py:104-105) rejects negative positions instead."""
    keyless = c8_attention.keyless_tokens
    # Request 0 lists 3 tokens over 1 key (positions -2, -1, 0).
    assert keyless([0, 3, 5, 6], [1, 900, 40], 6) == [True, True, False, False, False, False]
    assert keyless([0, 2, 3, 6, 6], [3000, 700, 0, 0], 6) == [False] * 3 + [True] * 3
    assert keyless([0, 2, 4, -1], [5000, 2600, 9000], 6) == [False] * 4 + [True] * 2
    assert keyless([1, 2], [10], 3) == [True, False, True]
    import oracle.oracle as ora
    from tests import workloads
    case = workloads.make_case(31, 4, [3, 2, 1], [1, 900, 40])
    with pytest.raises(ValueError, match="code -8"):
        ora.tiled_attention(workloads.oracle_case(case), tile=128, splits=1, return_lse=True)


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; --gpus N > 1 exits with a message before it
    touches a device."""
    import subprocess
    import sys
    run = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                         timeout=120)
    assert run.returncode == 2 and "measures one GPU" in run.stderr and not run.stdout


def test_c8_switch():
    import os
    old = os.environ.get("SHAREDKV_C8_DECODE")
    try:
        os.environ["SHAREDKV_C8_DECODE"] = "2"
        with pytest.raises(ValueError):
            c8_attention.enabled()
        os.environ["SHAREDKV_C8_DECODE"] = "1"
        assert c8_attention.enabled()
    finally:
        if old is None:
            os.environ.pop("SHAREDKV_C8_DECODE", None)
        else:
            os.environ["SHAREDKV_C8_DECODE"] = old


def cpu_case(**over):
    t, h = 2, 8
    q = torch.zeros((t, h, 512), dtype=torch.bfloat16)
    cache = torch.zeros((4, 32, 1, 512), dtype=torch.int8)
    fields = dict(q=q, ori=cache, ori_block_table=torch.zeros((1, 4), dtype=torch.int32),
                  cu_q=torch.tensor([0, 2], dtype=torch.int32), seq_lens=torch.tensor([40], dtype=torch.int32),
                  sink=torch.zeros(h), cmp=cache, cmp_block_table=torch.zeros((1, 4), dtype=torch.int32),
                  cmp_indices=torch.zeros((t, 1, 1024), dtype=torch.int32), ratio=4)
    fields.update(over)
    return SharedKVCase(**fields)


def test_attention_validation_errors():
    scale = torch.ones(512)
    with pytest.raises(ValueError, match="GPU"):
        PreparedAttention(cpu_case(), scale, scale)          # host tensors
    with pytest.raises(ValueError, match="implementation"):
        PreparedAttention(cpu_case(), scale, scale, implementation="npu")


def test_cache_write_validation_errors():
    cache = torch.zeros((4, 32, 1, 512), dtype=torch.int8)
    with pytest.raises(ValueError, match="GPU"):
        PreparedCacheWrite(cache, torch.zeros((2, 512), dtype=torch.bfloat16), torch.zeros(2, dtype=torch.int32),
                           torch.ones(512))


@pytest.mark.parametrize("bad", [0.0, -1.0, float("nan"), float("inf")])
def test_reject_invalid_frozen_scales(bad):
    """tests/unit/test_reference.py:15-20 of the reference."""
    scale = torch.ones(512)
    scale[17] = bad
    with pytest.raises(ValueError):
        CacheQuantization(scale)


def test_quantization_kat_and_append_invariance():
    """tests/unit/test_reference.py:22-40 of the reference."""
    quant = CacheQuantization(torch.ones(512))
    row = torch.zeros(1, 512)
    row[0, :8] = torch.tensor([-200.0, -127.0, -1.5, -0.5, 0.5, 1.5, 127.0, 200.0])
    assert quant.quantize(row)[0, :8].tolist() == [-127, -127, -2, 0, 0, 2, 127, 127]
    assert quant.quantize(row).dtype == torch.int8
    cal = CacheQuantization.calibrate([torch.ones(3, 512)])
    scale, inverse = cal.scale.clone(), cal.inverse_scale.clone()
    prefix = torch.linspace(-1, 1, 512).reshape(1, 512)
    before = cal.quantize(prefix)
    cal.quantize(torch.full((2, 512), 1000.0))
    assert torch.equal(cal.scale, scale) and torch.equal(cal.inverse_scale, inverse)
    assert torch.equal(cal.quantize(prefix), before)


def test_msmodelslim_requires_zero_offsets():
    """tests/unit/test_reference.py:42-48 of the reference."""
    tensors = {"layer.kv_cache_scale": torch.ones(512), "layer.kv_cache_offset": torch.zeros(512)}
    assert torch.equal(CacheQuantization.from_msmodelslim(tensors, "layer").scale, torch.ones(512))
    tensors["layer.kv_cache_offset"][0] = 1
    with pytest.raises(ValueError, match="nonzero offsets"):
        CacheQuantization.from_msmodelslim(tensors, "layer")


def test_contract_encoding_matches_checker():
    """The host encoding helper equals the checker's restatement on random rows."""
    import oracle.oracle as ora
    rng = np.random.default_rng(3)
    x = rng.standard_normal((64, 512)).astype(np.float32) * 4
    scale = np.abs(rng.standard_normal(512)).astype(np.float32) * 0.03 + 1e-3
    quant = CacheQuantization(torch.from_numpy(scale))
    np.testing.assert_array_equal(quant.inverse_scale.numpy(), ora.inverse_scale(scale))
    np.testing.assert_array_equal(quant.quantize(torch.from_numpy(x)).numpy(),
                                  ora.quantize(x, ora.inverse_scale(scale)))


def test_case_to_moves_every_tensor():
    case = cpu_case()
    moved = case.to("cpu")
    assert moved is not case and moved.ratio == 4 and torch.equal(moved.q, case.q)
