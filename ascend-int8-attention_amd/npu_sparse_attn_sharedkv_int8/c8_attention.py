"""C8 route: scratch sizing, KV-partition choice and launcher selection.

Interface counterpart: npu_sparse_attn_sharedkv_int8/c8_attention.py:18-138 of
the reference checkout (CORES, HEADS, MAX_SPLITS, enabled(), supported(),
prepare()).  The Ascend build plans tiles on the device from live metadata
for 24 cores.  This build plans a launch on the host from its capacity
(choose_splits: a pure function of tokens, ratio, top-k and max_seq_len),
and the kernel re-plans on the device only when graph padding leaves rows
idle (device_splits, the host mirror of that rule), so tests and the CPU
checker can recompute the plan, and hence the numerics, of every launch:

  tile   128 keys; a query's list is the window rows, then its compressed rows,
         cut into 128-key tiles numbered continuously across the two kinds
  splits KV partitions; tile k is folded into partition k % splits and the
         partitions are merged by log-sum-exp in the same launch

A query row is one work-group per partition, one work-group per compute unit
(its two-tile LDS ring takes most of the CU's 160 KiB).  More partitions mean
shorter partitions but a wider merge (each partition's state is written, and
read back by the one that folds the row).  Measured on MI355X with 9-tile C4
rows: 3 partitions beat 2, 4, 5, 6 and 8 for 32 and 64 query rows (B=32 x T=2:
19.4 us at 3, 20.6 at 4; 16 seqs x T=2: 16.6 at 3, 17.2 at 6); a lone query
row is fastest with 5 (13.3 us, against 14.4 at 9).  The launch keeps to one
wave of work-groups: tokens * splits <= CORES.
"""
import copy
import ctypes
import os

import torch

from types import SimpleNamespace

from .runtime import SharedKVArgs, native_launcher, library

CORES = 256                # MI355X compute units
HEADS = 8                  # heads per work-group; a launch takes 1..MAX_HEADS in groups of eight
MAX_HEADS = 128
DIM = 512
TILE = 128                 # keys per tile; matches SHAREDKV_C8_TILE in the C ABI
MAX_SPLITS = 16
WINDOW = 128
BLOCK = 32
MAX_TOPK = 1024
SMALL_TOKENS = 24          # C4 launches of fewer tokens go through the small-launch entry
SPLITS_FEW_ROWS = 5        # when rows x 5 work-groups fit one wave on the CUs
SPLITS_MANY_ROWS = 3
ONE_TILE_ITEMS = 112       # one partition per tile while rows x tiles stay within this
PARTIAL_FLOATS = 520       # per (token, partition, head): 512 numerator, max, denominator, pad

VARIANT_SPARSE, VARIANT_DENSE, VARIANT_SPARSE_SMALL = 20, 21, 22
VARIANT_DENSE_PAIRED = 23      # the query-grouped plans on 256-key tiles: two tokens per group
VARIANT_DENSE_PACKED = 24      # four tokens per group
VARIANT_PAIRED_NARROW = 25     # the same on 128-key tiles
VARIANT_PACKED_NARROW = 26
GROUPED_TILE = 256             # the reference's grouped plans' tile (attention.py:104-106 there)

# A workspace of this size serves any launch of up to WORKSPACE_ROWS rows (one
# uint32 merge ticket per row), for callers that size one shared workspace up
# front as the reference's constant allows (c8_attention.py:27-30 there);
# prepare() itself sizes each launch exactly (workspace_bytes).
WORKSPACE_ROWS = 1 << 16
WORKSPACE_BYTES = WORKSPACE_ROWS * 4


def enabled():
    """SHAREDKV_C8_DECODE: '1' (default) routes to this kernel; '0' asks for the
    legacy kernels, which this build does not have."""
    value = os.environ.get("SHAREDKV_C8_DECODE", "1")
    if value not in ("0", "1"):
        raise ValueError("SHAREDKV_C8_DECODE must be 0 or 1")
    return value == "1"


def max_tiles(ratio, topk, max_seq_len=None, ori_topk=0):
    """Upper bound on a query's tile count (window or explicit-slot tiles +
    compressed tiles)."""
    window_tiles = (max(WINDOW, ori_topk) + TILE - 1) // TILE
    if ratio == 4:
        return window_tiles + (min(topk, MAX_TOPK) + TILE - 1) // TILE
    if ratio == 128:
        if max_seq_len is None:
            return MAX_SPLITS
        return window_tiles + (max(0, int(max_seq_len)) // 128 + TILE - 1) // TILE
    return window_tiles


def plan_splits(rows, tiles, one_tile=True, room=None):
    """Partitions for `rows` query rows of at most `tiles` tiles each.

    One partition per tile while rows x tiles <= ONE_TILE_ITEMS, tiles <=
    MAX_SPLITS and tiles <= `room` (the work items a padded launch has per
    live row), if `one_tile`: every partition then waits for one tile before
    the merge (on MI355X 1-12 C4 rows of nine tiles take 0.1-0.8 us less
    than at five partitions, 14 and 16 rows more; eight partitions, where
    one holds two tiles, were slower than five).  Else five partitions while rows x 5
    work-groups fit one wave on the CUs (a row's nine tiles then take at
    most two per partition), else three; the fastest of 2..8 at 32 and 64
    rows.  The kernel applies the same rule to the live rows of a padded
    launch (c8_rows without the one-tile plan)."""
    if one_tile and rows * tiles <= ONE_TILE_ITEMS and tiles <= MAX_SPLITS and (room is None or tiles <= room):
        return max(1, tiles)
    wanted = SPLITS_FEW_ROWS if rows * SPLITS_FEW_ROWS <= CORES else SPLITS_MANY_ROWS
    wanted = min(wanted, max(1, CORES // rows))
    return max(1, min(wanted, tiles, MAX_SPLITS))


def choose_splits(tokens, ratio, topk, max_seq_len=None, ori_topk=0):
    """KV partitions for a launch of `tokens` query rows (host-side plan)."""
    if tokens <= 0:
        return 1
    return plan_splits(tokens, max_tiles(ratio, topk, max_seq_len, ori_topk))


def choose_paired_splits(tokens, ratio, max_seq_len=None):
    """KV partitions of a query-grouped launch (query_group 2 or 4): the plan
    of its work-groups (one per pair of tokens, at most ceil(tokens / 2) of
    them), whose window list can take a second tile (up to 129 or 131
    rows).  A C4 group lists every compressed row below its last position
    / 4 (max_seq_len // 4 rows at most).  Few work-groups with a known tile
    count take one partition per tile, as ungrouped launches do (config 2's
    C128 launch at G2: 17.4 us at 5 partitions, 14.7 at one per tile)."""
    if tokens <= 0:
        return 1
    if ratio == 4:
        tiles = MAX_SPLITS + 1 if max_seq_len is None else 2 + (max(0, int(max_seq_len)) // 4 + TILE - 1) // TILE
    else:
        tiles = max_tiles(ratio, 0, max_seq_len) + 1
    return plan_splits((tokens + 1) // 2, tiles)


def live_shape(cu_q, seq_lens, tokens):
    """(live tokens, longest live sequence) of a launch's metadata, as the
    kernel reads them (attention_impl.h:121-137): the last request with
    seq_len > 0 and cu_q[b + 1] >= 0 ends the live batch, its cu_q end
    (clamped to the launch's tokens) bounds the live tokens; the longest
    live sequence is the longest request that passes the same test."""
    cu_q = [int(x) for x in cu_q]
    seq_lens = [int(x) for x in seq_lens]
    live = [b for b, length in enumerate(seq_lens) if length > 0 and cu_q[b + 1] >= 0]
    if not live:
        return 0, 0
    end = cu_q[live[-1] + 1]
    return max(0, min(end, tokens)), max(seq_lens[b] for b in live)


def keyless_tokens(cu_q, seq_lens, tokens):
    """Query tokens whose output and LSE rows the kernel zero-fills: past the
    live tokens (graph padding, attention_impl.h:443-460), in no live
    request, or at a negative position (a request listing more query tokens
    than its sequence length; reference.py:104-105 rejects such metadata on
    the host, the device cannot read it back)."""
    cu = [int(x) for x in cu_q]
    lens = [int(x) for x in seq_lens]
    live_tokens, _ = live_shape(cu, lens, tokens)
    live_batch = max([b + 1 for b, n in enumerate(lens) if n > 0 and cu[b + 1] >= 0] + [0])
    keyless = [True] * tokens
    for t in range(live_tokens):
        for b in range(live_batch):
            if cu[b] <= t < cu[b + 1]:
                keyless[t] = lens[b] - cu[b + 1] + t < 0
    return keyless


def device_splits(splits, tokens, heads, ratio, topk, cu_q, seq_lens, ori_topk=0, fused=True, cmp_rows=None,
                  small=None):
    """The KV partitions the kernel runs a launch with, from its live metadata.

    A launch planned for `tokens` query tokens (graph capacity) at `splits`
    partitions has tokens x head groups x splits work-groups.  When fewer
    rows are live (graph padding), the kernel hands idle work-groups to the
    live rows as more partitions: plan_splits(live rows, tile count of the
    longest live row), at most work-groups // live rows and never below
    `splits`.  Only launches that merge in themselves re-plan (`fused`: the
    library's merge mode 0, with several partitions or with one partition
    and the re-plan's partition states supplied, which prepare() always
    does); one-partition C4 and window-only launches of more rows than CUs
    (rows_launch: c8_rows) apply the same rule with their rows as the
    work-groups, without the one-tile plan.  The kernel's numerics follow
    this count (tile k folds into partition k % count), so checkers use it
    in place of `splits`.

    Joint-plan launches (joint_launch; `cmp_rows` = the compressed block
    table's rows per sequence, width x 32) run as one partition per row
    instead.
    """
    live_tokens, longest = live_shape(cu_q, seq_lens, tokens)
    groups = head_groups(heads)
    live_rows, rows = live_tokens * groups, tokens * groups
    if joint_launch(splits, tokens, heads, ratio, cu_q, seq_lens, ori_topk, fused, cmp_rows, small):
        return 1
    if not fused or live_rows == 0 or live_rows >= rows:
        return splits
    tiles = (ori_topk + TILE - 1) // TILE if ori_topk else 1
    if ratio == 4:
        tiles += (min(longest // 4, topk) + TILE - 1) // TILE
    elif ratio == 128:
        tiles += (longest // 128 + TILE - 1) // TILE
    one_tile = not rows_launch(splits, tokens, heads, ratio, ori_topk, cmp_rows, small)
    room = rows * splits // live_rows
    return max(splits, min(plan_splits(live_rows, tiles, one_tile, room), room))


def rows_launch(splits, tokens, heads, ratio, ori_topk=0, cmp_rows=None, small=None):
    """Whether the kernel runs a launch on c8_rows (two four-wave work-groups
    per CU taking rows in turn): one partition, more rows than CUs, no
    explicit original slots, and window-only or C4 without joint rows
    compiled in (C4 kernels carry them for launches through the small-launch
    entry and for compressed block tables of at most one tile of rows per
    sequence)."""
    if small is None:
        small = tokens < SMALL_TOKENS
    joint4 = heads <= HEADS and (small or (cmp_rows is not None and cmp_rows <= TILE))
    return (splits == 1 and not ori_topk and tokens * head_groups(heads) > CORES
            and (ratio == 1 or (ratio == 4 and not joint4)))


def joint_launch(splits, tokens, heads, ratio, cu_q, seq_lens, ori_topk=0, fused=True, cmp_rows=None, small=None):
    """Whether the kernel runs a launch as a joint-plan launch: joint_plan
    holds, every live row fits one window tile and one compressed tile
    (longest live sequence // ratio <= 128), and the launch is fused or of
    one partition.  C4 launches need kernels with joint rows compiled in:
    those of the small-launch entry (`small`; by default the package's
    routing, fewer than SMALL_TOKENS tokens: launch_sharedkv_c8_sparse_small,
    which like the reference's small entry chooses from live lengths,
    c4_small.cpp:10-19), or whose compressed block table names at most 128
    rows per sequence (`cmp_rows` = table width x 32).  Such a launch runs
    one partition per row.  Its C128 rows with compressed rows, and all its
    C4 rows, are joint rows; C4 launches that are not joint-plan launches
    have none (reference.py:246 switches every C4 row of a joint_sparse plan
    to the dense multiplicity list)."""
    if small is None:
        small = tokens < SMALL_TOKENS
    if ratio == 4 and not small and (cmp_rows is None or cmp_rows > TILE):
        return False
    live_tokens, longest = live_shape(cu_q, seq_lens, tokens)
    return (joint_plan(ratio, heads, ori_topk > 0) and (fused or splits == 1) and live_tokens > 0
            and longest // ratio <= TILE)


def joint_plan(ratio, heads, explicit_slots):
    """Whether a launch's plan takes joint rows (reference.py:254-267):
    joint_dense for C128 (the reference device's two-kind pipeline at one
    partition, attention_impl.h:94-100) and joint_sparse for C4 (its short
    C4 task batches, c4.cpp:35-58).  When it does, every row of a
    one-partition launch whose window and compressed lists each fit one
    128-key tile runs one softmax over both kinds; other rows, and launches
    of more partitions, are tiled as usual.  C4 rows are joint only in a
    joint-plan launch (joint_launch), where each takes its compressed list
    densely with log(multiplicity) biases.
    Residual codes are required (at most eight heads), and explicit
    original slots keep the tiled plan."""
    return ratio in (4, 128) and heads <= HEADS and not explicit_slots


def supported(entry):
    """C8 ABI: 1..128 heads, ratio 1/4/128, window 128, block32 pages, top-k
    <= 1024, at most 1024 explicit original slots (reference
    c8_attention.py:56-71 requires 8 heads, top-k == 1024, ratio 4/128 and no
    explicit slots, leaving the rest to its legacy kernels; the HIP kernel
    covers them)."""
    if not getattr(entry, "blocks", 0) or getattr(entry, "args", None) is None:
        return False
    p = entry.args
    return (1 <= p.heads <= MAX_HEADS and p.tokens > 0 and p.batch > 0 and p.ratio in (1, 4, 128)
            and p.window == WINDOW and p.oriBlock == BLOCK and (p.ratio == 1 or p.cmpBlock == BLOCK)
            and (not p.oriIndices or 0 < p.oriTopk <= MAX_TOPK) and (p.ratio != 4 or 0 < p.topk <= MAX_TOPK)
            and 1 <= p.splits <= MAX_SPLITS and p.oriStride % 16 == 0 and p.cmpStride % 16 == 0)


def argument_type():
    """The ctypes argument block (reference c8_attention.py:40-43)."""
    return SharedKVArgs


def host_module():
    """The launcher object over the C ABI (the reference loads a pybind
    module here, c8_attention.py:123-129)."""
    return native_launcher()


def native_host(queued=False):
    """Launch entry of the C8 kernels (reference c8_attention.py:132-138);
    queued and direct launches are the same HIP launch here."""
    host = native_launcher()
    return SimpleNamespace(attention=host.attention_queued if queued else host.attention,
                           attention_args_size=host.attention_args_size, _owner=host)


def head_groups(heads):
    return (heads + HEADS - 1) // HEADS


def workspace_bytes(rows, splits):
    """rows = query tokens x head groups of eight."""
    return int(library().sharedkv_c8_workspace_bytes(rows, splits))


def partial_shape(rows, splits):
    """FP32 partition states: [rows, splits, 8, 520] with several partitions;
    with one, the room of the device re-plan of a padded launch (at most
    CORES row partitions: live rows x partitions <= CORES whenever the plan
    gives more than one), or nothing for a one-row launch."""
    if splits > 1:
        return (rows, splits, HEADS, PARTIAL_FLOATS)
    return (min(rows, CORES), HEADS, PARTIAL_FLOATS) if rows > 1 else (0,)


def prepare(entry, *, scratch_allocator=None, shared_storage=False):
    """Bind scratch and the launcher; returns a prepared copy of `entry`.

    A row is a query token's group of eight heads (tokens x ceil(heads / 8)
    rows; one row per token at 8 heads).
    workspace: one uint32 merge ticket per row (the last partition of a row
    to finish folds the row).  It is zeroed here, and every launch leaves it
    zero again, so a workspace must not be shared by launches that can run
    concurrently (separate streams get separate scratch through
    scratch_allocator's (name, stream) key).
    partial: FP32 [rows, splits, 8, 520] partition states (splits > 1), or
    with one partition the room of the device re-plan of a padded launch
    (partial_shape).
    """
    if getattr(entry, "c8_dynamic", False) or not supported(entry):
        return entry
    p = entry.args
    device = entry.case.q.device
    allocate = scratch_allocator or (lambda name, shape, dtype, dev: torch.empty(shape, dtype=dtype, device=dev))
    rows = p.tokens * head_groups(p.heads)
    need_ws = workspace_bytes(rows, p.splits)
    shape = partial_shape(rows, p.splits)
    need_partial = 1
    for extent in shape:
        need_partial *= extent
    has_partial = need_partial > 0 and shape != (0,)
    workspace, partial = entry.workspace, entry.partial
    if shared_storage:
        if workspace is None or workspace.numel() < need_ws or (
                has_partial and (partial is None or partial.numel() < need_partial)):
            raise ValueError("C8 shared controls require the full workspace and partial extents")
    else:
        if workspace is None or workspace.numel() < need_ws:
            workspace = allocate("workspace", (need_ws,), torch.uint8, device)
        if has_partial and (partial is None or partial.numel() < need_partial):
            partial = allocate("partial", shape, torch.float32, device)
    workspace[:need_ws].zero_()

    out = copy.copy(entry)
    out.args = type(p).from_buffer_copy(p)
    out.args.workspace = workspace.data_ptr()
    out.args.partial = partial.data_ptr() if (partial is not None and has_partial) else 0
    out.workspace, out.partial = workspace, partial
    out.blocks = rows * p.splits
    out.argument_address = ctypes.addressof(out.args)
    small = p.ratio == 4 and p.tokens < SMALL_TOKENS
    out.variant = VARIANT_SPARSE_SMALL if small else (VARIANT_SPARSE if p.ratio == 4 else VARIANT_DENSE)
    out.native = native_launcher()
    if out.native.attention_args_size != ctypes.sizeof(type(p)):
        raise RuntimeError("C8 host/device argument ABI mismatch")
    out.c8_dynamic = True
    return out
