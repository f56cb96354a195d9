"""Seeded random launches against the CPU checker: mixed ratios, head counts,
explicit original slots, C4 index modes, short contexts (joint rows),
prefill-like chunks of 260-400 tokens (c8_rows: work-groups taking rows in
turn), graph-capacity padding rows (a few, or enough that the device
re-plans the live rows, c8_rows capacities included), compressed block
tables as wide as a serving table, the grouped plans (query_group 2 and
4, 128- and 256-key tiles), KV partitions (1-16, the host plan included)
and both merge placements, all bit-exact (BF16 outputs) with the checker on the launch's own plan and
LSE within 2e-6."""
import os
import sys

import numpy as np
import pytest

from tests import workloads
from tests.device_cases import joint_flags, run_hip, run_oracle

pytestmark = pytest.mark.gpu

CASES = int(os.environ.get("SHAREDKV_FUZZ_CASES", "48"))   # more for a longer sweep


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def random_case(seed):
    rng = np.random.default_rng(1000 + seed)
    ratio = int(rng.choice([1, 4, 128]))
    batch = int(rng.integers(1, 6))
    queries = [int(q) for q in rng.integers(1, 5, batch)]
    # One launch in five is short-context (joint rows for C4 and C128).
    longest = 516 if rng.random() < 0.2 else 9000
    lengths = [int(max(q, rng.integers(1, longest))) for q in queries]
    prefill = rng.random() < 0.08
    if prefill:
        # Prefill-like: one long chunk of 260-400 query tokens (a
        # one-partition C4 launch of it runs c8_rows).
        queries[0] = int(rng.integers(260, 401))
        lengths[0] = int(queries[0] + rng.integers(0, 2500))
    heads = int(rng.choice([8, 8, 8, 4, 12, 16]))
    if prefill and rng.random() < 0.75:
        heads = 8
    mode = str(rng.choice(["uniform", "holes", "dups", "mixed"] + list(workloads.EDGE_MODES)))
    slots = rng.random() < 0.25 and not prefill      # a draft's slots cover at most 384 rows
    slot_mode = str(rng.choice(["draft", "shuffled", "pool"])) if slots else None
    splits = rng.choice([None, 1, 2, 3, 4, 5, 6, 8, 9, 12, 16])
    if prefill and rng.random() < 0.6:
        splits = None                                 # the host plan: one partition
    merge = int(rng.integers(0, 2))
    topk = int(rng.choice([1024, 512, 256]))
    need = max(q + 128 for q in queries) if slot_mode in ("draft", "shuffled") else 0
    ori_topk = 256 if need <= 256 else 384
    case = workloads.make_case(seed, ratio, queries, lengths, topk=topk, heads=heads, index_mode=mode,
                               ori_slots=slot_mode, ori_topk=ori_topk)
    # Graph capacity: a few padding rows, or (one launch in eight) enough that
    # the device re-plans the live rows of a one-partition or c8_rows launch.
    pad = int(rng.integers(1, 4)) if rng.random() < 0.3 else 0
    if not prefill and rng.random() < 0.125:
        pad = int(rng.integers(20, 300))
    # One C4 launch in six behind a serving-width compressed block table.
    wide = ratio == 4 and rng.random() < 1 / 6
    if wide:
        narrow = case["cmp"].table
        extra = int(rng.integers(1, 1055)) - narrow.shape[1]
        if extra > 0:
            case["cmp"].table = np.ascontiguousarray(
                np.concatenate([narrow, np.tile(narrow[:, :1], (1, extra))], axis=1))
    # One launch in four asks for a grouped plan (groups of two or four query
    # tokens).
    group = int(rng.choice([2, 4])) if heads <= 8 and not slot_mode and rng.random() < 0.25 else None
    tile = int(rng.choice([128, 256])) if group else None
    if pad:
        # Graph capacity: a synthetic request of `pad` NaN query rows with
        # seq_len 0 after the live ones (zero-filled by the kernel).
        live = int(case["cu_q"][-1])
        case["q"] = np.concatenate([case["q"], np.full((pad, heads, 512), 0x7FC0, np.uint16)])
        case["cu_q"] = np.concatenate([case["cu_q"], [live + pad]]).astype(np.int32)
        case["seq_lens"] = np.concatenate([case["seq_lens"], [0]]).astype(np.int32)
        case["ori"].table = np.concatenate([case["ori"].table, case["ori"].table[:1]])
        if case["cmp"] is not None:
            case["cmp"].table = np.concatenate([case["cmp"].table, case["cmp"].table[:1]])
        for key in ("cmp_indices", "ori_indices"):
            if case.get(key) is not None:
                filler = np.full((pad,) + case[key].shape[1:], -1, np.int32)
                case[key] = np.concatenate([case[key], filler])
    return case, (None if splits is None else int(splits)), merge, dict(
        ratio=ratio, queries=queries, lengths=lengths, heads=heads, mode=mode, slots=slot_mode, topk=topk,
        pad=pad, wide=case["cmp"].table.shape[1] if wide else 0, group=group, tile=tile,
        joint=bool(ratio != 1 and max(lengths) // ratio <= 128 and heads <= 8 and not slot_mode))


@pytest.mark.parametrize("seed", range(CASES))
def test_random_launch_matches_checker(seed):
    from npu_sparse_attn_sharedkv_int8.runtime import library
    case, splits, merge, desc = random_case(seed)
    say(f"[fuzz {seed}] splits={splits} merge={merge} {desc}")
    lib = library()
    try:
        assert lib.sharedkv_c8_set_merge_mode(merge) == 0
        out, lse, op = run_hip(case, splits=splits, query_group=desc["group"], tile_size=desc["tile"])
    finally:
        lib.sharedkv_c8_set_merge_mode(0)
    assert op.query_group == (desc["group"] or 1)
    plan = op.device_splits(merge_mode=merge)     # the kernel's re-plan under padding
    joint = joint_flags(case, op.splits, merge)   # judged on the launch as the kernel saw it
    live = int(case["cu_q"][-1]) - desc["pad"]
    if desc["pad"]:
        assert not out[live:].any() and not lse[live:].any(), "padding rows are not zero"
        case = dict(case, q=case["q"][:live], cu_q=case["cu_q"][:-1], seq_lens=case["seq_lens"][:-1])
    ref, ref_lse, _ = run_oracle(case, plan, joint=joint, query_group=op.query_group, tile=op.tile_size)
    diff = out[:live] != ref[:live]
    assert not diff.any(), f"seed {seed}: {int(diff.sum())} BF16 mismatches of {diff.size}"
    np.testing.assert_allclose(lse[:live], ref_lse[:live], rtol=0, atol=2e-6)
