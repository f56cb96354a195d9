"""The query-grouped plans (query_group 2 and 4) on the GPU against the CPU
checker.

reference.py:224-323 with query_group G: consecutive tokens G j .. G j + G - 1
of a request share one window list (positions max(0, p_first + 1 - 128) ..
p_last) and one compressed list (C128: rows below (p_last + 1) / 128; C4:
rows below (p_last + 1) / 4, each token weighing a row by its multiplicity
among its own valid top-k entries), each masking what it may not see.
PreparedAttention(query_group=G) runs it on 256-key tiles at one partition
(the reference operator's grouped plan: launch_sharedkv_c8_dense_paired /
_packed), or with tile_size=128 on 128-key tiles
(launch_sharedkv_c8_dense_paired_narrow / _packed_narrow); c8_pairs: one
work-group per pair of tokens within a group and partition, the group's
tiles fetched once per pair.  Every launch is checked bit for bit against
oracle.tiled_attention(tile, query_group=G) at the launch's partitions, and
shown to differ from the ungrouped plan (and G = 4 from G = 2, 256-key tiles
from 128-key ones) where the group's window makes the tiling differ.
"""
import sys

import numpy as np
import pytest

from tests import workloads
from tests.device_cases import bits_of, run_hip, run_oracle, to_device

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def check(case, splits, tag, group=2, tile=None, max_seq_len=None):
    out, lse, op = run_hip(case, splits=splits, query_group=group, tile_size=tile, max_seq_len=max_seq_len)
    assert op.query_group == group and op.device_splits() == op.splits and op.tile_size == (tile or 256)
    ref, ref_lse, _ = run_oracle(case, op.splits, query_group=group, tile=op.tile_size)
    live = int(case["cu_q"][-1])
    diff = out[:live] != ref[:live]
    assert not diff.any(), f"{tag}: {int(diff.sum())} BF16 mismatches of {diff[:live].size}"
    np.testing.assert_allclose(lse[:live], ref_lse[:live], rtol=0, atol=2e-6, err_msg=tag)
    return out, op


CASES = [
    # name, seed, ratio, queries per request, lengths
    ("mtp_pairs", 101, 128, [2] * 6, [130, 255, 256, 1000, 4097, 20000]),
    ("short_windows", 102, 128, [2, 2, 2], [2, 60, 129]),
    ("odd_groups", 103, 128, [3, 1, 5, 2], [3000, 700, 9000, 128]),
    ("prefill_chunk", 104, 128, [24], [6000]),
    ("window_only", 105, 1, [2, 3, 1, 4], [90, 700, 5, 300]),
    ("ragged_fours", 110, 128, [4, 7, 1, 6, 4], [131, 4000, 900, 20000, 256]),
    ("window_fours", 111, 1, [4, 5, 8, 3], [4, 133, 700, 2000]),
    # C4 groups: the dense list of the group's compressed rows, each token
    # weighing a row by its multiplicity among its own valid top-k entries.
    ("c4_short", 114, 4, [2, 3, 4], [300, 1000, 700]),
    ("c4_dups", 115, 4, [4, 2], [5000, 3000], "dups"),
    ("c4_holes", 116, 4, [3, 4, 1], [4200, 9000, 40], "holes"),
    ("c4_long_mixed", 117, 4, [4], [20000], "mixed"),
    ("c4_one_key", 118, 4, [2, 4, 2], [600, 2500, 9], "one_key_duplicates"),
]


@pytest.mark.parametrize("name,seed,ratio,queries,lengths,mode", [c + ("uniform",) * (6 - len(c)) for c in CASES],
                         ids=[c[0] for c in CASES])
@pytest.mark.parametrize("splits", [1, 2, 3, 5])
@pytest.mark.parametrize("group", [2, 4])
@pytest.mark.parametrize("tile", [256, 128])
def test_grouped_plan_matches_checker(name, seed, ratio, queries, lengths, mode, splits, group, tile):
    case = workloads.make_case(seed, ratio, queries, lengths, index_mode=mode)
    say(f"[grouped G{group} tile {tile}] {name} splits {splits}")
    out, op = check(case, splits, f"G{group} tile {tile} {name} splits {splits}", group, tile)
    if name in ("mtp_pairs", "ragged_fours"):
        # A later token's window starts later than the group's: on 128-key
        # tiles the tiling, and so the numerics, differ from the ungrouped
        # plan and between groups of two and of four (unless every request
        # has two tokens); a group's window list takes two 128-key tiles but
        # one 256-key tile (whose masked rows change nothing), so the tile
        # sizes differ too.
        ungrouped, _, _ = run_oracle(case, splits)
        assert (out != ungrouped).any()
        if tile == 128:
            other, _, _ = run_oracle(case, splits, query_group=6 - group, tile=tile)
            assert np.array_equal(out, other) == (name == "mtp_pairs")
        other_tile, _, _ = run_oracle(case, splits, query_group=group, tile=384 - tile)
        assert (out != other_tile).any()


@pytest.mark.parametrize("group", [2, 4])
@pytest.mark.parametrize("tile", [256, 128])
def test_grouped_plan_heads_and_default_partitions(group, tile):
    """Fewer than eight heads (the padding heads of the work-group are never
    written) and the default partition plan: one partition on 256-key tiles
    (the reference operator's), choose_paired_splits on 128-key tiles."""
    from npu_sparse_attn_sharedkv_int8 import c8_attention
    for heads in (4, 8):
        case = workloads.make_case(106, 128, [4] * 8, [2000 + 997 * i for i in range(8)], heads=heads)
        out, op = check(case, None, f"G{group} tile {tile} {heads} heads", group, tile)
        assert op.splits == (1 if tile == 256 else c8_attention.choose_paired_splits(32, 128))


@pytest.mark.parametrize("group", [2, 4])
def test_grouped_plan_one_partition_per_tile(group):
    """128-key grouped plans at one partition per tile: the library's choice
    for few work-groups with a known tile count (max_seq_len 66000: a
    window list of up to two tiles and five compressed tiles, 7 partitions
    for 6 work-groups of pairs), and 9 and 12 partitions (the fold above
    eight partitions, in groups of eight)."""
    from npu_sparse_attn_sharedkv_int8 import c8_attention
    case = workloads.make_case(119, 128, [2, 4, 2, 3], [66000, 41000, 20000, 9000])
    _, op = check(case, None, f"G{group} one tile per partition", group, 128, max_seq_len=66000)
    assert op.splits == c8_attention.choose_paired_splits(11, 128, 66000) == 7
    for splits in (9, 12):
        say(f"[grouped G{group}] tile 128 splits {splits}")
        check(case, splits, f"G{group} tile 128 splits {splits}", group, 128)


def test_packed_prefill_chunk():
    """A C128 prefill chunk (B = 1 x T = 256 at 9000 context) in groups of
    four, at one partition on 256-key tiles (the reference device's packed
    plan), and on 128-key tiles at one and two."""
    case = workloads.make_case(112, 128, [256], [9000])
    for tile, splits in ((256, 1), (128, 1), (128, 2)):
        say(f"[grouped G4] prefill chunk tile {tile} splits {splits}")
        check(case, splits, f"G4 prefill tile {tile} splits {splits}", 4, tile)


@pytest.mark.parametrize("tile", [256, 128])
@pytest.mark.parametrize("group", [2, 4])
@pytest.mark.parametrize("mode", [0, 1])
def test_grouped_plan_padding_and_merge_modes(mode, group, tile):
    """Graph-padding rows past the live tokens come back zero (NaN-poisoned
    Q), in both merge placements (fused, or the separate merge launch)."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    from npu_sparse_attn_sharedkv_int8.runtime import library
    case = workloads.make_case(107, 128, [2, 5, 3], [5000, 2600, 9000])
    live = int(case["cu_q"][-1])
    pad = 5
    padded = dict(case, q=np.concatenate([case["q"], np.full((pad, 8, 512), 0x7FC0, np.uint16)]))
    padded["cu_q"] = np.concatenate([case["cu_q"], [live + pad]]).astype(np.int32)
    padded["seq_lens"] = np.concatenate([case["seq_lens"], [0]]).astype(np.int32)
    padded["ori"].table = np.concatenate([case["ori"].table, case["ori"].table[:1]])
    padded["cmp"].table = np.concatenate([case["cmp"].table, case["cmp"].table[:1]])
    assert library().sharedkv_c8_set_merge_mode(mode) == 0
    try:
        dev, oscale, cscale, keep = to_device(padded)
        op = PreparedAttention(dev, oscale, cscale, splits=3, return_lse=True, query_group=group, tile_size=tile)
        op.out.fill_(float("nan"))
        op.lse.fill_(float("nan"))
        say(f"[grouped G{group} tile {tile} padding] merge mode {mode}")
        op.run()
        torch.cuda.synchronize()
    finally:
        library().sharedkv_c8_set_merge_mode(0)
    out, lse = bits_of(op.out), op.lse.cpu().numpy()
    assert not out[live:].any() and not lse[live:].any(), "padding rows are not zero"
    ref, ref_lse, _ = run_oracle(case, 3, query_group=group, tile=tile)
    assert np.array_equal(out[:live], ref)
    np.testing.assert_allclose(lse[:live], ref_lse, rtol=0, atol=2e-6)


@pytest.mark.parametrize("group", [2, 4])
def test_other_groupings_run_the_ungrouped_plan(group):
    """query_group 2 or 4 above eight heads or with explicit original slots
    runs (and reports) the ungrouped plan."""
    from npu_sparse_attn_sharedkv_int8 import c8_attention
    grouped = (c8_attention.VARIANT_DENSE_PAIRED, c8_attention.VARIANT_DENSE_PACKED,
               c8_attention.VARIANT_PAIRED_NARROW, c8_attention.VARIANT_PACKED_NARROW)
    for tag, case in (
            ("C4, 12 heads", workloads.make_case(108, 4, [2, 2], [3000, 5000], heads=12)),
            ("12 heads", workloads.make_case(109, 128, [4, 4], [3000, 5000], heads=12)),
            ("original slots", workloads.make_case(113, 128, [4, 2], [3000, 5000], ori_slots="draft"))):
        say(f"[grouped G{group}] {tag}: ungrouped")
        out, lse, op = run_hip(case, splits=3, query_group=group)
        assert op.query_group == 1 and op.tile_size == 128 and op.variant not in grouped, tag
        ref, _, _ = run_oracle(case, op.device_splits())
        assert np.array_equal(out, ref), tag
    # 256-key tiles exist only for the grouped plans.
    with pytest.raises(ValueError):
        run_hip(workloads.make_case(109, 128, [4, 4], [3000, 5000], heads=12), query_group=group, tile_size=256)
