"""GPU parity of the HIP attention kernels against the CPU checker.

Bar: INT8 Q codes, int32 QK partials, P codes and int32 PV partials bit-exact
(debug entry); BF16 outputs bit-exact with the checker run on the same plan
(128-key tiles, the launch's KV partitions) and within max-abs 2e-2 /
mean-abs 2e-3 of the reference's own reference.py vectors; LSE within 2e-6
absolute of the checker (log is the device's own).
"""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

from tests import workloads
from tests.device_cases import (effective_splits, joint_flags, query_subcase, run_hip, run_hip_debug, run_oracle,
                                to_device, bits_of,
                                torch_bf16,
                                default_cmp_capacity)

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def kinds_with_rows(case):
    """[tokens, 2] mask: the window always has rows; the compressed kind has
    rows when its (compacted or raw) list is non-empty."""
    cu, lens = case["cu_q"], case["seq_lens"]
    live = int(cu[-1])
    used = np.zeros((live, 2), bool)
    used[:, 0] = True
    for b in range(len(lens)):
        for t in range(cu[b], cu[b + 1]):
            pos = int(lens[b]) - int(cu[b + 1]) + t
            count = (pos + 1) // case["ratio"] if case["ratio"] != 1 else 0
            if case["ratio"] == 4:
                ix = case["cmp_indices"][t, 0]
                used[t, 1] = bool(((ix >= 0) & (ix < count)).any()) if count < len(ix) else True
            elif case["ratio"] == 128:
                used[t, 1] = count > 0
    return used


def compare(case, out, lse, splits, rows=None, tag="", merge_mode=0):
    """HIP output of a launch of `case` planned at `splits` (run with the
    library in `merge_mode`) against the checker on the partitions the
    kernel actually ran (effective_splits)."""
    joint = joint_flags(case, splits, merge_mode)
    splits = effective_splits(case, splits, merge_mode)
    ref, ref_lse, _ = run_oracle(case if rows is None else query_subcase(case, rows), splits, joint=joint)
    got = out if rows is None else out[rows]
    got_lse = lse if rows is None else lse[rows]
    live = ref.shape[0] if rows is not None else int(case["cu_q"][-1])
    diff = got[:live] != ref[:live]
    assert not diff.any(), f"{tag}: {int(diff.sum())} BF16 mismatches of {diff.size}"
    np.testing.assert_allclose(got_lse[:live], ref_lse[:live], rtol=0, atol=2e-6, err_msg=tag)


DEBUG_CASES = [
    ("c128_ctx4096", 0, 128, [1], [4096], "uniform"),
    ("c4_ctx16384", 1, 4, [1], [16384], "uniform"),
    ("c4_holes", 2, 4, [2], [4200], "holes"),
    ("c4_mixed_compact", 3, 4, [1, 2], [1500, 900], "mixed"),
    ("c4_dups", 4, 4, [1], [4400], "dups"),
    ("c128_mixed", 5, 128, [2, 1, 3], [100, 300, 1300], "uniform"),
    ("r1_window", 6, 1, [2, 1], [90, 700], "uniform"),
]


@pytest.mark.parametrize("splits", [1, 3])
@pytest.mark.parametrize("name,seed,ratio,queries,lengths,mode", DEBUG_CASES, ids=[c[0] for c in DEBUG_CASES])
def test_integer_partials_bit_exact(name, seed, ratio, queries, lengths, mode, splits):
    case = workloads.make_case(seed, ratio, queries, lengths, index_mode=mode)
    say(f"[debug parity] {name} splits={splits}")
    out, lse, dumps, op, (cap, tiles) = run_hip_debug(case, splits=splits)
    ref, ref_lse, rd = run_oracle(case, splits, debug=True, cmp_capacity=cap, tile_capacity=tiles)
    live = int(case["cu_q"][-1])
    # The kernel encodes Q for a kind only when the kind has rows to read;
    # compare Q codes of the kinds that do.
    used = kinds_with_rows(case)
    for key in ("qcodes", "alpha"):
        np.testing.assert_array_equal(dumps[key][:live][used], rd[key][:live][used], err_msg=f"{name} {key}")
    for key in ("scores", "probs", "values"):
        np.testing.assert_array_equal(dumps[key][:live], rd[key][:live], err_msg=f"{name} {key}")
    assert (out[:live] == ref[:live]).all(), name
    np.testing.assert_allclose(lse[:live], ref_lse[:live], rtol=0, atol=2e-6)


@pytest.mark.parametrize("name,seed,ratio,queries,lengths,mode", DEBUG_CASES, ids=[c[0] for c in DEBUG_CASES])
def test_default_plan_matches_checker(name, seed, ratio, queries, lengths, mode):
    """The production launch with its own KV-partition choice."""
    case = workloads.make_case(seed, ratio, queries, lengths, index_mode=mode)
    say(f"[parity] {name}")
    out, lse, op = run_hip(case)
    compare(case, out, lse, op.splits, tag=name)


SLOT_CASES = [
    # The reference's draft-slot shape (tests/npu/test_attention.py:37): window only,
    # four requests of five draft tokens, 256 slots per token.
    ("r1_draft", 51, 1, [5, 5, 5, 5], [8192, 700, 300, 4000], "draft", 256),
    ("c4_draft", 52, 4, [3, 2], [9000, 2000], "draft", 256),
    ("c128_shuffled", 53, 128, [2, 3], [5000, 900], "shuffled", 256),
    ("r1_pool", 54, 1, [2, 1], [300, 90], "pool", 384),
    # 8 slot tiles + 8 C4 tiles: with one partition, two chunks of row codes.
    ("c4_pool_wide", 55, 4, [2], [20000], "pool", 1024),
]


@pytest.mark.parametrize("splits", [None, 1, 3])
@pytest.mark.parametrize("name,seed,ratio,queries,lengths,slots,topk", SLOT_CASES, ids=[c[0] for c in SLOT_CASES])
def test_explicit_original_slots_match_checker(name, seed, ratio, queries, lengths, slots, topk, splits):
    """Explicit physical original slots (draft/MTP ori_indices,
    reference.py:236-239, 285): holes masked in place, no block table."""
    case = workloads.make_case(seed, ratio, queries, lengths, ori_slots=slots, ori_topk=topk)
    say(f"[slots] {name} splits={splits}")
    out, lse, op = run_hip(case, splits=splits)
    compare(case, out, lse, op.splits, tag=name)


@pytest.mark.parametrize("mode,ratio", [("window", 1), ("shuffled", 128), ("pool", 4)])
def test_explicit_slot_partials_bit_exact(mode, ratio):
    """Debug entry with one slot tile: Q codes, int32 QK partials, P codes
    and int32 PV partials equal the checker's."""
    case = workloads.make_case(56, ratio, [1, 1], [700, 3000], ori_slots=mode, ori_topk=128)
    say(f"[slots debug] {mode} ratio={ratio}")
    out, lse, dumps, op, (cap, tiles) = run_hip_debug(case, splits=2)
    ref, ref_lse, rd = run_oracle(case, 2, debug=True, cmp_capacity=cap, tile_capacity=tiles)
    used = kinds_with_rows(case)
    for key in ("qcodes", "alpha"):
        np.testing.assert_array_equal(dumps[key][used], rd[key][used], err_msg=key)
    for key in ("scores", "probs", "values"):
        np.testing.assert_array_equal(dumps[key], rd[key], err_msg=key)
    assert (out == ref).all()
    np.testing.assert_allclose(lse, ref_lse, rtol=0, atol=2e-6)


HEAD_CASES = [
    ("h1_c4", 61, 4, [2, 1], [3000, 900], 1, None),
    ("h4_c128", 62, 128, [1, 2], [5000, 700], 4, None),
    ("h12_r1", 63, 1, [3], [400], 12, None),
    ("h16_c4", 64, 4, [2, 2], [9000, 3000], 16, None),
    ("h24_c128_slots", 65, 128, [2], [2000], 24, "shuffled"),
    ("h128_c4", 66, 4, [1], [6000], 128, None),
]


@pytest.mark.parametrize("splits", [None, 1, 3])
@pytest.mark.parametrize("name,seed,ratio,queries,lengths,heads,slots", HEAD_CASES, ids=[c[0] for c in HEAD_CASES])
def test_head_counts_match_checker(name, seed, ratio, queries, lengths, heads, slots, splits):
    """1..128 heads in groups of eight per work-group; above eight heads
    without Q/P residuals (reference.py:221-222)."""
    case = workloads.make_case(seed, ratio, queries, lengths, heads=heads, ori_slots=slots, ori_topk=256)
    say(f"[heads] {name} splits={splits}")
    out, lse, op = run_hip(case, splits=splits)
    compare(case, out, lse, op.splits, tag=name)


@pytest.mark.parametrize("mode", [0, 1])
def test_head_groups_with_both_merge_placements(mode):
    from npu_sparse_attn_sharedkv_int8.runtime import library
    lib = library()
    try:
        assert lib.sharedkv_c8_set_merge_mode(mode) == 0
        case = workloads.make_case(67, 4, [2, 3], [4000, 2500], heads=20, index_mode="mixed")
        for splits in (2, 5):
            say(f"[heads merge mode {mode}] splits={splits}")
            out, lse, op = run_hip(case, splits=splits)
            compare(case, out, lse, splits, tag=f"heads 20 mode {mode} splits {splits}", merge_mode=mode)
    finally:
        lib.sharedkv_c8_set_merge_mode(0)


def _golden(name):
    from pathlib import Path
    return np.load(Path(__file__).resolve().parent / "golden" / "vectors" / f"{name}.npz")


@pytest.mark.parametrize("splits", [None, 1, 2])
@pytest.mark.parametrize("i", range(11))
def test_real_activations_match_checker(i, splits):
    """The reference's captured activations (tests/fixtures/activations) with
    the layer's frozen serving scales (data/scales_v1.pt), converted by
    tests/golden/make_fixtures.py: bit-exact with the checker, and inside the
    reference's gates against the sample's FP64 output (relative L2 < .04,
    min head cosine > .999; tests/npu/test_attention.py:56, 110)."""
    from pathlib import Path
    z = np.load(Path(__file__).resolve().parent / "golden" / "vectors" / "activations.npz")
    case = workloads.fixture_case(z, i)
    say(f"[real activations] {z[f'{i}_layer']} ratio {int(z[f'{i}_ratio'])} splits={splits}")
    out, lse, op = run_hip(case, splits=splits)
    compare(case, out, lse, op.splits, tag=str(z[f"{i}_layer"]))
    got = workloads.bf16_value(out[0]).astype(np.float64)
    want = z[f"{i}_reference"]
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    cos = ((got * want).sum(-1) / (np.linalg.norm(got, axis=-1) * np.linalg.norm(want, axis=-1))).min()
    assert rel < 0.04 and cos > 0.999, (rel, cos)


GOLDEN_NAMES = sorted(p.stem for p in (Path(__file__).resolve().parent / "golden" / "vectors").glob("c*.npz")
                      if p.stem != "calibrate")


def _golden_plans(z):
    return [tuple(int(v) for v in p) + (0, 1)[len(p) - 5:] for p in z["plans"]]


@pytest.mark.parametrize("heads", [8, 4, 16])
def test_joint_c128_rows(heads):
    """One-partition C128 launches take joint rows (reference.py:254-267,
    joint_dense) for rows whose window and compressed lists fit one tile
    each: bit-exact with the checker's joint plan, and different from the
    tiled plan's numbers (so the joint path is the one that ran).  Longer
    rows (more than 128 compressed rows) and rows without compressed rows
    stay tiled in the same launch; above eight heads every row is tiled."""
    import oracle.oracle as ora
    case = workloads.make_case(61, 128, [1, 2, 1, 1], [4096, 2000, 100, 17000], heads=heads)
    say(f"[joint] heads {heads}")
    out, lse, op = run_hip(case, splits=1)
    host = workloads.oracle_case(case)
    tiled, tiled_lse, _ = ora.tiled_attention(host, tile=128, splits=1, return_lse=True)
    want, want_lse = tiled, tiled_lse
    if heads <= 8:
        want, want_lse, _ = ora.tiled_attention(host, tile=128, splits=1, return_lse=True, joint_dense=True)
        joint_rows = [0, 1, 2]                 # counts 32, 15, 15; row 3 has none, row 4 has 132
        assert (want[joint_rows] != tiled[joint_rows]).any()
        np.testing.assert_array_equal(want[3:], tiled[3:])
    diff = out != want
    assert not diff.any(), f"{int(diff.sum())} BF16 mismatches"
    np.testing.assert_allclose(lse, want_lse, rtol=0, atol=2e-6)
    # Three partitions: tiled, whatever the row.
    out3, _, op3 = run_hip(case, splits=3)
    ref3, _, _ = ora.tiled_attention(host, tile=128, splits=3, return_lse=True)
    assert np.array_equal(out3, ref3)


@pytest.mark.parametrize("mode,heads", [("dups", 8), ("mixed", 8), ("uniform", 8), ("one_key_duplicates", 8),
                                        ("extended_duplicates", 4), ("holes", 8), ("mixed", 16)])
def test_joint_c4_rows(mode, heads):
    """Short C4 rows (at most 128 compressed rows below the position) take
    joint rows at one partition (reference.py:246-267, joint_sparse): the
    compressed list is every row some valid top-k entry names, once, in row
    order, with log(multiplicity) added to its logits, and one softmax spans
    both kinds.  Bit-exact with the checker's joint plan and different from
    the tiled plan (so the joint path is the one that ran).  The launch
    mixes partial windows (positions below 127), rows with no compressed
    row, and a request of three tokens.  Three planned partitions re-plan to
    one (every live row fits).  One long row makes the launch tiled
    throughout, its short rows on their top-k lists (reference.py:246
    switches every C4 row of a joint_sparse plan to the dense list, so the
    joint plan is per launch).  Above eight heads every row is tiled."""
    import oracle.oracle as ora
    queries, lengths = [1, 2, 1, 1, 3, 1], [300, 515, 100, 40, 200, 2]
    case = workloads.make_case(71, 4, queries, lengths, heads=heads, index_mode=mode)
    host = workloads.oracle_case(case)
    say(f"[joint c4] {mode} heads {heads}")
    tiled, _, _ = ora.tiled_attention(host, tile=128, splits=1, return_lse=True)
    for splits in (1, 3):
        out, lse, op = run_hip(case, splits=splits)
        assert op.device_splits() == (1 if heads <= 8 else splits)
        compare(case, out, lse, splits, tag=f"{mode} splits {splits}")
        if heads <= 8 and mode != "uniform":
            assert (out != tiled).any()
    # A long row in the same launch: tiled rows at the launch's plan.
    long_case = workloads.make_case(72, 4, queries + [1], lengths + [4096], heads=heads, index_mode=mode)
    for splits in (1, 3):
        out, lse, op = run_hip(long_case, splits=splits)
        assert op.device_splits() == splits
        compare(long_case, out, lse, splits, tag=f"{mode} with a long row, splits {splits}")


@pytest.mark.parametrize("mode", ["dups", "mixed", "holes"])
def test_joint_c4_rows_with_a_serving_width_table(mode):
    """Short C4 rows behind a block table as wide as a serving table (1055
    pages: every sequence of a 135 000-token model) take the joint route when
    the launch comes through the small-launch entry (fewer than 24 tokens,
    the package's routing), which like the reference's small entry chooses
    from live lengths (c4_small.cpp:10-19): bit-exact with the checker's
    joint_sparse plan and different from the tiled plan.  Short rows of a
    24-token launch (the sparse entry) behind the same table stay tiled."""
    import oracle.oracle as ora
    from npu_sparse_attn_sharedkv_int8 import c8_attention

    def widen(case):
        narrow = case["cmp"].table
        wide = np.concatenate([narrow, np.tile(narrow[:, :1], (1, 1055 - narrow.shape[1]))], axis=1)
        case["cmp"].table = np.ascontiguousarray(wide)
        return case

    case = widen(workloads.make_case(73, 4, [1, 2, 1, 1, 3, 1], [300, 515, 100, 40, 200, 2], index_mode=mode))
    say(f"[joint c4, serving-width table] {mode}")
    out, lse, op = run_hip(case, splits=1)
    assert op.variant == c8_attention.VARIANT_SPARSE_SMALL and op.args.cmpTableWidth == 1055
    assert joint_flags(case, 1) == (False, True) and op.device_splits() == 1
    compare(case, out, lse, 1, tag=f"{mode} wide table")
    tiled, _, _ = ora.tiled_attention(workloads.oracle_case(case), tile=128, splits=1, return_lse=True)
    assert (out != tiled).any()
    case = widen(workloads.make_case(74, 4, [4] * 6, [300, 515, 100, 40, 200, 20], index_mode=mode))
    out, lse, op = run_hip(case, splits=1)
    assert op.variant == c8_attention.VARIANT_SPARSE and joint_flags(case, 1) == (False, False)
    compare(case, out, lse, 1, tag=f"{mode} wide table, 24 tokens")


@pytest.mark.parametrize("heads", [8, 12])
def test_persistent_rows(heads):
    """One-partition C4 launches of more rows than CUs run c8_rows: two
    four-wave work-groups per CU taking rows in turn (up to two rows each
    here; twelve heads make two rows per token, the second with four live
    heads).  Bit-exact with the checker.  The launch mixes a long request, short ones, a request
    listing more query tokens than its sequence length (a keyless row, which
    ends early and loads nothing ahead) and graph-padding rows, so
    work-groups pass between rows with and without keys."""
    case = workloads.make_case(81, 4, [600, 5, 2], [3000, 40, 1], heads=heads, index_mode="holes")
    pad = 12
    live = int(case["cu_q"][-1])
    case["q"] = np.concatenate([case["q"], np.full((pad, heads, 512), 0x7FC0, np.uint16)])
    case["cu_q"] = np.concatenate([case["cu_q"], [live + pad]]).astype(np.int32)
    case["seq_lens"] = np.concatenate([case["seq_lens"], [0]]).astype(np.int32)
    case["ori"].table = np.concatenate([case["ori"].table, case["ori"].table[:1]])
    case["cmp"].table = np.concatenate([case["cmp"].table, case["cmp"].table[:1]])
    case["cmp_indices"] = np.concatenate([case["cmp_indices"], np.full((pad, 1, 1024), -1, np.int32)])
    say(f"[persistent] heads {heads}: {(live + pad) * ((heads + 7) // 8)} rows")
    out, lse, op = run_hip(case, splits=1)
    assert op.splits == 1 and op.device_splits() == 1
    assert not out[live:].any() and not lse[live:].any(), "padding rows are not zero"
    keyless = live - 2                                   # position -1
    assert not out[keyless].any() and not lse[keyless].any()
    # The checker rejects the keyless row's request (reference.py:104-105):
    # every other live row is checked as its own one-token request.
    live_case = dict(case, q=case["q"][:live], cu_q=case["cu_q"][:-1], seq_lens=case["seq_lens"][:-1],
                     cmp_indices=case["cmp_indices"][:live])
    rows = [r for r in range(live) if r != keyless]
    compare(live_case, out[:live], lse[:live], 1, rows=rows, tag=f"persistent heads {heads}")


@pytest.mark.parametrize("ratio,lengths,heads", [
    (128, [20000, 40, 1], 8),    # tiled rows of 151-156 compressed rows, short rows, a keyless row
    (128, [16990, 300, 1], 8),   # rows of 128 compressed rows (joint) and of 129-132 (tiled) in one chunk
    (128, [3000, 140, 1], 8),    # joint rows (1-23 compressed rows) and window-only rows (position < 127)
    (128, [20000, 40, 1], 12),   # two rows per token, no residual codes: tiled
    (1, [3000, 40, 1], 8),       # window-only cache
    (1, [3000, 40, 1], 12),      # window-only, two rows per token (c8_rows head groups)
])
def test_persistent_dense_rows(ratio, lengths, heads):
    """One-partition C128 and window-only launches of more rows than CUs:
    window-only launches run c8_rows (two four-wave work-groups per CU taking
    rows in turn), C128 launches one work-group per row, rows of 1-128
    compressed rows being joint rows.  Bit-exact with the checker's plan for
    the launch (joint_dense per row at one partition), with graph-padding
    rows and a keyless row as in the C4 case."""
    from npu_sparse_attn_sharedkv_int8 import c8_attention
    case = workloads.make_case(82, ratio, [600, 5, 2], lengths, heads=heads)
    pad = 12
    live = int(case["cu_q"][-1])
    case["q"] = np.concatenate([case["q"], np.full((pad, heads, 512), 0x7FC0, np.uint16)])
    case["cu_q"] = np.concatenate([case["cu_q"], [live + pad]]).astype(np.int32)
    case["seq_lens"] = np.concatenate([case["seq_lens"], [0]]).astype(np.int32)
    case["ori"].table = np.concatenate([case["ori"].table, case["ori"].table[:1]])
    if case["cmp"] is not None:
        case["cmp"].table = np.concatenate([case["cmp"].table, case["cmp"].table[:1]])
    rows = (live + pad) * ((heads + 7) // 8)
    say(f"[persistent dense] ratio {ratio}, lengths {lengths}, heads {heads}: {rows} rows")
    out, lse, op = run_hip(case, splits=1)
    assert op.splits == 1 and op.device_splits() == 1 and rows > c8_attention.CORES
    assert not out[live:].any() and not lse[live:].any(), "padding rows are not zero"
    keyless = live - 2                                   # position -1
    assert not out[keyless].any() and not lse[keyless].any()
    live_case = dict(case, q=case["q"][:live], cu_q=case["cu_q"][:-1], seq_lens=case["seq_lens"][:-1])
    compare(live_case, out[:live], lse[:live], 1, rows=[r for r in range(live) if r != keyless],
            tag=f"persistent dense ratio {ratio} heads {heads}")
    if ratio == 128 and heads == 8 and lengths[0] == 16990:
        # Both routes of the straddling chunk are taken: the tiled plan of
        # the same launch differs on the joint rows only.
        import oracle.oracle as ora
        chunk = query_subcase(live_case, list(range(600)))
        tiled, _, _ = ora.tiled_attention(workloads.oracle_case(chunk), tile=128, splits=1, return_lse=True)
        first = [t for t in range(600) if (16990 - 600 + t + 1) // 128 <= 128]
        rest = [t for t in range(600) if t not in first]
        assert first and rest and (out[first] != tiled[first]).any()
        assert not (out[rest] != tiled[rest]).any()


def test_rows_graph_c128_replayed_with_few_live_sequences():
    """A C128 decode launch of 256 requests x 2 tokens (512 one-partition
    rows) captured once and replayed with 256, 16, 64 and 3 live requests of
    16.6-30 K tokens (re-planned into partitions merged in the launch, spread
    over every XCD), then with 16 live requests of at most 16 511 tokens (a
    joint-plan launch: one partition per row, every row joint).  Outputs, LSE and partition states
    are NaN-poisoned before each state; padding rows come back zero, live
    rows bit-exact with the checker on the device plan."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    cap = 256
    rng = np.random.default_rng(34)
    long_lengths = [int(n) for n in rng.integers(16600, 30000, cap)]
    short_lengths = [int(n) for n in rng.integers(200, 16511, cap)]
    full = workloads.make_case(94, 128, [2] * cap, long_lengths)
    dev, oscale, cscale, keep = to_device(full)
    op = PreparedAttention(dev, oscale, cscale, return_lse=True)
    assert op.splits == 1 and op.partial is not None
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        op.run()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            op.run()
    torch.cuda.current_stream().wait_stream(stream)
    for batch, lengths in ((cap, long_lengths), (16, long_lengths), (64, long_lengths), (3, long_lengths),
                           (16, short_lengths)):
        cu = np.array([2 * min(b, batch) for b in range(cap + 1)], np.int32)
        lens = np.array(lengths[:batch] + [0] * (cap - batch), np.int32)
        q = full["q"].copy()
        q[2 * batch:] = 0x7FC0
        dev.q.copy_(torch_bf16(q, "cuda"))
        dev.cu_q.copy_(torch.from_numpy(cu))
        dev.seq_lens.copy_(torch.from_numpy(lens))
        op.out.fill_(float("nan"))
        op.lse.fill_(float("nan"))
        op.partial.fill_(float("nan"))
        torch.cuda.synchronize()
        plan = effective_splits(dict(full, q=q, cu_q=cu, seq_lens=lens), op.splits)
        assert (plan > 1) == (batch < cap and lengths is long_lengths), (batch, plan)
        say(f"[rows graph c128] {batch} live requests, {plan} partition(s)")
        graph.replay()
        torch.cuda.synchronize()
        out, lse = bits_of(op.out), op.lse.cpu().numpy()
        live = 2 * batch
        assert not out[live:].any() and not lse[live:].any(), "padding rows are not zero"
        assert not op.workspace.any(), "merge tickets must return to zero"
        sub = dict(full, q=q[:live], cu_q=cu[:batch + 1], seq_lens=lens[:batch])
        ref, ref_lse, _ = run_oracle(sub, plan)
        diff = out[:live] != ref
        assert not diff.any(), f"{batch} live: {int(diff.sum())} BF16 mismatches"
        np.testing.assert_allclose(lse[:live], ref_lse, rtol=0, atol=2e-6)
    del graph


@pytest.mark.parametrize("name", GOLDEN_NAMES)
def test_against_reference_vectors(name):
    """HIP output vs reference.py's own tiled_quantized_reference output on
    every stored plan: 64-512-key tiles, 1-5 partitions, the joint rows, the
    dense C4 multiplicity list and query groups, i.e. also the plans the
    reference's device picks for these shapes (512-key tiles, config 0's
    joint row, paired query groups).  The HIP launch runs its own plan
    (128-key tiles, one partition); every stored output is within the
    BASELINE tolerance of it (BF16 mean-abs 2e-3, max-abs 2e-2 or one BF16
    ulp of the reference value, whichever is larger; LSE within 2e-3).
    Where a stored plan is one the HIP launch can run (128-key ungrouped
    with the same joint rows, or query groups of 2 or 4 on 128- or 256-key
    tiles through the grouped entries: c4_prefill G2 and G4, c4_pairs G2 at
    128 and 256 keys, c4_raw_holes, c128_mixed and c1_group G2, c128_pairs
    G2 at 256 keys) the HIP launch also runs that plan's partitions and equals
    reference.py bit for bit except rare one-ulp exp flips (at most 0.1 %),
    LSE within 1e-5.
    Above eight heads (no residual codes) only the same-plan check applies."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention, SharedKVCase, c8_attention
    z = _golden(name)
    dev = "cuda"
    pool = lambda key, stride: torch.from_numpy(z[key]).to(dev).as_strided(  # noqa: E731
        (len(z[key]) // stride, 32, 1, 512), (stride, 512, 512, 1))
    ratio = int(z["ratio"])
    case = SharedKVCase(
        q=torch.from_numpy(z["q"].view(np.int16)).to(dev).view(torch.bfloat16),
        ori=pool("ori_pool", int(z["ori_stride"])), ori_block_table=torch.from_numpy(z["ori_table"]).to(dev),
        cu_q=torch.from_numpy(z["cu_q"]).to(dev), seq_lens=torch.from_numpy(z["seq_lens"]).to(dev),
        sink=torch.from_numpy(z["sink"]).to(dev),
        cmp=pool("cmp_pool", int(z["cmp_stride"])) if ratio != 1 else None,
        cmp_block_table=torch.from_numpy(z["cmp_table"]).to(dev) if ratio != 1 else None,
        cmp_indices=torch.from_numpy(z["cmp_indices"]).to(dev) if "cmp_indices" in z.files else None,
        ratio=ratio, window=int(z["window"]), softmax_scale=float(z["softmax_scale"]),
        ori_indices=torch.from_numpy(z["ori_indices"]).to(dev) if "ori_indices" in z.files else None)
    live = int(z["cu_q"][-1])

    def launch(splits, query_group=None, tile_size=None):
        op = PreparedAttention(case, torch.from_numpy(z["ori_scale"]).to(dev),
                               torch.from_numpy(z["cmp_scale"]).to(dev) if ratio != 1 else None, splits=splits,
                               return_lse=True, query_group=query_group, tile_size=tile_size)
        assert op.query_group == (query_group or 1) and op.tile_size == (tile_size or 128)
        op.run()
        torch.cuda.synchronize()
        return bits_of(op.out)[:live], op.lse.cpu().numpy()[:live]

    def as_f32(bits):
        return (bits.astype(np.uint32) << 16).view(np.float32)

    say(f"[reference vectors] {name}: own plan (128-key tiles, 1 partition)")
    own, own_lse = launch(1)
    # Above eight heads reference.py turns the Q and P residual codes off
    # (reference.py:221-222); its own plans then differ from each other by up
    # to 5e-2, so only the same-plan comparison below applies there.
    residual = z["q"].shape[1] <= 8
    for i, (tile, splits, jd, js, _, dense, group) in enumerate(_golden_plans(z)):
        want = z[f"out_{i}"][:live]
        err = np.abs(as_f32(own) - as_f32(want))
        if residual:
            # One BF16 ulp of slack per element on top of 2e-2: reference.py's
            # own plans differ from each other by one ulp on outputs of
            # magnitude 4-16 (the outlier channels), 0.03-0.06 absolute
            # (golden c4_prefill, c1_group, c4_pairs).
            ulp = np.spacing(np.abs(as_f32(want))) * 65536
            assert (err <= np.maximum(2e-2, ulp)).all() and err.mean() <= 2e-3, \
                (name, i, float(err.max()), float(err.mean()))
            np.testing.assert_allclose(own_lse, z[f"lse_{i}"][:live], rtol=0, atol=2e-3,
                                       err_msg=f"{name} plan {i}")
        # Same-plan check where the stored plan is the HIP launch's plan at
        # `splits`: 128-key tiles, ungrouped, and joint rows (C128
        # joint_dense, C4 joint_sparse) exactly when the HIP plan takes them
        # (one partition, at most eight heads, no explicit slots).
        # The grouped plans (query_group 2 and 4, launch_sharedkv_c8_dense_paired
        # / _packed) cover the stored 128-key, non-joint G2 and G4 plans.
        joint_here = splits == 1 and c8_attention.joint_plan(ratio, z["q"].shape[1], "ori_indices" in z.files)
        stored_joint = bool(jd) if ratio == 128 else bool(js) if ratio == 4 else False
        grouped = group in (2, 4) and not jd and z["q"].shape[1] <= 8 and "ori_indices" not in z.files
        if dense or not (tile == 128 and group == 1 and stored_joint == joint_here or grouped and tile in (128, 256)):
            continue
        say(f"[reference vectors] {name} plan {i}: tile={tile}, splits={splits}, query group {group}")
        got, got_lse = launch(splits, query_group=group if grouped else None, tile_size=tile if grouped else None)
        assert (got == want).mean() >= 0.999, (name, i)
        np.testing.assert_allclose(got_lse, z[f"lse_{i}"][:live], rtol=0, atol=1e-5)


# ------------------------------------------------------ BASELINE configs

SERVING_STRIDE = 622592     # vLLM compact page stride (38 layers x 16 KiB)


def config_specs(index):
    """The BASELINE.json configs at full shape (caches generated on the GPU);
    each entry is one launch: (seed, ratio, queries, lengths, page stride)."""
    rng = np.random.default_rng(100 + (index if isinstance(index, int) else 99))
    if index == 0:
        return [(0, 128, [1], [4096], 16384)]
    if index == 1:
        return [(1, 4, [1], [16384], 16384)]
    if index == 2:
        lengths = rng.integers(2048, 65537, 32)
        return [(2, 4, [2] * 16, lengths[:16], SERVING_STRIDE), (12, 128, [2] * 16, lengths[16:], SERVING_STRIDE)]
    if index == 3:
        return [(3, 4, [2048], [32768], 16384)]
    if index == 4:
        lengths = rng.integers(65536, 131073, 64)
        return [(4, 4, [1] * 64, lengths, 20480), (14, 128, [1] * 64, lengths, 20480)]
    if index == "headline":
        lengths = rng.integers(2048, 65537, 32)
        return [(7, 4, [2] * 32, lengths, SERVING_STRIDE)]
    raise ValueError(index)


@pytest.mark.parametrize("index", [0, 1, 2, 3, 4, "headline"])
def test_baseline_configs(index):
    """Full-size launches; every row is checked when the launch has <= 128
    rows, else 96 rows spread over the launch (each recomputed alone by the
    checker with an identical selection)."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    from tests.device_cases import DeviceCase
    for part, (seed, ratio, queries, lengths, stride) in enumerate(config_specs(index)):
        tokens = int(sum(queries))
        say(f"[config {index}.{part}] tokens={tokens} ratio={ratio} stride={stride}")
        dc = DeviceCase(seed, ratio, queries, lengths, page_stride=stride)
        op = PreparedAttention(dc.dev, dc.ori_scale, dc.cmp_scale, return_lse=True)
        op.run()
        torch.cuda.synchronize()
        rows = None if tokens <= 128 else np.linspace(0, tokens - 1, 96).astype(int)
        compare(dc.host(), bits_of(op.out), op.lse.cpu().numpy(), op.splits, rows=rows,
                tag=f"config {index}.{part}")
        del op, dc
        torch.cuda.empty_cache()


@pytest.mark.parametrize("batch,tokens", [(300, 1), (160, 2)])
def test_many_row_decode_launches(batch, tokens):
    """Decode-shaped C4 launches of more rows than CUs (one partition, KV
    copies with the non-temporal policy, work-groups taking rows in turn),
    at the serving page stride: 96 rows spread over the launch against the
    checker."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    from tests.device_cases import DeviceCase
    rng = np.random.default_rng(200 + batch)
    lengths = rng.integers(2048, 16385, batch)
    say(f"[many-row decode] {batch} x {tokens}")
    dc = DeviceCase(30 + tokens, 4, [tokens] * batch, lengths, page_stride=SERVING_STRIDE)
    op = PreparedAttention(dc.dev, dc.ori_scale, dc.cmp_scale, return_lse=True)
    assert op.splits == 1
    op.run()
    torch.cuda.synchronize()
    rows = np.linspace(0, batch * tokens - 1, 96).astype(int)
    compare(dc.host(), bits_of(op.out), op.lse.cpu().numpy(), op.splits, rows=rows, tag=f"{batch} x {tokens}")


@pytest.mark.parametrize("heads", [12, 16])
def test_many_row_decode_launches_with_head_groups(heads):
    """Decode-shaped C4 launches of more rows than CUs with more than eight
    heads (rows = tokens x groups of eight heads; non-temporal copies, no
    residual codes): 64 tokens spread over the launch against the checker."""
    batch, tokens = 150, 2
    rng = np.random.default_rng(300 + heads)
    lengths = [int(x) for x in rng.integers(200, 3000, batch)]
    case = workloads.make_case(310 + heads, 4, [tokens] * batch, lengths, heads=heads, index_mode="holes")
    say(f"[many-row decode] {batch} x {tokens}, {heads} heads")
    out, lse, op = run_hip(case, splits=None)
    assert op.splits == 1
    rows = np.linspace(0, batch * tokens - 1, 64).astype(int)
    compare(case, out, lse, op.splits, rows=rows, tag=f"{heads} heads")


@pytest.mark.parametrize("mode,heads", [(0, 8), (1, 8), (0, 12), (1, 12)])
def test_padded_graph_rows_are_zero_and_guards_hold(mode, heads):
    """Capacity rows past the live tokens (seq_len 0 / cu_q sentinel) are
    zero-filled; bytes around the output and LSE are untouched; with either
    merge placement (the separate merge launch must leave padded rows and
    rows finalized by one partition alone)."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    from npu_sparse_attn_sharedkv_int8.runtime import library
    assert library().sharedkv_c8_set_merge_mode(mode) == 0
    try:
        _padded_rows_case(heads, mode)
    finally:
        library().sharedkv_c8_set_merge_mode(0)


def _padded_rows_case(heads=8, mode=0):
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    case = workloads.make_case(21, 4, [2, 1, 0, 0], [3000, 700, 0, 0], index_mode="mixed", heads=heads)
    live = int(case["cu_q"][-1])
    # Capacity of 6 query rows: append 3 NaN-poisoned padding rows.
    q = np.concatenate([case["q"], np.full((3, heads, 512), 0x7FC0, np.uint16)])
    padded = dict(case, q=q, cmp_indices=np.concatenate([case["cmp_indices"],
                                                        np.full((3, 1, 1024), -1, np.int32)]))
    padded["cu_q"] = np.array([0, 2, 3, 6, 6], np.int32)      # graph pads a synthetic request
    padded["seq_lens"] = np.array([3000, 700, 0, 0], np.int32)
    dev, oscale, cscale, keep = to_device(padded)
    guard_out = torch.full((6 + 2, heads, 512), 123, dtype=torch.bfloat16, device="cuda")
    guard_lse = torch.full((6 + 2, heads), 123, dtype=torch.float32, device="cuda")
    say(f"[padding] capacity 6, live 3, heads {heads}")
    op = PreparedAttention(dev, oscale, cscale, output=guard_out[1:-1], lse_output=guard_lse[1:-1], splits=4)
    op.run()
    torch.cuda.synchronize()
    assert (guard_out[[0, -1]].float().cpu() == 123).all() and (guard_lse[[0, -1]].cpu() == 123).all()
    assert (op.out[live:].float().cpu() == 0).all() and (op.lse[live:].cpu() == 0).all()
    # Fused launches hand the padding rows' work-groups to the live rows.
    splits = op.device_splits(merge_mode=mode)
    # 3 (or 6) live rows of at most 1 + ceil(750 / 128) = 7 tiles: one
    # partition per tile, as an eager launch of those rows would choose.
    assert splits == (4 if mode else 7), splits
    compare(case, bits_of(op.out)[:live], op.lse.cpu().numpy()[:live], splits, tag="padding")


def test_metadata_views_and_scratch_guards():
    """Request metadata, block tables and indices passed as views at offset
    pointers inside buffers filled with -777, and workspace / partition
    scratch carved out of 0xA5-filled buffers: the results equal the checker,
    nothing outside the views is touched, and the workspace is zero again
    after each launch.  Flow of the reference's tests/npu/test_metadata_views.py
    :14-58 and the guard bytes of tests/support/attention_cases.py:36-54."""
    import dataclasses
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    case = workloads.make_case(25, 4, [2, 1, 3], [5000, 900, 12000], index_mode="mixed")
    dev, oscale, cscale, keep = to_device(case)
    sentinels = []

    def inside(t, pad=3):
        """t copied into the middle of a -777-filled buffer (pad rows on each side)."""
        big = torch.full((t.shape[0] + 2 * pad, *t.shape[1:]), -777, dtype=t.dtype, device=t.device)
        big[pad:pad + t.shape[0]] = t
        sentinels.append((big, pad, t.shape[0]))
        return big[pad:pad + t.shape[0]]

    views = dataclasses.replace(dev, cu_q=inside(dev.cu_q), seq_lens=inside(dev.seq_lens),
                                ori_block_table=inside(dev.ori_block_table),
                                cmp_block_table=inside(dev.cmp_block_table), cmp_indices=inside(dev.cmp_indices))
    assert views.cu_q.data_ptr() != dev.cu_q.data_ptr() and views.cu_q.is_contiguous()
    scratch = []

    def allocator(name, shape, dtype, device):
        n = int(np.prod(shape)) * torch.empty((), dtype=dtype).element_size()
        raw = torch.full((n + 512,), 0xA5, dtype=torch.uint8, device=device)
        scratch.append((name, raw, n))
        return raw[256:256 + n].view(dtype).view(shape)

    op = PreparedAttention(views, oscale, cscale, return_lse=True, splits=3, scratch_allocator=allocator)
    assert {name for name, _, _ in scratch} == {"workspace", "partial"}
    for rep in range(2):
        say(f"[views] launch {rep}")
        op.run()
        torch.cuda.synchronize()
        compare(case, bits_of(op.out), op.lse.cpu().numpy(), op.splits, tag=f"views {rep}")
        for big, pad, rows in sentinels:
            host = big.cpu()
            assert (host[:pad] == -777).all() and (host[pad + rows:] == -777).all()
        for name, raw, n in scratch:
            host = raw.cpu()
            assert (host[:256] == 0xA5).all() and (host[256 + n:] == 0xA5).all(), name
            if name == "workspace":
                assert (host[256:256 + n] == 0).all(), "merge tickets must return to zero"


def test_graph_replay_with_changing_live_metadata():
    """One captured launch replayed while the device-side live metadata
    changes; every replay equals an eager launch on the same inputs."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    case = workloads.make_case(22, 4, [2, 2, 2], [5000, 2600, 9000], index_mode="uniform")
    dev, oscale, cscale, keep = to_device(case)
    op = PreparedAttention(dev, oscale, cscale, return_lse=True)
    eager = PreparedAttention(dev, oscale, cscale, return_lse=True, splits=op.splits)
    stream = torch.cuda.Stream()
    say("[graph] capture")
    with torch.cuda.stream(stream):
        op.run()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            op.run()
    variants = [(np.array([0, 2, 4, 6]), np.array([5000, 2600, 9000])),
                (np.array([0, 2, 4, -1]), np.array([5000, 2600, 0])),
                (np.array([0, 1, 2, 2]), np.array([4000, 2600, 0])),
                (np.array([0, 2, 4, 6]), np.array([5000, 2600, 9000]))]
    for i, (cu, lens) in enumerate(variants):
        dev.cu_q.copy_(torch.from_numpy(cu.astype(np.int32)))
        dev.seq_lens.copy_(torch.from_numpy(lens.astype(np.int32)))
        op.out.fill_(7)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager.run()
        torch.cuda.synchronize()
        say(f"[graph] replay {i}")
        assert torch.equal(op.out, eager.out), i
        assert torch.equal(op.lse, eager.lse), i


@pytest.mark.parametrize("cap", [64, 160])
def test_graph_at_capacity_replayed_at_fewer_live_sequences(cap):
    """One launch captured at a capacity of 64 one-token C4 requests (3
    partitions: 192 work-groups) or 160 (one partition per row, with the
    re-plan's partition states supplied), replayed with 64, 8, 16, 32, 64
    and 8 live requests (graph padding: the rest seq_len 0).  The kernel
    re-plans from the live metadata (the idle work-groups become partitions
    of the live rows, placed on every XCD); every replay is bit-exact with
    the checker on that plan, padding rows are zero, and eager work runs
    between replays."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention, c8_attention
    rng = np.random.default_rng(5)
    lengths = [int(n) for n in rng.integers(2100, 3000, cap)]      # 6-7 tiles a row
    case = workloads.make_case(26, 4, [1] * cap, lengths, index_mode="uniform")
    dev, oscale, cscale, keep = to_device(case)
    op = PreparedAttention(dev, oscale, cscale, return_lse=True)
    assert op.splits == (3 if cap == 64 else 1)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        op.run()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            op.run()
    torch.cuda.current_stream().wait_stream(stream)
    other = PreparedAttention(dev, oscale, cscale, return_lse=True, splits=2)
    expected = {}
    for i, live in enumerate((64, 8, 16, 32, 64, 8)):
        cu = np.array(list(range(live + 1)) + [live] * (cap - live), np.int32)
        lens = np.array(lengths[:live] + [0] * (cap - live), np.int32)
        plan = c8_attention.device_splits(op.splits, cap, 8, 4, 1024, cu, lens)
        assert plan == {64: {64: 3, 8: 7, 16: 7, 32: 5}, 160: {64: 2, 8: 7, 16: 7, 32: 5}}[cap][live], plan
        dev.cu_q.copy_(torch.from_numpy(cu))
        dev.seq_lens.copy_(torch.from_numpy(lens))
        op.out.fill_(float("nan"))
        op.lse.fill_(float("nan"))
        other.run()                                     # eager work between replays
        torch.cuda.synchronize()
        say(f"[capacity graph] replay {i}: {live} live, {plan} partitions")
        graph.replay()
        torch.cuda.synchronize()
        out, lse = bits_of(op.out), op.lse.cpu().numpy()
        assert not out[live:].any() and not lse[live:].any(), "padding rows are not zero"
        if live not in expected:
            expected[live] = run_oracle(query_subcase(case, np.arange(live)), plan)[:2]
        ref, ref_lse = expected[live]
        diff = out[:live] != ref
        assert not diff.any(), f"{live} live: {int(diff.sum())} BF16 mismatches"
        np.testing.assert_allclose(lse[:live], ref_lse, rtol=0, atol=2e-6)
    del graph


def test_graph_switches_between_joint_and_tiled_c128_plans():
    """One C128 launch captured at a capacity of 16 one-token requests (5
    partitions), replayed while the live metadata changes: all rows short
    (the device runs one partition per row with joint rows), one row longer
    than 128 compressed rows (the launch's own 5 partitions), and 4 live
    requests (joint again, the rest padding).  Each replay is bit-exact with
    the checker on the plan c8_attention.device_splits names."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention, c8_attention
    cap = 16
    lengths = [4096 + 311 * i for i in range(cap - 1)] + [20000]
    case = workloads.make_case(27, 128, [1] * cap, lengths)
    dev, oscale, cscale, keep = to_device(case)
    op = PreparedAttention(dev, oscale, cscale, return_lse=True)
    assert op.splits == 5
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        op.run()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            op.run()
    torch.cuda.current_stream().wait_stream(stream)
    short = lengths[:-1] + [3000]
    variants = [("all short", list(range(cap + 1)), short, 1),
                ("one long", list(range(cap + 1)), lengths, 5),
                ("4 live", list(range(5)) + [4] * (cap - 4), short[:4] + [0] * (cap - 4), 1),
                ("all short again", list(range(cap + 1)), short, 1)]
    for tag, cu, lens, want in variants:
        cu, lens = np.array(cu, np.int32), np.array(lens, np.int32)
        plan = c8_attention.device_splits(op.splits, cap, 8, 128, 0, cu, lens)
        assert plan == want, (tag, plan)
        dev.cu_q.copy_(torch.from_numpy(cu))
        dev.seq_lens.copy_(torch.from_numpy(lens))
        op.out.fill_(float("nan"))
        op.lse.fill_(float("nan"))
        torch.cuda.synchronize()
        say(f"[joint graph] {tag}: {plan} partition(s)")
        graph.replay()
        torch.cuda.synchronize()
        live = int(cu[-1])
        out, lse = bits_of(op.out), op.lse.cpu().numpy()
        assert not out[live:].any() and not lse[live:].any()
        sub = dict(case, cu_q=cu[:live + 1] if live < cap else cu, seq_lens=lens[:live] if live < cap else lens,
                   q=case["q"][:live])
        ref, ref_lse, _ = run_oracle(sub, plan)
        diff = out[:live] != ref
        assert not diff.any(), f"{tag}: {int(diff.sum())} BF16 mismatches"
        np.testing.assert_allclose(lse[:live], ref_lse, rtol=0, atol=2e-6)
    del graph


@pytest.mark.parametrize("ratio", [4, 128])
def test_one_graph_across_live_batch_and_length_states(ratio):
    """Flow of the reference's tests/npu/test_dynamic.py:18-80: one launch
    captured at a capacity of 8 requests x 6 query tokens, replayed three
    times per live state while the live batch and lengths change (8, 4, 1, 6
    and 0 live requests; equal and mixed lengths).  Before each state the Q
    rows, outputs, LSE and partition states are poisoned with NaN; padding
    rows must come back zero and live rows bit-exact with the checker on the
    plan the device picks.  (The merge tickets in the workspace are not
    poisoned: this build's fused merge keeps them, zero between launches.)"""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    maximum = 8193 if ratio == 4 else 40000       # the reference runs C128 to 135000; 40000 keeps the case small
    full = workloads.make_case(70 + ratio, ratio, [6] * 8, [maximum] * 8, index_mode="uniform")
    dev, oscale, cscale, keep = to_device(full)
    op = PreparedAttention(dev, oscale, cscale, return_lse=True)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        op.run()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            op.run()
    torch.cuda.current_stream().wait_stream(stream)
    short = [1024, 1027, 1028, 8192] if ratio == 4 else [16384, 20000, 24000, 32768]
    mixed = [1024, 8192, 1028, 4097, 777] if ratio == 4 else [12289, 39999, 16000, 9001, 25129]
    states = [(8, [short[0]] * 8), (4, [short[1]] * 4), (1, [short[2]]), (6, [short[3]] * 6), (0, []),
              (8, [maximum] * 8), (5, mixed)]
    for batch, lengths in states:
        cu = np.array([min(6 * b, 6 * batch) for b in range(9)], np.int32)
        lens = np.array(lengths + [0] * (8 - batch), np.int32)
        # Q rows of this state: the case's own; rows past the live ones NaN.
        q = full["q"].copy()
        q[6 * batch:] = 0x7FC0
        dev.q.copy_(torch_bf16(q, "cuda"))
        dev.cu_q.copy_(torch.from_numpy(cu))
        dev.seq_lens.copy_(torch.from_numpy(lens))
        if op.partial is not None:
            op.partial.fill_(float("nan"))
        op.out.fill_(float("nan"))
        op.lse.fill_(float("nan"))
        torch.cuda.synchronize()
        say(f"[dynamic c{ratio}] {batch} live, lengths {lengths[:3]}")
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        out, lse = bits_of(op.out), op.lse.cpu().numpy()
        live = 6 * batch
        assert not out[live:].any() and not lse[live:].any(), "padding rows are not zero"
        if not batch:
            continue
        sub = dict(full, q=q[:live], cu_q=cu[:batch + 1], seq_lens=lens[:batch])
        plan = effective_splits(dict(full, q=q, cu_q=cu, seq_lens=lens), op.splits)
        ref, ref_lse, _ = run_oracle(sub, plan)
        diff = out[:live] != ref
        assert not diff.any(), f"{batch} live: {int(diff.sum())} BF16 mismatches"
        np.testing.assert_allclose(lse[:live], ref_lse, rtol=0, atol=2e-6)
    del graph


def test_persistent_graph_across_live_states():
    """A one-partition C4 launch of more rows than CUs (c8_rows work-groups
    taking rows in turn) captured at a capacity of 4 requests x 100 query tokens and
    replayed twice per live state while the live batch and lengths change
    (4, 2, 1, 0 and 3 live requests).  Outputs and LSE are poisoned with NaN
    before each state; padding rows must come back zero and live rows
    bit-exact with the checker on the device plan (one live request of 100
    two-tile rows re-plans to two partitions merged in the launch)."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    full = workloads.make_case(91, 4, [100] * 4, [1600] * 4, index_mode="holes")
    dev, oscale, cscale, keep = to_device(full)
    op = PreparedAttention(dev, oscale, cscale, return_lse=True)
    assert op.splits == 1
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        op.run()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            op.run()
    torch.cuda.current_stream().wait_stream(stream)
    states = [(4, [1600] * 4), (2, [1200, 1599]), (1, [101]), (0, []), (3, [1600, 350, 999])]
    for batch, lengths in states:
        cu = np.array([min(100 * b, 100 * batch) for b in range(5)], np.int32)
        lens = np.array(lengths + [0] * (4 - batch), np.int32)
        q = full["q"].copy()
        q[100 * batch:] = 0x7FC0
        dev.q.copy_(torch_bf16(q, "cuda"))
        dev.cu_q.copy_(torch.from_numpy(cu))
        dev.seq_lens.copy_(torch.from_numpy(lens))
        op.out.fill_(float("nan"))
        op.lse.fill_(float("nan"))
        torch.cuda.synchronize()
        say(f"[persistent graph] {batch} live, lengths {lengths}")
        for _ in range(2):
            graph.replay()
        torch.cuda.synchronize()
        out, lse = bits_of(op.out), op.lse.cpu().numpy()
        live = 100 * batch
        assert not out[live:].any() and not lse[live:].any(), "padding rows are not zero"
        if not batch:
            continue
        sub = dict(full, q=q[:live], cu_q=cu[:batch + 1], seq_lens=lens[:batch])
        plan = effective_splits(dict(full, q=q, cu_q=cu, seq_lens=lens), op.splits)
        assert plan == (2 if batch == 1 else 1), plan
        ref, ref_lse, _ = run_oracle(sub, plan)
        diff = out[:live] != ref
        assert not diff.any(), f"{batch} live: {int(diff.sum())} BF16 mismatches"
        np.testing.assert_allclose(lse[:live], ref_lse, rtol=0, atol=2e-6)
    del graph


def test_rows_graph_at_capacity_replayed_with_few_live_sequences():
    """A decode launch of 256 requests x 2 tokens (512 one-partition rows:
    c8_rows) captured once and replayed with 256, 16, 64, 3 and 256 live
    requests.  With few live rows the kernel re-plans them into partitions
    (c8_attention.device_splits: 4 for 32 rows of at most 4 tiles, 2 for
    128 rows, 4 for 6 rows), spread
    over every XCD and merged in the launch.  Outputs, LSE and partition
    states are NaN-poisoned before each state and eager launches run between
    replays; padding rows come back zero, live rows bit-exact with the
    checker on the device plan, and the merge tickets return to zero."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    cap = 256
    rng = np.random.default_rng(33)
    lengths = [int(n) for n in rng.integers(600, 1600, cap)]
    full = workloads.make_case(93, 4, [2] * cap, lengths, index_mode="uniform")
    dev, oscale, cscale, keep = to_device(full)
    op = PreparedAttention(dev, oscale, cscale, return_lse=True)
    assert op.splits == 1 and op.partial is not None and op.partial.shape == (256, 8, 520)
    other = PreparedAttention(dev, oscale, cscale, return_lse=True, splits=2)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        op.run()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            op.run()
    torch.cuda.current_stream().wait_stream(stream)
    for batch, want in ((cap, 1), (16, 4), (64, 2), (3, 4), (cap, 1)):
        cu = np.array([2 * min(b, batch) for b in range(cap + 1)], np.int32)
        lens = np.array(lengths[:batch] + [0] * (cap - batch), np.int32)
        q = full["q"].copy()
        q[2 * batch:] = 0x7FC0
        dev.q.copy_(torch_bf16(q, "cuda"))
        dev.cu_q.copy_(torch.from_numpy(cu))
        dev.seq_lens.copy_(torch.from_numpy(lens))
        op.out.fill_(float("nan"))
        op.lse.fill_(float("nan"))
        op.partial.fill_(float("nan"))
        other.run()                                     # eager work between replays
        torch.cuda.synchronize()
        plan = effective_splits(dict(full, q=q, cu_q=cu, seq_lens=lens), op.splits)
        assert plan == want, (batch, plan)
        say(f"[rows graph] {batch} live requests, {plan} partition(s)")
        graph.replay()
        torch.cuda.synchronize()
        out, lse = bits_of(op.out), op.lse.cpu().numpy()
        live = 2 * batch
        assert not out[live:].any() and not lse[live:].any(), "padding rows are not zero"
        assert not op.workspace.any(), "merge tickets must return to zero"
        sub = dict(full, q=q[:live], cu_q=cu[:batch + 1], seq_lens=lens[:batch])
        ref, ref_lse, _ = run_oracle(sub, plan)
        diff = out[:live] != ref
        assert not diff.any(), f"{batch} live: {int(diff.sum())} BF16 mismatches"
        np.testing.assert_allclose(lse[:live], ref_lse, rtol=0, atol=2e-6)
    del graph


@pytest.mark.parametrize("ratio", [1, 4, 128])
def test_queued_launches_with_rapid_rebinding(ratio):
    """Flow of the reference's tests/npu/test_queue.py:17-60: per stream (the
    current one, then an auxiliary one), 32 launches of one operator, each
    rebound to a query its producer (a scaling kernel) has just written and
    to a fresh output, with the case reference dropped right after the
    launch; one synchronisation at the end.  Every output is bit-exact with
    the checker on its own query (the reference asserts closeness to its
    CPU model; this build's bar is bit equality)."""
    import dataclasses
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    case = workloads.make_case(2801, ratio, [6], [513])
    dev, oscale, cscale, keep = to_device(case)
    op = PreparedAttention(dev, oscale, cscale)
    factors = (1.0, -0.75, 0.5, -1.25)
    expected = []
    for factor in factors:
        q_bits = bits_of((dev.q * factor).contiguous())
        expected.append(run_oracle(dict(case, q=q_bits), effective_splits(case, op.splits))[0])
    for auxiliary in (False, True):
        stream = torch.cuda.Stream() if auxiliary else torch.cuda.current_stream()
        stream.wait_stream(torch.cuda.current_stream())
        outputs = []
        with torch.cuda.stream(stream):
            for index in range(32):
                query = dev.q * factors[index % 4]
                output = torch.empty_like(query)
                op._rebind_same_geometry(dataclasses.replace(dev, q=query), output=output)
                op.run()
                outputs.append(output)
                op.case = None
        stream.synchronize()
        say(f"[queue] ratio {ratio} auxiliary {auxiliary}: 32 launches")
        for index, output in enumerate(outputs):
            assert np.array_equal(bits_of(output), expected[index % 4]), (auxiliary, index)


def test_rebind_same_geometry():
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    a = workloads.make_case(23, 128, [1, 2], [3000, 8000])
    b = workloads.make_case(24, 128, [1, 2], [3100, 7000])
    # Same geometry: scales stay bound across a rebind (as in the reference),
    # so b is read with a's scales, and b's block tables take a's widths.
    for kind in ("ori", "cmp"):
        b[kind].scale = a[kind].scale
        table = np.zeros_like(a[kind].table)
        table[:, :b[kind].table.shape[1]] = b[kind].table
        b[kind].table = table
    dev_a, oa, ca, ka = to_device(a)
    dev_b, ob, cb, kb = to_device(b)
    op = PreparedAttention(dev_a, oa, ca, return_lse=True, splits=4)
    op.run()
    torch.cuda.synchronize()
    first, first_lse = bits_of(op.out), op.lse.cpu().numpy()
    out_b = torch.empty_like(dev_b.q)
    lse_b = torch.empty((3, 8), dtype=torch.float32, device="cuda")
    op._rebind_same_geometry(dev_b, output=out_b, lse_output=lse_b)
    say("[rebind]")
    op.run()
    torch.cuda.synchronize()
    compare(a, first, first_lse, 4, tag="rebind-a")
    compare(b, bits_of(out_b), lse_b.cpu().numpy(), 4, tag="rebind-b")


EDGE_SHAPES = [(7, 129), (13, 513), (49, 129), (65, 513), (97, 1023)]   # test_sparse_edges.py:31-33


@pytest.mark.parametrize("mode", ("dups", "holes") + workloads.EDGE_MODES)
def test_sparse_edge_selections_match_checker(mode):
    """The reference's sparse-edge selections (tests/npu/test_sparse_edges.py
    :52-75: duplicates, holes, empty, more selected entries than the causal
    extent, a single key, one key twice, a permutation) over its batch x
    length shapes, one query per request: BF16 bit-exact with the checker
    and LSE within 2e-6, on the host plan's partitions."""
    for i, (batch, length) in enumerate(EDGE_SHAPES):
        say(f"[edges] {mode} batch={batch} length={length}")
        case = workloads.make_case(600 + i, 4, [1] * batch, [length] * batch, index_mode=mode)
        out, lse, op = run_hip(case)
        compare(case, out, lse, op.splits, tag=f"{mode} {batch}x{length}")


def test_splits_variants_match_checker():
    case = workloads.make_case(25, 4, [2, 1], [20000, 700], index_mode="holes")
    for splits in (1, 2, 5, 9, 16):
        say(f"[splits] {splits}")
        out, lse, op = run_hip(case, splits=splits)
        compare(case, out, lse, splits, tag=f"splits {splits}")


@pytest.mark.parametrize("name,ratio,queries,lengths,heads,want", [
    ("c4_one_row", 4, [1], [16384], 8, 9),                     # config 1's shape
    ("c4_seven_tiles", 4, [2, 2], [3000, 2900], 8, 9),          # two partitions own no tile
    ("c4_twelve_heads", 4, [2, 1], [30000, 9000], 12, 9),       # 3 tokens x 2 head groups
    ("c128_unknown_length", 128, [2], [131072], 8, 16),          # nine tiles; the bound is 16
    ("c4_twelve_rows", 4, [2] * 6, [4000 + 5000 * i for i in range(6)], 8, 9),
    ("c4_thirteen_rows", 4, [1] * 13, [4000 + 3000 * i for i in range(13)], 8, 5),
])
def test_one_partition_per_tile_plans(name, ratio, queries, lengths, heads, want):
    """The library's plan for launches of at most 112 row tiles: one KV
    partition per tile (nine for C4 top-k rows; sixteen, the bound, for C128
    rows whose length the launch was not told), the fold above eight
    partitions; thirteen rows of nine tiles take five.
    Bit-exact with the checker on that plan."""
    from npu_sparse_attn_sharedkv_int8 import c8_attention
    case = workloads.make_case(77, ratio, queries, lengths, heads=heads)
    say(f"[one tile] {name}")
    out, lse, op = run_hip(case)
    assert op.splits == want, (name, op.splits)
    assert effective_splits(case, op.splits) == want
    compare(case, out, lse, op.splits, tag=name)


def test_long_c128_rows_span_two_code_chunks():
    """C128 rows longer than twelve tiles per partition (ctx 300000: 2343
    compressed rows, 20 tiles) rebuild their row codes in a second chunk."""
    case = workloads.make_case(29, 128, [1, 2], [300000, 180000])
    for splits in (1, 2, 3):
        say(f"[long c128] splits={splits}")
        out, lse, op = run_hip(case, splits=splits)
        compare(case, out, lse, splits, tag=f"long c128 splits {splits}")


def test_ctypes_and_bridge_launches_agree():
    """The compiled launch bridge (the default) and the ctypes binding of the
    same C ABI (SHAREDKV_USE_CTYPES=1) launch the same kernels: identical
    outputs, and both raise on a rejected argument block."""
    import ctypes
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention, runtime
    case = workloads.make_case(33, 4, [2, 1], [5000, 900], index_mode="mixed")
    dev, oscale, cscale, keep = to_device(case)
    op = PreparedAttention(dev, oscale, cscale, return_lse=True)
    outs = []
    for use_ctypes in (False, True):
        host = runtime._Host(runtime.library(), use_ctypes=use_ctypes)
        op.out.fill_(0)
        host.attention(op.argument_address, op.blocks, op.variant, op.device_index)
        torch.cuda.synchronize()
        outs.append(bits_of(op.out))
        bad = type(op.args).from_buffer_copy(op.args)
        bad.splits = 0                                   # rejected by the C ABI's checks
        with pytest.raises(RuntimeError, match="hipError_t"):
            host.attention(ctypes.addressof(bad), op.blocks, op.variant, op.device_index)
    assert np.array_equal(outs[0], outs[1])
    compare(case, outs[0], op.lse.cpu().numpy(), op.splits, tag="bridge")


def test_empty_launch_is_a_no_op():
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    case = workloads.make_case(26, 4, [1], [600])
    dev, oscale, cscale, keep = to_device(case)
    dev.q = dev.q[:0]
    dev.cmp_indices = dev.cmp_indices[:0]
    op = PreparedAttention(dev, oscale, cscale)
    assert op.blocks == 0
    assert op.run().shape == (0, 8, 512)
    torch.cuda.synchronize()


def test_planner_knobs_report_the_plan_that_ran():
    """The Ascend planner's knobs (attention.py:27-30 of the reference) are
    validated; the planner switches are not applied (query_group is, in
    test_gpu_paired.py), and the operator reports the plan that ran
    (tile_size, query_group, splits), the fields the reference's tests
    rebuild their oracle plan from."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    case = workloads.make_case(27, 4, [2, 2], [700, 3000], index_mode="uniform")
    dev, oscale, cscale, keep = to_device(case)
    plain = PreparedAttention(dev, oscale, cscale, return_lse=True)
    plain.run()
    for kw in ({"query_group": 1}, {"tile_size": 128, "max_seq_len": 1024}, {"adaptive_splits": True},
               {"trim_cube_tails": True, "dynamic_c4": True}):
        op = PreparedAttention(dev, oscale, cscale, return_lse=True, **kw)
        assert (op.tile_size, op.query_group, op.splits) == (128, 1, plain.splits), kw
        op.run()
        torch.cuda.synchronize()
        assert torch.equal(op.out, plain.out) and torch.equal(op.lse, plain.lse), kw
    for kw in ({"query_group": 3}, {"tile_size": 256}, {"splits": 0}):
        with pytest.raises(ValueError):
            PreparedAttention(dev, oscale, cscale, **kw)
    compare(case, bits_of(plain.out), plain.lse.cpu().numpy(), plain.splits, tag="knobs")


@pytest.mark.parametrize("mode", [0, 1])
def test_merge_modes_match_checker(mode):
    """Partition states folded by the last partition of each row (mode 0,
    device-coherent state exchange across XCDs) or by a second launch
    (mode 1): both bit-exact with the checker."""
    from npu_sparse_attn_sharedkv_int8.runtime import library
    lib = library()
    try:
        assert lib.sharedkv_c8_set_merge_mode(mode) == 0
        case = workloads.make_case(27, 4, [2] * 12, list(range(3000, 3000 + 12 * 700, 700)), index_mode="mixed")
        for splits in (2, 3, 7, 16):
            say(f"[merge mode {mode}] splits={splits}")
            out, lse, op = run_hip(case, splits=splits)
            compare(case, out, lse, splits, tag=f"mode {mode} splits {splits}", merge_mode=mode)
        # Rows whose tiles all sit in partition 0 (no compressed rows yet) are
        # finalized by it; the others fold fewer partitions than launched.
        # (The 17000-key request keeps the launch off the joint C128 plan.)
        short = workloads.make_case(28, 128, [2, 1, 3, 1], [60, 130, 900, 17000])
        for splits in (3, 16):
            say(f"[merge mode {mode}] short rows splits={splits}")
            out, lse, op = run_hip(short, splits=splits)
            compare(short, out, lse, splits, tag=f"mode {mode} short splits {splits}", merge_mode=mode)
    finally:
        lib.sharedkv_c8_set_merge_mode(0)


def test_xcd_local_state_exchange():
    """The fused merge passes a row's partition states through one XCD's L2
    when the dispatch probe shows that work-groups agreeing in blockIdx
    modulo 8 share an XCD; launches of several partitions then place every
    row with all its partitions on one XCD (the headline shape: 8 rows x 3
    partitions per XCD; one row x 5 partitions: all on XCD 0; 5 rows x 5:
    one row on each of five XCDs).  With the exchange disabled every row
    uses device-coherent stores and loads.  Every launch is bit-exact with
    the checker either way, and the probe reports the exchange in use on
    MI355X."""
    from npu_sparse_attn_sharedkv_int8.runtime import library
    lib = library()
    cases = [
        ("headline-like", workloads.make_case(29, 4, [2] * 32, [2048 + 1999 * i for i in range(32)],
                                              index_mode="uniform"), None),
        ("one row", workloads.make_case(32, 4, [1], [16384], index_mode="uniform"), 5),
        ("five rows", workloads.make_case(30, 4, [1, 2, 2], [16384, 9000, 40000], index_mode="mixed"), 5),
        ("C128 rows", workloads.make_case(31, 128, [2] * 16, [2048 + 3999 * i for i in range(16)]), None),
    ]
    try:
        results = {}
        for enable in (1, 0):
            assert lib.sharedkv_c8_set_xcd_local(enable) == 0
            for tag, case, splits in cases:
                say(f"[xcd local {enable}] {tag}")
                out, lse, op = run_hip(case, splits=splits)
                compare(case, out, lse, op.splits, tag=f"xcd local {enable} {tag}")
                results[(enable, tag)] = (out, lse)
        assert lib.sharedkv_c8_xcd_local() == 1, "dispatch probe did not enable the XCD-local exchange"
        for tag, _, _ in cases:
            assert np.array_equal(results[(1, tag)][0], results[(0, tag)][0]), tag
            assert np.array_equal(results[(1, tag)][1], results[(0, tag)][1]), tag
    finally:
        lib.sharedkv_c8_set_xcd_local(int(os.environ.get("SHAREDKV_XCD_LOCAL", "1")))
    assert lib.sharedkv_c8_set_xcd_local(2) != 0


@pytest.mark.parametrize("mode", [0, 1])
@pytest.mark.parametrize("ratio", [4, 128, 1])
def test_rows_with_negative_position_are_zero(mode, ratio):
    """A request listing more query tokens than its sequence length gives its
    first tokens a negative position (reference.py:104-105 rejects such
    metadata; the device reads nothing back, so it cannot).  Such a token has
    no keys: its output and LSE rows are zero, in both merge placements and
    at one and several partitions, and the other tokens are untouched (equal
    to the checker on their own positions).  Explicit original slots do not
    change the rule."""
    import torch
    from npu_sparse_attn_sharedkv_int8.runtime import library
    lib = library()
    case = workloads.make_case(31, ratio, [3, 2, 1], [1, 900, 40])   # positions -2, -1, 0 | 898, 899 | 39
    bad, good = [0, 1], [2, 3, 4, 5]
    ref, ref_lse, _ = run_oracle(query_subcase(case, good), 1)
    try:
        assert lib.sharedkv_c8_set_merge_mode(mode) == 0
        for splits in (1, 3):
            say(f"[negative positions] ratio {ratio} mode {mode} splits {splits}")
            dev, oscale, cscale, keep = to_device(case)
            from npu_sparse_attn_sharedkv_int8 import PreparedAttention
            op = PreparedAttention(dev, oscale, cscale, splits=splits, return_lse=True)
            op.out.fill_(float("nan"))
            op.lse.fill_(float("nan"))
            op.run()
            torch.cuda.synchronize()
            out, lse = bits_of(op.out), op.lse.cpu().numpy()
            assert not out[bad].any() and not lse[bad].any()
            if splits == 1:
                assert np.array_equal(out[good], ref)
                np.testing.assert_allclose(lse[good], ref_lse, rtol=0, atol=2e-6)
            else:
                compare(query_subcase(case, good), out[good], lse[good], splits, tag="negative positions",
                        merge_mode=mode)
    finally:
        lib.sharedkv_c8_set_merge_mode(0)


def test_repeated_fused_merges_on_changing_inputs():
    """One prepared operator rebound to new inputs 24 times in a row, without
    host synchronisation between launches; every launch is checked, so a stale
    partition state or a ticket left behind by an earlier launch would show."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    # The 17000-key request keeps the C128 launches off the joint plan (more
    # than 128 compressed rows), so they fold partitions too.
    cases = [workloads.make_case(40 + i, 128 if i % 2 else 4, [2, 1, 2], [2500 + 97 * i, 7000 - 55 * i, 17000])
             for i in range(4)]
    # Same geometry within a ratio: shared scales, block tables of one width.
    for first in (0, 1):
        group = cases[first::2]
        for kind in ("ori", "cmp"):
            width = max(c[kind].table.shape[1] for c in group)
            for c in group:
                c[kind].scale = group[0][kind].scale
                table = np.zeros((c[kind].table.shape[0], width), np.int32)
                table[:, :c[kind].table.shape[1]] = c[kind].table
                c[kind].table = table
    devs = [to_device(c) for c in cases]
    outs = []
    ops = {}
    for i in range(24):
        c = i % 4
        dev, oscale, cscale, _ = devs[c]
        ratio = cases[c]["ratio"]
        if ratio not in ops:
            ops[ratio] = PreparedAttention(dev, oscale, cscale, splits=5, return_lse=True)
        op = ops[ratio]
        out = torch.empty_like(dev.q)
        lse = torch.empty((dev.q.shape[0], 8), dtype=torch.float32, device="cuda")
        op._rebind_same_geometry(dev, output=out, lse_output=lse)
        op.run()
        outs.append((c, out, lse))
    torch.cuda.synchronize()
    say("[repeated fused merges] 24 launches")
    refs = {}
    for c, out, lse in outs:
        if c not in refs:
            refs[c] = run_oracle(cases[c], effective_splits(cases[c], 5))[:2]
        ref, ref_lse = refs[c]
        assert (bits_of(out) == ref).all(), c
        np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, rtol=0, atol=2e-6)
