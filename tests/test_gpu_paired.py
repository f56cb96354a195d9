"""The paired plan (query_group 2) on the GPU against the CPU checker.

reference.py:224-323 with query_group 2: consecutive tokens 2j, 2j + 1 of a
request share one window list (positions max(0, p0 + 1 - 128) .. p1) and one
C128 compressed list (rows below (p1 + 1) / 128), each masking what it may
not see.  PreparedAttention(query_group=2) runs it through
launch_sharedkv_c8_dense_paired (c8_pairs: one work-group per group and
partition, the group's tiles fetched once).  Every launch is checked bit for
bit against oracle.tiled_attention(query_group=2) at the launch's
partitions, and shown to differ from the ungrouped plan where the window of
the second token makes the tiling differ.
"""
import sys

import numpy as np
import pytest

from tests import workloads
from tests.device_cases import bits_of, run_hip, run_oracle, to_device

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def check(case, splits, tag, merge_mode=0):
    out, lse, op = run_hip(case, splits=splits, query_group=2)
    assert op.query_group == 2 and op.device_splits() == op.splits
    ref, ref_lse, _ = run_oracle(case, op.splits, query_group=2)
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
]


@pytest.mark.parametrize("name,seed,ratio,queries,lengths", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("splits", [1, 2, 3, 5])
def test_paired_plan_matches_checker(name, seed, ratio, queries, lengths, splits):
    case = workloads.make_case(seed, ratio, queries, lengths)
    say(f"[paired] {name} splits {splits}")
    out, op = check(case, splits, f"{name} splits {splits}")
    if name == "mtp_pairs":
        # The second token's window starts one row later: the tiling, and so
        # the numerics, differ from the ungrouped plan.
        ungrouped, _, _ = run_oracle(case, splits)
        assert (out != ungrouped).any()


def test_paired_plan_heads_and_default_partitions():
    """Fewer than eight heads (the padding heads of the work-group are never
    written) and the library's own partition plan (choose_paired_splits)."""
    from npu_sparse_attn_sharedkv_int8 import c8_attention
    for heads in (4, 8):
        case = workloads.make_case(106, 128, [2] * 8, [2000 + 997 * i for i in range(8)], heads=heads)
        out, op = check(case, None, f"{heads} heads")
        assert op.splits == c8_attention.choose_paired_splits(16, 128)


@pytest.mark.parametrize("mode", [0, 1])
def test_paired_plan_padding_and_merge_modes(mode):
    """Graph-padding rows past the live tokens come back zero (NaN-poisoned
    Q), in both merge placements (fused, or the separate merge launch)."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    from npu_sparse_attn_sharedkv_int8.runtime import library
    case = workloads.make_case(107, 128, [2, 2, 3], [5000, 2600, 9000])
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
        op = PreparedAttention(dev, oscale, cscale, splits=3, return_lse=True, query_group=2)
        op.out.fill_(float("nan"))
        op.lse.fill_(float("nan"))
        say(f"[paired padding] merge mode {mode}")
        op.run()
        torch.cuda.synchronize()
    finally:
        library().sharedkv_c8_set_merge_mode(0)
    out, lse = bits_of(op.out), op.lse.cpu().numpy()
    assert not out[live:].any() and not lse[live:].any(), "padding rows are not zero"
    ref, ref_lse, _ = run_oracle(case, 3, query_group=2)
    assert np.array_equal(out[:live], ref)
    np.testing.assert_allclose(lse[:live], ref_lse, rtol=0, atol=2e-6)


def test_other_groupings_run_the_ungrouped_plan():
    """query_group 2 on C4 launches, query_group 4, or explicit original
    slots run (and report) the ungrouped plan."""
    from npu_sparse_attn_sharedkv_int8 import c8_attention
    case = workloads.make_case(108, 4, [2, 2], [3000, 5000], index_mode="uniform")
    out, lse, op = run_hip(case, splits=3, query_group=2)
    assert op.query_group == 1 and op.variant != c8_attention.VARIANT_DENSE_PAIRED
    ref, _, _ = run_oracle(case, op.device_splits())
    assert np.array_equal(out, ref)
    case = workloads.make_case(109, 128, [2, 2], [3000, 5000])
    out, lse, op = run_hip(case, splits=3, query_group=4)
    assert op.query_group == 1
