"""The allocation-free attention entry point (launch_sharedkv_c8_noalloc)
against the allocating one, through the C ABI.

Calls in a row on the library's per-GPU scratch array, each bit-exact with
launch_sharedkv_c8_sparse / _dense on the same arguments (output and LSE), in
both merge placements:
- inputs shrinking from call to call (300 rows, which run c8_rows, then 40,
  then 4 twice);
- inputs growing across fused launches whose tickets would reach past an
  earlier launch's rows (4 rows at 2 partitions, 20 at 5, 100 at 3, 300 at 1,
  100 at 3 and 100 at 2), the serving pattern of a batch that grows.
A launch whose partition states exceed the array is rejected before any work.
"""
import ctypes
import sys

import numpy as np
import pytest

from tests import workloads
from tests.device_cases import bits_of, to_device

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def _launch_both(case, splits):
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    from npu_sparse_attn_sharedkv_int8.runtime import library
    lib = library()
    dev, oscale, cscale, keep = to_device(case)
    op = PreparedAttention(dev, oscale, cscale, splits=splits, return_lse=True)
    op.run()
    out2 = torch.full_like(op.out, float("nan"))
    lse2 = torch.full_like(op.lse, float("nan"))
    args = type(op.args).from_buffer_copy(op.args)
    args.out, args.lse = out2.data_ptr(), lse2.data_ptr()
    args.workspace = args.partial = 0          # ignored by the allocation-free entry
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.launch_sharedkv_c8_noalloc(max(1, op.blocks), ctypes.c_void_p(stream), ctypes.byref(args))
    assert rc == 0, rc
    torch.cuda.synchronize()
    return (bits_of(op.out), op.lse.cpu().numpy()), (bits_of(out2), lse2.cpu().numpy()), keep


def _run_sequence(lib, mode, launches):
    try:
        assert lib.sharedkv_c8_set_merge_mode(mode) == 0
        for name, case, splits in launches:
            say(f"[no-alloc] merge mode {mode}: {name}")
            (ref, ref_lse), (got, got_lse), _ = _launch_both(case, splits)
            assert np.array_equal(got, ref), name
            assert np.array_equal(got_lse.view(np.uint32), ref_lse.view(np.uint32)), name
    finally:
        lib.sharedkv_c8_set_merge_mode(0)


def _c4_rows(seed, rows, tokens_per_seq=2):
    seqs = rows // tokens_per_seq
    return workloads.make_case(seed, 4, [tokens_per_seq] * seqs, [1500 + 211 * i for i in range(seqs)],
                               index_mode="mixed")


@pytest.mark.parametrize("mode", [0, 1])
def test_no_alloc_entry_equals_allocating_entry(mode):
    from npu_sparse_attn_sharedkv_int8.runtime import library
    chunk = workloads.make_case(70, 4, [300], [4000], index_mode="holes")   # c8_rows: more rows than CUs
    big = workloads.make_case(71, 4, [2] * 20, list(range(3000, 3000 + 20 * 900, 900)), index_mode="mixed")
    small = workloads.make_case(72, 128, [1, 2, 1], [900, 5000, 130])
    _run_sequence(library(), mode, (("300 C4 rows, 1 partition", chunk, 1), ("40 C4 rows, 3 partitions", big, 3),
                                    ("4 C128 rows, 2 partitions", small, 2), ("4 C128 rows, 1 partition", small, 1)))


@pytest.mark.parametrize("mode", [0, 1])
def test_no_alloc_entry_across_growing_launches(mode):
    """Fused launches that grow: each later launch's tickets cover rows whose
    bytes an earlier launch's partition states would have held under a
    layout that placed the states right after the tickets."""
    from npu_sparse_attn_sharedkv_int8.runtime import library
    four = _c4_rows(80, 4)
    twenty = _c4_rows(81, 20)
    hundred = _c4_rows(82, 100)
    chunk = workloads.make_case(83, 4, [300], [4000], index_mode="uniform")   # c8_rows
    _run_sequence(library(), mode, (("4 C4 rows, 2 partitions", four, 2), ("20 C4 rows, 5 partitions", twenty, 5),
                                    ("100 C4 rows, 3 partitions", hundred, 3), ("300 C4 rows, 1 partition", chunk, 1),
                                    ("100 C4 rows, 3 partitions again", hundred, 3),
                                    ("100 C4 rows, 2 partitions", hundred, 2)))


def test_no_alloc_entry_rejects_launches_past_its_scratch():
    """505 rows at two partitions need more partition states than the array
    holds: rejected.  The case has capacity for all 505 rows (Q, output and
    LSE) and none of them is live (every seq_len 0), so a launch that got
    past a broken guard would only zero-fill its own output rows in bounds,
    never write a partition state; the test sees it as a changed output."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    from npu_sparse_attn_sharedkv_int8.runtime import library
    lib = library()
    limit = lib.sharedkv_c8_noalloc_scratch_bytes()
    assert limit == 16 << 20
    rows = 505
    assert 4096 + rows * 2 * 8 * 520 * 4 > limit >= 4096 + (rows - 1) * 2 * 8 * 520 * 4
    case = workloads.make_case(73, 4, [rows], [rows + 100], index_mode="uniform")
    dev, oscale, cscale, keep = to_device(case)
    op = PreparedAttention(dev, oscale, cscale, splits=2, return_lse=True)
    dev.seq_lens.zero_()                       # no live row: graph padding only
    args = type(op.args).from_buffer_copy(op.args)
    assert args.tokens == rows and args.splits == 2
    op.out.fill_(float("nan"))
    before = bits_of(op.out).copy()
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.launch_sharedkv_c8_noalloc(1, ctypes.c_void_p(stream), ctypes.byref(args)) == 1
    torch.cuda.synchronize()
    assert np.array_equal(bits_of(op.out), before)
