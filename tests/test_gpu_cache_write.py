"""GPU parity of the INT8 cache writer (launch_cache_write) with the checker.

Bar: every byte of the pool equal to the CPU restatement's pool after the same
writes: codes of valid rows bit-exact, skipped rows (negative, past the pool,
offset past the page) leave their destination untouched, and guard bytes
outside each page's 16 KiB payload keep their value (73) at a serving page
stride.  Cases follow the reference's tests: cache_write.py:23-24 (4 slots
over 2 pages), test_queue.py:58-73 (repeated rebinds), test_adapter.py:186-189
(guard bytes at stride 622592), and BASELINE config 4 (4096 rows through a
random slot mapping).
"""
import sys

import numpy as np
import pytest

import oracle.oracle as ora
from tests import workloads

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def make_pool(pages, stride, fill=73):
    return np.full(pages * stride, fill, np.int8)


def run_writer(pool, pages, stride, updates_bits, slots, inverse, update_stride=512, three_d=False):
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedCacheWrite
    dev_pool = torch.from_numpy(pool.copy()).cuda()
    cache = dev_pool.as_strided((pages, 32, 1, 512), (stride, 512, 512, 1))
    rows = len(updates_bits)
    backing = np.zeros((rows, update_stride), np.uint16)
    backing[:, :512] = updates_bits
    upd = torch.from_numpy(backing.view(np.int16)).cuda().view(torch.bfloat16)[:, :512]
    if three_d:
        upd = upd.unsqueeze(1)
    sl = torch.from_numpy(np.ascontiguousarray(slots)).cuda()
    inv = torch.from_numpy(inverse).cuda()
    writer = PreparedCacheWrite(cache, upd, sl, inv)
    assert writer.run() is cache
    torch.cuda.synchronize()
    return dev_pool.cpu().numpy(), writer


@pytest.mark.parametrize("int64", [False, True])
@pytest.mark.parametrize("paired", [False, True])
@pytest.mark.parametrize("stride", [16384, 622592])
def test_writer_matches_checker(int64, paired, stride):
    rng = np.random.default_rng(int64 * 2 + paired + stride)
    pages, rows = 12, 300
    values = rng.standard_normal((rows, 512), dtype=np.float32)
    values[:, rng.choice(512, 16, replace=False)] *= 8
    bits = workloads.bf16_bits(values)
    scale = workloads.frozen_scale(workloads.bf16_value(bits))
    inverse = ora.inverse_scale(scale)
    flat = rng.permutation(pages * 32)[:rows].astype(np.int64)
    flat[5], flat[17], flat[40] = -1, pages * 32 + 3, -7
    if paired:
        slots = np.stack([flat // 32, flat % 32], 1)
        slots[17] = [pages, 1]
        slots[60] = [3, 32]
        slots[61] = [-1, 4]
    else:
        slots = flat
    slots = slots.astype(np.int64 if int64 else np.int32)
    pool = make_pool(pages, stride)
    say(f"[writer] int64={int64} paired={paired} stride={stride}")
    got, _ = run_writer(pool, pages, stride, bits, slots, inverse)
    expect = pool.copy()
    ora.cache_write(expect, stride, pages, 32, bits, slots, inverse, paired=paired)
    np.testing.assert_array_equal(got, expect)


def test_writer_row_strides_and_3d_updates():
    rng = np.random.default_rng(5)
    bits = workloads.bf16_bits(rng.standard_normal((40, 512), dtype=np.float32) * 2)
    inverse = ora.inverse_scale(workloads.frozen_scale(workloads.bf16_value(bits)))
    slots = rng.permutation(4 * 32)[:40].astype(np.int32)
    pool = make_pool(4, 20480)
    say("[writer] row stride 1024, [T,1,512] view")
    got, _ = run_writer(pool, 4, 20480, bits, slots, inverse, update_stride=1024, three_d=True)
    expect = pool.copy()
    ora.cache_write(expect, 20480, 4, 32, bits, slots, inverse)
    np.testing.assert_array_equal(got, expect)


def test_four_slots_across_two_pages():
    """examples/cache_write.py:23-24 of the reference: exact slot writes."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import CacheQuantization, PreparedCacheWrite
    cache = torch.zeros((2, 32, 1, 512), dtype=torch.int8, device="cuda")
    updates = (torch.arange(4 * 512, dtype=torch.float32).reshape(4, 512) % 23 - 11).to(torch.bfloat16).cuda()
    quant = CacheQuantization(torch.full((512,), 0.1))
    slots = torch.tensor([0, 31, 32, 63], dtype=torch.int32, device="cuda")
    PreparedCacheWrite(cache, updates, slots, quant.inverse_scale.cuda()).run()
    torch.cuda.synchronize()
    expect = quant.quantize(updates.cpu())
    flat = cache.cpu().reshape(64, 512)
    assert torch.equal(flat[[0, 31, 32, 63]], expect)
    mask = torch.ones(64, dtype=torch.bool)
    mask[[0, 31, 32, 63]] = False
    assert (flat[mask] == 0).all()


def test_rebind_writes_kat():
    """tests/npu/test_queue.py:58-73 of the reference: (v*10).round() over
    repeated rebinds of one prepared writer, token count changing."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedCacheWrite
    cache = torch.zeros((8, 32, 1, 512), dtype=torch.int8, device="cuda")
    inverse = torch.full((512,), 10.0, device="cuda")
    first = torch.zeros((4, 512), dtype=torch.bfloat16, device="cuda")
    writer = PreparedCacheWrite(cache, first, torch.zeros(4, dtype=torch.int32, device="cuda"), inverse)
    for step in range(32):
        n = 1 + step % 4
        v = torch.full((n, 512), (step % 25) / 10 - 1.2, dtype=torch.float32).to(torch.bfloat16).cuda()
        slots = torch.arange(step * 4, step * 4 + n, dtype=torch.int32, device="cuda") % 256
        writer._rebind_same_geometry(cache, v, slots)
        writer.run()
        torch.cuda.synchronize()
        got = cache.reshape(256, 512)[slots.long()].cpu()
        assert torch.equal(got, (v.cpu().float() * 10).round().clamp(-127, 127).to(torch.int8)), step


def test_config4_incremental_write():
    """4096 new rows through a random slot mapping into a
    stride-viewed pool that already holds data; bytes elsewhere unchanged."""
    rng = np.random.default_rng(4)
    pages, stride = 512, 20480
    values = rng.standard_normal((4096, 512), dtype=np.float32)
    values[:, rng.choice(512, 16, replace=False)] *= 8
    bits = workloads.bf16_bits(values)
    inverse = ora.inverse_scale(workloads.frozen_scale(workloads.bf16_value(bits)))
    slots = rng.permutation(pages * 32)[:4096].astype(np.int32)
    pool = rng.integers(-127, 128, pages * stride).astype(np.int8)
    say("[writer] config 4: 4096 rows")
    got, _ = run_writer(pool, pages, stride, bits, slots, inverse)
    expect = pool.copy()
    assert ora.cache_write(expect, stride, pages, 32, bits, slots, inverse) == 4096
    np.testing.assert_array_equal(got, expect)
