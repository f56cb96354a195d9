"""The serving adapter end to end on the GPU: compact page views, cache writes
through SharedKVLayer, attention through the same keyword contract vLLM
uses, streams, graph capture and the (out, lse) result shapes.

Flow of the reference's tests/npu/test_adapter.py:30-191: per ratio (window
only, C4, C128) a frozen scale file, caches written by the INT8 writer into
views of a sentinel-filled backing (compact stride 622592 B, layer offset
16384 B), attention compared with the checker on the op's own plan, two
query signs, a second stream with its own scratch, a captured graph replayed
after an eager call on the same op, the empty LSE, and sentinel bytes left
untouched.  The bar is this build's: BF16 outputs bit-exact with the checker
on the same plan, LSE within 2e-6.
"""
import sys
from types import SimpleNamespace

import numpy as np
import pytest

from tests import workloads
from tests.device_cases import bits_of, effective_splits, run_oracle, torch_bf16

pytestmark = pytest.mark.gpu

STRIDE, OFFSET = 622592, 16384


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def _expected(case, q_bits, splits):
    sub = dict(case)
    sub["q"] = q_bits
    ref, ref_lse, _ = run_oracle(sub, splits)
    return ref, ref_lse


def _check(case, q_bits, out, lse, splits, tag):
    ref, ref_lse = _expected(case, q_bits, effective_splits(case, splits))
    got = bits_of(out)
    mism = int((got != ref).sum())
    assert mism == 0, f"{tag}: {mism} BF16 mismatches"
    if lse is not None:
        np.testing.assert_allclose(lse.squeeze(-1).cpu().numpy(), ref_lse, rtol=0, atol=2e-6, err_msg=tag)


@pytest.mark.parametrize("ratio", [1, 4, 128])
def test_layer_end_to_end(ratio, tmp_path, monkeypatch):
    import torch
    from npu_sparse_attn_sharedkv_int8 import cache_layout, vllm_adapter

    say(f"[adapter] ratio={ratio}")
    case = workloads.make_case(991 + ratio, ratio, [5, 3], [260, 1300])
    prefix = f"unit.r{ratio}"
    kinds = ["ori"] + (["cmp"] if ratio != 1 else [])
    scales = {f"{prefix}.{k}": torch.from_numpy(case[k].scale) for k in kinds}
    path = tmp_path / "scales.pt"
    torch.save({"protocol": "sharedkv-c8-v1", "scales": scales}, path)
    monkeypatch.setenv("SHAREDKV_SCALES", str(path))
    vllm_adapter.load_scales.cache_clear()

    device = torch.device("cuda", torch.cuda.current_device())
    caches, raws, writes = {}, [], []
    for k in kinds:
        kind = case[k]
        raw = torch.full((kind.pages * STRIDE,), 73, dtype=torch.int8, device=device)
        cache = cache_layout.page_views(raw[OFFSET:], [(kind.pages, 32, 1, 512)], [torch.int8], STRIDE)[0]
        updates = torch_bf16(kind.values_bits, device).reshape(-1, 1, 512)
        slots = torch.arange(updates.shape[0], dtype=torch.int32, device=device)
        caches[k] = cache
        raws.append(raw)
        writes.append((cache, updates, slots, k))

    impl = SimpleNamespace(swa_cache_layer=SimpleNamespace(prefix=f"{prefix}.swa_cache"), head_dim=512,
                           turboquant=None, vllm_config=SimpleNamespace(parallel_config=SimpleNamespace(
                               decode_context_parallel_size=1, prefill_context_parallel_size=1)))
    state = vllm_adapter.runtime(impl)
    q0 = torch_bf16(case["q"], device)
    kw = dict(ori_kv=caches["ori"], cmp_kv=caches.get("cmp"),
              ori_block_table=torch.from_numpy(case["ori"].table).to(device),
              cmp_block_table=torch.from_numpy(case["cmp"].table).to(device) if ratio != 1 else None,
              cmp_sparse_indices=torch.from_numpy(case["cmp_indices"]).to(device) if ratio == 4 else None,
              cu_seqlens_q=torch.from_numpy(case["cu_q"]).to(device),
              seqused_kv=torch.from_numpy(case["seq_lens"]).to(device),
              sinks=torch.from_numpy(case["sink"]).to(device), cmp_ratio=ratio,
              ori_mask_mode=4, cmp_mask_mode=3, ori_win_left=127, ori_win_right=0,
              softmax_scale=case["softmax_scale"], layout_q="TND", layout_kv="PA_ND", return_softmax_lse=True)

    def run(query):
        for args in writes:
            state.write(*args)
        return state.attention(query, **kw)

    # Eager, two query signs (new Q pointer each time: the op is rebound).
    for multiplier in (1.0, -0.75):
        query = (q0 * multiplier).contiguous()
        out, lse = run(query)
        torch.cuda.synchronize()
        op = next(reversed(state.operators.values()))
        assert op.c8_dynamic and lse.shape == (*query.shape[:2], 1)
        _check(case, bits_of(query), out, lse, op.splits, f"eager x{multiplier}")
    for k in kinds:
        codes = torch.from_numpy(case[k].pool.reshape(case[k].pages, -1)[:, :32 * 512].copy())
        assert torch.equal(caches[k].reshape(case[k].pages, -1).cpu(), codes), k
    say(f"[adapter] ratio={ratio} eager ok")

    # A second stream gets its own stream key, op and scratch.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        key_side = vllm_adapter.stream_key(device)
        out_side, lse_side = state.attention(q0, **kw)
    side.synchronize()
    assert key_side != vllm_adapter.stream_key(device)
    side_op = next(reversed(state.operators.values()))
    _check(case, case["q"], out_side, lse_side, side_op.splits, "side stream")
    scratch_streams = {key[1] for key in vllm_adapter.StreamScratch.pools() if key[0] == device}
    assert key_side in scratch_streams or side_op.splits == 1

    # Capture writes + attention; an eager call on the same op between
    # capture and replay must not change the captured launch.
    query = q0.clone()
    capture = torch.cuda.Stream()
    capture.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(capture):
        with torch.cuda.graph(graph, stream=capture):
            g_out, g_lse = run(query)
    torch.cuda.current_stream().wait_stream(capture)
    captured = state.captured[-1]
    say(f"[adapter] ratio={ratio} captured (splits={captured.splits})")
    for i, sign in enumerate((1.0, -1.0, 1.0)):
        query.copy_(q0 * sign)
        negated = state.attention((-query).contiguous(), **kw)[0]       # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        _check(case, bits_of(query), g_out, g_lse, captured.splits, f"replay {i}")
        eager_op = next(reversed(state.operators.values()))
        _check(case, bits_of((-query).contiguous()), negated, None, eager_op.splits, f"eager {i}")
    say(f"[adapter] ratio={ratio} replays ok")

    _, empty = state.attention(q0, **{**kw, "return_softmax_lse": False})
    assert empty.shape == (0,) and empty.dtype == torch.float32 and empty.device == q0.device
    for cache, updates, slots, k in writes:
        state.write(cache, updates[:3], slots[:3], k)
    torch.cuda.synchronize()
    for k in kinds:
        codes = torch.from_numpy(case[k].pool.reshape(case[k].pages, -1)[:, :32 * 512].copy())
        assert torch.equal(caches[k].reshape(case[k].pages, -1).cpu(), codes), k
    for raw in raws:
        blocks = raw.view(-1, STRIDE).cpu()
        assert (blocks[:, :OFFSET] == 73).all() and (blocks[:, OFFSET + 16384:] == 73).all()
    assert all(op.case is None and op.out is None for op in state.operators.values())
    assert all(w.updates is None and w.slots is None for w in state.writers.values())
    del graph
    vllm_adapter.load_scales.cache_clear()


def test_scratch_allocator_grows_and_keys_by_stream():
    import torch
    from npu_sparse_attn_sharedkv_int8 import vllm_adapter
    device = torch.device("cuda", torch.cuda.current_device())
    a = vllm_adapter.scratch_allocator("t_ws", (100,), torch.uint8, device)
    b = vllm_adapter.scratch_allocator("t_ws", (60,), torch.uint8, device)
    assert a.data_ptr() == b.data_ptr() and b.shape == (60,)
    c = vllm_adapter.scratch_allocator("t_ws", (300,), torch.uint8, device)
    pool = vllm_adapter.StreamScratch.pools()[(device, vllm_adapter.stream_key(device))]
    assert c.data_ptr() != a.data_ptr() and [t.numel() for t in pool.buffers[("t_ws", torch.uint8)]] == [128, 512]
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        d = vllm_adapter.scratch_allocator("t_ws", (100,), torch.uint8, device)
    assert d.data_ptr() not in (a.data_ptr(), c.data_ptr())
    vllm_adapter.check_device(device)



def test_observer_on_device_reproduces_reference_calibrate(tmp_path):
    """The calibration observer on GPU tensors (device accumulators, one
    masked reduction per write), merged from two ranks' files: equal to the
    reference's CacheQuantization.calibrate output (golden calibrate.npz)
    bit for bit."""
    from tests.test_integration import observe_calibrate_vector
    got, want = observe_calibrate_vector(tmp_path, "cuda")
    np.testing.assert_array_equal(got.numpy(), want)
