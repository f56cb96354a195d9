"""Host side of the serving integration, without a GPU: calibration (observer,
merge, scale-file checks), the compact page planner, and the vLLM adapter and
plugin wiring driven with stand-in engine classes (vLLM is not installed
here; the reference drives its adapter with SimpleNamespace stand-ins too,
tests/npu/test_adapter.py:77-114).

Reference behaviour followed: the calibration workflow of docs/kv-cache.md:51-68
(marker-gated observation, rank_XX.pt payload, merge rule), the scale-file
checks of vllm_adapter.py:52-63, the sparse-attention keyword contract and
result of vllm_adapter.py:140-214, the plugin modes of vllm_plugin.py:13-30,
and the page planner of cache_layout.py:32-134.
"""
from dataclasses import dataclass
import json
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from npu_sparse_attn_sharedkv_int8 import cache_layout, calibration, vllm_adapter, vllm_plugin
from tests import workloads


# ------------------------------------------------------------ calibration

def _observer(tmp_path, collect=True):
    obs = calibration.CacheObserver(tmp_path)
    if collect:
        (tmp_path / "collect").touch()
    return obs


def test_observer_needs_the_marker(tmp_path):
    obs = _observer(tmp_path, collect=False)
    cache = torch.zeros(4, 32, 1, 512, dtype=torch.int8)
    obs.observe("model.layers.0.self_attn", "ori", cache, torch.ones(3, 512), torch.arange(3))
    assert obs.stats == {} and not (tmp_path / "rank_00.pt").exists()


def test_observer_counts_only_rows_the_writer_would_write(tmp_path):
    obs = _observer(tmp_path)
    cache = torch.zeros(2, 32, 1, 512, dtype=torch.int8)        # 64 slots
    rows = torch.zeros(5, 1, 512, dtype=torch.bfloat16)
    rows[:, 0, 7] = torch.tensor([1.0, -9.0, 3.0, 100.0, -2.5], dtype=torch.bfloat16)
    flat = torch.tensor([0, 63, -1, 64, 5])                        # -1 and 64 are skipped
    obs.observe("p", "ori", cache, rows, flat)
    peak, count = obs.stats["p.ori"]
    assert float(peak[7]) == 9.0 and int(count) == 3 and float(peak[:7].abs().sum()) == 0
    paired = torch.tensor([[0, 0], [1, 31], [2, 0], [1, 32], [0, -1]])   # only the first two are inside
    obs.observe("p", "ori", cache, rows, paired)
    peak, count = obs.stats["p.ori"]
    assert float(peak[7]) == 9.0 and int(count) == 5
    obs.flush()
    saved = torch.load(tmp_path / "rank_00.pt", weights_only=True)
    assert saved["version"] == 1 and saved["stats"]["p.ori"]["rows"] == 5
    assert float(saved["stats"]["p.ori"]["maximum"][7]) == 9.0


def test_observer_rejects_other_widths_and_nonfinite(tmp_path):
    obs = _observer(tmp_path)
    cache = torch.zeros(1, 32, 1, 512, dtype=torch.int8)
    with pytest.raises(ValueError):
        obs.observe("p", "ori", cache, torch.ones(2, 256), torch.arange(2))
    obs.observe("p", "cmp", cache, torch.full((1, 512), float("inf")), torch.arange(1))
    with pytest.raises(RuntimeError):
        obs.flush()
    obs.pending = False


def test_observer_checkpoints_when_the_marker_goes(tmp_path, monkeypatch):
    """The marker is looked up at most once per MARKER_POLL_SECONDS; once it
    is gone the next observation checkpoints what was collected and records
    nothing more."""
    monkeypatch.setattr(calibration, "MARKER_POLL_SECONDS", 0.0)
    obs = _observer(tmp_path)
    cache = torch.zeros(1, 32, 1, 512, dtype=torch.int8)
    obs.observe("p", "ori", cache, torch.full((2, 512), 3.0), torch.arange(2))
    assert not (tmp_path / "rank_00.pt").exists()
    (tmp_path / "collect").unlink()
    obs.observe("p", "ori", cache, torch.full((2, 512), 5.0), torch.arange(2))
    saved = torch.load(tmp_path / "rank_00.pt", weights_only=True)
    assert saved["stats"]["p.ori"]["rows"] == 2 and float(saved["stats"]["p.ori"]["maximum"][0]) == 3.0
    assert not obs.pending


def test_observer_marker_poll_is_cached(tmp_path, monkeypatch):
    monkeypatch.setattr(calibration, "MARKER_POLL_SECONDS", 3600.0)
    obs = _observer(tmp_path, collect=False)
    assert not obs.collecting()
    (tmp_path / "collect").touch()
    assert not obs.collecting()          # within the poll interval the old answer stands
    obs._marker_seen = (-1e9, False)
    assert obs.collecting()


def test_observer_refuses_graph_capture(tmp_path, monkeypatch):
    obs = _observer(tmp_path)
    monkeypatch.setattr(calibration, "_capturing", lambda: True)
    cache = torch.zeros(1, 32, 1, 512, dtype=torch.int8)
    with pytest.raises(RuntimeError):
        obs.observe("p", "ori", cache, torch.ones(2, 512), torch.arange(2))
    assert obs.stats == {}


def test_merge_takes_channel_maxima_over_ranks(tmp_path):
    rng = np.random.default_rng(5)
    a = rng.standard_normal((40, 512)).astype(np.float32)
    b = rng.standard_normal((30, 512)).astype(np.float32) * 3
    paths = []
    for rank, rows in enumerate((a, b)):
        payload = {"version": 1, "rank": rank, "pid": 1,
                   "stats": {"m.l0.ori": {"maximum": torch.from_numpy(np.abs(rows).max(0)), "rows": len(rows)}}}
        path = tmp_path / f"rank_{rank:02d}.pt"
        torch.save(payload, path)
        paths.append(path)
    merged = calibration.merge_observations(paths, margin=1.1, required=["m.l0.ori"])
    # The same rule as the synthetic workloads' frozen scale over all rows.
    expected = workloads.frozen_scale(np.concatenate([a, b]))
    np.testing.assert_array_equal(merged["scales"]["m.l0.ori"].numpy(), expected)
    assert merged["observed_rows_across_ranks"] == {"m.l0.ori": 70}
    assert sorted(merged["source_sha256"]) == ["rank_00.pt", "rank_01.pt"]
    assert calibration.validate_scales(merged) is merged["scales"]
    # Hand case: maximum 0 gives the floor; 127 / 1.1 gives 1.0 up to rounding.
    payload = {"version": 1, "stats": {"k": {"maximum": torch.zeros(512), "rows": 1}}}
    torch.save(payload, tmp_path / "z.pt")
    assert float(calibration.merge_observations([tmp_path / "z.pt"])["scales"]["k"][0]) == np.float32(1e-8)
    with pytest.raises(ValueError):
        calibration.merge_observations(paths, required=["missing"])


def observe_calibrate_vector(tmp_path, device):
    """The golden calibrate.npz samples (written by the reference's
    CacheQuantization.calibrate, reference.py:32-37) observed as cache writes
    by two ranks' observers on `device`, merged at margin 1: returns
    (merged scale, golden scale)."""
    from pathlib import Path
    import shutil
    z = np.load(Path(__file__).resolve().parent / "golden" / "vectors" / "calibrate.npz")
    samples = [torch.from_numpy(z["sample0"]),
               torch.from_numpy(z["sample1_bf16"].view(np.int16)).view(torch.bfloat16),
               torch.from_numpy(z["sample2"])]
    files = []
    for rank, group in enumerate((samples[:1], samples[1:])):
        directory = tmp_path / f"r{rank}"
        obs = calibration.CacheObserver(directory)
        (directory / "collect").touch()
        for sample in group:
            rows = sample.reshape(-1, 512).to(device)
            cache = torch.zeros(max(1, (rows.shape[0] + 31) // 32), 32, 1, 512, dtype=torch.int8, device=device)
            obs.observe("g.l0", "ori", cache, rows, torch.arange(rows.shape[0], device=device))
        obs.flush()
        files.append(shutil.copy(directory / "rank_00.pt", tmp_path / f"rank_{rank:02d}.pt"))
    merged = calibration.merge_observations(files, margin=1.0, required=["g.l0.ori"])
    return merged["scales"]["g.l0.ori"], z["scale"]


def test_observer_and_merge_reproduce_reference_calibrate(tmp_path):
    """Observer + merge at margin 1 equal CacheQuantization.calibrate on the
    same rows bit for bit (golden calibrate.npz, including the 1e-8 floor of
    an all-zero channel): the merge's FP32 sequence max -> fp32(margin *
    max) / 127 -> floor is the reference's at margin 1, and margin 1.1
    follows docs/kv-cache.md's formula left to right."""
    got, want = observe_calibrate_vector(tmp_path, "cpu")
    np.testing.assert_array_equal(got.numpy(), want)
    assert got[7] == np.float32(1e-8)


def test_scale_file_checks(tmp_path):
    good = {"protocol": "sharedkv-c8-v1", "scales": {"a.ori": torch.full((512,), 0.5)}}
    torch.save(good, tmp_path / "s.pt")
    assert set(calibration.load_scale_file(tmp_path / "s.pt")) == {"a.ori"}
    bad = [{"protocol": "v0", "scales": {}},
           {"protocol": "sharedkv-c8-v1", "scales": {"x": torch.full((511,), 0.5)}},
           {"protocol": "sharedkv-c8-v1", "scales": {"x": torch.full((512,), 0.5, dtype=torch.float64)}},
           {"protocol": "sharedkv-c8-v1", "scales": {"x": torch.zeros(512)}},
           {"protocol": "sharedkv-c8-v1", "scales": {"x": torch.full((512,), float("nan"))}}]
    for payload in bad:
        with pytest.raises(ValueError):
            calibration.validate_scales(payload)


def test_activation_fixture_scales_pass_the_loader_checks():
    """The frozen scales of the reference's scales_v1.pt kept in the fixture
    (layers' original and compressed vectors) satisfy the loader's checks."""
    z = np.load(workloads_fixture_path())
    scales = {f"l{i}.{k}": torch.from_numpy(z[f"{i}_{k}_scale"]) for i in range(int(z["count"]))
              for k in ("ori", "cmp") if f"{i}_{k}_scale" in z.files}
    assert len(scales) == 19
    assert calibration.validate_scales({"protocol": "sharedkv-c8-v1", "scales": scales}) is scales


def workloads_fixture_path():
    from pathlib import Path
    return Path(__file__).resolve().parent / "golden" / "vectors" / "activations.npz"


# ----------------------------------------------------------- page planner

@dataclass(frozen=True)
class Spec:
    page_size_bytes: int
    dtype: torch.dtype = torch.int8
    head_size: int = 512
    block_size: int = 32
    model_version: str = "deepseek_v4"
    scale_dim: int = 0
    scale_dtype: torch.dtype = torch.float32
    page_size_padded: int | None = None
    pages: int = 10

    def max_memory_usage_pages(self, config):
        return self.pages


def _grouped(*groups):
    return [cache_layout.UniformSpecs(dict(g)) for g in groups]


def test_group_specs_keep_c4_c128_and_cut_state_groups():
    c4 = {"l0.swa_cache": Spec(16384), "l0.attn": Spec(16384), "l0.indexer": Spec(8704, head_size=128)}
    c128 = {"l1.swa_cache": Spec(16384), "l1.attn": Spec(16384)}
    state = {f"l{i}.state": Spec(16384, dtype=torch.float32, head_size=None, page_size_padded=32768)
             for i in range(5)}
    groups = cache_layout.group_specs(_grouped(c4, c128, state))
    budget = cache_layout.round_up(max(41472, 32768), 16384)          # 49152
    assert [len(g.layer_names) for g in groups] == [3, 2, 3, 2]
    for g in groups:
        assert g.kv_cache_spec.page_size_bytes <= budget or len(g.layer_names) == 1
    assert all(s.page_size_padded is None for s in groups[2].kv_cache_spec.kv_cache_specs.values())
    with pytest.raises(ValueError):
        cache_layout.group_specs(_grouped({"a": Spec(16384)}, {"b": Spec(16384, block_size=64),
                                                               "c": Spec(16384, block_size=32)}))


def test_packed_layout_alignment_and_stride():
    specs = {"big": Spec(16384 * 3 + 100, dtype=torch.float32, head_size=None),
             "c8": Spec(16384),
             "idx": Spec(8704 + 2, head_size=128, scale_dim=1, scale_dtype=torch.float32),
             "odd": Spec(7, dtype=torch.bfloat16, head_size=64)}
    groups = [cache_layout.CacheGroup(list(specs), cache_layout.UniformSpecs(specs))]
    stride, offsets = cache_layout.packed_layout(groups)
    order = sorted(specs, key=lambda n: -specs[n].page_size_bytes)
    assert order == ["big", "c8", "idx", "odd"]
    end = 0
    for name in order:
        assert offsets[name] >= end
        assert offsets[name] % cache_layout.alignment_of(specs[name]) == 0
        end = offsets[name] + specs[name].page_size_bytes
    assert offsets["c8"] % 512 == 0 and cache_layout.alignment_of(specs["idx"]) == 4
    assert stride % 512 == 0 and stride >= end and stride - end < 512
    dup = [groups[0], cache_layout.CacheGroup(["c8"], cache_layout.UniformSpecs({"c8": specs["c8"]}))]
    with pytest.raises(ValueError):
        cache_layout.packed_layout(dup)


def test_cache_config_descriptors_and_backing():
    specs = {"a.swa": Spec(16384), "a.attn": Spec(16384), "a.state": Spec(4096, dtype=torch.float32, head_size=None)}
    groups = [cache_layout.CacheGroup(list(specs), cache_layout.UniformSpecs(specs))]
    config = SimpleNamespace(parallel_config=SimpleNamespace(), cache_config=SimpleNamespace())
    stride, offsets = cache_layout.packed_layout(groups)
    assert stride == 36864 and cache_layout.max_memory_usage(config, groups) == stride * 10
    blocks, descriptors = cache_layout.cache_config(config, groups, 10 * stride + 5)
    assert blocks == 10 and {d.layers[0]: d.offset for d in descriptors} == offsets
    config.cache_config.num_gpu_blocks_override = 3
    blocks, descriptors = cache_layout.cache_config(config, groups, 10 * stride)
    assert blocks == 3 and all(d.size == 3 * stride and d.block_stride == stride for d in descriptors)
    views = cache_layout.allocate_backing(groups, descriptors, 3, list(specs), "cpu")
    assert views["a.swa"].data_ptr() % cache_layout.BACKING_ALIGNMENT == offsets["a.swa"]
    bad = [cache_layout.CacheTensor(size=d.size, layers=d.layers, offset=d.offset + 512, block_stride=stride)
           for d in descriptors]
    with pytest.raises(ValueError):
        cache_layout.allocate_backing(groups, bad, 3, list(specs), "cpu")
    with pytest.raises(ValueError):
        cache_layout.allocate_backing(groups, descriptors[:2], 3, list(specs), "cpu")
    for name in ("pipeline_parallel_size", "decode_context_parallel_size"):
        cfg = SimpleNamespace(parallel_config=SimpleNamespace(**{name: 2}), cache_config=SimpleNamespace())
        with pytest.raises(ValueError):
            cache_layout.cache_config(cfg, groups, 10 * stride)


def test_page_views_address_page_times_stride():
    stride, offset, blocks = 622592, 16384, 3
    raw = torch.full((blocks * stride,), 73, dtype=torch.int8)
    cache, scales = cache_layout.page_views(raw[offset:], [(blocks, 32, 1, 512), (blocks, 32, 1)],
                                            [torch.int8, torch.float32], stride)
    assert cache.stride() == (stride, 512, 512, 1) and cache.data_ptr() == raw.data_ptr() + offset
    assert scales.stride() == (stride // 4, 1, 1) and scales.data_ptr() == raw.data_ptr() + offset + 16384
    cache.fill_(1)
    scales.fill_(2.0)
    per_block = raw.view(blocks, stride)
    assert (per_block[:, offset:offset + 16384] == 1).all()
    assert (per_block[:, offset + 16384:offset + 16384 + 128].view(torch.float32) == 2.0).all()
    assert (per_block[:, :offset] == 73).all() and (per_block[:, offset + 16384 + 128:] == 73).all()
    with pytest.raises(ValueError):
        cache_layout.page_views(raw[offset:], [(blocks, 32, 1, 512)], [torch.int8], 8192)


def test_uses_compact():
    groups = [cache_layout.CacheGroup(["x"], cache_layout.UniformSpecs({"x": Spec(16384)}))]
    assert cache_layout.uses_compact(groups)
    other = [cache_layout.CacheGroup(["x"], cache_layout.UniformSpecs({"x": Spec(16384, dtype=torch.bfloat16)}))]
    assert not cache_layout.uses_compact(other + [None])


# ------------------------------------------------------- adapter / plugin

def _impl(prefix="model.layers.3.self_attn", **parallel):
    return SimpleNamespace(swa_cache_layer=SimpleNamespace(prefix=prefix + ".swa_cache"), head_dim=512,
                           turboquant=None, vllm_config=SimpleNamespace(parallel_config=SimpleNamespace(**parallel)))


@pytest.fixture
def scale_file(tmp_path, monkeypatch):
    path = tmp_path / "scales.pt"
    torch.save({"protocol": "sharedkv-c8-v1",
                "scales": {"model.layers.3.self_attn.ori": torch.full((512,), 0.25)}}, path)
    monkeypatch.setenv("SHAREDKV_SCALES", str(path))
    vllm_adapter.load_scales.cache_clear()
    yield path
    vllm_adapter.load_scales.cache_clear()


def test_layer_contract_checks(scale_file):
    layer = vllm_adapter.runtime(_impl())
    assert layer.prefix == "model.layers.3.self_attn"
    for bad in ({"head_dim": 128}, {"turboquant": object()}):
        with pytest.raises(ValueError):
            vllm_adapter.runtime(SimpleNamespace(**{**vars(_impl()), **bad}))
    with pytest.raises(ValueError):
        vllm_adapter.runtime(_impl(decode_context_parallel_size=2))
    q = torch.zeros(1, 8, 512, dtype=torch.bfloat16)
    for kw in (dict(layout_q="BSND", layout_kv="PA_ND"), dict(layout_q="TND", layout_kv="PA_ND", ori_mask_mode=3),
               dict(layout_q="TND", layout_kv="PA_ND", ori_win_right=4),
               dict(layout_q="TND", layout_kv="PA_ND", cmp_ratio=4, cmp_mask_mode=1)):
        with pytest.raises(ValueError):
            layer.attention(q, **kw)
    layer.write(None, torch.zeros(0, 512), torch.zeros(0, dtype=torch.int32), "ori")   # empty: nothing
    with pytest.raises(ValueError):
        layer.write(None, torch.zeros(2, 512), torch.zeros(3, dtype=torch.int32), "ori")
    impl = _impl()
    assert vllm_adapter.runtime(impl) is vllm_adapter.runtime(impl)


def test_parse_and_launch_shape():
    """The keyword contract maps onto SharedKVCase; calls that differ only in
    device pointers share a launch shape, anything baked into the argument
    block (tokens, pages, strides, table widths, LSE) does not."""
    case = workloads.make_case(5, 4, [2, 1], [3000, 900])
    dev = SimpleNamespace()

    def kw(tokens=3, lse=True, stride=16384):
        q = torch.zeros(tokens, 8, 512, dtype=torch.bfloat16)
        pool = torch.zeros(40 * stride, dtype=torch.int8).as_strided((40, 32, 1, 512), (stride, 512, 512, 1))
        return q, dict(ori_kv=pool, cmp_kv=pool, ori_block_table=torch.zeros(2, 94, dtype=torch.int32),
                       cmp_block_table=torch.zeros(2, 24, dtype=torch.int32),
                       cmp_sparse_indices=torch.zeros(tokens, 1, 1024, dtype=torch.int32),
                       cu_seqlens_q=torch.tensor([0, 2, tokens], dtype=torch.int32),
                       seqused_kv=torch.tensor([3000, 900], dtype=torch.int32), sinks=torch.zeros(8),
                       cmp_ratio=4, ori_win_left=127, softmax_scale=0.04, layout_q="TND", layout_kv="PA_ND",
                       return_softmax_lse=lse)
    del case, dev
    c1, l1 = vllm_adapter.parse_attention_call(*kw())
    c2, l2 = vllm_adapter.parse_attention_call(*kw())
    assert c1.ratio == 4 and c1.window == 128 and l1 is True
    assert vllm_adapter.launch_shape(c1, l1) == vllm_adapter.launch_shape(c2, l2)
    for other in (kw(tokens=4), kw(lse=False), kw(stride=622592)):
        c3, l3 = vllm_adapter.parse_attention_call(*other)
        assert vllm_adapter.launch_shape(c3, l3) != vllm_adapter.launch_shape(c1, l1)


def test_operator_cache_is_lru():
    cache = vllm_adapter.OperatorCache(capacity=2)
    cache.put("a", 1)
    cache.put("b", 2)
    assert cache.get("a") == 1
    cache.put("c", 3)                       # "b" is the least recently used
    assert cache.get("b") is None and list(cache.values()) == [1, 3]


def test_load_scales_requires_the_file(monkeypatch, scale_file):
    assert set(vllm_adapter.load_scales()) == {"model.layers.3.self_attn.ori"}
    monkeypatch.delenv("SHAREDKV_SCALES")
    vllm_adapter.load_scales.cache_clear()
    with pytest.raises(ValueError):
        vllm_adapter.load_scales()


@dataclass(frozen=True)
class Plan:
    sparse_attn_op: object = None
    other: int = 7


@dataclass(frozen=True)
class BF16Spec:
    head_size: int = 512
    dtype: torch.dtype = torch.bfloat16
    page_size_bytes: int = 32768
    page_size_padded: int | None = None
    indexes_kv_by_block_stride: bool = False


def _engine_classes():
    class Impl:
        def __init__(self):
            self.__dict__.update(vars(_impl()))
            self.writes = []

        def get_kv_plan(self):
            return Plan()

        def _write_kv_cache(self, cache, kv, slot_mapping, *, quantize):
            self.writes.append((cache, kv, slot_mapping, quantize))
            return "bf16"

    class Cache:
        def get_kv_cache_spec(self, config):
            return BF16Spec()

    return Impl, Cache


def test_install_routes_plan_writes_and_specs(scale_file, monkeypatch):
    Impl, Cache = _engine_classes()
    vllm_adapter.install(vllm_adapter.EngineBinding(impl=Impl, cache_specs=(Cache,)))
    impl = Impl()
    plan = impl.get_kv_plan()
    assert plan.other == 7 and plan.sparse_attn_op == vllm_adapter.runtime(impl).attention
    assert impl.get_kv_plan() is plan
    calls = []
    monkeypatch.setattr(vllm_adapter.SharedKVLayer, "write", lambda self, *a: calls.append(a))
    impl._write_kv_cache("c", "kv", "s", quantize=True)
    impl._write_kv_cache("c", "kv", "s", quantize=False)
    assert calls == [("c", "kv", "s", "cmp"), ("c", "kv", "s", "ori")]
    spec = Cache().get_kv_cache_spec(None)
    assert spec.dtype == torch.int8 and spec.page_size_padded == 32768 and spec.indexes_kv_by_block_stride
    Impl2, Cache2 = _engine_classes()
    vllm_adapter.install(vllm_adapter.EngineBinding(impl=Impl2, cache_specs=(Cache2,), compact_pages=True))
    assert Cache2().get_kv_cache_spec(None).page_size_padded is None

    class Renamed:
        """Method and field names are the binding's, not fixed."""
        def __init__(self):
            self.__dict__.update(vars(_impl()))

        def plan(self):
            return SimpleNamespace(attention=None)

        def store(self, cache, kv, slot_mapping, *, quantize):
            return "bf16"

    @dataclass(frozen=True)
    class RenamedPlan:
        attention: object = None

    Renamed.plan = lambda self: RenamedPlan()
    vllm_adapter.install(vllm_adapter.EngineBinding(impl=Renamed, plan_method="plan", plan_field="attention",
                                                    write_method="store"))
    r = Renamed()
    assert r.plan().attention == vllm_adapter.runtime(r).attention
    r.store("c", "kv", "s", quantize=False)
    assert calls[-1] == ("c", "kv", "s", "ori")


def test_plugin_modes(tmp_path, scale_file, monkeypatch):
    monkeypatch.setattr(vllm_plugin.state, "mode", None)
    monkeypatch.delenv("SHAREDKV_INT8_MODE", raising=False)
    vllm_plugin.register(binding=object())       # unset: nothing happens, the binding is not used
    assert vllm_plugin.state.mode is None
    monkeypatch.setenv("SHAREDKV_INT8_MODE", "fp8")
    with pytest.raises(ValueError):
        vllm_plugin.register(binding=object())
    monkeypatch.setenv("SHAREDKV_INT8_MODE", "calibrate")
    monkeypatch.delenv("SHAREDKV_CALIBRATION_DIR", raising=False)
    with pytest.raises(ValueError):
        vllm_plugin.register(binding=object())

    Impl, Cache = _engine_classes()
    monkeypatch.setenv("SHAREDKV_CALIBRATION_DIR", str(tmp_path / "cal"))
    vllm_plugin.register(binding=vllm_adapter.EngineBinding(impl=Impl))
    assert vllm_plugin.state.mode == "calibrate"
    (tmp_path / "cal" / "collect").touch()
    vllm_plugin.state.observer._marker_seen = (-1e9, False)
    impl = Impl()
    cache = torch.zeros(2, 32, 1, 512, dtype=torch.int8)
    kv = torch.ones(3, 512, dtype=torch.bfloat16)
    assert impl._write_kv_cache(cache, kv, torch.arange(3), quantize=True) == "bf16"
    assert len(impl.writes) == 1 and int(vllm_plugin.state.observer.stats["model.layers.3.self_attn.cmp"][1]) == 3
    vllm_plugin.register(binding=object())       # registered once per process
    vllm_plugin.state.observer.pending = False

    monkeypatch.setattr(vllm_plugin.state, "mode", None)
    monkeypatch.setenv("SHAREDKV_INT8_MODE", "int8")
    Impl, Cache = _engine_classes()
    vllm_plugin.register(binding=vllm_adapter.EngineBinding(impl=Impl, cache_specs=(Cache,)))
    assert vllm_plugin.state.mode == "int8"
    assert Cache().get_kv_cache_spec(None).dtype == torch.int8


def test_plugin_binding_from_env(monkeypatch):
    monkeypatch.setenv(vllm_plugin.TARGETS_ENV, json.dumps({"impl": "collections:OrderedDict",
                                                            "cache_specs": ["types:SimpleNamespace"],
                                                            "compact_pages": True}))
    binding = vllm_plugin.binding_from_env()
    from collections import OrderedDict
    assert binding.impl is OrderedDict and binding.cache_specs == (SimpleNamespace,) and binding.compact_pages
    assert binding.plan_method == "get_kv_plan" and binding.write_method == "_write_kv_cache"
    monkeypatch.delenv(vllm_plugin.TARGETS_ENV)
    with pytest.raises(RuntimeError):
        vllm_plugin.binding_from_env()
    for bad in ("no_colon", ":Name", "collections:"):
        with pytest.raises(ValueError):
            vllm_plugin.resolve(bad)
