"""Pins the CPU checker (oracle/) before any GPU result is compared with it.

Sources of truth, in order:
  1. vectors written by the reference's own reference.py (tests/golden/):
     tiled_quantized_reference, joint_quantized_row, sharedkv_reference (FP64)
     and CacheQuantization, on seeded cases and several tiling plans;
  2. the reference's known-answer tests (tests/unit/test_reference.py of the
     reference checkout): rounding/clipping, shared sink denominator,
     padding indices, integer oracle vs FP64 attention;
  3. the reference's data fixtures (tests/fixtures/activations and the frozen
     serving scales data/scales_v1.pt, converted by
     tests/golden/make_fixtures.py): real captured activations with their
     FP64 attention outputs, and the reference's accuracy gates on them;
  4. what the mathematics fixes: exact integer dot products recomputed by
     brute force from the dumped codes and the gathered rows, the residual
     reconstruction bounds of the Q and P splits, the pairwise-sum tree,
     and exp against float64.
"""
import math
from pathlib import Path

import numpy as np
import pytest

import oracle.oracle as ora
from tests import workloads
from tests.device_cases import query_subcase

GOLDEN = Path(__file__).resolve().parent / "golden" / "vectors"
CASES = sorted(p.stem for p in GOLDEN.glob("c*.npz") if p.stem != "calibrate")


def golden_plans(z):
    """(tile, splits, joint_dense, joint_sparse, joint_tile_limit, dense_c4,
    query_group) of each stored output; older files carry the first five."""
    return [tuple(int(v) for v in p) + (0, 1)[len(p) - 5:] for p in z["plans"]]


def golden_case(z):
    has = lambda k: k in z.files  # noqa: E731
    return ora.Case(q=z["q"], ori=z["ori_pool"], ori_stride=int(z["ori_stride"]), ori_table=z["ori_table"],
                    cu_q=z["cu_q"], seq_lens=z["seq_lens"], sink=z["sink"], ori_scale=z["ori_scale"],
                    cmp=z["cmp_pool"] if has("cmp_pool") else None,
                    cmp_stride=int(z["cmp_stride"]) if has("cmp_stride") else 0,
                    cmp_table=z["cmp_table"] if has("cmp_table") else None,
                    cmp_scale=z["cmp_scale"] if has("cmp_scale") else None,
                    cmp_indices=z["cmp_indices"] if has("cmp_indices") else None,
                    ratio=int(z["ratio"]), window=int(z["window"]), softmax_scale=float(z["softmax_scale"]),
                    ori_indices=z["ori_indices"] if has("ori_indices") else None,
                    ori_pages=int(z["ori_pages"]) if has("ori_pages") else 0)


def bf16_ulps(a_bits, b_bits):
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    # Same sign region: the bit patterns are ordered like the values.
    return np.abs(a - b)


# ------------------------------------------------------------ golden vectors

@pytest.mark.parametrize("name", CASES)
def test_tiled_attention_matches_reference_vectors(name):
    """reference.py:210-323 outputs: bit-exact except rare 1-ulp BF16 flips
    from exp/summation ulps (torch.exp is not correctly rounded)."""
    z = np.load(GOLDEN / f"{name}.npz")
    case = golden_case(z)
    for i, (tile, splits, jd, js, limit, dense, group) in enumerate(golden_plans(z)):
        out, lse, _ = ora.tiled_attention(case, tile, splits, joint_dense=bool(jd), joint_sparse=bool(js),
                                          joint_tile_limit=limit, dense_c4=bool(dense), query_group=group)
        ref, ref_lse = z[f"out_{i}"], z[f"lse_{i}"]
        live = int(z["cu_q"][-1])
        ulps = bf16_ulps(out[:live], ref[:live])
        assert ulps.max() <= 1, (name, i)
        assert (ulps == 0).mean() >= 0.999, (name, i)
        np.testing.assert_allclose(lse[:live], ref_lse[:live], rtol=0, atol=2e-6)


def test_plan_families_are_covered():
    """The golden plans exercise every parameter the oracle restates:
    tile sizes 64-512, 1-5 partitions, both joint rows, the dense C4
    multiplicity list (with duplicates) and query groups of 2, 3 and 4."""
    plans = [p for name in CASES for p in golden_plans(np.load(GOLDEN / f"{name}.npz"))]
    assert {p[0] for p in plans} >= {64, 128, 256, 512}
    assert {p[1] for p in plans} >= {1, 2, 3, 4, 5}
    assert any(p[2] for p in plans) and any(p[3] for p in plans)
    assert any(p[5] for p in plans)
    assert {p[6] for p in plans} >= {1, 2, 3, 4}
    dense_dups = np.load(GOLDEN / "c4_dups.npz")
    assert any(p[5] for p in golden_plans(dense_dups))


def test_count_log_is_correctly_rounded():
    """The multiplicity bias log(count) (reference.py:249, 261; the checker's
    log_count and the kernel's, both the FP32 rounding of a double log):
    for every count 1..1024 the exact ln(k) (50 digits) lies at least 4e-4
    FP32 ulp from an FP32 rounding midpoint, so the double log rounds to the
    correctly rounded value, which torch.log gives too."""
    from decimal import Decimal, getcontext
    import torch
    getcontext().prec = 50
    ours = np.array([np.float32(math.log(k)) for k in range(1, 1025)])
    theirs = torch.log(torch.arange(1, 1025, dtype=torch.float32)).numpy()
    assert np.array_equal(ours, theirs)
    for k in range(2, 1025):
        exact = Decimal(k).ln()
        f = ours[k - 1]
        up, down = np.nextafter(f, np.float32(np.inf)), np.nextafter(f, np.float32(-np.inf))
        ulp = Decimal(float(up)) - Decimal(float(f))
        # f is the nearest float, and ln(k) is far from both midpoints.
        assert abs(exact - Decimal(float(f))) <= ulp / 2
        for other in (up, down):
            midpoint = (Decimal(float(f)) + Decimal(float(other))) / 2
            assert abs(exact - midpoint) >= Decimal("4e-4") * ulp, k
    assert ours[0] == 0.0


def test_joint_plans_need_residual_codes():
    """reference.py:258 asserts residual quantization (at most eight heads)
    for joint rows; the checker refuses such a plan outright."""
    case = workloads.oracle_case(workloads.make_case(4, 128, [1], [4096], heads=16))
    with pytest.raises(ValueError, match="code -11"):
        ora.tiled_attention(case, 128, 1, joint_dense=True)
    ora.tiled_attention(case, 128, 1)


def test_query_group_one_is_the_ungrouped_plan():
    """reference.py:229-231 with query_group = 1 reduces to each query's own
    window and list: the grouped code path at G = 1 equals the default."""
    case = golden_case(np.load(GOLDEN / "c4_pairs.npz"))
    a, la, _ = ora.tiled_attention(case, 128, 2)
    b, lb, _ = ora.tiled_attention(case, 128, 2, query_group=1)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(la, lb)


def test_query_group_masks_are_exact_for_window_only_rows():
    """A group's shared window (reference.py:233-234) only adds masked
    positions.  With 64-key tiles a query whose own window starts on a tile
    boundary sees the same tiles plus fully masked ones, which leave the
    state unchanged (weights 0, factor 1): its output equals the ungrouped
    plan's bit for bit.  Position 127 of a group of two starting at 126 has
    its window at 0..127, the group's list 0..127 as well."""
    case = workloads.oracle_case(workloads.make_case(3, 1, [2], [128]))
    a, la, _ = ora.tiled_attention(case, 64, 1)
    b, lb, _ = ora.tiled_attention(case, 64, 1, query_group=2)
    np.testing.assert_array_equal(a[1], b[1])
    np.testing.assert_array_equal(la[1], lb[1])


def test_calibrate_scale_matches_reference_vector():
    """CacheQuantization.calibrate (reference.py:32-37): channel abs-max over
    every sample (FP32 and BF16 inputs), / 127, floored at 1e-8 (a zero
    channel), bit for bit."""
    z = np.load(GOLDEN / "calibrate.npz")
    rows = np.concatenate([z["sample0"].reshape(-1, 512), ora.bf16_to_f32(z["sample1_bf16"]).reshape(-1, 512),
                           z["sample2"].reshape(-1, 512)])
    got = ora.calibrate_scale(rows)
    np.testing.assert_array_equal(got, z["scale"])
    assert got[7] == np.float32(1e-8)


def test_joint_row_matches_reference_vectors():
    z = np.load(GOLDEN / "joint_rows.npz")
    for tag, bias in (("plain", None), ("bias", z["bias"])):
        out, lse = ora.joint_row(z["q"], [z["rows0"], z["rows1"]], [z["scale0"], z["scale1"]], z["sink"],
                                 1 / math.sqrt(512), bias=bias)
        assert bf16_ulps(out, z[f"out_{tag}"]).max() <= 1
        assert (out == z[f"out_{tag}"]).mean() >= 0.999
        np.testing.assert_allclose(lse, z[f"lse_{tag}"], rtol=0, atol=2e-6)


@pytest.mark.parametrize("name", CASES)
def test_encoding_matches_reference_vectors(name):
    """CacheQuantization.inverse_scale and quantize (reference.py:47-53)."""
    z = np.load(GOLDEN / f"{name}.npz")
    np.testing.assert_array_equal(ora.inverse_scale(z["ori_scale"]), z["ori_inverse"])
    if "cmp_scale" in z.files:
        np.testing.assert_array_equal(ora.inverse_scale(z["cmp_scale"]), z["cmp_inverse"])
    values = ora.bf16_to_f32(z["quant_source_bits"])
    np.testing.assert_array_equal(ora.quantize(values, z["ori_inverse"]), z["quant_codes"])


@pytest.mark.parametrize("name", CASES)
def test_fp64_attention_matches_reference_vectors(name):
    """sharedkv_reference (reference.py:129-139) over decoded INT8 rows."""
    z = np.load(GOLDEN / f"{name}.npz")
    out, lse = ora.fp64_attention(golden_case(z))
    live = int(z["cu_q"][-1])
    np.testing.assert_allclose(out[:live], z["fp64_out"][:live], rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(lse[:live], z["fp64_lse"][:live], rtol=1e-6, atol=1e-6)


# ------------------------------------------- reference data fixtures

ACTIVATIONS = GOLDEN / "activations.npz"
ACT_LAYERS = 11
ACT_PATH_LAYERS = list(range(ACT_LAYERS))    # SWA128 + C4/C128 samples, and MTP samples on 133 explicit slots


def head_metrics(got, want):
    """tests/support/attention_cases.py:9-14 of the reference."""
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    a, b = got.reshape(-1, got.shape[-1]), want.reshape(-1, want.shape[-1])
    cos = (a * b).sum(-1) / (np.linalg.norm(a, axis=-1) * np.linalg.norm(b, axis=-1))
    return np.linalg.norm(got - want) / np.linalg.norm(want), cos.min()


@pytest.mark.parametrize("i", range(ACT_LAYERS))
def test_fp64_math_reproduces_fixture_reference(i):
    """The FP64 attention of reference.py:133-136 on each captured sample
    (query, original + compressed rows, sink) equals the sample's stored
    `reference` output."""
    z = np.load(ACTIVATIONS)
    q = workloads.bf16_value(z[f"{i}_q"]).astype(np.float64)
    kv = np.concatenate([workloads.bf16_value(z[f"{i}_ori"]), workloads.bf16_value(z[f"{i}_cmp"])]).astype(np.float64)
    out, _ = ora.fp64_rows(q, kv, z[f"{i}_sink"], float(z[f"{i}_softmax_scale"]))
    np.testing.assert_allclose(out, z[f"{i}_reference"], rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("splits", [1, 2])
@pytest.mark.parametrize("i", ACT_PATH_LAYERS)
def test_int8_path_meets_reference_gates_on_real_activations(i, splits):
    """The INT8 path (window + compressed rows encoded with the layer's frozen
    serving scales) against the sample's FP64 output, with the reference's
    gates: relative L2 < .04 and min head cosine > .999
    (tests/npu/test_attention.py:56, 110 of the reference)."""
    z = np.load(ACTIVATIONS)
    case = workloads.fixture_case(z, i)
    out, lse, _ = ora.tiled_attention(workloads.oracle_case(case), tile=128, splits=splits)
    rel, cos = head_metrics(ora.bf16_to_f32(out[0]), z[f"{i}_reference"])
    assert rel < 0.04 and cos > 0.999, (str(z[f"{i}_layer"]), rel, cos)
    assert np.isfinite(lse).all()


# ------------------------------------------------- reference known answers

def test_rounding_and_clipping_kat():
    """tests/unit/test_reference.py:22-28: half-even rounding, clamp at 127."""
    row = np.zeros((1, 512), np.float32)
    row[0, :8] = [-200.0, -127.0, -1.5, -0.5, 0.5, 1.5, 127.0, 200.0]
    codes = ora.quantize(row, ora.inverse_scale(np.ones(512, np.float32)))
    assert codes[0, :8].tolist() == [-127, -127, -2, 0, 0, 2, 127, 127]


def test_sink_shares_the_denominator_kat():
    """tests/unit/test_reference.py:50-58: q = 0, rows of 10 and 20, sink 0
    -> three equal weights, output exactly 10 (sink has no value), lse log 3."""
    q = np.zeros((2, 512), np.uint16)
    rows = [np.full((1, 512), 10, np.int8), np.full((1, 512), 20, np.int8)]
    ones = np.ones(512, np.float32)
    out, lse = ora.joint_row(q, rows, [ones, ones], np.zeros(2, np.float32), 1.0)
    assert np.all(ora.bf16_to_f32(out) == 10.0)
    np.testing.assert_allclose(lse, math.log(3), rtol=1e-6, atol=1e-6)


def test_padding_indices_do_not_contribute_kat():
    """tests/unit/test_reference.py:74-82: -1 and huge indices select nothing."""
    case = workloads.make_case(9, 4, [1], [257], index_mode="uniform")
    base = workloads.oracle_case(case)
    out_a, lse_a = ora.fp64_attention(base)
    padded = dict(case)
    ix = case["cmp_indices"].copy()
    ix[ix < 0] = 2 ** 30
    padded["cmp_indices"] = ix
    out_b, lse_b = ora.fp64_attention(workloads.oracle_case(padded))
    np.testing.assert_array_equal(out_a, out_b)
    np.testing.assert_array_equal(lse_a, lse_b)
    # The integer path agrees bit for bit too.
    a, la, _ = ora.tiled_attention(base)
    b, lb, _ = ora.tiled_attention(workloads.oracle_case(padded))
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(la, lb)


@pytest.mark.parametrize("ratio", [1, 4, 128])
def test_integer_oracle_close_to_fp64_attention(ratio):
    """tests/unit/test_reference.py:60-72: rel-L2 < 0.01, LSE within 2e-4."""
    case = workloads.make_case(23, ratio, [2, 1], [129, 257])
    c = workloads.oracle_case(case)
    out, lse, _ = ora.tiled_attention(c)
    ref, ref_lse = ora.fp64_attention(c)
    got = ora.bf16_to_f32(out).astype(np.float64)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 0.01
    np.testing.assert_allclose(lse, ref_lse, rtol=2e-4, atol=2e-4)


@pytest.mark.parametrize("ratio", [4, 128])
def test_many_partition_folds_close_to_fp64_attention(ratio):
    """The fold over 5-16 KV partitions (the one-partition-per-tile plans and
    the fold above eight partitions): rel-L2 < 0.01 and LSE within 2e-4 of
    FP64 attention at every partition count, as at one; and partitions that
    own no tile change nothing (rows of at most nine tiles give the same
    bits at 9, 12 and 16 partitions)."""
    lengths = [129, 9000, 70000] if ratio == 4 else [20000, 70000, 131072]
    case = workloads.make_case(41, ratio, [1, 2, 1], lengths)
    c = workloads.oracle_case(case)
    ref, ref_lse = ora.fp64_attention(c)
    outs = {}
    for splits in (5, 8, 9, 12, 16):
        out, lse, _ = ora.tiled_attention(c, splits=splits)
        got = ora.bf16_to_f32(out).astype(np.float64)
        assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 0.01, splits
        np.testing.assert_allclose(lse, ref_lse, rtol=2e-4, atol=2e-4, err_msg=f"S={splits}")
        outs[splits] = (out, lse)
    for splits in (12, 16):
        np.testing.assert_array_equal(outs[splits][0], outs[9][0])
        np.testing.assert_array_equal(outs[splits][1], outs[9][1])
    assert not np.array_equal(outs[5][0], outs[9][0])     # the partition count is part of the numerics


@pytest.mark.parametrize("mode", workloads.EDGE_MODES)
def test_edge_selections_close_to_fp64_attention(mode):
    """The reference's sparse-edge selections (tests/npu/test_sparse_edges.py
    :52-75) through the checker, one and three KV partitions: rel-L2 < 0.01
    and LSE within 2e-4 of FP64 attention over the same multiset of rows
    (duplicates count once per occurrence, reference.py:115-122)."""
    case = workloads.make_case(31, 4, [1] * 6, [129, 513, 1023, 1500, 4200, 9000], index_mode=mode)
    c = workloads.oracle_case(case)
    ref, ref_lse = ora.fp64_attention(c)
    for splits in (1, 3):
        out, lse, _ = ora.tiled_attention(c, splits=splits)
        got = ora.bf16_to_f32(out).astype(np.float64)
        assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 0.01, (mode, splits)
        np.testing.assert_allclose(lse, ref_lse, rtol=2e-4, atol=2e-4, err_msg=f"{mode} S={splits}")


def test_empty_selection_reduces_to_the_window_path():
    """A C4 row without a valid top-k entry is its window alone, whether the
    list is compacted away (count < topk) or kept as in-place holes (count >=
    topk: eight fully masked tiles): bit-exact with the window-only plan on
    the same window rows and scales."""
    case = workloads.make_case(32, 4, [1, 2], [700, 5000], index_mode="empty")
    window_only = dict(case, ratio=1, cmp=None, cmp_indices=None, topk=0)
    for splits in (1, 3):
        out_c4, lse_c4, _ = ora.tiled_attention(workloads.oracle_case(case), splits=splits)
        out_w, lse_w, _ = ora.tiled_attention(workloads.oracle_case(window_only), splits=1)
        assert np.array_equal(out_c4, out_w), splits
        assert np.array_equal(lse_c4, lse_w), splits


# ---------------------------------------------------- mathematical pins

def test_expf_against_float64():
    """sko_expf is within one ulp of the correctly rounded exponential (the
    float64 exp rounded once) and equals it on all but a small fraction of
    arguments: every 64th float32 in [-87, 0], plus a uniform grid.  The
    exhaustive survey (tests/golden/exp_survey.py, exp_survey.json) found
    0.45 % of all 1.12e9 such inputs not correctly rounded, none by more
    than one ulp."""
    bits = np.arange(0x80000000, 0xC2AE0000 + 1, 64, dtype=np.uint64).astype(np.uint32)
    x = np.concatenate([bits.view(np.float32), np.linspace(-87, 0, 200001, dtype=np.float32),
                        np.float32([-1e-30, -0.5, -1.0, -86.9])])
    got = ora.expf(x)
    want = np.exp(x.astype(np.float64)).astype(np.float32)
    diff = np.abs(got.view(np.int32).astype(np.int64) - want.view(np.int32).astype(np.int64))
    assert diff.max() <= 1
    assert (diff != 0).mean() < 0.006
    assert ora.expf(np.float32([0.0]))[0] == 1.0
    assert ora.expf(np.float32([-88.0, -1e30]))[0] == 0.0


def test_exp_survey_record():
    """The recorded survey of sko_expf against torch.exp (MKL on the CPU) and
    of the P codes it changes on the golden cases (tests/golden/exp_survey.py)
    stays consistent with the golden vectors it was taken on."""
    import json
    rec = json.loads((GOLDEN / "exp_survey.json").read_text())
    ex = rec["exhaustive_minus87_to_0"]
    assert ex["inputs"] == 0xC2AE0000 - 0x80000000 + 1
    assert ex["sko_vs_torch_over_1ulp"] == 0
    flips = rec["p_code_flips_total"]
    assert flips["weights"] > 200000 and flips["either"] <= flips["weights"] * 1e-4


def test_tree_sum_is_pairwise():
    import ctypes
    rng = np.random.default_rng(1)
    for count in (1, 5, 64, 100, 128):
        x = rng.random(count, dtype=np.float32)
        padded = 1 << (count - 1).bit_length()
        v = np.zeros(padded, np.float32)
        v[:count] = x
        while len(v) > 1:
            v = (v[0::2] + v[1::2]).astype(np.float32)
        got = ora.lib().sko_tree_sum(ctypes.c_void_p(x.ctypes.data), count, padded)
        assert np.float32(got) == v[0]


def _pin_case(seed, ratio, mode="uniform"):
    lengths = {4: [600, 5000], 128: [300, 9000], 1: [90, 700]}[ratio]
    return workloads.make_case(seed, ratio, [2, 1], lengths, index_mode=mode)


def _selection(case):
    """Brute-force reference.py:93-126 selection (+ compaction 250-252):
    per token, the list of (kind, logical row or None) in tile order."""
    cu, lens = case["cu_q"], case["seq_lens"]
    lists = []
    for b in range(len(lens)):
        for t in range(cu[b], cu[b + 1]):
            pos = int(lens[b]) - int(cu[b + 1]) + t
            ori = list(range(max(0, pos - 127), pos + 1))
            cmp = []
            if case["ratio"] != 1:
                count = (pos + 1) // case["ratio"]
                if case["ratio"] == 4:
                    raw = [int(i) for i in case["cmp_indices"][t, 0]]
                    if count < len(raw) <= 1024:
                        cmp = [i for i in raw if 0 <= i < count]
                    else:
                        cmp = [i if 0 <= i < count else None for i in raw]
                else:
                    cmp = list(range(count))
            lists.append((b, ori, cmp))
    return lists


@pytest.mark.parametrize("ratio,mode", [(4, "uniform"), (4, "holes"), (4, "dups"), (4, "mixed"), (128, None),
                                        (1, None)])
def test_integer_partials_by_brute_force(ratio, mode):
    """QK and PV int32 partials equal exact integer dot products of the dumped
    codes with the rows the selection rule picks; the Q and P splits
    reconstruct their inputs within the rounding bounds."""
    case = _pin_case(31, ratio, mode or "uniform")
    c = workloads.oracle_case(case)
    out, lse, dbg = ora.tiled_attention(c, tile=128, splits=2, debug=True)
    for t, (b, ori, cmp) in enumerate(_selection(case)):
        for kind, rows, kd in ((0, ori, case["ori"]), (1, cmp, case["cmp"])):
            if kd is None:
                continue
            qc = dbg["qcodes"][t, kind].astype(np.int64)
            alpha = dbg["alpha"][t, kind]
            # Q split: |q8| peaks at 127 per head and q8 + qlo/127 matches q*scale/alpha.
            folded = ora.bf16_to_f32(case["q"][t]).astype(np.float64) * kd.scale.astype(np.float64)
            assert np.all(np.abs(qc[:8]).max(1) == 127)
            recon = qc[:8] + qc[8:] / 127.0
            assert np.max(np.abs(recon - folded / alpha[:, None])) <= 0.5 / 127 + 1e-4
            for j, idx in enumerate(rows):
                base = 0 if kind == 0 else 128
                s = dbg["scores"][t, base + j]
                if idx is None:
                    continue
                row = ora.gather_rows(kd.pool, kd.page_stride, kd.table, b, [idx])[0].astype(np.int64)
                np.testing.assert_array_equal(s[:8], qc[:8] @ row)
                np.testing.assert_array_equal(s[8:], qc[8:] @ row)
        # PV: per tile, the dumped P codes times the tile's rows.
        tiles = []
        for kind, rows, kd in ((0, ori, case["ori"]), (1, cmp, case["cmp"])):
            for start in range(0, len(rows), 128):
                tiles.append((kind, rows[start:start + 128], start, kd))
        for number, (kind, rows, start, kd) in enumerate(tiles):
            if number >= dbg["values"].shape[1]:
                break
            base = (0 if kind == 0 else 128) + start
            p = dbg["probs"][t, base:base + len(rows)].astype(np.int64)   # [n, 16]
            assert p[:, :8].min() >= 0 and p[:, :8].max() <= 127
            kv = np.zeros((len(rows), 512), np.int64)
            for j, idx in enumerate(rows):
                if idx is not None:
                    kv[j] = ora.gather_rows(kd.pool, kd.page_stride, kd.table, b, [idx])[0]
            np.testing.assert_array_equal(dbg["values"][t, number], p.T @ kv)


@pytest.mark.parametrize("ratio", [1, 4, 128])
def test_window_slots_reproduce_the_window_path(ratio):
    """Explicit original slots (reference.py:236-239, 285) listing a query's
    own window rows in window order, then -1, put the same rows in the same
    tile places as the window path: identical bits."""
    lengths = [300, 2000] if ratio != 1 else [90, 700]
    plain = workloads.make_case(41, ratio, [3, 1], lengths)
    slots = workloads.make_case(41, ratio, [3, 1], lengths, ori_slots="window", ori_topk=128)
    assert slots["ori_indices"] is not None and (slots["ori_indices"] >= 0).sum() > 0
    for splits in (1, 3):
        a, la, _ = ora.tiled_attention(workloads.oracle_case(plain), splits=splits)
        b, lb, _ = ora.tiled_attention(workloads.oracle_case(slots), splits=splits)
        np.testing.assert_array_equal(a, b)
        np.testing.assert_array_equal(la, lb)


@pytest.mark.parametrize("ratio,mode", [(1, "draft"), (4, "draft"), (128, "shuffled"), (1, "shuffled")])
def test_slot_path_close_to_fp64_attention(ratio, mode):
    """Draft slots see the request's later rows too; shuffled slots carry
    holes, slots past the pool and a repeated slot.  The integer path stays
    within the reference's statistical gate of FP64 attention over the
    valid slots in order (reference.py:112-115)."""
    case = workloads.make_case(43, ratio, [4, 2], [600, 1500], ori_slots=mode, ori_topk=256)
    c = workloads.oracle_case(case)
    out, lse, _ = ora.tiled_attention(c, splits=2)
    ref, ref_lse = ora.fp64_attention(c)
    got = ora.bf16_to_f32(out).astype(np.float64)
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 0.01
    np.testing.assert_allclose(lse, ref_lse, rtol=2e-4, atol=2e-4)
    if mode == "draft":
        # Token 0 of request 0 sees rows up to the request's end: more than the window.
        assert (case["ori_indices"][0, 0] >= 0).sum() == 600 - (596 + 1 - 128)


def test_slot_integer_partials_by_brute_force():
    """QK int32 partials of explicit slots equal the codes times the rows at
    page = slot / 32, row = slot % 32 (no block table); holes score 0."""
    case = workloads.make_case(47, 128, [1, 1], [700, 300], ori_slots="shuffled", ori_topk=128)
    c = workloads.oracle_case(case)
    out, lse, dbg = ora.tiled_attention(c, splits=1, debug=True)
    kd = case["ori"]
    for t in range(2):
        qc = dbg["qcodes"][t, 0].astype(np.int64)
        for j, slot in enumerate(case["ori_indices"][t, 0]):
            s = dbg["scores"][t, j]
            if 0 <= slot < kd.pages * 32:
                row = ora.gather_slots(kd.pool, kd.page_stride, [slot])[0].astype(np.int64)
                np.testing.assert_array_equal(s[:8], qc[:8] @ row)
                np.testing.assert_array_equal(s[8:], qc[8:] @ row)
            else:
                assert not s.any()


def test_subcase_rows_reproduce_full_case_rows():
    """query_subcase (used to check large GPU launches on a row sample) keeps
    each row's selection, so the checker gives identical bits."""
    case = workloads.make_case(5, 4, [2, 3], [3000, 1200], index_mode="mixed")
    full, full_lse, _ = ora.tiled_attention(workloads.oracle_case(case), splits=3)
    rows = [0, 2, 4]
    sub = query_subcase(case, rows)
    part, part_lse, _ = ora.tiled_attention(workloads.oracle_case(sub), splits=3)
    np.testing.assert_array_equal(part, full[rows])
    np.testing.assert_array_equal(part_lse, full_lse[rows])


# ------------------------------------------------------------- cache writer

@pytest.mark.parametrize("int64,paired", [(False, False), (True, False), (False, True), (True, True)])
def test_cache_writer_oracle(int64, paired):
    """cache.py:16-69 + cache_write.cpp:38-73: codes of each valid row land at
    page*stride + offset*512; negative/out-of-range destinations are skipped;
    every other byte keeps its value."""
    rng = np.random.default_rng(7)
    pages, size, stride, rows = 6, 32, 32 * 512 + 4096, 40
    pool = np.full(pages * stride, 73, np.int8)
    upd = workloads.bf16_bits(rng.standard_normal((rows, 512), dtype=np.float32) * 3)
    scale = workloads.frozen_scale(workloads.bf16_value(upd))
    inv = ora.inverse_scale(scale)
    flat = rng.permutation(pages * size)[:rows].astype(np.int64)
    flat[3], flat[9] = -1, pages * size + 7
    if paired:
        slots = np.stack([flat // size, flat % size], 1)
        slots[9] = [pages, 0]
        slots[11] = [2, size]      # offset past the page
        slots[12] = [-5, 3]
    else:
        slots = flat
    slots = slots.astype(np.int64 if int64 else np.int32)
    written = ora.cache_write(pool, stride, pages, size, upd, slots, inv, paired=paired)
    expect = np.full_like(pool, 73)
    codes = workloads.encode(workloads.bf16_value(upd), scale)
    count = 0
    for r in range(rows):
        page, off = (int(slots[r, 0]), int(slots[r, 1])) if paired else (int(flat[r]) // size, int(flat[r]) % size)
        if (slots[r, 0] if paired else flat[r]) < 0 or page >= pages or not 0 <= off < size:
            continue
        expect[page * stride + off * 512: page * stride + off * 512 + 512] = codes[r]
        count += 1
    assert written == count
    np.testing.assert_array_equal(pool, expect)
