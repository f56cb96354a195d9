"""Write golden vectors from the reference's own CPU oracle.

Run in the build container only (the reference checkout is not on the GPU
box):  python tests/golden/make_golden.py [--reference /root/reference]

It imports npu_sparse_attn_sharedkv_int8.reference (reference.py) and records,
for seeded cases from tests/workloads.py, the inputs and the outputs of
  tiled_quantized_reference   reference.py:210-323  (BF16 out + FP32 LSE)
  joint_quantized_row         reference.py:175-207
  sharedkv_reference          reference.py:129-139  (FP64)
  CacheQuantization           reference.py:16-56    (inverse scale, codes)
  CacheQuantization.calibrate reference.py:32-37   (calibrate.npz)
These are the functions whose bits depend on torch's exp, log and reduction
order, which no test in the reference pins.  The vectors are data: inputs and
expected outputs, stored as .npz under tests/golden/vectors/.

Plans are (tile_size, splits, joint_dense, joint_sparse, joint_tile_limit,
dense_c4, query_group), the keyword arguments of tiled_quantized_reference.
Besides 128-key plans, every case family carries the plans the reference's
own device picks for that shape (the planners in the reference's
c4_wide.h:16-41, c128.cpp:79-105 and tests/support/attention_cases.py:56-111): config 0's
joint C128 row, config 1's 512-key tiles over 3 partitions, 512-key single
partition tiles for the batched, prefill and long-context C4/C128 slices,
and query groups of 2 (paired C4/C128 plans) and 4.
"""
import argparse
import sys
from dataclasses import replace
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from tests import workloads  # noqa: E402

# (name, seed, ratio, queries, lengths, index mode, page stride, plans)
# plan = (tile, splits, joint_dense, joint_sparse, joint_tile_limit[, dense_c4, query_group])
CASES = [
    # Config 0 of BASELINE (C128, B1, ctx 4096, seed 0); the reference device
    # runs it as one joint 128-key row (plan 2).
    ("c128_ctx4096", 0, 128, [1], [4096], None, 16384,
     [(128, 1, 0, 0, 256), (64, 3, 0, 0, 256), (128, 1, 1, 0, 256), (256, 2, 0, 0, 256)]),
    ("c4_raw_holes", 1, 4, [2], [4200], "holes", 16384,
     [(128, 1, 0, 0, 256), (256, 2, 0, 0, 256), (64, 5, 0, 0, 256), (128, 1, 0, 0, 256, 1, 1),
      (128, 1, 0, 0, 256, 0, 2)]),
    ("c4_compact_mixed", 2, 4, [1, 2], [1500, 900], "mixed", 20480,
     [(128, 1, 0, 0, 256), (64, 3, 0, 0, 256), (128, 2, 0, 0, 256, 1, 1)]),
    ("c4_joint_sparse", 5, 4, [1, 1], [600, 130], "mixed", 16384,
     [(256, 1, 0, 1, 256), (128, 1, 0, 0, 256)]),
    ("c128_mixed", 3, 128, [2, 1, 3], [100, 300, 1300], None, 16384,
     [(128, 1, 0, 0, 256), (64, 2, 0, 0, 256), (128, 1, 1, 0, 256), (128, 1, 0, 0, 256, 0, 2),
      (256, 1, 1, 0, 256, 0, 2)]),
    ("c4_dups", 4, 4, [1], [4400], "dups", 16384,
     [(128, 1, 0, 0, 256), (128, 3, 0, 0, 256), (128, 1, 0, 0, 256, 1, 1), (256, 2, 0, 0, 256, 1, 1)]),
    # Config 1 of BASELINE in full (C4, B1 T1, ctx 16384, 4096 compressed
    # rows, top-k 1024 uniform); the reference device splits it into 512-key
    # tiles over three partitions (plan 1).
    ("c4_cfg1", 10, 4, [1], [16384], "uniform", 16384,
     [(128, 1, 0, 0, 256), (512, 3, 0, 0, 256), (128, 5, 0, 0, 256)]),
    # Slice of the headline / config 2 C4 launch (two MTP pairs); reference
    # device plan: 512-key tiles, one partition (plan 1); plan 3 groups the
    # pairs (query_group 2, dense multiplicity list).
    ("c4_pairs", 11, 4, [2, 2], [3000, 6000], "uniform", 16384,
     [(128, 1, 0, 0, 256), (512, 1, 0, 0, 256), (128, 4, 0, 0, 256), (128, 1, 0, 0, 256, 0, 2),
      (256, 1, 0, 0, 256, 0, 2)]),
    # Slice of config 3 (chunked C4 prefill): four queries appended to a
    # cached prefix; reference device: 512-key tiles (plan 1); query groups
    # of 2 and 4 (plans 2, 3).
    ("c4_prefill", 12, 4, [4], [5000], "uniform", 16384,
     [(128, 1, 0, 0, 256), (512, 1, 0, 0, 256), (128, 1, 0, 0, 256, 0, 2), (128, 1, 0, 0, 256, 0, 4)]),
    # Slice of config 2 C128 / config 4 C128 (long contexts, MTP pairs); the
    # reference device's paired plans (256-key tiles, query_group 2) and
    # 512-key tiles.
    ("c128_pairs", 13, 128, [2, 2], [9000, 40000], None, 16384,
     [(128, 1, 0, 0, 256), (512, 1, 0, 0, 256), (256, 1, 0, 0, 256, 0, 2), (128, 3, 0, 0, 256)]),
    # Window-only (ratio 1) query groups.
    ("c1_group", 14, 1, [3, 2], [700, 90], None, 16384,
     [(128, 1, 0, 0, 256), (128, 1, 0, 0, 256, 0, 2), (64, 2, 0, 0, 256, 0, 3)]),
]
# Cases with other heads or explicit original slots:
# (name, seed, ratio, queries, lengths, index mode, page stride, plans, heads, ori slot mode, slots per row)
EXTRA = [
    # More than eight heads: reference.py:221-222 turns the Q/P residuals off.
    ("c128_heads16", 6, 128, [2, 1], [700, 2000], None, 16384, [(128, 1, 0, 0, 256), (128, 3, 0, 0, 256)],
     16, None, 0),
    ("c4_heads4", 7, 4, [1, 2], [3000, 1500], "uniform", 16384, [(128, 1, 0, 0, 256), (128, 2, 0, 0, 256)],
     4, None, 0),
    # Explicit physical original slots (reference.py:236-239, 285).
    ("c1_slots_shuffled", 8, 1, [2, 1], [600, 300], None, 16384, [(128, 1, 0, 0, 256), (128, 2, 0, 0, 256)],
     8, "shuffled", 256),
    ("c4_slots_draft", 9, 4, [3], [5000], "uniform", 16384, [(128, 1, 0, 0, 256), (128, 3, 0, 0, 256)],
     8, "draft", 256),
]


def torch_case(torch, ref, case):
    def cache(kind):
        pool = torch.from_numpy(kind.pool.copy())
        return pool.as_strided((kind.pages, 32, 1, 512), (kind.page_stride, 512, 512, 1))
    cmp = case["cmp"]
    return ref.SharedKVCase(
        q=torch.from_numpy(case["q"].view(np.int16).copy()).view(torch.bfloat16),
        ori=cache(case["ori"]), ori_block_table=torch.from_numpy(case["ori"].table),
        cu_q=torch.from_numpy(case["cu_q"]), seq_lens=torch.from_numpy(case["seq_lens"]),
        sink=torch.from_numpy(case["sink"]),
        cmp=cache(cmp) if cmp else None, cmp_block_table=torch.from_numpy(cmp.table) if cmp else None,
        cmp_indices=torch.from_numpy(case["cmp_indices"]) if case["cmp_indices"] is not None else None,
        ratio=case["ratio"], window=case["window"], softmax_scale=case["softmax_scale"],
        ori_indices=torch.from_numpy(case["ori_indices"]) if case.get("ori_indices") is not None else None)


def bits(t, torch):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument("--reference", default="/root/reference")
    parser.add_argument("--out", default=str(HERE / "vectors"))
    parser.add_argument("--only", nargs="*", help="write only these cases")
    args = parser.parse_args()
    sys.path.insert(0, args.reference)
    import torch
    from npu_sparse_attn_sharedkv_int8 import reference as ref

    torch.set_num_threads(4)
    out_dir = Path(args.out)
    out_dir.mkdir(parents=True, exist_ok=True)
    meta = dict(cpu_capability=torch.backends.cpu.get_cpu_capability(), torch=torch.__version__)
    cases = [c + (8, None, 0) for c in CASES] + EXTRA
    for name, seed, ratio, queries, lengths, mode, stride, plans, heads, slots, slot_count in cases:
        if args.only and name not in args.only:
            continue
        case = workloads.make_case(seed, ratio, queries, lengths, index_mode=mode or "uniform",
                                   page_stride=stride, heads=heads, ori_slots=slots, ori_topk=slot_count)
        tc = torch_case(torch, ref, case)
        oq = ref.CacheQuantization(torch.from_numpy(case["ori"].scale))
        cq = ref.CacheQuantization(torch.from_numpy(case["cmp"].scale)) if case["cmp"] else None
        record = dict(
            q=case["q"], ori_pool=case["ori"].pool, ori_stride=stride, ori_table=case["ori"].table,
            ori_scale=case["ori"].scale, cu_q=case["cu_q"], seq_lens=case["seq_lens"], sink=case["sink"],
            ratio=ratio, window=case["window"], softmax_scale=case["softmax_scale"],
            ori_inverse=oq.inverse_scale.numpy())
        # Codes of the first 64 source rows through CacheQuantization.quantize.
        src = workloads.bf16_value(case["ori"].values_bits[:64])
        record["quant_source_bits"] = case["ori"].values_bits[:64]
        record["quant_codes"] = oq.quantize(torch.from_numpy(src).bfloat16()).numpy()
        if cq is not None:
            record.update(cmp_pool=case["cmp"].pool, cmp_stride=stride, cmp_table=case["cmp"].table,
                          cmp_scale=case["cmp"].scale, cmp_inverse=cq.inverse_scale.numpy())
        if case["cmp_indices"] is not None:
            record["cmp_indices"] = case["cmp_indices"]
        if case.get("ori_indices") is not None:
            record.update(ori_indices=case["ori_indices"], ori_pages=case["ori"].pages)
        plans = [tuple(p) + (0, 1)[len(p) - 5:] for p in plans]
        record["plans"] = np.asarray(plans, dtype=np.int32)
        for i, (tile, splits, jd, js, limit, dense, group) in enumerate(plans):
            o, l = ref.tiled_quantized_reference(tc, oq, cq, tile_size=tile, splits=splits, return_lse=True,
                                                 joint_dense=bool(jd), joint_sparse=bool(js),
                                                 joint_tile_limit=limit, dense_c4=bool(dense),
                                                 query_group=group)
            record[f"out_{i}"] = bits(o, torch)
            record[f"lse_{i}"] = l.numpy()
        # FP64 attention over the decoded INT8 rows.
        decoded = replace(tc, ori=oq.dequantize(tc.ori), cmp=cq.dequantize(tc.cmp) if cq else None)
        o64, l64 = ref.sharedkv_reference(decoded)
        record["fp64_out"] = o64.numpy()
        record["fp64_lse"] = l64.numpy()
        np.savez_compressed(out_dir / f"{name}.npz", **record)
        print(name, {k: v.shape for k, v in record.items() if hasattr(v, "shape") and k.startswith("out")})

    if args.only:
        return
    # joint_quantized_row on explicit rows, with and without a bias.
    rng = np.random.default_rng(11)
    q = workloads.bf16_bits(rng.standard_normal((8, 512), dtype=np.float32))
    rows = [rng.integers(-127, 128, (n, 512)).astype(np.int8) for n in (37, 90)]
    scales = [np.abs(rng.standard_normal(512)).astype(np.float32) * 0.02 + 1e-3 for _ in range(2)]
    sink = np.linspace(-2, 2, 8, dtype=np.float32)
    bias = np.log(rng.integers(1, 4, 90).astype(np.float32))
    joint = dict(q=q, rows0=rows[0], rows1=rows[1], scale0=scales[0], scale1=scales[1], sink=sink, bias=bias)
    for tag, b in (("plain", None), ("bias", torch.from_numpy(bias))):
        o, l = ref.joint_quantized_row(torch.from_numpy(q.view(np.int16)).view(torch.bfloat16),
                                       [torch.from_numpy(r) for r in rows],
                                       [ref.CacheQuantization(torch.from_numpy(s)) for s in scales],
                                       torch.from_numpy(sink), 1 / np.sqrt(512),
                                       None if b is None else [None, b])
        joint[f"out_{tag}"] = bits(o, torch)
        joint[f"lse_{tag}"] = l.numpy()
    np.savez_compressed(out_dir / "joint_rows.npz", **joint)

    # CacheQuantization.calibrate over several samples (FP32 and BF16, with
    # and without a head axis), and a zero channel that the 1e-8 floor holds.
    rng = np.random.default_rng(12)
    samples = [rng.standard_normal((37, 512), dtype=np.float32) * 3,
               workloads.bf16_bits(rng.standard_normal((9, 1, 512), dtype=np.float32) * 20),
               rng.standard_normal((5, 512), dtype=np.float32)]
    samples[0][:, 7] = 0
    samples[1][..., 7] = 0
    samples[2][:, 7] = 0
    tensors = [torch.from_numpy(samples[0]),
               torch.from_numpy(samples[1].view(np.int16)).view(torch.bfloat16),
               torch.from_numpy(samples[2])]
    calib = dict(sample0=samples[0], sample1_bf16=samples[1], sample2=samples[2],
                 scale=ref.CacheQuantization.calibrate(tensors).scale.numpy())
    np.savez_compressed(out_dir / "calibrate.npz", **calib)
    (out_dir / "meta.txt").write_text("".join(f"{k}={v}\n" for k, v in meta.items()))
    print("meta", meta)


if __name__ == "__main__":
    main()
