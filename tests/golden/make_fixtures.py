"""Convert the reference's real-activation fixtures into a compact .npz.

Run in the build container only (the reference checkout is not on the GPU
box):  python tests/golden/make_fixtures.py [--reference /root/reference]

Sources, both loaded with torch.load(weights_only=True), nothing executed:
  tests/fixtures/activations/<layer>.call_1.pt   one captured sample per layer:
      query [8, 512], original [n, 512], compressed [m, 512] (BF16 values held
      as FP64), sink [8], softmax_scale, actual [8, 512] (the model's BF16
      output) and reference [8, 512] (FP64 attention over those rows)
  tests/fixtures/activations/metrics.jsonl      per-layer ratio and key counts
  npu_sparse_attn_sharedkv_int8/data/scales_v1.pt  frozen serving scales
      (protocol sharedkv-c8-v1), <layer>.ori / <layer>.cmp FP32 [512]
The reference's own tests build cases from these (tests/support/
serving_shapes.py:33-57) and gate the INT8 kernel with relative L2 < .04 and
min head cosine > .999 (tests/npu/test_attention.py:56, 110).

Output tests/golden/vectors/activations.npz: per layer <i>, q/ori/cmp/actual
as BF16 bits (uint16), reference FP64, sink FP32, softmax_scale, ratio, the
frozen scales FP32, and the layer name.
"""
import argparse
import json
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def bf16_bits_exact(t):
    """FP64 tensor holding BF16 values -> uint16 bits (asserts exactness)."""
    import torch
    b = t.to(torch.bfloat16)
    assert torch.equal(b.double(), t), "fixture values are not BF16"
    return b.view(torch.int16).numpy().view(np.uint16).copy()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    import torch
    ref = Path(args.reference)
    fixtures = ref / "tests" / "fixtures" / "activations"
    scales = torch.load(ref / "npu_sparse_attn_sharedkv_int8" / "data" / "scales_v1.pt",
                        map_location="cpu", weights_only=True)
    assert scales["protocol"] == "sharedkv-c8-v1"
    records = [json.loads(x) for x in (fixtures / "metrics.jsonl").read_text().splitlines()]
    out = {}
    for i, r in enumerate(records):
        layer = r["layer"]
        s = torch.load(fixtures / f"{layer}.call_{r['call']}.pt", map_location="cpu", weights_only=True)
        out[f"{i}_layer"] = np.array(layer)
        out[f"{i}_ratio"] = np.int32(r["ratio"])
        out[f"{i}_q"] = bf16_bits_exact(s["query"])
        out[f"{i}_ori"] = bf16_bits_exact(s["original"])
        out[f"{i}_cmp"] = bf16_bits_exact(s["compressed"])
        out[f"{i}_actual"] = bf16_bits_exact(s["actual"])
        out[f"{i}_reference"] = s["reference"].numpy().astype(np.float64)
        out[f"{i}_sink"] = s["sink"].float().numpy()
        out[f"{i}_softmax_scale"] = np.float64(s["softmax_scale"])
        out[f"{i}_ori_scale"] = scales["scales"][layer + ".ori"].numpy().astype(np.float32)
        if r["ratio"] != 1:
            out[f"{i}_cmp_scale"] = scales["scales"][layer + ".cmp"].numpy().astype(np.float32)
    out["count"] = np.int32(len(records))
    dest = HERE / "vectors" / "activations.npz"
    np.savez_compressed(dest, **out)
    print(f"wrote {dest} ({dest.stat().st_size} bytes, {len(records)} layers)")


if __name__ == "__main__":
    main()
