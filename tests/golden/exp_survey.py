"""How far the checker's exponential is from torch.exp, and what that does to
the P codes (run in the build container; writes exp_survey.json).

reference.py computes every softmax weight with torch.exp (reference.py:305,
317).  On the CPU, torch.exp of float32 is MKL's vector exponential: its bits
depend on the MKL code path the host CPU selects (AVX-512, AVX2, the
conditional-reproducibility modes), and it is not correctly rounded.  The
checker and the HIP kernels share sko_expf (Cody-Waite reduction, degree-8
Taylor polynomial).  This script measures

  1. sko_expf against torch.exp and against the correctly rounded exp
     (float64 exp rounded once) on every float32 in [-87, 0], the arguments
     the softmax produces (logit - running max <= 0; below -87 both sides
     give zero or a subnormal that rounds to zero P codes);
  2. the P-code flips on the golden cases: for every softmax weight of every
     non-joint, ungrouped golden plan with eight heads, the exponential's
     argument (oracle debug dump `weight_args`) is fed to both exponentials
     and the two-term codes p8 = rne(w * 127), p_low = rne((w * 127 - p8) *
     127) (reference.py:309-312) are compared.  The checker's own dumped P
     codes are first reproduced from sko_expf to make sure the arguments are
     the ones the tile loop used.

Usage: python tests/golden/exp_survey.py [--skip-exhaustive]
"""
import argparse
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

import oracle.oracle as ora  # noqa: E402
from tests.test_oracle import CASES, GOLDEN, golden_case, golden_plans  # noqa: E402


def p_codes(w):
    x = (w * np.float32(127)).astype(np.float32)
    hi = np.rint(x)
    lo = np.rint(((x - hi) * np.float32(127)).astype(np.float32))
    return hi.astype(np.int32), lo.astype(np.int32)


def exhaustive(torch):
    lo_bits, hi_bits = 0x80000000, 0xC2AE0000 + 1          # -0 .. -87
    chunk = 1 << 25
    stats = dict(inputs=0, sko_vs_torch=0, sko_vs_cr=0, torch_vs_cr=0, sko_vs_torch_over_1ulp=0)
    for start in range(lo_bits, hi_bits, chunk):
        x = np.arange(start, min(hi_bits, start + chunk), dtype=np.uint64).astype(np.uint32).view(np.float32)
        a = ora.expf(x).view(np.int32).astype(np.int64)
        t = torch.exp(torch.from_numpy(x)).numpy().view(np.int32).astype(np.int64)
        c = np.exp(x.astype(np.float64)).astype(np.float32).view(np.int32).astype(np.int64)
        stats["inputs"] += x.size
        stats["sko_vs_torch"] += int((a != t).sum())
        stats["sko_vs_cr"] += int((a != c).sum())
        stats["torch_vs_cr"] += int((t != c).sum())
        stats["sko_vs_torch_over_1ulp"] += int((np.abs(a - t) > 1).sum())
    return stats


def flips(torch):
    total = dict(weights=0, p8_flips=0, plo_flips=0, either=0)
    per_case = {}
    for name in CASES:
        z = np.load(GOLDEN / f"{name}.npz")
        if z["q"].shape[1] != 8 or ("ori_indices" in z.files and z["ori_indices"].shape[-1] > 128):
            continue
        case = golden_case(z)
        for i, (tile, splits, jd, js, limit, dense, group) in enumerate(golden_plans(z)):
            if jd or js or group != 1 or tile > 128:
                continue
            _, _, dbg = ora.tiled_attention(case, tile, splits, dense_c4=bool(dense), debug=True)
            live = int(z["cu_q"][-1])
            probs = dbg["probs"][:live]
            args = dbg["weight_args"][:live]
            visited = ~np.isnan(args).any(-1)          # positions the tile loop reached (NaN elsewhere)
            x = args[visited]                          # [n, 8]
            ours_hi, ours_lo = p_codes(ora.expf(x))
            assert np.array_equal(ours_hi, probs[visited][:, :8]), (name, i)
            assert np.array_equal(ours_lo, probs[visited][:, 8:]), (name, i)
            th, tl = p_codes(torch.exp(torch.from_numpy(np.ascontiguousarray(x))).numpy())
            f8, fl = int((th != ours_hi).sum()), int((tl != ours_lo).sum())
            n = int(x.size)
            per_case[f"{name}/plan{i}"] = dict(weights=n, p8_flips=f8, plo_flips=fl)
            total["weights"] += n
            total["p8_flips"] += f8
            total["plo_flips"] += fl
            total["either"] += int(((th != ours_hi) | (tl != ours_lo)).sum())
    return total, per_case


def main():
    parser = argparse.ArgumentParser()
    parser.add_argument("--skip-exhaustive", action="store_true")
    parser.add_argument("--out", default=str(GOLDEN / "exp_survey.json"))
    args = parser.parse_args()
    import torch
    torch.set_num_threads(8)
    result = dict(cpu_capability=torch.backends.cpu.get_cpu_capability(), torch=torch.__version__,
                  mkl=bool(torch.backends.mkl.is_available()))
    if not args.skip_exhaustive:
        result["exhaustive_minus87_to_0"] = exhaustive(torch)
    total, per_case = flips(torch)
    result["p_code_flips_total"] = total
    result["p_code_flips"] = per_case
    Path(args.out).write_text(json.dumps(result, indent=1) + "\n")
    print(json.dumps({k: v for k, v in result.items() if k != "p_code_flips"}, indent=1))


if __name__ == "__main__":
    main()
