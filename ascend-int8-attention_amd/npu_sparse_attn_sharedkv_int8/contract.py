"""Inputs of the shared-KV INT8 path: the frozen KV encoding and the case container.

Interface counterparts in the reference checkout (same names, fields and
error behaviour, so caller code is unchanged):
  CacheQuantization   npu_sparse_attn_sharedkv_int8/reference.py:16-56
  SharedKVCase        npu_sparse_attn_sharedkv_int8/reference.py:59-79

Encoding "sharedkv-c8-v1" (one FP32 scale per channel, K and V share the row):
  inverse[c] = fp32(1 / fp64(scale[c]))
  code       = clamp(round_half_even(fp32(x) * inverse[c]), -127, 127)
  value      = code * scale[c]
The GPU writer (PreparedCacheWrite) applies the same encoding in a HIP kernel;
the methods here are host conveniences for calibration and tests.  This
package has no CPU implementation of attention.
"""
from dataclasses import dataclass, fields
import math

import torch

DIM = 512
_FLOOR = 1e-8


def _validated(scale):
    if not isinstance(scale, torch.Tensor) or scale.dtype != torch.float32 or tuple(scale.shape) != (DIM,):
        raise ValueError("scale must be float32[512]")
    finite = torch.isfinite(scale).all()
    positive = (scale > 0).all()
    if not bool(finite and positive):
        raise ValueError("scale must be finite and strictly positive")
    return scale


@dataclass(frozen=True)
class CacheQuantization:
    """Frozen symmetric per-channel INT8 scales for one cache kind.

    Scales are fixed before the cache is populated and never move when tokens
    are appended, so codes already written stay valid.
    """

    scale: torch.Tensor

    def __post_init__(self):
        _validated(self.scale)

    @classmethod
    def calibrate(cls, samples):
        """Per-channel abs-max over the samples, divided by 127 (floor 1e-8)."""
        peak = torch.zeros(DIM, dtype=torch.float32)
        for rows in samples:
            batch_peak = rows.float().reshape(-1, DIM).abs().amax(dim=0).cpu()
            peak = torch.maximum(peak, batch_peak)
        return cls(torch.clamp(peak / 127, min=_FLOOR))

    @classmethod
    def from_msmodelslim(cls, tensors, prefix):
        """Scales exported by msModelSlim; only zero offsets (symmetric) are accepted."""
        offsets = tensors[prefix + ".kv_cache_offset"].float().reshape(-1)
        if bool((offsets != 0).any()):
            raise ValueError("Protocol v1 requires symmetric C8; nonzero offsets are unsupported")
        return cls(tensors[prefix + ".kv_cache_scale"].float().reshape(-1))

    @property
    def inverse_scale(self):
        """fp32(1 / fp64(scale)), computed once; the writer kernel consumes it."""
        return (1.0 / self.scale.to(torch.float64)).to(torch.float32)

    def quantize(self, x):
        inverse = self.inverse_scale.to(x.device)
        codes = torch.round(x.to(torch.float32) * inverse)   # torch.round is half-to-even
        return torch.clamp(codes, -127, 127).to(torch.int8)

    def dequantize(self, x):
        return x.to(torch.float32) * self.scale.to(x.device)


@dataclass
class SharedKVCase:
    """One attention launch's inputs.

    q                BF16 [T, H, 512], contiguous (TND layout)
    ori              INT8 [pages, 32, 1, 512] original (SWA) cache; page stride may exceed 16 KiB
    ori_block_table  INT32 [batch, logical pages] -> physical page
    cu_q             INT32 [batch + 1] query boundaries
    seq_lens         INT32 [batch] KV length of each request, new tokens included
    sink             FP32 [H] per-head sink logit (denominator only)
    cmp, cmp_block_table   compressed cache and its table (ratio 4 or 128)
    cmp_indices      INT32 [T, 1, topk] logical compressed rows for ratio 4; negative = padding
    ratio            1 (window only), 4 (C4 top-k) or 128 (C128 all rows)
    window           original window length (128 on the C8 path)
    softmax_scale    logit scale, default 1/sqrt(512)
    ori_indices      explicit physical original slots (not served by the C8 path)
    """

    q: torch.Tensor
    ori: torch.Tensor
    ori_block_table: torch.Tensor
    cu_q: torch.Tensor
    seq_lens: torch.Tensor
    sink: torch.Tensor
    cmp: torch.Tensor | None = None
    cmp_block_table: torch.Tensor | None = None
    cmp_indices: torch.Tensor | None = None
    ratio: int = 1
    window: int = 128
    softmax_scale: float = 1 / math.sqrt(DIM)
    ori_indices: torch.Tensor | None = None

    def to(self, device):
        """Copy of the case with every tensor moved to `device`."""
        moved = {}
        for f in fields(self):
            value = getattr(self, f.name)
            moved[f.name] = value.to(device) if isinstance(value, torch.Tensor) else value
        return SharedKVCase(**moved)
