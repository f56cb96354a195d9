"""Calibration of the frozen "sharedkv-c8-v1" scales: observe, merge, load.

Interface counterparts in the reference checkout:
  CacheObserver     npu_sparse_attn_sharedkv_int8/calibration.py:16-73
  merge step        docs/kv-cache.md:51-68 (steps 3-4: per-channel maximum
                    over ranks, scale = clamp_min(margin * maximum / 127, 1e-8))
  load_scales       npu_sparse_attn_sharedkv_int8/vllm_adapter.py:52-63

The observer watches the BF16 cache updates a serving engine writes (after
RoPE) without changing them, keeps a per-channel absolute maximum and a row
count per (layer prefix, cache kind), and checkpoints them to
<directory>/rank_XX.pt while <directory>/collect exists.  It synchronises the
device at every checkpoint, so it is a calibration tool, never a benchmark
configuration.  merge_observations() turns the rank files of one deployment
into the frozen scale file that load_scales() validates and the INT8 path
reads.  Every file here is written by this module and read with
torch.load(weights_only=True).
"""
import atexit
import hashlib
import os
from pathlib import Path
import time

import torch

PROTOCOL = "sharedkv-c8-v1"
DIM = 512
MARGIN = 1.1
FLOOR = 1e-8
CHECKPOINT_SECONDS = 10


def _capturing():
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


class CacheObserver:
    """Per-channel |x| maxima of the cache updates while `collect` exists."""

    def __init__(self, directory):
        self.directory = Path(directory)
        self.directory.mkdir(parents=True, exist_ok=True)
        self.marker = self.directory / "collect"
        self.stats = {}
        self.dirty = False
        self.last_save = time.monotonic()
        atexit.register(self.flush)

    @torch.inference_mode()
    def observe(self, prefix, kind, cache, updates, slots):
        """Record one cache write: `updates` [T,512] or [T,1,512], `slots` the
        writer's flat [T] or paired [T,2] slots into `cache` [pages,32,1,512].
        Rows whose slot the writer would skip are not counted."""
        if not self.marker.exists():
            self.flush()
            return
        if updates is None or updates.shape[0] == 0:
            return
        if _capturing():
            raise RuntimeError("Calibration needs eager execution; keep the marker absent during graph capture")
        if updates.shape[-1] != DIM or cache.shape[-1] != DIM:
            raise ValueError("Calibration expects the D=512 shared KV cache")
        pages, page_size = cache.shape[0], cache.shape[1]
        if slots.ndim == 1:
            valid = (slots >= 0) & (slots < pages * page_size)
        else:
            valid = (slots[:, 0] >= 0) & (slots[:, 0] < pages) & (slots[:, 1] >= 0) & (slots[:, 1] < page_size)
        rows = updates.reshape(-1, DIM).float()
        peak = torch.where(valid[:, None], rows, 0.0).abs().amax(0)
        count = valid.sum()
        key = f"{prefix}.{kind}"
        entry = self.stats.get(key)
        if entry is None:
            self.stats[key] = [peak, count]
        else:
            torch.maximum(entry[0], peak, out=entry[0])
            entry[1].add_(count)
        self.dirty = True
        if time.monotonic() - self.last_save >= CHECKPOINT_SECONDS:
            self.flush()

    def flush(self):
        """Checkpoint to rank_XX.pt (atomic rename); no-op when nothing changed."""
        if not self.dirty:
            return
        keys = sorted(self.stats)
        maxima = torch.stack([self.stats[k][0] for k in keys]).cpu()
        counts = torch.stack([self.stats[k][1] for k in keys]).cpu()
        if not bool(torch.isfinite(maxima).all()):
            raise RuntimeError("Non-finite cache values observed during calibration")
        rank = torch.distributed.get_rank() if torch.distributed.is_initialized() else 0
        payload = {"version": 1, "rank": rank, "pid": os.getpid(),
                   "stats": {k: {"maximum": maxima[i].clone(), "rows": int(counts[i])} for i, k in enumerate(keys)}}
        path = self.directory / f"rank_{rank:02d}.pt"
        temporary = path.with_suffix(f".tmp.{os.getpid()}")
        torch.save(payload, temporary)
        os.replace(temporary, path)
        self.dirty = False
        self.last_save = time.monotonic()


def _sha256(path):
    digest = hashlib.sha256()
    with open(path, "rb") as handle:
        for block in iter(lambda: handle.read(1 << 20), b""):
            digest.update(block)
    return digest.hexdigest()


def merge_observations(paths, margin=MARGIN, required=None, provenance=None):
    """Frozen scales from the observers' rank files.

    Per key: maximum over ranks of each channel's maximum, rows summed, and
    scale = max(fp32(margin * maximum) / 127, 1e-8) in FP32.  `required`
    (an iterable of keys) makes a missing or unobserved key an error.
    Returns the payload load_scales() accepts; torch.save() it to publish.
    """
    if not margin > 0:
        raise ValueError("margin must be positive")
    maxima, rows, sources = {}, {}, {}
    for path in sorted(str(p) for p in paths):
        payload = torch.load(path, map_location="cpu", weights_only=True)
        if payload.get("version") != 1 or not isinstance(payload.get("stats"), dict):
            raise ValueError(f"Not an observer checkpoint: {path}")
        for key, entry in payload["stats"].items():
            peak = entry["maximum"]
            if peak.shape != (DIM,) or peak.dtype != torch.float32 or not bool(torch.isfinite(peak).all()):
                raise ValueError(f"Invalid maximum for {key} in {path}")
            maxima[key] = torch.maximum(maxima[key], peak) if key in maxima else peak.clone()
            rows[key] = rows.get(key, 0) + int(entry["rows"])
        sources[os.path.basename(path)] = _sha256(path)
    for key in required or ():
        if rows.get(key, 0) == 0:
            raise ValueError(f"No observed rows for {key}")
    factor = torch.tensor(margin, dtype=torch.float32)
    scales = {key: torch.clamp((factor * peak) / 127, min=FLOOR) for key, peak in sorted(maxima.items())}
    return {"protocol": PROTOCOL, "scales": scales, "margin": float(margin),
            "observed_rows_across_ranks": dict(sorted(rows.items())), "source_sha256": sources,
            "provenance": dict(provenance or {})}


def validate_scales(payload):
    """The checks of the reference's load_scales: protocol name, then every
    vector FP32[512], finite and strictly positive.  Returns the scale dict."""
    if not isinstance(payload, dict) or payload.get("protocol") != PROTOCOL:
        raise ValueError("Wrong shared-KV scale protocol")
    scales = payload.get("scales")
    if not isinstance(scales, dict):
        raise ValueError("Scale file has no scale dictionary")
    for key, value in scales.items():
        if (not isinstance(value, torch.Tensor) or value.shape != (DIM,) or value.dtype != torch.float32
                or not bool(torch.isfinite(value).all() & (value > 0).all())):
            raise ValueError(f"Invalid scale vector: {key}")
    return scales


def load_scale_file(path):
    """Read a frozen scale file without executing anything from it."""
    return validate_scales(torch.load(path, map_location="cpu", weights_only=True))
