"""Calibration of the frozen "sharedkv-c8-v1" scales: observe, merge, load.

Documented workflow followed (docs/kv-cache.md:51-68 of the reference
checkout): while <directory>/collect exists, every rank records, per layer
prefix and cache kind, the channel-wise absolute maximum of the BF16 cache
updates it writes and how many rows it wrote, and checkpoints them to
<directory>/rank_XX.pt ({"version": 1, "rank", "pid", "stats": {key:
{"maximum": FP32[512], "rows": int}}}); merge_observations() combines the
rank files into the scale payload that load_scales() validates
(vllm_adapter.py:52-63 there).

This build's observer keeps all maxima of a rank in one device tensor
[keys, 512] and the row counts in one [keys] tensor (a key's row index is
assigned on first sight), so an observation is one masked reduction and two
in-place updates with no host round trip.  The collect marker is looked up
at most once per MARKER_POLL_SECONDS; when it disappears the statistics are
checkpointed once.  Checkpoints copy to the host (a device synchronisation),
so the observer is a calibration tool, never a benchmark configuration.
Every file here is written by this module and read with
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
CHECKPOINT_SECONDS = 10.0
MARKER_POLL_SECONDS = 1.0


def _capturing():
    return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()


def written_rows(cache, slots):
    """Mask of the update rows PreparedCacheWrite stores: flat slots in
    [0, pages * page_size), or (page, offset) pairs inside the cache
    (cache_write.cpp:53-63 of the reference)."""
    pages, page_size = cache.shape[0], cache.shape[1]
    if slots.ndim == 1:
        return (slots >= 0) & (slots < pages * page_size)
    page, offset = slots[:, 0], slots[:, 1]
    return (page >= 0) & (page < pages) & (offset >= 0) & (offset < page_size)


def write_rank_file(directory, rank, maxima, rows):
    """Atomically (re)write <directory>/rank_XX.pt from {key: maximum} and
    {key: rows}."""
    stats = {key: {"maximum": maxima[key], "rows": int(rows[key])} for key in sorted(maxima)}
    payload = {"version": 1, "rank": rank, "pid": os.getpid(), "stats": stats}
    target = Path(directory) / f"rank_{rank:02d}.pt"
    staging = target.with_name(f".{target.name}.{os.getpid()}.partial")
    torch.save(payload, staging)
    os.replace(staging, target)
    return target


class CacheObserver:
    """Channel maxima and row counts of observed cache writes, per
    "<layer prefix>.<kind>" key, while <directory>/collect exists."""

    def __init__(self, directory, checkpoint_seconds=CHECKPOINT_SECONDS):
        self.directory = Path(directory)
        self.directory.mkdir(parents=True, exist_ok=True)
        self.marker = self.directory / "collect"
        self.checkpoint_seconds = checkpoint_seconds
        self.keys = {}                # key -> row of maxima / rows
        self.maxima = None            # FP32 [keys, 512] on the observed device
        self.rows = None              # int64 [keys]
        self.pending = False          # observations not yet checkpointed
        self._marker_seen = (-1e9, False)
        self._checkpointed_at = time.monotonic()
        atexit.register(self.flush)

    @property
    def stats(self):
        """{key: (maximum FP32[512], rows)} (views of the accumulators)."""
        if self.maxima is None:
            return {}
        return {key: (self.maxima[i], self.rows[i]) for key, i in self.keys.items()}

    def collecting(self):
        now = time.monotonic()
        checked, present = self._marker_seen
        if now - checked >= MARKER_POLL_SECONDS:
            present = self.marker.exists()
            self._marker_seen = (now, present)
        return present

    def _slot(self, key, device):
        i = self.keys.get(key)
        if i is None:
            i = self.keys[key] = len(self.keys)
            grow = torch.zeros(1, DIM, dtype=torch.float32, device=device)
            count = torch.zeros(1, dtype=torch.int64, device=device)
            self.maxima = grow if self.maxima is None else torch.cat([self.maxima, grow])
            self.rows = count if self.rows is None else torch.cat([self.rows, count])
        return i

    @torch.inference_mode()
    def observe(self, prefix, kind, cache, updates, slots):
        """One cache write: `updates` [T, 512] or [T, 1, 512] going to
        `slots` (flat [T] or paired [T, 2]) of `cache` [pages, 32, 1, 512].
        Rows the writer would skip are not observed."""
        if not self.collecting():
            self.flush()
            return
        if updates is None or updates.shape[0] == 0:
            return
        if _capturing():
            raise RuntimeError("Calibration needs eager execution; keep the marker absent during graph capture")
        if updates.shape[-1] != DIM or cache.shape[-1] != DIM:
            raise ValueError("Calibration expects the D=512 shared KV cache")
        keep = written_rows(cache, slots)
        values = updates.reshape(-1, DIM).float().abs()
        peak = values.masked_fill(~keep[:, None], 0.0).amax(0)
        i = self._slot(f"{prefix}.{kind}", updates.device)
        torch.maximum(self.maxima[i], peak, out=self.maxima[i])
        self.rows[i] += keep.sum()
        self.pending = True
        if time.monotonic() - self._checkpointed_at >= self.checkpoint_seconds:
            self.flush()

    def flush(self):
        """Checkpoint to rank_XX.pt if anything was observed since the last one."""
        if not self.pending:
            return
        maxima, rows = self.maxima.cpu(), self.rows.cpu()
        if not bool(torch.isfinite(maxima).all()):
            raise RuntimeError("Non-finite cache values observed during calibration")
        rank = torch.distributed.get_rank() if torch.distributed.is_initialized() else 0
        write_rank_file(self.directory, rank, {k: maxima[i].clone() for k, i in self.keys.items()},
                        {k: rows[i] for k, i in self.keys.items()})
        self.pending = False
        self._checkpointed_at = time.monotonic()


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
