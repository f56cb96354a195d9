"""numpy/ctypes front end of the CPU oracle (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, as the checker.  The product package never does.

Functions mirror npu_sparse_attn_sharedkv_int8/reference.py of the reference
checkout:
  inverse_scale / quantize     reference.py:47-56 (CacheQuantization)
  calibrate_scale              reference.py:32-37 (+ docs/kv-cache.md margin rule)
  cache_write                  cache.py:16-69, csrc/kernels/cache_write.cpp:38-73
  tiled_attention              reference.py:210-323 (tiled_quantized_reference)
  joint_row                    reference.py:175-207 (joint_quantized_row)
  fp64_attention               reference.py:129-139 (sharedkv_reference)
"""
import ctypes
import math
import os
import subprocess
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "libsharedkv_oracle.so"
DIM = 512


def build():
    """Compile the oracle in place (make; gcc only)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        _lib = ctypes.CDLL(str(LIBRARY))
        _lib.sko_expf.restype = ctypes.c_float
        _lib.sko_expf.argtypes = [ctypes.c_float]
        _lib.sko_tree_sum.restype = ctypes.c_float
        _lib.sko_tree_sum.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_int32]
        _lib.sko_cache_write.restype = ctypes.c_int64
        _lib.sko_tiled_attention.restype = ctypes.c_int
    return _lib


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else ctypes.c_void_p(0)


# ---------------------------------------------------------------- bf16

def bf16_to_f32(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x):
    """Round to nearest even, as torch's .bfloat16()."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


# ---------------------------------------------------------------- encoding

def inverse_scale(scale):
    """reference.py:47-50: fp32(1 / fp64(scale))."""
    return (1.0 / np.asarray(scale, dtype=np.float32).astype(np.float64)).astype(np.float32)


def quantize(x, inverse):
    """reference.py:52-53 on fp32 values: round half-even, clamp to [-127, 127]."""
    v = np.rint(np.asarray(x, dtype=np.float32) * inverse.astype(np.float32))
    return np.clip(v, -127, 127).astype(np.int8)


def calibrate_scale(rows, margin=1.0):
    """reference.py:32-37 (margin 1.0) and the frozen-scale rule of
    docs/kv-cache.md: scale = max(margin * absmax / 127, 1e-8)."""
    amax = np.abs(np.asarray(rows, dtype=np.float32).reshape(-1, DIM)).max(0)
    return np.maximum((np.float32(margin) * amax) / np.float32(127), np.float32(1e-8)).astype(np.float32)


def cache_write(pool, page_stride, pages, page_size, updates_bf16, slots, inverse, paired=False):
    """Host restatement of the writer; pool is a flat int8 byte array."""
    updates_bf16 = np.ascontiguousarray(updates_bf16, dtype=np.uint16).reshape(len(updates_bf16), -1)
    slots = np.ascontiguousarray(slots)
    int64_slots = slots.dtype == np.int64
    assert slots.dtype in (np.int32, np.int64)
    slot_stride = 2 if paired else 1
    inverse = np.ascontiguousarray(inverse, dtype=np.float32)
    return lib().sko_cache_write(
        _ptr(pool), ctypes.c_int64(pages), ctypes.c_int64(page_size), ctypes.c_int64(page_stride),
        _ptr(updates_bf16), ctypes.c_int64(len(updates_bf16)), ctypes.c_int64(updates_bf16.shape[1]),
        _ptr(slots), ctypes.c_int(int(int64_slots)), ctypes.c_int(int(paired)),
        ctypes.c_int64(slot_stride), ctypes.c_int64(1 if paired else 0), _ptr(inverse))


def expf(x):
    """sko_expf elementwise (the checker's and the kernels' exponential)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().sko_expf_array(_ptr(x), _ptr(y), ctypes.c_int64(x.size))
    return y


# ---------------------------------------------------------------- attention

@dataclass
class Case:
    """Host copy of reference.py:59-73 SharedKVCase.

    ori / cmp are flat int8 byte pools; page p starts at p * *_stride bytes."""
    q: np.ndarray                  # uint16 bf16 bits [T, H, 512]
    ori: np.ndarray                # int8 flat pool
    ori_stride: int
    ori_table: np.ndarray          # int32 [B, W]
    cu_q: np.ndarray               # int32 [B + 1]
    seq_lens: np.ndarray           # int32 [B]
    sink: np.ndarray               # f32 [H]
    ori_scale: np.ndarray          # f32 [512]
    cmp: np.ndarray = None
    cmp_stride: int = 0
    cmp_table: np.ndarray = None
    cmp_scale: np.ndarray = None
    cmp_indices: np.ndarray = None  # int32 [T, 1, topk]
    ratio: int = 1
    window: int = 128
    softmax_scale: float = 1 / math.sqrt(DIM)
    block: int = 32
    extra: dict = field(default_factory=dict)
    ori_indices: np.ndarray = None  # int32 [T, 1, K] physical original slots (reference.py:73)
    ori_pages: int = 0              # pages of the original pool (slot capacity = pages * block)


class _Case(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p), ("ori", ctypes.c_void_p), ("ori_stride", ctypes.c_int64),
        ("ori_table", ctypes.c_void_p), ("ori_table_width", ctypes.c_int32),
        ("cmp", ctypes.c_void_p), ("cmp_stride", ctypes.c_int64),
        ("cmp_table", ctypes.c_void_p), ("cmp_table_width", ctypes.c_int32),
        ("cmp_indices", ctypes.c_void_p), ("topk", ctypes.c_int32),
        ("cu_q", ctypes.c_void_p), ("seq_lens", ctypes.c_void_p), ("batch", ctypes.c_int32),
        ("sink", ctypes.c_void_p), ("ori_scale", ctypes.c_void_p), ("cmp_scale", ctypes.c_void_p),
        ("tokens", ctypes.c_int32), ("heads", ctypes.c_int32), ("block", ctypes.c_int32),
        ("ratio", ctypes.c_int32), ("window", ctypes.c_int32), ("softmax_scale", ctypes.c_float),
        ("ori_slots", ctypes.c_void_p), ("ori_topk", ctypes.c_int32), ("ori_pages", ctypes.c_int32),
    ]


class _Plan(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("tile", "splits", "joint_dense", "joint_sparse", "joint_tile_limit", "dense_c4",
                 "query_group")]


class _Debug(ctypes.Structure):
    _fields_ = [("qcodes", ctypes.c_void_p), ("alpha", ctypes.c_void_p), ("scores", ctypes.c_void_p),
                ("probs", ctypes.c_void_p), ("values", ctypes.c_void_p),
                ("cmp_capacity", ctypes.c_int32), ("tile_capacity", ctypes.c_int32),
                ("weight_args", ctypes.c_void_p)]


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


def tiled_attention(case, tile=128, splits=1, return_lse=True, joint_dense=False, joint_sparse=False,
                    joint_tile_limit=256, dense_c4=False, debug=False, threads=None,
                    cmp_capacity=None, tile_capacity=None, query_group=1):
    """reference.py:210-323.  Returns (out_bf16_bits [T,H,512], lse [T,H], debug dict or None).
    debug (query_group 1, eight heads) adds the integer dumps and the
    softmax-weight exponential arguments (weight_args)."""
    q = _c(case.q, np.uint16)
    T, H, _ = q.shape
    keep = dict(q=q, ori=_c(case.ori, np.int8), ot=_c(case.ori_table, np.int32),
                cmp=_c(case.cmp, np.int8), ct=_c(case.cmp_table, np.int32),
                ix=_c(case.cmp_indices, np.int32), cu=_c(case.cu_q, np.int32),
                sl=_c(case.seq_lens, np.int32), sink=_c(case.sink, np.float32),
                os=_c(case.ori_scale, np.float32), cs=_c(case.cmp_scale, np.float32),
                oi=_c(case.ori_indices, np.int32))
    topk = keep["ix"].shape[-1] if keep["ix"] is not None else 0
    ori_topk = keep["oi"].shape[-1] if keep["oi"] is not None else 0
    if keep["oi"] is not None and not case.ori_pages:
        raise ValueError("explicit original slots need ori_pages")
    c = _Case(_ptr(q), _ptr(keep["ori"]), case.ori_stride, _ptr(keep["ot"]), keep["ot"].shape[1],
              _ptr(keep["cmp"]), case.cmp_stride, _ptr(keep["ct"]),
              keep["ct"].shape[1] if keep["ct"] is not None else 0, _ptr(keep["ix"]), topk,
              _ptr(keep["cu"]), _ptr(keep["sl"]), len(keep["sl"]), _ptr(keep["sink"]),
              _ptr(keep["os"]), _ptr(keep["cs"]), T, H, case.block, case.ratio, case.window,
              case.softmax_scale, _ptr(keep["oi"]), ori_topk, case.ori_pages)
    plan = _Plan(tile, splits, int(joint_dense), int(joint_sparse), joint_tile_limit, int(dense_c4),
                 int(query_group))
    out = np.zeros((T, H, DIM), dtype=np.uint16)
    lse = np.zeros((T, H), dtype=np.float32) if return_lse else None
    dbg = None
    dbg_arrays = None
    if debug:
        if cmp_capacity is None:
            cmp_capacity = max(topk, int(case.seq_lens.max()) // max(case.ratio, 1) + 1 if case.ratio != 1 else 0)
        if tile_capacity is None:
            tile_capacity = (128 + tile - 1) // tile + (cmp_capacity + tile - 1) // tile
        positions = 128 + cmp_capacity
        dbg_arrays = dict(
            qcodes=np.zeros((T, 2, 16, DIM), np.int8), alpha=np.zeros((T, 2, 8), np.float32),
            scores=np.zeros((T, positions, 16), np.int32), probs=np.zeros((T, positions, 16), np.int8),
            values=np.zeros((T, tile_capacity, 16, DIM), np.int32),
            weight_args=np.full((T, positions, 8), np.nan, np.float32))
        dbg = _Debug(*(_ptr(dbg_arrays[k]) for k in ("qcodes", "alpha", "scores", "probs", "values")),
                     cmp_capacity, tile_capacity, _ptr(dbg_arrays["weight_args"]))
    threads = threads or int(os.environ.get("SKO_THREADS", os.cpu_count() or 1))
    rc = lib().sko_tiled_attention(ctypes.byref(c), ctypes.byref(plan), _ptr(out), _ptr(lse),
                                   ctypes.byref(dbg) if dbg is not None else None, threads)
    if rc != 0:
        raise ValueError(f"oracle rejected the case (code {rc})")
    return out, lse, dbg_arrays


def joint_row(q_bf16, rows, scales, sink, softmax_scale, bias=None):
    """reference.py:175-207 on gathered INT8 rows (list of [n_k, 512])."""
    q = np.ascontiguousarray(q_bf16, dtype=np.uint16)
    H = q.shape[0]
    rows = [np.ascontiguousarray(r, dtype=np.int8).reshape(-1, DIM) for r in rows]
    scales = [np.ascontiguousarray(s, dtype=np.float32) for s in scales]
    row_ptrs = (ctypes.c_void_p * len(rows))(*[r.ctypes.data for r in rows])
    counts = (ctypes.c_int32 * len(rows))(*[len(r) for r in rows])
    scale_ptrs = (ctypes.c_void_p * len(rows))(*[s.ctypes.data for s in scales])
    sink = np.ascontiguousarray(sink, dtype=np.float32)
    bias = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    out = np.zeros((H, DIM), np.uint16)
    lse = np.zeros(H, np.float32)
    lib().sko_joint_row(_ptr(q), ctypes.c_int(H), row_ptrs, counts, scale_ptrs, ctypes.c_int(len(rows)),
                        _ptr(bias), _ptr(sink), ctypes.c_float(softmax_scale), _ptr(out), _ptr(lse))
    return out, lse


def gather_rows(pool, stride, table, batch, indices, block=32):
    """reference.py:82-85 on a flat byte pool."""
    indices = np.asarray(indices, dtype=np.int64)
    pages = table[batch, indices // block].astype(np.int64)
    offsets = pages * stride + (indices % block) * DIM
    return pool[offsets[:, None] + np.arange(DIM)[None, :]]


def gather_slots(pool, stride, slots, block=32):
    """reference.py:88-90 on a flat byte pool: physical slots, no table."""
    slots = np.asarray(slots, dtype=np.int64)
    offsets = (slots // block) * stride + (slots % block) * DIM
    return pool[offsets[:, None] + np.arange(DIM)[None, :]]


def selected_rows(case):
    """reference.py:93-126: yields (token, original rows, compressed rows or None)."""
    for b in range(len(case.seq_lens)):
        begin, end = int(case.cu_q[b]), int(case.cu_q[b + 1])
        length = int(case.seq_lens[b])
        if end - begin > length:
            raise ValueError("Query length cannot exceed sequence length")
        for t in range(begin, end):
            position = length - (end - begin) + (t - begin)
            if case.ori_indices is None:
                ori_idx = np.arange(max(0, position - case.window + 1), position + 1)
                ori = gather_rows(case.ori, case.ori_stride, case.ori_table, b, ori_idx, case.block)
            else:
                # reference.py:112-115: valid physical slots, in order, no table.
                slots = case.ori_indices[t, 0].astype(np.int64)
                slots = slots[(slots >= 0) & (slots < case.ori_pages * case.block)]
                ori = gather_slots(case.ori, case.ori_stride, slots, case.block)
            cmp = None
            if case.ratio != 1:
                count = (position + 1) // case.ratio
                if case.ratio == 4 and case.cmp_indices is not None:
                    idx = case.cmp_indices[t, 0].astype(np.int64)
                    idx = idx[(idx >= 0) & (idx < count)]
                else:
                    idx = np.arange(count)
                cmp = gather_rows(case.cmp, case.cmp_stride, case.cmp_table, b, idx, case.block)
            yield t, ori, cmp


def fp64_attention(case, ori_values=None, cmp_values=None):
    """reference.py:129-139 sharedkv_reference in FP64.

    ori_values / cmp_values map an int8 row block to real values (dequantize);
    by default rows are taken as the INT8 codes times their scale."""
    ori_values = ori_values or (lambda r: r.astype(np.float64) * case.ori_scale.astype(np.float64))
    cmp_values = cmp_values or (lambda r: r.astype(np.float64) * case.cmp_scale.astype(np.float64))
    T, H, _ = case.q.shape
    out = np.zeros((T, H, DIM), np.float64)
    lse = np.zeros((T, H), np.float64)
    q = bf16_to_f32(case.q).astype(np.float64)
    for t, ori, cmp in selected_rows(case):
        kv = ori_values(ori)
        if cmp is not None:
            kv = np.concatenate([kv, cmp_values(cmp)], 0)
        out[t], lse[t] = fp64_rows(q[t], kv, case.sink, case.softmax_scale)
    return out, lse


def fp64_rows(q, kv, sink, softmax_scale):
    """reference.py:133-136 for one query token: softmax over the rows `kv`
    plus one sink logit per head that enters the denominator only.
    q [H, 512], kv [n, 512] (FP64 values); returns (out [H, 512], lse [H])."""
    q = np.asarray(q, np.float64)
    kv = np.asarray(kv, np.float64)
    logits = q @ kv.T * softmax_scale
    ext = np.concatenate([logits, np.asarray(sink, np.float64)[:, None]], -1)
    m = ext.max(-1, keepdims=True)
    l = (m + np.log(np.exp(ext - m).sum(-1, keepdims=True)))[:, 0]
    return np.exp(logits - l[:, None]) @ kv, l
