"""Seeded synthetic shared-KV cases on the host (numpy).

Shapes follow the workloads of the reference's tests (tests/support/
serving_shapes.py, reference.py:326-354 make_case): BF16 Q ~ N(0,1); KV rows
~ N(0,1) with 16 outlier channels scaled x8, rounded to BF16, encoded with a
frozen per-channel scale max(1.1 * absmax / 127, 1e-8); block32 pages in a
shuffled pool; sink = linspace(-2, 2, H).

Only the pages a query can read are materialised; other logical pages map to
physical page 0, which the path never reads for them.
"""
import math

import numpy as np

DIM = 512
BLOCK = 32


def bf16_bits(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_value(bits):
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def kv_rows(rng, rows, outlier_channels):
    x = rng.standard_normal((rows, DIM), dtype=np.float32)
    x[:, outlier_channels] *= 8
    return bf16_bits(x)


def frozen_scale(values, margin=1.1):
    amax = np.abs(values).max(0).astype(np.float32)
    return np.maximum(np.float32(margin) * amax / np.float32(127), np.float32(1e-8)).astype(np.float32)


def encode(values, scale):
    inverse = (1.0 / scale.astype(np.float64)).astype(np.float32)
    return np.clip(np.rint(values * inverse), -127, 127).astype(np.int8)


class Kind:
    """One paged INT8 cache kind (original or compressed).  `rows`, when
    given, maps (batch, logical row) to that row's BF16 bits; the other rows
    of touched pages are zero.  `scale` then is the frozen scale to encode with."""

    def __init__(self, name, needed, rng, page_stride, table_width, pool_factor=1.25, rows=None, scale=None):
        self.name = name
        batch = len(needed)
        touched = [sorted(set(int(i) // BLOCK for i in rows)) for rows in needed]
        total = sum(len(t) for t in touched)
        pages = max(1, int(math.ceil(total * pool_factor)))
        physical = rng.permutation(pages)
        self.table = np.zeros((batch, max(1, table_width)), dtype=np.int32)
        k = 0
        for b, logical in enumerate(touched):
            for lp in logical:
                self.table[b, lp] = physical[k]
                k += 1
        self.pages = pages
        self.page_stride = page_stride
        if rows is None:
            outliers = rng.choice(DIM, 16, replace=False)
            self.values_bits = kv_rows(rng, pages * BLOCK, outliers)          # BF16 source rows
        else:
            self.values_bits = np.zeros((pages * BLOCK, DIM), dtype=np.uint16)
            for (b, logical), bits in rows.items():
                physical_page = self.table[b, logical // BLOCK]
                self.values_bits[physical_page * BLOCK + logical % BLOCK] = bits
        values = bf16_value(self.values_bits)
        self.scale = frozen_scale(values) if scale is None else np.asarray(scale, dtype=np.float32)
        codes = encode(values, self.scale)
        self.pool = np.zeros(pages * page_stride, dtype=np.int8)
        view = self.pool.reshape(pages, page_stride)[:, :BLOCK * DIM]
        view[:] = codes.reshape(pages, BLOCK * DIM)


# Sparse-edge selections of the reference's tests/npu/test_sparse_edges.py:52-75.
EDGE_MODES = ("empty", "single", "one_key_duplicates", "extended_duplicates", "permutation")


def edge_indices(mode, t, count, topk, rng):
    """One query's C4 index row (length topk, -1 = hole) for an edge mode:
    'empty'                no valid entry;
    'single'               one key, t mod count, in the last place;
    'one_key_duplicates'   that key in the first and the last place;
    'extended_duplicates'  every other place holds (place / 2) mod count, i.e.
                           more selected entries than the causal extent;
    'permutation'          a random order of all min(topk, count) keys."""
    row = np.full(topk, -1, np.int64)
    if count <= 0 or mode == "empty":
        return row
    if mode in ("single", "one_key_duplicates"):
        row[topk - 1] = t % count
        if mode == "one_key_duplicates":
            row[0] = t % count
    elif mode == "extended_duplicates":
        row[::2] = np.arange((topk + 1) // 2) % count
    else:
        extent = min(topk, count)
        row[:extent] = rng.permutation(extent)
    return row


def make_case(seed, ratio, queries, lengths, topk=1024, heads=8, window=128,
              page_stride=BLOCK * DIM, index_mode="uniform", softmax_scale=1 / math.sqrt(DIM),
              ori_slots=None, ori_topk=256):
    """Returns (oracle-style dict, metadata).  index_mode for C4:
    'uniform'  top-k drawn without replacement from the visible range, sorted;
    'holes'    as uniform with every 7th entry -1 and every 11th out of range;
    'dups'     indices i // 2 (duplicates);
    'mixed'    random with replacement plus -1 padding.
    EDGE_MODES (edge_indices): the reference's sparse-edge selections.
    ori_slots (explicit physical original slots, int32 [T, 1, ori_topk]):
    'window'   the physical slots of the query's own window rows, then -1
               (the same list, in the same places, as the window path);
    'draft'    the slots of logical rows max(0, pos - 127) .. len - 1 of the
               request, then -1 (tests/support/serving_shapes.py:96-105 of
               the reference: a draft token sees the whole draft);
    'shuffled' as 'draft', in a random order, with every 5th entry -1, every
               13th past the pool and a few repeated slots;
    'pool'     ori_topk slots drawn anywhere in the pool (physical slots need
               not belong to the request), 10 % of them -1 or past the pool."""
    rng = np.random.default_rng(seed)
    batch = len(queries)
    cu = np.zeros(batch + 1, dtype=np.int32)
    cu[1:] = np.cumsum(queries)
    tokens = int(cu[-1])
    seq = np.asarray(lengths, dtype=np.int32)
    q = bf16_bits(rng.standard_normal((tokens, heads, DIM), dtype=np.float32))
    sink = np.linspace(-2, 2, heads, dtype=np.float32)

    positions = []
    for b in range(batch):
        for t in range(cu[b], cu[b + 1]):
            positions.append((b, t, int(seq[b]) - int(cu[b + 1]) + t))

    ori_needed = [[] for _ in range(batch)]
    for b, t, pos in positions:
        ori_needed[b].extend(range(max(0, pos + 1 - window), pos + 1))
    ori = Kind("ori", ori_needed, rng, page_stride, (int(seq.max()) + BLOCK - 1) // BLOCK)

    out = dict(q=q, ori=ori, cu_q=cu, seq_lens=seq, sink=sink, ratio=ratio, window=window,
               softmax_scale=softmax_scale, cmp=None, cmp_indices=None, topk=0, ori_indices=None)
    if ratio != 1:
        indices = None
        cmp_needed = [[] for _ in range(batch)]
        if ratio == 4:
            indices = np.full((tokens, 1, topk), -1, dtype=np.int32)
            for b, t, pos in positions:
                count = (pos + 1) // 4
                if index_mode == "uniform":
                    ids = np.sort(rng.permutation(count)[:topk]) if count else np.zeros(0, np.int64)
                elif index_mode == "holes":
                    ids = np.sort(rng.permutation(count)[:topk]) if count else np.zeros(0, np.int64)
                    ids = ids.astype(np.int64)
                    ids[::7] = -1
                    ids[3::11] = count + 5
                elif index_mode == "dups":
                    ids = np.arange(min(topk, count)) // 2
                elif index_mode == "mixed":
                    n = min(topk, max(1, count))
                    ids = rng.integers(0, max(1, count), n) if count else np.full(n, -1)
                    ids[rng.random(n) < 0.2] = -1
                elif index_mode in EDGE_MODES:
                    ids = edge_indices(index_mode, t, count, topk, rng)
                else:
                    raise ValueError(index_mode)
                indices[t, 0, :len(ids)] = ids
                cmp_needed[b].extend(int(i) for i in ids if 0 <= i < count)
        else:
            for b, t, pos in positions:
                cmp_needed[b].extend(range((pos + 1) // ratio))
        width = (int(seq.max()) // ratio + BLOCK - 1) // BLOCK
        cmp = Kind("cmp", cmp_needed, rng, page_stride, width)
        out.update(cmp=cmp, cmp_indices=indices, topk=topk if ratio == 4 else 0)
    if ori_slots is not None:
        slots = np.full((tokens, 1, ori_topk), -1, dtype=np.int32)
        capacity = ori.pages * BLOCK
        for b, t, pos in positions:
            if ori_slots == "pool":
                row = rng.integers(0, capacity, ori_topk)
                bad = rng.random(ori_topk) < 0.1
                row[bad] = np.where(rng.random(int(bad.sum())) < 0.5, -1, capacity + 3)
                slots[t, 0] = row
                continue
            last = pos if ori_slots == "window" else int(seq[b]) - 1
            logical = np.arange(max(0, pos + 1 - window), last + 1)
            row = ori.table[b, logical // BLOCK].astype(np.int64) * BLOCK + logical % BLOCK
            if ori_slots == "shuffled":
                row = rng.permutation(row)
                if len(row) > 3:
                    row[1] = row[3]                 # a repeated slot
                row[::5] = -1
                row[2::13] = capacity + 7           # past the pool
            elif ori_slots not in ("window", "draft"):
                raise ValueError(ori_slots)
            if len(row) > ori_topk:
                raise ValueError("ori_topk too small for the request")
            slots[t, 0, :len(row)] = row
        out["ori_indices"] = slots
    return out


def oracle_case(case):
    """Adapter to oracle.Case."""
    import oracle.oracle as ora   # the checker; tests only
    cmp = case["cmp"]
    return ora.Case(q=case["q"], ori=case["ori"].pool, ori_stride=case["ori"].page_stride,
                    ori_table=case["ori"].table, cu_q=case["cu_q"], seq_lens=case["seq_lens"],
                    sink=case["sink"], ori_scale=case["ori"].scale,
                    cmp=cmp.pool if cmp else None, cmp_stride=cmp.page_stride if cmp else 0,
                    cmp_table=cmp.table if cmp else None, cmp_scale=cmp.scale if cmp else None,
                    cmp_indices=case["cmp_indices"], ratio=case["ratio"], window=case["window"],
                    softmax_scale=case["softmax_scale"], ori_indices=case.get("ori_indices"),
                    ori_pages=case["ori"].pages)


def fixture_case(z, i, seed=0, page_stride=BLOCK * DIM):
    """One query token built from real-activation fixture layer `i`
    (tests/golden/vectors/activations.npz, converted from the reference's
    tests/fixtures/activations): the token sits at position n - 1 of a
    sequence of n = 508 tokens, so its SWA128 window is the fixture's 128
    original rows and its compressed list is the fixture's compressed rows
    (all (n // ratio) visible entries; the C4 top-k holds every one of them).
    The MTP samples (ratio 1, 133 original rows) list their rows as explicit
    physical original slots (the draft path's ori_indices), in the sample's
    order, padded with -1 to 256.  Rows are encoded with the layer's frozen
    serving scales."""
    ratio = int(z[f"{i}_ratio"])
    ori_bits, cmp_bits = z[f"{i}_ori"], z[f"{i}_cmp"]
    window = ori_bits.shape[0]
    if ratio == 1:
        rng = np.random.default_rng(seed)
        n = window
        ori = Kind("ori", [range(n)], rng, page_stride, (n + BLOCK - 1) // BLOCK,
                   rows={(0, r): ori_bits[r] for r in range(n)}, scale=z[f"{i}_ori_scale"])
        logical = np.arange(n)
        slots = np.full((1, 1, 256), -1, dtype=np.int32)
        slots[0, 0, :n] = ori.table[0, logical // BLOCK] * BLOCK + logical % BLOCK
        return dict(q=z[f"{i}_q"].reshape(1, 8, DIM), ori=ori, cu_q=np.array([0, 1], np.int32),
                    seq_lens=np.array([n], np.int32), sink=z[f"{i}_sink"].astype(np.float32), ratio=1,
                    window=128, softmax_scale=float(z[f"{i}_softmax_scale"]), cmp=None, cmp_indices=None,
                    topk=0, ori_indices=slots)
    if window != 128:
        raise ValueError("only the SWA128 + compressed samples map onto this path")
    length = 508
    count = length // ratio
    assert cmp_bits.shape[0] == count
    rng = np.random.default_rng(seed)
    pos = length - 1
    first = pos + 1 - window
    ori_rows = {(0, first + r): ori_bits[r] for r in range(window)}
    ori = Kind("ori", [range(first, pos + 1)], rng, page_stride, (length + BLOCK - 1) // BLOCK,
               rows=ori_rows, scale=z[f"{i}_ori_scale"])
    cmp_rows = {(0, r): cmp_bits[r] for r in range(count)}
    cmp = Kind("cmp", [range(count)], rng, page_stride, (count + BLOCK - 1) // BLOCK,
               rows=cmp_rows, scale=z[f"{i}_cmp_scale"])
    indices = None
    topk = 0
    if ratio == 4:
        topk = 1024
        indices = np.full((1, 1, topk), -1, dtype=np.int32)
        indices[0, 0, :count] = np.arange(count)
    q = z[f"{i}_q"].reshape(1, 8, DIM)
    return dict(q=q, ori=ori, cu_q=np.array([0, 1], np.int32), seq_lens=np.array([length], np.int32),
                sink=z[f"{i}_sink"].astype(np.float32), ratio=ratio, window=128,
                softmax_scale=float(z[f"{i}_softmax_scale"]), cmp=cmp, cmp_indices=indices, topk=topk)
