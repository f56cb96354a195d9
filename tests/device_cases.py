"""Host/device plumbing shared by the GPU parity tests, smoke() and bench.py.

Builds SharedKVCase objects on the GPU from the seeded numpy cases of
tests/workloads.py, runs the HIP path through the package (C ABI underneath)
and runs the CPU checker (oracle/) with the same tiling plan.
"""
import ctypes

import numpy as np

from tests import workloads

DIM = 512


def torch_bf16(bits, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(device).view(torch.bfloat16)


def device_pool(kind, device):
    """The kind's flat byte pool on the device, viewed as [pages, 32, 1, 512]
    with its page stride (bytes == elements for INT8)."""
    import torch
    payload = workloads.BLOCK * DIM
    flat = torch.zeros(kind.pages * kind.page_stride, dtype=torch.int8, device=device)
    host = torch.from_numpy(kind.pool.reshape(kind.pages, kind.page_stride)[:, :payload].copy())
    flat.view(kind.pages, kind.page_stride)[:, :payload].copy_(host)
    return flat.as_strided((kind.pages, workloads.BLOCK, 1, DIM), (kind.page_stride, DIM, DIM, 1)), flat


def to_device(case, device="cuda"):
    """Returns (SharedKVCase on `device`, ori_scale, cmp_scale, keep-alive list)."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import SharedKVCase
    ori, ori_flat = device_pool(case["ori"], device)
    keep = [ori_flat]
    cmp = cmp_table = cmp_scale = indices = None
    if case["cmp"] is not None:
        cmp, cmp_flat = device_pool(case["cmp"], device)
        keep.append(cmp_flat)
        cmp_table = torch.from_numpy(case["cmp"].table).to(device)
        cmp_scale = torch.from_numpy(case["cmp"].scale).to(device)
    if case["cmp_indices"] is not None:
        indices = torch.from_numpy(case["cmp_indices"]).to(device)
    ori_indices = case.get("ori_indices")
    if ori_indices is not None:
        ori_indices = torch.from_numpy(ori_indices).to(device)
    dev = SharedKVCase(
        q=torch_bf16(case["q"], device), ori=ori, ori_block_table=torch.from_numpy(case["ori"].table).to(device),
        cu_q=torch.from_numpy(case["cu_q"]).to(device), seq_lens=torch.from_numpy(case["seq_lens"]).to(device),
        sink=torch.from_numpy(case["sink"]).to(device), cmp=cmp, cmp_block_table=cmp_table,
        cmp_indices=indices, ratio=case["ratio"], window=case["window"], softmax_scale=case["softmax_scale"],
        ori_indices=ori_indices)
    return dev, torch.from_numpy(case["ori"].scale).to(device), cmp_scale, keep


def bits_of(tensor):
    """BF16 tensor -> uint16 numpy bits (host copy)."""
    import torch
    return tensor.detach().cpu().view(torch.int16).numpy().view(np.uint16)


def run_hip(case, splits=None, return_lse=True, device="cuda", query_group=None, tile_size=None, max_seq_len=None):
    """One PreparedAttention launch; returns (out bits, lse, prepared)."""
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    dev, ori_scale, cmp_scale, keep = to_device(case, device)
    op = PreparedAttention(dev, ori_scale, cmp_scale, splits=splits, return_lse=return_lse, query_group=query_group,
                           tile_size=tile_size, max_seq_len=max_seq_len)
    op._keep = keep
    op.run()
    torch.cuda.synchronize()
    lse = op.lse.cpu().numpy() if op.lse is not None else None
    return bits_of(op.out), lse, op


def run_hip_debug(case, splits=None, cmp_capacity=None, device="cuda"):
    """The debug entry (integer dumps) with the same plan as run_hip."""
    import torch
    from npu_sparse_attn_sharedkv_int8.runtime import SharedKVDebug, library
    dev, ori_scale, cmp_scale, keep = to_device(case, device)
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    op = PreparedAttention(dev, ori_scale, cmp_scale, splits=splits, return_lse=True)
    T = case["q"].shape[0]
    if cmp_capacity is None:
        cmp_capacity = default_cmp_capacity(case)
    tiles = (128 + 127) // 128 + (cmp_capacity + 127) // 128
    positions = 128 + cmp_capacity
    buffers = dict(
        qcodes=torch.zeros((T, 2, 16, DIM), dtype=torch.int8, device=device),
        alpha=torch.zeros((T, 2, 8), dtype=torch.float32, device=device),
        scores=torch.zeros((T, positions, 16), dtype=torch.int32, device=device),
        probs=torch.zeros((T, positions, 16), dtype=torch.int8, device=device),
        values=torch.zeros((T, tiles, 16, DIM), dtype=torch.int32, device=device))
    dbg = SharedKVDebug(*(buffers[k].data_ptr() for k in ("qcodes", "alpha", "scores", "probs", "values")),
                        cmp_capacity, tiles)
    stream = torch.cuda.current_stream().cuda_stream
    rc = library().sharedkv_c8_attention_debug(ctypes.c_void_p(stream), ctypes.byref(op.args), ctypes.byref(dbg))
    if rc:
        raise RuntimeError(f"debug launch failed: {rc}")
    torch.cuda.synchronize()
    dumps = {k: v.cpu().numpy() for k, v in buffers.items()}
    return bits_of(op.out), op.lse.cpu().numpy(), dumps, op, (cmp_capacity, tiles)


def default_cmp_capacity(case):
    if case["ratio"] == 4:
        return case["cmp_indices"].shape[-1]
    if case["ratio"] == 128:
        return int(case["seq_lens"].max()) // 128 + 1
    return 0


def effective_splits(case, splits, merge_mode=0):
    """KV partitions the kernel runs for a launch of `case` (host numpy
    metadata) planned at `splits`, with the library in `merge_mode`
    (c8_attention.device_splits: the device's re-plan of padded launches and
    joint-row launches)."""
    from npu_sparse_attn_sharedkv_int8 import c8_attention
    slots = case.get("ori_indices")
    return c8_attention.device_splits(
        splits, case["q"].shape[0], case["q"].shape[1], case["ratio"],
        case["cmp_indices"].shape[-1] if case["ratio"] == 4 else 0, case["cu_q"], case["seq_lens"],
        slots.shape[-1] if slots is not None else 0, fused=merge_mode == 0, cmp_rows=cmp_rows(case))


def cmp_rows(case):
    """Rows per sequence the case's compressed block table names (width x 32),
    or None without a compressed cache."""
    return case["cmp"].table.shape[1] * 32 if case.get("cmp") is not None else None


def joint_flags(case, splits, merge_mode=0):
    """(joint_dense, joint_sparse) of the checker for a launch of `case`
    planned at `splits`: C128 rows are joint per row at one partition
    (c8_attention.joint_plan), C4 rows only in a joint-plan launch
    (c8_attention.joint_launch: short live rows and a compressed block
    table of at most 128 rows per sequence), judged on the whole launch's
    metadata."""
    from npu_sparse_attn_sharedkv_int8 import c8_attention
    slots = case.get("ori_indices")
    heads, ratio = case["q"].shape[1], case["ratio"]
    dense = ratio == 128 and c8_attention.joint_plan(ratio, heads, slots is not None)
    sparse = ratio == 4 and c8_attention.joint_launch(
        splits, case["q"].shape[0], heads, ratio, case["cu_q"], case["seq_lens"],
        slots.shape[-1] if slots is not None else 0, fused=merge_mode == 0, cmp_rows=cmp_rows(case))
    return bool(dense), bool(sparse)


def run_oracle(case, splits, debug=False, cmp_capacity=None, tile_capacity=None, threads=None, joint=None,
               query_group=1, tile=128):
    """The CPU checker with this build's plan: `tile`-key tiles (128; the
    grouped plans also 256), `splits` partitions (the ones the kernel runs),
    and joint rows where the kernel takes them: `joint` = joint_flags of the
    launch (default: those of `case` as its own launch at `splits`); the
    debug entry runs the tiled plan."""
    import oracle.oracle as ora
    if joint is None:   # a joint-plan launch runs one partition
        dense, sparse = joint_flags(case, splits)
        sparse = sparse and splits == 1
    else:
        dense, sparse = joint
    if query_group != 1:   # the paired plan has no joint rows
        dense = sparse = False
    return ora.tiled_attention(workloads.oracle_case(case), tile=tile, splits=splits, return_lse=True,
                               joint_dense=dense and not debug, joint_sparse=sparse and not debug, debug=debug,
                               cmp_capacity=cmp_capacity, tile_capacity=tile_capacity, threads=threads,
                               query_group=query_group)


def query_subcase(case, rows):
    """A case holding only query rows `rows` of `case`, each as its own
    one-token request with the same position, tables and index row, so every
    selected row computes exactly what it computes in the full case."""
    cu = case["cu_q"]
    owner = np.searchsorted(cu, np.arange(cu[-1]), side="right") - 1
    rows = np.asarray(rows)
    batch = owner[rows]
    positions = case["seq_lens"][batch] - cu[batch + 1] + rows
    sub = dict(case)
    sub["q"] = case["q"][rows]
    sub["cu_q"] = np.arange(len(rows) + 1, dtype=np.int32)
    sub["seq_lens"] = (positions + 1).astype(np.int32)
    sub["ori"] = _kind_rows(case["ori"], batch)
    if case["cmp"] is not None:
        sub["cmp"] = _kind_rows(case["cmp"], batch)
    if case["cmp_indices"] is not None:
        sub["cmp_indices"] = np.ascontiguousarray(case["cmp_indices"][rows])
    if case.get("ori_indices") is not None:
        sub["ori_indices"] = np.ascontiguousarray(case["ori_indices"][rows])   # physical: no table
    return sub


class _KindView:
    pass


def _kind_rows(kind, batch):
    view = _KindView()
    view.__dict__.update(kind.__dict__)
    view.table = np.ascontiguousarray(kind.table[batch])
    return view


# ------------------------------------------------- device-side large cases

class DeviceKind:
    """One paged INT8 cache kind generated on the GPU, for `layers` layers.

    The recipe of tests/workloads.py (KV ~ N(0,1) FP32, 16 outlier channels
    x8, rounded to BF16, frozen scale max(1.1 * absmax / 127, 1e-8), codes by
    the sharedkv-c8-v1 encoding) evaluated with torch on the device, so
    multi-GiB pools take milliseconds.  The block table maps the touched
    logical pages of each sequence to a random permutation of the pool
    (`pool_factor` slack).  Layers share the page numbering, as in a serving
    pool whose page stride holds every layer's 16 KiB page (layer l's page p
    starts at p * page_stride + l * 16384); each layer has its own data and
    scale.
    """

    PAGE_BYTES = workloads.BLOCK * DIM

    def __init__(self, touched, seed, page_stride, table_width, device, pool_factor=1.25, layers=1,
                 chunk_rows=1 << 18):
        import torch
        if page_stride < layers * self.PAGE_BYTES or page_stride % 16:
            raise ValueError("page stride cannot hold the layers' pages")
        rng = np.random.default_rng(seed)
        batch = len(touched)
        total = sum(len(t) for t in touched)
        self.pages = max(1, int(np.ceil(total * pool_factor)))
        self.page_stride, self.layers = page_stride, layers
        physical = rng.permutation(self.pages).astype(np.int32)
        self.table = np.zeros((batch, max(1, table_width)), dtype=np.int32)
        k = 0
        for b, logical in enumerate(touched):
            self.table[b, logical] = physical[k:k + len(logical)]
            k += len(logical)
        self.table_dev = torch.from_numpy(self.table).to(device)
        self.flat = torch.zeros(self.pages * page_stride, dtype=torch.int8, device=device)
        blocks = self.flat.view(self.pages, page_stride)
        rows = self.pages * workloads.BLOCK
        chunks = (rows + chunk_rows - 1) // chunk_rows
        gen = torch.Generator(device=device)
        self.scales, self.scales_dev, self.views = [], [], []
        for layer in range(layers):
            outliers = torch.from_numpy(rng.choice(DIM, 16, replace=False)).to(device)

            def chunk(i):
                gen.manual_seed((seed * 131 + layer) * 7919 + i)
                n = min(chunk_rows, rows - i * chunk_rows)
                x = torch.randn((n, DIM), generator=gen, device=device)
                x[:, outliers] *= 8
                return x.to(torch.bfloat16).float()

            amax = torch.zeros(DIM, device=device)
            for i in range(chunks):
                amax = torch.maximum(amax, chunk(i).abs().amax(0))
            scale = torch.clamp(amax * np.float32(1.1) / 127, min=1e-8)
            host_scale = scale.cpu().numpy().astype(np.float32)
            scale_dev = torch.from_numpy(host_scale).to(device)
            inverse = (1.0 / scale_dev.double()).float()
            base = layer * self.PAGE_BYTES
            for i in range(chunks):
                codes = torch.clamp(torch.round(chunk(i) * inverse), -127, 127).to(torch.int8)
                p0 = i * chunk_rows // workloads.BLOCK          # chunk_rows is a multiple of 32
                p1 = p0 + len(codes) // workloads.BLOCK
                blocks[p0:p1, base:base + self.PAGE_BYTES] = codes.view(p1 - p0, self.PAGE_BYTES)
            self.scales.append(host_scale)
            self.scales_dev.append(scale_dev)
            self.views.append(self.flat[base:].as_strided((self.pages, workloads.BLOCK, 1, DIM),
                                                          (page_stride, DIM, DIM, 1)))
        self._host = {}
        # Single-layer conveniences.
        self.view, self.scale, self.scale_dev = self.views[0], self.scales[0], self.scales_dev[0]

    def host_kind(self, layer=0):
        """Compact host copy (page stride 16 KiB) for the CPU checker."""
        if layer not in self._host:
            base = layer * self.PAGE_BYTES
            payload = self.flat.view(self.pages, self.page_stride)[:, base:base + self.PAGE_BYTES]
            self._host[layer] = payload.cpu().numpy().reshape(-1)
        view = _KindView()
        view.pages, view.table, view.scale = self.pages, self.table, self.scales[layer]
        view.pool, view.page_stride = self._host[layer], self.PAGE_BYTES
        return view


def c4_indices(rng, counts, topk):
    """Top-k logical compressed rows per query: drawn without replacement
    from the query's visible range [0, count), sorted, -1 padded (all rows
    when count <= topk)."""
    out = np.full((len(counts), 1, topk), -1, dtype=np.int32)
    for t, count in enumerate(counts):
        count = int(count)
        if count <= 0:
            continue
        ids = np.sort(rng.choice(count, topk, replace=False)) if count > topk else np.arange(count)
        out[t, 0, :len(ids)] = ids
    return out


class DeviceCase:
    """A full-size case: metadata on the host, caches generated on the GPU.

    cases[l] (SharedKVCase), ori_scales[l] and cmp_scales[l] feed
    PreparedAttention for layer l; host(l) returns the tests/workloads.py
    dict layout (compact host pools) for the checker.  Layers share
    sequences, positions and block tables and differ in Q, top-k indices,
    cache data and scales, like consecutive layers of one decode step.
    """

    def __init__(self, seed, ratio, queries, lengths, *, topk=1024, page_stride=workloads.BLOCK * DIM,
                 device="cuda", pool_factor=1.25, heads=8, window=128, layers=1):
        import torch
        from npu_sparse_attn_sharedkv_int8 import SharedKVCase
        rng = np.random.default_rng(seed)
        block = workloads.BLOCK
        batch = len(queries)
        cu = np.zeros(batch + 1, dtype=np.int32)
        cu[1:] = np.cumsum(queries)
        tokens = int(cu[-1])
        seq = np.asarray(lengths, dtype=np.int32)
        owner = np.repeat(np.arange(batch), queries)
        positions = seq[owner] - cu[owner + 1] + np.arange(tokens)
        counts = (positions + 1) // max(ratio, 1)
        self.q_bits = [workloads.bf16_bits(rng.standard_normal((tokens, heads, DIM), dtype=np.float32))
                       for _ in range(layers)]
        self.heads = heads
        self.sink = np.linspace(-2, 2, heads, dtype=np.float32)
        self.indices = [c4_indices(rng, counts, topk) for _ in range(layers)] if ratio == 4 else [None] * layers
        ori_touched, cmp_touched = [], []
        for b in range(batch):
            sel = owner == b
            own = positions[sel]
            if not len(own):
                ori_touched.append(np.zeros(0, np.int64))
                cmp_touched.append(np.zeros(0, np.int64))
                continue
            lo, hi = max(0, int(own.min()) - window + 1), int(own.max())
            ori_touched.append(np.arange(lo // block, hi // block + 1))
            if ratio == 4 and layers == 1:
                ids = self.indices[0][sel, 0].reshape(-1)
                cmp_touched.append(np.unique(ids[ids >= 0] // block))
            else:
                cmp_touched.append(np.arange((int(counts[sel].max()) + block - 1) // block))
        width = (int(seq.max()) + block - 1) // block
        self.ori = DeviceKind(ori_touched, seed * 2 + 1, page_stride, width, device, pool_factor, layers)
        self.cmp = None
        if ratio != 1:
            cwidth = max(1, (int(seq.max()) // ratio + block - 1) // block)
            self.cmp = DeviceKind(cmp_touched, seed * 2 + 2, page_stride, cwidth, device, pool_factor, layers)
        self.meta = dict(cu_q=cu, seq_lens=seq, ratio=ratio, window=window, softmax_scale=1 / np.sqrt(DIM),
                         topk=topk if ratio == 4 else 0, positions=positions, owner=owner)
        cu_dev, seq_dev = torch.from_numpy(cu).to(device), torch.from_numpy(seq).to(device)
        sink_dev = torch.from_numpy(self.sink).to(device)
        self.cases, self.ori_scales, self.cmp_scales = [], [], []
        for layer in range(layers):
            ix = self.indices[layer]
            self.cases.append(SharedKVCase(
                q=torch_bf16(self.q_bits[layer], device), ori=self.ori.views[layer],
                ori_block_table=self.ori.table_dev, cu_q=cu_dev, seq_lens=seq_dev, sink=sink_dev,
                cmp=self.cmp.views[layer] if self.cmp else None,
                cmp_block_table=self.cmp.table_dev if self.cmp else None,
                cmp_indices=torch.from_numpy(ix).to(device) if ix is not None else None,
                ratio=ratio, window=window, softmax_scale=float(1 / np.sqrt(DIM))))
            self.ori_scales.append(self.ori.scales_dev[layer])
            self.cmp_scales.append(self.cmp.scales_dev[layer] if self.cmp else None)
        self.dev, self.ori_scale, self.cmp_scale = self.cases[0], self.ori_scales[0], self.cmp_scales[0]

    def host(self, layer=0):
        m = self.meta
        return dict(q=self.q_bits[layer], ori=self.ori.host_kind(layer), cu_q=m["cu_q"], seq_lens=m["seq_lens"],
                    sink=self.sink, ratio=m["ratio"], window=m["window"], softmax_scale=m["softmax_scale"],
                    cmp=self.cmp.host_kind(layer) if self.cmp else None, cmp_indices=self.indices[layer],
                    topk=m["topk"])

    def selected_keys(self, layer=0):
        """Keys attended over all query tokens: the SWA window rows plus the
        compressed list (C4: valid top-k entries; C128: every visible entry)."""
        m = self.meta
        pos = m["positions"]
        keys = int(np.minimum(pos + 1, m["window"]).sum())
        if m["ratio"] == 4:
            ids = self.indices[layer][:, 0]
            keys += int(((ids >= 0) & (ids < ((pos + 1) // 4)[:, None])).sum())
        elif m["ratio"] == 128:
            keys += int(((pos + 1) // 128).sum())
        return keys

    def algorithmic_bytes(self, layer=0, lse=False):
        """Bytes one launch must move at minimum: each distinct KV row of a
        sequence and kind once (512 B), Q, output (+LSE), the index list, the
        distinct block-table entries, both scales, sinks and metadata."""
        m = self.meta
        block = workloads.BLOCK
        ix = self.indices[layer]
        rows = entries = 0
        for b in range(len(m["seq_lens"])):
            sel = m["owner"] == b
            pos = m["positions"][sel]
            if not len(pos):
                continue
            lo, hi = max(0, int(pos.min()) - m["window"] + 1), int(pos.max())
            rows += hi - lo + 1
            entries += hi // block - lo // block + 1
            if m["ratio"] == 4:
                ids = ix[sel, 0]
                valid = (ids >= 0) & (ids < ((pos + 1) // 4)[:, None])
                ids = np.unique(ids[valid])
            elif m["ratio"] == 128:
                ids = np.arange((int(pos.max()) + 1) // 128)
            else:
                ids = np.zeros(0, np.int64)
            rows += len(ids)
            entries += len(np.unique(ids // block))
        tokens = len(m["positions"])
        heads = self.heads
        q_out = tokens * heads * DIM * 2 * 2 + (tokens * heads * 4 if lse else 0)
        index_bytes = ix.size * 4 if ix is not None else 0
        scales = DIM * 4 * (2 if m["ratio"] != 1 else 1) + heads * 4
        meta = (len(m["cu_q"]) + len(m["seq_lens"])) * 4
        return rows * DIM + q_out + index_bytes + entries * 4 + scales + meta
