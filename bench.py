"""Benchmark: INT8 shared-KV decode queries/s and HBM GB/s on one MI355X.

Workload (BASELINE.json metric "INT8 sharedKV decode queries/s + HBM GB/s (% of
peak), B=32 C4 top-k1024"): B=32 sequences x T=2 query tokens (main + draft
slot), H=8, D=512, BF16 Q; contexts ~U[2048, 65536]; every sequence on the C4
launch: SWA128 window + top-k1024 compressed rows drawn from the visible range;
INT8 block32 pages at the serving page stride (622592 B) in a pool sized 1.25x
the need with shuffled block tables.  Synthetic data generated on the GPU.

A step is one attention launch (one layer of one decode step).  Steps rotate
over `--layers` layers (32 by default: over 1 GiB of distinct rows) whose
pages interleave in the 622592-B page stride the way a serving pool holds
every layer's 16 KiB page, so consecutive steps read different HBM (the
union of bytes read per rotation is four times the 256 MB MALL).  The K
timed steps are one captured HIP graph of K launches (serving runs decode in
graphs).  Protocol of the reference's capacity benchmark
(tests/npu/test_capacity.py:166-190 of the reference checkout): W eager
warmup launches, then the graph and its companions (below) are each
replayed 3 times untimed, then 9 rounds in alternating order each replay
every graph once between HIP events on the replay stream; the reported time
per launch is the median over the 9 rounds of (round time / K).
Companions, timed in the same rounds: the launch's data-movement floor
(csrc/gather_floor.hip: the exact rows each work item of the launch
gathers, copied into LDS with the same instructions, grid and two-tile
ring, with no metadata round trips, compute or merge), and a streaming read
of the same byte count through the same kernel.  The CPU baseline is the C
restatement (oracle/, "port") timed on a bounded sample on this host, rank 0
only.

Prints ONE JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "ascend-int8-attention_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "INT8 sharedKV decode queries/s + HBM GB/s (% of peak), B=32 C4 top-k1024"
PEAK_HBM_GBS = 8000.0
SERVING_STRIDE = 622592


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def workload(name, rng):
    """(seed, ratio, queries, lengths, page stride, description) of a launch.
    The BASELINE configs (seeds as recorded there: config 0 uses seed 0)."""
    s = SERVING_STRIDE
    if name == "headline":
        lengths = rng.integers(2048, 65537, 32)
        return (7, 4, [2] * 32, lengths, s,
                "headline: C4 top-k1024 decode, B=32 x T=2 (main + draft), ctx~U[2048,65536]")
    if name == "cfg0":
        return (0, 128, [1], [4096], s, "config 0: C128 decode, B=1 x T=1, ctx 4096")
    if name == "cfg1":
        return (1, 4, [1], [16384], s, "config 1: C4 top-k1024 decode, B=1 x T=1, ctx 16384")
    if name == "cfg2_c4":
        lengths = rng.integers(2048, 65537, 16)
        return (2, 4, [2] * 16, lengths, s, "config 2 C4 launch: 16 seqs x T=2, ctx~U[2048,65536]")
    if name == "cfg2_c128":
        lengths = rng.integers(2048, 65537, 16)
        return (12, 128, [2] * 16, lengths, s, "config 2 C128 launch: 16 seqs x T=2, ctx~U[2048,65536]")
    if name == "cfg3_prefill":
        return (3, 4, [2048], [32768], s, "config 3: C4 chunked prefill, B=1 x T=2048 on a 30720 prefix")
    if name == "cfg4_c4":
        lengths = rng.integers(65536, 131073, 64)
        return (4, 4, [1] * 64, lengths, s, "config 4 C4 layer: B=64 x T=1, ctx~U[65536,131072]")
    if name == "cfg4_c128":
        lengths = rng.integers(65536, 131073, 64)
        return (14, 128, [1] * 64, lengths, s, "config 4 C128 layer: B=64 x T=1, ctx~U[65536,131072]")
    if name == "c128":
        lengths = rng.integers(2048, 65537, 32)
        return (8, 128, [2] * 32, lengths, s, "C128 decode, B=32 x T=2, ctx~U[2048,65536]")
    raise SystemExit(f"unknown workload {name}")


WORKLOADS = ["headline", "cfg0", "cfg1", "cfg2_c4", "cfg2_c128", "cfg3_prefill", "cfg4_c4", "cfg4_c128", "c128",
             "cfg4_writer", "custom"]


def custom_workload(args, rng):
    """A decode or prefill shape outside the BASELINE configs (--workload
    custom): --batch sequences of --query-tokens each, lengths uniform in
    --ctx LO:HI, ratio --ratio, at the serving page stride."""
    lo, hi = (int(x) for x in args.ctx.split(":"))
    if not args.query_tokens <= lo <= hi:
        raise SystemExit("--ctx LO:HI needs query-tokens <= LO <= HI")
    lengths = rng.integers(lo, hi + 1, args.batch)
    return (20, args.ratio, [args.query_tokens] * args.batch, lengths, SERVING_STRIDE,
            f"custom: C{args.ratio}, B={args.batch} x T={args.query_tokens}, ctx~U[{lo},{hi}]")


def copy_calibration(mib, torch):
    """A plain device copy of `mib` MiB, four times: the reference dispatches
    for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes."""
    if not mib:
        return
    n = mib << 20
    src = torch.ones(n, dtype=torch.int8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"[bench] copy calibration: 4 copies of {n} bytes (read {n // 1024} KiB, write {n // 1024} KiB each)")


def bench_writer(args, torch):
    """Config 4's writer: 4096 BF16 rows quantised and scattered through a
    random unique slot mapping into a stride-viewed block32 pool (page stride
    622592 B), rotated over `--layers` update batches and pools."""
    import numpy as np
    from npu_sparse_attn_sharedkv_int8 import CacheQuantization, PreparedCacheWrite
    rows, pages, stride = 4096, 1024, SERVING_STRIDE
    layers = max(1, min(args.layers, stride // 16384))
    gen = torch.Generator(device="cuda").manual_seed(4)
    raw = torch.zeros(pages * stride, dtype=torch.int8, device="cuda")
    ops = []
    rng = np.random.default_rng(4)
    for layer in range(layers):
        cache = raw[layer * 16384:].as_strided((pages, 32, 1, 512), (stride, 512, 512, 1))
        updates = torch.randn((rows, 512), generator=gen, device="cuda").bfloat16()
        slots = torch.from_numpy(rng.choice(pages * 32, rows, replace=False).astype(np.int32)).cuda()
        quant = CacheQuantization.calibrate([updates.float().cpu()])
        ops.append(PreparedCacheWrite(cache, updates, slots, quant.inverse_scale.cuda()))
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for i in range(args.warmup):
            ops[i % layers].run()
    torch.cuda.synchronize()
    graph = capture(stream, args.steps, lambda i: ops[i % layers].run(), torch)
    medians, samples = timed_rounds({"writer": graph}, stream, args.steps, torch)
    ms_per_step = medians["writer"] / 1e3
    algorithmic = rows * (512 * 2 + 512 + 4) + 512 * 4
    achieved = algorithmic / (ms_per_step * 1e-3) / 1e9
    traffic, traffic_source = recorded_traffic("cfg4_writer")
    record = {
        "metric": "INT8 KV cache write rows/s + HBM GB/s, config 4 writer", "value": rows / (ms_per_step * 1e-3),
        "unit": "rows/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "i8",
        "data": "synthetic (GPU-generated, seeded)",
        "config": {"workload": "config 4 writer: 4096 BF16 rows, random unique int32 slots, page stride 622592",
                   "rows": rows, "pages": pages, "page_stride": stride, "layers_rotated": layers,
                   "timing": "median of 9 rounds, each one replay of a graph of K launches between HIP events"},
        "latency_us_per_launch": ms_per_step * 1e3,
        "rounds_us_per_launch": samples["writer"],
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS, "traffic": traffic, "traffic_source": traffic_source,
                     "algorithmic_bytes_per_launch": algorithmic},
    }
    if not args.no_cpu:
        log(f"[bench] writer CPU baseline ({args.cpu_seconds:.0f} s sample)")
        record["cpu_baseline"] = writer_cpu_baseline(rows, pages, stride, args.cpu_seconds)
    return record


def launch_rows(dc, layer, plan):
    """Per work item (query row, partition) of a tiled launch at `plan`
    partitions, the HBM row addresses it gathers, tile by tile, in the
    kernel's selection order: the SWA window rows, then the compressed list
    (C4: the valid top-k entries, compacted when the visible range is
    shorter than top-k, masked holes in place otherwise; C128: every visible
    compressed row), cut into 128-key tiles, tile k on partition k % plan.
    Masked places read the Q base, as the kernel's do.  Returns (addresses
    INT64 [items, max tiles, 128], tiles INT32 [items], bounds) where bounds
    lists the (low, high) byte ranges every address falls in."""
    import numpy as np
    m = dc.meta
    ratio, window, topk = m["ratio"], m["window"], m["topk"]
    pos_all, owner = m["positions"], m["owner"]
    q_base = dc.cases[layer].q.data_ptr()
    kinds = [(dc.ori, dc.ori.flat.data_ptr() + layer * dc.ori.PAGE_BYTES)]
    if dc.cmp is not None:
        kinds.append((dc.cmp, dc.cmp.flat.data_ptr() + layer * dc.cmp.PAGE_BYTES))
    rows = []
    for t, pos in enumerate(pos_all):
        b = int(owner[t])
        first = max(0, int(pos) + 1 - window)
        idx = np.arange(first, int(pos) + 1)
        lists = [(0, idx, np.ones(len(idx), bool))]
        count = (int(pos) + 1) // ratio if ratio != 1 else 0
        if ratio == 4:
            ix = dc.indices[layer][t, 0].astype(np.int64)
            ok = (ix >= 0) & (ix < count)
            if count < topk <= 1024:
                lists.append((1, ix[ok], np.ones(int(ok.sum()), bool)))
            else:
                lists.append((1, np.where(ok, ix, 0), ok))
        elif ratio == 128:
            lists.append((1, np.arange(count), np.ones(count, bool)))
        tiles = []
        for kind, ids, ok in lists:
            pool, base = kinds[kind]
            page = pool.table[b][ids // 32].astype(np.int64)
            addr = base + page * pool.page_stride + (ids % 32) * 512
            addr = np.where(ok, addr, q_base)
            for start in range(0, len(ids), 128):
                tile = np.full(128, q_base, np.int64)
                chunk = addr[start:start + 128]
                tile[:len(chunk)] = chunk
                tiles.append(tile)
        rows.append(tiles)
    items = [[tiles[k] for k in range(part, len(tiles), plan)] for tiles in rows for part in range(plan)]
    max_tiles = max(1, max(len(x) for x in items))
    out = np.zeros((len(items), max_tiles, 128), np.int64)
    counts = np.zeros(len(items), np.int32)
    for i, tiles in enumerate(items):
        counts[i] = len(tiles)
        for k, tile in enumerate(tiles):
            out[i, k] = tile
    bounds = [(q_base, q_base + 512)] + [(base, base + pool.pages * pool.page_stride) for pool, base in kinds]
    return out, counts, bounds


class FloorLegs:
    """The two companion legs of the timed rounds (csrc/gather_floor.hip,
    _native/libsharedkv_floor.so): `gather` copies each work item's rows of
    the attention launch (launch_rows, per layer) and `stream` reads the same
    number of bytes contiguously, with the same kernel, grid and ring.  Every
    address is checked on the host to lie inside the pool it names before
    any launch."""

    def __init__(self, dc, layers, plan, torch, non_temporal):
        import ctypes
        import numpy as np
        from npu_sparse_attn_sharedkv_int8._paths import NATIVE_DIR
        self.lib = ctypes.CDLL(str(NATIVE_DIR / "libsharedkv_floor.so"))
        self.lib.sharedkv_floor_gather.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                                   ctypes.c_uint32, ctypes.c_uint32, ctypes.c_int]
        self.lib.sharedkv_floor_gather.restype = ctypes.c_int
        self.nt = int(bool(non_temporal))
        self.gather, self.stream = [], []
        self.keep = []
        for layer in range(layers):
            addrs, tiles, bounds = launch_rows(dc, layer, plan)
            flat = addrs.reshape(-1, 128)
            live = np.repeat(np.arange(addrs.shape[1])[None, :], len(tiles), 0) < tiles[:, None]
            used = addrs[live].reshape(-1)
            inside = np.zeros(used.shape, bool)
            for lo, hi in bounds:
                inside |= (used >= lo) & (used + 512 <= hi)
            if not inside.all():
                raise SystemExit("floor leg: a row address falls outside its pool")
            self.gather.append((torch.from_numpy(addrs).cuda(), torch.from_numpy(tiles).cuda(), len(tiles),
                                addrs.shape[1]))
            del flat
        # Streaming read: each layer's tile count of contiguous 64 KiB tiles in
        # one buffer, layers one after another.
        tiles0 = self.gather[0][1].cpu().numpy()
        per_layer = int(tiles0.sum())
        self.bytes_per_launch = per_layer * 128 * 512
        self.buffer = torch.empty(layers * self.bytes_per_launch, dtype=torch.int8, device="cuda")
        base = self.buffer.data_ptr()
        for layer in range(layers):
            _, tiles_dev, items, max_tiles = self.gather[layer]
            tiles = tiles_dev.cpu().numpy()
            first = np.concatenate(([0], np.cumsum(tiles)[:-1]))
            k = first[:, None] + np.arange(max_tiles)[None, :]
            addrs = (base + layer * self.bytes_per_launch
                     + (k[:, :, None] * 128 + np.arange(128)[None, None, :]) * 512).astype(np.int64)
            addrs = np.where((np.arange(max_tiles)[None, :] < tiles[:, None])[:, :, None], addrs, base)
            self.stream.append((torch.from_numpy(addrs).cuda(), tiles_dev, items, max_tiles))

    def launch(self, which, layer, torch):
        addrs, tiles, items, max_tiles = (self.gather if which == "gather" else self.stream)[layer]
        rc = self.lib.sharedkv_floor_gather(torch.cuda.current_stream().cuda_stream, addrs.data_ptr(),
                                            tiles.data_ptr(), items, max_tiles, self.nt)
        if rc:
            raise RuntimeError(f"floor launch failed: {rc}")


def timed_rounds(graphs, stream, depth, torch, rounds=9, warm=3):
    """The reference's paired timing (test_capacity.py:166-190): every graph
    replayed `warm` times, then `rounds` rounds, each replaying every graph
    once in an order that rotates and reverses from round to round, between
    HIP events on `stream`.  Returns ({name: median us per launch},
    {name: [us per launch of each round]})."""
    import statistics
    names = list(graphs)
    with torch.cuda.stream(stream):
        for _ in range(warm):
            for graph in graphs.values():
                graph.replay()
        torch.cuda.synchronize()
        samples = {name: [] for name in names}
        for r in range(rounds):
            order = names[r % len(names):] + names[:r % len(names)]
            if r % 2:
                order = order[::-1]
            for name in order:
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                a.record(stream)
                graphs[name].replay()
                b.record(stream)
                b.synchronize()
                samples[name].append(a.elapsed_time(b) * 1e3 / depth)
    return {name: statistics.median(v) for name, v in samples.items()}, samples


def capture(stream, steps, launch, torch):
    """A HIP graph of `steps` calls launch(i) captured on `stream`."""
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for i in range(steps):
                launch(i)
    return graph


def host_cores():
    """Threads the CPU baseline may use: the job's CPU share (OMP_NUM_THREADS
    where the launcher sets it, else the process's CPU affinity)."""
    affinity = len(os.sched_getaffinity(0))
    share = int(os.environ.get("OMP_NUM_THREADS") or affinity)
    return max(1, min(share, affinity))


def cpu_baseline(dc, layers, splits, seconds, cmp_rows, query_group=1, tile=128):
    """Time the C restatement on whole launches of the same workload until
    about `seconds` of wall time have passed (bounded sample), on every host
    core of the job's share and then on one thread (half the time)."""
    import oracle.oracle as ora
    from npu_sparse_attn_sharedkv_int8 import c8_attention
    from tests import workloads
    hosts = [workloads.oracle_case(dc.host(layer)) for layer in range(min(layers, 2))]
    m = dc.meta
    joint_dense = c8_attention.joint_plan(m["ratio"], dc.heads, False) and m["ratio"] == 128 and query_group == 1
    joint_sparse = m["ratio"] == 4 and splits == 1 and query_group == 1 and c8_attention.joint_launch(
        splits, int(m["cu_q"][-1]), dc.heads, 4, m["cu_q"], m["seq_lens"], cmp_rows=cmp_rows)

    def timed(threads, budget):
        queries = launches = 0
        start = time.perf_counter()
        while time.perf_counter() - start < budget:
            ora.tiled_attention(hosts[launches % len(hosts)], tile=tile, splits=splits, return_lse=False,
                                joint_dense=joint_dense, joint_sparse=joint_sparse, threads=threads,
                                query_group=query_group)
            queries += int(dc.meta["cu_q"][-1])
            launches += 1
        elapsed = time.perf_counter() - start
        return queries / elapsed, (f"{launches} whole launches of the bench workload ({queries} queries, "
                                   f"{min(layers, 2)} layers' data) through oracle/libsharedkv_oracle.so, "
                                   f"{threads} OpenMP thread(s), {elapsed:.1f} s")

    cores = host_cores()
    value, sample = timed(cores, seconds)
    single, single_sample = timed(1, seconds / 2)
    return dict(value=value, unit="queries/s", cores=cores, kind="port", sample=sample,
                host={"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)),
                      "omp_num_threads": os.environ.get("OMP_NUM_THREADS")},
                single_thread={"value": single, "unit": "queries/s", "cores": 1, "sample": single_sample})


def writer_cpu_baseline(rows, pages, stride, seconds):
    """The writer's C restatement (oracle/, scalar, one thread) on the same
    shape: `rows` BF16 rows through a random unique slot mapping into a
    `pages`-page pool at `stride` bytes a page, repeated for ~`seconds`."""
    import numpy as np
    import oracle.oracle as ora
    from tests import workloads
    rng = np.random.default_rng(4)
    pool = np.zeros(pages * stride, np.int8)
    updates = workloads.bf16_bits(rng.standard_normal((rows, 512), dtype=np.float32))
    slots = rng.choice(pages * 32, rows, replace=False).astype(np.int32)
    inverse = ora.inverse_scale(workloads.frozen_scale(workloads.bf16_value(updates)))
    ora.cache_write(pool, stride, pages, 32, updates, slots, inverse)     # untimed: first touch of the pool
    calls = 0
    start = time.perf_counter()
    while time.perf_counter() - start < seconds:
        ora.cache_write(pool, stride, pages, 32, updates, slots, inverse)
        calls += 1
    elapsed = time.perf_counter() - start
    return dict(value=calls * rows / elapsed, unit="rows/s", cores=1, kind="port",
                sample=f"{calls} whole launches ({rows} rows each) through oracle/libsharedkv_oracle.so "
                       f"sko_cache_write, one thread, {elapsed:.1f} s")


def recorded_traffic(workload):
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary of this workload (scaled by a plain copy's reading),
    or None.  A recorded figure: bench.py itself does not run counters."""
    path = ROOT / "profiles" / f"traffic_{workload}.md"
    if path.exists():
        for line in path.read_text().splitlines():
            if line.startswith("bytes_per_launch:"):
                return int(line.split(":", 1)[1]), f"profiles/{path.name}"
    return None, None


def eager_latency(op, stream, torch, calls=50):
    """Per-call latency of single eager launches: HIP events around each
    launch on its stream (kernel time alone) and host wall time of run()
    plus synchronize (what a caller without graphs waits); medians."""
    import statistics
    kernel, wall = [], []
    with torch.cuda.stream(stream):
        for _ in range(calls):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            a.record(stream)
            op.run()
            b.record(stream)
            torch.cuda.synchronize()
            wall.append((time.perf_counter() - t0) * 1e6)
            kernel.append(a.elapsed_time(b) * 1e3)
    # The same wall-clock measure around a one-element torch add: the floor
    # of one eager launch plus synchronisation on this runtime.
    tiny = torch.zeros(1, device="cuda")
    floor = []
    with torch.cuda.stream(stream):
        for _ in range(calls):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            tiny.add_(1)
            torch.cuda.synchronize()
            floor.append((time.perf_counter() - t0) * 1e6)
    return {"calls": calls, "kernel_us_median": statistics.median(kernel),
            "call_us_median": statistics.median(wall), "null_call_us_median": statistics.median(floor),
            "note": "each launch alone: events on its stream around one run(); call = host wall of run() + "
                    "synchronize, launch overhead included; null call = the same around a one-element torch add"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=160)
    ap.add_argument("--warmup", type=int, default=32)
    ap.add_argument("--layers", type=int, default=32, help="layers rotated over (<= 38 in the page stride)")
    ap.add_argument("--workload", default="headline", choices=WORKLOADS)
    ap.add_argument("--splits", type=int, default=None, help="override the host plan's KV partitions")
    ap.add_argument("--page-stride", type=int, default=None, help="override the workload's page stride (bytes)")
    ap.add_argument("--merge", type=int, default=0, help="0: fused partition merge, 1: separate merge launch")
    ap.add_argument("--heads", type=int, default=8, help="query heads per token (the metric is quoted at 8)")
    ap.add_argument("--query-group", type=int, default=None, choices=[1, 2, 4],
                    help="2 or 4: the query-grouped plan (groups of 2 or 4 query tokens share one window and one "
                         "compressed list)")
    ap.add_argument("--tile-size", type=int, default=None, choices=[128, 256],
                    help="keys per tile of a grouped plan (default 256, the reference operator's; 128 also)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-floor", action="store_true", help="skip the gather-floor and streaming-read legs")
    ap.add_argument("--live", type=int, default=None, metavar="SEQS",
                    help="also replay the captured graph with only SEQS sequences live (graph padding; the "
                         "kernel re-plans partitions on the device); default 8 for the headline, 0 = skip")
    ap.add_argument("--ratio", type=int, default=4, choices=[1, 4, 128], help="custom workload: cache ratio")
    ap.add_argument("--batch", type=int, default=32, help="custom workload: sequences")
    ap.add_argument("--query-tokens", type=int, default=2, help="custom workload: query tokens per sequence")
    ap.add_argument("--ctx", default="2048:65536", help="custom workload: sequence lengths LO:HI (uniform)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="also run a plain device copy of MIB MiB four times (the reference kernel "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the path shards by sequence, each GPU running this kernel on its own rows", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch
    from npu_sparse_attn_sharedkv_int8 import PreparedAttention
    from tests.device_cases import DeviceCase

    torch.cuda.set_device(0)
    if args.workload == "cfg4_writer":
        record = bench_writer(args, torch)
        copy_calibration(args.copy_calibration, torch)
        print(json.dumps(record), flush=True)
        return
    from npu_sparse_attn_sharedkv_int8.runtime import library
    if library().sharedkv_c8_set_merge_mode(args.merge):
        raise SystemExit(f"unknown merge mode {args.merge}")
    rng = np.random.default_rng(2026)
    seed, ratio, queries, lengths, stride, description = (
        custom_workload(args, rng) if args.workload == "custom" else workload(args.workload, rng))
    stride = args.page_stride or stride
    layers = max(1, min(args.layers, stride // 16384))
    log(f"[bench] generating {description}; {layers} layers at page stride {stride}")
    t0 = time.perf_counter()
    dc = DeviceCase(seed, ratio, queries, lengths, page_stride=stride, layers=layers, heads=args.heads)
    torch.cuda.synchronize()
    log(f"[bench] generated in {time.perf_counter() - t0:.1f} s: ori pages {dc.ori.pages}, "
        f"cmp pages {dc.cmp.pages if dc.cmp else 0}")
    ops = [PreparedAttention(dc.cases[l], dc.ori_scales[l], dc.cmp_scales[l], splits=args.splits,
                             query_group=args.query_group, tile_size=args.tile_size)
           for l in range(layers)]
    splits = ops[0].splits
    group = ops[0].query_group
    from npu_sparse_attn_sharedkv_int8 import c8_attention
    # The partitions the kernel runs: the device re-plans joint C128 launches
    # (and padded ones, below) from the live metadata; the paired plan keeps
    # the launch's.
    cmp_rows = ops[0].args.cmpTableWidth * c8_attention.BLOCK
    device_plan = splits if group != 1 else c8_attention.device_splits(
        splits, int(dc.meta["cu_q"][-1]), args.heads, ratio, 1024, dc.meta["cu_q"], dc.meta["seq_lens"],
        fused=args.merge == 0, cmp_rows=cmp_rows)
    live_queries = int(sum(queries))
    bytes_per_launch = [dc.algorithmic_bytes(l) for l in range(layers)]

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        log(f"[bench] warmup {args.warmup} eager launches (splits={splits})")
        for i in range(args.warmup):
            ops[i % layers].run()
    torch.cuda.synchronize()
    graphs = {"attention": capture(stream, args.steps, lambda i: ops[i % layers].run(), torch)}
    tokens = int(dc.meta["cu_q"][-1])
    joint = group == 1 and device_plan == 1 and c8_attention.joint_launch(
        splits, tokens, args.heads, ratio, dc.meta["cu_q"], dc.meta["seq_lens"], cmp_rows=cmp_rows)
    rows_kernel = ratio == 4 and device_plan == 1 and tokens * ((args.heads + 7) // 8) > c8_attention.CORES
    floor = None
    if not args.no_floor and args.heads == 8 and not joint and not rows_kernel and group == 1:
        streamed = tokens <= (4 if ratio == 4 else 1 if ratio == 128 else 0) * len(queries)
        log(f"[bench] floor legs: gather of the launch's rows and a streaming read (non-temporal {streamed})")
        floor = FloorLegs(dc, layers, device_plan, torch, streamed)
        graphs["gather_floor"] = capture(stream, args.steps, lambda i: floor.launch("gather", i % layers, torch),
                                         torch)
        graphs["stream_read"] = capture(stream, args.steps, lambda i: floor.launch("stream", i % layers, torch),
                                        torch)
    wall0 = time.perf_counter()
    medians, samples = timed_rounds(graphs, stream, args.steps, torch)
    wall = time.perf_counter() - wall0
    ms_per_step = medians["attention"] / 1e3
    log(f"[bench] 9 rounds x {len(graphs)} graphs of {args.steps} launches in {wall * 1e3:.1f} ms wall; "
        + ", ".join(f"{k} {v:.2f} us" for k, v in medians.items()))
    mean_bytes = sum(bytes_per_launch[i % layers] for i in range(args.steps)) / args.steps
    achieved = mean_bytes / (ms_per_step * 1e-3) / 1e9
    floor_record = None
    if floor is not None:
        floor_record = {
            "gather_us": medians["gather_floor"], "stream_read_us": medians["stream_read"],
            "attention_us": medians["attention"], "bytes_per_launch": floor.bytes_per_launch,
            "gather_gbs": floor.bytes_per_launch / (medians["gather_floor"] * 1e-6) / 1e9,
            "stream_read_gbs": floor.bytes_per_launch / (medians["stream_read"] * 1e-6) / 1e9,
            "gather_frac_of_peak_algorithmic": mean_bytes / (medians["gather_floor"] * 1e-6) / 1e9 / PEAK_HBM_GBS,
            "note": "same 9 alternating rounds as the attention graph; gather = every row the launch's work items "
                    "copy (tiles of 128 x 512 B, masked places included), with the launch's grid, item order, "
                    "LDS DMA instruction and two-tile ring but no metadata round trips, compute or merge "
                    "(csrc/gather_floor.hip); stream_read = the same byte count read contiguously by the "
                    "same kernel"}

    # HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE
    # (scaled by a plain copy's reading); the summary states the commands.
    traffic, traffic_source = recorded_traffic(args.workload) if args.heads == 8 else (None, None)

    # The same graph replayed with only `live` sequences live: the rest get
    # seq_len 0 (graph padding) and the kernel hands their work-groups to the
    # live rows as extra partitions (c8_attention.device_splits).
    live_seqs = args.live if args.live is not None else (8 if args.workload == "headline" else 0)
    padded = None
    if 0 < live_seqs < len(queries) and args.merge == 0 and group == 1:
        import dataclasses
        cu_full, lens_full = dc.meta["cu_q"].copy(), dc.meta["seq_lens"].copy()
        cu = cu_full.copy()
        cu[live_seqs + 1:] = cu_full[live_seqs]
        lens = lens_full.copy()
        lens[live_seqs:] = 0
        live_rows = int(cu[live_seqs])
        padded_plan = c8_attention.device_splits(splits, int(cu_full[-1]), args.heads, ratio, 1024, cu, lens,
                                                 cmp_rows=cmp_rows)
        # The same layers' launches planned for the live sequences alone.
        live_ops = []
        for l in range(layers):
            c = dc.cases[l]
            live_case = dataclasses.replace(
                c, q=c.q[:live_rows], cu_q=c.cu_q[:live_seqs + 1], seq_lens=c.seq_lens[:live_seqs],
                ori_block_table=c.ori_block_table[:live_seqs],
                cmp_block_table=c.cmp_block_table[:live_seqs] if c.cmp_block_table is not None else None,
                cmp_indices=c.cmp_indices[:live_rows] if c.cmp_indices is not None else None)
            live_ops.append(PreparedAttention(live_case, dc.ori_scales[l], dc.cmp_scales[l]))
        with torch.cuda.stream(stream):
            for i in range(layers):
                live_ops[i].run()
        torch.cuda.synchronize()
        live_graph = capture(stream, args.steps, lambda i: live_ops[i % layers].run(), torch)
        dc.dev.cu_q.copy_(torch.from_numpy(cu))
        dc.dev.seq_lens.copy_(torch.from_numpy(lens))
        torch.cuda.synchronize()
        pad_medians, _ = timed_rounds({"padded": graphs["attention"], "live_only": live_graph}, stream, args.steps,
                                      torch)
        dc.dev.cu_q.copy_(torch.from_numpy(cu_full))
        dc.dev.seq_lens.copy_(torch.from_numpy(lens_full))
        torch.cuda.synchronize()
        us, live_us = pad_medians["padded"], pad_medians["live_only"]
        padded = {"capacity_sequences": len(queries), "live_sequences": live_seqs, "live_queries": live_rows,
                  "launch_splits": splits, "device_splits": padded_plan, "us_per_launch": us,
                  "queries_per_s": live_rows / (us * 1e-6), "live_only_us_per_launch": live_us,
                  "live_only_splits": live_ops[0].splits, "padded_over_live_only": us / live_us,
                  "note": "the timed graph replayed with the sequences past the live ones at seq_len 0, against a "
                          "graph of the same layers' launches planned for the live sequences alone; medians of 9 "
                          "alternating rounds"}
        log(f"[bench] padded graph: {live_seqs} of {len(queries)} sequences live, {padded_plan} partitions, "
            f"{us:.2f} us per launch; the live rows alone: {live_us:.2f} us ({live_ops[0].splits} partitions)")

    eager = eager_latency(ops[0], stream, torch)
    log(f"[bench] eager: kernel {eager['kernel_us_median']:.2f} us, call {eager['call_us_median']:.2f} us")

    # int8 MFMA work the launch performs: per selected key, QK and PV over
    # 16 rows (8 heads x {code, residual}) x 512 channels, 2 ops per MAC.
    keys = dc.selected_keys(0)
    int8_ops = keys * 16 * 512 * 2 * 2 * ((args.heads + 7) // 8)   # per group of eight heads
    metric = (METRIC if args.workload == "headline" and args.heads == 8 else
              f"INT8 sharedKV attention queries/s + HBM GB/s, {args.workload}, {args.heads} heads"
              + (", paired plan" if group == 2 else ""))
    record = {
        "metric": metric, "value": live_queries / (ms_per_step * 1e-3), "unit": "queries/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": ms_per_step, "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "i8", "data": "synthetic (GPU-generated, seeded)",
        "config": {"workload": description, "batch": len(queries), "query_tokens": live_queries, "heads": args.heads,
                   "dim": 512, "ratio": ratio, "topk": 1024 if ratio == 4 else 0, "window": 128,
                   "page_stride": stride, "layers_rotated": layers, "tile": ops[0].tile_size, "splits": splits,
                   "device_splits": device_plan,
                   "joint_rows": bool(joint), "query_group": group,
                   "lse": False, "merge": "fused" if args.merge == 0 else "separate launch",
                   "timing": "median of 9 alternating rounds (reference protocol), each one replay of a graph of "
                             "K launches between HIP events on its stream, after 3 untimed replays"},
        "latency_us_per_layer": ms_per_step * 1e3,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS, "traffic": traffic, "traffic_source": traffic_source,
                     "algorithmic_bytes_per_launch": mean_bytes},
        "mfma": {"int8_ops_per_launch": int8_ops, "achieved_tops": int8_ops / (ms_per_step * 1e-3) / 1e12,
                 "peak_tops": 5000.0, "frac": int8_ops / (ms_per_step * 1e-3) / 1e12 / 5000.0},
        "eager_latency": eager,
        "rounds_us_per_launch": samples["attention"],
    }
    if floor_record:
        record["floor"] = floor_record
    if padded:
        record["padded_graph"] = padded
    copy_calibration(args.copy_calibration, torch)
    if not args.no_cpu:
        log(f"[bench] CPU baseline ({args.cpu_seconds:.0f} s sample)")
        record["cpu_baseline"] = cpu_baseline(dc, layers, device_plan, args.cpu_seconds, cmp_rows, group,
                                              ops[0].tile_size)
    print(json.dumps(record), flush=True)


if __name__ == "__main__":
    main()
