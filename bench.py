"""Paged decode attention benchmark on one MI355X (gfx950).

One step = one gk_paged_decode call (C ABI) over the whole batch of the
workload: every sequence's new query row attends its paged K/V through the
block tables, split-K partitions plus log-sum-exp merge, bf16 output. Inputs
(pool, queries, block tables, lengths) are resident in HBM before timing
starts. Consecutive steps rotate over `--table-sets` disjoint block-table sets
of the same pool (same lengths, different blocks), so a step cannot be served
from the 256 MB last-level cache that the previous step filled.

Prints ONE JSON line: value = decode tokens/s (sequences per second of one
layer's attention step), the HBM roofline of the decode kernel measured with
HIP events on the launch stream, and the CPU baseline (the C oracle, a
restatement of the reference's direct_bf16_pv, on the host's cores). With the
default headline workload (c2) the same line carries `secondary`: the other
GPU configurations (c3 fused store + decode, c5 long-context decode: HBM
roofline; c4 prefix-shared prefill: MFMA roofline), each timed the same way,
`--steps` steps each (c3 and c5 after at least 100 warm-up steps, c4 after
1000), right after the headline, each by a child `bench.py --workload` process
of its own (a pool allocated after others were released ran ~4% slower); the
CPU baseline runs last.

    python bench.py [--gpus 1] [--steps 200] [--warmup 20 (c4: 1000)] [--workload c2] [--no-cpu]
                    [--no-secondary] [--host-overhead] [--page-size N]

--host-overhead instead times the drop-in op torch.ops.gaudirt.paged_attn on
C2's decode step (store of each row's new K/V, then attention), host side and
GPU side: per step, the host microseconds of building the metadata and
launching the op, for the reference's host constructor path
(PagedMetadata(locations, requests, positions, mapping, slots)) and for the
serving path (PagedMetadata._from_scheduler on device-resident inputs), next
to the GPU time of the same step. It prints its own JSON line.
"""

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "decode attn tokens/s + achieved KV-read HBM GB/s (% of 8 TB/s), 1 MI355X"
HBM_PEAK_GBPS = 8000.0

WORKLOADS = {
    "c2": "Llama-3-8B-shaped paged decode: batch 64, 32 q / 8 kv heads, head_dim 128, block 128, "
          "ctx U[512,4096], 4096-block bf16 pool",
    "c3": "fused KV store + decode: batch 256, 32 q / 8 kv heads, head_dim 128, block 128, len U[128,2048]",
    "c5": "70B-shaped long decode: batch 32, 64 q / 8 kv heads, head_dim 128, block 128, "
          "ctx log-U[1024,32768], 8192-block pool, split-K",
    "c4": "prefix-shared chunked prefill: 8 sequences x 512-row causal chunks on a shared 2048-token prefix, "
          "32 q / 8 kv heads, head_dim 128, block 128",
    "c2g2": "c2 at GQA group 2: batch 64, 16 q / 8 kv heads, head_dim 128, block 128, ctx U[512,4096], "
            "4096-block bf16 pool",
    "c2g1": "c2 at GQA group 1: batch 64, 8 q / 8 kv heads, head_dim 128, block 128, ctx U[512,4096], "
            "4096-block bf16 pool",
    "c2g3": "c2 at GQA group 3: batch 64, 24 q / 8 kv heads, head_dim 128, block 128, ctx U[512,4096], "
            "4096-block bf16 pool",
    "c4d256": "c4 at head_dim 256 (Gemma-2-9B-shaped heads): 8 sequences x 512-row causal chunks on a shared "
              "2048-token prefix, 16 q / 8 kv heads, head_dim 256, block 128",
}
# Prefill workloads: DevicePrefillCase arguments besides the C4 defaults.
PREFILL_WORKLOADS = {"c4": {}, "c4d256": {"heads": 16, "kv_heads": 8, "head_dim": 256}}
C4_WARMUP = 1000
MFMA_BF16_PEAK_TFLOPS = 2500.0


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=int(os.environ.get("WORLD_SIZE", "1")))
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=None,
                    help="untimed steps first (default 20; 1000 for c4, whose MFMA-bound kernel runs "
                         "~6%% slower until the GPU has been busy for ~0.1 s)")
    ap.add_argument("--workload", default="c2", choices=sorted(WORKLOADS))
    ap.add_argument("--table-sets", type=int, default=3)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--partition", type=int, default=0, help="split-K partition tokens (0 = library choice)")
    ap.add_argument("--page-size", type=int, default=0,
                    help="decode workloads: re-page the block tables to pages of this many tokens (same tokens; "
                         "1 = the token-granular map); 0 = the workload's block size")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-secondary", action="store_true",
                    help="headline workload only (no c3/c4/c5 entries after a c2 headline)")
    ap.add_argument("--host-overhead", action="store_true",
                    help="time the torch op's host side on C2 (metadata + launch) next to its GPU step")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="target CPU baseline sample time")
    return ap.parse_args()


# The dominant kernel of each workload with the library's own partition
# choice, as rocprofv3 names it (template arguments: head_dim, softcap,
# slot-lookup mode).
DOMINANT_KERNEL = {
    "c2": "decode_stream_kernel<128, false, 0>",
    "c3": "decode_stream_kernel<128, false, 0>",
    "c5": "decode_stream_kernel<128, false, 0>",
    "c4": "prefill_kernel<128, false, 0>",
    "c4d256": "prefill_kernel<256, false, 0>",
}


def measured_traffic(workload, partition=0, root=ROOT):
    """HBM bytes per launch of the workload's dominant kernel, as last measured with
    rocprofv3 PMC (FETCH_SIZE x2 + WRITE_SIZE) and recorded with its command in
    profiles/<kernel>_<workload>_traffic.md. None when no measurement exists, when
    the file measured another kernel than the one this build launches (its
    `kernel:` line must name DOMINANT_KERNEL[workload]), or when the decode step
    did not run the balanced schedule (`partition`, the library's
    gk_paged_decode_partition_tokens for the benchmarked parameters, non-zero:
    the partitioned kernel ran instead of DOMINANT_KERNEL)."""
    if partition != 0 or workload not in DOMINANT_KERNEL:
        return None
    kernel = DOMINANT_KERNEL[workload]
    path = os.path.join(root, "profiles", f"{kernel.split('<')[0]}_{workload}_traffic.md")
    recorded, traffic = None, None
    try:
        with open(path) as fh:
            for line in fh:
                if line.startswith("kernel:"):
                    recorded = line.split(":", 1)[1].strip()
                elif line.startswith("traffic_bytes_per_launch:"):
                    traffic = int(line.split(":", 1)[1])
    except OSError:
        return None
    return traffic if recorded == kernel else None


def cpu_baseline(dc, target_seconds):
    """Time the C oracle's direct_bf16_pv (reference restatement) on a bounded sample of the batch."""
    import numpy as np

    from oracle import oracle as orc

    threads = orc.host_threads()
    query, pool = dc.host_arrays()
    context = int(dc.lens.max())
    mapping = orc.mapping_from_block_table(dc.tables, dc.block_size, context)

    def run(rows):
        p = orc.Problem(query[:rows], pool, np.arange(rows), dc.lens[:rows].astype(np.int64) - 1, mapping,
                        dc.heads, dc.kv_heads, dc.head_dim, dc.scale)
        t0 = time.perf_counter()
        orc.direct_bf16_pv(p, threads)
        return time.perf_counter() - t0

    probe_rows = min(dc.batch, threads)
    probe = run(probe_rows)
    full = probe * dc.batch / probe_rows  # estimated seconds for the whole batch
    rows = dc.batch
    reps = max(1, min(50, int(target_seconds / max(full, 1e-6))))
    if full > target_seconds:
        rows = max(probe_rows, min(dc.batch, int(probe_rows * target_seconds / max(probe, 1e-6))))
        reps = 1
    times = [run(rows) for _ in range(reps)]
    t = statistics.median(times)
    kv_tokens = int(dc.lens[:rows].astype(np.int64).sum())
    return {
        "value": rows / t,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"first {rows} of {dc.batch} sequences ({kv_tokens} KV tokens), direct_bf16_pv C oracle, "
                  f"median of {reps} run(s), {t:.3f} s each, {threads} threads on {host_cpu()}",
    }


def host_cpu():
    """CPU model and logical CPU count of the host, for the baseline's record."""
    model = "unknown CPU"
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count()
    omp = os.environ.get("OMP_NUM_THREADS")
    return (f"{model} ({os.cpu_count()} logical CPUs, {usable} in this process's affinity mask"
            + (f", OMP_NUM_THREADS={omp}" if omp else "") + ")")


def prefill_run(lib, steps, warmup, seed, workload="c4"):
    """A prefill workload (C4): one gk_paged_prefill call per step, timed with HIP
    events on the launch stream. Returns (ms per step, TFLOP/s, the case)."""
    import torch

    from gaudirt_amd import capi, workloads

    pc = workloads.DevicePrefillCase(seed=seed, **PREFILL_WORKLOADS[workload])
    stream = torch.cuda.current_stream()
    p = capi.PrefillParams()
    p.query, p.q_row_stride = pc.query.data_ptr(), pc.query.stride(0)
    p.pool, p.slots = pc.pool.data_ptr(), pc.slots
    p.block_tables, p.bt_stride, p.block_size = pc.d_tables.data_ptr(), pc.d_tables.stride(0), pc.block_size
    p.seq_request, p.seq_first_row = pc.seq_request.data_ptr(), pc.seq_first_row.data_ptr()
    p.seq_rows, p.seq_prefix = pc.seq_rows.data_ptr(), pc.seq_prefix.data_ptr()
    p.seqs, p.max_rows = pc.seqs, pc.chunk
    p.q_heads, p.kv_heads, p.head_dim = pc.heads, pc.kv_heads, pc.head_dim
    p.scale, p.softcap, p.sliding_window = pc.scale, 0.0, -1
    p.out, p.out_row_stride = pc.out.data_ptr(), pc.out.stride(0)
    hstream = ctypes.c_void_p(stream.cuda_stream)
    for _ in range(warmup):
        capi.check(lib.gk_paged_prefill(ctypes.byref(p), hstream))
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        capi.check(lib.gk_paged_prefill(ctypes.byref(p), hstream))
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    tflops = pc.flops() / (ms * 1e-3) / 1e12
    print(f"[bench] {workload}: {ms * 1e3:.1f} us/step, {tflops:.1f} TFLOP/s ({tflops / MFMA_BF16_PEAK_TFLOPS:.1%} of "
          f"{MFMA_BF16_PEAK_TFLOPS:.0f}), {pc.rows / (ms * 1e-3):.4g} query rows/s", file=sys.stderr, flush=True)
    return ms, tflops, pc


def prefill_roofline(tflops, workload="c4"):
    return {"bound": "mfma", "achieved": tflops, "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": tflops / MFMA_BF16_PEAK_TFLOPS, "traffic": measured_traffic(workload)}


def prefill_bench(args):
    """A prefill workload as the headline: its own JSON line (MFMA roofline, causal-exact FLOPs)."""
    from gaudirt_amd import capi

    w = args.workload
    ms, tflops, pc = prefill_run(capi.load(), args.steps, args.warmup, args.seed, w)
    print(json.dumps({
        "metric": "prefix-shared chunked prefill attention TFLOP/s (causal-exact), 1 MI355X",
        "value": tflops, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic", "config": {"workload": f"{w}: {WORKLOADS[w]}", "flops_per_step": pc.flops()},
        "roofline": prefill_roofline(tflops, w), "cpu_baseline": None}), flush=True)


def decode_run(lib, workload, steps, warmup, table_sets, seed, partition, page_size=0):
    """One gk_paged_decode call per step over the whole batch of a decode workload,
    timed with HIP events on the launch stream; consecutive steps rotate over
    `table_sets` disjoint block-table sets (re-paged to `page_size` tokens per
    page when given). Returns a dict of the timing and the case."""
    import torch

    from gaudirt_amd import capi, workloads

    dc = workloads.DeviceDecodeCase(workload, seed=seed, table_sets=table_sets)
    stream = torch.cuda.current_stream()
    hstream = ctypes.c_void_p(stream.cuda_stream)
    page = page_size or dc.block_size
    table_sets_dev = dc.d_table_sets
    if page != dc.block_size:
        table_sets_dev = [torch.from_numpy(workloads.repage_tables(t, dc.lens, dc.block_size, page)).cuda()
                          for t in dc.table_sets]

    params = []
    for i, tables in enumerate(table_sets_dev):
        p = capi.DecodeParams()
        p.query, p.q_row_stride = dc.query.data_ptr(), dc.query.stride(0)
        p.pool, p.slots = dc.pool.data_ptr(), dc.slots
        p.block_tables, p.bt_stride, p.block_size = tables.data_ptr(), tables.stride(0), page
        p.row_request, p.row_context, p.rows = None, dc.d_lens.data_ptr(), dc.batch
        p.q_heads, p.kv_heads, p.head_dim = dc.heads, dc.kv_heads, dc.head_dim
        p.scale, p.softcap, p.sliding_window = dc.scale, 0.0, -1
        p.max_context, p.partition_tokens = int(dc.lens.max()), partition
        p.out, p.out_row_stride = dc.out.data_ptr(), dc.out.stride(0)
        if dc.store:
            p.new_key, p.new_value = dc.new_key.data_ptr(), dc.new_value.data_ptr()
            p.new_kv_row_stride = dc.new_key.stride(0)
            p.slot_mapping = dc.d_slot_mappings[i].data_ptr()
        params.append(p)
    need = max(lib.gk_paged_decode_workspace_bytes(ctypes.byref(p)) for p in params)
    workspace = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    chosen = lib.gk_paged_decode_partition_tokens(ctypes.byref(params[0]))

    def step(i):
        capi.check(lib.gk_paged_decode(ctypes.byref(params[i % len(params)]),
                                       ctypes.c_void_p(workspace.data_ptr()), need, hstream))

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        step(i)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_per_step = start.elapsed_time(end) / steps
    del workspace

    step_bytes = dc.step_bytes(page)
    kv_bytes = dc.kv_bytes()
    seconds = ms_per_step * 1e-3
    achieved = step_bytes / seconds / 1e9
    tokens_per_s = dc.batch / seconds
    print(f"[bench] {workload}: {ms_per_step * 1e3:.1f} us/step, {tokens_per_s:.4g} tokens/s, "
          f"{achieved:.1f} GB/s ({achieved / HBM_PEAK_GBPS:.1%} of peak), KV {kv_bytes / 1e9:.4f} GB/step, "
          f"partition {chosen}, wall {wall:.2f} s", file=sys.stderr, flush=True)
    return {
        "case": dc,
        "ms_per_step": ms_per_step,
        "tokens_per_s": tokens_per_s,
        "partition": int(chosen),
        "page_size": page,
        "table_sets": len(params),
        "kv_read_gbps": kv_bytes / seconds / 1e9,
        "roofline": {
            "bound": "hbm",
            "achieved": achieved,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBPS,
            # the recorded counters are for the workload's own block size (another
            # page size runs another variant of the kernel)
            "traffic": measured_traffic(workload, int(chosen)) if page == dc.block_size else None,
        },
    }


def secondary_runs(args):
    """C3, C5 (HBM roofline) and C4 (MFMA roofline) after the headline, each timed
    over `args.steps` steps by a child `bench.py --workload <w>` process whose JSON
    line is read back. A decode case set up in a process that had already
    allocated and released multi-GiB pools ran about 4% slower (the second of
    C3 / C5 in one process: C5 210.6 vs 202.4 us, C3 194.9 vs 187.8), so each
    case gets a process of its own, as a server allocates its pool once."""
    import subprocess

    out = {}
    for workload in ("c3", "c5", "c4"):
        # The first calls of a new case page in its pool and tables; C4's
        # MFMA-bound kernel also needs the clocks up.
        warmup = C4_WARMUP if workload == "c4" else max(args.warmup, 100)
        cmd = [sys.executable, "-u", os.path.abspath(__file__), "--workload", workload, "--no-cpu", "--no-secondary",
               "--steps", str(args.steps), "--warmup", str(warmup), "--seed", str(args.seed),
               "--table-sets", str(args.table_sets)]
        try:
            proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=900)
        except subprocess.TimeoutExpired:
            out[workload] = {"error": "timed out after 900 s"}
            continue
        sys.stderr.write(proc.stderr)
        sys.stderr.flush()
        if proc.returncode != 0 or not proc.stdout.strip():
            # The headline stands on its own: a failed leg is reported, not raised.
            out[workload] = {"error": f"exited with status {proc.returncode}"}
            continue
        line = json.loads(proc.stdout.strip().splitlines()[-1])
        entry = {"workload": line["config"]["workload"], "value": line["value"], "unit": line["unit"],
                 "ms_per_step": line["ms_per_step"], "steps": line["steps"], "warmup": line["warmup"]}
        if workload == "c4":
            entry["flops_per_step"] = line["config"]["flops_per_step"]
        else:
            entry.update(split_k_partition=line["config"]["split_k_partition"],
                         mean_context=line["config"]["mean_context"], max_context=line["config"]["max_context"])
        entry["roofline"] = line["roofline"]
        out[workload] = entry
    return out


def host_overhead(args):
    """Host and GPU time per decode step of torch.ops.gaudirt.paged_attn on C2."""
    import numpy as np
    import torch

    import gaudirt_amd
    from gaudirt_amd import workloads

    gaudirt_amd.load_extension()
    dc = workloads.DeviceDecodeCase("c2", seed=args.seed)
    rows, context, block = dc.batch, int(dc.lens.max()), dc.block_size
    # The token-granular request map of C2's block tables (-1 past each row's length).
    t = np.arange(context)
    mapping = np.where(t[None, :] < dc.lens[:, None],
                       dc.tables[:, np.minimum(t // block, dc.tables.shape[1] - 1)] * block + t % block, -1)
    mapping = np.ascontiguousarray(mapping.astype(np.int32))
    positions = dc.lens.astype(np.int64) - 1
    locations = mapping[np.arange(rows), positions].astype(np.int64)
    cpu = {"locations": torch.from_numpy(locations), "requests": torch.arange(rows, dtype=torch.int64),
           "positions": torch.from_numpy(positions), "mapping": torch.from_numpy(mapping)}
    dev = {k: v.cuda() for k, v in cpu.items()}
    prefixes, lengths = positions.tolist(), [1] * rows
    gen = torch.Generator(device="cuda")
    gen.manual_seed(args.seed)
    k = torch.randn((rows, dc.kv_heads * dc.head_dim), generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn((rows, dc.kv_heads * dc.head_dim), generator=gen, device="cuda").to(torch.bfloat16)
    key_pool, value_pool = dc.pool[0].transpose(0, 1), dc.pool[1].transpose(0, 1)
    op = torch.ops.gaudirt.paged_attn.default
    cls = torch.classes.gaudirt.PagedMetadata

    def host_ctor():
        m = cls(cpu["locations"], cpu["requests"], cpu["positions"], cpu["mapping"], dc.slots)
        return op(dc.query, k, v, key_pool, value_pool, m, dc.head_dim, dc.scale)

    def scheduler():
        m = cls._from_scheduler(dev["locations"], dev["requests"], dev["positions"], dev["mapping"], prefixes,
                                lengths, dc.slots, None, 0)
        return op(dc.query, k, v, key_pool, value_pool, m, dc.head_dim, dc.scale)

    def reused(meta):
        return lambda: op(dc.query, k, v, key_pool, value_pool, meta, dc.head_dim, dc.scale)

    stream = torch.cuda.current_stream()
    result = {}
    prebuilt = cls(cpu["locations"], cpu["requests"], cpu["positions"], cpu["mapping"], dc.slots)
    for name, fn in (("host_constructor", host_ctor), ("from_scheduler", scheduler),
                     ("metadata_reused", reused(prebuilt))):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        host = []
        start.record(stream)
        for _ in range(args.steps):
            t0 = time.perf_counter()
            fn()
            host.append(time.perf_counter() - t0)
        end.record(stream)
        torch.cuda.synchronize()
        wall_ms = start.elapsed_time(end) / args.steps
        result[name] = {"host_us_median": statistics.median(host) * 1e6,
                        "host_us_mean": statistics.fmean(host) * 1e6,
                        "stream_us_per_step": wall_ms * 1e3}
        print(f"[bench] host overhead {name}: host {result[name]['host_us_median']:.1f} us/step (median), "
              f"stream {wall_ms * 1e3:.1f} us/step", file=sys.stderr, flush=True)
    # The GPU time of one step alone: each step timed between its own events after a sync.
    gpu = []
    for _ in range(20):
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        reused(prebuilt)()
        end.record(stream)
        torch.cuda.synchronize()
        gpu.append(start.elapsed_time(end) * 1e3)
    result["gpu_step_us_median"] = statistics.median(gpu)
    print(f"[bench] host overhead: GPU step alone {result['gpu_step_us_median']:.1f} us", file=sys.stderr,
          flush=True)
    print(json.dumps({"metric": "paged_attn host overhead per decode step (c2), 1 MI355X", "unit": "us",
                      "steps": args.steps, "warmup": args.warmup, "rows": rows, "context": context,
                      "token_granular_map": True, **result}), flush=True)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the decode path does not shard across GPUs here", file=sys.stderr)
        sys.exit(2)
    if args.warmup is None:
        args.warmup = C4_WARMUP if args.workload in PREFILL_WORKLOADS else 20

    import torch

    assert torch.cuda.is_available(), "bench.py needs an MI355X"
    torch.cuda.set_device(0)
    if args.host_overhead:
        return host_overhead(args)
    if args.workload in PREFILL_WORKLOADS:
        return prefill_bench(args)

    from gaudirt_amd import capi

    lib = capi.load()
    r = decode_run(lib, args.workload, args.steps, args.warmup, args.table_sets, args.seed, args.partition,
                   args.page_size)
    dc = r["case"]
    # The GPU legs run back to back; the CPU baseline (about a second of host
    # work with the GPU idle) comes last.
    secondary = None
    if args.workload == "c2" and not args.no_secondary:
        secondary = secondary_runs(args)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(dc, args.cpu_seconds)
        print(f"[bench] cpu baseline: {cpu}", file=sys.stderr, flush=True)

    line = {
        "metric": METRIC,
        "value": r["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": r["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"{args.workload}: {WORKLOADS[args.workload]}",
            "batch": dc.batch,
            "q_heads": dc.heads,
            "kv_heads": dc.kv_heads,
            "head_dim": dc.head_dim,
            "block_size": r["page_size"],
            "mean_context": float(dc.lens.mean()),
            "max_context": int(dc.lens.max()),
            "split_k_partition": r["partition"],
            "table_sets": r["table_sets"],
            "seed": args.seed,
            "kv_read_gbps": r["kv_read_gbps"],
        },
        "roofline": r["roofline"],
        "cpu_baseline": cpu,
    }
    if secondary is not None:
        line["secondary"] = secondary
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
