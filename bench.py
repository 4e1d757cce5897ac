"""Decode-step benchmark of the MI355X KV-cache hot path.

Workload (the north-star shape): Llama-3-8B KV
geometry (32 layers, 32 query / 8 KV heads, head_dim 128), f16 paged KV with
32-token pages, batch 64, every sequence at context 8192.  One step = the
decode step of the reference generator for every layer: append one token per
sequence (K/V rows fp32 -> f16 into the paged pool) and split-K GQA attention
over the 8193 cached tokens.  Pages are placed by a seeded random permutation
of the pool (installed through the actor's free stack); cache contents are
synthetic N(0,1) f16 written straight into the pool (the append kernel writes
the step's new token); Q is N(0,1)/sqrt(128), the kernel scale 1/sqrt(128)
(the reference always applies 1/sqrt(head_dim), detail.hpp:3163).

Each timed step re-appends at position 8192 and attends over 8193 tokens, so
every step does identical work.  `value` is KV-read GB/s: K+V bytes the
attention must read per step / step time.  The roofline object covers the
dominant kernel (split-K decode attention), timed with HIP events on the
stream it runs on.  The CPU baseline is the oracle's restatement of the
reference's paged decode route, timed on this host on a bounded sample.

With no --config, the same run also measures the other BASELINE configs
under the same clock and reports them in a "configs" object of the one JSON
line: config 4 (q8_0 decode, B=32, ctx 16k), config 5 (chunked prefill on
MFMA + eviction/compaction, f16 and q8_0 pools), config 2 (Llama-3.2-1B
ragged decode) and config 1 (Qwen3-0.6B contiguous decode), each with its
roofline, a parity sample and a bounded CPU baseline.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "emel.cpp_amd"))

HBM_PEAK_GBS = 8000.0

# HBM bytes per launch of the measured kernels (decode_kernel + combine_kernel
# per layer for decode, prefill_kernel per layer for the chunked prefill),
# from the two rocprofv3 PMC runs (FETCH_SIZE, WRITE_SIZE) summarised in the
# profiles/ file of each workload, each scaled by the same counter's reading
# on a plain 1 GiB copy (bench.py --copy-calibration): FETCH_SIZE x2.000,
# WRITE_SIZE x1.000.
PMC_TRAFFIC_BYTES = {  # workload -> bytes; source: profiles/<kernel>_<workload>.md
    "llama3-8b-b64-ctx8k": 2157021798,
    "llama3-8b-q8_0-b32-ctx16k": 1150230950,
    "llama3-8b-prefill512-evict25": 287648388,
    "llama3-8b-q8_0-prefill512-evict25": 292694400,
    "llama3.2-1b-b16-ctx1k-4k": 96741730,
    "qwen3-0.6b-b1-ctx512": 2627852,
    "gemma4-d256-prefill512-evict25": 105300848,
    "gemma4-d256-q8_0-prefill512-evict25": 87734776,
    "gemma4-d512-prefill512-evict25": 285765904,
}

CONFIGS = {
    # name: (n_layer, n_head, n_kv, head_dim, block_tokens, batch, ctx, kv_type)
    "llama3-8b-b64-ctx8k": (32, 32, 8, 128, 32, 64, 8192, "f16"),
    "llama3-8b-q8_0-b32-ctx16k": (32, 32, 8, 128, 32, 32, 16384, "q8_0"),
    "llama3.2-1b-b16-ctx1k-4k": (16, 32, 8, 64, 16, 16, None, "f16"),
    "qwen3-0.6b-b1-ctx512": (28, 16, 8, 128, 16, 1, 512, "f16"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default=None,
                    choices=sorted(CONFIGS) + ["llama3-8b-prefill512-evict25",
                                               "llama3-8b-q8_0-prefill512-evict25",
                                               "gemma4-d256-prefill512-evict25",
                                               "gemma4-d256-q8_0-prefill512-evict25",
                                               "gemma4-d512-prefill512-evict25",
                                               "llama3-8b-b64-ctx8k-generator"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--headline-only", action="store_true",
                    help="with no --config: measure config 3 only (no 'configs' object)")
    ap.add_argument("--cpu-budget", type=float, default=10.0,
                    help="seconds of CPU-baseline work for the headline config")
    ap.add_argument("--kernel-split", action="store_true",
                    help="decode configs: add per-kernel durations of one eager step from "
                         "torch.profiler (a diagnostic, not the roofline basis)")
    ap.add_argument("--no-kernel-split", action="store_true",
                    help="accepted for older command lines; the split is off by default")
    ap.add_argument("--separate-append", action="store_true",
                    help="append with emelk_kv_append, then emelk_attn_decode (two launches per "
                         "layer) instead of emelk_attn_decode_append")
    ap.add_argument("--cpu-threads", type=int, default=0)
    ap.add_argument("--seed", type=int, default=1234)
    ap.add_argument("--no-prime", action="store_true",
                    help="start each event-timed block right after the spin kernel, "
                         "without an untimed block first")
    ap.add_argument("--eager", action="store_true",
                    help="time the step as eager launches instead of one replayed HIP graph")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only copy 1 GiB device-to-device three times (the reference kernel "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings)")
    ap.add_argument("--launch-floor", type=int, default=0, metavar="N",
                    help="only time a replayed HIP graph of N back-to-back one-element kernels "
                         "(the launch floor of a step of N dependent launches)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU only: the KV hot path shards by "
                          "sequence with no exchange between GPUs; run with --gpus 1"}))
        sys.exit(2)

    import torch

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        a = torch.ones(1 << 30, dtype=torch.uint8, device=dev)
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": 1 << 30, "copies": 3}))
        return
    if args.launch_floor > 0:
        # each launch depends on the one before (same stream), as the
        # decode + combine launches of a step do
        x = torch.zeros(1, dtype=torch.float32, device=dev)
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for _ in range(args.launch_floor):
                    x.add_(1.0)
        torch.cuda.current_stream().wait_stream(side)
        for _ in range(max(1, args.warmup)):
            graph.replay()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            graph.replay()
        torch.cuda.synchronize()
        ms = 1e3 * (time.perf_counter() - t0) / args.steps
        print(json.dumps({"launch_floor_launches": args.launch_floor, "ms_per_graph": round(ms, 4),
                          "us_per_launch": round(1e3 * ms / args.launch_floor, 3),
                          "steps": args.steps}))
        return
    import emelk

    if args.config is None:
        args.config = "llama3-8b-b64-ctx8k"
        # the sub-configs first, each in a child process, before this
        # process allocates anything; then the headline here
        configs = None if args.headline_only else other_configs(args, torch)
        result = run_config(args, torch, emelk, dev)
        if configs is not None:
            result["configs"] = configs
    else:
        result = run_config(args, torch, emelk, dev)
    if TIMING_NOTES:
        result["timing_notes"] = sorted(TIMING_NOTES)
    print(json.dumps(result), flush=True)
    bad = parity_failures(result)
    if bad:
        log(f"[bench] PARITY FAILED at {bad}")
        sys.exit(3)
    failed = [k for k, v in result.get("configs", {}).items() if "error" in v]
    if failed:
        log(f"[bench] sub-configs failed: {failed}")
        sys.exit(4)


PREFILL_CONFIGS = ("llama3-8b-prefill512-evict25", "llama3-8b-q8_0-prefill512-evict25",
                   "gemma4-d256-prefill512-evict25", "gemma4-d256-q8_0-prefill512-evict25",
                   "gemma4-d512-prefill512-evict25")

# The other BASELINE configs in the default run: (label, workload, steps, warmup)
SUB_CONFIGS = [
    ("config4_q8_0_decode", "llama3-8b-q8_0-b32-ctx16k", 10, 2),
    ("config5_prefill_evict_f16", "llama3-8b-prefill512-evict25", 3, 1),
    ("config5_prefill_evict_q8_0", "llama3-8b-q8_0-prefill512-evict25", 3, 1),
    ("config2_llama1b_ragged", "llama3.2-1b-b16-ctx1k-4k", 20, 3),
    ("config1_qwen3_contiguous", "qwen3-0.6b-b1-ctx512", 20, 3),
]
SUB_KEYS = ("metric", "value", "unit", "ms_per_step", "steps", "warmup", "steps_per_s",
            "step_launch", "dtype", "kv_type", "config", "roofline", "kernel_split",
            "cpu_baseline", "parity_full_size", "parity_sample", "compaction")


def other_configs(args, torch):
    """Each sub-config in a child process of its own (`bench.py --config`),
    so every line is measured as a standalone run: inside one process a
    workload whose pools are allocated after another workload's pools were
    freed ran about 5% slower (config 4: frac 0.737 first, 0.703 after
    config 3; config 3: 0.825 first, 0.770 after config 4), and a child
    started while the parent held freed pools of config 3 still lost it
    (0.706); processes that start after the previous one has exited show
    no order effect.  So the children run first, while this process has
    allocated nothing."""
    import subprocess
    out = {}
    for label, workload, steps, warmup in SUB_CONFIGS:
        cmd = [sys.executable, os.path.abspath(__file__), "--config", workload, "--steps",
               str(steps), "--warmup", str(warmup), "--cpu-budget", "3.0", "--seed", str(args.seed)]
        for flag in ("no_cpu_baseline", "no_prime", "eager", "separate_append", "kernel_split"):
            if getattr(args, flag):
                cmd.append("--" + flag.replace("_", "-"))
        if args.cpu_threads:
            cmd += ["--cpu-threads", str(args.cpu_threads)]
        log(f"[bench] sub-config {label} ({workload}) in a child process")
        res = subprocess.run(cmd, stdout=subprocess.PIPE, text=True, timeout=900)
        lines = [ln for ln in res.stdout.splitlines() if ln.startswith("{")]
        if res.returncode not in (0, 3) or not lines:
            out[label] = {"error": f"child exited with {res.returncode}"}
            continue
        r = json.loads(lines[-1])
        out[label] = {k: r[k] for k in SUB_KEYS if k in r}
        out[label]["process"] = "child (fresh GPU context and allocator)"
    return out


TIMING_NOTES = set()


def gpu_head_start(torch, cycles=40_000_000):
    """Queue a spin kernel (tens of ms) ahead of an event-timed block, so the
    host has enqueued the block's launches before the GPU reaches them: each
    event interval then holds GPU time only, never host launch overhead.
    False when this torch build has no spin kernel."""
    sleep = getattr(torch.cuda, "_sleep", None)
    if sleep is None:
        return False
    sleep(cycles)
    return True


def timed_blocks(torch, stream, launch, reps, prime=None):
    """HIP event time (ms) of `launch()` (a block of back-to-back calls on
    `stream`), `reps` times.  Each block is queued behind a spin kernel; a
    block whose launches were not all queued before the GPU reached its
    start event (the host stalled, e.g. freeing a large array) may hold host
    gaps and is measured again.  Without a spin kernel every interval is
    kept and the line says that they may hold host gaps.  `prime()`, queued
    between the spin and the start event, runs untimed work first, so the
    timed block does not start on a GPU that has just idled in the spin (its
    clocks ramp back up)."""
    times, tries = [], 0
    while len(times) < reps and tries < 4 * reps:
        tries += 1
        spun = gpu_head_start(torch)
        if prime is not None:
            prime()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        launch()
        e1.record(stream)
        ahead = not e0.query()  # the GPU was still spinning when the last call was queued
        torch.cuda.synchronize()
        if not spun:
            TIMING_NOTES.add("no spin kernel in this torch build: event intervals may hold "
                             "host launch gaps")
        if ahead or not spun:
            times.append(e0.elapsed_time(e1))
    if not times:
        raise RuntimeError("could not queue a timed block ahead of the GPU")
    return times


def graph_event_ms(torch, graph, stream, reps):
    """(HIP event ms, host ms) per replay of a captured graph, replayed
    `reps` times back to back: one event pair on `stream` around the
    replays (no host gap can fall between the graph's kernels), and the host
    clock around the same replays with a synchronisation on either side, so
    the event figure never exceeds the host one."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        e0.record(stream)
        for _ in range(reps):
            graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    host = 1e3 * (time.perf_counter() - t0) / reps
    return e0.elapsed_time(e1) / reps, host


def parity_failures(obj, path=""):
    """Paths of every `within_tolerance: false` in a result."""
    bad = []
    if isinstance(obj, dict):
        for k, v in obj.items():
            if k == "within_tolerance" and v is False:
                bad.append(path or "/")
            else:
                bad += parity_failures(v, f"{path}/{k}")
    elif isinstance(obj, list):
        for i, v in enumerate(obj):
            bad += parity_failures(v, f"{path}/{i}")
    return bad


def baseline_threads(args, lanes):
    """One thread per sequence lane (or per row lane of a chunk), up to the
    host threads this process may use and the box's share of 16."""
    if args.cpu_threads:
        return args.cpu_threads
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count() or 1
    return max(1, min(lanes, usable, 16))


def cpu_info(threads):
    """Provenance of a CPU-baseline figure: the threads used and the host."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = None
    return {"cores": threads, "cpu_model": model, "nproc": os.cpu_count(),
            "usable_cpus": usable}


def kernel_split(args, torch, fn, names):
    """Average device time per launch (ms) of each named kernel over one
    eager call of fn, from torch.profiler's device trace (outside the timed
    region).  Lets the line report the dominant kernel apart from its
    helpers (e.g. decode_kernel vs combine_kernel)."""
    if args.no_kernel_split or not args.kernel_split:
        return None
    try:
        from torch.profiler import ProfilerActivity, profile
        torch.cuda.synchronize()
        with profile(activities=[ProfilerActivity.CUDA]) as prof:
            fn()
            torch.cuda.synchronize()
        res = {}
        for ev in prof.key_averages():
            for n in names:
                if n + "<" in ev.key or ev.key.endswith(n):
                    total = getattr(ev, "device_time_total", None)
                    if total is None:
                        total = getattr(ev, "cuda_time_total", 0.0)
                    r = res.setdefault(n, {"launches": 0, "total_us": 0.0})
                    r["launches"] += int(ev.count)
                    r["total_us"] += float(total)
        return {n: {"launches": r["launches"],
                    "avg_ms": round(r["total_us"] / max(1, r["launches"]) / 1e3, 5)}
                for n, r in res.items()} or None
    except Exception as e:  # the profiler is a reporting aid, never a gate
        log(f"[bench] kernel split unavailable: {e!r}")
        return None


def run_config(args, torch, emelk, dev):
    if args.config in PREFILL_CONFIGS:
        return prefill_evict(args, torch, emelk, dev)
    if args.config == "llama3-8b-b64-ctx8k-generator":
        return generator(args, torch, emelk, dev)
    return decode_run(args, torch, emelk, dev)


def decode_run(args, torch, emelk, dev):
    L, H, HK, D, BT, B, CTX, kvt = CONFIGS[args.config]
    kv_type = emelk.KV_F16 if kvt == "f16" else emelk.KV_Q8_0
    rng = np.random.default_rng(args.seed)
    if CTX is None:
        ctx = rng.integers(1024, 4097, size=B).astype(np.int64)
    else:
        ctx = np.full(B, CTX, dtype=np.int64)
    lens = ctx + 1  # tokens attended after the step's append
    pages_per_seq = -(-lens // BT)
    max_blocks = int(pages_per_seq.sum()) + 1
    assert max_blocks <= emelk.MAX_BLOCKS

    # ---- block map through the actor (seeded page permutation) ----
    actor = emelk.KvActor()
    ok, err = actor.reserve(B, max_blocks, BT)
    assert ok, err
    # config 1 is a contiguous cache: the actor's own ascending pops give the
    # one sequence the identity page map (the reference's flash route);
    # every other config places its pages by a seeded permutation
    contiguous = args.config == "qwen3-0.6b-b1-ctx512"
    if not contiguous:
        actor.set_free_order(rng.permutation(max_blocks).astype(np.uint16))
    for s in range(B):
        assert actor.allocate_sequence(s)[0]
        assert actor.allocate_slots(s, int(ctx[s]))[0]
    for s in range(B):
        ok, err, _ = actor.allocate_slots(s, 1)  # the decode step's slot
        assert ok, err
    stride = int(pages_per_seq.max()) + 1
    tables_h = actor.export_block_tables(list(range(B)), stride)
    tables = torch.from_numpy(tables_h.view(np.int16)).to(dev)

    g = emelk.geometry(L, H, HK, D, BT, max_blocks, kv_type)
    pool_bytes = emelk.pool_bytes(g)
    log(f"[bench] config={args.config} pools 2 x {pool_bytes / 1e9:.2f} GB, "
        f"pages={max_blocks}")
    k_pool = torch.empty(pool_bytes, dtype=torch.uint8, device=dev)
    v_pool = torch.empty(pool_bytes, dtype=torch.uint8, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    chunk = 1 << 30
    t0 = time.time()
    for pool in (k_pool, v_pool):
        if kv_type == emelk.KV_F16:
            h = pool.view(torch.float16)
            for i in range(0, h.numel(), chunk):
                n = min(chunk, h.numel() - i)
                h[i:i + n].normal_(generator=gen)
        else:
            # q8_0 pages are written by quantizing N(0,1) rows (1% x20
            # outliers) with the append kernel, one layer and page range at
            # a time.
            pass
    if kv_type == emelk.KV_Q8_0:
        for layer in range(L):
            for s0 in range(0, B, 8):
                s1 = min(B, s0 + 8)
                n = int(ctx.max())
                kr = torch.randn((s1 - s0, n, HK * D), generator=gen, device=dev)
                vr = torch.randn((s1 - s0, n, HK * D), generator=gen, device=dev)
                for t in (kr, vr):
                    m = torch.rand(t.shape, generator=gen, device=dev) < 0.01
                    t[m] *= 20.0
                pos = torch.zeros(s1 - s0, dtype=torch.int32, device=dev)
                emelk.append(g, k_pool, v_pool, layer, kr, vr, pos, tables[s0:s1])
                del kr, vr
    torch.cuda.synchronize()
    log(f"[bench] pools filled in {time.time() - t0:.1f}s")

    q = [(torch.randn((B, H, D), generator=gen, device=dev) / np.sqrt(D)).contiguous()
         for _ in range(L)]
    new_k = [torch.randn((B, 1, HK * D), generator=gen, device=dev) for _ in range(L)]
    new_v = [torch.randn((B, 1, HK * D), generator=gen, device=dev) for _ in range(L)]
    out = [torch.empty((B, H, D), dtype=torch.float32, device=dev) for _ in range(L)]
    positions = torch.from_numpy(ctx.astype(np.int32)).to(dev)
    kv_lens = torch.from_numpy(lens.astype(np.int32)).to(dev)
    max_len = int(lens.max())
    ws = torch.empty(emelk.decode_workspace_bytes(g, B, max_len) // 4 + 1, dtype=torch.float32,
                     device=dev)
    scale = float(1.0 / np.sqrt(D))
    stream = torch.cuda.current_stream()

    new_k2 = [t.view(B, HK * D) for t in new_k]
    new_v2 = [t.view(B, HK * D) for t in new_v]
    if contiguous:
        # the one sequence sits on pages 0.. of every region: the flash
        # route's contiguous cache, attended without a block table
        seq_stride = int(pages_per_seq.max()) * BT
        assert np.array_equal(tables_h[0, :pages_per_seq[0]], np.arange(pages_per_seq[0]))

    def attend(layer, store):
        """The step's attention for one layer; store: the new token is
        written in the same launch."""
        if contiguous:
            emelk.decode_contiguous(g, k_pool, v_pool, layer, q[layer], out[layer], kv_lens,
                                    max_len, seq_stride, scale, ws,
                                    k_rows=new_k2[layer] if store else None,
                                    v_rows=new_v2[layer] if store else None)
        elif store:
            emelk.decode_append(g, k_pool, v_pool, layer, new_k2[layer], new_v2[layer],
                                q[layer], out[layer], kv_lens, max_len, tables, scale, ws)
        else:
            emelk.decode(g, k_pool, v_pool, layer, q[layer], out[layer], kv_lens, max_len,
                         tables, scale, ws)

    def step():
        for layer in range(L):
            if args.separate_append:
                emelk.append(g, k_pool, v_pool, layer, new_k[layer], new_v[layer], positions,
                             tables)
                attend(layer, False)
            else:  # the step's store of the new token and its attention in one launch
                attend(layer, True)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # eager step time (host launch path included)
    K = args.steps
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for k in range(K):
        step()
    torch.cuda.synchronize()
    eager_ms = 1e3 * (time.perf_counter() - t_start) / K
    # Step timing: the L-layer step captured once as a HIP graph and replayed
    # K times, as a serving loop would run it (host clock for ms_per_step).
    # Kernel timing (roofline): one HIP event pair on the replay stream
    # around K more back-to-back replays, per layer call: decode (with the
    # fused store) + combine, nothing else in the graph, no host gap.
    graph_ms = None
    attn_avg_ms = None
    if not args.eager:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                step()
        torch.cuda.current_stream().wait_stream(side)
        for _ in range(args.warmup):
            graph.replay()
        ev_ms, graph_ms = graph_event_ms(torch, graph, side, K)
        if not args.separate_append:
            attn_avg_ms = ev_ms / L
    if attn_avg_ms is None:
        # eager or --separate-append: one HIP event pair around the L
        # back-to-back decode calls of a step after a GPU head start (the
        # appends of --separate-append left out: their rows are stored)
        def decode_block():
            for layer in range(L):
                attend(layer, not args.separate_append)

        attn_avg_ms = float(np.mean(timed_blocks(
            torch, stream, decode_block, K,
            prime=None if args.no_prime else decode_block))) / L
    timing_basis = ("HIP events around K replays of the step's graph, per layer call"
                    if graph_ms is not None and not args.separate_append else
                    "HIP events around the L eager decode calls of a step after a GPU head "
                    "start, per call")
    ms_per_step = graph_ms if graph_ms is not None else eager_ms

    # ---- algorithmic bytes ----
    if kv_type == emelk.KV_F16:
        row_bytes = HK * D * 2
    else:
        row_bytes = HK * (D + D // 32 * 2)
    kv_read_layer = int(lens.sum()) * row_bytes * 2          # K and V rows attended
    q_bytes = B * H * D * 4
    o_bytes = B * H * D * 4
    table_bytes = 0 if contiguous else int(pages_per_seq.sum()) * 2  # contiguous: no table
    append_bytes = B * HK * D * 4 * 2 + B * row_bytes * 2
    step_kv_bytes = kv_read_layer * L
    step_bytes = (kv_read_layer + q_bytes + o_bytes + table_bytes + append_bytes) * L
    kernel_bytes = kv_read_layer + q_bytes + o_bytes + table_bytes
    if not args.separate_append:  # the decode launch also stores the new token
        kernel_bytes += append_bytes
    kv_gbs = step_kv_bytes / (ms_per_step * 1e-3) / 1e9
    achieved = kernel_bytes / (attn_avg_ms * 1e-3) / 1e9

    split = kernel_split(args, torch, step, ["decode_kernel", "combine_kernel", "append_f16_kernel",
                                             "append_q8_0_kernel"])

    # ---- full-size parity check + CPU baseline (oracle built -O3
    # -march=native on this host) ----
    parity = None
    cpu = None
    if not args.no_cpu_baseline and contiguous:
        # the reference's route for an identity map: the flash decode with an
        # f16 accumulator (kernel/detail.hpp:5238-5291), one thread, every layer
        import oracle
        nlib, build = oracle.native_lib()
        lb = pool_bytes // L
        worst, within, secs = 0.0, True, 0.0
        n = int(lens[0])
        for layer in range(L):
            heads = []
            for p_ in (k_pool, v_pool):
                h = p_[layer * lb:(layer + 1) * lb].cpu().numpy().view(np.uint16)
                # pool [page][kv_head][t][D] -> head-major [kv_head][token][D]
                h = h.reshape(max_blocks, HK, BT, D).transpose(1, 0, 2, 3).reshape(HK, -1, D)
                heads.append(np.ascontiguousarray(h[:, :n]))
            qh = q[layer].view(B, H * D).cpu().numpy()
            t1 = time.perf_counter()
            want = oracle.flash_attn_f16acc(qh[0], heads[0], heads[1], D, H, HK, n, n, scale,
                                            lib_=nlib)
            secs += time.perf_counter() - t1
            got = out[layer].view(B, H * D).cpu().numpy()[0]
            err = np.abs(got.astype(np.float64) - want)
            worst = max(worst, float(err.max()))
            within = within and bool(np.all(err <= 2e-3 + 1e-2 * np.abs(want)))
        parity = {"layers": L, "sequences": B, "route": "flash, f16 accumulator",
                  "max_abs_err": worst, "within_tolerance": within}
        cpu_step_s = secs
        cpu = {"value": round(step_kv_bytes / cpu_step_s / 1e9, 4), "unit": "GB/s",
               **cpu_info(1), "kind": "port", "build": build,
               "sample": f"all {L} layers of the step ({secs:.3f}s); oracle restatement of the "
                         "flash route with an f16 accumulator, 1 thread (one sequence lane)",
               "steps_per_s": round(1.0 / cpu_step_s, 4)}
    elif not args.no_cpu_baseline:
        # the reference route (compute_attention; the oracle's q8_0 route for
        # q8_0 pools) over every sequence of whole layers, one thread per
        # sequence lane, layer after layer until the CPU budget is spent;
        # every layer's GPU output of the last step is checked
        import oracle
        nlib, build = oracle.native_lib()
        nthreads = baseline_threads(args, B)
        kind = "f16" if kv_type == emelk.KV_F16 else "q8_0"
        worst, within, secs, layers_done = 0.0, True, 0.0, 0
        for layer in range(L):
            kc, vc = (pool_token_major(p_, layer, L, max_blocks, HK, BT, D,
                                       kv_type == emelk.KV_Q8_0, oracle)
                      for p_ in (k_pool, v_pool))
            qh = q[layer].view(B, H * D).cpu().numpy()
            want, t_layer = oracle.attention_rows(kind, qh, kc, vc, tables_h, lens, BT, H, HK, D,
                                                  scale, nthreads, n_ctx=int(lens.max()),
                                                  lib_=nlib)
            del kc, vc
            got = out[layer].view(B, H * D).cpu().numpy()
            err = np.abs(got.astype(np.float64) - want)
            worst = max(worst, float(err.max()))
            within = within and bool(np.all(err <= 2e-3 + 1e-2 * np.abs(want)))
            secs += t_layer
            layers_done += 1
            if secs >= args.cpu_budget:
                break
        parity = {"layers": layers_done, "sequences": B, "max_abs_err": worst,
                  "within_tolerance": within}
        cpu_step_s = secs / layers_done * L  # sample = whole layers; scaled to L layers
        cpu = {"value": round(step_kv_bytes / cpu_step_s / 1e9, 4), "unit": "GB/s",
               **cpu_info(nthreads), "kind": "port", "build": build,
               "sample": f"{layers_done} layer(s) x {B} sequences of the same step "
                         f"({secs:.2f}s wall), scaled to {L} layers; oracle restatement of "
                         f"compute_attention ({kind} route), one thread per sequence lane, "
                         f"{nthreads} threads",
               "steps_per_s": round(1.0 / cpu_step_s, 6)}

    metric = ("KV-read HBM GB/s (% of peak) + decode steps/s, 8B-shape b64 ctx8k"
              if args.config == "llama3-8b-b64-ctx8k" else
              f"KV-read HBM GB/s (% of peak) + decode steps/s, {args.config}")
    traffic = None if args.separate_append else PMC_TRAFFIC_BYTES.get(args.config)
    result = {
        "metric": metric,
        "value": round(kv_gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "steps_per_s": round(1e3 / ms_per_step, 3),
        "step_launch": "hip graph replay" if graph_ms is not None else "eager",
        "eager_ms_per_step": round(eager_ms, 4),
        "pct_of_hbm_peak": round(100.0 * kv_gbs / HBM_PEAK_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if kv_type == emelk.KV_F16 else "q8_0",
        "data": "synthetic (seeded N(0,1) K/V/Q, seeded random page permutation)",
        "config": {"workload": args.config, "n_layer": L, "n_head": H, "n_head_kv": HK,
                   "head_dim": D, "block_tokens": BT, "batch": B,
                   "ctx": int(ctx[0]) if CTX else "U[1024,4096]", "kv": kvt,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic,
                     "traffic_source": (f"profiles/decode_kernel_{args.config}.md (rocprofv3 "
                                        "--pmc FETCH_SIZE / WRITE_SIZE of an earlier run of this "
                                        "workload, copy-calibrated)") if traffic else None,
                     "kernel": (("decode_kernel + combine_kernel"
                                 if args.separate_append else
                                 "decode_kernel with the fused append + combine_kernel") +
                                (", emelk_attn_decode_contiguous (no block table)"
                                 if contiguous else "")),
                     "bytes_per_launch": kernel_bytes, "avg_launch_ms": round(attn_avg_ms, 4),
                     "timing": timing_basis},
        "kernel_split": ({"source": "torch.profiler device trace of one eager step "
                                    "(diagnostic; not the roofline basis)", **split}
                         if split else None),
        "cpu_baseline": cpu,
        "parity_full_size": parity,
    }
    return result


def pool_token_major(pool, layer, n_layer, max_blocks, n_kv, bt, d, q8, oracle):
    """One layer of a device pool in the reference's token-major paged
    layout (key_cache[phys][kv_dim], text/generator/detail.hpp:2984-3005):
    uint16 halves for f16 pools, BLOCK_Q8_0 rows for q8_0 pools (whose
    regions hold values [bt][d] then scales [bt][d/32])."""
    lb = pool.numel() // n_layer
    raw = pool[layer * lb:(layer + 1) * lb].cpu().numpy().reshape(max_blocks, n_kv, -1)
    if not q8:
        h = raw.view(np.uint16).reshape(max_blocks, n_kv, bt, d)
        return np.ascontiguousarray(h.transpose(0, 2, 1, 3)).reshape(max_blocks * bt, n_kv * d)
    qs = raw[:, :, :bt * d].view(np.int8).reshape(max_blocks, n_kv, bt, d // 32, 32)
    ds = raw[:, :, bt * d:].view(np.uint16).reshape(max_blocks, n_kv, bt, d // 32)
    out = np.empty((max_blocks, bt, n_kv, d // 32), oracle.BLOCK_Q8_0)
    out["qs"] = qs.transpose(0, 2, 1, 3, 4)
    out["d"] = ds.transpose(0, 2, 1, 3)
    return out.reshape(max_blocks * bt, n_kv * d // 32)


def prefill_evict(args, torch, emelk, dev):
    """8 sequences with 4096 cached tokens each
    append a 512-token chunk (per layer: chunk append + causal chunk attention
    on MFMA, f16 in, fp32 accumulate), then 25% of each sequence's pages are
    evicted and the survivors compacted by a generated move list.  The
    q8_0 variant runs the same workload on q8_0 pools (the prefix is stored
    through the quantizing append; K/V are dequantized to fp16 while staged
    for the MFMAs)."""
    L, H, HK, D, BT, B, P0, NQ = 32, 32, 8, 128, 32, 8, 4096, 512
    if args.config.startswith("gemma4-d256"):
        # Gemma-4's sliding-window attention layers: 8 query heads on one KV
        # head of 256 (src/emel/model/gemma4/detail.cpp:24-29); 8 layers
        L, H, HK, D = 8, 8, 1, 256
    elif args.config.startswith("gemma4-d512"):
        # its global layers: key length 512 (row-by-row route); 8 layers
        L, H, HK, D = 8, 8, 1, 512
    q8 = "q8_0" in args.config
    rng = np.random.default_rng(args.seed)
    total = P0 + NQ
    pages = -(-total // BT)
    max_blocks = B * pages + 1
    actor = emelk.KvActor()
    assert actor.reserve(B, max_blocks, BT)[0]
    actor.set_free_order(rng.permutation(max_blocks).astype(np.uint16))
    for s in range(B):
        assert actor.allocate_sequence(s)[0]
        assert actor.allocate_slots(s, P0)[0]
    for s in range(B):
        assert actor.allocate_slots(s, NQ)[0]  # the chunk's slots
    stride = pages + 1
    tables = torch.from_numpy(actor.export_block_tables(list(range(B)), stride).view(np.int16)).to(dev)
    g = emelk.geometry(L, H, HK, D, BT, max_blocks, emelk.KV_Q8_0 if q8 else emelk.KV_F16)
    pb = emelk.pool_bytes(g)
    page_bytes = pb // (L * max_blocks)
    k_pool = torch.empty(pb, dtype=torch.uint8, device=dev)
    v_pool = torch.empty(pb, dtype=torch.uint8, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    if q8:
        # the prefix through the quantizing append (1% outliers x20, as config 4)
        zero = torch.zeros((B,), dtype=torch.int32, device=dev)
        for layer in range(L):
            rows = []
            for _ in range(2):
                x = torch.randn((B, P0, HK * D), generator=gen, device=dev)
                x = torch.where(torch.rand(x.shape, generator=gen, device=dev) < 0.01, x * 20.0, x)
                rows.append(x)
            emelk.append(g, k_pool, v_pool, layer, rows[0], rows[1], zero, tables)
            del rows
        torch.cuda.synchronize()
    else:
        k_pool.view(torch.float16).normal_(generator=gen)
        v_pool.view(torch.float16).normal_(generator=gen)
    q = [torch.randn((B, NQ, H, D), generator=gen, device=dev) for _ in range(L)]
    ck = [torch.randn((B, NQ, HK * D), generator=gen, device=dev) for _ in range(L)]
    cv = [torch.randn((B, NQ, HK * D), generator=gen, device=dev) for _ in range(L)]
    out = torch.empty((B, NQ, H, D), dtype=torch.float32, device=dev)
    qs = torch.full((B,), P0, dtype=torch.int32, device=dev)
    scale = float(1.0 / np.sqrt(D))
    stream = torch.cuda.current_stream()

    def step():
        for layer in range(L):
            emelk.append(g, k_pool, v_pool, layer, ck[layer], cv[layer], qs, tables)
            emelk.prefill_chunk(g, k_pool, v_pool, layer, q[layer], out, qs, tables, scale)

    def chunk_block():
        for layer in range(L):
            emelk.prefill_chunk(g, k_pool, v_pool, layer, q[layer], out, qs, tables, scale)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    K = args.steps
    # Step: the L layers' append + chunk attention captured as one HIP graph
    # and replayed K times (host clock).  Kernel timing (roofline): a graph
    # of the L chunk-attention calls alone (the chunk rows are appended),
    # replayed K times between one HIP event pair, per call.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    g_step, g_attn = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(g_step, stream=side):
            step()
        with torch.cuda.graph(g_attn, stream=side):
            chunk_block()
    torch.cuda.current_stream().wait_stream(side)
    g_step.replay()
    g_attn.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for k in range(K):
        g_step.replay()
    torch.cuda.synchronize()
    ms_step = 1e3 * (time.perf_counter() - t0) / K
    attn_ms = graph_event_ms(torch, g_attn, side, K)[0] / L
    # bytes the kernel must move per launch: the unique K/V of the layer
    # (prefix + chunk, every KV head), the fp32 queries and the fp32 output
    prefill_bytes = (B * HK * (P0 + NQ) * (page_bytes // (HK * BT)) * 2
                     + 2 * B * NQ * H * D * 4)
    rows = np.arange(NQ, dtype=np.float64)
    flops_layer = 4.0 * D * H * B * float(np.sum(P0 + rows + 1))
    tflops = flops_layer / (attn_ms * 1e-3) / 1e12

    # parity sample + CPU baseline: the last layer's output (out is reused
    # per layer) for seeded (sequence, row) pairs against the oracle's
    # per-row route (text/generator/detail.hpp:4297-4372), one thread per
    # sequence lane, batches of rows until the CPU budget is spent
    parity = cpu = None
    if not args.no_cpu_baseline:
        import oracle
        nlib, build = oracle.native_lib()
        nthreads = baseline_threads(args, B)
        layer = L - 1
        kc, vc = (pool_token_major(p_, layer, L, max_blocks, HK, BT, D, q8, oracle)
                  for p_ in (k_pool, v_pool))
        tables_h = tables.cpu().numpy().view(np.uint16)
        prng = np.random.default_rng(args.seed + 2)
        qh = q[layer].cpu().numpy()
        got = out.cpu().numpy()
        worst, ok_all, t_cpu, keys, pick = 0.0, True, 0.0, 0, []
        # seeded (sequence, row) pairs, the chunk's first and last rows
        # first, two rows per thread per batch
        cand = [(0, 0), (B - 1, NQ - 1)] + [(int(prng.integers(B)), int(prng.integers(NQ)))
                                            for _ in range(4096)]
        per = 2 * nthreads
        for i0 in range(0, len(cand), per):
            if pick and t_cpu >= args.cpu_budget:
                break
            batch = cand[i0:i0 + per]
            lims = np.array([P0 + r_ + 1 for _, r_ in batch], np.int32)
            qb = np.stack([qh[s_, r_].ravel() for s_, r_ in batch])
            want, secs = oracle.attention_rows("q8_0" if q8 else "f16", qb, kc, vc, tables_h,
                                               lims, BT, H, HK, D, scale, nthreads,
                                               row_table=[s_ for s_, _ in batch], lib_=nlib)
            t_cpu += secs
            keys += int(lims.sum())
            pick += batch
            for j, (s_, r_) in enumerate(batch):
                e = np.abs(got[s_, r_].ravel().astype(np.float64) - want[j])
                worst = max(worst, float(e.max()))
                ok_all = ok_all and bool(np.all(e <= 2e-3 + 1e-2 * np.abs(want[j])))
        parity = {"layer": layer, "n_rows": len(pick), "first_rows": pick[:6],
                  "max_abs_err": worst, "within_tolerance": ok_all}
        # the per-row route's time per attended key, scaled to a layer's keys
        layer_keys = B * float(np.sum(P0 + rows + 1))
        cpu_layer_s = t_cpu / keys * layer_keys
        cpu = {"value": round(flops_layer / cpu_layer_s / 1e12, 6), "unit": "TFLOP/s",
               **cpu_info(nthreads), "kind": "port", "build": build,
               "sample": f"{len(pick)} rows of layer {layer} ({t_cpu:.2f}s wall), scaled by "
                         f"attended keys to the layer's {B * NQ} rows; oracle per-row route, "
                         f"one thread per sequence lane, {nthreads} threads"}
        del kc, vc

    # eviction + compaction
    evicted = 0
    for s in range(B):
        ev_blocks = sorted(rng.choice(pages - 1, size=pages // 4, replace=False).tolist())
        ok, err, removed = actor.evict_blocks(s, ev_blocks)
        assert ok, err
        evicted += len(ev_blocks)
    ok, err, moves = actor.compact()
    assert ok, err
    mv = torch.tensor(moves, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()
    # one untimed launch, then repeats of the same move list, each between
    # its own HIP event pair after a GPU head start (the pools' contents are
    # not used after this point)
    copy_reps = 5
    copy_times = timed_blocks(torch, stream, lambda: emelk.copy_blocks(g, k_pool, v_pool, mv),
                              copy_reps,
                              prime=lambda: emelk.copy_blocks(g, k_pool, v_pool, mv))
    copy_ms = float(np.mean(copy_times))
    copy_bytes = 2 * 2 * len(moves) * L * page_bytes  # read + write, K and V
    traffic = PMC_TRAFFIC_BYTES.get(args.config)
    res = {
        "metric": "chunked-prefill attention TFLOP/s (MFMA f16, fp32 acc) + compaction GB/s",
        "kv_type": "q8_0" if q8 else "f16",
        "value": round(tflops, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True,
        "dtype": "f16", "data": "synthetic (seeded N(0,1), seeded page permutation)",
        "config": {"workload": args.config, "batch": B, "prefix": P0,
                   "chunk": NQ, "n_layer": L, "block_tokens": BT},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": 2500.0,
                     "unit": "TFLOP/s", "frac": round(tflops / 2500.0, 4),
                     "traffic": traffic,
                     "traffic_source": (f"profiles/prefill_kernel_{args.config}.md (rocprofv3 "
                                        "--pmc FETCH_SIZE / WRITE_SIZE of an earlier run of this "
                                        "workload, copy-calibrated)") if traffic else None,
                     "algorithmic_bytes": prefill_bytes,
                     "kernel": "prefill_kernel",
                     "timing": "HIP events around K replays of a graph of the L chunk-attention "
                               "calls, per call",
                     "flops_per_launch": flops_layer, "avg_launch_ms": round(attn_ms, 4)},
        "cpu_baseline": cpu,
        "parity_sample": parity,
        "compaction": {"pages_evicted": evicted, "moves": len(moves), "ms": round(copy_ms, 4),
                       "timing": f"mean of {len(copy_times)} event-timed launches after an "
                                 "untimed one (min "
                                 f"{min(copy_times):.4f} ms, max {max(copy_times):.4f} ms)",
                       "GB/s": round(copy_bytes / (copy_ms * 1e-3) / 1e9, 1),
                       "bytes": copy_bytes,
                       "roofline": {"bound": "hbm", "kernel": "copy_blocks_kernel (HIP events)",
                                    "achieved": round(copy_bytes / (copy_ms * 1e-3) / 1e9, 1),
                                    "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                    "frac": round(copy_bytes / (copy_ms * 1e-3) / 1e9
                                                  / HBM_PEAK_GBS, 4)}},
    }
    return res


def generator(args, torch, emelk, dev):
    """The multi-sequence step executor (emelk_batch_decoder) at the
    Llama-3-8B shape: 64 sequences are prefilled to 8192 tokens through it in
    chunks of 512 (per layer: RoPE + append, then chunked-prefill attention),
    then each timed step extends every sequence by one token (allocate_slots
    for the batch, block-table upload) and runs, per layer, RoPE + append and
    decode attention.  The timed steps replay the 32 layers' launches as one
    HIP graph (graph-stable plan), with begin_step's host work and uploads
    in every step; the eager rate is reported beside it."""
    L, H, HK, D, BT, B, CTX = 32, 32, 8, 128, 32, 64, 8192
    chunk = 512
    steps = args.steps
    max_len = CTX + args.warmup + 2 * steps + 2  # warmup, eager and graph-replayed steps
    pages = B * (-(-max_len // BT)) + 8
    g = emelk.geometry(L, H, HK, D, BT, pages, emelk.KV_F16)
    actor = emelk.KvActor()
    ok, err = actor.reserve(B, pages, BT)
    assert ok, err
    rng = np.random.default_rng(args.seed)
    actor.set_free_order(rng.permutation(pages).astype(np.uint16))
    for s in range(B):
        assert actor.allocate_sequence(s)[0]
    side = torch.cuda.Stream()  # graph capture needs a non-default stream
    torch.cuda.set_stream(side)
    sid = side.cuda_stream
    cache = emelk.KvCache(g, stream=sid)
    rope = emelk.RopeTable(D, D, max_len + 1, 500000.0, emelk.NORMAL_PAIRING, stream=sid)
    dec = emelk.BatchDecoder(g, actor, cache, rope, max_batch=B, max_kv_len=max_len, stream=sid)
    dec.set_fixed_plan(True)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    ids = list(range(B))
    scale = float(1.0 / np.sqrt(D))
    # prefill (untimed): one set of random projections reused for every chunk and layer
    qc = torch.randn((B, chunk, H * D), generator=gen, device=dev)
    kc = torch.randn((B, chunk, HK * D), generator=gen, device=dev)
    vc = torch.randn((B, chunk, HK * D), generator=gen, device=dev)
    qr = torch.empty_like(qc)
    oc = torch.empty_like(qc)
    t0 = time.time()
    for _ in range(CTX // chunk):
        dec.begin_step(ids, chunk)
        for layer in range(L):
            dec.layer(layer, qc, qr, kc, vc, oc, scale)
    torch.cuda.synchronize()
    log(f"[bench] generator prefill of {B} x {CTX} tokens in {time.time() - t0:.1f}s")
    del qc, kc, vc, qr, oc
    q1 = torch.randn((B, 1, H * D), generator=gen, device=dev)
    k1 = torch.randn((B, 1, HK * D), generator=gen, device=dev)
    v1 = torch.randn((B, 1, HK * D), generator=gen, device=dev)
    q1r = torch.empty_like(q1)
    o1 = torch.empty_like(q1)

    def layers():
        for layer in range(L):
            dec.layer(layer, q1, q1r, k1, v1, o1, scale)

    def step():
        dec.begin_step(ids, 1)
        layers()

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    eager_ms = 1e3 * (time.perf_counter() - t_start) / steps
    # capture one step's layers, then replay them after each begin_step
    dec.begin_step(ids, 1)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        layers()
    graph.replay()
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    for _ in range(steps):
        dec.begin_step(ids, 1)
        graph.replay()
    torch.cuda.synchronize()
    ms_step = 1e3 * (time.perf_counter() - t_start) / steps
    ctx_mean = CTX + args.warmup + steps + 1 + (steps + 1) / 2.0  # the graph-replayed steps
    kv_bytes = B * ctx_mean * HK * D * 2 * 2 * L
    res = {
        "metric": "multi-sequence decode step through emelk_batch_decoder (tokens/s)",
        "value": round(B / (ms_step * 1e-3), 1), "unit": "tokens/s", "n_gpus": 1,
        "steps": steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic (seeded N(0,1) projections, seeded page permutation)",
        "config": {"workload": "llama3-8b-b64-ctx8k-generator", "n_layer": L, "batch": B,
                   "ctx": CTX, "prefill_chunk": chunk,
                   "step_launch": "begin_step + one HIP graph of the 32 layers",
                   "parallelism": "single GPU"},
        "kv_read_GBps": round(kv_bytes / (ms_step * 1e-3) / 1e9, 1),
        "eager_ms_per_step": round(eager_ms, 4),
    }
    dec.close()
    return res


if __name__ == "__main__":
    main()
