#!/usr/bin/env python3
"""Benchmark of the token-mixing hot path on one MI355X.

Default run: the BASELINE metric on config 3 — paged GQA decode attention, batch 64, bf16 KV pool, lengths
U[128, 8192], 8/2 heads x 256, block 16, sigmoid output gate fused. One step = one RocmBackend.paged_attention call
over the whole batch (split-K kernel + merge/gate kernel), inputs already resident in HBM. Prints ONE JSON line, whose
"configs" holds the same record (value, roofline, cpu_baseline) for configs 1, 2, 4 and 5, and whose
"access_pattern_ceiling" entries (config 3 here, config 2 under configs) give what the memory system delivers for
each decode kernel's own access pattern with no arithmetic (librk_probe.so).

  value           decode-attention tokens/s = batch / step time (one attention-layer call per decode token)
  roofline        the split-K kernel (the dominant launch): its algorithmic bytes (every visible K/V byte once, q,
                  the block-table entries and lens it reads) / its average duration, measured with HIP events over
                  back-to-back launches on the stream it runs on; peak = 8 TB/s HBM
  cpu_baseline    the CPU oracle (TorchBackend.paged_attention + gate restated in torch fp32) on the same seeded
                  inputs, timed on this host's cores

Other workloads print the same record for: c1, the config-1 decode (parity/latency case); c2, the config-2 DeltaNet
decode step (batch 8; state slots rotated so reads come from HBM, not the 256 MB Infinity Cache); c4, the config-4
chunked gated delta prefill (4 x 4096 tokens, both kernels); c5, the config-5 packed prefill attention (c5f: the
same batch in fp32, on the fp32-operand kernel; c5g: at 14/2 heads x 64, on the 16-query bf16 kernel); lp, the
DeltaNet prefill companions (fused conv / norms / beta, g front and the gated RMSNorm) on the config-4 batch; ap,
the config-3 decode attention layer with its q / k norm, RoPE and KV write (rk_attn_prep) in front; wd, the
sliding-window decode (window 4096) through the grouped pool's rings; mv, every linear of a Qwen3.5-2B decode step at
batch 8 (INT4 layers, INT8 head).
Timing: W untimed warm-up steps, then K timed steps captured in one HIP graph and replayed between two events
after a device synchronize (the eager, Python-issued rate is reported beside it).
"""
import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (str(ROOT), str(ROOT / "metal-inference-engine_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

HBM_PEAK_GBS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "traffic.json"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cpu_threads() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def traffic_for(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc summary (FETCH_SIZE + WRITE_SIZE,
    scaled by the copy-kernel calibration), or None when no summary covers it."""
    if not TRAFFIC_FILE.exists():
        return None
    data = json.loads(TRAFFIC_FILE.read_text())
    entry = data.get(kernel)
    return entry.get("bytes_per_launch") if entry else None


def time_region(fn, steps: int, warmup: int, stream) -> float:
    """Average ms per call of fn over `steps` back-to-back calls on `stream` (after `warmup` calls)."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for _ in range(steps):
        fn()
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps


USE_GRAPHS = True
SETTLE_MS = 60.0


def settle(fn, stream, target_ms: float = None) -> None:
    """Run fn untimed for about target_ms of device time before a workload's warm-up: the shader clock ramps up over
    the first tens of milliseconds of load (measured on config 4: 288 us per call timed after 3 warm-up calls, 238 us
    after 100), and every workload is timed at the clock it runs at under sustained load."""
    import torch
    target = SETTLE_MS if target_ms is None else target_ms
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    fn()
    t1.record(stream)
    torch.cuda.synchronize()
    per = max(t0.elapsed_time(t1), 1e-3)
    for _ in range(min(int(target / per), 20000)):
        fn()
    torch.cuda.synchronize()


def graph_time(fn, steps: int, stream) -> float:
    """Average ms per step of `steps` calls of fn captured in one HIP graph (no host work between launches); with
    --no-graph (counter-collection runs) the eager back-to-back rate instead. The timed replay is queued behind one
    untimed replay of the same graph, so the host's graph-launch latency (about 0.1 ms, which the first event would
    otherwise count against the K steps) overlaps device work; every timed step still runs in full."""
    import torch
    if not USE_GRAPHS:
        return time_region(fn, steps, 0, stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(steps):
            fn()
    graph.replay()                                  # first replay uploads the graph
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    w0 = time.perf_counter()
    graph.replay()                                  # untimed: the timed replay is queued behind it
    t0.record(stream)
    graph.replay()
    t1.record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - w0) * 1e3
    GRAPH_WALL_MS.append(wall / (2 * steps))        # host clock over both replays, from the first launch
    return t0.elapsed_time(t1) / steps


GRAPH_WALL_MS: list[float] = []


CPU_SAMPLE_S = 10.0


def cpu_time(fn, runs: int = 3) -> tuple[float, int, float]:
    """Median seconds per call of fn on the host cores, over at least `runs` calls after a warm-up and until about
    CPU_SAMPLE_S seconds of calls have run (a bounded sample). Returns (median, calls, total seconds)."""
    fn()                                   # warm-up
    ts = []
    while len(ts) < runs or (sum(ts) < CPU_SAMPLE_S and len(ts) < 10000):
        t = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t)
    return statistics.median(ts), len(ts), sum(ts)


PLAN_LAYERS = 6     # full-attention layers of Qwen3.5-2B: the decode-step layers that share one batch layout plan


def bench_paged_decode(case, args, backend, workload_name: str, config: dict, plan_layers: int = 0):
    import torch
    from native import kernels
    from native.rocm_native import load
    dev = backend.device
    stream = torch.cuda.current_stream(dev)
    log(f"[bench] {workload_name}: copying inputs to {dev}")
    sets = []
    for i in range(args.sets):                       # distinct copies: consecutive steps never re-read a cache
        c = case.to(dev)
        if i:
            c.k_pool, c.v_pool = c.k_pool.clone(), c.v_pool.clone()
        sets.append(c)
    torch.cuda.synchronize()
    B, Hq, d = case.q.shape
    it = [0]
    NB0, bs0, Hkv0, _ = case.k_pool.shape

    def call():
        c = sets[it[0] % len(sets)]
        it[0] += 1
        backend.paged_attention(c.q, c.k_pool, c.v_pool, c.tables, c.lens, c.block_size, c.window, gate=c.gate)

    def make_plan(c):
        return backend.decode_plan(c.tables, c.lens, c.block_size, Hq, Hkv0, d, NB0, c.window)

    def planned_step():
        # one decode step's attention work: the batch layout plan once, then the model's attention layers, each on
        # its own pool (the sets alternate, so consecutive layers never re-read a cache), all with that plan
        c0 = sets[0]                                 # the step's tables and lens, shared by its layers
        plan = make_plan(c0)
        for layer in range(plan_layers):
            c = sets[(it[0] + layer) % len(sets)]
            backend.paged_attention(c.q, c.k_pool, c.v_pool, c0.tables, c0.lens, c.block_size, c.window, gate=c.gate,
                                    plan=plan)
        it[0] += plan_layers

    per = plan_layers if plan_layers else 1
    step = planned_step if plan_layers else call
    settle(step, stream)
    log(f"[bench] {workload_name}: timing {args.steps} steps after {args.warmup} warm-up")
    eager_ms = time_region(step, args.steps, args.warmup, stream) / per
    t = time.perf_counter()
    for _ in range(args.steps):
        step()
    host_us = (time.perf_counter() - t) / (args.steps * per) * 1e6
    torch.cuda.synchronize()
    ms = graph_time(step, args.steps, stream) / per
    single_ms = graph_time(call, args.steps, stream) if plan_layers else ms

    # the split-K launch alone: back-to-back launches through the C ABI with prebuilt arguments (with the step's
    # plan when the step has one: the plan is made once per step, outside the layers' split launches)
    lib = load()
    outs = [torch.empty(B, Hq, d, device=dev) for _ in sets]
    NB, bs, Hkv, _ = case.k_pool.shape
    max_nb = case.tables.shape[1]
    need = lib.lib.rk_paged_decode_workspace_bytes(B, Hq, Hkv, d, bs, max_nb)
    ws = kernels.workspace(dev, need)
    plan = make_plan(sets[0]) if plan_layers else None
    pl = (plan.buf.data_ptr(), plan.buf.numel()) if plan is not None else (None, 0)

    def argsets_for(pl):
        t = sets[0]                                  # one batch layout (tables, lens) for every pool copy
        return [(0, o.data_ptr(), c.q.data_ptr(), c.k_pool.data_ptr(), c.v_pool.data_ptr(),
                 kernels.DTYPE_CODES[c.k_pool.dtype], t.tables.data_ptr(), t.lens.data_ptr(), B, Hq, Hkv, d, bs,
                 max_nb, NB, int(c.window or 0), c.gate.data_ptr(), c.gate.stride(0), *pl, ws.data_ptr(),
                 ws.numel(), stream.cuda_stream)
                for o, c in zip(outs, sets)]
    fn = lib.lib.rk_paged_decode_phase

    def split_of(argsets):
        j = [0]

        def split():
            a = argsets[j[0] % len(argsets)]
            j[0] += 1
            if fn(*a) != 0:
                raise RuntimeError(lib.last_error())
        return split

    split_ms = time_region(split_of(argsets_for(pl)), args.steps, args.warmup, stream)
    split_unplanned_ms = time_region(split_of(argsets_for((None, 0))), args.steps, args.warmup, stream) \
        if plan_layers else split_ms
    plan_ms = graph_time(lambda: make_plan(sets[0]), args.steps, stream) if plan_layers else 0.0
    ceiling = block_stream_ceiling(case, sets, args, stream) if getattr(args, "ceiling", False) else None
    kv = case.kv_bytes()
    split_bytes = kv + B * Hq * d * 4 + 4 * case.table_entries() + 4 * B
    achieved = split_bytes / (split_ms * 1e-3) / 1e9
    step_gbs = case.algorithmic_bytes() / (ms * 1e-3) / 1e9
    log(f"[bench] {workload_name}: step {ms * 1e3:.1f} us in a graph ({step_gbs:.0f} GB/s algorithmic), "
        f"{eager_ms * 1e3:.1f} us eager (host {host_us:.1f} us per call), split kernel {split_ms * 1e3:.1f} us "
        f"({achieved:.0f} GB/s)")
    if plan_layers:
        log(f"[bench] {workload_name}: per layer call with the step's plan shared by {plan_layers} layers; "
            f"plan {plan_ms * 1e3:.1f} us per step, one call without a plan {single_ms * 1e3:.1f} us, split kernel "
            f"without a plan {split_unplanned_ms * 1e3:.1f} us")

    cpu = None
    if not args.no_cpu:
        from oracle import backend_ref
        torch.set_num_threads(cpu_threads())
        log(f"[bench] {workload_name}: CPU oracle on {torch.get_num_threads()} threads")

        def cpu_run():
            o = backend_ref.paged_attention(case.q, case.k_pool, case.v_pool, case.tables, case.lens,
                                            case.block_size, case.window)
            backend_ref.gate(o, case.gate)

        t, calls, total = cpu_time(cpu_run)
        cpu = {"value": B / t, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"the full {workload_name} batch ({B} sequences, {int(case.lens.sum())} positions): "
                         f"median of {calls} runs after 1 warm-up ({total:.1f} s in all), {t:.4f} s per batch"}
    return {
        "metric": "decode attn tokens/s @ batch 64 + achieved HBM GB/s (% of 8 TB/s), 1 GPU",
        "value": B / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) inputs; no model weights are involved)",
        "config": config,
        "hbm_gbs_step": step_gbs, "hbm_frac_step": step_gbs / HBM_PEAK_GBS,
        "timing": "value and ms_per_step: K steps captured in one HIP graph, replayed between two events behind one "
                  "untimed replay (after about 60 ms of untimed steps to settle the clock); eager_ms_per_step: the "
                  "same K steps issued from Python" + (
                      f"; a step is one decode step's attention work for a model with {plan_layers} attention "
                      f"layers: the batch layout plan (rk_paged_decode_plan) once, then {plan_layers} paged "
                      f"attention calls over alternating pools that read it; ms_per_step is per attention-layer call "
                      f"(the step's time / {plan_layers})" if plan_layers else ""),
        "eager_ms_per_step": eager_ms, "host_us_per_call": host_us,
        **({"plan": {"layers_per_plan": plan_layers, "plan_ms": plan_ms, "single_call_ms": single_ms,
                     "split_ms_without_plan": split_unplanned_ms}} if plan_layers else {}),
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic_for(f"paged_decode_split/{workload_name}"),
                     "kernel": "paged_decode_split", "bytes_per_launch": split_bytes, "avg_ms": split_ms},
        "cpu_baseline": cpu,
        **({"access_pattern_ceiling": ceiling} if ceiling else {}),
    }


def block_stream_ceiling(case, sets, args, stream) -> dict:
    """What HBM delivers for this batch's K / V tiles with no arithmetic (rk_probe_block_stream over the same
    device pools): the tiles in table order (the decode's scattered 16 KiB blocks) and sorted by address (a
    near-sequential stream of the same bytes), best of three grid sizes each."""
    import torch
    from native.rocm_native import load_probes
    probes = load_probes()
    NB, bs, Hkv, d = case.k_pool.shape
    esz = case.k_pool.element_size()
    if (bs * Hkv * d * esz) not in (4096, 8192, 16384):
        return None
    tile_bytes = bs * Hkv * d * esz
    offs = [int(case.tables[i, b]) * tile_bytes for i, n in enumerate(case.lens.tolist())
            for b in range(((n - case.window) // bs if case.window and n > case.window else 0), -(-n // bs))]
    dev = sets[0].q.device
    lists = {"table_order": torch.tensor(offs, dtype=torch.int64, device=dev),
             "address_order": torch.tensor(sorted(offs), dtype=torch.int64, device=dev)}
    sink = torch.empty(1024 * 512, dtype=torch.int32, device=dev)
    moved = 2 * tile_bytes * len(offs)
    out = {"kernel": "probe_block_stream", "tiles": len(offs), "bytes_per_launch": moved,
           "kv_bytes_visible": case.kv_bytes()}
    # persistent grids of 256 / 512 / 1024 workgroups (8 waves each), and one-shot workgroups over runs of
    # 8 / 16 / 32 consecutive tiles; the fastest of each kind is kept
    shapes = [("persistent", w, 0) for w in (256, 512, 1024)] + [("one_shot", 0, n) for n in (8, 16, 32)]
    for name, lst in lists.items():
        res = {}
        for kind, wgs, per in shapes:
            j = [0]

            def run():
                c = sets[j[0] % len(sets)]
                j[0] += 1
                probes.call("rk_probe_block_stream", c.k_pool.data_ptr(), c.v_pool.data_ptr(), lst.data_ptr(),
                            len(offs), tile_bytes, wgs, per, sink.data_ptr(), stream.cuda_stream)
            ms = time_region(run, args.steps, args.warmup, stream)
            log(f"[bench] ceiling ({name}, {kind}, {wgs or per}): {ms * 1e3:.1f} us")
            if kind not in res or ms < res[kind]["avg_ms"]:
                gbs = moved / (ms * 1e-3) / 1e9
                res[kind] = {"avg_ms": ms, "workgroups" if wgs else "tiles_per_workgroup": wgs or per, "gbs": gbs,
                             "frac": gbs / HBM_PEAK_GBS}
        out[name] = res
    return out


class SlotState:
    """A DeltaNet state holder for the CPU oracle: S [n_linear, H, dk, dv], conv_tail [n_linear, K-1, C]."""

    def __init__(self, S, conv_tail):
        self.S, self.conv_tail = S, conv_tail


def bench_deltanet(args, backend):
    import torch
    import workloads as wl
    from native import kernels
    from oracle import backend_ref
    dev = backend.device
    stream = torch.cuda.current_stream(dev)
    B, n_linear, max_seqs = 8, 6, 64                  # 64 x 6 slots x 1 MiB per head-set = 384 MiB of state
    case = wl.c2_deltanet_step(batch=B, max_seqs=max_seqs, n_linear=n_linear)
    c = case.to(dev)
    gen = torch.Generator().manual_seed(22)
    perms = [torch.randperm(max_seqs, generator=gen)[:B].to(torch.int32).to(dev) for _ in range(8)]
    combos = [(p, s) for p in perms for s in range(n_linear)]      # 48 distinct (slot set, layer) state blocks
    torch.cuda.synchronize()
    k = [0]

    def step():
        seqs, slot = combos[k[0] % len(combos)]
        k[0] += 1
        kernels.deltanet_decode(c.qkv, c.z, c.b, c.a, c.conv, c.S, seqs, slot, c.conv_w, c.A_log, c.dt_bias,
                                c.norm_w, c.eps, c.dims)

    # launch-bound at this size: capture the timed steps in a HIP graph and time one replay
    settle(step, stream)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ms = graph_time(step, args.steps, stream)
    nbytes = case.algorithmic_bytes()
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"[bench] c2: {ms * 1e3:.2f} us per step, {gbs:.0f} GB/s algorithmic")
    ceiling = None
    if getattr(args, "ceiling", False):
        # the step's state traffic alone (read, scale, write back each head's 64 KiB block), same rotation
        from native.rocm_native import load_probes
        probes = load_probes()
        H, dk, dv, _ = case.dims
        state_bytes = 2 * B * H * dk * dv * 4
        ceiling = {"kernel": "probe_state_rmw", "bytes_per_launch": state_bytes}
        for split in (1, 2, 4, 8, 16):
            def rmw():
                seqs, slot = combos[k[0] % len(combos)]
                k[0] += 1
                probes.call("rk_probe_state_rmw", c.S.data_ptr(), seqs.data_ptr(), B, n_linear, slot, H, dk, dv,
                            split, 1.0, torch.cuda.current_stream(dev).cuda_stream)   # the capture stream
            t = graph_time(rmw, args.steps, stream)
            ceiling[f"split_{split}"] = {"workgroups": B * H * split, "avg_ms": t,
                                         "gbs": state_bytes / (t * 1e-3) / 1e9,
                                         "frac_of_step_bytes": nbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS}
            log(f"[bench] c2 state ceiling, {split} workgroups per head: {t * 1e3:.2f} us")
    cpu = None
    if not args.no_cpu:
        torch.set_num_threads(cpu_threads())
        states = [SlotState(case.S[int(s)].clone(), case.conv[int(s)].clone()) for s in case.seq_index]

        def cpu_run():
            backend_ref.deltanet_decode_batch(case.qkv, case.z, case.b, case.a, states, 0, case.conv_w, case.A_log,
                                              case.dt_bias, case.norm_w, case.eps, case.dims)
        t, calls, total = cpu_time(cpu_run, runs=5)
        cpu = {"value": B / t, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"one batch-{B} step (state carried between calls), median of {calls} calls after 1 "
                         f"warm-up ({total:.1f} s in all), {t * 1e3:.2f} ms per step"}
    return {
        "metric": "DeltaNet decode step tokens/s @ batch 8 + achieved HBM GB/s (% of 8 TB/s), 1 GPU",
        "value": B / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded)", "config": {"workload": "config 2: DeltaNet decode step, batch 8, 16 heads x "
                                                             "128 x 128 fp32 state, conv 4 over 6144 channels"},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
                     "traffic": traffic_for("deltanet_step/c2"), "kernel": "deltanet_step_kernel",
                     "bytes_per_launch": nbytes, "avg_ms": ms},
        "cpu_baseline": cpu,
        **({"access_pattern_ceiling": ceiling} if ceiling else {}),
    }


FP32_MFMA_PEAK_TFLOPS = 157.3     # MI355X dense fp32 matrix peak


def bench_prefill(args, backend, chunk: bool = False, fp32: bool = False, g7: bool = False):
    """Config 5 (chunk False), or one 512-token chunk over a 32,768-token history (chunk True: the grid without
    split key ranges would fill 32 of 256 CUs). fp32: config 5's batch in the Qwen3.5 engine's own fp32 pool and
    activations, which runs on the fp32-operand kernel (fp32 MFMA), priced against the fp32 matrix peak. g7: config
    5's batch at 14/2 heads x 64 (the reference's own kernel-test shape, tests/test_kernels.py:107-114), bf16, which
    runs on the 16-query bf16-operand kernel."""
    import torch
    import workloads as wl
    from native import kernels
    dev = backend.device
    stream = torch.cuda.current_stream(dev)
    if chunk:
        case = wl.chunk_prefill()
    elif g7:
        case = wl.c5_prefill(Hq=14, Hkv=2, d=64)
    else:
        case = wl.c5_prefill(dtype=torch.float32 if fp32 else torch.bfloat16)
    tag = "ck" if chunk else ("c5f" if fp32 else ("c5g" if g7 else "c5"))
    c = case.to(dev)
    torch.cuda.synchronize()

    def step():
        kernels.paged_prefill(c.q, c.k_new, c.v_new, c.k_pool, c.v_pool, c.tables, c.cu_seqlens, c.starts,
                              c.block_size, gate=c.gate)

    settle(step, stream)
    ms = time_region(step, args.steps, args.warmup, stream)
    flops = case.flops()
    tflops = flops / (ms * 1e-3) / 1e12
    N = case.q.shape[0]
    peak = FP32_MFMA_PEAK_TFLOPS if fp32 else 2500.0
    log(f"[bench] {tag}: {ms * 1e3:.1f} us per packed prefill, {tflops:.1f} TFLOP/s ({tflops / peak:.1%} of peak)")
    cpu = None
    if not args.no_cpu:
        from oracle import prefill_ref
        torch.set_num_threads(cpu_threads())
        # sample: the shortest segment (of the chunk: its first 64 tokens), scaled to the whole batch by flops
        s = min(range(len(case.starts)), key=lambda i: case.lengths()[i] * (case.starts[i] + case.lengths()[i]))
        lo, hi = case.cu_seqlens[s], case.cu_seqlens[s + 1]
        if chunk:
            hi = lo + 64
        one = wl.PrefillCase(case.q[lo:hi], case.k_new[lo:hi], case.v_new[lo:hi], case.gate[lo:hi],
                             case.k_pool.clone(), case.v_pool.clone(), case.tables[s:s + 1], [0, hi - lo],
                             [case.starts[s]], case.block_size)
        # repeated calls rewrite the same rows into the cloned pool: every call does identical work
        t, calls, total = cpu_time(lambda: prefill_ref.packed_prefill(one.q, one.k_new, one.v_new, one.k_pool,
                                                                      one.v_pool, one.tables, one.cu_seqlens,
                                                                      one.starts, one.block_size, one.gate), runs=1)
        t_full = t * flops / one.flops()
        cpu = {"value": N / t_full, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"segment {s} alone ({hi - lo} new tokens on a {case.starts[s]}-token prefix): median of "
                         f"{calls} calls ({total:.1f} s in all), {t:.3f} s per call, scaled to the whole pack by "
                         f"flops"}
    work, n_slots = kernels.prefill_work(case.lengths(), case.starts, None, True, kernels.PREFILL_SPLIT_TILES,
                                         case.k_pool.shape[2], kernels.device_cus(dev))
    if fp32:
        return {
            "metric": "packed prefill attention tokens/s (config 5 batch, fp32 pool and activations) + TFLOP/s "
                      "(% of fp32 MFMA peak), 1 GPU",
            "value": N / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic (seeded)",
            "config": {"workload": "config 5's batch with the fp32 pool, q, new K/V and gate of the Qwen3.5 engine "
                                   "(src/models/qwen3_5.py:70-71): 8 packed segments, 8/2 heads x 256, block 16, "
                                   "causal, gate, KV write-back; fp32 operands (fp32 MFMA)",
                       "new_tokens": N, "flops": flops},
            "roofline": {"bound": "mfma", "achieved": tflops, "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": tflops / FP32_MFMA_PEAK_TFLOPS, "traffic": traffic_for("prefill_attention_f32/c5f"),
                         "kernel": "prefill_attention_f32 (+ prefill_kv_write)", "avg_ms": ms},
            "cpu_baseline": cpu,
        }
    if g7:
        return {
            "metric": "packed prefill attention tokens/s (config 5 batch at 14/2 heads x 64) + TFLOP/s (% of bf16 "
                      "MFMA peak), 1 GPU",
            "value": N / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded)",
            "config": {"workload": "config 5's segments (8 packed, new U[64, 2048] on prefixes U[0, 16384]) at 14/2 "
                                   "heads x 64, the reference's kernel-test shape (group 7: the 16-query bf16 "
                                   "kernel, two head chunks), block 16, causal, gate, KV write-back",
                       "new_tokens": N, "flops": flops},
            "roofline": {"bound": "mfma", "achieved": tflops, "peak": 2500.0, "unit": "TFLOP/s",
                         "frac": tflops / 2500.0, "traffic": traffic_for("prefill_attention_b16/c5g"),
                         "kernel": "prefill_attention_b16 (+ prefill_kv_write)", "avg_ms": ms},
            "cpu_baseline": cpu,
        }
    if chunk:
        return {
            "metric": "chunked-prefill attention tokens/s (512 new on 32,768 cached) + TFLOP/s, 1 GPU",
            "value": N / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded)",
            "config": {"workload": "one 512-token chunk after 32,768 cached positions, 8/2 heads x 256, block 16, "
                                   "causal, gate, KV write-back", "new_tokens": N, "flops": flops,
                       "work_entries": len(work) // 5, "split_pieces": n_slots},
            "roofline": {"bound": "mfma", "achieved": tflops, "peak": 2500.0, "unit": "TFLOP/s",
                         "frac": tflops / 2500.0, "traffic": None,
                         "kernel": "prefill_attention (+ prefill_kv_write)", "avg_ms": ms},
            "cpu_baseline": cpu,
        }
    return {
        "metric": "packed prefill attention tokens/s (config 5) + TFLOP/s (% of bf16 MFMA peak), 1 GPU",
        "value": N / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded)",
        "config": {"workload": "config 5: 8 packed segments, new U[64, 2048] on prefixes U[0, 16384], 8/2 heads x 256, "
                               "block 16, causal, gate, KV write-back", "new_tokens": N, "flops": flops},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": 2500.0, "unit": "TFLOP/s", "frac": tflops / 2500.0,
                     "traffic": traffic_for("prefill_attention/c5"), "kernel": "prefill_attention (+ prefill_kv_write)",
                     "avg_ms": ms},
        "cpu_baseline": cpu,
    }


def bench_chunked_delta(args, backend):
    """Config 4: one packed call over 4 sequences x 4096 tokens (both kernels), captured in a HIP graph. Consecutive
    steps alternate between two seeded input sets (403 MB of q, k, v together, beyond the 256 MB Infinity Cache) and
    carry one state, so every step reads its inputs from HBM and depends on the step before."""
    import torch
    import workloads as wl
    from native import kernels
    from native.rocm_native import load
    from native.kernels import to_device
    dev = backend.device
    stream = torch.cuda.current_stream(dev)
    case = wl.c4_chunked_delta()
    sets = [case.to(dev), wl.c4_chunked_delta(seed=44).to(dev)]
    N, H, dk = case.q.shape
    dv = case.v.shape[2]
    cu = case.cu_seqlens
    cuc = [0]
    for a, b in zip(cu, cu[1:]):
        cuc.append(cuc[-1] + -(-(b - a) // kernels.DELTA_CHUNK))
    meta = to_device(torch.tensor(cu + cuc, dtype=torch.int32), dev)
    lib = load()
    ws = torch.empty(lib.lib.rk_gated_delta_workspace_bytes(cuc[-1], H), dtype=torch.uint8, device=dev)
    out = torch.empty(N, H, dv, dtype=torch.float32, device=dev)
    S = sets[0].S.clone()
    n = len(cu) - 1
    torch.cuda.synchronize()
    turn = [0]

    def step():      # the state is carried from step to step; its values do not change the work
        c = sets[turn[0] % 2]
        turn[0] += 1
        lib.call("rk_gated_delta_chunked", out.data_ptr(), S.data_ptr(), S.stride(0), c.q.data_ptr(), c.k.data_ptr(),
                 c.v.data_ptr(), 1, c.beta.data_ptr(), c.g.data_ptr(), meta.data_ptr(), meta.data_ptr() + 4 * (n + 1),
                 None, n, cuc[-1], H, dk, dv, ws.data_ptr(), ws.numel(), torch.cuda.current_stream(dev).cuda_stream)

    settle(step, stream)
    eager = time_region(step, args.steps, args.warmup, stream)
    ms = graph_time(step, args.steps, stream)
    flops = case.flops()
    tflops = flops / (ms * 1e-3) / 1e12
    gbs = case.hbm_bytes() / (ms * 1e-3) / 1e9
    if GRAPH_WALL_MS:                                # (graph_time times eager launches under --no-graph)
        log(f"[bench] c4: graph replays {GRAPH_WALL_MS[-1] * 1e3:.1f} us per call by the host clock (both replays)")
    log(f"[bench] c4: {ms * 1e3:.1f} us per packed call (eager {eager * 1e3:.1f} us), {tflops:.1f} TFLOP/s "
        f"({tflops / 25:.1f}% of bf16 MFMA peak), {gbs:.0f} GB/s algorithmic ({gbs / HBM_PEAK_GBS:.1%} of HBM)")
    cpu = None
    if not args.no_cpu:
        from oracle import ops_ref
        torch.set_num_threads(cpu_threads())
        lo, hi = cu[0], cu[1]
        f = lambda x: x[lo:hi].float()
        t, calls, total = cpu_time(lambda: ops_ref.gated_delta_chunked(f(case.q), f(case.k), f(case.v), f(case.beta),
                                                                       f(case.g), case.S[0].clone()), runs=1)
        t_full = t * n
        cpu = {"value": N / t_full, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"sequence 0 alone ({hi - lo} tokens, {H} heads): median of {calls} calls ({total:.1f} s "
                         f"in all), {t:.3f} s per call, times {n} sequences"}
    return {
        "metric": "chunked gated delta prefill tokens/s (config 4) + TFLOP/s (% of bf16 MFMA peak), 1 GPU",
        "value": N / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded)",
        "config": {"workload": "config 4: chunked gated delta rule, 4 x 4096 tokens packed, 16 heads, dk = dv = 128, "
                               "chunk 64, bf16 inputs, fp32 state from zero", "tokens": N, "flops": flops,
                   "hbm_bytes": case.hbm_bytes(), "input_sets": 2},
        "roofline": {"bound": "mfma", "achieved": tflops, "peak": 2500.0, "unit": "TFLOP/s", "frac": tflops / 2500.0,
                     "traffic": traffic_for("chunked_delta/c4"), "kernel": "delta_chunk_prep + delta_chunk_scan",
                     "avg_ms": ms, "hbm_frac": gbs / HBM_PEAK_GBS},
        "cpu_baseline": cpu,
    }


def bench_linear_prefill(args, backend):
    """The DeltaNet prefill companions on the config-4 batch: one step = the fused front (conv + split + l2norm +
    beta / g, conv tails handed over) and the gated RMSNorm over 4 x 4096 packed tokens; the whole layer (front +
    chunked delta rule + norm) is timed beside it."""
    import torch
    import workloads as wl
    from native import kernels
    from native.rocm_native import RK_F32, load
    from native.kernels import to_device
    dev = backend.device
    stream = torch.cuda.current_stream(dev)
    case = wl.lp_linear_prefill()
    c = case.to(dev)
    H, dk, dv, _ = case.dims
    C, K = case.conv_w.shape
    N = case.y.shape[0]
    cu = case.cu_seqlens
    n = len(cu) - 1
    cuc = [0]
    for a, b in zip(cu, cu[1:]):
        cuc.append(cuc[-1] + -(-(b - a) // kernels.DELTA_CHUNK))
    meta = to_device(torch.tensor(cu + cuc + list(range(n)), dtype=torch.int32), dev)
    seqs = meta.data_ptr() + 4 * (2 * n + 2)
    lib = load()
    ws = torch.empty(lib.lib.rk_gated_delta_workspace_bytes(cuc[-1], H), dtype=torch.uint8, device=dev)
    qkv, z, b, a = c.cols()
    q = torch.empty(N, H, dk, dtype=torch.float32, device=dev)
    k, v = torch.empty_like(q), torch.empty(N, H, dv, dtype=torch.float32, device=dev)
    beta, g = torch.empty(N, H, dtype=torch.float32, device=dev), torch.empty(N, H, dtype=torch.float32, device=dev)
    o = torch.empty(N, H, dv, dtype=torch.float32, device=dev)
    out = torch.empty(N * H, dv, dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    sp = lambda: torch.cuda.current_stream(dev).cuda_stream

    def front():      # conv tails are handed over in place each step; their values do not change the work
        lib.call("rk_deltanet_prefill_front", q.data_ptr(), k.data_ptr(), v.data_ptr(), beta.data_ptr(),
                 g.data_ptr(), qkv.data_ptr(), b.data_ptr(), a.data_ptr(), RK_F32, qkv.stride(0), c.conv.data_ptr(),
                 c.conv.stride(0), c.conv_w.data_ptr(), c.A_log.data_ptr(), c.dt_bias.data_ptr(), meta.data_ptr(),
                 seqs, n, N, H, dk, dv, K, sp())

    def norm():
        lib.call("rk_rms_norm_gated", out.data_ptr(), o.data_ptr(), z.data_ptr(), RK_F32, z.stride(0), H,
                 c.norm_w.data_ptr(), N * H, dv, case.eps, sp())

    def delta():
        lib.call("rk_gated_delta_chunked", o.data_ptr(), c.S.data_ptr(), c.S.stride(0), q.data_ptr(), k.data_ptr(),
                 v.data_ptr(), RK_F32, beta.data_ptr(), g.data_ptr(), meta.data_ptr(), meta.data_ptr() + 4 * (n + 1),
                 seqs, n, cuc[-1], H, dk, dv, ws.data_ptr(), ws.numel(), sp())

    def step():
        front()
        norm()

    def layer():
        front()
        delta()
        norm()

    for _ in range(args.warmup):
        layer()
    torch.cuda.synchronize()
    ms_front = graph_time(front, args.steps, stream)
    ms_norm = graph_time(norm, args.steps, stream)
    ms = graph_time(step, args.steps, stream)
    ms_layer = graph_time(layer, max(1, args.steps // 5), stream)
    fb, nb = case.front_bytes(), case.norm_bytes()
    gbs = fb / (ms_front * 1e-3) / 1e9
    log(f"[bench] lp: front {ms_front * 1e3:.1f} us ({gbs:.0f} GB/s, {gbs / HBM_PEAK_GBS:.1%}), norm "
        f"{ms_norm * 1e3:.1f} us ({nb / (ms_norm * 1e-3) / 1e9:.0f} GB/s), companions {ms * 1e3:.1f} us, whole layer "
        f"{ms_layer * 1e3:.1f} us")
    cpu = None
    if not args.no_cpu:
        from oracle import backend_ref, ops_ref
        torch.set_num_threads(cpu_threads())
        lo, hi = cu[0], cu[1]
        xq, xz, xb, xa = (t[lo:hi] for t in case.cols())
        o_cpu = torch.randn(hi - lo, H, dv, generator=torch.Generator().manual_seed(0))

        def cpu_run():
            backend_ref.linear_attention_front(xq, xb, xa, case.conv[0], case.conv_w, case.A_log, case.dt_bias,
                                               case.dims)
            ops_ref.rms_norm_gated(o_cpu.reshape(-1, dv), xz.reshape(-1, dv), case.norm_w, case.eps)
        t, calls, total = cpu_time(cpu_run, runs=3)
        cpu = {"value": (hi - lo) / t, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"segment 0 alone ({hi - lo} tokens): conv + split + l2norm + beta / g and the gated "
                         f"RMSNorm, median of {calls} calls ({total:.1f} s in all), {t * 1e3:.1f} ms per call"}
    return {
        "metric": "DeltaNet prefill companions tokens/s (config-4 batch) + achieved HBM GB/s (% of 8 TB/s), 1 GPU",
        "value": N / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (seeded)",
        "config": {"workload": "linear-attention prefill around the delta rule: 4 x 4096 packed tokens, fp32 in_proj "
                               "output, conv 4 over 6144 channels, 16 heads x 128, states in place",
                   "tokens": N, "front_bytes": fb, "norm_bytes": nb, "front_ms": ms_front, "norm_ms": ms_norm,
                   "layer_ms": ms_layer, "layer_tokens_per_s": N / (ms_layer * 1e-3)},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
                     "traffic": traffic_for("deltanet_prefill_front/lp"),
                     "kernel": "prefill_front_kernel + tail_handoff_kernel", "bytes_per_launch": fb,
                     "avg_ms": ms_front},
        "cpu_baseline": cpu,
    }


def bench_attn_prep(args, backend):
    """The decode attention layer at config 3 with its pre-processing: rk_attn_prep (q / k RMSNorm, partial RoPE,
    KV write of the 64 new tokens) + the paged decode with the fused gate. The prep kernel is also timed at the
    config-5 prefill size (N packed tokens, q / k / v written out), where it is bandwidth-bound."""
    import torch
    import workloads as wl
    from native import kernels
    dev = backend.device
    stream = torch.cuda.current_stream(dev)
    Hq, Hkv, d, rot, theta = wl.HQ, wl.HKV, wl.HEAD_DIM, 64, 1e7
    case = wl.c3_paged_decode()
    B, bs = case.q.shape[0], case.block_size
    gen = torch.Generator().manual_seed(12)
    y = torch.randn(B, (2 * Hq + 2 * Hkv) * d, generator=gen)
    qw, kw = 1 + 0.1 * torch.randn(d, generator=gen), 1 + 0.1 * torch.randn(d, generator=gen)
    pos = (case.lens - 1).to(torch.int32)
    last = pos.long()
    slots = case.tables.long().gather(1, (last // bs)[:, None])[:, 0] * bs + last % bs
    log(f"[bench] ap: copying inputs to {dev}")
    sets = []
    for i in range(args.sets):
        c = case.to(dev)
        if i:
            c.k_pool, c.v_pool = c.k_pool.clone(), c.v_pool.clone()
        sets.append(c)
    yd, qwd, kwd, posd, slotsd = y.to(dev), qw.to(dev), kw.to(dev), pos.to(dev), slots.to(dev)
    torch.cuda.synchronize()
    it = [0]

    def prep():
        c = sets[it[0] % len(sets)]
        return backend.attention_prep(yd, qwd, kwd, 1e-6, posd, theta, rot, (Hq, Hkv, d), c.k_pool, c.v_pool, slotsd)

    def layer():
        c = sets[it[0] % len(sets)]
        it[0] += 1
        q, gate = backend.attention_prep(yd, qwd, kwd, 1e-6, posd, theta, rot, (Hq, Hkv, d), c.k_pool, c.v_pool,
                                         slotsd)
        backend.paged_attention(q, c.k_pool, c.v_pool, c.tables, c.lens, bs, gate=gate)

    for _ in range(args.warmup):
        layer()
    torch.cuda.synchronize()
    ms_prep = graph_time(prep, args.steps, stream)
    ms = graph_time(layer, args.steps, stream)
    # prefill size: the config-5 packed tokens, q / k / v written out (the paged prefill writes the pool itself)
    c5 = wl.c5_prefill()
    N = c5.q.shape[0]
    yp = torch.randn(N, (2 * Hq + 2 * Hkv) * d, generator=gen).to(dev)
    posp = torch.randint(0, 16384, (N,), generator=gen, dtype=torch.int32).to(dev)
    ms_pf = graph_time(lambda: kernels.attn_prep(yp, qwd, kwd, 1e-6, posp, theta, rot, (Hq, Hkv, d)), args.steps,
                       stream)
    pf_bytes = N * (Hq + 2 * Hkv) * d * (4 + 4) + N * 4 + 2 * d * 4
    pf_gbs = pf_bytes / (ms_pf * 1e-3) / 1e9
    log(f"[bench] ap: prep {ms_prep * 1e3:.1f} us at B = {B}, prep + decode {ms * 1e3:.1f} us; prep at N = {N}: "
        f"{ms_pf * 1e3:.1f} us ({pf_gbs:.0f} GB/s, {pf_gbs / HBM_PEAK_GBS:.1%})")
    cpu = None
    if not args.no_cpu:
        from oracle import backend_ref
        torch.set_num_threads(cpu_threads())
        kp, vp = case.k_pool.clone(), case.v_pool.clone()
        blocks, offsets = (slots // bs), (slots % bs)

        def cpu_run():
            q, k, v, gate = backend_ref.attention_prep(y, qw, kw, 1e-6, pos, theta, rot, (Hq, Hkv, d))
            kp[blocks, offsets] = k.to(kp.dtype)
            vp[blocks, offsets] = v.to(vp.dtype)
            o = backend_ref.paged_attention(q, kp, vp, case.tables, case.lens, bs)
            backend_ref.gate(o.reshape(B, Hq * d), gate)
        t, calls, total = cpu_time(cpu_run)
        cpu = {"value": B / t, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"the full config-3 batch ({B} sequences): norms, RoPE, KV write, paged attention, gate; "
                         f"median of {calls} runs ({total:.1f} s in all), {t:.4f} s per batch"}
    return {
        "metric": "decode attention layer tokens/s @ batch 64 (q/k norm + RoPE + KV write + paged attention + gate), "
                  "1 GPU",
        "value": B / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded)",
        "config": {"workload": "config 3 decode batch with the layer's pre-processing: fp32 projection rows, "
                               "8/2 heads x 256, 64 rotary dims, theta 1e7, bf16 pool", "prep_ms": ms_prep,
                   "prefill_prep_tokens": N, "prefill_prep_ms": ms_pf, "prefill_prep_bytes": pf_bytes},
        "roofline": {"bound": "hbm", "achieved": pf_gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": pf_gbs / HBM_PEAK_GBS, "traffic": traffic_for("attn_prep/ap"),
                     "kernel": "attn_prep_kernel (at the config-5 prefill size)", "bytes_per_launch": pf_bytes,
                     "avg_ms": ms_pf},
        "cpu_baseline": cpu,
    }


QWEN35_2B = {"layers": 24, "linear_layers": 18, "hidden": 2048, "intermediate": 6144, "vocab": 248320,
             "in_proj": 8224, "qkvg": 5120}


def bench_linears(args, backend):
    """Every linear of one Qwen3.5-2B decode step at batch 8 (the reference's INT4 policy: INT4 layers, INT8 tied
    head; src/quant.py:115-121): per layer the mixer's input projection (DeltaNet in_proj [8224, 2048] on 18 layers,
    attention qkvg [5120, 2048] on 6) and output projection [2048, 2048], the MLP's gate_up [12288, 2048] and down
    [2048, 6144]; then the head [248320, 2048]. Weights are random codes / scales generated on the GPU (a bandwidth
    workload: the values do not change the work); one step = the 97 rk_linear_rows launches, in a HIP graph."""
    import torch
    from quant import QuantTensor
    dev = backend.device
    stream = torch.cuda.current_stream(dev)
    c = QWEN35_2B
    M, H, I = 8, c["hidden"], c["intermediate"]
    gen = torch.Generator(device=dev).manual_seed(14)

    def qt(N, K, scheme):
        if scheme == "int8":
            data = torch.randint(-127, 128, (N, K), generator=gen, device=dev, dtype=torch.int8)
        else:
            data = torch.randint(0, 256, (N, K // 2), generator=gen, device=dev, dtype=torch.uint8)
        scales = (torch.rand(N, K // 32, generator=gen, device=dev) * 1e-3 + 1e-4).to(torch.float16)
        mins = (torch.rand(N, K // 32, generator=gen, device=dev) * -0.01).to(torch.float16) if scheme == "int4" else None
        return QuantTensor(scheme, data, scales, (N, K), 32, mins)

    mats = []
    for i in range(c["layers"]):
        mixer_in = c["in_proj"] if i % 4 != 3 else c["qkvg"]       # 3 of every 4 layers are DeltaNet
        mats += [qt(mixer_in, H, "int4"), qt(H, H, "int4"), qt(2 * I, H, "int4"), qt(H, I, "int4")]
    mats.append(qt(c["vocab"], H, "int8"))
    wbytes = sum(m.nbytes for m in mats)
    xs = {K: torch.randn(M, K, generator=gen, device=dev) for K in (H, I)}
    outs = [torch.empty(M, m.shape[0], device=dev) for m in mats]
    from native import kernels
    torch.cuda.synchronize()

    def step():
        for m, o in zip(mats, outs):
            kernels.linear_rows(xs[m.shape[1]], m, out=o)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ms = graph_time(step, max(1, args.steps // 5), stream)
    head = mats[-1]
    # the head alone (skipped under --no-graph, the counter-collection mode, so that every dispatch is one of a step)
    ms_head = None if args.no_graph else graph_time(lambda: kernels.linear_rows(xs[H], head, out=outs[-1]),
                                                     args.steps, stream)
    io = sum(M * (m.shape[1] + m.shape[0]) * 4 for m in mats)
    gbs = (wbytes + io) / (ms * 1e-3) / 1e9
    head_gbs = head.nbytes / (ms_head * 1e-3) / 1e9 if ms_head else None
    head_note = f"; head alone {ms_head * 1e3:.1f} us ({head_gbs:.0f} GB/s)" if ms_head else ""
    log(f"[bench] mv: {ms * 1e3:.1f} us per step of {len(mats)} linears ({wbytes / 1e9:.2f} GB of weights, "
        f"{gbs:.0f} GB/s = {gbs / HBM_PEAK_GBS:.1%}){head_note}")
    cpu = None
    if not args.no_cpu:
        from oracle import quant_ref
        torch.set_num_threads(cpu_threads())
        layer = [m.to("cpu") for m in mats[:4]]
        xc = {K: v.cpu() for K, v in xs.items()}

        def cpu_run():
            for m in layer:
                quant_ref.linear(xc[m.shape[1]], quant_ref.dequantize(m.scheme, m.data, m.scales, m.mins))
        t, calls, total = cpu_time(cpu_run, runs=3)
        lbytes = sum(m.nbytes for m in layer)
        t_step = t * wbytes / lbytes
        cpu = {"value": M / t_step, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"one DeltaNet layer's 4 linears (dequantize + fp32 matmul, {lbytes / 1e6:.1f} MB of weights): "
                         f"median of {calls} calls ({total:.1f} s in all), {t * 1e3:.1f} ms, scaled by weight bytes to "
                         f"the step ({wbytes / lbytes:.1f}x)"}
    return {
        "metric": "decode-step linears tokens/s @ batch 8 (Qwen3.5-2B shapes, INT4 + INT8 head) + achieved HBM GB/s, "
                  "1 GPU",
        "value": M / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (random codes and scales)",
        "config": {"workload": "all 97 linears of a Qwen3.5-2B decode step at batch 8: INT4 (block 32) layers, INT8 "
                               "head, fp32 activations", "weight_bytes": wbytes, "head_ms": ms_head,
                   "head_gbs": head_gbs},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
                     "traffic": traffic_for("linear_rows/mv"), "kernel": "linear_rows_kernel (97 launches)",
                     "bytes_per_launch": (wbytes + io) / len(mats), "avg_ms": ms / len(mats)},
        "cpu_baseline": cpu,
    }


def bench_decode_step(args, backend):
    """A whole Qwen3.5-2B decode step at batch 8 through RocmBackend (INT4 weights, INT8 tied embedding / head, the
    reference's policy): the backend calls of Qwen3_5Model.decode_batch (src/models/qwen3_5.py:228-290) for 24 layers
    (18 DeltaNet, 6 gated attention over bf16 paged KV with histories of 512-4096 positions) plus the head. Weights
    are random codes / scales generated on the GPU (the values do not change the work); one step is captured in a
    HIP graph and replayed (the sequences are not advanced, so every replay does the same work)."""
    import dataclasses
    import torch
    import workloads as wl
    from backend.rocm import RocmBackend
    dev = backend.device
    stream = torch.cuda.current_stream(dev)
    be = RocmBackend(dev, scheme="int4")
    cfg, B = wl.QWEN35_2B, 8
    gen = torch.Generator().manual_seed(33)
    lens = torch.randint(512, 4097, (B,), generator=gen).tolist()
    log(f"[bench] ds: building the model and states on {dev}")
    w = wl.random_device_weights(cfg, "int4", dev, seed=31)
    st = wl.HybridDecodeState(cfg, lens, dev, seed=32)
    layout = st.layout()
    tokens = torch.randint(0, cfg.vocab, (B,), generator=gen).to(dev)
    torch.cuda.synchronize()

    def step():
        wl.hybrid_decode_step(be, w, st, tokens, layout)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ms = graph_time(step, max(1, args.steps // 5), stream)
    n_full = sum(cfg.is_full(i) for i in range(cfg.layers))
    wbytes = sum(t.nbytes if hasattr(t, "scheme") else 0 for t in w.values())
    kv_bytes = n_full * sum(L + 1 for L in lens) * cfg.Hkv * cfg.d * 2 * 2
    state_bytes = (cfg.layers - n_full) * B * (cfg.H * cfg.dk * cfg.dv * 4 * 2 + (cfg.conv_k - 1) * cfg.conv_dim * 4 * 2)
    step_bytes = wbytes + kv_bytes + state_bytes
    gbs = step_bytes / (ms * 1e-3) / 1e9
    log(f"[bench] ds: {ms * 1e3:.1f} us per decode step at batch {B} ({B / (ms * 1e-3):.0f} tokens/s); "
        f"{step_bytes / 1e9:.3f} GB per step (weights {wbytes / 1e9:.3f}, KV {kv_bytes / 1e6:.1f} MB, DeltaNet states "
        f"{state_bytes / 1e6:.1f} MB): {gbs:.0f} GB/s = {gbs / HBM_PEAK_GBS:.1%}")
    cpu = None
    if not args.no_cpu:
        # the oracle on the host: 4 of the 24 layers (3 DeltaNet + 1 attention) and the head, fp32 weights dequantized
        # once (the reference's CPU path holds fp32 weights), scaled to the 24 layers
        from oracle import decode_ref, ops_ref, quant_ref
        torch.set_num_threads(cpu_threads())
        cfg4 = dataclasses.replace(cfg, layers=4)
        names = [n for n in wl.hybrid_weight_shapes(cfg4)]

        def host(t):
            if hasattr(t, "scheme"):
                return quant_ref.dequantize(t.scheme, t.data.cpu(), t.scales.cpu(),
                                            t.mins.cpu() if t.mins is not None else None)
            return t.float().cpu()
        wh = {n: host(w[n]) for n in names}
        kh, vh = st.k.cpu(), st.v.cpu()
        Sh, convh = st.pool.S.cpu(), st.pool.conv.cpu()
        seq_index = torch.tensor([q.seq for q in st.seqs])
        lay = [t.cpu() for t in layout]
        tok = tokens.cpu()
        h = torch.randn(B, cfg.hidden, generator=gen)

        def run4():
            decode_ref.hybrid_decode_step(cfg4, wh, kh, vh, Sh, convh, seq_index, st.slot, *lay, tok)

        def head():
            quant_ref.linear(ops_ref.rms_norm(h, wh["norm.weight"], cfg.eps), wh["embed_tokens.weight"])
        t4, calls, total = cpu_time(run4)
        th, _, _ = cpu_time(head)
        t_step = th + (cfg.layers / 4) * (t4 - th)
        cpu = {"value": B / t_step, "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
               "sample": f"the oracle's decode step over 4 of the 24 layers (3 DeltaNet + 1 attention) plus "
                         f"embedding and head, fp32 weights: median {t4:.3f} s over {calls} calls ({total:.1f} s); "
                         f"head alone {th:.3f} s; step = head + 6 x (4 layers)"}
    return {
        "metric": "decode step tokens/s @ batch 8 (Qwen3.5-2B, INT4 weights, whole step: 24 layers + head) + "
                  "achieved HBM GB/s, 1 GPU",
        "value": B / (ms * 1e-3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": ms, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic (random INT4 / INT8 codes and scales, seeded states and KV)",
        "config": {"workload": "Qwen3.5-2B decode_batch at batch 8: 18 DeltaNet + 6 gated-attention layers, "
                               "INT4 linears (INT8 tied head), bf16 paged KV, histories U[512, 4096]",
                   "lens": lens, "step_bytes": step_bytes, "weight_bytes": wbytes, "kv_bytes": kv_bytes,
                   "state_bytes": state_bytes},
        "roofline": {"bound": "hbm", "achieved": gbs, "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": gbs / HBM_PEAK_GBS,
                     "traffic": None, "kernel": "the whole step (97 linears, 6 paged decodes, 18 DeltaNet steps, "
                                                "norms, SwiGLU)", "bytes_per_launch": step_bytes, "avg_ms": ms},
        "cpu_baseline": cpu,
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="all",
                    choices=["all", "c1", "c2", "c3", "c4", "c5", "c5f", "c5g", "ck", "lp", "ap", "wd", "mv", "ds"],
                    help="all (default): the config-3 headline record with configs 1, 2, 4, 5 as sub-records and "
                         "the measured access-pattern ceilings")
    ap.add_argument("--sets", type=int, default=2, help="distinct input copies rotated between steps")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-graph", action="store_true", help="time eager launches only (for counter collection)")
    ap.add_argument("--no-ceiling", action="store_true", help="skip the access-pattern probes")
    args = ap.parse_args()
    args.ceiling = not args.no_ceiling
    global USE_GRAPHS
    USE_GRAPHS = not args.no_graph
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}); "
              "the sequences of a batch shard across GPUs with no exchange, so N GPUs run N independent copies "
              "of this benchmark.", file=sys.stderr)
        return 2
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    import workloads as wl
    from backend.rocm import RocmBackend
    backend = RocmBackend("cuda:0")

    def c3():
        case = wl.c3_paged_decode()
        lens = case.lens
        config = {"workload": "config 3: paged GQA decode, batch 64, bf16 KV, fp32 accumulate, 8/2 heads x 256, "
                              "block 16, lengths U[128, 8192], pool 1.25 x positions, sigmoid gate",
                  "batch": 64, "total_positions": int(lens.sum()), "num_blocks": int(case.k_pool.shape[0]),
                  "kv_bytes": case.kv_bytes()}
        return bench_paged_decode(case, args, backend, "c3", config, plan_layers=PLAN_LAYERS)

    def c1():
        case = wl.c1_paged_decode()
        sets = args.sets
        args.sets = max(args.sets, 64)                 # 64 x 8 MiB pools > the 256 MB Infinity Cache
        ceiling, args.ceiling = args.ceiling, False
        rec = bench_paged_decode(case, args, backend, "c1",
                                 {"workload": "config 1: paged GQA decode, batch 1, fp32 KV, 512 positions"})
        args.sets, args.ceiling = sets, ceiling
        rec["metric"] = "decode attn tokens/s @ batch 1 (config 1 latency case), 1 GPU"
        rec["dtype"] = "f32"
        return rec

    if args.workload == "all":
        global CPU_SAMPLE_S
        rec = c3()
        torch.cuda.empty_cache()
        CPU_SAMPLE_S = 5.0                             # the sub-records' CPU samples: about 5 s each
        keep = ("metric", "value", "unit", "ms_per_step", "dtype", "config", "roofline", "cpu_baseline",
                "access_pattern_ceiling", "eager_ms_per_step")
        subs = {}
        for name, fn in (("c1", c1), ("c2", lambda: bench_deltanet(args, backend)),
                         ("c4", lambda: bench_chunked_delta(args, backend)),
                         ("c5", lambda: bench_prefill(args, backend)),
                         ("c5_fp32", lambda: bench_prefill(args, backend, fp32=True)),
                         ("c5_g7", lambda: bench_prefill(args, backend, g7=True))):
            sub = fn()
            subs[name] = {k: v for k, v in sub.items() if k in keep}
            torch.cuda.empty_cache()
        rec["configs"] = subs
    elif args.workload == "c3":
        rec = c3()
    elif args.workload == "c1":
        rec = c1()
    elif args.workload == "wd":
        case = wl.wd_windowed_decode()
        rec = bench_paged_decode(case, args, backend, "wd",
                                 {"workload": "sliding-window decode through the grouped pool: batch 64, 16/4 heads "
                                              "x 128, window 4096, bf16 KV in per-sequence rings, lengths "
                                              "U[128, 8192] (config 3's), sigmoid gate",
                                  "batch": 64, "window": wl.WD_WINDOW, "visible_positions":
                                      int(case.lens.long().clamp(max=wl.WD_WINDOW).sum()),
                                  "units": case.meta["units"], "kv_bytes": case.kv_bytes()})
        rec["metric"] = "sliding-window decode attn tokens/s @ batch 64 (grouped pool rings) + achieved HBM GB/s, 1 GPU"
    elif args.workload == "c5":
        rec = bench_prefill(args, backend)
    elif args.workload == "c5f":
        rec = bench_prefill(args, backend, fp32=True)
    elif args.workload == "c5g":
        rec = bench_prefill(args, backend, g7=True)
    elif args.workload == "ck":
        rec = bench_prefill(args, backend, chunk=True)
    elif args.workload == "c4":
        rec = bench_chunked_delta(args, backend)
    elif args.workload == "lp":
        rec = bench_linear_prefill(args, backend)
    elif args.workload == "ap":
        rec = bench_attn_prep(args, backend)
    elif args.workload == "mv":
        rec = bench_linears(args, backend)
    elif args.workload == "ds":
        rec = bench_decode_step(args, backend)
    else:
        rec = bench_deltanet(args, backend)
    print(json.dumps(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
