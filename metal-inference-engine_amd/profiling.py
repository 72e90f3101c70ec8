"""Helpers behind the rocprofv3 summaries under profiles/: a copy kernel of known size for calibrating the HBM traffic
counters, and converters from rocprofv3 CSV output to the short text summaries and profiles/traffic.json.

  python metal-inference-engine_amd/profiling.py copy [--mib N]
      one fp32 elementwise copy (torch.mul(x, 1, out=y)) of N MiB, the known-size kernel: under rocprofv3 --pmc its
      FETCH_SIZE / WRITE_SIZE readings give the scale between the counters and bytes actually moved.
  python metal-inference-engine_amd/profiling.py stats <kernel_stats.csv> <out.txt> <command...>
      kernel-trace statistics (--kernel-trace --stats --output-format csv) as a text table, with the command.
  python metal-inference-engine_amd/profiling.py table <traffic.json> <out.txt>
      the human-readable summary of traffic.json (profiles/hbm_traffic.txt), regenerated from it so the two agree.
  python metal-inference-engine_amd/profiling.py traffic <out.json> <copy_mib> <copy_fetch.csv> <copy_write.csv>
          <name>=<pattern>:<fetch.csv>:<write.csv> ...
      HBM bytes per launch of the kernels whose names contain <pattern> (summed over kernels when the pattern
      matches several per step; averaged over all matching dispatches when it starts with '*'), from one FETCH_SIZE pass and one WRITE_SIZE pass (KiB per dispatch), each scaled
      by what the same counter reads for the copy kernel. Entries for other names already in <out.json> are kept.
"""
import csv
import json
import statistics
import sys
from collections import defaultdict


def copy_kernel(mib: int) -> None:
    import torch
    n = mib * (1 << 20) // 4
    x = torch.ones(n, device="cuda")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    torch.mul(x, 1.0, out=y)
    torch.cuda.synchronize()
    print(f"copy kernel: read {mib} MiB, wrote {mib} MiB", flush=True)


def stats_table(stats_csv: str, out_txt: str, command: str) -> None:
    rows = list(csv.DictReader(open(stats_csv)))
    lines = [f"# rocprofv3 kernel-trace statistics", f"# command: {command}", "",
             f"{'kernel':<72} {'calls':>6} {'avg_us':>9} {'min_us':>9} {'max_us':>9} {'pct':>6}"]
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        name = r["Name"].replace("rk::(anonymous namespace)::", "")
        lines.append(f"{name[:72]:<72} {int(r['Calls']):>6} {float(r['AverageNs']) / 1e3:>9.2f} "
                     f"{float(r['MinNs']) / 1e3:>9.2f} {float(r['MaxNs']) / 1e3:>9.2f} "
                     f"{float(r['Percentage']):>6.2f}")
    open(out_txt, "w").write("\n".join(lines) + "\n")


def _per_dispatch(counter_csv: str, pattern: str, counter: str) -> tuple[float, int]:
    """Median over steps of the counter summed over the dispatches of one step (kernels matching pattern), KiB.
    A pattern starting with '*' instead averages over every matching dispatch (a step of many launches of one
    kernel family over different shapes: the mean bytes per launch)."""
    if pattern.startswith("*"):
        vals = [float(r["Counter_Value"]) for r in csv.DictReader(open(counter_csv))
                if r["Counter_Name"] == counter and pattern[1:] in r["Kernel_Name"]]
        if not vals:
            raise SystemExit(f"{counter_csv}: no {counter} rows for kernels matching {pattern[1:]!r}")
        return sum(vals) / len(vals), len(vals)
    by_kernel = defaultdict(list)
    for r in csv.DictReader(open(counter_csv)):
        if r["Counter_Name"] == counter and pattern in r["Kernel_Name"]:
            by_kernel[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    if not by_kernel:
        raise SystemExit(f"{counter_csv}: no {counter} rows for kernels matching {pattern!r}")
    total = sum(statistics.median(v) for v in by_kernel.values())
    return total, min(len(v) for v in by_kernel.values())


def traffic(out_json: str, copy_mib: int, copy_fetch: str, copy_write: str, specs: list[str]) -> None:
    nbytes = copy_mib * (1 << 20)
    cf, _ = _per_dispatch(copy_fetch, "MulFunctor", "FETCH_SIZE")      # the copy, not the fill that made its input
    cw, _ = _per_dispatch(copy_write, "MulFunctor", "WRITE_SIZE")
    f_scale, w_scale = nbytes / (cf * 1024), nbytes / (cw * 1024)
    # entries of other workloads already in the file are kept (each was scaled by the calibration of its own run)
    try:
        out = json.loads(open(out_json).read())
    except FileNotFoundError:
        out = {}
    out["_calibration"] = {"copy_bytes": nbytes, "fetch_kib": cf, "write_kib": cw, "fetch_scale": f_scale,
                           "write_scale": w_scale}
    for spec in specs:
        name, rest = spec.split("=", 1)
        pattern, fetch_csv, write_csv = rest.split(":")
        f, nf = _per_dispatch(fetch_csv, pattern, "FETCH_SIZE")
        w, nw = _per_dispatch(write_csv, pattern, "WRITE_SIZE")
        fb, wb = f * 1024 * f_scale, w * 1024 * w_scale
        out[name] = {"kernels": pattern.lstrip("*"), "fetch_bytes": fb, "write_bytes": wb, "bytes_per_launch": fb + wb,
                     "dispatches": min(nf, nw)}
    open(out_json, "w").write(json.dumps(out, indent=1) + "\n")


# algorithmic bytes per launch (MB) of each traffic.json entry and what makes up the measured bytes; the
# algorithmic figures are the workloads' own counts (workloads.py), printed beside the counters
ALGORITHMIC = {
    "paged_decode_split/c3": (544.1, "K/V 543.6 + q, tables, lens; partials written"),
    "paged_decode_merge/c3": (None, "partials read, out written"),
    "paged_decode_split/c1": (2.1, "fp32 K/V of 512 positions + q, table; partials written"),
    "paged_decode_merge/c1": (None, ""),
    "deltanet_step/c2": (18.4, "state 2 x 8.4 + conv tails, inputs, out"),
    "chunked_delta/c4": (346.0, "q, k, v bf16, beta, g, o fp32, final states; + the T / coefficient workspace"),
    "delta_chunk_scan/c4": (None, "the scan alone"),
    "prefill_attention/c5": (356.7, "bf16 operands; K / V re-read once per 32-query block"),
    "prefill_attention_f32/c5f": (631.7, "fp32 pool and q; K / V re-read once per 32-query block; balance-split "
                                         "pieces write partial records"),
    "prefill_attention_b16/c5g": (119.9, "14/2 x 64 heads: K / V re-read once per 32-query block and head chunk"),
    "deltanet_prefill_front/lp": (810.2, "qkv / b / a columns + K-1 rows per 32-token run; q, k, v, beta, g written"),
    "rms_norm_gated/lp": (402.7, "x and z read, out written once"),
    "linear_rows/mv": (14.8, "mean of the step's 97 launches; x re-read per row group, K-split partials"),
    "attn_prep/ap": (245.4, "projection rows read, q / k / v written (config-5 token count)"),
    "paged_decode_split/wd": (406.0, "the window's K/V"),
}


def traffic_table(traffic_json: str, out_txt: str) -> None:
    data = json.loads(open(traffic_json).read())
    cal = data.get("_calibration", {})
    lines = [
        "# HBM bytes per launch from rocprofv3 counters (FETCH_SIZE and WRITE_SIZE, one counter per run), per kernel",
        "# and workload. Generated from profiles/traffic.json (which bench.py reads for its roofline \"traffic\"",
        "# field) by: python3 metal-inference-engine_amd/profiling.py table profiles/traffic.json profiles/hbm_traffic.txt",
        "#",
        "# calibration (the known-size kernel: one fp32 elementwise copy of 1 GiB, torch.mul(x, 1, out=y)):",
        "#   cd /tmp && export TMPDIR=/tmp && rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir> -o copy -- "
        "python3 /root/repo/metal-inference-engine_amd/profiling.py copy --mib 1024",
        "#   (the same with --pmc WRITE_SIZE)",
        f"#   FETCH_SIZE read {cal.get('fetch_kib', 0):,.0f} KiB for {cal.get('copy_bytes', 0) / 1024:,.0f} KiB read"
        f"  -> fetch scale {cal.get('fetch_scale', 0):.3f}",
        f"#   WRITE_SIZE read {cal.get('write_kib', 0):,.0f} KiB for {cal.get('copy_bytes', 0) / 1024:,.0f} KiB "
        f"written -> write scale {cal.get('write_scale', 0):.3f}",
        "#",
        "# per workload w (eager launches, no graph, so every dispatch is counted):",
        "#   cd /tmp && export TMPDIR=/tmp && rocprofv3 --pmc FETCH_SIZE --output-format csv -d <dir> -o w -- python3 "
        "/root/repo/bench.py --workload w --steps 3 --warmup 1 --no-cpu --no-graph",
        "#   (the same with --pmc WRITE_SIZE); then python3 metal-inference-engine_amd/profiling.py traffic "
        "profiles/traffic.json 1024 <copy csvs> <name>=<kernel pattern>:<fetch csv>:<write csv> ...",
        "#",
        f"# {'entry':<28} {'kernels':<36} {'fetch MB':>9} {'write MB':>9} {'total MB':>9} {'algo MB':>8}  note",
    ]
    for name, e in data.items():
        if name.startswith("_"):
            continue
        algo, note = ALGORITHMIC.get(name, (None, ""))
        lines.append(f"  {name:<28} {e['kernels'][:36]:<36} {e['fetch_bytes'] / 1e6:>9.1f} {e['write_bytes'] / 1e6:>9.1f}"
                     f" {e['bytes_per_launch'] / 1e6:>9.1f} {('%.1f' % algo) if algo else '-':>8}  {note}")
    open(out_txt, "w").write("\n".join(lines) + "\n")


if __name__ == "__main__":
    cmd = sys.argv[1]
    if cmd == "copy":
        copy_kernel(int(sys.argv[sys.argv.index("--mib") + 1]) if "--mib" in sys.argv else 1024)
    elif cmd == "stats":
        stats_table(sys.argv[2], sys.argv[3], " ".join(sys.argv[4:]))
    elif cmd == "table":
        traffic_table(sys.argv[2], sys.argv[3])
    elif cmd == "traffic":
        traffic(sys.argv[2], int(sys.argv[3]), sys.argv[4], sys.argv[5], sys.argv[6:])
    else:
        raise SystemExit(__doc__)
