"""Helpers behind the rocprofv3 summaries under profiles/: a copy kernel of known size for calibrating the HBM traffic
counters, and converters from rocprofv3 CSV output to the short text summaries and profiles/traffic.json.

  python metal-inference-engine_amd/profiling.py copy [--mib N]
      one fp32 elementwise copy (torch.mul(x, 1, out=y)) of N MiB, the known-size kernel: under rocprofv3 --pmc its
      FETCH_SIZE / WRITE_SIZE readings give the scale between the counters and bytes actually moved.
  python metal-inference-engine_amd/profiling.py stats <kernel_stats.csv> <out.txt> <command...>
      kernel-trace statistics (--kernel-trace --stats --output-format csv) as a text table, with the command.
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


if __name__ == "__main__":
    cmd = sys.argv[1]
    if cmd == "copy":
        copy_kernel(int(sys.argv[sys.argv.index("--mib") + 1]) if "--mib" in sys.argv else 1024)
    elif cmd == "stats":
        stats_table(sys.argv[2], sys.argv[3], " ".join(sys.argv[4:]))
    elif cmd == "traffic":
        traffic(sys.argv[2], int(sys.argv[3]), sys.argv[4], sys.argv[5], sys.argv[6:])
    else:
        raise SystemExit(__doc__)
