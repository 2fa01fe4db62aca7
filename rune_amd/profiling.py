"""Summaries of rocprofv3 output for the committed profiles.

``python -m rune_amd.profiling trace DIR --records E --calls K`` reads the
``*_kernel_stats.csv`` / ``*_kernel_trace.csv`` of a ``--kernel-trace --stats``
run and prints a markdown table per kernel plus the per-launch averages of the
kernel groups that bench.py reports (per-record GEMMs, per-record message
kernels).

``python -m rune_amd.profiling traffic FETCH_DIR WRITE_DIR --records E`` reads
the ``*_counter_collection.csv`` of two ``--pmc`` runs (FETCH_SIZE, WRITE_SIZE;
KiB per dispatch) and prints JSON with the HBM bytes per launch of each group.
Each counter is scaled by what it reads for the run's largest plain copy
kernel (``bench.py --copy-calibration``: 256 MiB read and 256 MiB written).
"""

from __future__ import annotations

import argparse
import collections
import csv
import json
import math
import os
import sys

COPY_BYTES = 256 << 20
COPY_KERNEL = "__amd_rocclr_copyBuffer"

# per-record message kernels of the MP and EQ blocks (bench.py "edge_kernels")
EDGE_KERNELS = ("k_eq_edge_nbr", "k_eq_edge_centre", "k_eq_aggregate", "k_eq_pair_dir",
                "k_eq_pair_grp", "k_eq_pair_grp_c", "k_eq_edge_adj", "k_eq_harmonic_backward", "k_edge_prep",
                "k_gather_f", "k_edge_rb_backward", "k_edge_direct", "k_mp_aggregate",
                "k_mp_edge_backward", "k_mp_neighbor_backward", "k_mp_aggregate_c",
                "k_mp_edge_backward_c", "k_mp_neighbor_backward_c")
# fused per-record MLP kernels (bench.py "edge_gemm", with the per-record GEMMs)
EDGE_GEMM_KERNELS = ("k_mp_edge_forward", "k_mp_edge_reverse")


def short_name(name):
    """Kernel name without namespaces and argument list."""
    base = name
    for prefix in ("void ", "rune::", "(anonymous namespace)::"):
        base = base.replace(prefix, "")
    return base.split("(")[0].strip()


def group_of(name, grid_threads, records):
    """bench.py group of one dispatch: GEMMs over at least `records` rows
    (64-row tiles of 256 threads) are per-record GEMMs."""
    base = short_name(name)
    if any(base == k or base.startswith(k + "<") for k in EDGE_GEMM_KERNELS):
        return "edge_gemm"
    if base.startswith("k_gemm<"):
        return "edge_gemm" if grid_threads >= 256 * math.ceil(records / 64) else None
    for k in EDGE_KERNELS:
        if base == k or base.startswith(k + "<"):
            return "edge_kernels"
    return None


def trace_summary(directory, records, calls):
    stats = list(csv.DictReader(open(_find(directory, "_kernel_stats.csv"))))
    trace = list(csv.DictReader(open(_find(directory, "_kernel_trace.csv"))))
    total = sum(float(r["TotalDurationNs"]) for r in stats)
    lines = ["| kernel | calls | avg us | total ms | % |", "|---|---:|---:|---:|---:|"]
    for r in stats:
        if float(r["Percentage"]) < 0.1:
            continue
        lines.append(f"| `{short_name(r['Name'])}` | {r['Calls']} | "
                     f"{float(r['AverageNs']) / 1e3:.1f} | "
                     f"{float(r['TotalDurationNs']) / 1e6:.2f} | {float(r['Percentage']):.1f} |")
    groups = collections.defaultdict(list)
    for r in trace:
        grid = int(r.get("Grid_Size", r.get("Grid_Size_X", 0)) or 0)
        g = group_of(r["Kernel_Name"], grid, records)
        if g:
            groups[g].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    lines += ["", "Kernel groups (launches of all traced calls):", "",
              "| group | launches | launches/call | avg us | ms/call |",
              "|---|---:|---:|---:|---:|"]
    for g, d in sorted(groups.items()):
        lines.append(f"| {g} | {len(d)} | {len(d) / calls:.1f} | {sum(d) / len(d) / 1e3:.1f} | "
                     f"{sum(d) / calls / 1e6:.2f} |")
    lines += ["", f"All kernels: {total / 1e6 / calls:.2f} ms per call ({calls} calls traced)."]
    return "\n".join(lines)


def _find(directory, suffix):
    for root, _, files in os.walk(directory):
        for f in files:
            if f.endswith(suffix):
                return os.path.join(root, f)
    raise SystemExit(f"no *{suffix} under {directory}")


def _counters(path, counter):
    """{dispatch id: (kernel name, grid threads, value summed over instances)}."""
    out = {}
    for r in csv.DictReader(open(path)):
        if r["Counter_Name"] != counter:
            continue
        d = int(r["Dispatch_Id"])
        name, grid, v = out.get(d, (r["Kernel_Name"], int(r["Grid_Size"]), 0.0))
        out[d] = (name, grid, v + float(r["Counter_Value"]))
    return out


def traffic(fetch_dir, write_dir, records):
    fetch = _counters(_find(fetch_dir, "_counter_collection.csv"), "FETCH_SIZE")
    write = _counters(_find(write_dir, "_counter_collection.csv"), "WRITE_SIZE")

    def calibration(counts):
        copies = [v for (n, _, v) in counts.values() if short_name(n) == COPY_KERNEL]
        if not copies:
            raise SystemExit("no copy kernel in the run (use bench.py --copy-calibration)")
        return COPY_BYTES / (max(copies) * 1024.0)

    ff, fw = calibration(fetch), calibration(write)
    groups = collections.defaultdict(lambda: [0.0, 0.0, 0])
    kernels = collections.defaultdict(lambda: [0.0, 0.0, 0])
    for counts, slot in ((fetch, 0), (write, 1)):
        for name, grid, v in counts.values():
            b = v * 1024.0 * (ff if slot == 0 else fw)
            k = kernels[short_name(name)]
            k[slot] += b
            k[2] += slot == 0
            g = group_of(name, grid, records)
            if g:
                groups[g][slot] += b
                if slot == 0:
                    groups[g][2] += 1
    out = {"copy_calibration": {"fetch_factor": round(ff, 4), "write_factor": round(fw, 4),
                                "copy_bytes": COPY_BYTES},
           "groups": {}}
    for g, (fb, wb, n) in groups.items():
        out["groups"][g] = {"launches": n, "fetch_bytes_per_launch": int(fb / n),
                            "write_bytes_per_launch": int(wb / n),
                            "bytes_per_launch": int((fb + wb) / n)}
    # every kernel moving at least 1 MB per launch, largest first
    out["kernels"] = {}
    for name, (fb, wb, n) in sorted(kernels.items(), key=lambda kv: -(kv[1][0] + kv[1][1])):
        if n and (fb + wb) / n >= 1e6 and name != COPY_KERNEL:
            out["kernels"][name] = {"launches": n, "fetch_bytes_per_launch": int(fb / n),
                                    "write_bytes_per_launch": int(wb / n)}
    return out


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("dir")
    t.add_argument("--records", type=int, required=True)
    t.add_argument("--calls", type=int, required=True)
    c = sub.add_parser("traffic")
    c.add_argument("fetch_dir")
    c.add_argument("write_dir")
    c.add_argument("--records", type=int, required=True)
    args = ap.parse_args(argv)
    if args.cmd == "trace":
        print(trace_summary(args.dir, args.records, args.calls))
    else:
        print(json.dumps(traffic(args.fetch_dir, args.write_dir, args.records), indent=1))


if __name__ == "__main__":
    sys.exit(main())
