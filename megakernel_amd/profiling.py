"""Summaries of rocprofv3 output for the decode kernel.

Two jobs, both on files rocprofv3 wrote (``--output-format csv``):

* ``stats``: turn ``*_kernel_stats.csv`` into a short text table (the form
  kept under ``profiles/``), prefixed with the command that produced it;
* ``launches``: per-launch durations from ``*_kernel_trace.csv``, grouped by
  kernel and grid size (the operator microbench launches each op kernel both
  with many instances and with one);
* ``traffic``: combine four ``--pmc`` runs -- FETCH_SIZE and WRITE_SIZE of the
  decode launch, and the same two counters of a plain device copy of known
  size -- into HBM bytes per decode launch.  Each counter is scaled by
  (known copy bytes / what that counter read for the copy), which absorbs the
  counter's unit and any per-XCD aggregation quirk.  Written as JSON for
  ``bench.py`` (``roofline.traffic``).

Usage:
  python -m megakernel_amd.profiling stats STATS.csv --command "..." -o OUT.txt
  python -m megakernel_amd.profiling launches TRACE.csv --match mk::ops:: --command "..." -o OUT.txt
  python -m megakernel_amd.profiling traffic --decode-fetch A.csv --decode-write B.csv \
      --copy-fetch C.csv --copy-write D.csv --copy-bytes N --ctx 1024 --tokens 256 \
      --algorithmic-bytes X -o profiles/decode_traffic.json
"""
from __future__ import annotations

import argparse
import csv
import json
import statistics
import sys

DECODE_KERNEL = "decode_kernel"


def _rows(path: str) -> list[dict]:
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def kernel_stats(path: str) -> list[dict]:
    """Rows of a rocprofv3 kernel_stats.csv as dicts with numeric fields."""
    out = []
    for r in _rows(path):
        out.append({"name": r.get("Name", ""), "calls": int(r.get("Calls", 0)),
                    "total_ns": float(r.get("TotalDurationNs", 0)), "avg_ns": float(r.get("AverageNs", 0)),
                    "min_ns": float(r.get("MinNs", 0)), "max_ns": float(r.get("MaxNs", 0)),
                    "pct": float(r.get("Percentage", 0))})
    return out


def counter_values(path: str, counter: str, kernel_substr: str) -> list[float]:
    """Per-dispatch values of one counter for kernels whose name contains
    kernel_substr (summed over rows of the same dispatch)."""
    acc: dict[str, float] = {}
    for r in _rows(path):
        if r.get("Counter_Name") != counter or kernel_substr not in r.get("Kernel_Name", ""):
            continue
        key = r.get("Dispatch_Id") or r.get("Correlation_Id") or str(len(acc))
        acc[key] = acc.get(key, 0.0) + float(r["Counter_Value"])
    return [acc[k] for k in sorted(acc, key=lambda s: int(s) if s.isdigit() else 0)]


def stats_text(path: str, cmd: str, top: int = 8) -> str:
    rows = sorted(kernel_stats(path), key=lambda r: -r["total_ns"])[:top]
    lines = [f"# command: {cmd}", "",
             f"{'kernel':60s} {'calls':>6s} {'avg us':>10s} {'min us':>10s} {'max us':>10s} {'% time':>7s}"]
    for r in rows:
        name = r["name"] if len(r["name"]) <= 60 else r["name"][:57] + "..."
        lines.append(f"{name:60s} {r['calls']:6d} {r['avg_ns'] / 1e3:10.1f} {r['min_ns'] / 1e3:10.1f} "
                     f"{r['max_ns'] / 1e3:10.1f} {r['pct']:7.2f}")
    return "\n".join(lines) + "\n"


def launch_text(path: str, cmd: str, substr: str) -> str:
    """Per (kernel, grid size) launch durations from a rocprofv3
    kernel_trace.csv, for kernels whose name contains substr: launches of one
    kernel with different work (e.g. many instances vs one) have different
    grids, so each group is one kind of launch."""
    groups: dict[tuple[str, int], list[float]] = {}
    for r in _rows(path):
        name = r.get("Kernel_Name", "")
        if substr not in name:
            continue
        grid = int(r.get("Grid_Size_X", 0)) // max(1, int(r.get("Workgroup_Size_X", 1)))
        dur = (float(r["End_Timestamp"]) - float(r["Start_Timestamp"])) / 1e3
        groups.setdefault((name, grid), []).append(dur)
    lines = [f"# command: {cmd}", f"# launches of kernels matching '{substr}', grouped by grid (workgroups)", "",
             f"{'kernel':60s} {'grid':>6s} {'calls':>6s} {'median us':>10s} {'min us':>10s} {'max us':>10s}"]
    for (name, grid), d in sorted(groups.items(), key=lambda kv: (kv[0][0], -kv[0][1])):
        short = name if len(name) <= 60 else name[:57] + "..."
        lines.append(f"{short:60s} {grid:6d} {len(d):6d} {statistics.median(d):10.2f} {min(d):10.2f} "
                     f"{max(d):10.2f}")
    return "\n".join(lines) + "\n"


def traffic(args) -> dict:
    dec_f = counter_values(args.decode_fetch, "FETCH_SIZE", DECODE_KERNEL)
    dec_w = counter_values(args.decode_write, "WRITE_SIZE", DECODE_KERNEL)
    cp_f = counter_values(args.copy_fetch, "FETCH_SIZE", args.copy_kernel)
    cp_w = counter_values(args.copy_write, "WRITE_SIZE", args.copy_kernel)
    if not (dec_f and dec_w and cp_f and cp_w):
        raise SystemExit("missing counter rows (decode fetch/write, copy fetch/write): "
                         f"{len(dec_f)} {len(dec_w)} {len(cp_f)} {len(cp_w)}")
    # the timed launches are the largest decode dispatches (warm-up launches
    # of the same length are included; shorter ones are not)
    f_launch = max(dec_f)
    w_launch = max(dec_w)
    scale_f = args.copy_bytes / statistics.median(cp_f)
    scale_w = args.copy_bytes / statistics.median(cp_w)
    fetch_b = f_launch * scale_f
    write_b = w_launch * scale_w
    return {
        "ctx": args.ctx, "tokens": args.tokens,
        "decode_fetch_counter_per_launch": f_launch, "decode_write_counter_per_launch": w_launch,
        "copy_bytes": args.copy_bytes,
        "copy_fetch_counter": statistics.median(cp_f), "copy_write_counter": statistics.median(cp_w),
        "fetch_scale_bytes_per_unit": scale_f, "write_scale_bytes_per_unit": scale_w,
        "fetch_bytes_per_launch": fetch_b, "write_bytes_per_launch": write_b,
        "hbm_bytes_per_launch": fetch_b + write_b,
        "algorithmic_bytes_per_launch": args.algorithmic_bytes,
        "traffic_over_algorithmic": (fetch_b + write_b) / args.algorithmic_bytes if args.algorithmic_bytes else None,
    }


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="what", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("--command", required=True, help="the command that produced the csv")
    s.add_argument("-o", "--out")
    s.add_argument("--top", type=int, default=8, help="kernels listed")
    ln = sub.add_parser("launches")
    ln.add_argument("csv", help="kernel_trace.csv")
    ln.add_argument("--command", required=True)
    ln.add_argument("--match", required=True, help="substring of the kernel names to list")
    ln.add_argument("-o", "--out")
    t = sub.add_parser("traffic")
    for k in ("decode-fetch", "decode-write", "copy-fetch", "copy-write"):
        t.add_argument(f"--{k}", required=True)
    t.add_argument("--copy-kernel", default="", help="substring of the copy kernel's name")
    t.add_argument("--copy-bytes", type=float, required=True, help="bytes read (= bytes written) by one copy")
    t.add_argument("--ctx", type=int, required=True)
    t.add_argument("--tokens", type=int, required=True)
    t.add_argument("--algorithmic-bytes", type=float, default=0.0)
    t.add_argument("-o", "--out", required=True)
    a = ap.parse_args(argv)
    if a.what == "stats":
        txt = stats_text(a.csv, a.command, a.top)
        if a.out:
            with open(a.out, "w") as f:
                f.write(txt)
        sys.stdout.write(txt)
    elif a.what == "launches":
        txt = launch_text(a.csv, a.command, a.match)
        if a.out:
            with open(a.out, "w") as f:
                f.write(txt)
        sys.stdout.write(txt)
    else:
        res = traffic(a)
        with open(a.out, "w") as f:
            json.dump(res, f, indent=1)
        print(json.dumps(res, indent=1))


if __name__ == "__main__":
    main()
