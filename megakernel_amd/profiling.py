"""Summaries of rocprofv3 output for the decode kernel.

Two jobs, both on files rocprofv3 wrote (``--output-format csv``):

* ``stats``: turn ``*_kernel_stats.csv`` into a short text table (the form
  kept under ``profiles/``), prefixed with the command that produced it;
* ``launches``: per-launch durations from ``*_kernel_trace.csv``, grouped by
  kernel and grid size (the operator microbench launches each op kernel both
  with many instances and with one);
* ``counters``: per-launch and per-token totals of other ``--pmc`` counters
  (L2 hits / misses, wave waits, instruction cache) of the decode launch, as
  a markdown table with the derived ratios;
* ``traffic``: combine four ``--pmc`` runs -- FETCH_SIZE and WRITE_SIZE of the
  decode launch, and the same two counters of a plain device copy of known
  size -- into HBM bytes per decode launch.  Each counter is scaled by
  (known copy bytes / what that counter read for the copy), which absorbs the
  counter's unit and any per-XCD aggregation quirk.  Written as JSON for
  ``bench.py`` (``roofline.traffic``);
* ``step-traffic``: the same scaling for work that runs as many kernels --
  a batched decode step, a prefill -- summing FETCH_SIZE / WRITE_SIZE over
  every dispatch whose name matches ``--kernels`` and dividing by the number
  of dispatches of ``--unit-kernel`` (one per step or per prompt).  The
  bench line of the profiled run supplies the algorithmic bytes per unit and
  the workload key that ``bench.py`` matches before it reports the traffic.

Usage:
  python -m megakernel_amd.profiling stats STATS.csv --command "..." -o OUT.txt
  python -m megakernel_amd.profiling launches TRACE.csv --match mk::ops:: --command "..." -o OUT.txt
  python -m megakernel_amd.profiling counters A.csv [B.csv ...] --tokens 256 --command "..." -o OUT.md
  python -m megakernel_amd.profiling traffic --decode-fetch A.csv --decode-write B.csv \
      --copy-fetch C.csv --copy-write D.csv --copy-bytes N --ctx 1024 --tokens 256 \
      --algorithmic-bytes X -o profiles/decode_traffic.json
  python -m megakernel_amd.profiling step-traffic --fetch A.csv --write B.csv --copy-fetch C.csv \
      --copy-write D.csv --copy-bytes N --kernels mk::batch:: --unit-kernel bk_tok \
      --bench-json BENCH.json -o profiles/batch16_traffic.json
"""
from __future__ import annotations

import argparse
import csv
import json
import statistics
import sys

DECODE_KERNELS = ("decode_kernel", "decode_cls_kernel")  # spread / class-specialised decode kernels


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


def counter_values(path: str, counter: str, kernel_substr) -> list[float]:
    """Per-dispatch values of one counter for kernels whose name contains
    kernel_substr (a string or a tuple of alternatives; summed over rows of the
    same dispatch)."""
    subs = (kernel_substr,) if isinstance(kernel_substr, str) else tuple(kernel_substr)
    acc: dict[str, float] = {}
    for r in _rows(path):
        if r.get("Counter_Name") != counter or not any(k in r.get("Kernel_Name", "") for k in subs):
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
    dec_f = counter_values(args.decode_fetch, "FETCH_SIZE", DECODE_KERNELS)
    dec_w = counter_values(args.decode_write, "WRITE_SIZE", DECODE_KERNELS)
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
        "hbm_bytes_per_token": (fetch_b + write_b) / args.tokens,
        "algorithmic_bytes_per_launch": args.algorithmic_bytes,
        "traffic_over_algorithmic": (fetch_b + write_b) / args.algorithmic_bytes if args.algorithmic_bytes else None,
    }


def step_traffic(args) -> dict:
    """HBM bytes per unit (step / prompt) summed over many kernels' dispatches."""
    f = counter_values(args.fetch, "FETCH_SIZE", args.kernels)
    w = counter_values(args.write, "WRITE_SIZE", args.kernels)
    nf = len(counter_values(args.fetch, "FETCH_SIZE", args.unit_kernel))
    nw = len(counter_values(args.write, "WRITE_SIZE", args.unit_kernel))
    cp_f = counter_values(args.copy_fetch, "FETCH_SIZE", args.copy_kernel)
    cp_w = counter_values(args.copy_write, "WRITE_SIZE", args.copy_kernel)
    if not (f and w and nf and nw and cp_f and cp_w) or nf != nw:
        raise SystemExit("missing counter rows (fetch / write dispatches, units, copy fetch / write): "
                         f"{len(f)} {len(w)} {nf} {nw} {len(cp_f)} {len(cp_w)}")
    bench = None
    with open(args.bench_json) as fh:  # the bench line among whatever else the run printed
        for line in fh:
            if line.startswith("{") and '"traffic_key"' in line:
                bench = json.loads(line)
    if bench is None:
        raise SystemExit(f"no bench line with a traffic_key in {args.bench_json}")
    alg = float(bench["algorithmic_bytes_per_unit"])
    scale_f = args.copy_bytes / statistics.median(cp_f)
    scale_w = args.copy_bytes / statistics.median(cp_w)
    fetch_b = sum(f) / nf * scale_f
    write_b = sum(w) / nw * scale_w
    return {
        "traffic_key": bench["traffic_key"], "units": nf, "dispatches": len(f),
        "kernels": args.kernels, "unit_kernel": args.unit_kernel,
        "copy_bytes": args.copy_bytes,
        "copy_fetch_counter": statistics.median(cp_f), "copy_write_counter": statistics.median(cp_w),
        "fetch_scale_bytes_per_unit": scale_f, "write_scale_bytes_per_unit": scale_w,
        "fetch_bytes_per_unit": fetch_b, "write_bytes_per_unit": write_b,
        "hbm_bytes_per_unit": fetch_b + write_b,
        "algorithmic_bytes_per_unit": alg,
        "traffic_over_algorithmic": (fetch_b + write_b) / alg,
    }


# derived quantities of the counter summary: (label, numerator, denominator)
DERIVED = [
    ("L2 (TCC) hit rate", ("TCC_HIT_sum",), ("TCC_HIT_sum", "TCC_MISS_sum")),
    ("wave-cycles waiting on anything / wave-cycles", ("SQ_WAIT_ANY",), ("SQ_WAVE_CYCLES",)),
    ("wave-cycles waiting for issue / wave-cycles", ("SQ_WAIT_INST_ANY",), ("SQ_WAVE_CYCLES",)),
    ("average L2 -> memory read latency (TCC cycles)", ("TCC_EA0_RDREQ_LEVEL_sum",), ("TCC_EA0_RDREQ_sum",)),
    ("memory reads counted as DRAM requests / all memory reads", ("TCC_EA0_RDREQ_DRAM_sum",), ("TCC_EA0_RDREQ_sum",)),
    ("instruction-cache hit rate", ("SQC_ICACHE_HITS",), ("SQC_ICACHE_HITS", "SQC_ICACHE_MISSES")),
]


def counters_text(paths: list[str], cmd: str, tokens: int) -> str:
    """Per-launch totals of every counter in the given --pmc csv files for the
    largest decode dispatch, per token, and the derived ratios above."""
    vals: dict[str, float] = {}
    for p in paths:
        names = sorted({r["Counter_Name"] for r in _rows(p)})
        for c in names:
            v = counter_values(p, c, DECODE_KERNELS)
            if v:
                vals[c] = max(v)
    lines = [f"# command: {cmd}", "", f"decode launch of {tokens} tokens (largest decode dispatch of each pass)", "",
             "| counter | per launch | per token |", "|---|---|---|"]
    for c in sorted(vals):
        lines.append(f"| {c} | {vals[c]:,.0f} | {vals[c] / tokens:,.1f} |")
    lines += ["", "| derived | value |", "|---|---|"]
    for label, num, den in DERIVED:
        if all(k in vals for k in num + den):
            n, d = sum(vals[k] for k in num), sum(vals[k] for k in den)
            lines.append(f"| {label} | {n / d:.4f} |")
    return "\n".join(lines) + "\n"


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
    st = sub.add_parser("step-traffic")
    for k in ("fetch", "write", "copy-fetch", "copy-write", "bench-json"):
        st.add_argument(f"--{k}", required=True)
    st.add_argument("--copy-kernel", default="", help="substring of the copy kernel's name")
    st.add_argument("--copy-bytes", type=float, required=True, help="bytes read (= bytes written) by one copy")
    st.add_argument("--kernels", required=True, help="substring of the kernels whose counters are summed")
    st.add_argument("--unit-kernel", required=True, help="substring of the kernel dispatched once per unit")
    st.add_argument("-o", "--out", required=True)
    c = sub.add_parser("counters")
    c.add_argument("csv", nargs="+", help="counter_collection.csv of one or more --pmc passes")
    c.add_argument("--command", required=True, help="the commands that produced the csv files")
    c.add_argument("--tokens", type=int, required=True)
    c.add_argument("-o", "--out")
    a = ap.parse_args(argv)
    if a.what == "stats":
        txt = stats_text(a.csv, a.command, a.top)
        if a.out:
            with open(a.out, "w") as f:
                f.write(txt)
        sys.stdout.write(txt)
    elif a.what == "counters":
        txt = counters_text(a.csv, a.command, a.tokens)
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
        res = traffic(a) if a.what == "traffic" else step_traffic(a)
        with open(a.out, "w") as f:
            json.dump(res, f, indent=1)
        print(json.dumps(res, indent=1))


if __name__ == "__main__":
    main()
