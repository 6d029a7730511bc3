"""Summarise rocprofv3 output of a bench.py run (kernel times and HBM traffic).

    python -m mimansm1_v1_amd.profsum --trace DIR/prof_trace/trace_results.db \\
        --fetch DIR/pmc_fetch/fetch_counter_collection.csv \\
        --write DIR/pmc_write/write_counter_collection.csv \\
        --copy-fetch DIR/pmc_copy_fetch/cf_counter_collection.csv \\
        --copy-write DIR/pmc_copy_write/cw_counter_collection.csv \\
        --copy-bytes 1073741824 [--json profiles/traffic_config3.json]

Kernel times come from the ``--kernel-trace --stats`` database: calls, mean
and share from its ``top_kernels`` view, and from the per-dispatch ``kernels``
view the median and the same figures over the dispatches that ran alone (no
other dispatch of the trace overlapped them in time; a backward that runs dQ
on a second stream beside dK/dV gives both kinds).  FETCH_SIZE / WRITE_SIZE (KiB per dispatch, averaged over a
kernel's dispatches) are scaled by the factors that make the same counters read
``--copy-bytes`` for the plain device copy of that many bytes (the largest
dispatch of the calibration runs).
"""
from __future__ import annotations

import argparse
import re
import csv
import json
import sqlite3
from collections import defaultdict

SHORT = {
    "attn_fwd_kernel": "fwd",
    "attn_fwd_pp_kernel": "fwd",
    "attn_dkdv_pipe_kernel": "dkdv",
    "attn_dkdv_kernel": "dkdv",
    "attn_dq_kernel": "dq",
    "attn_dkdv_reduce_kernel": "reduce",
    "attn_delta_kernel": "delta",
    "attn_delta16_kernel": "delta16",
    "attn_do16_kernel": "do16",
    "attn_cvt16_kernel": "cvt16",
}


def demangle(name: str) -> str:
    """`mm1::kernel<args>` for this library's mangled kernel names (the
    profiler records some of them mangled, and binutils' demangler predates
    the _Float16 mangling they contain); other names unchanged."""
    m = re.match(r"_ZN3mm1(\d+)", name)
    if not m:
        return name
    n = int(m.group(1))
    rest = name[m.end():]
    base = rest[:n]
    rest = rest[n:]
    if not rest.startswith("I"):
        return f"mm1::{base}"
    args = []
    for kind, val in re.findall(r"L([ib])(\d+)E", rest[:rest.find("EEv") + 1] if "EEv" in rest else rest):
        args.append(("true" if val == "1" else "false") if kind == "b" else val)
    return f"mm1::{base}<{', '.join(args)}>"


def kernel_key(name: str) -> str:
    base = demangle(name).replace("void ", "").split("(")[0].split("<")[0]
    return base.split("::")[-1]


def trace_table(db: str):
    con = sqlite3.connect(db)
    rows = con.execute("select name, total_calls, average, percentage from top_kernels").fetchall()
    return [(kernel_key(n), demangle(n).split("(")[0].replace("void ", ""), c, avg, pct) for n, c, avg, pct in rows]


def _median(xs):
    xs = sorted(xs)
    n = len(xs)
    return None if n == 0 else (xs[n // 2] if n % 2 else 0.5 * (xs[n // 2 - 1] + xs[n // 2]))


def dispatch_stats(spans):
    """spans: (name, start, end) per dispatch, in ns.  Returns {name: (all
    durations, durations of the dispatches no other dispatch overlapped)} in
    µs."""
    order = sorted(range(len(spans)), key=lambda i: spans[i][1])
    alone = [True] * len(spans)
    reach, owner = None, None   # latest end among the dispatches started so far, and whose
    for i in order:
        _, start, end = spans[i]
        if reach is not None and start < reach:
            alone[i] = False
            alone[owner] = False
        if reach is None or end > reach:
            reach, owner = end, i
    out = defaultdict(lambda: ([], []))
    for i, (name, start, end) in enumerate(spans):
        us = (end - start) / 1e3
        out[name][0].append(us)
        if alone[i]:
            out[name][1].append(us)
    return dict(out)


def trace_dispatches(db: str):
    con = sqlite3.connect(db)
    spans = con.execute("select name, start, end from kernels").fetchall()
    return dispatch_stats([(demangle(n).split("(")[0].replace("void ", ""), s, e) for n, s, e in spans])


def counter_means(path: str):
    vals = defaultdict(list)
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            vals[kernel_key(r["Kernel_Name"])].append(float(r["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in vals.items()}


def counter_table(path: str):
    """{kernel: {counter: mean per dispatch}} of a --pmc CSV with any counters."""
    vals = defaultdict(lambda: defaultdict(list))
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            vals[kernel_key(r["Kernel_Name"])][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return {k: {c: sum(v) / len(v) for c, v in cs.items()} for k, cs in vals.items()}


def copy_kib(path: str) -> float:
    with open(path, newline="") as f:
        return max(float(r["Counter_Value"]) for r in csv.DictReader(f))


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--trace")
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--copy-fetch")
    ap.add_argument("--copy-write")
    ap.add_argument("--copy-bytes", type=int, default=1 << 30)
    ap.add_argument("--json", help="write {short kernel name: HBM bytes per launch} here")
    ap.add_argument("--pmc", nargs="+", default=[],
                    help="LABEL=CSV ...: per-kernel means of every counter in each --pmc CSV")
    args = ap.parse_args(argv)

    if args.trace:
        per = trace_dispatches(args.trace)
        print("| kernel | calls | avg µs | median µs | share | calls alone | avg alone µs | median alone µs |\n"
              "|---|---:|---:|---:|---:|---:|---:|---:|")
        for _, full, calls, avg, pct in trace_table(args.trace):
            every, solo = per.get(full, ([], []))
            med = _median(every)
            solo_avg = sum(solo) / len(solo) if solo else None
            fmt = lambda x: "-" if x is None else f"{x:.1f}"
            print(f"| `{full}` | {calls} | {avg:.1f} | {fmt(med)} | {pct:.1f}% | {len(solo)} | "
                  f"{fmt(solo_avg)} | {fmt(_median(solo))} |")
        print()
    if args.fetch and args.write and args.copy_fetch and args.copy_write:
        kib = args.copy_bytes / 1024
        f_scale = kib / copy_kib(args.copy_fetch)
        w_scale = kib / copy_kib(args.copy_write)
        fetch, write = counter_means(args.fetch), counter_means(args.write)
        print(f"calibration: FETCH_SIZE x {f_scale:.4f}, WRITE_SIZE x {w_scale:.4f} "
              f"(copy of {args.copy_bytes} bytes)\n")
        print("| kernel | FETCH_SIZE KiB | WRITE_SIZE KiB | HBM bytes/launch (scaled) |\n|---|---:|---:|---:|")
        traffic = {}
        for k in sorted(fetch):
            if k not in SHORT or k not in write:
                continue
            total = (fetch[k] * f_scale + write[k] * w_scale) * 1024
            traffic[SHORT[k]] = int(round(total))
            print(f"| `{k}` | {fetch[k]:,.0f} | {write[k]:,.0f} | {total / 1e6:,.1f} MB |")
        if args.json:
            traffic["_note"] = (f"HBM-side bytes per launch: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE "
                                f"(KiB per dispatch, mean over dispatches) scaled by {f_scale:.4f} and "
                                f"{w_scale:.4f}, the factors that make the same counters read "
                                f"{args.copy_bytes} bytes for a device copy of that size")
            with open(args.json, "w") as f:
                json.dump(traffic, f, indent=1)
                f.write("\n")


    if args.pmc:
        rows, names = [], []
        for item in args.pmc:
            label, path = item.split("=", 1)
            for k, cs in sorted(counter_table(path).items()):
                if k in SHORT:
                    rows.append((label, k, cs))
                    names += [c for c in cs if c not in names]
        print("| run | kernel | " + " | ".join(names) + " |")
        print("|---|---|" + "---:|" * len(names))
        for label, k, cs in rows:
            print(f"| {label} | `{k}` | " + " | ".join(f"{cs[c]:,.0f}" if c in cs else "" for c in names) + " |")


if __name__ == "__main__":
    main()
