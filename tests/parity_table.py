"""Formats the parity records a GPU test run leaves (MM1_PARITY_LOG, one JSON
object per checked output, written by tests/parity.py) as a markdown table.

    MM1_PARITY_LOG=/tmp/parity.jsonl python -m pytest tests -m gpu ...
    python tests/parity_table.py /tmp/parity.jsonl [--cases config,golden,ragged] [--summary]

--summary prints, over every record of the log, the count of O/dQ/dK/dV
checks per gate and the largest error per output (the bf16 output where it
passed as `bf16`, the pre-cast values where it passed as `precast`).
"""
from __future__ import annotations

import argparse
import json

ORDER = {"O": 0, "lse2": 1, "dQ": 2, "dK": 3, "dV": 4, "delta": 5}


def fmt(x):
    return "" if x is None else f"{x:.2e}"


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("log")
    ap.add_argument("--cases", default="config,golden,ragged,smoke",
                    help="comma-separated prefixes of the case names to include")
    ap.add_argument("--summary", action="store_true", help="gate counts and largest errors only")
    args = ap.parse_args(argv)
    prefixes = tuple(args.cases.split(","))
    recs = [json.loads(line) for line in open(args.log) if line.strip()]
    if args.summary:
        summary(recs)
        return
    recs = [r for r in recs if r.get("case", "").startswith(prefixes)]
    seen, rows = set(), []
    for r in recs:
        key = (r["case"], r["out"])
        if key in seen:
            continue
        seen.add(key)
        rows.append(r)
    rows.sort(key=lambda r: (r["case"], ORDER.get(r["out"], 9)))
    print("| case | out | max-abs | rel-L2 | floor | pre-cast max-abs | pre-cast rel-L2 "
          "| reference-kernel rounding max-abs | ... rel-L2 | gate |")
    print("|---|---|---:|---:|---:|---:|---:|---:|---:|---|")
    for r in rows:
        print(f"| {r['case']} | {r['out']} | {fmt(r['max_abs'])} | {fmt(r['rel_l2'])} | {fmt(r.get('floor'))} "
              f"| {fmt(r.get('precast_max_abs'))} | {fmt(r.get('precast_rel_l2'))} | {fmt(r.get('alg'))} "
              f"| {fmt(r.get('alg_rel'))} | {r.get('gate')} |")


def summary(recs):
    outs = ("O", "dQ", "dK", "dV")
    gates = {}
    worst = {}
    for r in recs:
        if r.get("out") not in outs:
            continue
        gates[r.get("gate")] = gates.get(r.get("gate"), 0) + 1
        pre = r.get("gate") == "precast"
        err = (r.get("precast_max_abs") if pre else r["max_abs"], r.get("precast_rel_l2") if pre else r["rel_l2"])
        if r["out"] not in worst or err[0] > worst[r["out"]][0][0]:
            worst[r["out"]] = (err, r["case"], r.get("gate"))
    print(f"Gates over the O/dQ/dK/dV rows of this run: {gates}.")
    print()
    print("| out | max-abs | rel-L2 | case | gate |")
    print("|---|---:|---:|---|---|")
    for o in outs:
        if o in worst:
            (ma, rl), case, gate = worst[o]
            print(f"| {o} | {fmt(ma)} | {fmt(rl)} | {case} | {gate} |")


if __name__ == "__main__":
    main()
