"""Shared pieces of the drop-in modules' harnesses (check_math, check_gpu,
benchmark, tune of attention.py, swiglu.py, lm_head.py).

The reference ships a check/benchmark harness next to each TileLang module
(attention_tilelang.py:544-788, swiglu_tilelang.py:368-643,
lm_head_tilelang.py:338-590): a script a user runs after changing a kernel.
Here the three modules share one implementation of the parts that do not
depend on the kernel:

* ``Report``: named checks grouped in sections; each records whether it held
  and a measured value, prints one line, and the whole report is returned to
  the caller (tests assert on it) rather than only printed.
* ``compare``: the error figures every GPU check reports -- max-abs, the
  reference harness's max|d| / max|ref| (attention_tilelang.py:664-669), and
  relative L2.
* ``time_cuda``: median milliseconds of a callable over repeated HIP-event
  timed loops on the current stream.
* ``main``: the command line (``check``, ``gpu``, ``bench``, ``tune``; the
  reference's ``--check``/``--gpu``/``--bench``/``--tune`` flags work too).
"""
from __future__ import annotations

import argparse
import statistics
from dataclasses import dataclass, field

import torch


@dataclass
class Outcome:
    section: str
    label: str
    ok: bool
    value: object = None


@dataclass
class Report:
    """Collects check outcomes; ``ok`` is True when every check held."""
    title: str
    quiet: bool = False
    outcomes: list = field(default_factory=list)
    _section: str = ""

    def section(self, name: str) -> "Report":
        self._section = name
        if not self.quiet:
            print(f"\n[{self.title}] {name}")
        return self

    def expect(self, label: str, ok, value=None) -> bool:
        ok = bool(ok)
        self.outcomes.append(Outcome(self._section, label, ok, value))
        if not self.quiet:
            shown = "" if value is None else f" = {value:.3e}" if isinstance(value, float) else f" = {value}"
            print(f"    [{'pass' if ok else 'FAIL'}] {label}{shown}")
        return ok

    def note(self, text: str) -> None:
        if not self.quiet:
            print(f"    {text}")

    @property
    def ok(self) -> bool:
        return all(o.ok for o in self.outcomes)

    def failures(self):
        return [o for o in self.outcomes if not o.ok]

    def finish(self) -> "Report":
        if not self.quiet:
            bad = self.failures()
            print(f"\n[{self.title}] {len(self.outcomes) - len(bad)}/{len(self.outcomes)} checks passed"
                  + ("" if not bad else ": " + "; ".join(f"{o.section}/{o.label}" for o in bad)))
        return self


def compare(got: torch.Tensor, want: torch.Tensor) -> dict:
    """Error of `got` against the reference values `want` (any dtypes)."""
    g, w = got.detach().float(), want.detach().float()
    d = g - w
    max_abs = d.abs().max().item() if d.numel() else 0.0
    ref_max = w.abs().max().item() if w.numel() else 0.0
    wn = w.norm().item()
    return {
        "max_abs": max_abs,
        "max_rel": max_abs / max(ref_max, 1e-12),     # the reference harness's figure
        "rel_l2": d.norm().item() / wn if wn > 0 else d.norm().item(),
        "finite": bool(torch.isfinite(g).all()),
    }


def time_cuda(fn, warmup: int = 5, iters: int = 20, repeats: int = 3, device=None) -> float:
    """Median over `repeats` loops of the mean ms per call of fn(), timed with
    HIP events on the current stream after `warmup` untimed calls."""
    stream = torch.cuda.current_stream(device)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize(device)
    per_call = []
    for _ in range(repeats):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for _ in range(iters):
            fn()
        stop.record(stream)
        torch.cuda.synchronize(device)
        per_call.append(start.elapsed_time(stop) / iters)
    return statistics.median(per_call)


def needs_gpu(what: str) -> bool:
    if torch.cuda.is_available():
        return True
    print(f"{what}: no HIP device")
    return False


def main(module: str, actions: dict, argv=None) -> int:
    """``python -m <module> [check|gpu|bench|tune ...]``; with no action,
    ``check``.  `actions` maps each action name to a callable."""
    ap = argparse.ArgumentParser(prog=f"python -m {module}")
    ap.add_argument("actions", nargs="*", metavar="ACTION",
                    help=f"any of {', '.join(actions)} (default: check)")
    for name in actions:
        ap.add_argument(f"--{name}", dest=f"flag_{name}", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args(argv)
    unknown = sorted(set(args.actions) - set(actions))
    if unknown:
        ap.error(f"unknown action(s) {', '.join(unknown)}")
    chosen = [a for a in actions if a in args.actions or getattr(args, f"flag_{a}")] or ["check"]
    status = 0
    for name in chosen:
        result = actions[name]()
        if isinstance(result, Report) and not result.ok:
            status = 1
    return status
