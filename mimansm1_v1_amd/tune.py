"""Tune the attention kernels once, for the shapes the run actually uses.

The counterpart of CODE/mimans/training/tune.py:30-128.  The run trains at
seq 2048 with micro batch 8 (CODE/mimans/training/train.py:22-23) and switches
to seq 8192 for the long-context stages, dividing the micro batch by four to
keep the tokens per micro step fixed (CODE/mimans/data.py:71-78,
tune.py:30-46): so both 8 x 2048 and 2 x 8192 are tuned.  A tiling that wins
at one is not necessarily the one that wins at the other.

For each shape and kernel (attention_fwd, attention_bwd -- keyed
``(micro_batch, heads, seq_len, dim, True, groups)`` as in tune.py:54-58) the
compiled gfx950 tilings are timed on synthetic inputs and the winner is
written to the tile store at once, so an interrupted run keeps what it
measured and a re-run skips what is known.  The reference's SwiGLU and LM-head
jobs (tune.py:59-64) are not run: this library builds those kernels
(`csrc/swiglu.hip`, `csrc/lm_head.hip`) with one gfx950 tiling each, so there
is nothing to choose; their `get_kernel` handles return that tiling.

    python -m mimansm1_v1_amd.tune                 # both shapes
    python -m mimansm1_v1_amd.tune --stage 0       # just 8 x 2048
    python -m mimansm1_v1_amd.tune --force         # re-measure known entries
    python -m mimansm1_v1_amd.tune --store mimansm1_v1_amd/tuned_tiles.json
                                                   # refresh the shipped table
"""
from __future__ import annotations

import argparse
import time

# (name, seq_len) of the reference's training stages, in order (data.py:71-78).
STAGES = (("foundation", 2048), ("code_spec", 2048), ("long_ctx", 8192), ("anneal", 8192))
MICRO_BATCH, SEQ_LEN = 8, 2048          # TrainConfig defaults (train.py:22-23)


def stage_shapes(micro_batch=MICRO_BATCH, seq_len=SEQ_LEN, stages=STAGES):
    """(stage name, micro_batch, seq_len) for each distinct context length,
    holding tokens per micro step fixed as the stage switch does (tune.py:30-46)."""
    seen, out = set(), []
    micro, seq = micro_batch, seq_len
    for name, stage_seq in stages:
        if stage_seq != seq:
            micro = max(1, micro * seq // stage_seq)
            seq = stage_seq
        if seq in seen:
            continue
        seen.add(seq)
        out.append((name, micro, seq))
    return out


def jobs(micro_batch, seq_len, cfg):
    shape = (micro_batch, cfg.n_heads, seq_len, cfg.head_dim, True, cfg.groups)
    return [("attention_fwd", "fwd", shape), ("attention_bwd", "bwd", shape)]


def tune_all(micro_batch, seq_len, cfg, force=False, store=None, lookup=None, search=None,
             record=None, out=print):
    """Tune each job of one shape; returns {name: (config, ms) or None}.  The
    lookup / search / record hooks default to the tile store and the GPU
    search; they are parameters so the control flow runs without a GPU."""
    from . import attention, tuned
    lookup = lookup or tuned.lookup
    search = search or (lambda kind, shape: attention.autotune(kind, shape, verbose=True)[:2])
    record = record or (lambda name, shape, config: tuned.record(name, shape, config, store=store))
    done = {}
    for name, kind, shape in jobs(micro_batch, seq_len, cfg):
        if not force and lookup(name, shape) is not None:
            out(f"  {name:14s} already known, skipping")
            done[name] = None
            continue
        out(f"  {name:14s} tuning {shape} ...")
        started = time.time()
        try:
            config, ms = search(kind, shape)
            record(name, shape, config)
            terse = " ".join(f"{k}={v}" for k, v in sorted(config.items()))
            out(f"  {name:14s} {time.time() - started:6.1f}s  {ms:.3f} ms  {terse}")
            done[name] = (config, ms)
        except Exception as exc:   # keep going: the other jobs are independent
            out(f"  {name:14s} FAILED after {time.time() - started:.1f}s: "
                f"{type(exc).__name__}: {exc}")
            done[name] = None
    return done


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--stage", type=int, default=None,
                        help="tune only one context length, by index")
    parser.add_argument("--force", action="store_true",
                        help="re-measure kernels that are already known")
    parser.add_argument("--store", default=None,
                        help="tile store to write (default: the per-user store)")
    args = parser.parse_args(argv)

    import torch

    from . import attention, tuned
    if not torch.cuda.is_available():
        raise SystemExit("tuning needs the gpu it will run on")
    attention.AUTOTUNE = True
    cfg = attention.AttnConfig()
    shapes = stage_shapes()
    if args.stage is not None:
        shapes = [shapes[args.stage]]
    store = args.store or tuned.STORE
    print(f"tuning on {tuned.device_key()}")
    print(f"store: {store}\n")

    def lookup(name, shape):   # only what the target store already holds counts as known
        return tuned._read(store).get(tuned.device_key(), {}).get(tuned._shape_key(name, shape))

    ok = True
    for name, micro, seq in shapes:
        print(f"{name}: micro_batch {micro} x seq {seq} = {micro * seq:,} tokens per micro step")
        done = tune_all(micro, seq, cfg, force=args.force, store=store, lookup=lookup)
        ok &= all(v is not None or lookup(n, s) is not None
                  for (n, _, s), v in zip(jobs(micro, seq, cfg), done.values()))
        print()
    print(tuned.summary([store]))
    return ok


if __name__ == "__main__":
    raise SystemExit(0 if main() else 1)
