#!/usr/bin/env python3
"""Causal GQA flash-attention fwd+bwd throughput on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config 3] [--no-cpu]

A step is one forward + backward of the attention op over one batch of the
BASELINE.json workload (default config 3: batch 2, seq 8192, 10 query heads,
2 KV heads, head_dim 128, causal, bf16, synthetic N(0,1) inputs resident in
HBM).  The step runs exactly the kernels ``FlashAttention`` runs -- the
forward (K/V conversion, attention), the backward's prep (Delta, fp16 dO),
dK/dV, dQ with the dK/dV group sum in its tail -- through the library's C
ABI, and a second loop records HIP events between the stages on the launch
stream so every stage's average duration is measured live.

Printed: one JSON line.  ``value`` is algorithmic TFLOP/s of the whole step
(7 * B * H * S^2 * D for causal fwd+bwd: fwd 2 GEMMs + bwd 5 GEMMs of
2*S^2*D/2 each per head), from the median of --repeats timed loops of
--steps steps; ``roofline`` is the dominant kernel's algorithmic TFLOP/s
against the bf16 dense MFMA peak (the fp16 products of the kernels run at the
same rate); ``cpu_baseline`` is the fp32 reference math (oracle, torch
autograd) timed on this host's cores on the same workload (or one batch
element of it when host RAM is short), and each extra config carries its own;
``gpu_clock`` is the shader clock the GPU holds under the same step run back
to back for two seconds after the timed loops (``pct_of_clock_peak`` relates
the value to the MFMA peak at that clock).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA, published
HBM_TBPS = 8.0

CONFIGS = {
    1: dict(batch=1, seq=512),      # forward only
    2: dict(batch=8, seq=2048),
    3: dict(batch=2, seq=8192),
    4: dict(batch=4, seq=4096),
}
HEADS, KV_HEADS, DIM = 10, 2, 128
SUBLAYER_CONFIG = 5           # the attention sublayer, reported beside


def gemm_unit(batch, seq, heads=HEADS, dim=DIM, causal=True):
    """One causal attention GEMM over all heads: 2*S*S*D/2 * B*H flops."""
    return 2.0 * batch * heads * seq * seq * dim * (0.5 if causal else 1.0)


def parse(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=3, choices=[2, 3, 4])
    ap.add_argument("--also", type=int, nargs="*", default=[1, 2, 4, 5],
                    help="extra configs reported beside the main one (1 = forward only, 5 = the "
                         "attention sublayer)")
    ap.add_argument("--repeats", type=int, default=5,
                    help="timed loops of --steps steps; the reported figures are their median")
    ap.add_argument("--tiles", default=None, metavar="FWD,DKDV,DQ",
                    help="tiling indices (mm1_attn_tile_desc) for the stage calls instead of the "
                         "tile table's choice for the workload (A/B runs)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-ffn", action="store_true",
                    help="skip the SwiGLU feed-forward leg (reported beside the attention line)")
    ap.add_argument("--no-head", action="store_true",
                    help="skip the fused cross-entropy head leg (reported beside the attention line)")
    ap.add_argument("--ffn-tokens", type=int, default=16384,
                    help="tokens of the SwiGLU leg (8 x 2048, the reference benchmark's default)")
    ap.add_argument("--no-autograd", action="store_true", help="skip the autograd cross-check")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="only run --steps device-to-device copies of MIB MiB (a plain copy "
                         "kernel of known size, to scale rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    ap.add_argument("--mfma-ceiling", action="store_true",
                    help="only run the matrix-core issue-rate probe (probe/mfma_ceiling.hip): "
                         "FLOP/s of fp16 32x32x16 products alone and with fixed mixes of VALU / LDS "
                         "instructions, and the clock under each")
    ap.add_argument("--traffic", default=None,
                    help="JSON with HBM bytes per launch from rocprofv3 --pmc "
                         "(default profiles/traffic_config<N>.json if present)")
    return ap.parse_args(argv)


# Kernel launched by each tiling index of a stage (mm1_attn_tile_desc order).
KERNEL_NAMES = {"fwd": ("attn_fwd_pp_kernel", "attn_fwd_kernel", "attn_fwd_kernel"),
                "dkdv": ("attn_dkdv_pipe_kernel", "attn_dkdv_pipe_kernel"),
                "dq": ("attn_dq_kernel", "attn_dq_kernel")}


def select_tiles(batch, seq, override=None):
    """The tilings the tile record (this machine's store, then the shipped
    gfx950 table) holds for this workload -- what get_kernel's handles launch
    -- or `override` ("FWD,DKDV,DQ", one stream).  Returns {stage: index}
    plus "overlap" (the backward record's dQ side-stream switch, else
    attention.OVERLAP_DQ); the stage calls pass them explicitly."""
    from mimansm1_v1_amd import attention as A
    if override:
        f, k, q = (int(x) for x in override.split(","))
        return {"fwd": f, "dkdv": k, "dq": q, "overlap": False}
    from mimansm1_v1_amd import tuned
    shape = (batch, HEADS, seq, DIM, True, HEADS // KV_HEADS)
    fwd_cfg = tuned.lookup("attention_fwd", shape)
    bwd_cfg = tuned.lookup("attention_bwd", shape)
    fwd = A.tile_index("fwd", fwd_cfg) if fwd_cfg else None
    bwd = A.tile_index("bwd", bwd_cfg) if bwd_cfg else None
    overlap = bool((bwd_cfg or {}).get("overlap_dq", A.OVERLAP_DQ)) if bwd else A.OVERLAP_DQ
    return {"fwd": fwd or 0, "dkdv": (bwd or (0, 0))[0], "dq": (bwd or (0, 0))[1],
            "overlap": overlap}


def rope_rotate(x, theta=10_000.0):
    """Rotate-half RoPE in fp32 at positions 0..S-1: pair (x_i, x_{i+D/2})
    turned by angle pos * theta^(-2i/D) (the form of AT:533-541)."""
    import torch
    B, S, H, D = x.shape
    half = D // 2
    inv = theta ** (-2.0 * torch.arange(half, dtype=torch.float64) / D)
    ang = torch.arange(S, dtype=torch.float64)[:, None] * inv[None, :]
    c = ang.cos().float().view(1, S, 1, half)
    sn = ang.sin().float().view(1, S, 1, half)
    lo, hi = x[..., :half], x[..., half:]
    return torch.cat([lo * c - hi * sn, lo * sn + hi * c], dim=-1)


class Workload:
    """One batch of a BASELINE.json config resident in HBM, and the stage
    calls of one fwd+bwd step.  Inputs are drawn on the CPU from one seeded
    generator in the order Q, K, V, dO; with rope_sigma (config 4) a scale
    sigma ~ U(0.5, 3) per query head and per KV head follows, Q and K are
    scaled by it and rotated by RoPE (base 10000) in fp32, then all are cast
    to bf16."""

    def __init__(self, lib, batch, seq, device, tiles, seed=0, rope_sigma=False):
        import torch
        self.lib, self.B, self.S = lib, batch, seq
        self.H, self.Hkv, self.D = HEADS, KV_HEADS, DIM
        self.tiles = tiles
        gen = torch.Generator().manual_seed(seed)
        q = torch.randn(batch, seq, HEADS, DIM, generator=gen)
        k = torch.randn(batch, seq, KV_HEADS, DIM, generator=gen)
        v = torch.randn(batch, seq, KV_HEADS, DIM, generator=gen)
        do = torch.randn(batch, seq, HEADS, DIM, generator=gen)
        if rope_sigma:
            sq = torch.empty(HEADS).uniform_(0.5, 3.0, generator=gen)
            sk = torch.empty(KV_HEADS).uniform_(0.5, 3.0, generator=gen)
            q = rope_rotate(q * sq.view(1, 1, HEADS, 1))
            k = rope_rotate(k * sk.view(1, 1, KV_HEADS, 1))
        dev = lambda t: t.to(torch.bfloat16).to(device)
        self.q, self.k, self.v, self.do = dev(q), dev(k), dev(v), dev(do)
        self.o = torch.empty_like(self.q)
        self.lse = torch.empty(batch, HEADS, seq, dtype=torch.float32, device=device)
        self.dq = torch.empty_like(self.q)
        self.dk = torch.empty_like(self.k)
        self.dv = torch.empty_like(self.v)
        self.st_bytes = lib.mm1_attn_fwd_state_size(batch, seq, HEADS, KV_HEADS, DIM)
        self.state = torch.empty(self.st_bytes, dtype=torch.uint8, device=device)
        self.ws_bytes = lib.mm1_attn_bwd_workspace_size(batch, seq, HEADS, KV_HEADS, DIM)
        self.ws = torch.empty(self.ws_bytes, dtype=torch.uint8, device=device)
        self.scale = DIM ** -0.5
        self.stream = torch.cuda.current_stream(device)
        self.side = torch.cuda.Stream(device)   # default priority

    STAGES = ("fwd", "prep", "dkdv", "dq")

    def step(self, marks=None):
        """One fwd+bwd; if `marks` is given, records an event after each stage.
        Without `marks`, and when the tile record says so (tiles["overlap"]),
        the backward runs as BwdKernel then does: dQ on a second stream beside
        dK/dV, the dK/dV partial sum after dK/dV on the launch stream.  With
        `marks` the stages run one after the other on the launch stream (dQ
        with the partial sum in its tail), for the per-stage times."""
        L, B, S, H, Hkv, D, sp = self.lib, self.B, self.S, self.H, self.Hkv, self.D, self.stream.cuda_stream
        p = lambda t: t.data_ptr()

        def chk(rc, name):
            if rc != 0:
                raise RuntimeError(f"{name}: {L.mm1_attn_strerror(rc).decode()}")

        t = self.tiles
        st = (p(self.state), self.st_bytes)
        ws = (p(self.ws), self.ws_bytes)
        shape = (B, S, H, Hkv, D, 1, self.scale)
        chk(L.mm1_attn_fwd_tiles(p(self.q), p(self.k), p(self.v), p(self.o), p(self.lse), *st, *shape,
                                 t["fwd"], sp), "fwd")
        if marks is not None:
            marks[0].record(self.stream)
        chk(L.mm1_attn_bwd_prep(p(self.o), p(self.do), p(self.lse), *st, *ws, B, S, H, Hkv, D, self.scale, sp),
            "prep")
        if marks is not None:
            marks[1].record(self.stream)
        if marks is None and t.get("overlap"):
            import torch
            fork = torch.cuda.Event()
            fork.record(self.stream)
            self.side.wait_event(fork)
            chk(L.mm1_attn_bwd_dq_tiles(*st, p(self.dq), *ws, *shape, t["dq"], self.side.cuda_stream), "dq")
            chk(L.mm1_attn_bwd_dkdv_tiles(*st, p(self.dk), p(self.dv), *ws, *shape, t["dkdv"], sp), "dkdv")
            chk(L.mm1_attn_bwd_dkdv_reduce_tiles(*ws, p(self.dk), p(self.dv), B, S, H, Hkv, D, 1, t["dkdv"], sp),
                "dkdv reduce")
            join = torch.cuda.Event()
            join.record(self.side)
            self.stream.wait_event(join)
            return
        chk(L.mm1_attn_bwd_dkdv_tiles(*st, p(self.dk), p(self.dv), *ws, *shape, t["dkdv"], sp), "dkdv")
        if marks is not None:
            marks[2].record(self.stream)
        # dQ, with the dK/dV group sum folded into the same launch (what
        # mm1_attn_bwd runs after the dK/dV stage)
        chk(L.mm1_attn_bwd_dq_reduce_tiles(*st, p(self.dq), p(self.dk), p(self.dv), *ws, *shape, t["dkdv"],
                                           t["dq"], sp), "dq")
        if marks is not None:
            marks[3].record(self.stream)


def _clock_reader():
    """A function returning the GPU's current shader (GFX) clock in MHz, and
    its source: amdsmi's GPU metrics (the mean over the XCDs), else its clock
    info, else the sysfs DPM table's current level; (None, None) if none."""
    try:
        import amdsmi
        amdsmi.amdsmi_init()
        handle = amdsmi.amdsmi_get_processor_handles()[0]

        def metrics():
            clks = [c for c in amdsmi.amdsmi_get_gpu_metrics_info(handle)["current_gfxclks"]
                    if isinstance(c, (int, float)) and 0 < c < 65535]
            return sum(clks) / len(clks)

        def info():
            return float(amdsmi.amdsmi_get_clock_info(handle, amdsmi.AmdSmiClkType.GFX)["clk"])

        for read, src in ((metrics, "amdsmi gpu_metrics current_gfxclks (mean over XCDs)"),
                          (info, "amdsmi clock info (GFX)")):
            try:
                read()
                return read, src
            except Exception:
                pass
    except Exception:
        pass
    import glob
    import re
    paths = sorted(glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk"))
    if paths:
        def sysfs():
            for line in open(paths[0]):
                if line.strip().endswith("*"):
                    return float(re.search(r"(\d+)\s*Mhz", line, re.I).group(1))
            return float("nan")
        try:
            sysfs()
            return sysfs, f"sysfs {paths[0]}"
        except Exception:
            pass
    return None, None


def sustained_clock(step, seconds=2.0, settle=0.5):
    """The shader clock the GPU holds under the timed workload: runs `step`
    back to back for `seconds` and reads the clock after each batch of steps
    (a device synchronisation apart) once `settle` seconds have passed -- the
    SMU's readings lag the load by a fraction of a second, so samples taken
    during a short timed loop read the idle clock.  Median, min, max in MHz."""
    import time
    import torch
    read, source = _clock_reader()
    if read is None:
        return None
    samples = []
    t0 = time.perf_counter()
    while True:
        for _ in range(4):
            step()
        torch.cuda.synchronize()
        t = time.perf_counter() - t0
        if t >= settle:
            try:
                samples.append(read())
            except Exception:
                break
        if t >= seconds:
            break
    vals = sorted(v for v in samples if v == v and v > 0)
    if not vals:
        return None
    med = vals[len(vals) // 2]
    return {"median_mhz": round(med, 1), "min_mhz": round(vals[0], 1), "max_mhz": round(vals[-1], 1),
            "samples": len(vals), "seconds": seconds, "source": source,
            "peak_at_this_clock_tflops": round(PEAK_BF16_TFLOPS * med / 2400.0, 1)}


MFMA_CEILING_MODES = ("products only", "+4 fma", "+4 fma +1 exp", "A from LDS (b128)",
                      "A and B from LDS (b128 + 2 tr_b64)",
                      "dK/dV mix (2 LDS, 3 fma, 0.5 exp)", "LDS reads only (b128)",
                      "LDS reads only (tr_b64)", "products only, 1 dependent chain",
                      "products only, 2 dependent chains")
MFMA_CEILING_LDS_ONLY = (6, 7)   # no products: LDS bytes per second instead


def mfma_ceiling(device, seconds=1.5, settle=0.5):
    """The matrix-core issue-rate probe (probe/mfma_ceiling.hip, built into
    _lib/libmm1probe.so): for each instruction mix, 512 workgroups of 4
    waves (two waves per SIMD, as the attention kernels run) issue 4
    independent fp16 32x32x16 product chains for `seconds`, launch after
    launch; the median launch time gives TFLOP/s, and the clock is read after
    each launch once `settle` seconds have passed."""
    import ctypes
    import time
    import torch
    from mimansm1_v1_amd import build as B
    path = B.probe_path()
    if not path.exists():
        raise RuntimeError(f"{path} is missing: run python -m mimansm1_v1_amd.build")
    lib = ctypes.CDLL(str(path))
    fn = lib.mm1_probe_mfma_ceiling
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    blocks, iters = 512, 20000
    out = torch.empty(blocks * 256, dtype=torch.float32, device=device)
    read, source = _clock_reader()
    flop = blocks * 4 * iters * 4 * 32768.0
    rows = []
    for mode, name in enumerate(MFMA_CEILING_MODES):
        stream = torch.cuda.current_stream().cuda_stream
        if fn(mode, out.data_ptr(), blocks, iters, stream) != 0:
            raise RuntimeError(f"probe mode {mode} failed to launch")
        torch.cuda.synchronize()
        times, clocks = [], []
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < seconds:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn(mode, out.data_ptr(), blocks, iters, stream)
            e1.record()
            torch.cuda.synchronize()
            times.append(e0.elapsed_time(e1))
            if read is not None and time.perf_counter() - t0 >= settle:
                try:
                    clocks.append(read())
                except Exception:
                    pass
        ms = sorted(times)[len(times) // 2]
        clk = sorted(clocks)[len(clocks) // 2] if clocks else None
        if mode in MFMA_CEILING_LDS_ONLY:
            nbytes = blocks * 4 * iters * 4096.0      # 4 KiB of LDS reads per wave and trip
            tbs = nbytes / ms / 1e9
            per_clk = nbytes / (ms * 1e-3) / (clk * 1e6) / 256 if clk else None
            rows.append({"mode": mode, "mix": name, "ms": round(ms, 4), "lds_tbytes_per_s": round(tbs, 2),
                         "bytes_per_clk_per_cu": round(per_clk, 1) if per_clk else None,
                         "clock_mhz": round(clk, 1) if clk else None})
            print(f"[mfma-ceiling] {name:36s} {tbs:7.2f} TB/s of LDS reads, "
                  f"{per_clk or float('nan'):5.1f} B/clk/CU  clock {clk or float('nan'):6.0f} MHz",
                  file=sys.stderr, flush=True)
            continue
        tf = flop / ms / 1e9
        rows.append({"mode": mode, "mix": name, "ms": round(ms, 4), "tflops": round(tf, 1),
                     "pct_of_peak": round(100 * tf / PEAK_BF16_TFLOPS, 1),
                     "clock_mhz": round(clk, 1) if clk else None})
        print(f"[mfma-ceiling] {name:36s} {tf:7.1f} TFLOP/s ({100 * tf / PEAK_BF16_TFLOPS:4.1f}% of "
              f"{PEAK_BF16_TFLOPS:.0f})  clock {clk or float('nan'):6.0f} MHz", file=sys.stderr, flush=True)
    return {"probe": "mfma_ceiling", "instruction": "v_mfma_f32_32x32x16_f16", "workgroups": blocks,
            "waves_per_simd": 2, "products_per_launch": blocks * 4 * iters * 4, "clock_source": source,
            "modes": rows}


def time_forward(batch, seq, device, steps, warmup):
    """The forward alone through the drop-in kernel handle (config 1: the
    GPU side of the CPU forward baseline): median of five timed loops."""
    import torch
    import mimansm1_v1_amd as mm
    gen = torch.Generator().manual_seed(0)
    mk = lambda h: torch.randn(batch, seq, h, DIM, generator=gen).to(torch.bfloat16).to(device)
    q, k, v = mk(HEADS), mk(KV_HEADS), mk(KV_HEADS)
    kern = mm.get_kernel("fwd", batch, HEADS, seq, DIM, True, HEADS // KV_HEADS)
    loops = []
    for _ in range(5):
        loops.append(_timed(lambda: kern(q, k, v), steps, warmup))
    ms = sorted(loops)[2]
    return {"batch": batch, "seq_len": seq, "ms_fwd": round(ms, 4),
            "fwd_tflops": round(2 * gemm_unit(batch, seq) / (ms * 1e-3) / 1e12, 2)}


def time_workload(wl, steps, warmup, repeats=5):
    """W warm-up steps, then `repeats` rounds of two loops of exactly `steps`
    steps, each loop bracketed by a device synchronisation: the first times
    the steps alone (HIP events before and after the loop only), the second
    records an event on the launch stream after every stage for the per-stage
    times (about 2.5 us per event, which is why the step itself is timed
    without them).  Returns the median round's ms per step, that round's
    per-stage ms, and every round's ms per step."""
    import torch
    for _ in range(warmup):
        wl.step()
    torch.cuda.synchronize()
    ev = lambda: torch.cuda.Event(enable_timing=True)
    loops = []
    for _ in range(repeats):
        start, end = ev(), ev()
        torch.cuda.synchronize()
        start.record(wl.stream)
        for _ in range(steps):
            wl.step()
        end.record(wl.stream)
        torch.cuda.synchronize()
        step_ms = start.elapsed_time(end) / steps
        marks = [[ev() for _ in Workload.STAGES] for _ in range(steps)]
        begins = [ev() for _ in range(steps)]
        torch.cuda.synchronize()
        for i in range(steps):
            begins[i].record(wl.stream)
            wl.step(marks[i])
        torch.cuda.synchronize()
        per_stage = {name: 0.0 for name in Workload.STAGES}
        for i in range(steps):
            prev = begins[i]
            for name, mk in zip(Workload.STAGES, marks[i]):
                per_stage[name] += prev.elapsed_time(mk)
                prev = mk
        loops.append((step_ms, {k: v / steps for k, v in per_stage.items()}))
    order = sorted(range(repeats), key=lambda i: loops[i][0])
    ms, stages = loops[order[repeats // 2]]
    return ms, stages, [round(x[0], 4) for x in loops]


def time_autograd(batch, seq, device, steps, warmup, repeats=5):
    """The same step through the drop-in autograd op (cross-check): W warm-up
    steps, then the median of `repeats` timed loops of `steps` steps, as for
    the kernels' own step (a single loop reads the clock's ramp as well)."""
    import torch
    import mimansm1_v1_amd as mm
    gen = torch.Generator().manual_seed(0)
    mk = lambda *s: torch.randn(*s, generator=gen).to(torch.bfloat16).to(device).requires_grad_(True)
    q, k, v = mk(batch, seq, HEADS, DIM), mk(batch, seq, KV_HEADS, DIM), mk(batch, seq, KV_HEADS, DIM)
    do = torch.randn(batch, seq, HEADS, DIM, generator=gen).to(torch.bfloat16).to(device)

    def run():
        mm.flash_attention(q, k, v, True, HEADS // KV_HEADS).backward(do)
        q.grad = k.grad = v.grad = None

    for _ in range(warmup):
        run()
    loops = []
    for _ in range(repeats):
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(steps):
            run()
        t1.record()
        torch.cuda.synchronize()
        loops.append(t0.elapsed_time(t1) / steps)
    return sorted(loops)[repeats // 2]


def _timed(fn, steps, warmup):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        fn()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps


def time_sublayer(batch, seq, device, steps, warmup):
    """the attention sublayer (d_model 1280, fused QKV
    projection, QK-norm + RoPE, causal flash attention, wo) forward + backward
    under bf16 autocast, x ~ N(0,1), weights ~ N(0, 0.02^2).  Besides the whole
    step, its parts are timed on the same tensors: the attention kernels (fwd +
    bwd), the projection GEMMs (QKV and wo, fwd + both backward products, as
    BF16Linear runs them on hipBLASLt) and the QK-norm + RoPE kernels (fwd +
    bwd)."""
    import torch
    import torch.nn.functional as F
    from mimansm1_v1_amd import attention as A
    gen = torch.Generator().manual_seed(0)
    cfg = A.AttnConfig(max_seq_len=seq)
    mod = A.Attention(cfg, A.Rotary(cfg.head_dim, seq, cfg.rope_theta))
    with torch.no_grad():
        for lin in (mod.wq, mod.wk, mod.wv, mod.wo):
            lin.weight.copy_(torch.randn(lin.weight.shape, generator=gen) * 0.02)
    mod = mod.to(device)
    x = torch.randn(batch, seq, cfg.d_model, generator=gen).to(device).requires_grad_(True)
    dy = torch.randn(batch, seq, cfg.d_model, generator=gen).to(torch.bfloat16).to(device)
    ac = lambda: torch.autocast("cuda", dtype=torch.bfloat16)

    def full():
        with ac():
            y = mod(x)
        y.backward(dy)
        x.grad = None
        mod.zero_grad(set_to_none=True)

    ms_full = _timed(full, steps, warmup)
    # parts, on tensors of the same shapes and values
    w_cat = torch.cat((mod.wq.weight, mod.wk.weight, mod.wv.weight), 0).detach().requires_grad_(True)
    wo = mod.wo.weight.detach().requires_grad_(True)
    with torch.no_grad(), ac():
        qkv = F.linear(x, w_cat).contiguous()
    qkv.requires_grad_(True)
    qn, kn = (m.weight.detach().requires_grad_(True) for m in (mod.q_norm, mod.k_norm))
    with torch.no_grad():
        q, k, v = A.qknorm_rope(qkv, qn, kn, mod.rope.cos, mod.rope.sin, cfg.n_heads, cfg.n_kv_heads,
                                cfg.norm_eps)
    g = [torch.randn(t.shape, generator=gen).to(torch.bfloat16).to(device) for t in (q, k, v)]
    for t in (q, k, v):
        t.requires_grad_(True)
    o = torch.randn(batch, seq, cfg.d_model, generator=gen).to(torch.bfloat16).to(device).requires_grad_(True)
    dqkv = torch.randn(qkv.shape, generator=gen).to(torch.bfloat16).to(device)

    def attention():
        A.flash_attention(q, k, v, True, cfg.groups).backward(g[0])
        q.grad = k.grad = v.grad = None

    # the QK-norm + RoPE kernels through the C ABI on preallocated buffers (the
    # autograd wrapper's allocations would otherwise time the host, not the GPU)
    from mimansm1_v1_amd import _lib
    lib = _lib.load()
    qo, ko, vo = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dqkv_o = torch.empty_like(qkv)
    dwq, dwk = torch.empty(cfg.head_dim, device=device), torch.empty(cfg.head_dim, device=device)
    ws_bytes = lib.mm1_qknorm_rope_bwd_workspace_size()
    ws = torch.empty(ws_bytes // 4, device=device)
    qnf, knf = qn.detach().float().contiguous(), kn.detach().float().contiguous()
    cos_t, sin_t = mod.rope.cos, mod.rope.sin
    sp = torch.cuda.current_stream(device).cuda_stream
    H, Hkv, D, rot = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cos_t.shape[0]

    def norm_rope():
        _lib.check(lib.mm1_qknorm_rope_fwd(qkv.data_ptr(), qnf.data_ptr(), knf.data_ptr(), cos_t.data_ptr(),
                                           sin_t.data_ptr(), qo.data_ptr(), ko.data_ptr(), vo.data_ptr(),
                                           batch, seq, H, Hkv, D, rot, cfg.norm_eps, sp), "qknorm fwd")
        _lib.check(lib.mm1_qknorm_rope_bwd(qkv.data_ptr(), qnf.data_ptr(), knf.data_ptr(), cos_t.data_ptr(),
                                           sin_t.data_ptr(), g[0].data_ptr(), g[1].data_ptr(), g[2].data_ptr(),
                                           dqkv_o.data_ptr(), dwq.data_ptr(), dwk.data_ptr(), ws.data_ptr(),
                                           ws_bytes, batch, seq, H, Hkv, D, rot, cfg.norm_eps, sp), "qknorm bwd")

    def gemms():
        # the projections as the step runs them (BF16Linear under autocast)
        with ac():
            a = A.BF16Linear.apply(x, w_cat)
            b = A.BF16Linear.apply(o, wo)
        torch.autograd.backward((a, b), (dqkv, dy))
        x.grad = w_cat.grad = o.grad = wo.grad = None

    parts = {"attention": _timed(attention, steps, warmup), "gemm": _timed(gemms, steps, warmup),
             "qknorm_rope": _timed(norm_rope, steps, warmup)}
    tokens = batch * seq
    gemm_flops = 6.0 * tokens * cfg.d_model * (cfg.n_heads + 2 * cfg.n_kv_heads) * cfg.head_dim \
        + 6.0 * tokens * cfg.d_model * cfg.d_model
    attn_flops = 7 * gemm_unit(batch, seq)
    return {
        "batch": batch, "seq_len": seq, "d_model": cfg.d_model,
        "ms_per_step": round(ms_full, 4),
        "tflops": round((attn_flops + gemm_flops) / (ms_full * 1e-3) / 1e12, 2),
        "part_ms": {k: round(v, 4) for k, v in parts.items()},
        "other_ms": round(ms_full - sum(parts.values()), 4),
        "attention_tflops": round(attn_flops / (parts["attention"] * 1e-3) / 1e12, 2),
        "gemm_tflops": round(gemm_flops / (parts["gemm"] * 1e-3) / 1e12, 2),
        "flops": {"attention": attn_flops, "gemm": gemm_flops},
        "note": "bf16 autocast; attention = flash_attention fwd+bwd kernels, gemm = QKV (1280->1792) and "
                "wo (1280->1280) fwd + dX + dW as the step runs them (BF16Linear: hipBLASLt GEMMs, dW over 8 "
                "token chunks with fp32 outputs), qknorm_rope = fwd+bwd kernels; "
                "other = casts, weight concatenation and autograd bookkeeping of the whole step",
    }


def time_swiglu(tokens, device, steps, warmup):
    """The SwiGLU feed-forward (d_model 1280, ffn 3328) on `tokens` tokens:
    fused_swiglu forward + backward (autograd, bf16), and its two HIP kernels
    alone through the C ABI on preallocated buffers: the gate/up GEMM with the
    SwiGLU epilogue (training mode: gate, up, act out) and the gradient
    kernel.  Inputs ~ N(0,1), weights ~ N(0, 0.02^2), synthetic."""
    import torch
    from mimansm1_v1_amd import _lib
    from mimansm1_v1_amd import swiglu as SG
    cfg = SG.FFNConfig()
    T, d, Fh = tokens, cfg.d_model, cfg.ffn_hidden
    gen = torch.Generator().manual_seed(0)
    mk = lambda *shape, s=1.0: (torch.randn(*shape, generator=gen) * s).to(torch.bfloat16).to(device)
    x, wg, wu, wd = mk(T, d), mk(d, Fh, s=0.02), mk(d, Fh, s=0.02), mk(Fh, d, s=0.02)
    go = mk(T, d)
    leaves = [t.clone().requires_grad_(True) for t in (x, wg, wu, wd)]

    def full():
        SG.fused_swiglu(*leaves).backward(go)
        for t in leaves:
            t.grad = None

    lib = _lib.load()
    sp = torch.cuda.current_stream(device).cuda_stream
    gate, up, act = (torch.empty(T, Fh, dtype=torch.bfloat16, device=device) for _ in range(3))
    dgu = torch.empty(T, 2 * Fh, dtype=torch.bfloat16, device=device)
    dact = mk(T, Fh)

    def gate_up():
        _lib.check(lib.mm1_swiglu_gate_up(x.data_ptr(), wg.data_ptr(), wu.data_ptr(), gate.data_ptr(),
                                          up.data_ptr(), act.data_ptr(), T, d, Fh, SG.MODE_TRAIN, sp),
                   "mm1_swiglu_gate_up")

    def grad():
        _lib.check(lib.mm1_swiglu_grad(dact.data_ptr(), gate.data_ptr(), up.data_ptr(), dgu.data_ptr(),
                                       dgu.data_ptr() + 2 * Fh, T, Fh, 2 * Fh, sp), "mm1_swiglu_grad")

    ms_full = _timed(full, steps, warmup)
    ms_gu = _timed(gate_up, steps, warmup)
    ms_grad = _timed(grad, steps, warmup)
    gu_flops = 4.0 * T * d * Fh
    gu_bytes = 2.0 * (T * d + 2 * d * Fh + 3 * T * Fh)
    grad_bytes = 2.0 * 5 * T * Fh
    return {
        "tokens": T, "d_model": d, "ffn": Fh,
        "ms_per_step": round(ms_full, 4),
        "tflops": round(SG.swiglu_flops(T, cfg) / (ms_full * 1e-3) / 1e12, 2),
        "gate_up_ms": round(ms_gu, 4),
        "gate_up_tflops": round(gu_flops / (ms_gu * 1e-3) / 1e12, 2),
        "gate_up_frac_of_peak": round(gu_flops / (ms_gu * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "gate_up_hbm_gbps": round(gu_bytes / (ms_gu * 1e-3) / 1e9, 1),
        "grad_ms": round(ms_grad, 4),
        "grad_gbps": round(grad_bytes / (ms_grad * 1e-3) / 1e9, 1),
        "grad_frac_of_hbm": round(grad_bytes / (ms_grad * 1e-3) / 1e12 / HBM_TBPS, 4),
        "note": "fwd+bwd flops 18*T*d*F (3 GEMMs forward, 6 backward, as swiglu_tilelang.benchmark "
                "counts); gate_up = the fused gate/up GEMM + SwiGLU epilogue kernel (4*T*d*F flops, "
                "gate/up/act written); grad = the elementwise gradient kernel (3 reads + 2 writes of "
                "T*F bf16)",
    }


def time_lm_head(tokens, device, steps, warmup):
    """The fused cross-entropy head (d_model 1280, vocabulary 49,152) on
    `tokens` tokens: fused_cross_entropy forward + backward (whole-vocabulary
    chunk), and its two GEMM-pass kernels alone through the C ABI: the
    log-sum-exp pass (with target logits and per-token losses) and the
    d_logits pass.  hidden ~ N(0, 0.1^2), weight ~ N(0, 0.02^2) (the
    reference benchmark's scales), uniform targets; synthetic."""
    import torch
    from mimansm1_v1_amd import _lib
    from mimansm1_v1_amd import lm_head as LH
    cfg = LH.HeadConfig()
    T, d, V = tokens, cfg.d_model, cfg.vocab
    gen = torch.Generator().manual_seed(0)
    hidden = (torch.randn(T, d, generator=gen) * 0.1).to(torch.bfloat16).to(device)
    weight = (torch.randn(d, V, generator=gen) * 0.02).to(torch.bfloat16).to(device)
    targets = torch.randint(0, V, (T,), generator=gen).to(device)
    h_leaf, w_leaf = hidden.clone().requires_grad_(True), weight.clone().requires_grad_(True)

    def full():
        LH.fused_cross_entropy(h_leaf, w_leaf, targets).backward()
        h_leaf.grad = w_leaf.grad = None

    lib = _lib.load()
    sp = torch.cuda.current_stream(device).cuda_stream
    lse, tl, loss = (torch.empty(T, dtype=torch.float32, device=device) for _ in range(3))
    ws_bytes = lib.mm1_lm_head_workspace_size(T, V)
    ws = torch.empty(ws_bytes // 4 + 1, dtype=torch.float32, device=device)
    scale = torch.tensor([1.0 / T], device=device)
    dl = torch.empty(T, V, dtype=torch.bfloat16, device=device)

    def lse_pass():
        _lib.check(lib.mm1_lm_head_lse(hidden.data_ptr(), weight.data_ptr(), targets.data_ptr(), -100,
                                       lse.data_ptr(), tl.data_ptr(), loss.data_ptr(), ws.data_ptr(), ws_bytes,
                                       T, d, V, sp), "mm1_lm_head_lse")

    def dlogits_pass():
        _lib.check(lib.mm1_lm_head_dlogits(hidden.data_ptr(), weight.data_ptr(), targets.data_ptr(), -100,
                                           lse.data_ptr(), scale.data_ptr(), dl.data_ptr(), V, T, d, V, 0, V,
                                           sp), "mm1_lm_head_dlogits")

    ms_full = _timed(full, steps, warmup)
    ms_lse = _timed(lse_pass, steps, warmup)
    ms_dl = _timed(dlogits_pass, steps, warmup)
    unit = 2.0 * T * d * V
    return {
        "tokens": T, "d_model": d, "vocab": V,
        "ms_per_step": round(ms_full, 4),
        "tflops": round(4 * unit / (ms_full * 1e-3) / 1e12, 2),
        "lse_ms": round(ms_lse, 4),
        "lse_tflops": round(unit / (ms_lse * 1e-3) / 1e12, 2),
        "lse_frac_of_peak": round(unit / (ms_lse * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
        "dlogits_ms": round(ms_dl, 4),
        "dlogits_tflops": round(unit / (ms_dl * 1e-3) / 1e12, 2),
        "note": "fwd+bwd flops 4 * 2*T*d*V (log-sum-exp pass; d_logits pass, d_hidden and d_weight "
                "GEMMs); the [T, V] logits are never stored in the forward; lse = the log-sum-exp "
                "kernel pass (2*T*d*V flops, partials + combine), dlogits = the d_logits GEMM pass",
    }


def cpu_baseline(config):
    """The reference's CPU attention path: the fp32 reference math (the
    oracle's restatement of AT:521-530, autograd for the backward) on this
    host's cores, on the bench workload itself when host RAM allows (autograd
    keeps about four fp32 [B, H, S, S] score-sized tensors), else on one batch
    element (reported per batch element).  One warm-up run, then the median of
    three timed runs."""
    import torch
    from oracle import reference as R
    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    B, S = CONFIGS[config]["batch"], CONFIGS[config]["seq"]
    need = 4 * 4.0 * B * HEADS * S * S + (16 << 30)
    try:
        import psutil
        avail = psutil.virtual_memory().available
    except ImportError:
        avail = 0
    full = avail >= need
    batch = B if full else 1
    q, k, v, do = R.make_inputs(batch, S, HEADS, KV_HEADS, DIM, seed=0, dtype=torch.float32,
                                rope_sigma=(config == 4))
    groups = HEADS // KV_HEADS
    fwd_only = config == 1
    if fwd_only:
        flops = 2 * gemm_unit(batch, S)
        run = lambda: R.attention(q, k, v, True, groups)
    else:
        flops = 7 * gemm_unit(batch, S)   # algorithmic 7*B*H*S^2*D (gemm_unit holds the causal 1/2)
        run = lambda: R.grads(q, k, v, do, True, groups)
    run()                                 # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run()
        times.append(time.perf_counter() - t0)
    med = sorted(times)[1]
    model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    what = (f"the full config {config} workload (batch {B})" if full else
            f"batch 1 of config {config} (host RAM {avail / 2**30:.0f} GiB < {need / 2**30:.0f} GiB "
            f"for the full batch of {B}; the rate is per batch element)")
    return {
        "value": round(flops / med / 1e12, 5),
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"fp32 torch {'forward' if fwd_only else 'autograd'} of the reference math "
                   f"(oracle/reference.py, AT:521-530) on {what}: seq {S}, 10 query / 2 KV heads, d 128, "
                   f"causal {'fwd' if fwd_only else 'fwd+bwd'}; 1 warm-up run, median of 3 runs = "
                   f"{med:.3f} s per {'fwd' if fwd_only else 'fwd+bwd'}; algorithmic flops "
                   f"{'2' if fwd_only else '7'}*B*H*S^2*D (causal halves counted) = {flops / 1e9:.2f} GFLOP; "
                   f"CPU: {model}"),
    }


def main(argv=None):
    args = parse(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: every box in this setup has one MI355X, so "
              f"--gpus {args.gpus} is not supported (the attention would shard per (batch, KV "
              f"head), each GPU computing its share with no exchange).", file=sys.stderr)
        return 2
    sys.path.insert(0, str(ROOT))
    import torch
    from mimansm1_v1_amd import _lib
    lib = _lib.load()
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 1
    device = torch.device("cuda:0")

    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes": n * 4, "launches": args.steps}), flush=True)
        return 0

    if args.mfma_ceiling:
        print(json.dumps(mfma_ceiling(device)), flush=True)
        return 0

    results = {}
    clock = None
    for cfg in [args.config] + [c for c in args.also if c != args.config]:
        if cfg == 1:
            res = time_forward(CONFIGS[1]["batch"], CONFIGS[1]["seq"], device, args.steps, args.warmup)
            results[cfg] = res
            print(f"[bench] config 1 (forward only): {res['ms_fwd']:.4f} ms, {res['fwd_tflops']:.1f} TFLOP/s",
                  file=sys.stderr, flush=True)
            continue
        if cfg == SUBLAYER_CONFIG:
            res = time_sublayer(2, 8192, device, args.steps, args.warmup)
            results[cfg] = res
            torch.cuda.empty_cache()
            print(f"[bench] config 5 (sublayer): {res['ms_per_step']:.3f} ms/step, {res['tflops']:.1f} TFLOP/s, "
                  f"parts {res['part_ms']}, other {res['other_ms']:.3f}", file=sys.stderr, flush=True)
            continue
        B, S = CONFIGS[cfg]["batch"], CONFIGS[cfg]["seq"]
        tiles = select_tiles(B, S, args.tiles)
        wl = Workload(lib, B, S, device, tiles, rope_sigma=(cfg == 4))
        ms, stages, loops = time_workload(wl, args.steps, args.warmup, args.repeats)
        if cfg == args.config:
            clock = sustained_clock(wl.step)
        unit = gemm_unit(B, S)
        flops = {"fwd": 2 * unit, "dkdv": 4 * unit, "dq": 3 * unit}
        one_stream = sum(stages.values())
        res = {
            "ms_per_step": ms,
            "tflops": 7 * unit / (ms * 1e-3) / 1e12,
            "stage_ms": stages,
            "ms_per_step_one_stream": one_stream,
            "fwd_tflops": 2 * unit / (stages["fwd"] * 1e-3) / 1e12,
            "bwd_tflops": 5 * unit / ((one_stream - stages["fwd"]) * 1e-3) / 1e12,
            "kernel_tflops": {k: flops[k] / (stages[k] * 1e-3) / 1e12 for k in flops},
            "kernel_flops": flops,
            "tiles": tiles,
            "loops_ms_per_step": loops,
        }
        if not args.no_autograd:
            res["ms_per_step_autograd"] = time_autograd(B, S, device, args.steps, args.warmup, args.repeats)
        results[cfg] = res
        del wl
        torch.cuda.empty_cache()
        print(f"[bench] config {cfg}: {ms:.3f} ms/step, {res['tflops']:.1f} TFLOP/s, "
              f"stages {', '.join(f'{k} {v:.3f}' for k, v in stages.items())}",
              file=sys.stderr, flush=True)

    ffn_res = None
    if not args.no_ffn:
        ffn_res = time_swiglu(args.ffn_tokens, device, args.steps, args.warmup)
        torch.cuda.empty_cache()
        print(f"[bench] swiglu: {ffn_res['ms_per_step']:.3f} ms/step, {ffn_res['tflops']:.1f} TFLOP/s; "
              f"gate_up {ffn_res['gate_up_ms']:.3f} ms ({ffn_res['gate_up_tflops']:.1f} TFLOP/s), "
              f"grad {ffn_res['grad_ms']:.3f} ms ({ffn_res['grad_gbps']:.0f} GB/s)",
              file=sys.stderr, flush=True)

    head_res = None
    if not args.no_head:
        head_res = time_lm_head(args.ffn_tokens, device, args.steps, args.warmup)
        torch.cuda.empty_cache()
        print(f"[bench] lm head: {head_res['ms_per_step']:.3f} ms/step, {head_res['tflops']:.1f} TFLOP/s; "
              f"lse {head_res['lse_ms']:.3f} ms ({head_res['lse_tflops']:.1f} TFLOP/s), "
              f"dlogits {head_res['dlogits_ms']:.3f} ms ({head_res['dlogits_tflops']:.1f} TFLOP/s)",
              file=sys.stderr, flush=True)

    main_res = results[args.config]
    B, S = CONFIGS[args.config]["batch"], CONFIGS[args.config]["seq"]
    dom = max(("fwd", "dkdv", "dq"), key=lambda k: main_res["stage_ms"][k])
    achieved = main_res["kernel_tflops"][dom]
    traffic = None
    tpath = Path(args.traffic) if args.traffic else ROOT / "profiles" / f"traffic_config{args.config}.json"
    if tpath.exists():
        try:
            traffic = json.loads(tpath.read_text()).get(dom)
        except ValueError:
            traffic = None

    out = {
        "metric": "causal GQA attn fwd+bwd TFLOP/s and % of MI355X bf16 MFMA peak, seq 2048/8192",
        "value": round(main_res["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(main_res["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"config {args.config}: causal GQA flash attention fwd+bwd, batch {B}, "
                        f"seq {S}, 10 query heads / 2 KV heads, head_dim 128, bf16",
            "batch": B, "seq_len": S, "heads": HEADS, "kv_heads": KV_HEADS, "head_dim": DIM,
            "causal": True, "parallelism": "single GPU",
        },
        "pct_of_peak": round(100 * main_res["tflops"] / PEAK_BF16_TFLOPS, 2),
        "gpu_clock": clock,
        "pct_of_clock_peak": (round(100 * main_res["tflops"] / clock["peak_at_this_clock_tflops"], 2)
                              if clock else None),
        "stage_schedule": ("stage_ms, fwd/bwd_tflops, kernel_tflops and the roofline's launch time come "
                           "from the per-stage loop, every stage on one stream with an event after each; "
                           "ms_per_step (and value) from the step loop, which runs dQ beside dK/dV on a "
                           "second stream when the tile record says so (tiles.overlap)"),
        "ms_per_step_one_stream": round(main_res["ms_per_step_one_stream"], 4),
        "fwd_tflops": round(main_res["fwd_tflops"], 2),
        "bwd_tflops": round(main_res["bwd_tflops"], 2),
        "stage_ms": {k: round(v, 4) for k, v in main_res["stage_ms"].items()},
        "tiles": main_res["tiles"],
        "repeats": args.repeats,
        "loops_ms_per_step": main_res["loops_ms_per_step"],
        "reference_flop_count_tflops": round(main_res["tflops"] * 5 / 7, 2),
        "roofline": {
            "bound": "mfma",
            "kernel": KERNEL_NAMES[dom][main_res["tiles"][dom]],
            "achieved": round(achieved, 2),
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": traffic,
            "flops_per_launch": main_res["kernel_flops"][dom],
            "avg_launch_ms": round(main_res["stage_ms"][dom], 4),
            "launch_timing": "HIP events on the launch stream around the stage in the one-stream per-stage loop",
        },
    }
    if "ms_per_step_autograd" in main_res:
        out["ms_per_step_autograd"] = round(main_res["ms_per_step_autograd"], 4)
    for cfg, res in results.items():
        if cfg == args.config:
            continue
        if cfg == SUBLAYER_CONFIG:
            out["config5"] = res
            continue
        if cfg == 1:
            out["config1"] = dict(res, note="forward only (BASELINE.json config 1), the drop-in kernel handle")
            continue
        out[f"config{cfg}"] = {
            "batch": CONFIGS[cfg]["batch"], "seq_len": CONFIGS[cfg]["seq"],
            "tflops": round(res["tflops"], 2),
            "pct_of_peak": round(100 * res["tflops"] / PEAK_BF16_TFLOPS, 2),
            "ms_per_step": round(res["ms_per_step"], 4),
            "ms_per_step_one_stream": round(res["ms_per_step_one_stream"], 4),
            "fwd_tflops": round(res["fwd_tflops"], 2), "bwd_tflops": round(res["bwd_tflops"], 2),
            "stage_ms": {k: round(v, 4) for k, v in res["stage_ms"].items()},
            "tiles": res["tiles"],
            "loops_ms_per_step": res["loops_ms_per_step"],
        }
        if cfg == 4:
            out[f"config{cfg}"]["inputs"] = ("RoPE-rotated Q, K with sigma ~ U(0.5, 3) per head (BASELINE.json "
                                             "config 4), V, dO ~ N(0,1)")
    if ffn_res is not None:
        out["swiglu"] = ffn_res
    if head_res is not None:
        out["lm_head"] = head_res
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.config)
        for cfg in results:
            if cfg in (1, 2, 4) and cfg != args.config:
                out[f"config{cfg}"]["cpu_baseline"] = cpu_baseline(cfg)
                print(f"[bench] cpu baseline config {cfg}: {out[f'config{cfg}']['cpu_baseline']['value']} TFLOP/s",
                      file=sys.stderr, flush=True)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
