"""Build the gfx950 attention library in-tree with hipcc.

    python -m mimansm1_v1_amd.build [--verbose] [--resource-usage]

Compiles every ``csrc/*.hip`` for ``--offload-arch=gfx950`` and links them into
``mimansm1_v1_amd/_lib/libmm1attn.so``, and ``probe/mfma_ceiling.hip`` into
``_lib/libmm1probe.so`` (the matrix-core issue-rate probe that
``bench.py --mfma-ceiling`` runs; not part of the attention ABI).  No GPU is
needed (hipcc cross-compiles).  The libraries are loaded with ctypes.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_lib"
LIB_NAME = "libmm1attn.so"
PROBE_SRC = PKG / "probe" / "mfma_ceiling.hip"
PROBE_LIB = "libmm1probe.so"
ARCH = "gfx950"

# Packed fp32 VALU ops are disabled for all device code (the hardware pool
# this builds for has shown silent wrong results from some of their forms).
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    "-ffp-contract=fast",
]


# Per-source extra flags (none at present).
EXTRA_FLAGS: dict = {}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def library_path() -> Path:
    return OUT_DIR / LIB_NAME


def build(verbose: bool = False, resource_usage: bool = False) -> Path:
    cc = hipcc()
    obj_dir = OUT_DIR / "obj"
    obj_dir.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")

    def compile_one(src: Path) -> Path:
        obj = obj_dir / (src.stem + ".o")
        cmd = [cc, *DEVICE_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
        if resource_usage:
            cmd.insert(1, "-Rpass-analysis=kernel-resource-usage")
        res = subprocess.run(cmd, capture_output=True, text=True)
        log = "\n".join(
            ln for ln in (res.stdout + res.stderr).splitlines()
            if "packed-fp32-ops" not in ln
        )
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{log}")
        if verbose or resource_usage:
            print(f"[build] {src.name}\n{log}" if log.strip() else f"[build] {src.name}")
        return obj

    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objs = list(pool.map(compile_one, sources))

    out = library_path()
    tmp = out.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"[build] wrote {out}")
    build_probe(cc)
    return out


def probe_path() -> Path:
    return OUT_DIR / PROBE_LIB


def build_probe(cc: str) -> Path:
    out = probe_path()
    tmp = out.with_suffix(".so.tmp")
    cmd = [cc, *DEVICE_FLAGS, "-shared", str(PROBE_SRC), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {PROBE_SRC.name}:\n{res.stdout}{res.stderr}")
    os.replace(tmp, out)
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--verbose", action="store_true")
    ap.add_argument("--resource-usage", action="store_true",
                    help="print per-kernel VGPR/AGPR/LDS/scratch usage")
    args = ap.parse_args(argv)
    build(verbose=args.verbose, resource_usage=args.resource_usage)
    return 0


if __name__ == "__main__":
    sys.exit(main())
