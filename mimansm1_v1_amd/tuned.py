"""Tile records: (device, kernel, shape) -> the tiling that won there.

The counterpart of CODE/mimans/model/tuned.py:31-104 (device_key / lookup /
record / config_of / summary, same nesting: device -> "kernel:shape" ->
config).  A config names one of the tilings compiled into the library
(``mm1_attn_tile_desc``): block_M, block_N, waves, stages, schedule -- for the
backward the dK/dV and dQ kernels' fields prefixed ``dkdv_`` and ``dq_``.

Two files are consulted, this machine's own store first:

* ``STORE`` -- ``$MM1_TUNED_STORE`` or ``~/.cache/mimansm1_v1_amd/tuned_tiles.json``;
  ``record`` writes here, immediately and atomically, so an interrupted tuning
  run keeps what it measured;
* ``TABLE`` -- ``tuned_tiles.json`` beside this file: the measured gfx950
  table shipped with the package (written by ``python -m mimansm1_v1_amd.tune
  --store <this file>``), so a fresh MI355X starts from tuned tiles without a
  search.

A device missing from both simply misses: its kernels search (``AUTOTUNE``)
or use the defaults, never tiles measured on other hardware.

    python -m mimansm1_v1_amd.tune      # fill the store for the run's shapes
    python -m mimansm1_v1_amd.tuned     # show what is remembered
"""
from __future__ import annotations

import json
import os
import threading
from pathlib import Path

TABLE = Path(__file__).with_name("tuned_tiles.json")
STORE = Path(os.environ.get("MM1_TUNED_STORE",
                            Path.home() / ".cache" / "mimansm1_v1_amd" / "tuned_tiles.json"))
_lock = threading.Lock()


def device_key() -> str:
    """Architecture and CU count, e.g. ``gfx950-256cu``: tiles are only valid
    for the kind of card they were measured on."""
    try:
        import torch
        if not torch.cuda.is_available():
            return "no-hip"
        props = torch.cuda.get_device_properties(torch.cuda.current_device())
        arch = getattr(props, "gcnArchName", "") or props.name.replace(" ", "-")
        return f"{arch.split(':')[0]}-{props.multi_processor_count}cu"
    except Exception:
        return "no-hip"


def _shape_key(kernel: str, shape) -> str:
    return f"{kernel}:{','.join(str(s) for s in shape)}"


def _read(path: Path) -> dict:
    try:
        data = json.loads(Path(path).read_text())
        return data if isinstance(data, dict) else {}
    except (OSError, ValueError):
        return {}


def lookup(kernel: str, shape, device: str | None = None):
    """The remembered config for this kernel and shape, or None."""
    device = device or device_key()
    key = _shape_key(kernel, shape)
    for path in (STORE, TABLE):
        hit = _read(path).get(device, {}).get(key)
        if hit:
            return dict(hit)
    return None


def record(kernel: str, shape, config: dict, device: str | None = None, store=None) -> None:
    """Remember a tuned config (written at once; empty configs are ignored)."""
    if not config:
        return
    path = Path(store or STORE)
    device = device or device_key()
    with _lock:
        data = _read(path)
        data.setdefault(device, {})[_shape_key(kernel, shape)] = dict(config)
        path.parent.mkdir(parents=True, exist_ok=True)
        tmp = path.with_suffix(".json.tmp")
        tmp.write_text(json.dumps(data, indent=2, sort_keys=True) + "\n")
        os.replace(tmp, path)


def config_of(kernel):
    """The tiling a kernel handle settled on, if it reports one."""
    config = getattr(kernel, "config", None)
    return dict(config) if isinstance(config, dict) else None


def summary(paths=None) -> str:
    """What each store holds, one line per record:
    ``<store>  <device>  <kernel>  <shape>  key=value ...``."""
    rows = []
    for path in paths or (STORE, TABLE):
        data = _read(path)
        records = [(device, key, config) for device, entries in sorted(data.items())
                   for key, config in sorted(entries.items())]
        if not records:
            rows.append(f"{path}  (no records)")
        for device, key, config in records:
            kernel, _, shape = key.partition(":")
            fields = " ".join(f"{name}={value}" for name, value in sorted(config.items()))
            rows.append(f"{path}  {device}  {kernel}  ({shape})  {fields}")
    return "\n".join(rows)


if __name__ == "__main__":
    print(f"this gpu: {device_key()}\n")
    print(summary())
