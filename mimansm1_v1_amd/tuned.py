"""Tile record: (device, kernel, shape) -> chosen tile variant.

The counterpart of CODE/mimans/model/tuned.py:31-104 (device_key / lookup /
record), keyed by the HIP architecture name (e.g. "gfx950") instead of the
CUDA compute capability.  Records live in ``tuned_tiles.json`` next to this
file and are replaced atomically.
"""
from __future__ import annotations

import json
import os
import threading
from pathlib import Path

STORE = Path(os.environ.get("MM1_TUNED_STORE", Path(__file__).with_name("tuned_tiles.json")))
_lock = threading.Lock()


def device_key() -> str:
    try:
        import torch
        if torch.cuda.is_available():
            props = torch.cuda.get_device_properties(torch.cuda.current_device())
            return getattr(props, "gcnArchName", props.name).split(":")[0]
    except Exception:
        pass
    return "gfx950"


def _load() -> dict:
    try:
        return json.loads(STORE.read_text())
    except (OSError, ValueError):
        return {}


def _key(name, shape) -> str:
    return f"{device_key()}|{name}|{','.join(str(int(s)) for s in shape)}"


def lookup(name, shape):
    return _load().get(_key(name, shape))


def record(name, shape, config) -> None:
    with _lock:
        data = _load()
        data[_key(name, shape)] = dict(config)
        tmp = STORE.with_suffix(".tmp")
        tmp.write_text(json.dumps(data, indent=1, sort_keys=True))
        os.replace(tmp, STORE)
