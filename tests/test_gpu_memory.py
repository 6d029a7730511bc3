"""Device memory the library holds by itself: its code objects and the
static scratch array of mm1_attn_bwd_noalloc (MM1_NOALLOC_SCRATCH_BYTES), a
device-side static of the code object.  Measured in a fresh child process (so
no earlier test has loaded the library), with hipMemGetInfo's free bytes read
before the library is loaded, after it is loaded, after its first kernel
launch (a small forward) and after a first mm1_attn_bwd_noalloc call, each
net of what torch's caching allocator reserved in between."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent

CHILD = r"""
import json, sys
sys.path.insert(0, sys.argv[1])
import torch
dev = torch.device("cuda:0")
torch.empty(1, device=dev)                      # context, allocator warm
def point():
    torch.cuda.synchronize()
    return torch.cuda.mem_get_info(0)[0], torch.cuda.memory_reserved(0)
f0, r0 = point()
from mimansm1_v1_amd import _lib
lib = _lib.load()
f1, r1 = point()
B, S, H, Hkv, D = 1, 64, 10, 2, 128
q = torch.zeros(B, S, H, D, dtype=torch.bfloat16, device=dev)
k = torch.zeros(B, S, Hkv, D, dtype=torch.bfloat16, device=dev)
v = torch.zeros_like(k)
o = torch.empty_like(q)
lse = torch.empty(B, H, S, dtype=torch.float32, device=dev)
st = torch.empty(lib.mm1_attn_fwd_state_size(B, S, H, Hkv, D), dtype=torch.uint8, device=dev)
f1b, r1b = point()
rc = lib.mm1_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr(),
                      st.data_ptr(), st.numel(), B, S, H, Hkv, D, 1, D ** -0.5,
                      torch.cuda.current_stream(dev).cuda_stream)
f2, r2 = point()
# the no-allocation backward, once, on the same small shape
dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
do = torch.zeros_like(q)
f2b, r2b = point()
rc2 = lib.mm1_attn_bwd_noalloc(o.data_ptr(), do.data_ptr(), lse.data_ptr(), st.data_ptr(), st.numel(),
                               dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), B, S, H, Hkv, D, 1, D ** -0.5,
                               torch.cuda.current_stream(dev).cuda_stream)
f3, r3 = point()
print(json.dumps({"rc": rc, "rc_noalloc": rc2, "load": (f0 - f1) - (r1 - r0),
                  "first_launch": (f1b - f2) - (r2 - r1b), "noalloc": (f2b - f3) - (r3 - r2b),
                  "scratch": 256 << 20}))
"""


@pytest.mark.gpu
def test_static_scratch_is_mapped_by_the_first_no_alloc_call():
    out = subprocess.run([sys.executable, "-c", CHILD, str(ROOT)], capture_output=True, text=True,
                         timeout=300)
    assert out.returncode == 0, out.stderr[-2000:]
    rec = json.loads(out.stdout.strip().splitlines()[-1])
    print(f"    device bytes taken by loading the library: {rec['load']:,}; by its first kernel "
          f"launch: {rec['first_launch']:,}; by the first mm1_attn_bwd_noalloc call: {rec['noalloc']:,}")
    assert rec["rc"] == 0 and rec["rc_noalloc"] == 0
    mib = 1 << 20
    # loading the library and running its ordinary entry points maps its
    # code objects (a few MiB) but not the scratch array ...
    assert rec["load"] + rec["first_launch"] <= 32 * mib, rec
    # ... which the first no-allocation call maps (its hipGetSymbolAddress
    # and first use), and which stays mapped from then on
    assert rec["scratch"] <= rec["noalloc"] <= rec["scratch"] + 32 * mib, rec
