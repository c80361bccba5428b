"""GPU: soupk_lora_bwd_params_noalloc, the allocation-free form of soupk_lora_bwd_params (its
partial sums in the library's static per-GPU scratch instead of a caller workspace), called
through the C ABI.  It runs the same kernels over the same partial layout, so its parameter
gradients must equal the workspace entry point's bit for bit: checked on consecutive calls,
each smaller than the one before (so a call that read a slice left over from the previous one
would differ), down to no rows at all (zero gradients)."""

import pytest
import torch

from testt_amd import _ext, lora

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
H, NQ, NV, R = 1536, 1536, 256, 16


def _inputs(M, seed):
    g = torch.Generator().manual_seed(seed)

    def mk(cols, scale):
        return (torch.randn(M, cols, generator=g) * scale).to(torch.float16).to(DEV)

    return mk(H, 1.0), mk(2 * R, 0.5), mk(2 * R, 0.1), mk(NQ, 0.1), mk(NV, 0.1)


def _noalloc(y, t, dt, g_q, g_v, scaling):
    M = y.shape[0]
    outs = [torch.full(shape, float("nan"), dtype=torch.float32, device=DEV)
            for shape in ((R, H), (R, H), (NQ, R), (NV, R))]
    _ext.call("soupk_lora_bwd_params_noalloc", *[_ext.ptr(x) for x in (y, t, dt)],
              _ext.ptr(g_q), g_q.stride(0), _ext.ptr(g_v), g_v.stride(0), float(scaling),
              *[_ext.ptr(o) for o in outs], M, H, NQ, NV, R, _ext.stream_of(y))
    return outs


@pytest.mark.parametrize("sizes", [(2048, 333, 0), (6784, 129)])
def test_noalloc_matches_workspace_entry(sizes):
    for i, M in enumerate(sizes):
        print(f"lora params no-alloc call {i}: M={M}", flush=True)
        ins = (*_inputs(M, seed=100 + M), 2.0)
        got = _noalloc(*ins)
        want = lora.lora_bwd_params(*ins)
        for name, a, b in zip(("d_aq", "d_av", "d_bq", "d_bv"), got, want):
            assert torch.equal(a, b), f"{name} differs at M={M}"
        if M == 0:
            assert all(bool((a == 0).all()) for a in got)
    torch.cuda.synchronize()


_CAPTURE_CHILD = r'''
import sys
import torch
sys.path.insert(0, sys.argv[1])
from testt_amd import _ext, lora
from tests.test_zz_no_alloc import _inputs, H, NQ, NV, R

DEV = torch.device("cuda")
_ext.lib()                                  # loads the library and sets up device 0
M = 1000
ins = _inputs(M, seed=7)
want = lora.lora_bwd_params(*ins, 2.0)
outs = [torch.empty_like(w) for w in want]
y, t, dt, g_q, g_v = ins
args = ([_ext.ptr(x) for x in (y, t, dt)] + [_ext.ptr(g_q), g_q.stride(0), _ext.ptr(g_v),
        g_v.stride(0), 2.0] + [_ext.ptr(o) for o in outs] + [M, H, NQ, NV, R])
torch.cuda.synchronize()
s = torch.cuda.Stream()
s.wait_stream(torch.cuda.current_stream())
graph = torch.cuda.CUDAGraph()
with torch.cuda.graph(graph, stream=s):     # this process's first no-alloc call
    _ext.call("soupk_lora_bwd_params_noalloc", *args, _ext.stream_of(y))
torch.cuda.synchronize()
for rep in range(3):
    for o in outs:
        o.fill_(float("nan"))
    scratch_user = lora.lora_bwd_params(*_inputs(333, seed=rep), 2.0)   # eager work between
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    for name, a, b in zip(("d_aq", "d_av", "d_bq", "d_bv"), outs, want):
        assert torch.equal(a, b), (rep, name)
print("CAPTURE_OK", flush=True)
'''


def test_noalloc_first_call_under_graph_capture():
    """The entry point's first call in a process made inside HIP graph capture (the scratch
    address was looked up when the library was loaded, soupk_init_device), then the graph
    replayed three times with other eager work between the replays: every replay equals the
    workspace entry point's gradients bit for bit.  Run in a fresh child process, so that no
    earlier call of this session has made the lookup."""
    import os
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("lora params no-alloc under graph capture (child process)", flush=True)
    proc = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, root], capture_output=True,
                          text=True, timeout=300, cwd=root)
    print(proc.stdout[-2000:], proc.stderr[-2000:], flush=True)
    assert proc.returncode == 0 and "CAPTURE_OK" in proc.stdout
