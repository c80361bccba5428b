"""GPU: one decoder layer's forward + backward (testt_amd/layer.py) captured in a HIP graph with
torch.cuda.graph and replayed.  The kernels, torch's ops and hipBLASLt's chosen solutions are
deterministic, so every replay must reproduce the eager step bit for bit: outputs, the input
gradients and the LoRA gradients.  Replays alternate with eager work on another layer and with
synchronisations, so state left behind by one replay (a cleared buffer, a flag) that the next
one relies on would show up as a mismatch."""

import pytest
import torch

from testt_amd import layer, workloads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def inputs(batch, seq, seed):
    g = torch.Generator().manual_seed(seed)
    H = workloads.HIDDEN
    m = batch * seq
    s0 = torch.randn(m, H, generator=g).to(DEV)
    d0 = (0.5 * torch.randn(m, H, generator=g)).to(torch.float16).to(DEV)
    gs = (1e-2 * torch.randn(m, H, generator=g)).to(DEV)
    gd = (1e-2 * torch.randn(m, H, generator=g)).to(torch.float16).to(DEV)
    return s0, d0, gs, gd


@pytest.mark.parametrize("batch,seq", [(2, 128), (2, 32)])
def test_layer_graph_replays_match_eager(batch, seq):
    """(2, 128): the layer on unpacked weights + hipBLASLt; (2, 32), 64 tokens: the layer on its
    NF4 weights (fused NF4-dequant products with split partials, layer.nf4_resident)."""
    print(f"layer graph capture B={batch} T={seq}", flush=True)
    w = layer.synthetic_layer(DEV, seed=9)
    w_other = layer.synthetic_layer(DEV, seed=10)
    params = (*w.lora_q, *w.lora_v)
    pos = torch.arange(batch * seq, device=DEV)
    groups = ((w.q, w.k, w.v), (w.o,), (w.gate, w.up), (w.down,))
    assert layer.nf4_resident(batch * seq, groups, pos.device) == (batch * seq <= 128)
    cos, sin = (t.to(DEV) for t in workloads.rope_tables(seq))
    s0, d0, gs, gd = inputs(batch, seq, 1)
    s_in = s0.clone().requires_grad_(True)
    d_in = d0.clone().requires_grad_(True)

    def step(ww, si, di, gsi, gdi):
        s, d = layer.decoder_layer(si, di, ww, pos, batch, seq, cos, sin, None)
        torch.autograd.backward([s, d], [gsi, gdi])
        return s, d

    def clear():
        for t in (s_in, d_in, *params):
            t.grad = None

    s_ref, d_ref = (t.detach().clone() for t in step(w, s_in, d_in, gs, gd))
    grads_ref = [t.grad.clone() for t in (s_in, d_in, *params)]
    clear()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            step(w, s_in, d_in, gs, gd)
            clear()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        s_out, d_out = step(w, s_in, d_in, gs, gd)
    torch.cuda.synchronize()

    o0, o1, o2, o3 = inputs(batch, seq, 2)
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize()
        got = [s_out, d_out] + [t.grad for t in (s_in, d_in, *params)]
        want = [s_ref, d_ref] + grads_ref
        for name, a, b in zip(("s", "d", "ds", "ddelta", "dA_q", "dB_q", "dA_v", "dB_v"),
                              got, want):
            assert torch.equal(a, b), (r, name)
        # eager work on another layer between replays
        oi = o0.clone().requires_grad_(True)
        step(w_other, oi, o1.clone().requires_grad_(True), o2, o3)
        for t in (*w_other.lora_q, *w_other.lora_v):
            t.grad = None
        torch.cuda.synchronize()
