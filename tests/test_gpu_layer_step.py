"""GPU: one full decoder layer built from the drop-in ops (testt_amd/layer.py, the per-layer body
of solution/model.py:235-255) against an fp32 eager layer with the same weights (dequantized by
the oracle), on a ragged, padded batch; forward outputs and the gradients of the residual
input, the previous block output and the LoRA parameters.

The fused layer runs its GEMMs in fp16 (as the reference does under autocast), so the check is
the reference step test's relative-norm tolerance (solution/test_model.py:118-127: 2e-2)."""

import numpy as np
import pytest
import torch

from oracle.nf4 import dequant_state
from oracle.rope import apply_rotary
from testt_amd import layer, layer_native, mlp, nf4, workloads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def rel_err(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def reference_layer(s0, d0, w, wd, pos, batch, seq, cos, sin, amask):
    """fp32 eager layer: the same wiring with every GEMM and the attention in fp32.  With LoRA
    dropout the two branches draw their masks in the fused layer's order (q, then v) on the
    padded [B, T, H] input, so a generator reseeded alike gives both layers the same masks."""
    H = s0.shape[1]
    nh, nkv, hd = w.n_heads, w.n_kv, w.head_dim
    padded = batch * seq

    def norm(x, weight):
        return weight * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + w.eps))

    s = s0 + d0.float()
    y = norm(s, w.input_norm)
    qkv = y @ torch.cat([wd["q"], wd["k"], wd["v"]]).t() + w.qkv_bias.float()
    y_pad = torch.zeros(padded, H, device=DEV).index_copy(0, pos, y)

    def lora_rows():
        x = y_pad
        if w.dropout > 0:
            x = torch.nn.functional.dropout(y_pad.view(batch, seq, H), w.dropout,
                                            training=True).view(padded, H)
        return x.index_select(0, pos)

    rows_q = lora_rows()
    rows_v = lora_rows()
    lq = (rows_q @ w.lora_q[0].t()) @ w.lora_q[1].t() * w.scaling
    lv = (rows_v @ w.lora_v[0].t()) @ w.lora_v[1].t() * w.scaling
    q = qkv[:, :nh * hd] + lq
    k = qkv[:, nh * hd:(nh + nkv) * hd]
    v = qkv[:, (nh + nkv) * hd:] + lv

    def pad(flat, heads):
        out = torch.zeros(padded, heads * hd, device=DEV).index_copy(0, pos, flat)
        return out.view(batch, seq, heads, hd).transpose(1, 2)

    qp, kp = apply_rotary(pad(q, nh), pad(k, nkv), cos, sin)
    vp = pad(v, nkv)
    rep = nh // nkv
    kp = kp.repeat_interleave(rep, dim=1)
    vp = vp.repeat_interleave(rep, dim=1)
    scores = (qp @ kp.transpose(-1, -2).contiguous()) / np.sqrt(hd)
    allowed = torch.ones(seq, seq, dtype=torch.bool, device=DEV).tril()[None, None] & \
        amask.bool()[:, None, None, :]
    scores = scores.masked_fill(~allowed, float("-inf"))
    a = torch.softmax(scores, -1).nan_to_num(0.0) @ vp
    a = a.transpose(1, 2).reshape(padded, nh * hd).index_select(0, pos)
    s2 = s + a @ wd["o"].t()
    y2 = norm(s2, w.post_norm)
    d = (torch.nn.functional.silu(y2 @ wd["gate"].t()) * (y2 @ wd["up"].t())) @ wd["down"].t()
    return s2, d


@pytest.mark.parametrize("lengths,dropout", [((64, 40), 0.0), ((64, 64), 0.0), ((64, 40), 0.1)])
def test_decoder_layer_matches_fp32_eager(lengths, dropout):
    print(f"decoder layer lengths={lengths} dropout={dropout}", flush=True)
    batch, seq = len(lengths), 64
    w = layer.synthetic_layer(DEV, seed=9, dropout=dropout)
    wd = {n: torch.from_numpy(dequant_state(getattr(w, n)).astype(np.float32)).to(DEV)
          for n in ("q", "k", "v", "o", "gate", "up", "down")}
    amask = torch.zeros(batch, seq, dtype=torch.int64, device=DEV)
    for b, n in enumerate(lengths):
        amask[b, :n] = 1
    pos = amask.reshape(-1).nonzero().squeeze(1)
    m = pos.numel()
    cos, sin = (t.to(DEV) for t in workloads.rope_tables(seq, w.head_dim))
    g = torch.Generator().manual_seed(3)
    s0 = torch.randn(m, workloads.HIDDEN, generator=g).to(DEV)
    d0 = (0.5 * torch.randn(m, workloads.HIDDEN, generator=g)).to(torch.float16).to(DEV)
    gs = (1e-2 * torch.randn(m, workloads.HIDDEN, generator=g)).to(DEV)
    gd = (1e-2 * torch.randn(m, workloads.HIDDEN, generator=g)).to(torch.float16).to(DEV)

    s_in = s0.clone().requires_grad_(True)
    d_in = d0.clone().requires_grad_(True)
    torch.manual_seed(1234)
    s, d = layer.decoder_layer(s_in, d_in, w, pos, batch, seq, cos, sin,
                               layer.key_valid_of(amask))
    torch.autograd.backward([s, d], [gs, gd])
    fused = [s_in.grad, d_in.grad] + [p.grad for p in (*w.lora_q, *w.lora_v)]
    for p in (*w.lora_q, *w.lora_v):
        p.grad = None

    rs_in = s0.clone().requires_grad_(True)
    rd_in = d0.float().clone().requires_grad_(True)
    torch.manual_seed(1234)
    rs, rd = reference_layer(rs_in, rd_in, w, wd, pos, batch, seq, cos, sin, amask)
    torch.autograd.backward([rs, rd], [gs, gd.float()])
    ref = [rs_in.grad, rd_in.grad] + [p.grad for p in (*w.lora_q, *w.lora_v)]

    assert rel_err(s, rs) < 2e-2 and rel_err(d.float(), rd) < 2e-2
    for name, a, b in zip(("d s_in", "d delta", "d A_q", "d B_q", "d A_v", "d B_v"), fused, ref):
        assert a is not None and b is not None, name
        assert rel_err(a, b) < 2e-2, (name, rel_err(a, b))


@pytest.mark.parametrize("keep", [True, False])
def test_unpack_per_layer_is_bit_identical(monkeypatch, keep):
    """All seven projections unpacked by one launch before the layer (UNPACK_PER_LAYER) or each
    stack where it is used: the same fp16 weights, so the same outputs and gradients, bit for
    bit, with the weights kept for backward or unpacked again there.  (The fused NF4 GEMM,
    which a projection without an unpacked weight may take at this row count, sums in another
    order; it is off here, so that both runs use the unpacked weights.)"""
    batch, seq, lengths = 2, 64, (64, 37)
    w = layer.synthetic_layer(DEV, seed=11)
    amask = torch.zeros(batch, seq, dtype=torch.int64, device=DEV)
    for b, n in enumerate(lengths):
        amask[b, :n] = 1
    pos = amask.reshape(-1).nonzero().squeeze(1)
    m = pos.numel()
    cos, sin = (t.to(DEV) for t in workloads.rope_tables(seq, w.head_dim))
    g = torch.Generator().manual_seed(5)
    s0 = torch.randn(m, workloads.HIDDEN, generator=g).to(DEV)
    d0 = (0.5 * torch.randn(m, workloads.HIDDEN, generator=g)).to(torch.float16).to(DEV)
    gs = (1e-2 * torch.randn(m, workloads.HIDDEN, generator=g)).to(DEV)
    gd = (1e-2 * torch.randn(m, workloads.HIDDEN, generator=g)).to(torch.float16).to(DEV)
    monkeypatch.setattr(nf4, "KEEP_UNPACKED_FOR_BACKWARD", keep)
    monkeypatch.setattr(nf4, "USE_FUSED_NF4_GEMM", False)
    runs = []
    for per_layer in (True, False):
        monkeypatch.setattr(layer, "UNPACK_PER_LAYER", per_layer)
        s_in = s0.clone().requires_grad_(True)
        d_in = d0.clone().requires_grad_(True)
        s, d = layer.decoder_layer(s_in, d_in, w, pos, batch, seq, cos, sin,
                                   layer.key_valid_of(amask))
        torch.autograd.backward([s, d], [gs, gd])
        runs.append([s.detach(), d.detach(), s_in.grad, d_in.grad] +
                    [p.grad.clone() for p in (*w.lora_q, *w.lora_v)])
        for p in (*w.lora_q, *w.lora_v):
            p.grad = None
    for name, a, b in zip(("s", "d", "d s_in", "d delta", "d A_q", "d B_q", "d A_v", "d B_v"),
                          *runs):
        assert torch.equal(a, b), name


@pytest.mark.parametrize("lengths", [(64, 37), (64, 64), (0, 9)])
def test_varlen_attention_path_is_bit_identical(monkeypatch, lengths):
    """The layer's varlen path (RopeAttention over the real tokens) against its padded path
    (RopePack, attention with key flags, gather): for right-padded rows the same arithmetic in
    the same order, so the same outputs and gradients, bit for bit."""
    batch, seq = len(lengths), 64
    w = layer.synthetic_layer(DEV, seed=13)
    amask = torch.zeros(batch, seq, dtype=torch.int64, device=DEV)
    for b, n in enumerate(lengths):
        amask[b, :n] = 1
    pos = amask.reshape(-1).nonzero().squeeze(1)
    m = pos.numel()
    cos, sin = (t.to(DEV) for t in workloads.rope_tables(seq, w.head_dim))
    g = torch.Generator().manual_seed(6)
    s0 = torch.randn(m, workloads.HIDDEN, generator=g).to(DEV)
    d0 = (0.5 * torch.randn(m, workloads.HIDDEN, generator=g)).to(torch.float16).to(DEV)
    gs = (1e-2 * torch.randn(m, workloads.HIDDEN, generator=g)).to(DEV)
    gd = (1e-2 * torch.randn(m, workloads.HIDDEN, generator=g)).to(torch.float16).to(DEV)
    runs = []
    for varlen in (True, False):
        monkeypatch.setattr(layer, "USE_VARLEN_ATTENTION", varlen)
        s_in = s0.clone().requires_grad_(True)
        d_in = d0.clone().requires_grad_(True)
        s, d = layer.decoder_layer(s_in, d_in, w, pos, batch, seq, cos, sin,
                                   layer.key_valid_of(amask))
        torch.autograd.backward([s, d], [gs, gd])
        runs.append([s.detach(), d.detach(), s_in.grad, d_in.grad] +
                    [p.grad.clone() for p in (*w.lora_q, *w.lora_v)])
        for p in (*w.lora_q, *w.lora_v):
            p.grad = None
    for name, a, b in zip(("s", "d", "d s_in", "d delta", "d A_q", "d B_q", "d A_v", "d B_v"),
                          *runs):
        assert torch.equal(a, b), name


@pytest.mark.parametrize("keep", [False, True])
def test_unpacked_weights_freed_after_forward_without_keep(monkeypatch, keep):
    """With nf4.KEEP_UNPACKED_FOR_BACKWARD = False (the reference's memory profile), no fp16
    projection outlives its layer's forward: four layer forwards with grad (each keeping what
    its backward needs) grow the allocated memory by far less than one layer's unpacked weights
    (94 MB at Qwen2.5-1.5B's shapes) per layer.  The LoRA parameters' fp16 staging, which the
    backward keeps, is its own small allocation, not a view that holds the unpack buffer.  With
    True the weights are kept for the backward, one buffer per layer."""
    monkeypatch.setattr(nf4, "KEEP_UNPACKED_FOR_BACKWARD", keep)
    w = layer.synthetic_layer(DEV, seed=21)
    unpacked = sum(int(np.prod(nf4.weight_shape(p))) * 2
                   for p in (w.q, w.k, w.v, w.o, w.gate, w.up, w.down))
    B, T = 4, 128
    pos = workloads.ragged_positions((T,) * B, T).to(DEV)
    M = pos.numel()
    g = torch.Generator().manual_seed(4)
    s = torch.randn(M, workloads.HIDDEN, generator=g).to(DEV).requires_grad_(True)
    cos, sin = workloads.rope_tables(T, workloads.HEAD_DIM, workloads.ROPE_THETA, device=DEV)
    d = None
    outs = []
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated(DEV)
    for _ in range(4):
        s, d = layer.decoder_layer(s, d, w, pos, B, T, cos, sin, None)
        outs.append((s, d))
    torch.cuda.synchronize()
    per_layer = (torch.cuda.memory_allocated(DEV) - before) / 4
    print(f"keep={keep}: {per_layer / 1e6:.1f} MB per layer (unpacked weights "
          f"{unpacked / 1e6:.1f} MB)", flush=True)
    if keep:
        assert per_layer > unpacked
    else:
        assert per_layer < 0.5 * unpacked
    (s.float().sum() + d.float().sum()).backward()
    assert w.lora_q[0].grad is not None


@pytest.mark.parametrize("lengths,with_delta", [((64, 37), True), ((64, 64), True),
                                               ((64, 37), False)])
def test_one_node_layer_is_bit_identical(monkeypatch, lengths, with_delta):
    """The layer as one autograd node -- issued from C (layer_native.NativeDecoderLayer,
    soupk_layer_fwd / _bwd) or from Python (layer.DecoderLayer, calling the five nodes' forward
    and backward in order) -- against the five nodes themselves: the same outputs and
    gradients, bit for bit, and the same parameter gradients after two steps accumulate; also
    for the first layer, whose input norm has no residual delta."""
    batch, seq = 2, 64
    # the one-node forms take the unpacked weights; at this token count the layer would run on
    # its NF4 weights (test_nf4_resident_layer)
    monkeypatch.setattr(layer, "NF4_RESIDENT_SMALL_BATCHES", False)
    w = layer.synthetic_layer(DEV, seed=12)
    amask = torch.zeros(batch, seq, dtype=torch.int64, device=DEV)
    for b, n in enumerate(lengths):
        amask[b, :n] = 1
    pos = amask.reshape(-1).nonzero().squeeze(1)
    m = pos.numel()
    cos, sin = (t.to(DEV) for t in workloads.rope_tables(seq, w.head_dim))
    g = torch.Generator().manual_seed(6)
    s0 = torch.randn(m, workloads.HIDDEN, generator=g).to(DEV)
    d0 = (0.5 * torch.randn(m, workloads.HIDDEN, generator=g)).to(torch.float16).to(DEV)
    gs = (1e-2 * torch.randn(m, workloads.HIDDEN, generator=g)).to(DEV)
    gd = (1e-2 * torch.randn(m, workloads.HIDDEN, generator=g)).to(torch.float16).to(DEV)
    runs = []
    for one_node, native in ((True, True), (True, False), (False, False)):
        monkeypatch.setattr(layer, "ONE_NODE_LAYER", one_node)
        monkeypatch.setattr(layer_native, "NATIVE_LAYER", native)
        node = ("NativeDecoderLayerBackward" if native else
                "DecoderLayerBackward" if one_node else None)
        out = []
        for _ in range(2):
            s_in = s0.clone().requires_grad_(True)
            d_in = d0.clone().requires_grad_(True) if with_delta else None
            s, d = layer.decoder_layer(s_in, d_in, w, pos, batch, seq, cos, sin,
                                       layer.key_valid_of(amask))
            assert (type(s.grad_fn).__name__ == node) == one_node
            torch.autograd.backward([s, d], [gs, gd])
            out += [s.detach(), d.detach(), s_in.grad,
                    d_in.grad if with_delta else torch.zeros(())]
        runs.append(out + [p.grad.clone() for p in (*w.lora_q, *w.lora_v)])
        for p in (*w.lora_q, *w.lora_v):
            p.grad = None
    names = ["s", "d", "d s_in", "d delta"] * 2 + ["d A_q", "d B_q", "d A_v", "d B_v"]
    for ref in runs[1:]:
        for name, a, b in zip(names, runs[0], ref):
            assert torch.equal(a, b), name


@pytest.mark.parametrize("lengths", [(64, 37), (16, 0)])
def test_nf4_resident_layer(monkeypatch, lengths):
    """At few tokens the layer runs its products on the NF4 weights (the fused NF4-dequant GEMM
    forward and input gradient, layer.NF4_RESIDENT_SMALL_BATCHES): no unpack in the forward or
    the backward, and outputs and gradients within fp16 rounding of the same layer on unpacked
    weights (the fused kernels sum in another order than hipBLASLt, and the q|k|v input
    gradient is added to the LoRA part after its own rounding).  The fp32 comparison of
    test_decoder_layer_matches_fp32_eager covers this path too (104 tokens)."""
    print(f"nf4-resident layer lengths={lengths}", flush=True)
    batch, seq = len(lengths), 64
    w = layer.synthetic_layer(DEV, seed=14)
    amask = torch.zeros(batch, seq, dtype=torch.int64, device=DEV)
    for b, n in enumerate(lengths):
        amask[b, :n] = 1
    pos = amask.reshape(-1).nonzero().squeeze(1)
    m = pos.numel()
    cos, sin = (t.to(DEV) for t in workloads.rope_tables(seq, w.head_dim))
    g = torch.Generator().manual_seed(8)
    s0 = torch.randn(m, workloads.HIDDEN, generator=g).to(DEV)
    d0 = (0.5 * torch.randn(m, workloads.HIDDEN, generator=g)).to(torch.float16).to(DEV)
    gs = (1e-2 * torch.randn(m, workloads.HIDDEN, generator=g)).to(DEV)
    gd = (1e-2 * torch.randn(m, workloads.HIDDEN, generator=g)).to(torch.float16).to(DEV)
    calls = []

    def counting(mod, name):
        real = getattr(mod, name)

        def wrapped(*a, **k):
            calls.append(name)
            return real(*a, **k)
        monkeypatch.setattr(mod, name, wrapped)

    for mod, name in ((nf4, "unpack_concat"), (mlp, "unpack_concat"), (layer, "unpack_concat"),
                      (layer, "unpack_groups"), (layer, "unpack_groups_lora")):
        counting(mod, name)
    assert layer.nf4_resident(m, ((w.q, w.k, w.v), (w.o,), (w.gate, w.up), (w.down,)),
                              s0.device)
    runs = []
    for resident in (True, False):
        monkeypatch.setattr(layer, "NF4_RESIDENT_SMALL_BATCHES", resident)
        calls.clear()
        s_in = s0.clone().requires_grad_(True)
        d_in = d0.clone().requires_grad_(True)
        s, d = layer.decoder_layer(s_in, d_in, w, pos, batch, seq, cos, sin,
                                   layer.key_valid_of(amask))
        torch.autograd.backward([s, d], [gs, gd])
        torch.cuda.synchronize()
        if resident:
            assert calls == [], calls
        else:
            assert calls, "the unpacked run unpacks"
        runs.append([s.detach(), d.detach(), s_in.grad, d_in.grad] +
                    [p.grad.clone() for p in (*w.lora_q, *w.lora_v)])
        for p in (*w.lora_q, *w.lora_v):
            p.grad = None
    for name, a, b in zip(("s", "d", "d s_in", "d delta", "d A_q", "d B_q", "d A_v", "d B_v"),
                          *runs):
        assert torch.isfinite(a.float()).all(), name
        assert rel_err(a, b) < 5e-3, (name, rel_err(a, b))


@pytest.mark.parametrize("lengths,with_delta", [((64, 37), True), ((16, 0), True),
                                               ((64, 37), False)])
def test_nf4_resident_native_is_bit_identical(monkeypatch, lengths, with_delta):
    """The layer on its NF4 weights issued from C (NativeDecoderLayer with dims.nf4:
    soupk_layer_fwd / _bwd calling the fused NF4 GEMMs) against the same layer's per-operation
    nodes on the NF4 weights: the same outputs and gradients, bit for bit, over two steps
    (parameter gradients accumulating), also for a first layer without residual delta."""
    print(f"nf4-resident native layer lengths={lengths} delta={with_delta}", flush=True)
    monkeypatch.setattr(layer, "NF4_RESIDENT_SMALL_BATCHES", True)
    batch, seq = len(lengths), 64
    w = layer.synthetic_layer(DEV, seed=15)
    amask = torch.zeros(batch, seq, dtype=torch.int64, device=DEV)
    for b, n in enumerate(lengths):
        amask[b, :n] = 1
    pos = amask.reshape(-1).nonzero().squeeze(1)
    m = pos.numel()
    cos, sin = (t.to(DEV) for t in workloads.rope_tables(seq, w.head_dim))
    g = torch.Generator().manual_seed(9)
    s0 = torch.randn(m, workloads.HIDDEN, generator=g).to(DEV)
    d0 = (0.5 * torch.randn(m, workloads.HIDDEN, generator=g)).to(torch.float16).to(DEV)
    gs = (1e-2 * torch.randn(m, workloads.HIDDEN, generator=g)).to(DEV)
    gd = (1e-2 * torch.randn(m, workloads.HIDDEN, generator=g)).to(torch.float16).to(DEV)
    runs = []
    for native in (True, False):
        monkeypatch.setattr(layer_native, "NATIVE_LAYER", native)
        out = []
        for _ in range(2):
            s_in = s0.clone().requires_grad_(True)
            d_in = d0.clone().requires_grad_(True) if with_delta else None
            s, d = layer.decoder_layer(s_in, d_in, w, pos, batch, seq, cos, sin,
                                       layer.key_valid_of(amask))
            assert (type(s.grad_fn).__name__ == "NativeDecoderLayerBackward") == native
            torch.autograd.backward([s, d], [gs, gd])
            out += [s.detach(), d.detach(), s_in.grad,
                    d_in.grad if with_delta else torch.zeros(())]
        runs.append(out + [p.grad.clone() for p in (*w.lora_q, *w.lora_v)])
        for p in (*w.lora_q, *w.lora_v):
            p.grad = None
    names = ["s", "d", "d s_in", "d delta"] * 2 + ["d A_q", "d B_q", "d A_v", "d B_v"]
    for name, a, b in zip(names, *runs):
        assert torch.equal(a, b), name
