"""GPU: the rank-16 LoRA kernels (testt_amd/csrc/lora.hip) against float64 restatements of the
rounding steps of the fp16 GEMMs they replace (peft's branch under fp16 autocast,
solution/model.py:195-206).  Each fp16 result is one rounding of a sum of exact fp16 products
accumulated in fp32, so it lies within n fp16 ulps of the exact sum (n = 1, or 2 where a
scaling multiplies an already rounded value) plus the fp32 summation error, bounded by
32 * 2^-24 * sum|terms| (the sums are at most ~16 additions deep: 32-product MFMA steps, then
four partial sums); the second term matters only where the sum cancels to a small result.
gs = fp16(g * scaling) is elementwise and exact.  The fused QKVLora is also checked against its
separate-GEMM path."""

import pytest
import torch

from testt_amd import layer, lora, workloads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def within_ulps(got, exact, n, abs_terms):
    """|got - exact| <= n fp16 ulps of exact + 32 * 2^-24 * abs_terms (float64 tensors)."""
    h = exact.to(torch.float16)
    inf = torch.tensor(float("inf"), dtype=torch.float16, device=h.device)
    ulp = (torch.nextafter(h.abs(), inf) - h.abs()).double()
    err = (got.double() - exact).abs()
    bad = err > n * ulp + 32 * 2.0 ** -24 * abs_terms
    assert not bool(bad.any()), (f"{int(bad.sum())} of {bad.numel()} beyond the bound, "
                                 f"max err {float(err.max()):.3g}")


def params(H, NQ, NV, seed):
    g = torch.Generator().manual_seed(seed)
    a_q = (torch.randn(16, H, generator=g) / H ** 0.5).to(DEV)
    a_v = (torch.randn(16, H, generator=g) / H ** 0.5).to(DEV)
    b_q = (0.05 * torch.randn(NQ, 16, generator=g)).to(DEV)
    b_v = (0.05 * torch.randn(NV, 16, generator=g)).to(DEV)
    return a_q, a_v, b_q, b_v


def f64_16(t):
    return t.to(torch.float16).double()


@pytest.mark.parametrize("H,NQ,NV", [(1536, 1536, 256), (256, 384, 128)])
def test_stage_layouts(H, NQ, NV):
    """soupk_lora_stage: the fp16 casts of the parameters (torch's rounding), in the four
    layouts, in order: [A_q; A_v], its transpose, [B_q; B_v], B_q^T, B_v^T."""
    print(f"lora stage H={H} NQ={NQ} NV={NV}", flush=True)
    a_q, a_v, b_q, b_v = params(H, NQ, NV, H + NQ)
    st = lora.stage(a_q, a_v, b_q, b_v)
    assert st.numel() == lora.staged_elems(H, NQ, NV)
    a16 = torch.cat([a_q, a_v]).to(torch.float16)
    b16 = torch.cat([b_q, b_v]).to(torch.float16)
    want = torch.cat([a16.flatten(), a16.t().flatten(), b16.flatten(),
                      b_q.to(torch.float16).t().flatten(), b_v.to(torch.float16).t().flatten()])
    assert torch.equal(st, want)


@pytest.mark.parametrize("M,H,NQ,NV,scaling", [(2048, 1536, 1536, 256, 2.0), (37, 512, 512, 256, 0.7),
                                               (1, 256, 256, 128, 2.0)])
def test_lora_fwd(M, H, NQ, NV, scaling):
    print(f"lora fwd M={M} H={H} NQ={NQ} NV={NV} s={scaling}", flush=True)
    a_q, a_v, b_q, b_v = params(H, NQ, NV, M + H)
    g = torch.Generator().manual_seed(1)
    y = torch.randn(M, H, generator=g).to(torch.float16).to(DEV)
    t, lq, lv = lora.lora_fwd(y, a_q, a_v, b_q, b_v, scaling)
    a16 = f64_16(torch.cat([a_q, a_v]))
    within_ulps(t, y.double() @ a16.t(), 1, y.double().abs() @ a16.abs().t())
    for out, tt, b in ((lq, t[:, :16], b_q), (lv, t[:, 16:], b_v)):
        b16 = f64_16(b)
        inner = (tt.double() @ b16.t()).to(torch.float16).double()   # one GEMM rounding
        within_ulps(out, inner * scaling, 2, scaling * (tt.double().abs() @ b16.abs().t()))


@pytest.mark.parametrize("M,H,NQ,NV,scaling,strided", [(2048, 1536, 1536, 256, 2.0, True),
                                                       (37, 512, 512, 256, 0.7, False),
                                                       (1, 256, 256, 128, 2.0, True)])
def test_lora_bwd_rows(M, H, NQ, NV, scaling, strided):
    print(f"lora bwd rows M={M} H={H} NQ={NQ} NV={NV} s={scaling} strided={strided}", flush=True)
    a_q, a_v, b_q, b_v = params(H, NQ, NV, M + NQ)
    g = torch.Generator().manual_seed(2)
    if strided:      # the layout RopePack's backward hands over: views of one [M, NQ+2NV+...]
        wide = (1e-2 * torch.randn(M, NQ + 2 * NV, generator=g)).to(torch.float16).to(DEV)
        g_q, g_v = wide[:, :NQ], wide[:, NQ + NV:]
    else:
        g_q = (1e-2 * torch.randn(M, NQ, generator=g)).to(torch.float16).to(DEV)
        g_v = (1e-2 * torch.randn(M, NV, generator=g)).to(torch.float16).to(DEV)
    dt, dy = lora.lora_bwd_rows(g_q, g_v, a_q, a_v, b_q, b_v, scaling)
    gs_q = (g_q.float() * scaling).to(torch.float16)   # formed in the kernel, not stored
    gs_v = (g_v.float() * scaling).to(torch.float16)
    bq16, bv16 = f64_16(b_q), f64_16(b_v)
    exact_dt = torch.cat([gs_q.double() @ bq16, gs_v.double() @ bv16], dim=1)
    terms_dt = torch.cat([gs_q.double().abs() @ bq16.abs(), gs_v.double().abs() @ bv16.abs()],
                         dim=1)
    within_ulps(dt, exact_dt, 1, terms_dt)
    a16 = f64_16(torch.cat([a_q, a_v]))
    within_ulps(dy, dt.double() @ a16, 1, dt.double().abs() @ a16.abs())


def rel(a, b):
    a, b = a.detach().double(), b.detach().double()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def test_qkvlora_fused_matches_gemm_path(monkeypatch):
    """The same QKVLora step through the kernels and through separate fp16 GEMMs: outputs and
    every gradient agree to fp16 GEMM rounding (relative L2 < 2e-3)."""
    w = layer.synthetic_layer(DEV, seed=9)
    M = 300
    g = torch.Generator().manual_seed(3)
    y = torch.randn(M, workloads.HIDDEN, generator=g).to(torch.float16).to(DEV)
    gq = (1e-2 * torch.randn(M, 2048, generator=g)).to(torch.float16).to(DEV)
    glq = (1e-2 * torch.randn(M, 1536, generator=g)).to(torch.float16).to(DEV)
    glv = (1e-2 * torch.randn(M, 256, generator=g)).to(torch.float16).to(DEV)
    results = []
    for fused in (True, False):
        monkeypatch.setattr(layer, "USE_FUSED_LORA", fused)
        yi = y.clone().requires_grad_(True)
        for p in (*w.lora_q, *w.lora_v):
            p.grad = None
        qkv, lq, lv = layer.QKVLora.apply(yi, w.qkv_bias, *w.lora_q, *w.lora_v, w.scaling,
                                          (w.q, w.k, w.v))
        torch.autograd.backward([qkv, lq, lv], [gq, glq, glv])
        results.append([qkv, lq, lv, yi.grad] + [p.grad.clone() for p in (*w.lora_q, *w.lora_v)])
    assert torch.equal(results[0][0], results[1][0])          # the projection itself: one GEMM
    for name, a, b in zip(("lq", "lv", "dy", "dA_q", "dB_q", "dA_v", "dB_v"), results[0][1:],
                          results[1][1:]):
        assert rel(a, b) < 2e-3, (name, rel(a, b))


@pytest.mark.parametrize("M,H,NQ,NV,scaling,strided", [(2048, 1536, 1536, 256, 2.0, True),
                                                       (300, 512, 512, 256, 0.7, False),
                                                       (37, 256, 256, 128, 2.0, True),
                                                       (1, 256, 256, 128, 1.0, False)])
def test_lora_bwd_params(M, H, NQ, NV, scaling, strided):
    """The parameter gradients (reductions over the rows, per-128-row slices added in order):
    fp16 roundings of the exact sums, as fp32, with gs = fp16(g * scaling) formed from g (rows
    of a wider buffer, as the attention backward hands them over, or contiguous)."""
    print(f"lora bwd params M={M} H={H} NQ={NQ} NV={NV} s={scaling} strided={strided}",
          flush=True)
    g = torch.Generator().manual_seed(M + H)

    def f16(*shape, sd):
        return (sd * torch.randn(*shape, generator=g)).to(torch.float16).to(DEV)

    y, t, dt = f16(M, H, sd=1.0), f16(M, 32, sd=0.5), f16(M, 32, sd=0.01)
    if strided:
        wide = f16(M, NQ + 2 * NV, sd=0.01)
        g_q, g_v = wide[:, :NQ], wide[:, NQ + NV:]
    else:
        g_q, g_v = f16(M, NQ, sd=0.01), f16(M, NV, sd=0.01)
    d_aq, d_av, d_bq, d_bv = lora.lora_bwd_params(y, t, dt, g_q, g_v, scaling)
    gs_q = (g_q.float() * scaling).to(torch.float16)
    gs_v = (g_v.float() * scaling).to(torch.float16)
    assert d_aq.dtype == torch.float32 and d_bq.shape == (NQ, 16) and d_bv.shape == (NV, 16)
    yd, td, dtd = y.double(), t.double(), dt.double()
    within_ulps(torch.cat([d_aq, d_av]), dtd.t() @ yd, 1, dtd.abs().t() @ yd.abs())
    within_ulps(d_bq, gs_q.double().t() @ td[:, :16], 1, gs_q.double().abs().t() @ td[:, :16].abs())
    within_ulps(d_bv, gs_v.double().t() @ td[:, 16:], 1, gs_v.double().abs().t() @ td[:, 16:].abs())


def test_lora_bwd_params_no_rows():
    e = torch.empty(0, 256, dtype=torch.float16, device=DEV)
    e32 = torch.empty(0, 32, dtype=torch.float16, device=DEV)
    out = lora.lora_bwd_params(e, e32, e32, e, torch.empty(0, 128, dtype=torch.float16,
                                                          device=DEV), 2.0)
    for x in out:
        assert torch.equal(x, torch.zeros_like(x))


def _bits(t):
    return t.detach().contiguous().view(torch.int16)


@pytest.mark.parametrize("lengths,T,NH,NKV,scaling", [
    ((512, 512, 512, 512), 512, 12, 2, 2.0),      # the step shape (M = 2048)
    ((512, 152, 128, 96), 512, 12, 2, 2.0),       # the BASELINE ragged batch (M = 888)
    ((17,), 40, 4, 2, 0.7),                        # one partial row block, a second part
    ((33, 0, 20), 64, 2, 1, 1.0)])                 # an empty row, one head pair per part
def test_lora_rope_fwd_matches_lora_then_rope(lengths, T, NH, NKV, scaling):
    """soupk_lora_rope_fwd writes t as soupk_lora_fwd does and the rows
    soupk_rope_pack_tokens writes from lora_fwd's lq / lv: both bit for bit.  One position is
    made invalid: its row is zeros in both."""
    print(f"lora+rope fwd lengths={lengths} T={T} NH={NH} NKV={NKV} s={scaling}", flush=True)
    from testt_amd import rope

    D, H = 128, 512 if NH < 12 else 1536
    NQ, NV = NH * D, NKV * D
    a_q, a_v, b_q, b_v = params(H, NQ, NV, sum(lengths) + NH)
    qkv, _, _, pos = workloads.rope_inputs(lengths, T, NH, NKV, D, seed=T + NH, device=DEV)
    M = pos.numel()
    if M > 3:
        pos[3] = -1
    g = torch.Generator().manual_seed(M)
    y = torch.randn(M, H, generator=g).to(torch.float16).to(DEV)
    cos, sin = workloads.rope_tables(T, D, workloads.ROPE_THETA, device=DEV)
    B = len(lengths)
    st = lora.stage(a_q, a_v, b_q, b_v)
    t_ref, lq, lv = lora.lora_fwd(y, a_q, a_v, b_q, b_v, scaling, staged=st)
    rows_ref, _, _, _ = rope.rope_pack_tokens(qkv, lq, lv, cos, sin, pos, B, T, NH, NKV, D)
    t, rows, _, _, _ = lora.lora_rope_fwd(y, a_q, a_v, b_q, b_v, scaling, qkv, cos, sin, pos, B,
                                          T, NH, NKV, staged=st)
    assert torch.equal(_bits(t), _bits(t_ref))
    assert torch.equal(_bits(rows), _bits(rows_ref))
    if M > 3:
        assert not bool(rows[3].any())


@pytest.mark.parametrize("lengths", [(512, 512, 512, 512), (512, 152, 128, 96), (40, 0, 7)])
def test_fused_lora_rope_layer_matches_unfused(monkeypatch, lengths):
    """decoder_layer with the q|k|v GEMM, LoRA + RoPE and attention in one node
    (QKVLoraRopeAttention) against QKVLora followed by RopeAttention: the layer's outputs and
    the gradients of the input and of every LoRA parameter are bit-identical."""
    print(f"fused LoRA+RoPE layer lengths={lengths}", flush=True)
    w = layer.synthetic_layer(DEV, seed=9)
    B, T = len(lengths), max(max(lengths), 1)
    pos = workloads.ragged_positions(lengths, T).to(DEV)
    M = pos.numel()
    g = torch.Generator().manual_seed(M)
    s0 = torch.randn(M, workloads.HIDDEN, generator=g).to(DEV)
    d0 = (0.5 * torch.randn(M, workloads.HIDDEN, generator=g)).to(torch.float16).to(DEV)
    gs = (1e-2 * torch.randn(M, workloads.HIDDEN, generator=g)).to(DEV)
    gd = (1e-2 * torch.randn(M, workloads.HIDDEN, generator=g)).to(torch.float16).to(DEV)
    cos, sin = workloads.rope_tables(T, workloads.HEAD_DIM, workloads.ROPE_THETA, device=DEV)
    results = []
    for fused in (True, False):
        monkeypatch.setattr(layer, "FUSE_LORA_ROPE", fused)
        s = s0.clone().requires_grad_(True)
        d = d0.clone().requires_grad_(True)
        for p in (*w.lora_q, *w.lora_v):
            p.grad = None
        so, do = layer.decoder_layer(s, d, w, pos, B, T, cos, sin, None)
        torch.autograd.backward([so, do], [gs, gd])
        results.append([so, do, s.grad, d.grad] + [p.grad.clone() for p in (*w.lora_q,
                                                                              *w.lora_v)])
    for name, a, b in zip(("s", "d", "ds", "dd", "dA_q", "dB_q", "dA_v", "dB_v"), *results):
        assert torch.equal(a.detach(), b.detach()), name
