"""GPU parity: the varlen path of the layer -- the token-major RoPE pack (soupk_rope_pack_tokens),
the causal GQA attention over each sequence's real tokens (soupk_attention_varlen_fwd/_bwd) and
its backward with RoPE's backward fused in -- against the padded path it replaces
(soupk_rope_pack_fwd, soupk_attention_fwd/_bwd with key flags, soupk_rope_pack_bwd), and the
attention against float32.

For right-padded rows a sequence's tokens sit at the same offsets in both layouts, so the two
paths run the same arithmetic in the same order: every output and gradient must be
bit-identical (torch.equal on the fp16 / fp32 bits).  The float32 comparison uses the
tolerances of tests/test_gpu_attention.py (outputs 2e-3 absolute, lse 1e-4 relative)."""

import math

import pytest
import torch

from tests.test_gpu_attention import reference
from testt_amd import attention, rope, workloads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
D = 128

# (lengths of the rows, padded row length T, query heads, key/value heads)
CASES = [
    ((512, 152, 128, 96), 512, 12, 2),     # the BASELINE ragged batch (M = 888)
    ((512, 512, 512, 512), 512, 12, 2),    # every position real (M = 2048)
    ((77, 0, 33, 1), 77, 12, 2),           # an empty row, T = 77, a one-token row
    ((130, 64), 130, 4, 4),
    ((1,), 1, 2, 1),
]


def _inputs(lengths, T, NH, NKV, seed, lora_dtype=torch.float32):
    qkv, lq, lv, pos = workloads.rope_inputs(lengths, T, NH, NKV, D, lora_dtype, seed=seed,
                                             device=DEV)
    cos, sin = workloads.rope_tables(T, D, workloads.ROPE_THETA, device=DEV)
    return qkv, lq, lv, pos, cos, sin


def _key_valid(lengths, T):
    valid = torch.zeros(len(lengths), T, dtype=torch.uint8)
    for b, n in enumerate(lengths):
        valid[b, :n] = 1
    return valid.to(DEV)


def _bits(t):
    return t.detach().contiguous().view(torch.int16) if t.dtype == torch.float16 else t.detach()


@pytest.mark.parametrize("lengths,T,NH,NKV", CASES)
@pytest.mark.parametrize("lora_dtype", [torch.float32, torch.float16])
def test_rope_pack_tokens_matches_padded(lengths, T, NH, NKV, lora_dtype):
    print(f"rope tokens lengths={lengths} T={T} NH={NH} NKV={NKV} lora={lora_dtype}", flush=True)
    B = len(lengths)
    qkv, lq, lv, pos, cos, sin = _inputs(lengths, T, NH, NKV, seed=sum(lengths) + T,
                                         lora_dtype=lora_dtype)
    rows, _, _, _ = rope.rope_pack_tokens(qkv, lq, lv, cos, sin, pos, B, T, NH, NKV, D)
    q, k, v = rope.rope_pack(qkv, lq, lv, cos, sin, pos, B, T, NH, NKV, D)
    M = pos.numel()
    bb, tt = pos // T, pos % T
    padded = torch.cat([q[bb, :, tt].reshape(M, -1), k[bb, :, tt].reshape(M, -1),
                        v[bb, :, tt].reshape(M, -1)], dim=1)
    assert torch.equal(_bits(rows), _bits(padded))


def test_rope_pack_tokens_position_outside_rows():
    """A token whose position has no place gets a zero row; the others are unaffected."""
    qkv, lq, lv, pos, cos, sin = _inputs((20, 7), 20, 12, 2, seed=5)
    ref, _, _, _ = rope.rope_pack_tokens(qkv, lq, lv, cos, sin, pos, 2, 20, 12, 2, D)
    bad = pos.clone()
    bad[3], bad[10] = -1, 2 * 20
    rows, _, _, _ = rope.rope_pack_tokens(qkv, lq, lv, cos, sin, bad, 2, 20, 12, 2, D)
    keep = torch.ones(pos.numel(), dtype=torch.bool, device=DEV)
    keep[3] = keep[10] = False
    assert torch.equal(_bits(rows[keep]), _bits(ref[keep]))
    assert not bool(rows[~keep].any())


def _padded_qkv(rows, lengths, T, NH, NKV, pos):
    """The padded q, k, v holding the token rows at their positions (zeros elsewhere)."""
    B, M = len(lengths), pos.numel()
    bb, tt = pos // T, pos % T
    q = torch.zeros(B, NH, T, D, dtype=torch.float16, device=DEV)
    k = torch.zeros(B, NKV, T, D, dtype=torch.float16, device=DEV)
    v = torch.zeros(B, NKV, T, D, dtype=torch.float16, device=DEV)
    q[bb, :, tt] = rows[:, :NH * D].reshape(M, NH, D)
    k[bb, :, tt] = rows[:, NH * D:(NH + NKV) * D].reshape(M, NKV, D)
    v[bb, :, tt] = rows[:, (NH + NKV) * D:].reshape(M, NKV, D)
    return q, k, v


@pytest.mark.parametrize("lengths,T,NH,NKV", CASES)
def test_varlen_forward_matches_padded_and_fp32(lengths, T, NH, NKV):
    print(f"varlen fwd lengths={lengths} T={T} NH={NH} NKV={NKV}", flush=True)
    B = len(lengths)
    g = torch.Generator().manual_seed(7 * T + NH)
    pos = workloads.ragged_positions(lengths, T).to(DEV)
    M = pos.numel()
    rows = torch.randn(M, (NH + 2 * NKV) * D, generator=g).to(torch.float16).to(DEV)
    cu = attention.cu_seqlens_of(pos, B, T)
    assert cu.tolist() == [0] + torch.tensor(lengths).cumsum(0).tolist()
    scale = 1.0 / math.sqrt(D)
    out, lse = attention.attention_varlen_fwd(rows, cu, NH, NKV, scale)
    q, k, v = _padded_qkv(rows, lengths, T, NH, NKV, pos)
    valid = _key_valid(lengths, T)
    p_out, p_lse = attention.attention_fwd(q, k, v, valid, scale)
    assert torch.equal(_bits(out), _bits(p_out.index_select(0, pos)))
    bb, tt = pos // T, pos % T
    assert torch.equal(lse, p_lse[bb, :, tt].t())
    r_out, r_lse = reference(q.cpu(), k.cpu(), v.cpu(), valid.cpu(), scale)
    r_rows = r_out.reshape(B * T, -1)[pos.cpu()]
    err = (out.cpu().float() - r_rows).abs().max().item() if M else 0.0
    print(f"  max |out - fp32| = {err:.2e}", flush=True)
    assert err < 2e-3
    rl = r_lse[bb.cpu(), :, tt.cpu()].t()
    assert ((lse.cpu() - rl).abs() <= 1e-4 * rl.abs() + 1e-5).all()


def test_varlen_sequences_from_bounds_alone():
    """The varlen kernels need only the sequence bounds: a sequence of 700 tokens and one of
    188 (no padded row length involved; the grid covers any split of the M tokens) match the
    padded kernels on rows of T = 700, forward and backward, bit for bit."""
    lengths, T, NH, NKV = (700, 188), 700, 12, 2
    B = len(lengths)
    g = torch.Generator().manual_seed(21)
    pos = workloads.ragged_positions(lengths, T).to(DEV)
    M = pos.numel()
    rows = torch.randn(M, (NH + 2 * NKV) * D, generator=g).to(torch.float16).to(DEV)
    dout = torch.randn(M, NH * D, generator=g).to(torch.float16).to(DEV)
    cu = torch.tensor([0, 700, 888], dtype=torch.int32, device=DEV)
    scale = 1.0 / math.sqrt(D)
    out, lse = attention.attention_varlen_fwd(rows, cu, NH, NKV, scale)
    dqkv = attention.attention_varlen_bwd(rows, cu, out, lse, dout, scale, NH, NKV)
    q, k, v = _padded_qkv(rows, lengths, T, NH, NKV, pos)
    valid = _key_valid(lengths, T)
    p_out, p_lse = attention.attention_fwd(q, k, v, valid, scale)
    assert torch.equal(_bits(out), _bits(p_out.index_select(0, pos)))
    p_dout = torch.zeros(B * T, NH * D, dtype=torch.float16, device=DEV)
    p_dout[pos] = dout
    dq, dk, dv = attention.attention_bwd(q, k, v, valid, p_out, p_lse, p_dout, scale)
    bb, tt = pos // T, pos % T
    gathered = torch.cat([dq[bb, :, tt].reshape(M, -1), dk[bb, :, tt].reshape(M, -1),
                          dv[bb, :, tt].reshape(M, -1)], dim=1)
    assert torch.equal(_bits(dqkv), _bits(gathered))


@pytest.mark.parametrize("lengths,T,NH,NKV", CASES)
def test_varlen_backward_matches_padded(lengths, T, NH, NKV):
    """Without tables the varlen backward's rows are the padded backward's dq, dk, dv at the
    tokens' positions; with the RoPE tables they are soupk_rope_pack_bwd of those."""
    print(f"varlen bwd lengths={lengths} T={T} NH={NH} NKV={NKV}", flush=True)
    B = len(lengths)
    g = torch.Generator().manual_seed(5 * T + NH)
    pos = workloads.ragged_positions(lengths, T).to(DEV)
    M = pos.numel()
    rows = torch.randn(M, (NH + 2 * NKV) * D, generator=g).to(torch.float16).to(DEV)
    dout = torch.randn(M, NH * D, generator=g).to(torch.float16).to(DEV)
    cos, sin = workloads.rope_tables(T, D, workloads.ROPE_THETA, device=DEV)
    cu = attention.cu_seqlens_of(pos, B, T)
    scale = 1.0 / math.sqrt(D)
    out, lse = attention.attention_varlen_fwd(rows, cu, NH, NKV, scale)
    plain = attention.attention_varlen_bwd(rows, cu, out, lse, dout, scale, NH, NKV)
    fused = attention.attention_varlen_bwd(rows, cu, out, lse, dout, scale, NH, NKV,
                                           rope=(cos, sin, pos, B, T))
    q, k, v = _padded_qkv(rows, lengths, T, NH, NKV, pos)
    valid = _key_valid(lengths, T)
    p_out, p_lse = attention.attention_fwd(q, k, v, valid, scale)
    p_dout = torch.zeros(B * T, NH * D, dtype=torch.float16, device=DEV)
    p_dout[pos] = dout
    dq, dk, dv = attention.attention_bwd(q, k, v, valid, p_out, p_lse, p_dout, scale)
    bb, tt = pos // T, pos % T
    gathered = torch.cat([dq[bb, :, tt].reshape(M, -1), dk[bb, :, tt].reshape(M, -1),
                          dv[bb, :, tt].reshape(M, -1)], dim=1)
    assert torch.equal(_bits(plain), _bits(gathered))
    composed = torch.empty_like(rows)
    from testt_amd import _ext
    if M:
        _ext.call("soupk_rope_pack_bwd", _ext.ptr(dq), _ext.ptr(dk), _ext.ptr(dv),
                  _ext.ptr(cos), _ext.ptr(sin), _ext.ptr(pos), _ext.ptr(composed), M, B, T, NH,
                  NKV, D, _ext.stream_of(composed))
    assert torch.equal(_bits(fused), _bits(composed))


@pytest.mark.parametrize("lengths,T", [((512, 152, 128, 96), 512), ((77, 0, 33, 1), 77)])
def test_rope_attention_autograd_matches_padded_path(lengths, T):
    """RopeAttention (one node: token-major pack, varlen attention, fused backward) against
    the layer's former path RopePack -> CausalAttention -> gather of the real rows: the output
    and the gradients of qkv, lora_q and lora_v are bit-identical."""
    NH, NKV, B = 12, 2, len(lengths)
    qkv, lq, lv, pos, cos, sin = _inputs(lengths, T, NH, NKV, seed=3 * T + B,
                                         lora_dtype=torch.float16)
    M = pos.numel()
    g = torch.Generator().manual_seed(T)
    dout = torch.randn(M, NH * D, generator=g).to(torch.float16).to(DEV)
    cu = attention.cu_seqlens_of(pos, B, T)

    leaves_a = [t.clone().requires_grad_(True) for t in (qkv, lq, lv)]
    out_a = attention.rope_attention(*leaves_a, cos, sin, pos, cu, B, T, NH, NKV)
    out_a.backward(dout)

    leaves_b = [t.clone().requires_grad_(True) for t in (qkv, lq, lv)]
    q, k, v = rope.rope_pack(*leaves_b, cos, sin, pos, B, T, NH, NKV, D)
    out_b = attention.causal_attention(q, k, v, _key_valid(lengths, T)).index_select(0, pos)
    out_b.backward(dout)

    assert torch.equal(_bits(out_a), _bits(out_b))
    for name, a, b in zip(("qkv", "lora_q", "lora_v"), leaves_a, leaves_b):
        assert torch.equal(_bits(a.grad), _bits(b.grad)), name


def test_varlen_backward_rejects_mismatched_inputs():
    """attention_varlen_bwd checks every tensor it hands the kernels (shapes, dtypes, the RoPE
    tables' rows) before launching: a short lse or table would be read past its end."""
    M, NH, NKV, D = 40, 4, 2, 128
    W = (NH + 2 * NKV) * D
    qkv = torch.zeros(M, W, dtype=torch.float16, device=DEV)
    cu = torch.tensor([0, 25, 40], dtype=torch.int32, device=DEV)
    out = torch.zeros(M, NH * D, dtype=torch.float16, device=DEV)
    lse = torch.zeros(NH, M, dtype=torch.float32, device=DEV)
    dout = torch.zeros_like(out)
    cos = torch.ones(32, D, device=DEV)
    sin = torch.zeros(32, D, device=DEV)
    pos = torch.arange(M, device=DEV)
    good = dict(qkv_r=qkv, cu_seqlens=cu, out=out, lse=lse, dout=dout, scale=0.1, n_heads=NH,
                n_kv=NKV, rope=(cos, sin, pos, 2, 32))
    attention.attention_varlen_bwd(**good)
    torch.cuda.synchronize()
    bad = [dict(lse=lse[:, :M - 1].contiguous()), dict(lse=lse.t().contiguous()),
           dict(out=out[:M - 1]), dict(cu_seqlens=cu.long()),
           dict(rope=(cos[:20].contiguous(), sin, pos, 2, 32)),
           dict(rope=(cos, sin, pos[:M - 1], 2, 32)), dict(qkv_r=qkv[:, :W - 8].contiguous())]
    for change in bad:
        with pytest.raises((ValueError, TypeError)):
            attention.attention_varlen_bwd(**{**good, **change})


def _rope32(x, cos_t, sin_t, heads):
    """float32 rotation of [M, heads*D] rows by per-token tables [M, D] (rotate_half form)."""
    M = x.shape[0]
    h = x.view(M, heads, D)
    rot = torch.cat([-h[..., D // 2:], h[..., :D // 2]], dim=-1)
    return (h * cos_t[:, None] + rot * sin_t[:, None]).reshape(M, heads * D)


def _reference_rope_attention(qkv, lq, lv, cos, sin, pos, mask, NH, NKV, dout, scale):
    """float32 (CPU) RoPE + causal GQA attention over the padded layout with the key-padding
    mask of `mask`, gathered at the real tokens, and its gradients for qkv, lq, lv."""
    B, T = mask.shape
    M = pos.numel()
    leaves = [t.detach().cpu().float().requires_grad_(True) for t in (qkv, lq, lv)]
    x, lq32, lv32 = leaves
    pos = pos.cpu()
    tt = pos % T
    c, s = cos.cpu()[tt], sin.cpu()[tt]
    q = _rope32(x[:, :NH * D] + lq32, c, s, NH)
    k = _rope32(x[:, NH * D:(NH + NKV) * D], c, s, NKV)
    v = x[:, (NH + NKV) * D:] + lv32

    def padded(rows, heads):
        flat = torch.zeros(B * T, heads * D).index_copy(0, pos, rows)
        return flat.view(B, T, heads, D).transpose(1, 2)

    qp, kp, vp = padded(q, NH), padded(k, NKV), padded(v, NKV)
    rep = NH // NKV
    kp, vp = kp.repeat_interleave(rep, 1), vp.repeat_interleave(rep, 1)
    allowed = torch.ones(T, T, dtype=torch.bool).tril()[None, None] & \
        mask.cpu().bool()[:, None, None, :]
    allowed = allowed | torch.eye(T, dtype=torch.bool)[None, None]   # pad queries: finite rows
    sc = (qp @ kp.transpose(-1, -2)) * scale
    p = torch.softmax(sc.masked_fill(~allowed, float("-inf")), -1)
    out = (p @ vp).transpose(1, 2).reshape(B * T, NH * D)[pos]
    out.backward(dout.detach().cpu().float())
    return out.detach(), [t.grad for t in leaves]


def _mask(kind, B, T):
    m = torch.zeros(B, T, dtype=torch.int64)
    if kind == "left":          # the BASELINE ragged lengths, left-aligned (prompt padding)
        for b, n in enumerate((512, 152, 128, 96)[:B]):
            m[b, T - n:] = 1
    else:                       # pads inside rows, at both ends and in runs of several lengths
        m[0, 20:] = 1
        m[1, :10] = 1
        m[1, 30:61] = 1
        m[2] = (torch.arange(T) % 3 != 1).long()
        m[3, 5:6] = 1
    return m.to(DEV)


@pytest.mark.parametrize("kind,T", [("left", 512), ("gaps", 77)])
def test_rope_attention_left_padding_and_gaps(kind, T):
    """Masks whose real tokens are not a prefix of each row: left padding (TRL's padded
    prompts) and pads between real tokens.  The varlen path attends within each row's real
    tokens in index order (= position order); RoPE uses the tokens' true positions.  Against
    the padded path (RopePack -> causal attention with the key flags -> gather) and the float32
    reference: outputs within 2e-3 absolute, the qkv / LoRA gradients within 1e-2 relative
    (L2 norm)."""
    NH, NKV, B = 12, 2, 4
    mask = _mask(kind, B, T)
    pos = mask.reshape(-1).nonzero().squeeze(1)
    M = pos.numel()
    print(f"rope attention {kind} mask T={T} M={M}", flush=True)
    g = torch.Generator().manual_seed(17 + T)
    width = (NH + 2 * NKV) * D
    qkv = torch.randn(M, width, generator=g).to(torch.float16).to(DEV)
    lq = (1e-2 * torch.randn(M, NH * D, generator=g)).to(torch.float16).to(DEV)
    lv = (1e-2 * torch.randn(M, NKV * D, generator=g)).to(torch.float16).to(DEV)
    dout = torch.randn(M, NH * D, generator=g).to(torch.float16).to(DEV)
    cos, sin = workloads.rope_tables(T, D, workloads.ROPE_THETA, device=DEV)
    cu = attention.cu_seqlens_of(pos, B, T)
    assert cu.tolist() == [0] + mask.sum(1).cumsum(0).tolist()
    scale = 1.0 / math.sqrt(D)

    leaves_a = [t.clone().requires_grad_(True) for t in (qkv, lq, lv)]
    out_a = attention.rope_attention(*leaves_a, cos, sin, pos, cu, B, T, NH, NKV)
    out_a.backward(dout)

    leaves_b = [t.clone().requires_grad_(True) for t in (qkv, lq, lv)]
    q, k, v = rope.rope_pack(*leaves_b, cos, sin, pos, B, T, NH, NKV, D)
    key_valid = (mask != 0).to(torch.uint8).contiguous()
    out_b = attention.causal_attention(q, k, v, key_valid).index_select(0, pos)
    out_b.backward(dout)

    r_out, r_grads = _reference_rope_attention(qkv, lq, lv, cos, sin, pos, mask, NH, NKV,
                                               dout, scale)
    err_ref = (out_a.detach().cpu().float() - r_out).abs().max().item()
    err_pad = (out_a.detach().float() - out_b.detach().float()).abs().max().item()
    print(f"  max |out - fp32| = {err_ref:.2e}, |varlen - padded| = {err_pad:.2e}", flush=True)
    assert err_ref < 2e-3 and err_pad < 2e-3
    for name, a, b, r in zip(("qkv", "lora_q", "lora_v"), leaves_a, leaves_b, r_grads):
        ga = a.grad.cpu().float()
        rel_ref = float((ga - r).norm() / r.norm())
        rel_pad = float((ga - b.grad.cpu().float()).norm() / b.grad.cpu().float().norm())
        print(f"  grad {name}: rel to fp32 {rel_ref:.1e}, to padded {rel_pad:.1e}", flush=True)
        assert rel_ref < 1e-2 and rel_pad < 1e-2, name
