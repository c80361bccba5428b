"""One Qwen2 decoder layer of the QLoRA training step, wired from the drop-in ops.

Mirrors the per-layer body of the reference's fused_forward (solution/model.py:235-255) on the
real (non-pad) tokens:

  s, y, y_pad = add_rmsnorm(s, d)               residual add + input RMSNorm (HIP)
  (all seven NF4 projections unpacked by one HIP launch: UNPACK_PER_LAYER; with few tokens
   the products read the NF4 weights through the fused NF4-dequant GEMM instead:
   NF4_RESIDENT_SMALL_BATCHES)
  qkv        = y @ [Wq;Wk;Wv]^T + b               one hipBLASLt GEMM
  lq, lv     = B(A(dropout(y_pad))) * scaling     LoRA on q/v (HIP, or fp16 GEMMs with dropout)
  a          = rope_attention(qkv, lq, lv)        LoRA add + RoPE into token-major rows, then
                                                  causal GQA flash attention over each row's
                                                  real tokens (HIP; varlen, no padding)
  o          = a @ Wo^T                           hipBLASLt
  s, y2, _   = add_rmsnorm(s, o)                  residual add + post-attention RMSNorm (HIP)
  d          = mlp(y2)                            GEMM + SwiGLU (HIP) + GEMM

The reference takes these modules from a PEFT/bitsandbytes model; here they are plain tensors
(`LayerWeights`), so one layer can be built from synthetic NF4 weights for measurement and
tests.  The LoRA branch follows peft's `lora_B(lora_A(dropout(x))) * scaling` under fp16
autocast (the matmuls in fp16, on the fp32 padded norm output so the dropout draws match).

Without dropout the LoRA input fp16(y_pad[pos]) is exactly the fp16 norm output y that the
projection GEMM reads (the norm kernel rounds the same fp32 value into both), so `QKVLora`
runs the projection and both LoRA branches on y in one autograd node: A_q|A_v as one skinny
GEMM, no padded fp32 copy, gather, casts or scatter-add, and in backward the LoRA input
gradient accumulated into the projection's input-gradient GEMM.  The norm then writes no padded
output at all.  With dropout the reference's path is kept (the padded layout fixes the draws).
"""

import math
from dataclasses import dataclass

import torch

from . import attention as _attention
from . import blas as _blas
from . import layer_native as _native
from . import lora as _lora
from . import workloads
from .mlp import FusedNF4MLP, fused_mlp
from .nf4 import (FrozenNF4Linear, frozen_linear, fused_grad_input, fused_linear,
                  keep_for_backward, unpack_concat, unpack_groups,
                  unpack_groups_lora, unpacked_for_backward)
from .rmsnorm import AddRMSNorm, RMSNormNoAdd, add_rmsnorm
from .rope import rope_pack


@dataclass
class LayerWeights:
    input_norm: torch.Tensor        # fp32 [H]
    post_norm: torch.Tensor         # fp32 [H]
    q: object                       # Params4bit-like NF4 weights (.data, .quant_state)
    k: object
    v: object
    o: object
    gate: object
    up: object
    down: object
    qkv_bias: torch.Tensor          # fp16 [(NH + 2*NKV) * D], or None
    lora_q: tuple                   # (A fp32 [r, H], B fp32 [NH*D, r]) trainable, or None
    lora_v: tuple                   # (A fp32 [r, H], B fp32 [NKV*D, r]) trainable, or None
    scaling: float                  # LoRA scaling of q (and of v unless scaling_v is given)
    n_heads: int
    n_kv: int
    head_dim: int
    eps: float = 1e-6
    dropout: float = 0.0            # LoRA dropout probability (when lora_dropout is None)
    o_bias: torch.Tensor = None     # fp16 [H], or None
    scaling_v: float = None         # LoRA scaling of v when it differs from q's
    lora_dropout: tuple = None      # (q, v) dropout modules to call (peft's), instead of dropout
    attn_scale: float = None        # attention softmax scale (None: 1/sqrt(head_dim))


def synthetic_layer(device, hidden=workloads.HIDDEN, inter=workloads.INTER,
                    n_heads=workloads.N_HEADS, n_kv=workloads.N_KV, head_dim=workloads.HEAD_DIM,
                    rank=16, alpha=32, dropout=0.0, seed=9):
    """A Qwen2.5-1.5B-shaped layer: synthetic NF4 projections, LoRA r=16 on q/v."""
    g = workloads.gen(seed)
    qd, kvd = n_heads * head_dim, n_kv * head_dim
    shapes = {"q": (qd, hidden), "k": (kvd, hidden), "v": (kvd, hidden), "o": (hidden, qd),
              "gate": (inter, hidden), "up": (inter, hidden), "down": (hidden, inter)}
    nf4w = {name: workloads.nf4_weight(*shape, seed=seed * 100 + i, device=device,
                                       absmax2_range=(0.005, 0.02), offset=0.01)
            for i, (name, shape) in enumerate(shapes.items())}

    def lora(out_dim):
        a = (torch.randn(rank, hidden, generator=g) / math.sqrt(hidden)).to(device)
        b = (0.05 * torch.randn(out_dim, rank, generator=g)).to(device)
        return a.requires_grad_(True), b.requires_grad_(True)

    return LayerWeights(
        input_norm=(1 + 0.02 * torch.randn(hidden, generator=g)).to(device),
        post_norm=(1 + 0.02 * torch.randn(hidden, generator=g)).to(device),
        qkv_bias=(0.1 * torch.randn(qd + 2 * kvd, generator=g)).to(torch.float16).to(device),
        lora_q=lora(qd), lora_v=lora(kvd), scaling=alpha / rank, n_heads=n_heads, n_kv=n_kv,
        head_dim=head_dim, dropout=dropout, **nf4w)


# Rank-16 LoRA through testt_amd/csrc/lora.hip (False: the separate fp16 GEMMs below).
USE_FUSED_LORA = True

# Attention over each sequence's real tokens (attention.RopeAttention: token-major RoPE pack,
# varlen attention, RoPE's backward inside the attention backward) for head dim 128; False
# keeps the padded path (RopePack into [B, heads, T, D], attention with key flags, a gather of
# the real rows), which gives bit-identical results for right-padded batches.
USE_VARLEN_ATTENTION = True

# The seven projections of a layer unpacked by one launch before its forward (one buffer, the
# row stacks q|k|v, o, gate|up, down as views), instead of one launch per stack where each is
# used (the reference's order, solution/nf4.py:125 and solution/mlp.py:105-108).  The fp16
# values are the same; the whole buffer lives until the last stack is released (the backward
# of q|k|v when the weights are kept for backward, the end of the layer's forward otherwise).
UNPACK_PER_LAYER = True
# A layer whose token count is small enough that each of its products takes the fused
# NF4-dequant GEMM, forward and input gradient (nf4_gemm's measured window: up to 128 rows at
# Qwen2.5-1.5B's shapes on MI355X), skips that unpack and runs on the NF4 weights: no fp16 copy
# of the layer's weights (94 MB in Qwen2.5-1.5B) is written or read.  Issued from C like the
# unpacked layer (layer_native, dims.nf4).  Measured (bench.py --nf4-resident, forward +
# backward at 16 / 64 / 128 tokens): eager 222 / 220 / 221 us against 303 us unpacked, GPU
# time (graph replay) 186 / 201 / 218 us against 232 / 218 / 232 us.
NF4_RESIDENT_SMALL_BATCHES = True
# Up to this many tokens the layer runs on its NF4 weights whenever their layout allows, also
# where single products measured faster through unpack + hipBLASLt (the layer's sum is what
# counts: it saves the unpack launch, and the products it loses are offset by those it wins).
NF4_RESIDENT_MAX_TOKENS = 0


def nf4_resident(tokens, groups, device):
    """True when a layer of `tokens` rows runs on its NF4 weights (NF4_RESIDENT_SMALL_BATCHES).
    The answer is remembered on the first weight per token count, device and weight state."""
    from . import nf4, nf4_gemm

    if tokens <= 0 or not nf4.USE_FUSED_NF4_GEMM:
        return False
    key = (tokens, device, tuple(nf4._plan_key(x, device) for g in groups for x in g))
    first = groups[0][0]
    memo = getattr(first, "_soupk_resident", None)
    if memo is None:
        memo = {}
        try:
            setattr(first, "_soupk_resident", memo)
        except AttributeError:        # an object that takes no attributes: not remembered
            pass
    key = key + (tokens <= NF4_RESIDENT_MAX_TOKENS,)
    hit = memo.get(key)
    if hit is None:
        if len(memo) > 256:
            memo.clear()
        hit = memo[key] = nf4_gemm.prefers_fused_all(tokens, groups, device,
                                                     window=not key[-1])
    return hit


def _qkv_forward(ctx, y16, weights, w16, bias):
    """y16 @ [Wq;Wk;Wv]^T + b: without the caller's unpacked stack `w16`, the fused NF4-dequant
    GEMM where it is the faster path (few rows); else hipBLASLt on the unpacked stack, which is
    kept for backward (nf4.KEEP_UNPACKED_FOR_BACKWARD)."""
    qkv = fused_linear(y16, weights, bias) if w16 is None else None
    if qkv is not None:
        ctx.unpacked = None
        return qkv
    w = w16 if w16 is not None else unpack_concat(weights, y16.device)
    qkv = _blas.linear(y16, w, bias)
    keep_for_backward(ctx, w)
    return qkv


def _add_qkv_input_grad(ctx, g_qkv, dy):
    """dy += g_qkv @ [Wq;Wk;Wv] (fp16): one accumulating hipBLASLt GEMM on the kept or
    re-unpacked stack, or, where no stack was kept and it is the faster path, the fused NF4
    input gradient added to dy (rounded twice: the product, then the sum)."""
    g = g_qkv.to(torch.float16)
    dx = fused_grad_input(g, ctx.weights) if getattr(ctx, "unpacked", None) is None else None
    if dx is not None:
        dy += dx
        return dy
    w = unpacked_for_backward(ctx, ctx.weights, dy.device)
    _blas.matmul(g, w, out=dy, accumulate=True)
    return dy


class QKVLora(torch.autograd.Function):
    """(qkv, lora_q, lora_v) from the fp16 norm output y, for LoRA without dropout:
    qkv = y @ [Wq;Wk;Wv]^T + b (frozen NF4; the unpacked weight kept for backward, or unpacked
    again there: nf4.KEEP_UNPACKED_FOR_BACKWARD) and
    lora_x = fp16(fp16(fp16(y @ fp16(A_x)^T) @ fp16(B_x)^T) * scaling), peft's branch under fp16
    autocast (solution/model.py:195-206 with dropout p = 0)."""

    @staticmethod
    def forward(ctx, y16, bias, a_q, b_q, a_v, b_v, scaling, weights, w16=None, staged=None):
        qkv = _qkv_forward(ctx, y16, weights, w16, bias)
        ctx.weights, ctx.scaling = weights, scaling
        params = (a_q.detach(), a_v.detach(), b_q.detach(), b_v.detach())
        ctx.fused = USE_FUSED_LORA and _lora.supported(y16, *params)
        if ctx.fused:       # testt_amd/csrc/lora.hip: the parameters' fp16 casts, then t, lq, lv
            if staged is None:   # (else staged by the layer's weight launch, unpack_groups_lora)
                staged = _lora.stage(*params)
            t, lq, lv = _lora.lora_fwd(y16, *params, scaling, staged=staged)
            ctx.save_for_backward(y16, t, *params, staged)
            return qkv, lq, lv
        r = a_q.shape[0]
        a16 = torch.cat([a_q.detach(), a_v.detach()]).to(torch.float16)
        t = y16 @ a16.t()
        bq16 = b_q.detach().to(torch.float16)
        bv16 = b_v.detach().to(torch.float16)
        lq = t[:, :r] @ bq16.t()
        lv = t[:, r:] @ bv16.t()
        if scaling != 1.0:
            lq.mul_(scaling)
            lv.mul_(scaling)
        ctx.save_for_backward(y16, t, a16, bq16, bv16)
        ctx.rank = r
        return qkv, lq, lv

    @staticmethod
    def backward(ctx, g_qkv, g_lq, g_lv):
        if ctx.fused:
            return QKVLora._backward_fused(ctx, g_qkv, g_lq, g_lv)
        y16, t, a16, bq16, bv16 = ctx.saved_tensors
        s, r = ctx.scaling, ctx.rank
        m = y16.shape[0]
        dt = torch.zeros((m, 2 * r), dtype=torch.float16, device=y16.device)
        grads = [None, None, None, None]   # dA_q, dB_q, dA_v, dB_v
        for i, (g, b16) in enumerate(((g_lq, bq16), (g_lv, bv16))):
            if g is None:
                continue
            g = g.to(torch.float16)
            if s != 1.0:
                g = g * s                  # the grad of `* scaling` (fp16, as autograd does)
            torch.mm(g, b16, out=dt[:, i * r:(i + 1) * r])
            # fp16 products cast to the fp32 parameters, as autocast's backward gives them
            grads[2 * i + 1] = (g.t() @ t[:, i * r:(i + 1) * r]).float()
        da = (dt.t() @ y16).float()
        grads[0], grads[2] = da[:r], da[r:]
        dy = dt @ a16
        if g_qkv is not None:
            _add_qkv_input_grad(ctx, g_qkv, dy)
        return dy, None, grads[0], grads[1], grads[2], grads[3], None, None, None, None

    @staticmethod
    def _backward_fused(ctx, g_qkv, g_lq, g_lv):
        y16, t, a_q, a_v, b_q, b_v, staged = ctx.saved_tensors
        m, dev = y16.shape[0], y16.device
        g_lq = _lora.rows_view(g_lq, b_q.shape[0], m, dev)
        g_lv = _lora.rows_view(g_lv, b_v.shape[0], m, dev)
        dt, dy = _lora.lora_bwd_rows(g_lq, g_lv, a_q, a_v, b_q, b_v, ctx.scaling, staged=staged)
        # fp16 products cast to the fp32 parameters, as autocast's backward gives them
        d_aq, d_av, d_bq, d_bv = _lora.lora_bwd_params(y16, t, dt, g_lq, g_lv, ctx.scaling)
        if g_qkv is not None:
            _add_qkv_input_grad(ctx, g_qkv, dy)
        return dy, None, d_aq, d_bq, d_av, d_bv, None, None, None, None


# The rank-16 LoRA forward and the RoPE pack of the varlen attention in one launch
# (soupk_lora_rope_fwd: the rotated q|k|v rows written directly, no lq / lv in memory and no
# rope_pack_tokens launch), with the q|k|v GEMM, the LoRA and the attention in one autograd node
# (QKVLoraRopeAttention).  False: QKVLora then attention.RopeAttention, bit-identical values.
FUSE_LORA_ROPE = True


class QKVLoraRopeAttention(torch.autograd.Function):
    """out [M, NH*128] = varlen causal GQA attention of rotate(y @ [Wq;Wk;Wv]^T + b + LoRA), the
    forward of QKVLora followed by attention.RopeAttention in one node, for rank-16 LoRA without
    dropout and head dim 128: the q|k|v GEMM (hipBLASLt), soupk_lora_rope_fwd (t, and the
    rotated rows with the LoRA deltas added), the varlen attention.  The backward is theirs:
    the attention backward with RoPE's backward fused in gives the gradient of the q|k|v GEMM
    output, whose q and v columns are the LoRA deltas' gradients (views, as RopePack's backward
    returns them); then the LoRA backward and the frozen projection's input gradient."""

    @staticmethod
    def forward(ctx, y16, bias, a_q, b_q, a_v, b_v, scaling, weights, w16, staged, cos, sin,
                pos_idx, cu_seqlens, batch, seq, n_heads, n_kv, scale):
        qkv = _qkv_forward(ctx, y16, weights, w16, bias)
        params = (a_q.detach(), a_v.detach(), b_q.detach(), b_v.detach())
        if staged is None:
            staged = _lora.stage(*params)
        t, qkv_r, cos32, sin32, pos = _lora.lora_rope_fwd(y16, *params, scaling, qkv, cos, sin,
                                                          pos_idx, batch, seq, n_heads, n_kv,
                                                          staged=staged)
        del qkv
        out, lse = _attention.attention_varlen_fwd(qkv_r, cu_seqlens, n_heads, n_kv, scale)
        ctx.save_for_backward(y16, t, *params, staged, qkv_r, out, lse, cos32, sin32, pos,
                              cu_seqlens)
        ctx.weights, ctx.scaling = weights, scaling
        ctx.dims = (batch, seq, n_heads, n_kv, scale)
        return out

    @staticmethod
    def backward(ctx, dout):
        (y16, t, a_q, a_v, b_q, b_v, staged, qkv_r, out, lse, cos, sin, pos,
         cu) = ctx.saved_tensors
        batch, seq, n_heads, n_kv, scale = ctx.dims
        dqkv = _attention.attention_varlen_bwd(qkv_r, cu, out, lse, dout, scale, n_heads, n_kv,
                                               rope=(cos, sin, pos, batch, seq))
        del qkv_r, out, lse
        m, dev = y16.shape[0], y16.device
        NQ, NV = b_q.shape[0], b_v.shape[0]
        g_lq = _lora.rows_view(dqkv[:, :NQ], NQ, m, dev)
        g_lv = _lora.rows_view(dqkv[:, NQ + NV:], NV, m, dev)
        dt, dy = _lora.lora_bwd_rows(g_lq, g_lv, a_q, a_v, b_q, b_v, ctx.scaling, staged=staged)
        # fp16 products cast to the fp32 parameters, as autocast's backward gives them
        d_aq, d_av, d_bq, d_bv = _lora.lora_bwd_params(y16, t, dt, g_lq, g_lv, ctx.scaling)
        _add_qkv_input_grad(ctx, dqkv, dy)
        return (dy, None, d_aq, d_bq, d_av, d_bv) + (None,) * 13


def lora_branch(y_pad, ab, scaling, dropout, batch, seq, pos_idx):
    """peft's B(A(dropout(x))) * scaling for the real tokens, fp16 matmuls (solution/model.py:
    195-206): the dropout runs on the padded fp32 norm output, A and B on the real rows.
    `dropout` is a probability or a dropout module to call (peft's own, so that its training
    flag and the random draws are the unpatched model's)."""
    a, b = ab
    hidden = y_pad.shape[-1]
    x = y_pad.view(batch, seq, hidden)
    if callable(dropout):
        dropped = dropout(x)
    else:
        dropped = torch.nn.functional.dropout(x, dropout, training=dropout > 0)
    dropped = dropped.view(batch * seq, hidden)
    rows = dropped.index_select(0, pos_idx).to(torch.float16)
    return (rows @ a.to(torch.float16).t()) @ b.to(torch.float16).t() * scaling


def attention(q, k, v, key_valid, scale=None):
    """Causal GQA attention of the padded [B, heads, T, D] layout -> token-major [B*T, NH*D].

    Query i of row b sees key j iff j <= i and the key is real (key_valid[b, j] != 0; every key
    when key_valid is None): transformers' causal + padding mask.  Head dim 128 (Qwen2.5) runs
    testt_amd/csrc/attention.hip; other head dims torch's scaled_dot_product_attention on the
    same mask, as the reference runs every shape (solution/model.py:246-247)."""
    B, NH, T, D = q.shape
    if _attention.supported(q, k, v):
        return _attention.causal_attention(q, k, v, key_valid, scale)
    mask = None if key_valid is None else causal_pad_mask(key_valid)
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    if mask is None:
        a = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True,
                                                             scale=scale, enable_gqa=True)
    else:
        a = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=mask,
                                                             scale=scale, enable_gqa=True)
    return a.transpose(1, 2).reshape(B * T, NH * D)


def key_valid_of(attention_mask):
    """uint8 [B, T] key-is-real flags of a [B, T] attention_mask, or None when nothing is
    padded (the kernels then skip the flag reads)."""
    if bool(attention_mask.all()):
        return None
    return (attention_mask != 0).to(torch.uint8).contiguous()


def causal_pad_mask(attention_mask):
    """Boolean [B, 1, T, T] mask: causal and key-not-padding (None when nothing is padded)."""
    if bool(attention_mask.all()):
        return None
    batch, seq = attention_mask.shape
    causal = torch.ones(seq, seq, dtype=torch.bool, device=attention_mask.device).tril()
    mask = causal[None, None] & attention_mask.bool()[:, None, None, :]
    # a fully padded query row would be all False; let it see itself so SDPA stays finite
    eye = torch.eye(seq, dtype=torch.bool, device=attention_mask.device)[None, None]
    return mask | (eye & ~attention_mask.bool()[:, None, :, None])


def _dropout_p(module):
    if isinstance(module, torch.nn.Dropout) and module.training:
        return float(module.p)
    return 0.0


def lora_without_dropout(w):
    """True when the layer's LoRA runs as QKVLora: adapters on both q and v with one rank and
    one scaling, and no dropout drawn (p = 0, Identity, or a dropout module in eval mode)."""
    if w.lora_q is None or w.lora_v is None:
        return False
    if w.scaling_v is not None and w.scaling_v != w.scaling:
        return False
    if w.lora_q[0].shape[0] != w.lora_v[0].shape[0]:
        return False
    if w.lora_dropout is not None:
        return all(m is None or _dropout_p(m) == 0.0 for m in w.lora_dropout)
    return w.dropout == 0.0


# The layer's five autograd nodes (input norm, q|k|v + LoRA + RoPE + attention, o projection,
# post-attention norm, MLP) as one node whose forward and backward call theirs in order: the
# same kernels and the same values, bit for bit, with one node for the autograd engine to run
# instead of five (measured on the eager layer: the engine's per-node work and the Python around
# each node are host time the GPU waits for at the ragged batch).
ONE_NODE_LAYER = True


class _SubCtx:
    """The ctx of a node run inside another node's forward and backward: records what the node
    saves (the outer node saves it, so that outputs among it hold no reference cycle)."""

    def __init__(self, need):
        self.needs_input_grad = (need,) * 32
        self.saved = ()

    def save_for_backward(self, *tensors):
        self.saved = tensors


class DecoderLayer(torch.autograd.Function):
    """(s, d) of the fused path of decoder_layer as one autograd node."""

    @staticmethod
    def forward(ctx, s_in, delta, a_q, b_q, a_v, b_v, w, w_qkv, w_o, w_gu, w_d, staged, cos, sin,
                pos_idx, cu, batch, seq, scale):
        need = any(ctx.needs_input_grad)
        subs = [_SubCtx(need) for _ in range(5)]
        ctx.no_add = delta is None      # the first layer: the input norm without a residual add
        if ctx.no_add:
            s1 = s_in
            y, _ = RMSNormNoAdd.forward(subs[0], s_in, w.input_norm, w.eps, None, 0)
        else:
            s1, y, _ = AddRMSNorm.forward(subs[0], s_in, delta, w.input_norm, w.eps, None, 0)
        a = QKVLoraRopeAttention.forward(subs[1], y, w.qkv_bias, a_q, b_q, a_v, b_v, w.scaling,
                                         (w.q, w.k, w.v), w_qkv, staged, cos, sin, pos_idx, cu,
                                         batch, seq, w.n_heads, w.n_kv, scale)
        del y
        o = FrozenNF4Linear.forward(subs[2], a, w.o_bias, (w.o,), w_o)
        del a
        s2, y2, _ = AddRMSNorm.forward(subs[3], s1, o, w.post_norm, w.eps, None, 0)
        del s1, o
        d = FusedNF4MLP.forward(subs[4], y2, w.gate, w.up, w.down, w_gu, w_d)
        flat, counts = [], []
        for c in subs:
            flat.extend(c.saved)
            counts.append(len(c.saved))
            c.saved = ()
        ctx.save_for_backward(*flat)
        ctx.subs, ctx.counts = subs, counts
        return s2, d

    @staticmethod
    def backward(ctx, g_s, g_d):
        subs, saved, i = ctx.subs, ctx.saved_tensors, 0
        ctx.subs = None
        for c, n in zip(subs, ctx.counts):
            c.saved_tensors = saved[i:i + n]
            i += n
        del saved
        # each gradient in the dtype of the tensor it belongs to, as the engine casts it between
        # nodes: s fp32; the norm outputs, a and o fp16
        g_y2 = FusedNF4MLP.backward(subs[4], g_d)[0]
        g_s1, g_o = AddRMSNorm.backward(subs[3], g_s, g_y2.to(torch.float16), None)[:2]
        del g_y2
        g_a = FrozenNF4Linear.backward(subs[2], g_o.to(torch.float16))[0]
        del g_o
        r = QKVLoraRopeAttention.backward(subs[1], g_a.to(torch.float16))
        del g_a
        if ctx.no_add:
            # s_in is also the residual: its gradient adds the norm's (two terms, either order)
            g_s_in = RMSNormNoAdd.backward(subs[0], r[0].to(torch.float16), None)[0] + g_s1
            g_delta = None
        else:
            g_s_in, g_delta = AddRMSNorm.backward(subs[0], g_s1.to(torch.float32),
                                                  r[0].to(torch.float16), None)[:2]
        return (g_s_in, g_delta, r[2], r[3], r[4], r[5]) + (None,) * 13


def decoder_layer(s, delta, w, pos_idx, batch, seq, cos, sin, key_valid):
    """(s, d): the residual stream and the MLP output of one layer (the next layer's delta).
    key_valid: uint8 [batch, seq] (key_valid_of(attention_mask)), or None when nothing is
    padded."""
    padded = batch * seq
    nh, nkv, hd = w.n_heads, w.n_kv, w.head_dim
    plain = lora_without_dropout(w)
    params = (w.lora_q[0], w.lora_v[0], w.lora_q[1], w.lora_v[1]) if plain else None
    w_qkv = w_o = w_gu = w_d = staged = None
    groups = ((w.q, w.k, w.v), (w.o,), (w.gate, w.up), (w.down,))
    on_nf4 = NF4_RESIDENT_SMALL_BATCHES and nf4_resident(s.shape[0], groups, s.device)
    if UNPACK_PER_LAYER and not on_nf4:
        if plain and USE_FUSED_LORA and _lora.params_supported(*params, s.device):
            # the LoRA parameters' fp16 staging rides on the same launch as the unpack
            (w_qkv, w_o, w_gu, w_d), staged = unpack_groups_lora(
                groups, s.device, tuple(p.detach() for p in params))
        else:
            w_qkv, w_o, w_gu, w_d = unpack_groups(groups, s.device)
    if plain and FUSE_LORA_ROPE and USE_FUSED_LORA and USE_VARLEN_ATTENTION and \
            hd == _attention.HEAD_DIM and nkv > 0 and nh % nkv == 0 and \
            w.lora_q[1].shape[0] == nh * hd and w.lora_v[1].shape[0] == nkv * hd and \
            _lora.params_supported(*params, s.device):
        cu = _attention.cu_seqlens_of(pos_idx, batch, seq)
        scale = 1.0 / math.sqrt(hd) if w.attn_scale is None else float(w.attn_scale)
        native = _native.supported(s, delta, w, w_qkv, w_o, w_gu, w_d, staged)
        if on_nf4 and _native.supported_nf4(s, delta, w):
            # the C-issued layer on the NF4 weights; the LoRA parameters staged here, as the
            # unpack launch does for the unpacked layer
            staged = _lora.stage(*(p.detach() for p in params))
            native = True
        if ONE_NODE_LAYER and native:
            from .rope import _table
            from ._index import as_index

            return _native.NativeDecoderLayer.apply(
                s.contiguous(), None if delta is None else delta.contiguous(), *w.lora_q,
                *w.lora_v, w, w_qkv, w_o, w_gu, w_d, staged, _table(cos, seq, hd, "cos", s.device),
                _table(sin, seq, hd, "sin", s.device), as_index(pos_idx), cu, batch, seq, scale)
        if ONE_NODE_LAYER and w_o is not None and w_gu is not None and w_d is not None:
            return DecoderLayer.apply(s.contiguous(),
                                      None if delta is None else delta.contiguous(),
                                      *w.lora_q, *w.lora_v,
                                      w, w_qkv, w_o, w_gu, w_d, staged, cos, sin, pos_idx, cu,
                                      batch, seq, scale)
        s, y, _ = add_rmsnorm(s, delta, w.input_norm, w.eps)
        a = QKVLoraRopeAttention.apply(y, w.qkv_bias, *w.lora_q, *w.lora_v, w.scaling,
                                       (w.q, w.k, w.v), w_qkv, staged, cos, sin, pos_idx, cu,
                                       batch, seq, nh, nkv, scale)
        del w_qkv, staged
        return _layer_tail(s, a, w, w_o, w_gu, w_d)
    if plain:
        s, y, _ = add_rmsnorm(s, delta, w.input_norm, w.eps)
        qkv, lq, lv = QKVLora.apply(y, w.qkv_bias, *w.lora_q, *w.lora_v, w.scaling,
                                    (w.q, w.k, w.v), w_qkv, staged)
    else:
        any_lora = w.lora_q is not None or w.lora_v is not None
        if any_lora:
            s, y, y_pad = add_rmsnorm(s, delta, w.input_norm, w.eps, pos_idx, padded)
        else:
            s, y, _ = add_rmsnorm(s, delta, w.input_norm, w.eps)
        qkv = frozen_linear(y, (w.q, w.k, w.v), w.qkv_bias, w_qkv)
        drops = w.lora_dropout if w.lora_dropout is not None else (w.dropout, w.dropout)
        scales = (w.scaling, w.scaling if w.scaling_v is None else w.scaling_v)
        lq, lv = (None if ab is None else
                  lora_branch(y_pad, ab, sc, dr, batch, seq, pos_idx)
                  for ab, sc, dr in zip((w.lora_q, w.lora_v), scales, drops))
        if any_lora:
            del y_pad
    if USE_VARLEN_ATTENTION and _attention.varlen_supported(qkv, hd, nh, nkv):
        # the real tokens only: rows of batch row b are cu[b] .. cu[b+1] of the sorted pos_idx
        cu = _attention.cu_seqlens_of(pos_idx, batch, seq)
        a = _attention.rope_attention(qkv, lq, lv, cos, sin, pos_idx, cu, batch, seq, nh, nkv,
                                      w.attn_scale)
        del qkv, lq, lv, w_qkv
    else:
        q, k, v = rope_pack(qkv, lq, lv, cos, sin, pos_idx, batch, seq, nh, nkv, hd)
        del qkv, lq, lv, w_qkv
        a = attention(q, k, v, key_valid, w.attn_scale)
        del q, k, v
        if pos_idx.numel() != padded:       # nonzero() indices are sorted: all slots = identity
            a = a.index_select(0, pos_idx)
    return _layer_tail(s, a, w, w_o, w_gu, w_d)


def _layer_tail(s, a, w, w_o, w_gu, w_d):
    """o-projection, residual add + post-attention RMSNorm, MLP: (s, d)."""
    o = frozen_linear(a, (w.o,), w.o_bias, w_o)
    del a, w_o
    s, y2, _ = add_rmsnorm(s, o, w.post_norm, w.eps)
    d = fused_mlp(y2, w.gate, w.up, w.down, w_gu, w_d)
    return s, d
