"""Causal grouped-query attention on gfx950 (testt_amd/csrc/attention.hip), forward and
backward, in place of torch's scaled_dot_product_attention in the decoder layer
(solution/model.py:246-247 runs transformers' sdpa_attention_forward there).

Two layouts.  Varlen (what the layer runs): `RopeAttention` takes the q|k|v GEMM output of the
M real tokens and the LoRA deltas, builds the rotated token-major q|k|v rows
(rope.rope_pack_tokens) and runs the attention over each sequence's own tokens -- sequence b is
tokens cu_seqlens[b] .. cu_seqlens[b+1] of the sorted padded positions, query i of it sees its
keys j <= i -- so nothing is computed for, or written to, padding; its backward writes the
gradient of the q|k|v GEMM output directly, RoPE's transposed rotation applied inside the
attention backward (no separate RoPE-pack backward pass).  Padded (the drop-in for the padded
layout of solution/rope.py's RopePack):

Inputs are RopePack's outputs, q [B, NH, T, D] and k, v [B, NKV, T, D] fp16 (D = 128); query i of
row b sees key j iff j <= i and attention_mask[b, j] == 1 (the causal + key-padding mask of
transformers' create_causal_mask).  The output is token-major, [B*T, NH*D] fp16: the rows the
o-projection reads, with no transpose copy.  Other head dims, or CPU tensors, are not handled
here (the caller keeps torch's SDPA for them, as the reference does for every shape)."""

import math

import torch

from . import _ext

HEAD_DIM = 128


_CU_ATTR = "_soupk_cu_seqlens"


def cu_seqlens_of(pos_idx, batch, seq):
    """int32 [batch + 1]: where each batch row's tokens start in the sorted padded positions
    pos_idx (attention_mask.nonzero() order), and the token count at the end.  Every layer of
    a step uses one pos_idx, so the result is cached on it (rebuilt when the tensor changes)."""
    key = (int(batch), int(seq), pos_idx._version, pos_idx.data_ptr(), pos_idx.numel())
    cached = getattr(pos_idx, _CU_ATTR, None)
    if cached is not None and cached[0] == key:
        return cached[1]
    bounds = torch.arange(batch + 1, device=pos_idx.device, dtype=torch.int64) * seq
    cu = torch.searchsorted(pos_idx.to(torch.int64), bounds).to(torch.int32)
    try:
        setattr(pos_idx, _CU_ATTR, (key, cu))
    except AttributeError:
        pass
    return cu


def varlen_supported(qkv, head_dim, n_heads, n_kv):
    return (qkv.is_cuda and qkv.dtype == torch.float16 and qkv.dim() == 2
            and head_dim == HEAD_DIM and n_kv > 0 and n_heads % n_kv == 0)


def attention_varlen_fwd(qkv_r, cu_seqlens, n_heads, n_kv, scale):
    """(out [M, NH*D] fp16, lse [NH, M] fp32) of the token-major rotated rows qkv_r [M, W]."""
    _ext.require(qkv_r, "qkv_r", dtype=torch.float16, ndim=2)
    M = qkv_r.shape[0]
    dev = qkv_r.device
    if qkv_r.shape[1] != (n_heads + 2 * n_kv) * HEAD_DIM:
        raise ValueError(f"qkv_r width {qkv_r.shape[1]} != {(n_heads + 2 * n_kv) * HEAD_DIM}")
    _ext.require(cu_seqlens, "cu_seqlens", dtype=torch.int32, ndim=1, device=dev)
    B = cu_seqlens.numel() - 1
    out = torch.empty((M, n_heads * HEAD_DIM), dtype=torch.float16, device=dev)
    lse = torch.empty((n_heads, M), dtype=torch.float32, device=dev)
    _ext.call("soupk_attention_varlen_fwd", _ext.ptr(qkv_r), _ext.ptr(cu_seqlens), B,
              _ext.ptr(out), _ext.ptr(lse), M, n_heads, n_kv, HEAD_DIM, float(scale),
              _ext.stream_of(qkv_r))
    return out, lse


def attention_varlen_bwd(qkv_r, cu_seqlens, out, lse, dout, scale, n_heads, n_kv, rope=None):
    """dqkv [M, W] fp16: the gradient of qkv_r's rows, or -- with rope = (cos, sin, pos, batch,
    seq) (fp32 tables [>= seq, 128], int64 padded positions b*seq + t) -- of the q|k|v rows
    before the rotation, RoPE's backward applied inside the kernels."""
    _ext.require(qkv_r, "qkv_r", dtype=torch.float16, ndim=2)
    M = qkv_r.shape[0]
    dev = qkv_r.device
    if qkv_r.shape[1] != (n_heads + 2 * n_kv) * HEAD_DIM:
        raise ValueError(f"qkv_r width {qkv_r.shape[1]} != {(n_heads + 2 * n_kv) * HEAD_DIM}")
    _ext.require(cu_seqlens, "cu_seqlens", dtype=torch.int32, ndim=1, device=dev)
    _ext.require(out, "out", dtype=torch.float16, ndim=2, device=dev)
    if tuple(out.shape) != (M, n_heads * HEAD_DIM):
        raise ValueError(f"out has shape {tuple(out.shape)}, expected {(M, n_heads * HEAD_DIM)}")
    _ext.require(lse, "lse", dtype=torch.float32, ndim=2, device=dev)
    if tuple(lse.shape) != (n_heads, M):
        raise ValueError(f"lse has shape {tuple(lse.shape)}, expected {(n_heads, M)}")
    dout = dout.to(torch.float16).contiguous()
    _ext.require(dout, "dout", dtype=torch.float16, ndim=2, device=dev)
    if tuple(dout.shape) != tuple(out.shape):
        raise ValueError(f"dout has shape {tuple(dout.shape)}, expected {tuple(out.shape)}")
    B = cu_seqlens.numel() - 1
    dqkv = torch.empty_like(qkv_r)
    n_delta = (M * n_heads + 3) // 4 * 4
    workspace = torch.empty(n_delta + 2 * M * n_heads * HEAD_DIM, dtype=torch.float32,
                            device=dev)
    cos = sin = pos = None
    slots, t_rope = 0, 0
    if rope is not None:
        cos, sin, pos, batch, seq = rope
        for name, t in (("cos", cos), ("sin", sin)):
            _ext.require(t, name, dtype=torch.float32, ndim=2, device=dev)
            if t.shape[0] < seq or t.shape[1] != HEAD_DIM:
                raise ValueError(f"{name} must be [>= {seq}, {HEAD_DIM}], got {tuple(t.shape)}")
        _ext.require(pos, "pos", dtype=torch.int64, ndim=1, device=dev)
        if pos.numel() != M:
            raise ValueError(f"pos has {pos.numel()} entries for {M} rows")
        slots, t_rope = batch * seq, seq
    _ext.call("soupk_attention_varlen_bwd", _ext.ptr(qkv_r), _ext.ptr(cu_seqlens), B,
              _ext.ptr(out), _ext.ptr(dout), _ext.ptr(lse), _ext.ptr(cos),
              _ext.ptr(sin), _ext.ptr(pos), int(slots), int(t_rope), _ext.ptr(workspace),
              _ext.ptr(dqkv), M, n_heads, n_kv, HEAD_DIM, float(scale), _ext.stream_of(dqkv))
    return dqkv


class RopeAttention(torch.autograd.Function):
    """out [M, NH*D] = causal GQA attention of the rotated q|k|v of the real tokens (rope +
    attention in one autograd node; the backward returns the gradients of qkv and of the two
    LoRA deltas, the latter as views of the first, as RopePack does)."""

    @staticmethod
    def forward(ctx, qkv, lora_q, lora_v, cos, sin, pos_idx, cu_seqlens, batch, seq, n_heads,
                n_kv, scale):
        from .rope import rope_pack_tokens

        qkv_r, cos32, sin32, pos = rope_pack_tokens(qkv, lora_q, lora_v, cos, sin, pos_idx,
                                                    batch, seq, n_heads, n_kv, HEAD_DIM)
        out, lse = attention_varlen_fwd(qkv_r, cu_seqlens, n_heads, n_kv, scale)
        ctx.save_for_backward(qkv_r, out, lse, cos32, sin32, pos, cu_seqlens)
        ctx.dims = (batch, seq, n_heads, n_kv, scale)
        return out

    @staticmethod
    def backward(ctx, dout):
        need_qkv, need_lq, need_lv = ctx.needs_input_grad[:3]
        none = (None,) * 9
        if not (need_qkv or need_lq or need_lv):
            return (None, None, None) + none
        qkv_r, out, lse, cos, sin, pos, cu = ctx.saved_tensors
        batch, seq, n_heads, n_kv, scale = ctx.dims
        dqkv = attention_varlen_bwd(qkv_r, cu, out, lse, dout, scale, n_heads, n_kv,
                                    rope=(cos, sin, pos, batch, seq))
        q_cols = n_heads * HEAD_DIM
        v_start = (n_heads + n_kv) * HEAD_DIM
        return ((dqkv if need_qkv else None), (dqkv[:, :q_cols] if need_lq else None),
                (dqkv[:, v_start:] if need_lv else None)) + none


def rope_attention(qkv, lora_q, lora_v, cos, sin, pos_idx, cu_seqlens, batch, seq, n_heads,
                   n_kv, scale=None):
    """Differentiable RoPE + causal GQA attention over the real tokens: out [M, NH*D] fp16,
    token-major in pos_idx order (the rows the o-projection reads)."""
    scale = 1.0 / math.sqrt(HEAD_DIM) if scale is None else float(scale)
    return RopeAttention.apply(qkv.contiguous(),
                               lora_q.contiguous() if lora_q is not None else None,
                               lora_v.contiguous() if lora_v is not None else None,
                               cos, sin, pos_idx, cu_seqlens, batch, seq, n_heads, n_kv, scale)


def supported(q, k, v):
    return (q.is_cuda and q.dtype == torch.float16 and q.dim() == 4 and q.shape[-1] == HEAD_DIM
            and k.shape[1] > 0 and q.shape[1] % k.shape[1] == 0)


def attention_fwd(q, k, v, key_valid=None, scale=None):
    """(out [B*T, NH*D] fp16, lse [B, NH, T] fp32)."""
    B, NH, T, D = q.shape
    NKV = k.shape[1]
    dev = q.device
    for t, name, heads in ((q, "q", NH), (k, "k", NKV), (v, "v", NKV)):
        _ext.require(t, name, dtype=torch.float16, ndim=4, device=dev)
        if tuple(t.shape) != (B, heads, T, D):
            raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {(B, heads, T, D)}")
    if key_valid is not None:
        _ext.require(key_valid, "key_valid", dtype=torch.uint8, ndim=2, device=dev)
        if tuple(key_valid.shape) != (B, T):
            raise ValueError(f"key_valid has shape {tuple(key_valid.shape)}, expected {(B, T)}")
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    out = torch.empty((B * T, NH * D), dtype=torch.float16, device=dev)
    lse = torch.empty((B, NH, T), dtype=torch.float32, device=dev)
    _ext.call("soupk_attention_fwd", _ext.ptr(q), _ext.ptr(k), _ext.ptr(v), _ext.ptr(key_valid),
              _ext.ptr(out), _ext.ptr(lse), B, T, NH, NKV, D, scale, _ext.stream_of(q))
    return out, lse


def attention_bwd(q, k, v, key_valid, out, lse, dout, scale):
    """(dq [B, NH, T, D], dk, dv [B, NKV, T, D]) fp16, from the forward's out and lse."""
    B, NH, T, D = q.shape
    NKV = k.shape[1]
    dev = q.device
    dout = dout.to(torch.float16).contiguous()
    _ext.require(dout, "dout", dtype=torch.float16, ndim=2, device=dev)
    if tuple(dout.shape) != (B * T, NH * D):
        raise ValueError(f"dout has shape {tuple(dout.shape)}, expected {(B * T, NH * D)}")
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    n_delta = (B * NH * T + 3) // 4 * 4
    workspace = torch.empty(n_delta + 2 * B * NH * T * D, dtype=torch.float32, device=dev)
    _ext.call("soupk_attention_bwd", _ext.ptr(q), _ext.ptr(k), _ext.ptr(v), _ext.ptr(key_valid),
              _ext.ptr(out), _ext.ptr(dout), _ext.ptr(lse), _ext.ptr(workspace), _ext.ptr(dq),
              _ext.ptr(dk), _ext.ptr(dv), B, T, NH, NKV, D, float(scale), _ext.stream_of(q))
    return dq, dk, dv


class CausalAttention(torch.autograd.Function):
    """out = causal GQA attention of q, k, v (token-major [B*T, NH*D]); gradients for q, k, v."""

    @staticmethod
    def forward(ctx, q, k, v, key_valid, scale):
        out, lse = attention_fwd(q, k, v, key_valid, scale)
        ctx.save_for_backward(q, k, v, key_valid, out, lse)
        ctx.scale = scale
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, key_valid, out, lse = ctx.saved_tensors
        dq, dk, dv = attention_bwd(q, k, v, key_valid, out, lse, dout, ctx.scale)
        return dq, dk, dv, None, None


def causal_attention(q, k, v, key_valid=None, scale=None):
    """Differentiable causal GQA attention: out [B*T, NH*D] fp16 (token-major)."""
    scale = 1.0 / math.sqrt(q.shape[-1]) if scale is None else float(scale)
    return CausalAttention.apply(q, k, v, key_valid, scale)
