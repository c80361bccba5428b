"""Q/K/V assembly for attention on gfx950: LoRA add + rotary embedding + scatter to the padded
layout.  Drop-in for solution/rope.py.

The fused q/k/v GEMM output (fp16, unpadded tokens) is read once per token by
testt_amd/csrc/rope_pack.hip, which adds the LoRA outputs in fp32, rotates q and k in fp32 and
writes fp16 q/k/v directly into [batch, heads, seq, head_dim] at the token's padded position,
the layout SDPA takes; padded positions with no token are zeroed by the same launch.  Backward
is the transposed rotation, gathering per token and writing the fp16 gradient of the q/k/v GEMM
output; the LoRA branches get views of the same buffer.
"""

import torch

from . import _ext
from ._common import next_pow2
from ._index import as_index, inverse_map


def _consts(n_heads, n_kv, head_dim):
    """The reference's compile-time constants (solution/rope.py:131-133), kept for callers."""
    return dict(NH=n_heads, NKV=n_kv, HALF=head_dim // 2, NH_P=next_pow2(n_heads),
                NKV_P=next_pow2(n_kv))


def _table(t, seq, head_dim, name, device):
    t = t.detach()
    if t.dtype != torch.float32:
        t = t.float()
    t = _ext.require(t.contiguous(), name, ndim=2, device=device)
    if t.shape[0] < seq or t.shape[1] != head_dim:
        raise ValueError(f"{name} must be [>= {seq}, {head_dim}], got {tuple(t.shape)}")
    return t


def _lora_pair(lora_q, lora_v):
    """Both LoRA deltas in one element type (fp16 or fp32) and its ABI code."""
    ts = [t for t in (lora_q, lora_v) if t is not None]
    if not ts:
        return lora_q, lora_v, _ext.DTYPE_F16
    if all(t.dtype == torch.float16 for t in ts):
        dtype, code = torch.float16, _ext.DTYPE_F16
    else:
        dtype, code = torch.float32, _ext.DTYPE_F32
    conv = [None if t is None else t.detach().to(dtype).contiguous() for t in (lora_q, lora_v)]
    return conv[0], conv[1], code


class RopePack(torch.autograd.Function):
    @staticmethod
    def forward(ctx, qkv, lora_q, lora_v, cos, sin, pos_idx, batch, seq, n_heads, n_kv, head_dim):
        _ext.require(qkv, "qkv", dtype=torch.float16, ndim=2)
        rows = qkv.shape[0]
        dev = qkv.device
        width = (n_heads + 2 * n_kv) * head_dim
        if qkv.shape[1] != width:
            raise ValueError(f"qkv width {qkv.shape[1]} != (n_heads + 2*n_kv) * head_dim = {width}")
        if head_dim % 2:
            raise ValueError("head_dim must be even")
        pos = as_index(pos_idx)
        if pos.numel() != rows:
            raise ValueError(f"pos_idx has {pos.numel()} entries for {rows} rows")
        lq, lv, code = _lora_pair(lora_q, lora_v)
        if lq is not None and tuple(lq.shape) != (rows, n_heads * head_dim):
            raise ValueError(f"lora_q shape {tuple(lq.shape)} != {(rows, n_heads * head_dim)}")
        if lv is not None and tuple(lv.shape) != (rows, n_kv * head_dim):
            raise ValueError(f"lora_v shape {tuple(lv.shape)} != {(rows, n_kv * head_dim)}")
        cos32 = _table(cos, seq, head_dim, "cos", dev)
        sin32 = _table(sin, seq, head_dim, "sin", dev)
        q = torch.empty((batch, n_heads, seq, head_dim), dtype=torch.float16, device=dev)
        k = torch.empty((batch, n_kv, seq, head_dim), dtype=torch.float16, device=dev)
        v = torch.empty((batch, n_kv, seq, head_dim), dtype=torch.float16, device=dev)
        slots = batch * seq
        # Positions without a token are zeroed by the kernel; with as many (distinct) tokens as
        # positions there are none.
        inv = inverse_map(pos, slots) if rows != slots else None
        if rows or inv is not None:
            _ext.call("soupk_rope_pack_fwd", _ext.ptr(qkv), _ext.ptr(lq), _ext.ptr(lv), code,
                      _ext.ptr(cos32), _ext.ptr(sin32), _ext.ptr(pos), _ext.ptr(inv), _ext.ptr(q),
                      _ext.ptr(k), _ext.ptr(v), rows, batch, seq, n_heads, n_kv, head_dim,
                      _ext.stream_of(qkv))
        ctx.save_for_backward(cos32, sin32, pos)
        ctx.dims = (rows, batch, seq, n_heads, n_kv, head_dim)
        return q, k, v

    @staticmethod
    def backward(ctx, grad_q, grad_k, grad_v):
        cos, sin, pos_idx = ctx.saved_tensors
        rows, batch, seq, n_heads, n_kv, head_dim = ctx.dims
        need_qkv, need_lq, need_lv = ctx.needs_input_grad[:3]
        if not (need_qkv or need_lq or need_lv):
            return (None,) * 11
        width = (n_heads + 2 * n_kv) * head_dim
        dqkv = torch.empty((rows, width), dtype=torch.float16, device=pos_idx.device)
        grads = [g.to(torch.float16).contiguous() if g is not None else None
                 for g in (grad_q, grad_k, grad_v)]
        if rows:
            _ext.call("soupk_rope_pack_bwd", _ext.ptr(grads[0]), _ext.ptr(grads[1]),
                      _ext.ptr(grads[2]), _ext.ptr(cos), _ext.ptr(sin), _ext.ptr(pos_idx),
                      _ext.ptr(dqkv), rows, batch, seq, n_heads, n_kv, head_dim,
                      _ext.stream_of(dqkv))
        q_cols = n_heads * head_dim
        v_start = (n_heads + n_kv) * head_dim
        return ((dqkv if need_qkv else None),
                (dqkv[:, :q_cols] if need_lq else None),
                (dqkv[:, v_start:] if need_lv else None),
                None, None, None, None, None, None, None, None)


def rope_pack(qkv, lora_q, lora_v, cos, sin, pos_idx, batch, seq, n_heads, n_kv, head_dim):
    return RopePack.apply(qkv.contiguous(),
                          lora_q.contiguous() if lora_q is not None else None,
                          lora_v.contiguous() if lora_v is not None else None,
                          cos.contiguous(), sin.contiguous(), pos_idx, batch, seq,
                          n_heads, n_kv, head_dim)


def rope_pack_tokens(qkv, lora_q, lora_v, cos, sin, pos_idx, batch, seq, n_heads, n_kv,
                     head_dim):
    """The RoPE pack forward without the scatter: fp16 [rows, (n_heads + 2*n_kv) * head_dim] in
    qkv's own token-major layout -- q + lora_q rotated, k rotated, v + lora_v -- with the same
    arithmetic as RopePack (bit-identical values), for the varlen attention, which reads the
    real tokens where they are (no padded layout, no zero rows).  head_dim 128.  A token whose
    position lies outside [0, batch*seq) gets a row of zeros.  Not differentiable by itself:
    attention.RopeAttention carries its backward (fused into the attention backward)."""
    _ext.require(qkv, "qkv", dtype=torch.float16, ndim=2)
    rows = qkv.shape[0]
    dev = qkv.device
    width = (n_heads + 2 * n_kv) * head_dim
    if qkv.shape[1] != width:
        raise ValueError(f"qkv width {qkv.shape[1]} != (n_heads + 2*n_kv) * head_dim = {width}")
    if head_dim != 128:
        raise ValueError("rope_pack_tokens handles head_dim 128 (use RopePack otherwise)")
    pos = as_index(pos_idx)
    if pos.numel() != rows:
        raise ValueError(f"pos_idx has {pos.numel()} entries for {rows} rows")
    lq, lv, code = _lora_pair(lora_q, lora_v)
    if lq is not None and tuple(lq.shape) != (rows, n_heads * head_dim):
        raise ValueError(f"lora_q shape {tuple(lq.shape)} != {(rows, n_heads * head_dim)}")
    if lv is not None and tuple(lv.shape) != (rows, n_kv * head_dim):
        raise ValueError(f"lora_v shape {tuple(lv.shape)} != {(rows, n_kv * head_dim)}")
    cos32 = _table(cos, seq, head_dim, "cos", dev)
    sin32 = _table(sin, seq, head_dim, "sin", dev)
    out = torch.empty((rows, width), dtype=torch.float16, device=dev)
    if rows:
        _ext.call("soupk_rope_pack_tokens", _ext.ptr(qkv), _ext.ptr(lq),
                  _ext.ptr(lv), code, _ext.ptr(cos32), _ext.ptr(sin32), _ext.ptr(pos),
                  _ext.ptr(out), rows, batch, seq, n_heads, n_kv, head_dim, _ext.stream_of(out))
    return out, cos32, sin32, pos
