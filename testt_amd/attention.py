"""Causal grouped-query attention on gfx950 (testt_amd/csrc/attention.hip), forward and
backward, in place of torch's scaled_dot_product_attention in the decoder layer
(solution/model.py:246-247 runs transformers' sdpa_attention_forward there).

Inputs are RopePack's outputs, q [B, NH, T, D] and k, v [B, NKV, T, D] fp16 (D = 128); query i of
row b sees key j iff j <= i and attention_mask[b, j] == 1 (the causal + key-padding mask of
transformers' create_causal_mask).  The output is token-major, [B*T, NH*D] fp16: the rows the
o-projection reads, with no transpose copy.  Other head dims, or CPU tensors, are not handled
here (the caller keeps torch's SDPA for them, as the reference does for every shape)."""

import math

import torch

from . import _ext

HEAD_DIM = 128


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
