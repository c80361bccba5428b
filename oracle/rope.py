"""LoRA add + RoPE + pack into the padded [B, heads, T, D] layout, eager PyTorch on the CPU.
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Forward follows solution/rope.py:24-75 as its own test builds the reference
(solution/test_kernels.py:145-158): q = qkv_q + lora_q, k = qkv_k, v = qkv_v + lora_v in fp32,
index_copy of each into zeros [B*T, heads*D] at pos_idx, view/transpose to [B, heads, T, D],
then transformers' apply_rotary_pos_emb (modeling_qwen2.py:105-135): q*cos + rotate_half(q)*sin
with rotate_half(x) = cat(-x2, x1); fp16 at the end.  Backward is torch autograd through the
same graph (solution/test_kernels.py:159-163); the fp32 gradient of the fused qkv row is then
cast to fp16 as the kernel stores it (solution/rope.py:78-128).

Pinned by: transformers' own apply_rotary_pos_emb on the same padded tensors, and the
invariants of tests/test_oracle_rope.py (t = 0 is the identity, pair norms are preserved, the
backward of the rotation is its transpose, pad positions are exactly zero).
"""

import torch


def rotate_half(x):
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rotary(q, k, cos, sin):
    """q*cos + rotate_half(q)*sin for q, k [B, heads, T, D] and cos, sin [T, D]."""
    c, s = cos[None, None], sin[None, None]
    return q * c + rotate_half(q) * s, k * c + rotate_half(k) * s


def _padded(flat, pos_idx, batch, seq, heads, head_dim):
    out = torch.zeros(batch * seq, heads * head_dim, dtype=flat.dtype)
    out = out.index_copy(0, pos_idx.long(), flat)
    return out.view(batch, seq, heads, head_dim).transpose(1, 2)


def _leaves(qkv, lora_q, lora_v):
    leaves = [None if t is None else t.detach().float().clone().requires_grad_(True)
              for t in (qkv, lora_q, lora_v)]
    return leaves


def _graph(leaves, cos, sin, pos_idx, batch, seq, nh, nkv, d):
    fqkv, flq, flv = leaves
    fq = fqkv[:, :nh * d] + flq if flq is not None else fqkv[:, :nh * d]
    fk = fqkv[:, nh * d:(nh + nkv) * d]
    fv = fqkv[:, (nh + nkv) * d:] + flv if flv is not None else fqkv[:, (nh + nkv) * d:]
    cos, sin = cos[:seq].float(), sin[:seq].float()
    rq, rk = apply_rotary(_padded(fq, pos_idx, batch, seq, nh, d),
                          _padded(fk, pos_idx, batch, seq, nkv, d), cos, sin)
    rv = _padded(fv, pos_idx, batch, seq, nkv, d)
    return rq, rk, rv


def rope_pack_fwd(qkv, lora_q, lora_v, cos, sin, pos_idx, batch, seq, nh, nkv, d):
    """(q, k, v) fp16 in the padded layout."""
    with torch.no_grad():
        rq, rk, rv = _graph(_leaves(qkv, lora_q, lora_v), cos, sin, pos_idx, batch, seq, nh,
                            nkv, d)
    return rq.to(torch.float16), rk.to(torch.float16), rv.to(torch.float16)


def rope_pack_bwd(qkv, lora_q, lora_v, cos, sin, pos_idx, batch, seq, nh, nkv, d, dq, dk, dv):
    """fp16 dqkv [M, (nh+2nkv)*d]: the gradient of the fused qkv row for incoming dq/dk/dv
    (each may be None = zero), by autograd.  The LoRA gradients are its q and v column blocks."""
    leaves = _leaves(qkv, None, None)
    rq, rk, rv = _graph(leaves, cos, sin, pos_idx, batch, seq, nh, nkv, d)
    outs, grads = [], []
    for out, g in ((rq, dq), (rk, dk), (rv, dv)):
        if g is not None:
            outs.append(out)
            grads.append(g.float())
    if outs:
        torch.autograd.backward(outs, grads)
    grad = leaves[0].grad
    if grad is None:
        grad = torch.zeros_like(leaves[0])
    return grad.detach().to(torch.float16)
