"""Writes the small golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

Each fixture holds seeded inputs and expected outputs produced by a route independent of the
oracle's own code: hand-derived known answers and float64 arithmetic for NF4, transformers'
Qwen2RMSNorm and apply_rotary_pos_emb (the third-party eager path the reference replaces,
installed here as transformers 5.15.0), float64 closed forms for SwiGLU, and float64
torch.nn.functional.cross_entropy / log_softmax for the head.  The reference itself is not run.
"""

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from testt_amd import workloads  # noqa: E402


def f64_dequant(packed, absmax_u8, code2, absmax2, offset, nf4, qblock, qblock2):
    """NF4 dequant by the float64 route: exact products in float64, rounded to fp32 once."""
    packed = packed.reshape(-1).astype(np.int64)
    n = packed.size
    blk = np.arange(n) // (qblock // 2)
    prod = (code2.astype(np.float64)[absmax_u8[blk]] *
            absmax2.astype(np.float64)[blk // qblock2]).astype(np.float32)
    scale = (prod.astype(np.float64) + np.float64(np.float32(offset))).astype(np.float32)
    hi = (nf4.astype(np.float64)[packed >> 4] * scale.astype(np.float64)).astype(np.float32)
    lo = (nf4.astype(np.float64)[packed & 15] * scale.astype(np.float64)).astype(np.float32)
    out = np.empty(2 * n, np.float16)
    out[0::2], out[1::2] = hi.astype(np.float16), lo.astype(np.float16)
    return out


def nf4_fixture():
    g = np.random.default_rng(11)
    nf4 = np.asarray(workloads.NF4_LEVELS, np.float32)
    code2 = workloads.dynamic_code_signed().numpy()
    # 1) every byte value under several absmax blocks (qblock 64 -> 32 bytes per block)
    packed = np.tile(np.arange(256, dtype=np.uint8), 8)            # 2048 bytes, 64 blocks
    absmax_u8 = g.integers(0, 256, size=64).astype(np.uint8)
    absmax2 = np.array([0.0371, 0.0917], np.float32)               # qblock2 = 32 -> 2 groups
    offset = np.float32(0.0312)
    expected = f64_dequant(packed, absmax_u8, code2, absmax2, offset, nf4, 64, 32)
    return dict(packed=packed, absmax_u8=absmax_u8, code2=code2, absmax2=absmax2,
                offset=np.array([offset], np.float32), nf4=nf4, qblock=np.int64(64),
                qblock2=np.int64(32), expected=expected)


def rmsnorm_fixture():
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

    x, delta, w, pad_idx, padded = workloads.rmsnorm_inputs(rows=24, hidden=256, padded=40,
                                                            seed=12)
    norm = Qwen2RMSNorm(256, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(w)
        s = x + delta.float()
        y = norm(s)                                   # fp32 in -> fp32 out
        rstd = torch.rsqrt(s.double().pow(2).mean(-1) + 1e-6)
    return dict(x=x.numpy(), delta=delta.numpy(), w=w.numpy(), pad_idx=pad_idx.numpy(),
                padded=np.int64(padded), eps=np.float32(1e-6), y32=y.numpy(),
                y16=y.to(torch.float16).numpy(), rstd64=rstd.numpy())


def rope_fixture():
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

    batch, seq, nh, nkv, d = 2, 6, 3, 1, 16
    lengths = (6, 4)
    qkv, lq, lv, pos = workloads.rope_inputs(lengths=lengths, seq=seq, n_heads=nh, n_kv=nkv,
                                             head_dim=d, lora_dtype=torch.float32, seed=13)
    cos, sin = workloads.rope_tables(seq=seq, head_dim=d, theta=1e4)
    fq = qkv[:, :nh * d].float() + lq
    fk = qkv[:, nh * d:(nh + nkv) * d].float()
    fv = qkv[:, (nh + nkv) * d:].float() + lv

    def padded(flat, heads):
        out = torch.zeros(batch * seq, heads * d).index_copy(0, pos, flat)
        return out.view(batch, seq, heads, d).transpose(1, 2)

    rq, rk = apply_rotary_pos_emb(padded(fq, nh), padded(fk, nkv), cos[None], sin[None])
    rv = padded(fv, nkv)
    return dict(qkv=qkv.numpy(), lq=lq.numpy(), lv=lv.numpy(), pos=pos.numpy(),
                cos=cos.numpy(), sin=sin.numpy(), dims=np.array([batch, seq, nh, nkv, d]),
                q=rq.to(torch.float16).numpy(), k=rk.to(torch.float16).numpy(),
                v=rv.to(torch.float16).numpy())


def swiglu_fixture():
    gu = workloads.swiglu_inputs(rows=8, inter=64, seed=14, scale=3.0)
    dact = workloads.swiglu_grad(rows=8, inter=64, seed=15) * 100
    g = gu[:, :64].double()
    u = gu[:, 64:].double()
    sig = 1.0 / (1.0 + torch.exp(-g))
    act = g * sig * u
    d = dact.double()
    dg = d * u * sig * (1.0 + g * (1.0 - sig))
    du = d * g * sig
    return dict(gu=gu.numpy(), dact=dact.numpy(), act=act.to(torch.float16).numpy(),
                dgu=torch.cat([dg, du], 1).to(torch.float16).numpy())


def head_fixture():
    rows, vocab = 6, 1003                       # odd vocab: unaligned rows, scalar head/tail
    g = workloads.gen(16)
    z = (2.0 * torch.randn(rows, vocab, generator=g)).to(torch.float16)
    z[2, 17] = z[2, 900] = 30.0                 # tie: first index wins
    targets = torch.tensor([5, -100, 17, 1002, 0, 900], dtype=torch.int64)
    zd = z.double()
    logp = torch.log_softmax(zd, -1)
    entropy = -(logp.exp() * logp).sum(-1)
    lab = targets != -100
    ce = torch.nn.functional.cross_entropy(zd, targets, ignore_index=-100, reduction="none")
    lse = torch.logsumexp(zd, -1)
    correct = (zd.argmax(-1) == targets) & lab
    scale = 64.0 / 5.0
    onehot = torch.zeros_like(zd)
    onehot[lab, targets[lab]] = 1.0
    grad = ((logp.exp() - onehot) * scale).to(torch.float16)
    new = torch.where(lab[:, None], grad, z)
    return dict(z=z.numpy(), targets=targets.numpy(), entropy=entropy.numpy(),
                loss=ce.numpy(), lse=lse.numpy(), correct=correct.numpy(),
                grad_scale=np.float32(scale), new_logits=new.numpy())


def main():
    for name, fn in (("nf4_kat", nf4_fixture), ("rmsnorm_qwen2", rmsnorm_fixture),
                     ("rope_hf", rope_fixture), ("swiglu_f64", swiglu_fixture),
                     ("head_f64", head_fixture)):
        path = os.path.join(HERE, f"{name}.npz")
        np.savez_compressed(path, **fn())
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
