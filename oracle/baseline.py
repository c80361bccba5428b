"""The reference's eager PyTorch path for each kernel, run on the CPU, for bench.py's CPU
baseline.  TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): timed beside the GPU kernels,
never shipped.

Each function computes what the corresponding kernel produces, the way base Soup's eager path
does: bitsandbytes-style dequant (numpy fp32, oracle.nf4), Qwen2RMSNorm + autograd,
index_copy + apply_rotary_pos_emb + autograd, silu * up + autograd, and log_softmax / argmax /
softmax - onehot over fp32-cast logits.
"""

import torch

from . import nf4 as onf4
from . import rope as orope


def nf4_unpack(w):
    return onf4.dequant_state(w)


def rmsnorm_fwd(x, delta, w, eps, pad_idx, padded):
    s = x + delta.float()
    y = w * (s * torch.rsqrt(s.pow(2).mean(-1, keepdim=True) + eps))
    ypad = torch.zeros(padded, x.shape[1])
    ypad[pad_idx] = y
    return s, y.to(torch.float16), ypad


def rmsnorm_bwd(x, delta, w, eps, pad_idx, dy, dypad, ds):
    xr = x.clone().requires_grad_(True)
    dr = delta.clone().requires_grad_(True)
    s = xr + dr.float()
    y = w * (s * torch.rsqrt(s.pow(2).mean(-1, keepdim=True) + eps))
    torch.autograd.backward([y, s], [dy.float() + dypad[pad_idx], ds])
    return xr.grad, dr.grad


def rope_fwd(qkv, lq, lv, cos, sin, pos, batch, seq, nh, nkv, d):
    return orope.rope_pack_fwd(qkv, lq, lv, cos, sin, pos, batch, seq, nh, nkv, d)


def rope_bwd(qkv, cos, sin, pos, batch, seq, nh, nkv, d, dq, dk, dv):
    return orope.rope_pack_bwd(qkv, None, None, cos, sin, pos, batch, seq, nh, nkv, d, dq, dk, dv)


def swiglu_fwd(gu):
    inter = gu.shape[1] // 2
    return (torch.nn.functional.silu(gu[:, :inter].float()) * gu[:, inter:].float()).half()


def swiglu_bwd(dact, gu):
    inter = gu.shape[1] // 2
    g = gu[:, :inter].float().requires_grad_(True)
    u = gu[:, inter:].float().requires_grad_(True)
    (torch.nn.functional.silu(g) * u).backward(dact.float())
    return torch.cat([g.grad, u.grad], 1).half()


def head_stats_grad(logits, targets, grad_scale):
    z = logits.float()
    logp = torch.log_softmax(z, -1)
    p = logp.exp()
    entropy = -(p * logp).sum(-1)
    lab = targets != -100
    safe = targets.clamp(min=0)
    loss = torch.where(lab, -logp.gather(1, safe[:, None]).squeeze(1), torch.zeros(()))
    correct = (z.argmax(-1) == targets) & lab
    p[lab, safe[lab]] -= 1.0
    grad = (p * grad_scale).half()
    return entropy, loss, correct, grad
