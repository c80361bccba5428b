"""Residual add + Qwen2RMSNorm, forward and backward, eager PyTorch on the CPU.
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Forward follows solution/rmsnorm.py:24-43 and transformers' Qwen2RMSNorm
(transformers/models/qwen2/modeling_qwen2.py:247-252): s = x + fp32(delta),
y = w * (s * rsqrt(mean(s^2) + eps)); y in fp16 for the GEMMs, y in fp32 scattered to
ypad[pad_idx] (the rest zero).  Backward is torch autograd through that eager graph with the
three incoming gradients of solution/rmsnorm.py:46-69 (fp16 dy, fp32 dypad gathered at pad_idx,
fp32 ds), exactly as solution/test_kernels.py:67-86 builds its reference.

Pinned by: transformers' own Qwen2RMSNorm module (installed third-party code, the reference's
eager path) on the same inputs, a float64 recomputation of rstd and of the closed-form gradient
dx = (g - n * mean(g * n)) * rstd + ds, and the invariants of tests/test_oracle_rmsnorm.py.
"""

import torch


def rmsnorm_fwd(x, delta, weight, eps, pad_idx=None, padded_rows=0):
    """(s fp32, y fp16, ypad fp32 [padded_rows, H], rstd fp32 [rows])."""
    x = x.detach().float()
    s = x + delta.detach().float() if delta is not None else x
    variance = s.pow(2).mean(-1, keepdim=True)
    rstd = torch.rsqrt(variance + eps)
    y = weight.detach().float() * (s * rstd)
    ypad = torch.zeros((padded_rows, x.shape[1]), dtype=torch.float32)
    if pad_idx is not None:
        ypad[pad_idx.long()] = y
    return s, y.to(torch.float16), ypad, rstd.squeeze(-1)


def rmsnorm_fwd_bwd(x, delta, weight, eps, pad_idx, padded_rows, dy, dypad, ds):
    """Forward outputs and (dx fp32, ddelta fp16 or None) by autograd.

    dy (fp16, grad of y16), dypad (fp32, grad of ypad; needs pad_idx) and ds (fp32, grad of s;
    needs delta) may each be None."""
    xr = x.detach().float().clone().requires_grad_(True)
    dr = delta.detach().clone().requires_grad_(True) if delta is not None else None
    s = xr + dr.float() if dr is not None else xr
    variance = s.pow(2).mean(-1, keepdim=True)
    rstd = torch.rsqrt(variance + eps)
    y = weight.detach().float() * (s * rstd)
    total = torch.zeros_like(y)
    if dy is not None:
        total = total + dy.float()
    if dypad is not None and pad_idx is not None:
        total = total + dypad.float()[pad_idx.long()]
    outs, grads = [y], [total]
    if ds is not None and dr is not None:
        outs.append(s)
        grads.append(ds.float())
    torch.autograd.backward(outs, grads)
    ddelta = dr.grad if dr is not None else None
    return xr.grad.detach(), ddelta
