"""Residual add + RMSNorm on gfx950, forward and backward.  Drop-in for solution/rmsnorm.py.

One wavefront per token row (testt_amd/csrc/rmsnorm.hip):
  s = x + delta            (the residual stream, fp32; delta is the fp16 output of the block)
  y = w * s * rsqrt(mean(s^2) + eps)         (transformers' Qwen2RMSNorm)
written once in fp16 for the GEMMs and, when asked, once in fp32 into the padded
[batch * seq, hidden] layout that the LoRA dropout reads; rows of that layout with no token are
zeroed by the same launch.  Backward is one wavefront per row as well: it sums the fp16 gradient
of the GEMM path and the fp32 gradient of the LoRA path in fp32 and adds the residual gradient.
"""

import torch

from . import _ext
from ._index import as_index, inverse_map


def _weight32(weight, hidden, device):
    """The norm weight as a contiguous fp32 device vector (the kernels read fp32)."""
    w = weight.detach()
    if w.dtype != torch.float32:
        w = w.float()
    w = _ext.require(w.contiguous(), "weight", ndim=1, device=device)
    if w.numel() != hidden:
        raise ValueError(f"weight has {w.numel()} elements, hidden size is {hidden}")
    return w


def _launch_fwd(x, delta, weight, eps, pad_idx, padded_rows):
    """(s, y16, ypad32, rstd) of solution/rmsnorm.py:76-92."""
    _ext.require(x, "x", dtype=torch.float32, ndim=2)
    rows, hidden = x.shape
    dev = x.device
    if delta is not None:
        _ext.require(delta, "delta", dtype=torch.float16, ndim=2, device=dev)
        if tuple(delta.shape) != (rows, hidden):
            raise ValueError(f"delta shape {tuple(delta.shape)} != x shape {(rows, hidden)}")
    w = _weight32(weight, hidden, dev)
    s = torch.empty_like(x) if delta is not None else x
    y = torch.empty((rows, hidden), dtype=torch.float16, device=dev)
    rstd = torch.empty((rows,), dtype=torch.float32, device=dev)
    inv = None
    if pad_idx is not None:
        pad_idx = as_index(pad_idx)
        if pad_idx.numel() != rows:
            raise ValueError(f"pad_idx has {pad_idx.numel()} entries for {rows} rows")
        padded_rows = int(padded_rows)
        # Rows of ypad that no token lands on are zeroed in the same launch; with as many
        # (distinct) tokens as padded rows there are none.
        ypad = torch.empty((padded_rows, hidden), dtype=torch.float32, device=dev)
        if rows != padded_rows:
            inv = inverse_map(pad_idx, padded_rows)
    else:
        padded_rows = 0
        ypad = torch.empty((0, hidden), dtype=torch.float32, device=dev)
    if rows or inv is not None:
        _ext.call("soupk_rmsnorm_fwd", _ext.ptr(x), _ext.ptr(delta), _ext.ptr(w),
                  _ext.ptr(s) if delta is not None else None, _ext.ptr(y),
                  _ext.ptr(ypad) if pad_idx is not None else None, _ext.ptr(pad_idx),
                  _ext.ptr(inv), _ext.ptr(rstd), rows, padded_rows, hidden, float(eps),
                  _ext.stream_of(x))
    return s, y, ypad, rstd


def _launch_bwd(s, rstd, weight, pad_idx, grad_s, grad_y, grad_ypad, want_delta):
    """(dx, ddelta or None) of solution/rmsnorm.py:95-112."""
    _ext.require(s, "s", dtype=torch.float32, ndim=2)
    rows, hidden = s.shape
    dev = s.device
    w = _weight32(weight, hidden, dev)
    dx = torch.empty_like(s)
    ddelta = torch.empty((rows, hidden), dtype=torch.float16, device=dev) if want_delta else None
    has_pad = grad_ypad is not None and pad_idx is not None and grad_ypad.numel() > 0
    dy = grad_y.to(torch.float16).contiguous() if grad_y is not None else None
    dpad = grad_ypad.to(torch.float32).contiguous() if has_pad else None
    ds = grad_s.to(torch.float32).contiguous() if grad_s is not None else None
    idx = as_index(pad_idx) if has_pad else None
    for t, name in ((dy, "grad_y"), (ds, "grad_s")):
        if t is not None and tuple(t.shape) != (rows, hidden):
            raise ValueError(f"{name} shape {tuple(t.shape)} != {(rows, hidden)}")
    if has_pad and (dpad.dim() != 2 or dpad.shape[1] != hidden or idx.numel() != rows):
        raise ValueError("grad_ypad / pad_idx do not match the saved rows")
    if rows:
        _ext.call("soupk_rmsnorm_bwd", _ext.ptr(s), _ext.ptr(rstd), _ext.ptr(w), _ext.ptr(dy),
                  _ext.ptr(dpad), _ext.ptr(idx), _ext.ptr(ds), _ext.ptr(dx), _ext.ptr(ddelta),
                  rows, dpad.shape[0] if has_pad else 0, hidden, _ext.stream_of(s))
    return dx, ddelta


class AddRMSNorm(torch.autograd.Function):
    """(s, y16, ypad32) = (x + delta, norm(x + delta) in fp16, the same in fp32 at padded rows)."""

    @staticmethod
    def forward(ctx, x, delta, weight, eps, pad_idx, padded_rows):
        s, y, ypad, rstd = _launch_fwd(x, delta, weight, eps, pad_idx, padded_rows)
        ctx.save_for_backward(s, rstd, weight, pad_idx)
        return s, y, ypad

    @staticmethod
    def backward(ctx, grad_s, grad_y, grad_ypad):
        s, rstd, weight, pad_idx = ctx.saved_tensors
        need_x, need_delta = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if not (need_x or need_delta):
            return None, None, None, None, None, None
        dx, ddelta = _launch_bwd(s, rstd, weight, pad_idx, grad_s, grad_y, grad_ypad, need_delta)
        return (dx if need_x else None), ddelta, None, None, None, None


class RMSNormNoAdd(torch.autograd.Function):
    """(y16, ypad32) = norm(x) without a residual add (the first layer's input norm)."""

    @staticmethod
    def forward(ctx, x, weight, eps, pad_idx, padded_rows):
        _s, y, ypad, rstd = _launch_fwd(x, None, weight, eps, pad_idx, padded_rows)
        ctx.save_for_backward(x, rstd, weight, pad_idx)
        return y, ypad

    @staticmethod
    def backward(ctx, grad_y, grad_ypad):
        x, rstd, weight, pad_idx = ctx.saved_tensors
        if not ctx.needs_input_grad[0]:
            return None, None, None, None, None
        dx, _ = _launch_bwd(x, rstd, weight, pad_idx, None, grad_y, grad_ypad, False)
        return dx, None, None, None, None


def add_rmsnorm(x, delta, weight, eps, pad_idx=None, padded_rows=0):
    """Returns (s, y16, ypad32); with delta=None, s is x itself."""
    x = x.contiguous()
    if delta is None:
        y, ypad = RMSNormNoAdd.apply(x, weight, eps, pad_idx, padded_rows)
        return x, y, ypad
    return AddRMSNorm.apply(x, delta.contiguous(), weight, eps, pad_idx, padded_rows)
