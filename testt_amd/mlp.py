"""The Qwen2 MLP, down(silu(gate(x)) * up(x)), with frozen NF4 weights, as one autograd node.
Drop-in for solution/mlp.py.

- gate and up are one hipBLASLt GEMM against both weights unpacked into one [2I, H] buffer
  (with few rows, where the fused NF4-dequant GEMM of testt_amd/nf4_gemm.py is the faster
  path, each product runs on the NF4 weights instead: nf4.fused_linear / fused_grad_input);
- testt_amd/csrc/swiglu.hip reads the fp16 [tokens, 2I] result and writes silu(g) * u in fp16
  (computed in fp32, rounded once to fp16 where the down projection reads it);
- backward turns the incoming gradient into the gate/up gradients in place, in the [tokens, 2I]
  gate/up buffer, so the input gradient is again a single product (split along K over
  batched GEMMs with fp32 partials, summed by a HIP kernel; split_parts, as the down
  projection's forward).

RECOMPUTE_GATE_UP (solution/mlp.py:27) chooses where that buffer comes from.  The reference
recomputes it in backward (one more [tokens, H] x [H, 2I] GEMM) to keep nothing of size
[tokens, I] alive between the passes.  On MI355X the buffer of the 2048-token step is 73 MB per
layer (2 GB for 28 layers, under 1% of 288 GB of HBM) while the recompute GEMM is 113 GFLOP
per layer, so the default here keeps the forward's buffer; True restores the reference's
memory profile.  Both give identical results (the same GEMM on the same inputs).  The kept
buffer is consumed by the in-place backward, so a second backward through the same graph
raises instead of reading gradients as activations.
"""

import torch

from . import _ext
from . import blas as _blas
from ._common import kernels_ok
from .nf4 import fused_grad_input, fused_linear, keep_for_backward, unpack_concat

RECOMPUTE_GATE_UP = False  # True: keep only the [tokens, H] input, recompute gate/up

# Split of the gate|up input-gradient GEMM (d(gate|up) [tokens, 2I] @ [W_gate; W_up] [2I, H])
# along K into batched hipBLASLt GEMMs with fp32 outputs, summed in order and rounded once to
# fp16 by soupk_sum_partials, and of the down projection's forward (act [tokens, I] @ W_down^T)
# the same way: both contract deep (17,920 / 8,960) into a [tokens, H] output of few tiles.
# None: split_parts() picks the count by rows; an int forces it (1 = one fp16 GEMM, the
# reference's).
SPLIT_K_GATE_UP = None
SPLIT_K_DOWN = None


def split_parts(rows, out_cols, depth, kind):
    """Slices of K for the split products, measured on MI355X (hipBLASLt's tuned or heuristic
    solutions, 256 to 4096 rows at Qwen2.5-1.5B's shapes):
    - the gate|up input gradient: the largest of 1, 2, 4, 8 that keeps the output's
      256 x 256 tiles times the slices within 256 (8 up to 1024 rows: 888 rows 67.8 us against
      88.3 with 4 and 202.3 unsplit; 4 at 2048 rows: 130.7 against 161.1 / 146.8 with 2 / 8);
    - the down projection's forward: 2 up to 2048 rows (2048 rows 63.4 against 69.7 us
      unsplit, 888 rows 38.7 against 43.7), one GEMM above (3072 rows 92.5 against 97.3)."""
    if rows <= 0:
        return 1
    if kind == "gate_up":
        tiles = -(-rows // 256) * -(-out_cols // 256)
        parts = 1
        while parts < 8 and tiles * parts * 2 <= 256 and depth % (parts * 2) == 0:
            parts *= 2
        return parts
    return 2 if rows <= 2048 and depth % 2 == 0 else 1
# Columns one workgroup step covers per row in the reference's tiling (solution/mlp.py:28);
# the HIP kernels stream the flat [rows, I] space in 16-byte chunks instead.
COLS_PER_PROGRAM = 1024


def gated_silu(gu):
    """act[r, c] = fp16(silu(gu[r, c]) * gu[r, I + c]) for gu = [gate | up] fp16 [rows, 2I]."""
    _ext.require(gu, "gu", dtype=torch.float16, ndim=2)
    rows, two_i = gu.shape
    if two_i % 2:
        raise ValueError(f"gu width {two_i} is odd; expected [gate | up]")
    inter = two_i // 2
    act = torch.empty((rows, inter), dtype=torch.float16, device=gu.device)
    if rows and inter:
        _ext.call("soupk_swiglu_fwd", _ext.ptr(gu), _ext.ptr(act), rows, inter,
                  _ext.stream_of(gu))
    return act


def gated_silu_backward_(dact, gu):
    """Overwrites gu = [gate | up] with [d gate | d up] for the incoming gradient dact."""
    _ext.require(gu, "gu", dtype=torch.float16, ndim=2)
    rows, two_i = gu.shape
    inter = two_i // 2
    dact = dact.to(torch.float16).contiguous()
    _ext.require(dact, "dact", dtype=torch.float16, ndim=2, device=gu.device)
    if tuple(dact.shape) != (rows, inter):
        raise ValueError(f"dact shape {tuple(dact.shape)} != {(rows, inter)}")
    if rows and inter:
        _ext.call("soupk_swiglu_bwd_inplace", _ext.ptr(dact), _ext.ptr(gu), rows, inter,
                  _ext.stream_of(gu))
    return gu


def _mm(a, b):
    """a @ b: the direct hipBLASLt GEMM (testt_amd/blas.py: torch.matmul's solution without
    its per-call setup) for the 2-d operands of the layer, torch.matmul otherwise."""
    return _blas.matmul(a, b) if a.dim() == 2 and b.dim() == 2 else torch.matmul(a, b)


def matmul_split_k(a, b, parts):
    """fp16 a [M, K] @ b [K, N] as `parts` GEMMs over equal slices of K (batched, fp32
    outputs), summed in slice order and rounded once to fp16.  K % parts == 0; a with unit
    column stride, b with unit column stride or the transpose of such a matrix."""
    M, K = a.shape
    N = b.shape[1]
    if K % parts or a.stride(1) != 1 or (b.stride(1) != 1 and b.stride(0) != 1):
        raise ValueError(f"matmul_split_k: K={K} must split into {parts} slices, unit strides")
    out = _blas.split_k(a, b, parts)
    if out is not None:
        return out
    c = K // parts
    a3 = a.as_strided((parts, M, c), (c, a.stride(0), 1))
    b3 = b.as_strided((parts, c, N), (c * b.stride(0), b.stride(0), b.stride(1)))
    partial = _blas.bmm_f32(a3, b3)                                 # [parts, M, N] fp32
    out = torch.empty((M, N), dtype=torch.float16, device=a.device)
    if M * N:
        _ext.call("soupk_sum_partials", partial.data_ptr(), parts, M * N, M * N,
                  out.data_ptr(), _ext.stream_of(out))
    return out


class FusedNF4MLP(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, gate_w, up_w, down_w, gate_up16=None, down16=None):
        # Without the caller's unpacked stacks, each product runs on the NF4 weights through
        # the fused NF4-dequant GEMM where that is the faster path (nf4.fused_linear: few
        # rows), else on W unpacked here.
        gate_up = gate_up16
        gu = fused_linear(x, (gate_w, up_w)) if gate_up is None and x.dim() == 2 else None
        if gu is None:
            if gate_up is None:
                gate_up = unpack_concat((gate_w, up_w), x.device)
            gu = _mm(x, gate_up.t())
        act = gated_silu(gu)
        ctx.recompute = RECOMPUTE_GATE_UP
        ctx.consumed = False
        if ctx.recompute:
            del gu
            ctx.save_for_backward(x)
        else:
            ctx.save_for_backward(x, gu)
        down = down16
        out = fused_linear(act, (down_w,)) if down is None and act.dim() == 2 else None
        if out is None:
            if down is None:
                down = unpack_concat((down_w,), x.device)
            parts = SPLIT_K_DOWN
            if parts is None and act.dim() == 2:
                parts = split_parts(act.shape[0], down.shape[0], act.shape[1], "down")
            if parts and parts > 1 and act.dim() == 2 and act.shape[1] % parts == 0 and \
                    act.shape[0] > 0:
                out = matmul_split_k(act, down.t(), parts)
            else:
                out = _mm(act, down.t())
        ctx.weights = (gate_w, up_w, down_w)
        keep_for_backward(ctx, (gate_up, down))
        return out

    @staticmethod
    def backward(ctx, grad_out):
        if not ctx.needs_input_grad[0]:
            return None, None, None, None, None, None
        gate_w, up_w, down_w = ctx.weights
        saved = ctx.saved_tensors
        x = saved[0]
        grad_out = grad_out.to(torch.float16)
        kept = getattr(ctx, "unpacked", None)
        ctx.unpacked = None
        gate_up, down = kept if kept is not None else (None, None)
        # a stack the forward did not unpack: the fused input gradient where it is the faster
        # path, else W unpacked here
        dact = None
        if down is None:
            dact = fused_grad_input(grad_out, (down_w,)) if grad_out.dim() == 2 else None
            if dact is None:
                down = unpack_concat((down_w,), grad_out.device)
        if dact is None:
            dact = _mm(grad_out, down)
        del down
        if ctx.recompute:
            gu = fused_linear(x, (gate_w, up_w)) if gate_up is None else None
            if gu is None:
                if gate_up is None:
                    gate_up = unpack_concat((gate_w, up_w), grad_out.device)
                gu = _mm(x, gate_up.t())
        else:
            if ctx.consumed:
                raise RuntimeError("FusedNF4MLP: backward ran twice through a graph whose kept "
                                   "gate/up buffer the first backward overwrote; set "
                                   "mlp.RECOMPUTE_GATE_UP = True to backpropagate twice")
            ctx.consumed = True
            gu = saved[1]
        gated_silu_backward_(dact, gu)
        del dact
        grad_x = None
        if gate_up is None:
            grad_x = fused_grad_input(gu, (gate_w, up_w)) if gu.dim() == 2 else None
            if grad_x is None:
                gate_up = unpack_concat((gate_w, up_w), grad_out.device)
        if grad_x is None:
            parts = SPLIT_K_GATE_UP
            if parts is None:
                parts = split_parts(gu.shape[0], gate_up.shape[1], gu.shape[1], "gate_up")
            if parts > 1 and gu.shape[1] % parts == 0 and gu.shape[0] > 0:
                grad_x = matmul_split_k(gu, gate_up, parts)
            else:
                grad_x = _mm(gu, gate_up)
        return grad_x, None, None, None, None, None


def fused_mlp(x, gate_w, up_w, down_w, gate_up16=None, down16=None):
    """down(silu(gate(x)) * up(x)); gate_up16 / down16, when given, are the gate|up and down
    stacks already unpacked (nf4.unpack_groups)."""
    if not kernels_ok(x):
        raise ValueError("fused_mlp: x must be a HIP device tensor (no CPU path)")
    return FusedNF4MLP.apply(x.contiguous(), gate_w, up_w, down_w, gate_up16, down16)
