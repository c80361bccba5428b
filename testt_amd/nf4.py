"""NF4 (bitsandbytes 4-bit, double quant) weight unpacking on gfx950, and the frozen 4-bit linear
that uses it.  Drop-in for solution/nf4.py (same names, arguments and fallbacks).

bitsandbytes stores a frozen projection as NF4: two 4-bit codes per byte (high nibble first),
one absmax per `blocksize` (64) values, and with double quant ("nested") the absmax itself is
an 8-bit code into a 256-entry table, scaled per 256 absmax blocks and shifted by one offset:

    absmax[b] = code2[absmax_u8[b]] * absmax2[b // 256] + offset
    w[i]      = nf4[q[i]] * absmax[i // 64]          (fp32, rounded once to fp16)

`soupk_nf4_unpack` (testt_amd/csrc/nf4_unpack.hip) does this in one HBM pass, rounding each
product and sum separately as bitsandbytes does, so the fp16 values are bit-identical to
bitsandbytes' dequantize_4bit.  Several projections are unpacked into one buffer so that q/k/v
or gate/up run as a single hipBLASLt GEMM (torch.matmul).
"""

import ctypes
import weakref

import torch

from . import _ext
from . import blas
from ._common import kernels_ok

# One workgroup step of the unpack kernel: 256 threads x 4 chunks x 16 packed bytes.
# (solution/nf4.py:24 names the per-program tile of the Triton kernel the same way.)
BYTES_PER_PROGRAM = 16384

# The reference unpacks every frozen weight twice per step, in forward and again in backward
# (solution/nf4.py:125, solution/mlp.py:105-108), so that no fp16 weight outlives its GEMM.
# On MI355X the fp16 weights of all 28 layers of Qwen2.5-1.5B are 2.6 GB (under 1% of 288 GB
# of HBM), so by default the forward's unpacked weight is kept for the backward GEMM and
# dropped there: one unpack pass per step instead of two, identical results (the unpack is
# deterministic).  False restores the reference's memory profile.
KEEP_UNPACKED_FOR_BACKWARD = True

# FrozenNF4Linear through the fused NF4-dequant GEMM (testt_amd/nf4_gemm.py: W read as NF4,
# dequantised in the GEMM's tile loads, no fp16 W in HBM) where it measured ahead of unpack +
# hipBLASLt on MI355X (nf4_gemm.prefer_fused, prefer_fused_grad_input: a grid of half to one
# wave of the compute units and a contraction of at most 2048, e.g. the q|k|v and o forward at
# 1024-2048 rows, the gate|up forward at up to 128 rows, the q|k|v and o input gradient at
# 1024 rows, down's input gradient at up to 128 rows; and below half a wave with the
# contraction split, e.g. the q|k|v, o and down forward and the q|k|v, o and gate|up input
# gradient at up to 256 rows); elsewhere unpack + hipBLASLt runs.  Only
# a forward that unpacks W itself uses it: a caller that passes the unpacked weight (the
# decoder layer's one-launch unpack of all seven projections) keeps hipBLASLt, and so does a
# backward that has the forward's unpacked weight (KEEP_UNPACKED_FOR_BACKWARD).
USE_FUSED_NF4_GEMM = True


def keep_for_backward(ctx, weight):
    """Hold the forward's unpacked fp16 `weight` in ctx when a backward may read it (an input
    needs a gradient; a forward outside autograd frees ctx, and the weight, with its outputs).
    Grad mode is always off inside autograd.Function.forward, so it is not consulted."""
    keep = KEEP_UNPACKED_FOR_BACKWARD and any(ctx.needs_input_grad)
    ctx.unpacked = weight if keep else None


def unpacked_for_backward(ctx, weights, device):
    """The weight the forward kept (released from ctx), else `weights` unpacked again."""
    weight = getattr(ctx, "unpacked", None)
    ctx.unpacked = None
    return weight if weight is not None else unpack_concat(weights, device)


def _quant_state(weight):
    return getattr(weight, "quant_state", None)


def supports_fast_unpack(weight):
    """True for the layout the kernel handles: NF4, nested absmax with 256-blocks, even sizes.

    Same predicate as solution/nf4.py:52-62."""
    state = _quant_state(weight)
    if state is None or getattr(state, "quant_type", None) != "nf4" or not state.nested:
        return False
    if state.state2 is None or state.state2.blocksize != 256 or state.blocksize % 2:
        return False
    shape = tuple(state.shape)
    if len(shape) != 2 or (shape[0] * shape[1]) % state.blocksize:
        return False
    return weight.data.dtype == torch.uint8 and weight.data.is_contiguous()


def _on_device(weight, device):
    state = _quant_state(weight)
    tensors = (weight.data, state.absmax, state.code, state.state2.code, state.state2.absmax)
    return all(t.device == device for t in tensors) and \
        (not torch.is_tensor(state.offset) or state.offset.device == device)


def _offset_tensor(state, device):
    off = state.offset
    if torch.is_tensor(off):
        off = off.reshape(-1)[:1]
        return off if off.dtype == torch.float32 else off.float()
    return torch.tensor([float(off)], dtype=torch.float32, device=device)


def _f32(t):
    return t if t.dtype == torch.float32 and t.is_contiguous() else t.float().contiguous()


def _plan_key(weight, device):
    """What a cached plan of `weight` depends on: the addresses of its packed data and state
    tensors and the offset object (None for an object that is not an NF4 weight)."""
    state = _quant_state(weight)
    try:
        return (device, weight.data.data_ptr(), state.absmax.data_ptr(), state.code.data_ptr(),
                state.state2.code.data_ptr(), state.state2.absmax.data_ptr(), id(state.offset))
    except AttributeError:
        return None


def _plan(weight, device):
    """The kernel arguments of one weight on `device` (pointers into its quant state, converted
    tables kept alive), checked once and cached on the weight; None for a layout or device the
    kernel does not take.  The cache is keyed by the addresses of the state tensors, so a
    weight whose state is replaced is checked again."""
    key = _plan_key(weight, device)
    if key is None:
        return None
    state = _quant_state(weight)
    cached = getattr(weight, "_soupk_plan", None)
    if cached is not None and cached[0] == key:
        return cached[1]
    if not (supports_fast_unpack(weight) and _on_device(weight, device)):
        return None
    if state.absmax.dtype != torch.uint8:
        raise TypeError(f"nested absmax must be uint8, got {state.absmax.dtype}")
    n_bytes = weight.data.numel()
    absmax = state.absmax.contiguous()
    code2 = _f32(state.state2.code)
    absmax2 = _f32(state.state2.absmax)
    nf4 = _f32(state.code)
    if code2.numel() < 256 or nf4.numel() < 16:
        raise ValueError("quant state tables are too small (code2 needs 256, nf4 16 entries)")
    n_blocks = -(-n_bytes // (state.blocksize // 2))
    if absmax.numel() < n_blocks or absmax2.numel() < -(-n_blocks // 256):
        raise ValueError("quant state absmax arrays do not cover the weight")
    offset = _offset_tensor(state, device)
    plan = ((_ext.ptr(weight.data), _ext.ptr(absmax), _ext.ptr(code2), _ext.ptr(absmax2),
             _ext.ptr(offset), _ext.ptr(nf4)), n_bytes, int(state.blocksize),
            int(state.state2.blocksize), (absmax, code2, absmax2, nf4, offset))
    try:
        weight._soupk_plan = (key, plan)
    except AttributeError:          # objects without a __dict__ are checked on every call
        pass
    return plan


def unpack_into(weight, out):
    """Write the fp16 values of one bitsandbytes 4-bit weight ([N, K]) into `out` ([N, K]).

    Mirrors solution/nf4.py:72-89: the HIP kernel for the supported layout on the device,
    bitsandbytes' own dequantize_4bit for other layouts (as the reference does).  CPU tensors
    are rejected: this build has no CPU path."""
    if not kernels_ok(out):
        raise ValueError("unpack_into: `out` must be a HIP device tensor (no CPU path)")
    plan = _plan(weight, out.device)
    if plan is not None:
        ptrs, n_bytes, qblock, qblock2, _ = plan
        _ext.require(out, "out", dtype=torch.float16)
        if out.numel() != 2 * n_bytes:
            raise ValueError(f"out has {out.numel()} elements, the weight holds {2 * n_bytes}")
        _ext.call("soupk_nf4_unpack", *ptrs, out.data_ptr(), n_bytes, qblock, qblock2,
                  _ext.stream_of(out))
        return out
    import bitsandbytes.functional as bnb_functional

    state = _quant_state(weight)
    out.copy_(bnb_functional.dequantize_4bit(weight.data, state).to(out.dtype).view_as(out))
    return out


def weight_shape(weight):
    return tuple(_quant_state(weight).shape)


# Most weights soupk_nf4_unpack_multi takes in one launch.
MAX_PARTS_PER_LAUNCH = 8


def unpack_many(weights, outs):
    """unpack_into(w, o) for every pair, as few launches as the kernel allows: the weights with
    a kernel plan that share one (qblock, qblock2) go through soupk_nf4_unpack_multi, up to
    MAX_PARTS_PER_LAUNCH per launch, the rest through unpack_into."""
    if not outs:
        return
    if not all(kernels_ok(o) for o in outs):
        raise ValueError("unpack_many: outputs must be HIP device tensors (no CPU path)")
    groups = {}
    for weight, out in zip(weights, outs, strict=True):
        plan = _plan(weight, out.device)
        if plan is None or out.device != outs[0].device:
            unpack_into(weight, out)
            continue
        _ext.require(out, "out", dtype=torch.float16)
        if out.numel() != 2 * plan[1] or not out.is_contiguous():
            raise ValueError(f"out has {out.numel()} elements (contiguous: "
                             f"{out.is_contiguous()}), the weight holds {2 * plan[1]}")
        groups.setdefault((plan[2], plan[3]), []).append((plan, out))
    for (qblock, qblock2), items in groups.items():
        for c in range(0, len(items), MAX_PARTS_PER_LAUNCH):
            chunk = items[c:c + MAX_PARTS_PER_LAUNCH]
            n = len(chunk)
            arrays = [(ctypes.c_void_p * n)(*[p[0][i] for p, _ in chunk]) for i in range(6)]
            outs_a = (ctypes.c_void_p * n)(*[o.data_ptr() for _, o in chunk])
            sizes = (ctypes.c_int64 * n)(*[p[1] for p, _ in chunk])
            _ext.call("soupk_nf4_unpack_multi", n, *[ctypes.addressof(a) for a in arrays],
                      ctypes.addressof(outs_a), ctypes.addressof(sizes), qblock, qblock2,
                      _ext.stream_of(chunk[0][1]))


def unpack_concat(weights, device):
    """fp16 [sum N_i, K]: the weights stacked by rows, unpacked in place (one launch)."""
    rows = [weight_shape(w)[0] for w in weights]
    cols = weight_shape(weights[0])[1]
    out = torch.empty((sum(rows), cols), dtype=torch.float16, device=device)
    views, start = [], 0
    for n in rows:
        views.append(out[start:start + n])
        start += n
    unpack_many(weights, views)
    return out


# Row stacks placed in one buffer by unpack_groups start at multiples of this many elements
# (512 bytes), the alignment the GEMM kernels are given for separately allocated weights.
_GROUP_ALIGN = 256


def _weak(obj):
    """A weak reference to `obj` (a callable giving it back), or a strong one for objects that
    take no weak reference."""
    try:
        return weakref.ref(obj)
    except TypeError:
        return lambda: obj


class _GroupPlan:
    """unpack_groups' launches for one list of weight groups, prepared once: the buffer size,
    each stack's place in it, and per launch the NF4 state pointer tables and sizes (ctypes
    arrays) and the byte offsets of the outputs; a call allocates the buffer and adds its
    address.

    One plan is kept on the first weight of the list (a later list that starts with the same
    weight replaces it).  It holds the weights only weakly, so it keeps no replaced weight
    alive and forms no reference cycle with the weight that carries it, and it is used only for
    the same device, the same grouping and the same weights (by identity), each with an
    unchanged plan key (its packed data and state tensors, _plan_key)."""

    def __init__(self, device, sizes, flat_w, offsets, stacks, total):
        plans = [_plan(w, device) for w in flat_w]
        self.ok = all(pl is not None for pl in plans) and len({(pl[2], pl[3]) for pl in plans}) == 1
        self.total, self.stacks = total, stacks
        self.device, self.sizes = device, sizes
        self.check = [(_weak(w), _plan_key(w, device)) for w in flat_w]
        self.launches = []
        if not self.ok:
            return
        self.qblock, self.qblock2 = plans[0][2], plans[0][3]
        self.keep = [pl[4] for pl in plans]
        for c in range(0, len(plans), MAX_PARTS_PER_LAUNCH):
            chunk = plans[c:c + MAX_PARTS_PER_LAUNCH]
            n = len(chunk)
            arrays = [(ctypes.c_void_p * n)(*[pl[0][i] for pl in chunk]) for i in range(6)]
            sizes = (ctypes.c_int64 * n)(*[pl[1] for pl in chunk])
            self.launches.append((n, arrays, sizes, [2 * o for o in offsets[c:c + n]]))

    def matches(self, device, sizes, flat_w):
        if device != self.device or sizes != self.sizes or len(flat_w) != len(self.check):
            return False
        return all(ref() is w and _plan_key(w, device) == key
                   for (ref, key), w in zip(self.check, flat_w))

    def run(self, device, lora_params=None):
        """The stacks; with lora_params (a_q, a_v, b_q, b_v), also their fp16 staging
        (lora.stage) by the same launch, placed after the stacks: (stacks, staged)."""
        extra = 0
        if lora_params is not None:
            from . import lora as _lora

            a_q = lora_params[0]
            H = a_q.shape[1]
            NQ, NV = _lora._check_params(*lora_params, H, device)
            extra = _lora.staged_elems(H, NQ, NV)
        buf = torch.empty(self.total, dtype=torch.float16, device=device)
        # The staged parameters get an allocation of their own (304 KB at Qwen2.5-1.5B's
        # shapes): the LoRA backward keeps them, and a view into `buf` would keep all seven
        # fp16 projections (94 MB per layer) alive with them until that layer's backward.
        staged = torch.empty(extra, dtype=torch.float16, device=device) if extra else None
        base = buf.data_ptr()
        stream = _ext.stream_of(buf)
        last = len(self.launches) - 1
        for c, (n, arrays, sizes, out_offsets) in enumerate(self.launches):
            outs = (ctypes.c_void_p * n)(*[base + o for o in out_offsets])
            args = (n, *[ctypes.addressof(a) for a in arrays], ctypes.addressof(outs),
                    ctypes.addressof(sizes), self.qblock, self.qblock2)
            if extra and c == last:
                _ext.call("soupk_nf4_unpack_multi_lora", *args,
                          *[p.data_ptr() for p in lora_params], staged.data_ptr(), extra,
                          H, NQ, NV, _lora.RANK, stream)
            else:
                _ext.call("soupk_nf4_unpack_multi", *args, stream)
        stacks = [buf[st:st + rows * cols].view(rows, cols) for st, rows, cols in self.stacks]
        if lora_params is None:
            return stacks
        return stacks, staged


def _group_plan(groups, device, flat_w, offsets, stacks, total):
    sizes = tuple(len(g) for g in groups)
    plan = getattr(flat_w[0], "_soupk_groups", None)
    if plan is None or not plan.matches(device, sizes, flat_w):
        plan = _GroupPlan(device, sizes, flat_w, offsets, stacks, total)
        try:
            flat_w[0]._soupk_groups = plan
        except AttributeError:      # an object without a __dict__: planned on every call
            pass
    return plan


def unpack_groups_lora(groups, device, lora_params):
    """unpack_groups plus the fp16 staging of a decoder layer's LoRA parameters
    lora_params = (a_q, a_v, b_q, b_v) (testt_amd.lora.stage's buffer) in the same launch:
    (stacks, staged)."""
    device = _hip_device(device)
    flat_w, offsets, stacks, total = _group_layout(groups)
    if flat_w:
        plan = _group_plan(groups, device, flat_w, offsets, stacks, total)
        if plan.ok and plan.launches:
            return plan.run(device, lora_params)
    from . import lora as _lora

    return _unpack_groups_generic(groups, device), _lora.stage(*lora_params)


def unpack_groups(groups, device):
    """One fp16 [sum N_i, K] row stack per group of weights (unpack_concat of each group), all
    unpacked by one launch into a single buffer: the projections of a decoder layer
    (q|k|v, o, gate|up, down) before its forward.  Returns the stacks, views of the buffer.
    The launch arguments are prepared once per list of weights (_GroupPlan) and checked on each
    call with the same key as each weight's own plan."""
    device = _hip_device(device)
    flat_w, offsets, stacks, total = _group_layout(groups)
    if flat_w:
        plan = _group_plan(groups, device, flat_w, offsets, stacks, total)
        if plan.ok:
            return plan.run(device)
    return _unpack_groups_generic(groups, device)


def _hip_device(device):
    device = torch.device(device)
    if device.type != "cuda":
        raise ValueError("unpack_groups: the device must be a HIP device (no CPU path)")
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    return device


def _group_layout(groups):
    """The weights in order, each one's element offset in the buffer, each stack's
    (offset, rows, cols), and the buffer's size (stacks at multiples of _GROUP_ALIGN)."""
    flat_w, offsets, stacks, total = [], [], [], 0
    for weights in groups:
        rows = [weight_shape(w)[0] for w in weights]
        cols = weight_shape(weights[0])[1]
        if any(weight_shape(w)[1] != cols for w in weights):
            raise ValueError("weights of one group must have the same number of columns")
        stacks.append((total, sum(rows), cols))
        r0 = 0
        for w, n in zip(weights, rows):
            flat_w.append(w)
            offsets.append(total + r0 * cols)
            r0 += n
        total += -(-sum(rows) * cols // _GROUP_ALIGN) * _GROUP_ALIGN
    return flat_w, offsets, stacks, total


def _unpack_groups_generic(groups, device):
    """unpack_groups through unpack_many (layouts or devices a prepared launch does not take)."""
    shapes, total = [], 0
    for weights in groups:
        rows = [weight_shape(w)[0] for w in weights]
        cols = weight_shape(weights[0])[1]
        if any(weight_shape(w)[1] != cols for w in weights):
            raise ValueError("weights of one group must have the same number of columns")
        shapes.append((total, rows, cols))
        total += -(-sum(rows) * cols // _GROUP_ALIGN) * _GROUP_ALIGN
    buf = torch.empty(total, dtype=torch.float16, device=device)
    stacks, flat_w, flat_o = [], [], []
    for weights, (start, rows, cols) in zip(groups, shapes):
        stack = buf[start:start + sum(rows) * cols].view(sum(rows), cols)
        stacks.append(stack)
        r0 = 0
        for w, n in zip(weights, rows):
            flat_w.append(w)
            flat_o.append(stack[r0:r0 + n])
            r0 += n
    unpack_many(flat_w, flat_o)
    return stacks


def fused_linear(x2, weights, bias=None):
    """x2 [M, K] @ W^T (+ bias), W the row stack of the NF4 `weights`, through the fused
    NF4-dequant GEMM where that is the faster path for this problem (nf4_gemm.prefer_fused);
    None elsewhere, and the caller unpacks W."""
    if not USE_FUSED_NF4_GEMM:
        return None
    from . import nf4_gemm

    if nf4_gemm.supported(x2, weights, bias) and nf4_gemm.prefer_fused(x2, weights):
        return nf4_gemm.nf4_linear(x2, weights, bias)
    return None


def fused_grad_input(g2, weights):
    """g2 [M, N] @ W (the input gradient of fused_linear's product) through the fused NF4
    input-gradient GEMM where that is the faster path (nf4_gemm.prefer_fused_grad_input); None
    elsewhere."""
    if not USE_FUSED_NF4_GEMM:
        return None
    from . import nf4_gemm

    if nf4_gemm.grad_input_supported(g2, weights) and \
            nf4_gemm.prefer_fused_grad_input(g2, weights):
        return nf4_gemm.nf4_grad_input(g2, weights)
    return None


class FrozenNF4Linear(torch.autograd.Function):
    """y = x @ W^T (+ b) for frozen 4-bit weights stacked by rows, fp16 in and out.

    No input is kept because W does not train (solution/nf4.py:108-127); the unpacked weight
    (`w16` when the caller unpacked it already) is kept for backward or unpacked again there
    (KEEP_UNPACKED_FOR_BACKWARD)."""

    @staticmethod
    def forward(ctx, x, bias, weights, w16=None):
        ctx.weights = weights
        if w16 is None:
            out = fused_linear(x.reshape(-1, x.shape[-1]), weights, bias)
            if out is not None:
                ctx.unpacked = None
                return out.view(*x.shape[:-1], out.shape[-1])
        weight = w16 if w16 is not None else unpack_concat(weights, x.device)
        if x.dim() == 2 or x.is_contiguous():
            out = blas.linear(x.reshape(-1, x.shape[-1]), weight, bias)
            out = out.view(*x.shape[:-1], out.shape[-1])
        else:
            out = torch.nn.functional.linear(x, weight, bias)
        keep_for_backward(ctx, weight)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        grad_x = None
        if ctx.needs_input_grad[0]:
            g = grad_out.to(torch.float16)
            if getattr(ctx, "unpacked", None) is None:
                # no unpacked weight kept: the fused input gradient where it is the faster path
                dx = fused_grad_input(g.reshape(-1, g.shape[-1]), ctx.weights)
                if dx is not None:
                    return dx.view(*g.shape[:-1], dx.shape[-1]), None, None, None
            weight = unpacked_for_backward(ctx, ctx.weights, grad_out.device)
            if g.dim() == 2:
                grad_x = blas.matmul(g, weight)
            else:
                grad_x = g @ weight
        return grad_x, None, None, None


def frozen_linear(x, weights, bias=None, w16=None):
    """x @ W^T (+ bias), W the row stack of `weights`; `w16`, when given, is that stack already
    unpacked (unpack_groups), used instead of unpacking again."""
    return FrozenNF4Linear.apply(x, bias, tuple(weights), w16)
