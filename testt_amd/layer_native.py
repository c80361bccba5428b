"""The decoder layer's fused path as one native call each way (soupk_layer_fwd / _bwd).

testt_amd/layer.py's DecoderLayer runs the layer's five autograd nodes inside one, each
operation still issued from Python: its checks, its allocation, its ctypes call.  On the
MI355X box that made the eager layer host-bound at the ragged batch (about 485 us of issue time
against 420 us of GPU time).  NativeDecoderLayer issues the same launches from C with the same
arguments (csrc/layer_exec.hip), so the values are DecoderLayer's bit for bit; Python allocates
the buffers (one arena for what the backward reads, one for the forward's temporaries, one for
the backward's scratch) and fills two argument structs.

Used by layer.decoder_layer when NATIVE_LAYER is set and the layer takes the fused path with its
weights unpacked once for forward and backward (the default): LoRA rank 16 on q and v without
dropout, head dim 128, no o-projection bias, the direct hipBLASLt GEMMs on, the unpacked weights
kept for backward and the gate|up buffer kept (not recomputed).
"""

import ctypes

import torch

from . import _ext
from . import blas as _blas
from . import mlp as _mlp

NATIVE_LAYER = True

_p, _i32, _i64, _f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float


class Nf4Group(ctypes.Structure):
    _fields_ = ([("n_parts", _i32), ("rows", _i32 * 4)] +
                [(n, _p * 4) for n in ("packed", "absmax", "code2", "absmax2", "offset", "nf4")])


class LayerNf4(ctypes.Structure):
    _fields_ = ([(n, Nf4Group) for n in ("qkv", "o", "gu", "down")] +
                [("split_fwd", _i32 * 4), ("split_bwd", _i32 * 4), ("partials", _p),
                 ("partials_floats", _i64)])


class LayerDims(ctypes.Structure):
    _fields_ = ([("M", _i64)] +
                [(n, _i32) for n in ("H", "NH", "NKV", "D", "I", "r", "batch", "seq", "p_down",
                                     "p_gu")] +
                [(n, _f32) for n in ("eps", "scaling", "scale")] +
                [(n, _p) for n in ("norm1", "norm2", "qkv_bias", "w_qkv", "w_o", "w_gu", "w_d",
                                   "staged", "cos", "sin", "pos", "cu", "gemm_ws")] +
                [("gemm_ws_bytes", _i64), ("nf4", _p)])


class LayerFwd(ctypes.Structure):
    _fields_ = ([("s_in", _p), ("delta", _p)] +
                [(n, _i32) for n in ("algo_qkv", "algo_o", "algo_gu", "algo_down")] +
                [(n, _p) for n in ("s1", "y", "rstd1", "t", "qkv_r", "attn", "lse", "s2", "y2",
                                   "rstd2", "gu", "qkv", "o", "act", "down_part", "d")])


class LayerBwd(ctypes.Structure):
    _fields_ = ([(n, _p) for n in ("s_in", "s1", "rstd1", "y", "t", "qkv_r", "attn", "lse", "s2",
                                   "rstd2", "y2", "gu")] +
                [(n, _i32) for n in ("has_delta", "algo_down_dx", "algo_gu_dx", "algo_o_dx",
                                     "algo_qkv_dx")] +
                [(n, _p) for n in ("g_s", "g_d", "dact", "gu_part", "g_y2", "g_s1", "g_o", "g_a",
                                   "attn_ws", "dqkv", "dt", "dy", "lora_ws")] +
                [("lora_ws_floats", _i64)] +
                [(n, _p) for n in ("g_s_in", "g_delta", "d_aq", "d_av", "d_bq", "d_bv")])


_F16, _F32 = 2, 4


def _arena(device, parts):
    """One uint8 allocation holding `parts` ([(name, bytes)], each 256-byte aligned): the
    tensor and {name: device address}."""
    offs, total = {}, 0
    for name, nbytes in parts:
        offs[name] = total
        total += (nbytes + 255) // 256 * 256
    buf = torch.empty(max(total, 256), dtype=torch.uint8, device=device)
    base = buf.data_ptr()
    return buf, {n: base + o for n, o in offs.items()}


def _common(s, delta, w, inter):
    from . import lora as _lora
    from . import mlp

    return (NATIVE_LAYER and not mlp.RECOMPUTE_GATE_UP and w.o_bias is None and
            s.dtype == torch.float32 and (delta is None or delta.dtype == torch.float16) and
            w.head_dim == 128 and _lora.RANK == 16 and s.dim() == 2 and s.shape[1] % 8 == 0 and
            inter % 8 == 0 and s.is_cuda)


def supported(s, delta, w, w_qkv, w_o, w_gu, w_d, staged):
    """The layer on its unpacked fp16 stacks (hipBLASLt products)."""
    from . import nf4

    return (_blas.USE_GEMM_LT and nf4.KEEP_UNPACKED_FOR_BACKWARD and staged is not None and
            all(x is not None for x in (w_qkv, w_o, w_gu, w_d)) and w_d.dim() == 2 and
            _common(s, delta, w, w_d.shape[1]))


def supported_nf4(s, delta, w):
    """The layer on its NF4 weights (fused NF4-dequant products; the caller checked their
    layout, layer.nf4_resident)."""
    from . import nf4

    return nf4.USE_FUSED_NF4_GEMM and _common(s, delta, w, nf4.weight_shape(w.down)[1])


def _nf4_group(weights, dev):
    from . import nf4

    g = Nf4Group()
    g.n_parts = len(weights)
    for i, x in enumerate(weights):
        g.rows[i] = nf4.weight_shape(x)[0]
        (g.packed[i], g.absmax[i], g.code2[i], g.absmax2[i], g.offset[i],
         g.nf4[i]) = nf4._plan(x, dev)[0]
    return g


def _nf4_layer(w, M, dev):
    """The LayerNf4 of a layer's NF4 weights at M tokens: the split counts nf4_gemm's
    nf4_linear and nf4_grad_input pick, and the floats of the largest split's partials
    (partials unset).  Remembered on the q weight per token count, device and weight state (the
    addresses of the seven weights' NF4 data and tables, as nf4's plan cache keys them), so
    that it lives as long as the weights whose tables it points at; a fresh copy of the
    remembered struct per call."""
    from . import nf4

    weights = (w.q, w.k, w.v, w.o, w.gate, w.up, w.down)
    key = (M, dev, tuple(nf4._plan_key(x, dev) for x in weights))
    memo = getattr(w.q, "_soupk_layer_nf4", None)
    if memo is None:
        memo = {}
        setattr(w.q, "_soupk_layer_nf4", memo)
    hit = memo.get(key)
    if hit is None:
        if len(memo) > 64:
            memo.clear()
        n4, fwd, bwd = _build_nf4_layer(w, M, dev)
        hit = memo[key] = (bytes(n4), fwd, bwd)
    return LayerNf4.from_buffer_copy(hit[0]), hit[1], hit[2]


def _build_nf4_layer(w, M, dev):
    from . import nf4, nf4_gemm

    groups = ((w.q, w.k, w.v), (w.o,), (w.gate, w.up), (w.down,))
    cus = nf4_gemm._cu_count(dev)
    n4 = LayerNf4()
    fwd_floats = bwd_floats = 4
    for i, (name, weights) in enumerate(zip(("qkv", "o", "gu", "down"), groups)):
        setattr(n4, name, _nf4_group(weights, dev))
        rows = sum(nf4.weight_shape(x)[0] for x in weights)
        cols = nf4.weight_shape(weights[0])[1]
        fwd = nf4_gemm.split_count(M, rows, cols, cus)
        bwd = nf4_gemm.split_count(M, cols, rows, cus, nf4_gemm.GRAD_TILE)
        n4.split_fwd[i], n4.split_bwd[i] = fwd, bwd
        if fwd > 1:
            fwd_floats = max(fwd_floats, nf4_gemm._split_used(cols // 64, fwd)[1] * M * rows)
        if bwd > 1:
            bwd_floats = max(bwd_floats, nf4_gemm._split_used(rows // 64, bwd)[1] * M * cols)
    return n4, fwd_floats, bwd_floats


class NativeDecoderLayer(torch.autograd.Function):
    """(s, d) of the layer's fused path, forward and backward each one soupk call."""

    @staticmethod
    def forward(ctx, s_in, delta, a_q, b_q, a_v, b_v, w, w_qkv, w_o, w_gu, w_d, staged, cos32,
                sin32, pos, cu, batch, seq, scale):
        from . import nf4
        from .rmsnorm import _weight32

        dev = s_in.device
        M, H = s_in.shape
        on_nf4 = w_qkv is None          # the products on the NF4 weights (few tokens)
        I = nf4.weight_shape(w.down)[1] if on_nf4 else w_d.shape[1]
        NH, NKV, D, r = w.n_heads, w.n_kv, 128, 16
        NQ, NV = NH * D, NKV * D
        W = NQ + 2 * NV
        if on_nf4:
            p_down = p_gu = 1
            n4, floats, ctx.bwd_floats = _nf4_layer(w, M, dev)
            partials = torch.empty(floats, dtype=torch.float32, device=dev)
            n4.partials, n4.partials_floats = partials.data_ptr(), partials.numel()
        else:
            n4 = partials = None
            p_down = _mlp.SPLIT_K_DOWN or _mlp.split_parts(M, H, I, "down")
            p_gu = _mlp.SPLIT_K_GATE_UP or _mlp.split_parts(M, H, 2 * I, "gate_up")
            if I % p_down:
                p_down = 1
            if (2 * I) % p_gu:
                p_gu = 1
        st = _ext.stream_of(s_in)
        ws = None if on_nf4 else _blas._ws(dev)
        norm1, norm2 = _weight32(w.input_norm, H, dev), _weight32(w.post_norm, H, dev)
        bias = w.qkv_bias
        dims = LayerDims(M, H, NH, NKV, D, I, r, batch, seq, p_down, p_gu, float(w.eps),
                         float(w.scaling), float(scale), norm1.data_ptr(), norm2.data_ptr(),
                         _ext.ptr(bias), _ext.ptr(w_qkv), _ext.ptr(w_o), _ext.ptr(w_gu),
                         _ext.ptr(w_d), staged.data_ptr(), cos32.data_ptr(), sin32.data_ptr(),
                         pos.data_ptr(), cu.data_ptr(), _ext.ptr(ws),
                         0 if on_nf4 else _blas.WORKSPACE_BYTES,
                         ctypes.addressof(n4) if on_nf4 else None)
        has_delta = delta is not None
        keep, kp = _arena(dev, [("s1", M * H * _F32 if has_delta else 0), ("y", M * H * _F16),
                                ("rstd1", M * _F32), ("t", M * 2 * r * _F16),
                                ("qkv_r", M * W * _F16), ("attn", M * NQ * _F16),
                                ("lse", NH * M * _F32), ("y2", M * H * _F16),
                                ("rstd2", M * _F32), ("gu", M * 2 * I * _F16)])
        tmp, tp = _arena(dev, [("qkv", M * W * _F16), ("o", M * H * _F16),
                               ("act", M * I * _F16),
                               ("down_part", p_down * M * H * _F32 if p_down > 1 else 0)])
        s2 = torch.empty((M, H), dtype=torch.float32, device=dev)
        d = torch.empty((M, H), dtype=torch.float16, device=dev)
        t = _blas._table
        args = LayerFwd(
            s_in.data_ptr(), _ext.ptr(delta),
            t.get(("tn", W, M, H, H, H, W, bias is not None), -1),
            t.get(("tn", H, M, NQ, NQ, NQ, H, False), -1),
            t.get(("tn", 2 * I, M, H, H, H, 2 * I, False), -1),
            t.get(("tn", H, M, I, I, I, H, False), -1),
            kp["s1"], kp["y"], kp["rstd1"], kp["t"], kp["qkv_r"], kp["attn"], kp["lse"],
            s2.data_ptr(), kp["y2"], kp["rstd2"], kp["gu"], tp["qkv"], tp["o"], tp["act"],
            tp["down_part"], d.data_ptr())
        _ext.call("soupk_layer_fwd", ctypes.addressof(dims), ctypes.addressof(args), st)
        del tmp, ws, partials
        ctx.save_for_backward(s_in, s2)
        ctx.keep, ctx.kp = keep, kp
        ctx.nf4 = n4                    # dims.nf4 points at it
        # what the backward reads besides: the weights, LoRA parameters and tables (inputs)
        ctx.inputs = (w_qkv, w_o, w_gu, w_d, staged, cos32, sin32, pos, cu, norm1, norm2, bias,
                      a_q, a_v, b_q, b_v, w)      # w: the NF4 weights dims.nf4 points into
        ctx.dims = dims
        ctx.has_delta = has_delta
        ctx.consumed = False
        return s2, d

    @staticmethod
    def backward(ctx, g_s, g_d):
        if ctx.consumed:
            raise RuntimeError("NativeDecoderLayer: backward ran twice through a graph whose kept "
                               "gate/up buffer the first backward overwrote; set "
                               "mlp.RECOMPUTE_GATE_UP = True to backpropagate twice")
        ctx.consumed = True
        s_in, s2 = ctx.saved_tensors
        dims, kp, keep = ctx.dims, ctx.kp, ctx.keep
        dev = s_in.device
        M, H, NH, NKV, I, r = dims.M, dims.H, dims.NH, dims.NKV, dims.I, dims.r
        NQ, NV = NH * 128, NKV * 128
        W = NQ + 2 * NV
        p_gu = dims.p_gu
        g_s = g_s.to(torch.float32).contiguous()
        g_d = g_d.to(torch.float16).contiguous()
        slices = (M + 127) // 128
        lora_ws_floats = max(slices * (2 * r * H + r * (NQ + NV)), 4)
        n_delta = (M * NH + 3) // 4 * 4
        scratch, sp = _arena(dev, [
            ("dact", M * I * _F16), ("gu_part", p_gu * M * H * _F32 if p_gu > 1 else 0),
            ("g_y2", M * H * _F16), ("g_s1", M * H * _F32), ("g_o", M * H * _F16),
            ("g_a", M * NQ * _F16), ("attn_ws", (n_delta + 2 * M * NQ) * _F32),
            ("dqkv", M * W * _F16), ("dt", M * 2 * r * _F16), ("dy", M * H * _F16),
            ("lora_ws", lora_ws_floats * _F32)])
        g_s_in = torch.empty((M, H), dtype=torch.float32, device=dev)
        g_delta = torch.empty((M, H), dtype=torch.float16, device=dev) if ctx.has_delta else None
        d_aq = torch.empty((r, H), dtype=torch.float32, device=dev)
        d_av = torch.empty((r, H), dtype=torch.float32, device=dev)
        d_bq = torch.empty((NQ, r), dtype=torch.float32, device=dev)
        d_bv = torch.empty((NV, r), dtype=torch.float32, device=dev)
        t = _blas._table
        args = LayerBwd(
            s_in.data_ptr(), kp["s1"], kp["rstd1"], kp["y"], kp["t"], kp["qkv_r"], kp["attn"],
            kp["lse"], s2.data_ptr(), kp["rstd2"], kp["y2"], kp["gu"], int(ctx.has_delta),
            t.get(("nn", I, M, H, I, H, I, False), -1),
            t.get(("nn", H, M, 2 * I, H, 2 * I, H, False), -1),
            t.get(("nn", NQ, M, H, NQ, H, NQ, False), -1),
            t.get(("nn", H, M, W, H, W, H, False), -1),
            g_s.data_ptr(), g_d.data_ptr(), sp["dact"], sp["gu_part"], sp["g_y2"], sp["g_s1"],
            sp["g_o"], sp["g_a"], sp["attn_ws"], sp["dqkv"], sp["dt"], sp["dy"], sp["lora_ws"],
            lora_ws_floats, g_s_in.data_ptr(), _ext.ptr(g_delta), d_aq.data_ptr(),
            d_av.data_ptr(), d_bq.data_ptr(), d_bv.data_ptr())
        st = _ext.stream_of(g_s_in)
        n4 = ctx.nf4
        if n4 is not None:
            # the split products' partials, from the stream the backward runs on
            ws = torch.empty(ctx.bwd_floats, dtype=torch.float32, device=dev)
            n4.partials, n4.partials_floats = ws.data_ptr(), ws.numel()
        else:
            ws = _blas._ws(dev)       # a workspace of the stream the backward runs on
            dims.gemm_ws = ws.data_ptr()
        _ext.call("soupk_layer_bwd", ctypes.addressof(dims), ctypes.addressof(args), st)
        del ws
        if not ctx.has_delta:
            # s_in is also the residual: its gradient adds the residual's (two terms, so the
            # order the engine would sum them in does not matter)
            g_s_in.add_(_view_f32(scratch, sp["g_s1"], M, H))
        ctx.keep = ctx.kp = ctx.inputs = ctx.nf4 = None
        del keep, scratch
        return (g_s_in, g_delta, d_aq, d_bq, d_av, d_bv) + (None,) * 13


def _view_f32(buf, addr, rows, cols):
    """The fp32 [rows, cols] tensor at device address `addr` inside the uint8 arena `buf`."""
    off = addr - buf.data_ptr()
    return buf[off:off + rows * cols * _F32].view(torch.float32).view(rows, cols)
