"""The LoRA branch of the q and v projections for rank 16 on gfx950 (testt_amd/csrc/lora.hip):
peft's lora_B(lora_A(x)) * scaling under fp16 autocast (solution/model.py:195-206, dropout 0),
in one launch forward and one backward, in place of the separate fp16 GEMMs, casts and
scalings.  `layer.QKVLora` uses it when `supported` holds and keeps its GEMM path otherwise.

    stage(a_q, a_v, b_q, b_v)                         -> the fp16 casts of the parameters
    lora_fwd(y16, a_q, a_v, b_q, b_v, scaling, st)    -> t [M, 32], lq [M, NQ], lv [M, NV] fp16
    lora_bwd_rows(g_q, g_v, a_q, a_v, b_q, b_v, s, st) -> dt [M, 32], dy [M, H] fp16
    lora_bwd_params(y16, t, dt, g_q, g_v, s)          -> dA_q, dA_v [16, H], dB_q, dB_v fp32

with t = fp16(y A^T), lq = fp16(fp16(t_q B_q^T) * s), gs = fp16(g * s),
dt = fp16(gs_q B_q | gs_v B_v), dy = fp16(dt A), dA = fp32(fp16(dt^T y)),
dB_x = fp32(fp16(gs_x^T t_x)): the rounding steps of the fp16 GEMMs they replace (fp32 sums in
another order).  gs is never stored: both backward kernels form it from g as they read it.
A and B enter the products as their fp16 casts (autocast's), which `stage`
makes in one launch, in the layouts the kernels read; the forward's staged buffer serves its
backward too (the parameters do not change in between).  Without `st` the functions stage
the parameters themselves."""

import torch

from . import _ext

RANK = 16


def params_supported(a_q, a_v, b_q, b_v, device):
    """Rank 16 fp32 contiguous parameters on `device`, H, NQ, NV multiples of 128."""
    for p in (a_q, a_v, b_q, b_v):
        if p.dtype != torch.float32 or p.device != device or not p.is_contiguous() or \
                p.dim() != 2:
            return False
    H = a_q.shape[1]
    return (tuple(a_q.shape) == (RANK, H) and tuple(a_v.shape) == (RANK, H)
            and b_q.shape[1] == RANK and b_v.shape[1] == RANK and H % 128 == 0
            and b_q.shape[0] % 128 == 0 and b_v.shape[0] % 128 == 0)


def supported(y16, a_q, a_v, b_q, b_v):
    """Rank 16, fp16 y and fp32 parameters on one HIP device, H, NQ, NV multiples of 128."""
    if not (y16.is_cuda and y16.dtype == torch.float16 and y16.dim() == 2):
        return False
    return params_supported(a_q, a_v, b_q, b_v, y16.device) and a_q.shape[1] == y16.shape[1]


def _check_params(a_q, a_v, b_q, b_v, H, dev):
    """The four LoRA parameters must be contiguous fp32 tensors on `dev` of shapes (16, H),
    (16, H), (NQ, 16), (NV, 16) with H, NQ and NV multiples of 128 (the kernels' tiling)."""
    for p, name in ((a_q, "a_q"), (a_v, "a_v"), (b_q, "b_q"), (b_v, "b_v")):
        _ext.require(p, name, dtype=torch.float32, ndim=2, device=dev)
    if tuple(a_q.shape) != (RANK, H) or tuple(a_v.shape) != (RANK, H):
        raise ValueError(f"a_q {tuple(a_q.shape)} and a_v {tuple(a_v.shape)} must be "
                         f"({RANK}, {H})")
    if b_q.shape[1] != RANK or b_v.shape[1] != RANK:
        raise ValueError(f"b_q {tuple(b_q.shape)} and b_v {tuple(b_v.shape)} must have "
                         f"{RANK} columns")
    if H % 128 or b_q.shape[0] % 128 or b_v.shape[0] % 128:
        raise ValueError(f"H ({H}), NQ ({b_q.shape[0]}) and NV ({b_v.shape[0]}) must be "
                         "multiples of 128")
    return b_q.shape[0], b_v.shape[0]


def staged_elems(H, NQ, NV):
    """Halves of the staged parameter buffer: [A_q; A_v] and its transpose, [B_q; B_v], and
    B_q^T, B_v^T."""
    return 4 * RANK * H + 2 * RANK * (NQ + NV)


def stage(a_q, a_v, b_q, b_v):
    """fp16 [staged_elems] device tensor: the parameters' fp16 casts in the kernels' layouts."""
    H = a_q.shape[-1] if a_q.dim() == 2 else 0
    dev = a_q.device
    NQ, NV = _check_params(a_q, a_v, b_q, b_v, H, dev)
    st = torch.empty(staged_elems(H, NQ, NV), dtype=torch.float16, device=dev)
    _ext.call("soupk_lora_stage", _ext.ptr(a_q), _ext.ptr(a_v), _ext.ptr(b_q), _ext.ptr(b_v),
              _ext.ptr(st), st.numel(), H, NQ, NV, RANK, _ext.stream_of(st))
    return st


def _staged(st, a_q, a_v, b_q, b_v, H, NQ, NV, dev):
    if st is None:
        return stage(a_q, a_v, b_q, b_v)
    _ext.require(st, "staged", dtype=torch.float16, ndim=1, device=dev)
    if st.numel() < staged_elems(H, NQ, NV):
        raise ValueError(f"staged holds {st.numel()} values, {staged_elems(H, NQ, NV)} needed")
    return st


def lora_fwd(y16, a_q, a_v, b_q, b_v, scaling, staged=None):
    _ext.require(y16, "y16", dtype=torch.float16, ndim=2)
    M, H = y16.shape
    dev = y16.device
    NQ, NV = _check_params(a_q, a_v, b_q, b_v, H, dev)
    st = _staged(staged, a_q, a_v, b_q, b_v, H, NQ, NV, dev)
    t = torch.empty((M, 2 * RANK), dtype=torch.float16, device=dev)
    lq = torch.empty((M, NQ), dtype=torch.float16, device=dev)
    lv = torch.empty((M, NV), dtype=torch.float16, device=dev)
    _ext.call("soupk_lora_fwd", _ext.ptr(y16), _ext.ptr(st), float(scaling), _ext.ptr(t),
              _ext.ptr(lq), _ext.ptr(lv), M, H, NQ, NV, RANK, _ext.stream_of(y16))
    return t, lq, lv


def lora_rope_fwd(y16, a_q, a_v, b_q, b_v, scaling, qkv, cos, sin, pos_idx, batch, seq,
                  n_heads, n_kv, staged=None):
    """The LoRA forward fused with the RoPE pack of the varlen attention's rows
    (soupk_lora_rope_fwd): t [M, 32] and out [M, (n_heads + 2 n_kv) * 128] fp16 = rotated
    (q + lq) | rotated k | v + lv, where lq, lv are lora_fwd's deltas and qkv the q|k|v GEMM
    output; the values of rope.rope_pack_tokens(qkv, lq, lv, ...) bit for bit, without lq and lv
    in memory.  Returns (t, out, cos32, sin32, pos) (the tables and positions as the attention
    backward takes them)."""
    from . import rope as _rope

    _ext.require(y16, "y16", dtype=torch.float16, ndim=2)
    M, H = y16.shape
    dev = y16.device
    NQ, NV = _check_params(a_q, a_v, b_q, b_v, H, dev)
    D = 128
    if NQ != n_heads * D or NV != n_kv * D:
        raise ValueError(f"B_q / B_v rows ({NQ}, {NV}) != heads x 128 ({n_heads * D}, {n_kv * D})")
    width = NQ + 2 * NV
    _ext.require(qkv, "qkv", dtype=torch.float16, ndim=2, device=dev)
    if tuple(qkv.shape) != (M, width):
        raise ValueError(f"qkv shape {tuple(qkv.shape)} != {(M, width)}")
    pos = _rope.as_index(pos_idx)
    if pos.numel() != M or pos.device != dev:
        raise ValueError(f"pos_idx has {pos.numel()} entries on {pos.device} for {M} rows")
    cos32 = _rope._table(cos, seq, D, "cos", dev)
    sin32 = _rope._table(sin, seq, D, "sin", dev)
    st = _staged(staged, a_q, a_v, b_q, b_v, H, NQ, NV, dev)
    t = torch.empty((M, 2 * RANK), dtype=torch.float16, device=dev)
    out = torch.empty((M, width), dtype=torch.float16, device=dev)
    _ext.call("soupk_lora_rope_fwd", _ext.ptr(y16), _ext.ptr(st), float(scaling), _ext.ptr(qkv),
              _ext.ptr(cos32), _ext.ptr(sin32), _ext.ptr(pos), _ext.ptr(t), _ext.ptr(out), M, H,
              n_heads, n_kv, D, RANK, batch, seq, _ext.stream_of(y16))
    return t, out, cos32, sin32, pos


def _rows(g, n, m, dev):
    """g as an fp16 [m, n] view with unit column stride (zeros for a missing gradient)."""
    if g is None:
        return torch.zeros((m, n), dtype=torch.float16, device=dev)
    if not g.is_cuda or g.device != dev or g.dim() != 2:
        raise ValueError(f"a LoRA output gradient must be a 2-d tensor on {dev}, got "
                         f"{tuple(g.shape)} on {g.device}")
    g = g.to(torch.float16)
    if g.stride(1) != 1 or g.stride(0) % 8 or g.data_ptr() % 16:
        g = g.contiguous()
    return g


def lora_bwd_rows(g_q, g_v, a_q, a_v, b_q, b_v, scaling, staged=None):
    ref = g_q if g_q is not None else g_v
    if ref is None:
        raise ValueError("lora_bwd_rows needs at least one of g_q, g_v")
    M, dev = ref.shape[0], ref.device
    NQ, NV = _check_params(a_q, a_v, b_q, b_v, a_q.shape[-1], dev)
    H = a_q.shape[1]
    st = _staged(staged, a_q, a_v, b_q, b_v, H, NQ, NV, dev)
    g_q, g_v = rows_view(g_q, NQ, M, dev), rows_view(g_v, NV, M, dev)
    dt = torch.empty((M, 2 * RANK), dtype=torch.float16, device=dev)
    dy = torch.empty((M, H), dtype=torch.float16, device=dev)
    _ext.call("soupk_lora_bwd_rows", _ext.ptr(g_q), g_q.stride(0), _ext.ptr(g_v), g_v.stride(0),
              _ext.ptr(st), float(scaling), _ext.ptr(dt), _ext.ptr(dy), M, H, NQ, NV, RANK,
              _ext.stream_of(dy))
    return dt, dy


SLICE_ROWS = 128   # rows per partial sum of soupk_lora_bwd_params


def rows_view(g, n, m, dev):
    """g_q / g_v as the backward kernels read them: fp16 [m, n] with unit column stride and a
    16-byte aligned row stride (a view of the attention backward's q|k|v gradient stays one;
    a missing gradient becomes zeros)."""
    g = _rows(g, n, m, dev)
    if tuple(g.shape) != (m, n):
        raise ValueError(f"a LoRA output gradient has shape {tuple(g.shape)}, expected {(m, n)}")
    return g


def lora_bwd_params(y16, t, dt, g_q, g_v, scaling):
    """dA_q, dA_v, dB_q, dB_v from the forward's y16 and t, the row backward's dt and the
    gradients g_q, g_v of lq, lv (gs = fp16(g * scaling) formed as they are read)."""
    M, H = y16.shape
    dev = y16.device
    for x, name, cols in ((y16, "y16", H), (t, "t", 2 * RANK), (dt, "dt", 2 * RANK)):
        _ext.require(x, name, dtype=torch.float16, ndim=2, device=dev)
        if tuple(x.shape) != (M, cols):
            raise ValueError(f"{name} has shape {tuple(x.shape)}, expected {(M, cols)}")
    if g_q is None or g_v is None:
        raise ValueError("lora_bwd_params needs g_q and g_v (pass zeros for a missing one)")
    NQ, NV = g_q.shape[1], g_v.shape[1]
    g_q, g_v = rows_view(g_q, NQ, M, dev), rows_view(g_v, NV, M, dev)
    slices = (M + SLICE_ROWS - 1) // SLICE_ROWS
    n_ws = slices * (2 * RANK * H + RANK * (NQ + NV))
    ws = torch.empty(max(n_ws, 4), dtype=torch.float32, device=dev)
    d_aq = torch.empty((RANK, H), dtype=torch.float32, device=dev)
    d_av = torch.empty((RANK, H), dtype=torch.float32, device=dev)
    d_bq = torch.empty((NQ, RANK), dtype=torch.float32, device=dev)
    d_bv = torch.empty((NV, RANK), dtype=torch.float32, device=dev)
    _ext.call("soupk_lora_bwd_params", _ext.ptr(y16), _ext.ptr(t), _ext.ptr(dt), _ext.ptr(g_q),
              g_q.stride(0), _ext.ptr(g_v), g_v.stride(0), float(scaling), _ext.ptr(ws),
              ws.numel(), _ext.ptr(d_aq), _ext.ptr(d_av), _ext.ptr(d_bq), _ext.ptr(d_bv), M, H,
              NQ, NV, RANK, _ext.stream_of(y16))
    return d_aq, d_av, d_bq, d_bv
