"""y = x W^T (+ bias) with the frozen NF4 weight dequantised inside the GEMM
(testt_amd/csrc/gemm_nf4.hip), the fused NF4-dequant GEMM the reference names as its next step
(README.md:190-192), in place of unpack_concat + torch.matmul (solution/nf4.py:108-127).

    nf4_linear(x, weights, bias=None)   x fp16 [M, K]; weights: 1-4 Params4bit-like parts
                                        stacked by rows (q|k|v, gate|up), each a multiple of
                                        128 rows, blocksize 64, nested 256; -> fp16 [M, N]
    gemm_tn(x, w16, bias=None)          the same GEMM on an fp16 W [N, K]

The weight values are the unpack kernel's bit for bit (same arithmetic), so nf4_linear equals
gemm_tn(x, unpack_concat(weights)) exactly."""

import ctypes

import torch

from . import _ext
from . import nf4 as _nf4

MAX_PARTS = 4


def supported(x, weights, bias=None):
    if not (x.is_cuda and x.dtype == torch.float16 and x.dim() == 2):
        return False
    if not 1 <= len(weights) <= MAX_PARTS:
        return False
    K = x.shape[1]
    for w in weights:
        if not _nf4.supports_fast_unpack(w):
            return False
        st = w.quant_state
        rows, cols = _nf4.weight_shape(w)
        if cols != K or rows % 128 or st.blocksize != 64 or st.state2.blocksize != 256:
            return False
        if _nf4._plan(w, x.device) is None:
            return False
    if bias is not None and (bias.dtype != torch.float16 or not bias.is_cuda):
        return False
    return K % 64 == 0 and x.stride(1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0


# Where the fused kernels measured ahead of unpack + hipBLASLt on MI355X (bench.py --nf4-gemm,
# Qwen2.5-1.5B's projections at 16 to 2048 rows): where their grid fills between half and one
# wave of the compute units and the contraction is short.  With fewer tiles a workgroup walks
# its whole contraction alone (q|k|v forward at 16 rows: 21.6 against 14.1 us); with a second
# wave of tiles, or a long contraction (down's forward over 8960 columns, gate|up's input
# gradient over 17920 rows), this build's MFMA core is behind hipBLASLt's.  Inside the window:
# gate|up forward at 16 / 64 rows 23.3 / 23.8 against 57.2 / 38.1 us; q|k|v and o forward at
# 2048 rows 27.1 / 25.3 against 28.0 / 25.6 us; q|k|v and o input gradient at 1024 rows
# 30.4 / 19.9 against 32.7 / 25.3 us; down's input gradient at 16 / 64 rows 19.2 / 19.6
# against 24.8 / 26.6 us.
FUSED_MAX_CONTRACTION = 2048
FWD_TILE = (128, 128)    # rows of x, rows of W per workgroup of soupk_gemm_tn_nf4
GRAD_TILE = (128, 64)    # rows of dy, columns of W per workgroup of soupk_gemm_nn_nf4


def fused_fits(rows, out_cols, contraction, tile, cus):
    """The fused kernels' window: a grid of half to one wave of the `cus` compute units and a
    contraction of at most FUSED_MAX_CONTRACTION."""
    tiles = -(-rows // tile[0]) * -(-out_cols // tile[1])
    return contraction <= FUSED_MAX_CONTRACTION and cus // 2 <= tiles <= cus


def _cu_count(device):
    cached = _cu_count.cache.get(device)
    if cached is None:
        cached = _cu_count.cache[device] = torch.cuda.get_device_properties(device)\
            .multi_processor_count
    return cached


_cu_count.cache = {}


def prefer_fused(x, weights):
    """True where the fused NF4 forward y = x W^T is the faster path (fused_fits)."""
    M, K = x.shape
    N = sum(_nf4.weight_shape(w)[0] for w in weights)
    return fused_fits(M, N, K, FWD_TILE, _cu_count(x.device))


def prefer_fused_grad_input(dy, weights):
    """True where the fused NF4 input gradient dx = dy W is the faster path (fused_fits: dx has
    W's columns, the contraction runs over W's rows)."""
    M, N = dy.shape
    K = _nf4.weight_shape(weights[0])[1]
    return fused_fits(M, K, N, GRAD_TILE, _cu_count(dy.device))


def gemm_tn(x, w16, bias=None):
    _ext.require(w16, "w16", dtype=torch.float16, ndim=2, device=x.device)
    M, K = x.shape
    N = w16.shape[0]
    y = torch.empty((M, N), dtype=torch.float16, device=x.device)
    if bias is not None:
        _ext.require(bias, "bias", dtype=torch.float16, ndim=1, device=x.device)
    _ext.call("soupk_gemm_tn", x.data_ptr(), x.stride(0), w16.data_ptr(), _ext.ptr(bias),
              y.data_ptr(), M, N, K, _ext.stream_of(x))
    return y


def _nf4_args(weights, device):
    plans = [_nf4._plan(w, device) for w in weights]
    rows = [_nf4.weight_shape(w)[0] for w in weights]
    n = len(weights)
    arrays = [(ctypes.c_void_p * n)(*[p[0][i] for p in plans]) for i in range(6)]
    part_rows = (ctypes.c_int32 * n)(*rows)
    return plans, rows, arrays, part_rows


def grad_input_supported(dy, weights):
    """nf4_grad_input takes these: fp16 dy [M, N] with unit column stride and 16-byte aligned
    rows, 1-4 NF4 parts (blocksize 64, nested 256) of one column count, each a multiple of 128
    rows, W's columns a multiple of 128."""
    if not (dy.is_cuda and dy.dtype == torch.float16 and dy.dim() == 2):
        return False
    if not 1 <= len(weights) <= MAX_PARTS:
        return False
    cols = None
    total = 0
    for w in weights:
        if not _nf4.supports_fast_unpack(w):
            return False
        st = w.quant_state
        r, c = _nf4.weight_shape(w)
        if r % 128 or st.blocksize != 64 or st.state2.blocksize != 256 or \
                (cols is not None and c != cols):
            return False
        if _nf4._plan(w, dy.device) is None:
            return False
        cols, total = c, total + r
    return (cols % 128 == 0 and dy.shape[1] == total and dy.stride(1) == 1 and
            dy.stride(0) % 8 == 0 and dy.data_ptr() % 16 == 0)


def nf4_grad_input(dy, weights):
    """dx = dy @ W (fp16 [M, K]) for W the row stack of `weights` ([N, K]), dequantised in the
    GEMM (soupk_gemm_nn_nf4): the input gradient of nf4_linear without an fp16 W in memory."""
    M, N = dy.shape
    plans, rows, arrays, part_rows = _nf4_args(weights, dy.device)
    if sum(rows) != N:
        raise ValueError(f"dy has {N} columns, the weights {sum(rows)} rows")
    K = _nf4.weight_shape(weights[0])[1]
    dx = torch.empty((M, K), dtype=torch.float16, device=dy.device)
    _ext.call("soupk_gemm_nn_nf4", dy.data_ptr(), dy.stride(0), len(weights),
              *[ctypes.addressof(a) for a in arrays], ctypes.addressof(part_rows),
              plans[0][2], plans[0][3], dx.data_ptr(), M, K, N, _ext.stream_of(dy))
    return dx


def nf4_linear(x, weights, bias=None):
    """x @ W^T (+ bias) for W the row stack of `weights`, dequantised in the GEMM."""
    M, K = x.shape
    plans = [_nf4._plan(w, x.device) for w in weights]
    rows = [_nf4.weight_shape(w)[0] for w in weights]
    N = sum(rows)
    if bias is not None:
        _ext.require(bias, "bias", dtype=torch.float16, ndim=1, device=x.device)
        if bias.numel() != N:
            raise ValueError(f"bias has {bias.numel()} entries, the weights {N} rows")
    n = len(weights)
    arrays = [(ctypes.c_void_p * n)(*[p[0][i] for p in plans]) for i in range(6)]
    part_rows = (ctypes.c_int32 * n)(*rows)
    y = torch.empty((M, N), dtype=torch.float16, device=x.device)
    _ext.call("soupk_gemm_tn_nf4", x.data_ptr(), x.stride(0), n,
              *[ctypes.addressof(a) for a in arrays], ctypes.addressof(part_rows),
              plans[0][2], plans[0][3], _ext.ptr(bias), y.data_ptr(), M, N, K,
              _ext.stream_of(x))
    return y
