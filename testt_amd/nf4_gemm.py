"""y = x W^T (+ bias) with the frozen NF4 weight dequantised inside the GEMM
(testt_amd/csrc/gemm_nf4.hip), the fused NF4-dequant GEMM the reference names as its next step
(README.md:190-192), in place of unpack_concat + torch.matmul (solution/nf4.py:108-127).

    nf4_linear(x, weights, bias=None, splits=None)
                                        x fp16 [M, K]; weights: 1-4 Params4bit-like parts
                                        stacked by rows (q|k|v, gate|up), each a multiple of
                                        128 rows, blocksize 64, nested 256; -> fp16 [M, N];
                                        splits: cuts of the contraction (default split_count)
    gemm_tn(x, w16, bias=None)          the same GEMM on an fp16 W [N, K]

The weight values are the unpack kernel's bit for bit (same arithmetic), so nf4_linear with
one split equals gemm_tn(x, unpack_concat(weights)) exactly; with more, the same products are
summed in another order (fp32 partials per split, added in split order)."""

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
# against 24.8 / 26.6 us.  Below half a wave the forward cuts its contraction (split_count),
# which puts it ahead up to an eighth of a wave of tiles (a quarter for down's 8960 columns):
# q|k|v / o / down at 16 rows 7.9 / 7.6 / 13.3 against 14.2 / 13.4 / 38.4 us, q|k|v and o at
# 256 rows 14.8 / 13.6 against 17.9 / 14.2 us, down at 512 rows 36.7 against 53.3 us; at 512
# rows q|k|v and o are 3% behind (19.4 / 17.6 against 18.8 / 17.1 us) and left out.
FUSED_MAX_CONTRACTION = 2048
FWD_TILE = (128, 128)    # rows of x, rows of W per workgroup of soupk_gemm_tn_nf4
GRAD_TILE = (128, 64)    # rows of dy, columns of W per workgroup of soupk_gemm_nn_nf4


def fused_fits(rows, out_cols, contraction, tile, cus, split_tiles=0):
    """The fused kernels' window: a grid of half to one wave of the `cus` compute units and a
    contraction of at most FUSED_MAX_CONTRACTION, or a grid of at most `split_tiles` tiles,
    whose contraction the split kernels cut (split_count)."""
    tiles = -(-rows // tile[0]) * -(-out_cols // tile[1])
    if contraction <= FUSED_MAX_CONTRACTION and cus // 2 <= tiles <= cus:
        return True
    return tiles <= split_tiles


def forward_split_tiles(contraction, cus):
    """Grids up to which the split forward measured ahead of unpack + hipBLASLt: an eighth of a
    wave of tiles (q|k|v and o at 256 rows), a quarter for contractions past
    FUSED_MAX_CONTRACTION (down at 512 rows).  Beyond it the partials' traffic, which grows with
    the rows, puts it behind (q|k|v / o at 512 rows 3% behind)."""
    return cus // 8 if contraction <= FUSED_MAX_CONTRACTION else cus // 4


def grad_split_tiles(contraction, cus):
    """Grids up to which the split input gradient measured ahead of unpack + hipBLASLt: a
    quarter of a wave of tiles (q|k|v and o at 256 rows), one wave for contractions past
    FUSED_MAX_CONTRACTION (gate|up at 1024 rows, 192 tiles over 17920 rows: 150.7 against
    220.0 us).  At 512 rows q|k|v is 3% behind and o level."""
    return cus // 4 if contraction <= FUSED_MAX_CONTRACTION else cus


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
    cus = _cu_count(x.device)
    return fused_fits(M, N, K, FWD_TILE, cus, forward_split_tiles(K, cus))


def prefer_fused_grad_input(dy, weights):
    """True where the fused NF4 input gradient dx = dy W is the faster path (fused_fits: dx has
    W's columns, the contraction runs over W's rows)."""
    M, N = dy.shape
    K = _nf4.weight_shape(weights[0])[1]
    cus = _cu_count(dy.device)
    return fused_fits(M, K, N, GRAD_TILE, cus, grad_split_tiles(N, cus))


def prefers_fused_all(rows, groups, device, window=True):
    """True when every group of `groups` (each a row stack of NF4 weights, as one product
    reads it) takes the fused kernels at `rows` rows in both directions -- the window of
    prefer_fused and of prefer_fused_grad_input -- and has the layout they read (with
    window=False: the layout alone).  A decoder layer with this token count then runs on its
    NF4 weights without unpacking them."""
    cus = _cu_count(device)
    for weights in groups:
        if not 1 <= len(weights) <= MAX_PARTS:
            return False
        cols, n = None, 0
        for w in weights:
            if not _nf4.supports_fast_unpack(w):
                return False
            st = w.quant_state
            r, c = _nf4.weight_shape(w)
            if r % 128 or c % 128 or st.blocksize != 64 or st.state2.blocksize != 256 or \
                    (cols is not None and c != cols) or _nf4._plan(w, device) is None:
                return False
            cols, n = c, n + r
        if window and not (
                fused_fits(rows, n, cols, FWD_TILE, cus, forward_split_tiles(cols, cus)) and
                fused_fits(rows, cols, n, GRAD_TILE, cus, grad_split_tiles(n, cus))):
            return False
    return True


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


def nf4_grad_input(dy, weights, splits=None):
    """dx = dy @ W (fp16 [M, K]) for W the row stack of `weights` ([N, K]), dequantised in the
    GEMM (soupk_gemm_nn_nf4): the input gradient of nf4_linear without an fp16 W in memory.
    `splits` cuts the contraction over W's rows (soupk_gemm_nn_nf4_split; default: split_count
    for this device and the 128 x 64 tiles)."""
    M, N = dy.shape
    plans, rows, arrays, part_rows = _nf4_args(weights, dy.device)
    if sum(rows) != N:
        raise ValueError(f"dy has {N} columns, the weights {sum(rows)} rows")
    K = _nf4.weight_shape(weights[0])[1]
    dx = torch.empty((M, K), dtype=torch.float16, device=dy.device)
    if splits is None:
        splits = split_count(M, K, N, _cu_count(dy.device), GRAD_TILE) if M > 0 else 1
    args = (dy.data_ptr(), dy.stride(0), len(weights), *[ctypes.addressof(a) for a in arrays],
            ctypes.addressof(part_rows), plans[0][2], plans[0][3], dx.data_ptr(), M, K, N)
    if splits > 1:
        ws = torch.empty(_split_used(N // 64, splits)[1] * M * K, dtype=torch.float32,
                         device=dy.device)
        _ext.call("soupk_gemm_nn_nf4_split", *args, splits, ws.data_ptr(), ws.numel(),
                  _ext.stream_of(dy))
        return dx
    _ext.call("soupk_gemm_nn_nf4", *args, _ext.stream_of(dy))
    return dx


MAX_SPLITS = 32   # the limit of soupk_gemm_tn_nf4_split and soupk_gemm_nn_nf4_split
# Cost model of the split kernels (microseconds), fitted to split-count sweeps on MI355X at
# Qwen2.5-1.5B's projections, 16-1024 rows (forward: q|k|v, o, down; input gradient: q|k|v, o,
# gate|up): a 64-wide contraction step of a workgroup alone on its CU (latency-bound at these
# grids), the slowdown of each step when two workgroups share a CU, each MB of fp32 partials
# written and summed, and the summing launch.  Its pick is the measured best, or within 4% of
# it, in each of the 27 sweep cases that measured it.
SPLIT_STEP_US = 0.72
SPLIT_SHARED_CU = 1.5
SPLIT_PARTIAL_US_PER_MB = 0.2
SPLIT_SUM_US = 2.5


def _split_used(kt, splits):
    per = -(-kt // splits)
    return per, -(-kt // per)


_split_memo = {}


def split_count(rows, out_cols, contraction, cus, tile=FWD_TILE):
    """split_count for these arguments and the cost model's present constants, remembered
    (the decoder layer asks for eight counts per step)."""
    key = (rows, out_cols, contraction, cus, tuple(tile), SPLIT_STEP_US, SPLIT_SHARED_CU,
           SPLIT_PARTIAL_US_PER_MB, SPLIT_SUM_US, FUSED_MAX_CONTRACTION, MAX_SPLITS)
    hit = _split_memo.get(key)
    if hit is None:
        if len(_split_memo) > 4096:
            _split_memo.clear()
        hit = _split_memo[key] = _split_count(rows, out_cols, contraction, cus, tile)
    return hit


def _split_count(rows, out_cols, contraction, cus, tile=FWD_TILE):
    """Contraction splits of a fused kernel's grid of `tile` tiles (the forward's 128 x 128, the
    input gradient's 128 x 64): 1 when the tiles alone fill half a wave of the `cus` compute
    units and the contraction is at most FUSED_MAX_CONTRACTION, else the count (each split at
    least two 64-wide contraction steps) that minimises the cost model above: the steps of one
    workgroup, slowed where tiles x splits puts two on a CU (and repeated per further round of
    two per CU), plus the partials' traffic and the summing launch."""
    tiles = -(-rows // tile[0]) * -(-out_cols // tile[1])
    kt = contraction // 64
    if kt < 2 or (2 * tiles >= cus and contraction <= FUSED_MAX_CONTRACTION):
        return 1

    def cost(s):
        per, used = _split_used(kt, s)
        w = tiles * used
        t = SPLIT_STEP_US * per * (1 if w <= cus else SPLIT_SHARED_CU * -(-w // (2 * cus)))
        if used > 1:
            t += SPLIT_SUM_US + SPLIT_PARTIAL_US_PER_MB * used * rows * out_cols * 8e-6
        return t

    return min(range(1, min(kt // 2, MAX_SPLITS) + 1), key=cost)


def nf4_linear(x, weights, bias=None, splits=None):
    """x @ W^T (+ bias) for W the row stack of `weights`, dequantised in the GEMM; `splits`
    cuts the contraction (default: split_count for this device)."""
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
    if splits is None:
        splits = split_count(M, N, K, _cu_count(x.device)) if M > 0 else 1
    if splits > 1:
        ws = torch.empty(_split_used(K // 64, splits)[1] * M * N, dtype=torch.float32,
                         device=x.device)
        _ext.call("soupk_gemm_tn_nf4_split", x.data_ptr(), x.stride(0), n,
                  *[ctypes.addressof(a) for a in arrays], ctypes.addressof(part_rows),
                  plans[0][2], plans[0][3], _ext.ptr(bias), y.data_ptr(), M, N, K, splits,
                  ws.data_ptr(), ws.numel(), _ext.stream_of(x))
        return y
    _ext.call("soupk_gemm_tn_nf4", x.data_ptr(), x.stride(0), n,
              *[ctypes.addressof(a) for a in arrays], ctypes.addressof(part_rows),
              plans[0][2], plans[0][3], _ext.ptr(bias), y.data_ptr(), M, N, K,
              _ext.stream_of(x))
    return y
