"""Row-major fp16 GEMMs of the training step on hipBLASLt through soupk_gemm_lt.

The dense GEMMs stay on hipBLASLt, as the reference keeps them on the vendor BLAS through
torch.matmul (solution/nf4.py:108-127, solution/mlp.py:80-113).  torch's path builds the
hipBLASLt descriptors and queries the algorithm on every call, about 19 us of host time per
GEMM on the MI355X box, which made the eager layer host-bound at the ragged batch (issue 602 us
against 455 us of GPU time).  soupk_gemm_lt keeps one plan per problem and runs it with one
hipblasLtMatmul.  Its algorithm is the one torch.matmul runs: the tuned table's solution
(gemm_tuning.enable() hands the table over once TunableOp has accepted it for this system) or,
for problems the table does not list, hipBLASLt's first heuristic choice -- so the result is
torch.matmul's, bit for bit, where the same solution runs.

    matmul(a, b, bias=None, out=None, accumulate=False)
        a [M, K] @ b [K, N] (+ bias [N]) -> [M, N] fp16, or into `out` (+= with accumulate);
        a with unit column stride, b either row-major or the transpose of a row-major [N, K]
    linear(x, w, bias=None)                  x @ w^T (+ bias)
    bmm_f32(a3, b3)                          [P, M, K] @ [P, K, N] -> fp32 [P, M, N]

Operands outside these layouts go to torch (the same library, its own per-call setup).
"""

import csv
import threading

import torch

from . import _ext

WORKSPACE_BYTES = 64 << 20
USE_GEMM_LT = True

_lock = threading.Lock()
_table = {}        # ("tn" | "nn", m, n, k, lda, ldb, ldd, bias) -> hipBLASLt solution index


def load_table(path):
    """The tuned solutions of a TunableOp table (its hipBLASLt rows; 'Default' rows keep the
    heuristic).  Call only for a table TunableOp accepted for this system: the indices name
    solutions of the hipBLASLt build its validators list."""
    table = {}
    with open(path) as f:
        for row in csv.reader(f):
            if len(row) < 3 or row[0] == "Validator":
                continue
            op, sig, sol = row[0], row[1], row[2]
            if not sol.startswith("Gemm_Hipblaslt_") or "_Half_" not in op:
                continue
            bias = op.startswith("GemmAndBias")
            if not (bias or op.startswith("GemmTunableOp")):
                continue
            parts = sig.split("_")      # tn_m_n_k_ld_lda_ldb_ldc
            if len(parts) != 8 or parts[4] != "ld":
                continue
            key = (parts[0], *(int(x) for x in parts[1:4]), *(int(x) for x in parts[5:8]), bias)
            table[key] = int(sol[len("Gemm_Hipblaslt_"):])
    with _lock:
        _table.clear()
        _table.update(table)
    return len(table)


def clear_table():
    with _lock:
        _table.clear()


def _ws(device):
    """hipBLASLt's workspace for one call, from torch's caching allocator on the current stream
    (about 1 us: a cached block; freed when the caller drops it, and reused only in that
    stream's order, so that no two streams' GEMMs share it)."""
    return torch.empty(WORKSPACE_BYTES, dtype=torch.uint8, device=device)


def _aligned(*ts):
    # 16-byte operands, as every solution may assume: the plan is chosen per problem, not per
    # address
    return all(t.data_ptr() % 16 == 0 for t in ts)


def _fits(t):
    return t.is_cuda and t.dtype == torch.float16 and t.dim() == 2


def matmul(a, b, bias=None, out=None, accumulate=False):
    """a [M, K] @ b [K, N] (+ bias [N]); see the module docstring."""
    M, K = a.shape
    N = b.shape[1]
    if b.shape[0] != K:
        raise ValueError(f"matmul: {tuple(a.shape)} @ {tuple(b.shape)}")
    # b row-major [K, N] (leading dimension b.stride(0)), or b = w^T for w row-major [N, K]
    # (leading dimension b.stride(1)); a leading dimension of a size-1 extent is free
    b_rows = b.stride(1) == 1 and (K == 1 or b.stride(0) >= N)
    b_cols = not b_rows and b.stride(0) == 1 and (N == 1 or b.stride(1) >= K)
    ok = (USE_GEMM_LT and _fits(a) and _fits(b) and a.stride(1) == 1 and (b_rows or b_cols)
          and a.device == b.device and K > 0 and (M == 1 or a.stride(0) >= K)
          and (bias is None or (bias.dtype == torch.float16 and bias.is_contiguous()
                                and bias.numel() == N and not accumulate
                                and bias.data_ptr() % 8 == 0)))
    if out is not None:
        ok = (ok and _fits(out) and out.stride(1) == 1 and tuple(out.shape) == (M, N)
              and (M == 1 or out.stride(0) >= N))
    elif accumulate:
        raise ValueError("matmul: accumulate needs `out`")
    if not ok:
        return _torch_matmul(a, b, bias, out, accumulate)
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=a.device)
    if M == 0 or N == 0:
        return out
    # column-major: out^T [N, M] = op(b^T) [N, K] @ a^T [K, M]
    ta = 0 if b_rows else 1
    lda = max(b.stride(0), N) if b_rows else max(b.stride(1), K)
    ldb = max(a.stride(0), K)
    ldd = max(out.stride(0), N)
    if not _aligned(a, b, out) or (lda | ldb | ldd) % 8:
        return _torch_matmul(a, b, bias, out, accumulate)
    key = ("tn" if ta else "nn", N, M, K, lda, ldb, ldd, bias is not None)
    st = _ext.stream_of(a)
    ws = _ws(a.device)
    _ext.call("soupk_gemm_lt", ta, 0, N, M, K, b.data_ptr(), lda, 0, a.data_ptr(), ldb, 0,
              out.data_ptr(), ldd, 0, 0, 1, 1 if accumulate else 0, _ext.ptr(bias),
              _table.get(key, -1), ws.data_ptr(), WORKSPACE_BYTES, st)
    return out


def linear(x, w, bias=None):
    """x [M, K] @ w [N, K]^T (+ bias [N])."""
    return matmul(x, w.t(), bias)


def bmm_f32(a3, b3):
    """Batched a3 [P, M, K] @ b3 [P, K, N] -> fp32 [P, M, N]: a3 with unit column stride, b3
    with unit column stride or unit row stride (slices of a transposed matrix), each with
    strides of its own (slices of one matrix, as matmul_split_k makes)."""
    P, M, K = a3.shape
    N = b3.shape[2]
    b_rows = b3.stride(2) == 1 and b3.stride(1) >= N     # each slice row-major [K, N]
    b_cols = not b_rows and b3.stride(1) == 1 and b3.stride(2) >= K   # transposed [N, K]
    ok = (USE_GEMM_LT and a3.is_cuda and a3.dtype == torch.float16 and
          b3.dtype == torch.float16 and a3.dim() == 3 and b3.dim() == 3 and
          b3.shape[:2] == (P, K) and a3.stride(2) == 1 and (b_rows or b_cols) and K > 0 and
          a3.stride(1) >= K and P > 0)
    ld_b = b3.stride(1) if b_rows else b3.stride(2)
    if not ok or not _aligned(a3, b3) or (a3.stride(0) | a3.stride(1) | b3.stride(0) |
                                          ld_b) % 8:
        return torch.ops.aten.bmm.dtype(a3, b3, torch.float32)
    out = torch.empty((P, M, N), dtype=torch.float32, device=a3.device)
    if M == 0 or N == 0:
        return out
    st = _ext.stream_of(a3)
    ws = _ws(a3.device)
    # column-major per problem: out_p^T [N, M] = op(b3_p^T) [N, K] @ a3_p^T [K, M]
    _ext.call("soupk_gemm_lt", 0 if b_rows else 1, 0, N, M, K, b3.data_ptr(), ld_b,
              b3.stride(0), a3.data_ptr(), a3.stride(1), a3.stride(0), out.data_ptr(), N, M * N,
              1, P, 0, None, -1, ws.data_ptr(), WORKSPACE_BYTES, st)
    return out


def split_k(a, b, parts):
    """fp16 a [M, K] @ b [K, N] as `parts` batched GEMMs over equal slices of K with fp32
    partials, summed in slice order and rounded once (soupk_sum_partials) -> fp16 [M, N]; b
    row-major or the transpose of a row-major [N, K].  None where the operands do not fit
    (mlp.matmul_split_k then builds the slices as views).  The same two launches as the views
    through bmm_f32, with the slices' strides computed here rather than by two as_strided
    views and their checks (host time: the layer issues two of these per step)."""
    M, K = a.shape
    N = b.shape[1]
    if not (USE_GEMM_LT and parts > 0 and K % parts == 0 and M > 0 and N > 0 and _fits(a)
            and _fits(b) and a.device == b.device and a.stride(1) == 1 and a.stride(0) >= K):
        return None
    c = K // parts
    if b.stride(1) == 1 and b.stride(0) >= N:
        ta, ld_b = 0, b.stride(0)          # slice p: rows p*c .. of b
    elif b.stride(0) == 1 and b.stride(1) >= K:
        ta, ld_b = 1, b.stride(1)          # slice p: columns p*c .. of b^T
    else:
        return None
    if not _aligned(a, b) or (a.stride(0) | ld_b | c) % 8:
        return None
    st = _ext.stream_of(a)
    ws = _ws(a.device)
    part = torch.empty((parts, M, N), dtype=torch.float32, device=a.device)
    out = torch.empty((M, N), dtype=torch.float16, device=a.device)
    _ext.call("soupk_gemm_lt", ta, 0, N, M, c, b.data_ptr(), ld_b, c * b.stride(0), a.data_ptr(),
              a.stride(0), c, part.data_ptr(), N, M * N, 1, parts, 0, None, -1, ws.data_ptr(),
              WORKSPACE_BYTES, st)
    _ext.call("soupk_sum_partials", part.data_ptr(), parts, M * N, M * N, out.data_ptr(), st)
    return out


def _torch_matmul(a, b, bias, out, accumulate):
    if accumulate:
        return out.addmm_(a, b)
    if out is not None:
        torch.mm(a, b, out=out)
        if bias is not None:
            out += bias
        return out
    return torch.nn.functional.linear(a, b.t(), bias) if bias is not None else torch.mm(a, b)
