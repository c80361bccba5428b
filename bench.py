"""Benchmark of the MI355X kernel set of the QLoRA step (BASELINE.json metric), one GPU.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--cpu-seconds S]

A step is one pass of the hot path over one batch of synthetic input: every kernel of the
solution/ set, forward and backward, once, at the 2048-token shape of Qwen2.5-1.5B
(config 1, the CPU-runnable RMSNorm case, is the same RMSNorm
shape).  Inputs are resident in HBM before the timed region; 20 warm-up steps, 200 timed.
Each launch carries a pair of HIP events on the stream it runs on (torch's current stream),
recorded by the kernel dispatch itself (soupk_time_next_launch -> hipExtLaunchKernelGGL), so
they time the kernel exactly as rocprofv3's kernel trace does; launches go straight through
the C ABI with preallocated buffers.  Each kernel rotates through enough input sets that one
rotation's inputs exceed twice the 256 MB Infinity Cache (rotation_sets), so no launch finds its
inputs there: they come from HBM, as the roofline assumes.

Prints ONE JSON line: value = the set's aggregate compulsory HBM bytes / summed kernel time
(GB/s), per-kernel us / GB/s / fraction of the 8 TB/s peak, the roofline of the dominant kernel,
and the CPU baseline (the reference's eager PyTorch path on the host cores, oracle/baseline.py).
"""

import argparse
import ctypes
import json
import math
import os
import re
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import testt_amd  # noqa: E402
from testt_amd import _ext, workloads  # noqa: E402

PEAK_HBM_GBPS = 8000.0
PEAK_MFMA_F16_TFLOPS = 2500.0   # MI355X dense fp16 MFMA
METRIC = json.load(open(os.path.join(ROOT, "BASELINE.json")))["metric"]
# HBM bytes per launch measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (written by
# `bench.py --summarize-pmc`); the roofline's "traffic" field is read from this table.
TRAFFIC_TABLE = os.path.join(ROOT, "profiles", "hbm_traffic_step2048_pmc.md")


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Case:
    """One kernel at its BASELINE shape: algorithmic bytes and per-input-set launch args."""

    def __init__(self, name, kernel, entry, nbytes, sets, cpu=None, lib=None):
        self.name, self.kernel, self.entry, self.nbytes = name, kernel, entry, nbytes
        self.sets = sets            # list of (tensors kept alive, ctypes args without stream)
        self.cpu = cpu              # cpu(ob) -> callable running the CPU eager path once, given
                                    # the oracle.baseline module (imported by the CPU leg only)
        self.fn = getattr(lib if lib is not None else _ext.lib(), entry)
        self.times = []

    def launch(self, i, stream):
        status = self.fn(*self.sets[i % len(self.sets)][1], stream)
        if status:
            raise _ext.SoupkError(f"{self.entry} failed with status {status}")


def p(t):
    return t.data_ptr() if t is not None else None


# Input bytes one rotation of a kernel's input sets spans: twice the 256 MB Infinity Cache
# (MALL).  With a fixed three sets, the RoPE forward (whose loads allocate in the MALL) found
# its 23 MB of inputs there and ran 5.6 us against 6.45 us from HBM.
ROTATION_BYTES = 512 << 20


def rotation_sets(in_bytes, n_sets=None):
    """Number of input sets a kernel with `in_bytes` of input per launch rotates through:
    `n_sets` if given (quick probes), else enough to span ROTATION_BYTES, at least 3."""
    if n_sets is not None:
        return n_sets
    return max(3, -(-ROTATION_BYTES // in_bytes))


def build_cases(dev, n_sets=None, lib=None):
    """The eight kernels at the step shape; `lib` selects the soupk library (default: the
    package's)."""
    cases = []
    H, I, NH, NKV, D, B, T = (workloads.HIDDEN, workloads.INTER, workloads.N_HEADS,
                              workloads.N_KV, workloads.HEAD_DIM, workloads.BATCH, workloads.SEQ)
    M = B * T

    # nf4_unpack: gate|up [17920, 1536]
    sets = []
    for i in range(rotation_sets(2 * I * H // 2 + 2 * I * H // 64, n_sets)):
        w = workloads.nf4_weight(2 * I, H, seed=1 + i, device=dev)
        st = w.quant_state
        out = torch.empty((2 * I, H), dtype=torch.float16, device=dev)
        sets.append(((w, out), (p(w.data), p(st.absmax), p(st.state2.code), p(st.state2.absmax),
                                p(st.offset), p(st.code), p(out), w.data.numel(), 64, 256)))
    st = sets[0][0][0].quant_state
    nbytes = (sets[0][0][0].data.numel() + st.absmax.numel() + 4 * st.state2.absmax.numel()
              + 4 * 256 + 4 * 16 + 4 + 2 * 2 * sets[0][0][0].data.numel())

    def nf4_cpu(ob):
        w_cpu = workloads.nf4_weight(2 * I, H, seed=1)
        return lambda: ob.nf4_unpack(w_cpu)

    cases.append(Case("nf4_unpack", "nf4_unpack_vec_kernel", "soupk_nf4_unpack", nbytes, sets,
                      cpu=nf4_cpu, lib=lib))

    # add + RMSNorm forward (delta, pad output) and backward at [2048, 1536]
    fsets, bsets = [], []
    n_f, n_b = rotation_sets(6 * M * H, n_sets), rotation_sets(14 * M * H, n_sets)
    for i in range(max(n_f, n_b)):
        x, delta, w, pad_idx, padded = workloads.rmsnorm_inputs(M, H, M, seed=2 + 10 * i,
                                                                device=dev)
        s = torch.empty_like(x)
        y = torch.empty((M, H), dtype=torch.float16, device=dev)
        ypad = torch.empty((M, H), dtype=torch.float32, device=dev)
        rstd = torch.empty(M, dtype=torch.float32, device=dev)
        if i < n_f:
            fsets.append(((x, delta, w, pad_idx, s, y, ypad, rstd),
                          (p(x), p(delta), p(w), p(s), p(y), p(ypad), p(pad_idx), None, p(rstd),
                           M, M, H, 1e-6)))
        if i >= n_b:
            continue
        dy, dypad, ds = workloads.rmsnorm_grads(M, H, M, seed=3 + 10 * i, device=dev)
        s_b = x + delta.float()
        rstd_b = torch.rsqrt(s_b.pow(2).mean(-1) + 1e-6)
        dx = torch.empty_like(x)
        dd = torch.empty((M, H), dtype=torch.float16, device=dev)
        bsets.append(((s_b, rstd_b, w, dy, dypad, pad_idx, ds, dx, dd),
                      (p(s_b), p(rstd_b), p(w), p(dy), p(dypad), p(pad_idx), p(ds), p(dx), p(dd),
                       M, M, H)))
    row_elems = M * H

    def rms_cpu(ob, backward):
        xc, dc, wc, pc, _ = workloads.rmsnorm_inputs(M, H, M, seed=2)
        gyc, gpc, gsc = workloads.rmsnorm_grads(M, H, M, seed=3)
        if backward:
            return lambda: ob.rmsnorm_bwd(xc, dc, wc, 1e-6, pc, gyc, gpc, gsc)
        return lambda: ob.rmsnorm_fwd(xc, dc, wc, 1e-6, pc, M)

    cases.append(Case("rmsnorm_fwd", "rmsnorm_fwd_kernel", "soupk_rmsnorm_fwd",
                      16 * row_elems + 4 * H + 4 * M + 8 * M, fsets,
                      cpu=lambda ob: rms_cpu(ob, False), lib=lib))
    cases.append(Case("rmsnorm_bwd", "rmsnorm_bwd_kernel", "soupk_rmsnorm_bwd",
                      20 * row_elems + 4 * H + 4 * M + 8 * M, bsets,
                      cpu=lambda ob: rms_cpu(ob, True), lib=lib))

    # LoRA-add + RoPE + QKV pack forward / backward at M = 2048 (fp32 LoRA deltas)
    fsets, bsets = [], []
    cos, sin = workloads.rope_tables(T, D, workloads.ROPE_THETA, device=dev)
    W = (NH + 2 * NKV) * D
    # forward: qkv fp16 + fp32 LoRA deltas; backward: dq, dk, dv fp16
    n_f = rotation_sets(M * W * 2 + M * (NH + NKV) * D * 4, n_sets)
    n_b = rotation_sets(M * W * 2, n_sets)
    for i in range(max(n_f, n_b)):
        qkv, lq, lv, pos = workloads.rope_inputs((T,) * B, T, NH, NKV, D, torch.float32,
                                                 seed=6 + 10 * i, device=dev)
        if i < n_f:
            q = torch.empty((B, NH, T, D), dtype=torch.float16, device=dev)
            k = torch.empty((B, NKV, T, D), dtype=torch.float16, device=dev)
            v = torch.empty((B, NKV, T, D), dtype=torch.float16, device=dev)
            fsets.append(((qkv, lq, lv, pos, q, k, v),
                          (p(qkv), p(lq), p(lv), _ext.DTYPE_F32, p(cos), p(sin), p(pos), None,
                           p(q), p(k), p(v), M, B, T, NH, NKV, D)))
        if i >= n_b:
            continue
        dq, dk, dv = workloads.rope_grads(B, T, NH, NKV, D, seed=7 + 10 * i, device=dev)
        dqkv = torch.empty((M, W), dtype=torch.float16, device=dev)
        bsets.append(((dq, dk, dv, pos, dqkv),
                      (p(dq), p(dk), p(dv), p(cos), p(sin), p(pos), p(dqkv), M, B, T, NH, NKV,
                       D)))
    tab = 2 * T * D * 4

    def rope_cpu(ob, backward):
        qc, lqc, lvc, posc = workloads.rope_inputs((T,) * B, T, NH, NKV, D, torch.float32,
                                                   seed=6)
        cc, sc = workloads.rope_tables(T, D, workloads.ROPE_THETA)
        if backward:
            dqc, dkc, dvc = workloads.rope_grads(B, T, NH, NKV, D, seed=7)
            return lambda: ob.rope_bwd(qc, cc, sc, posc, B, T, NH, NKV, D, dqc, dkc, dvc)
        return lambda: ob.rope_fwd(qc, lqc, lvc, cc, sc, posc, B, T, NH, NKV, D)

    cases.append(Case("rope_pack_fwd", "rope_pack_fwd_kernel", "soupk_rope_pack_fwd",
                      M * W * 2 + M * NH * D * 4 + M * NKV * D * 4 + tab + 8 * M + M * W * 2,
                      fsets, cpu=lambda ob: rope_cpu(ob, False), lib=lib))
    cases.append(Case("rope_pack_bwd", "rope_pack_bwd_kernel", "soupk_rope_pack_bwd",
                      M * W * 2 + tab + 8 * M + M * W * 2, bsets,
                      cpu=lambda ob: rope_cpu(ob, True), lib=lib))

    # SwiGLU forward and in-place backward at [2048, 2 x 8960]
    fsets, bsets = [], []
    for i in range(rotation_sets(M * 2 * I * 2, n_sets)):
        gu = workloads.swiglu_inputs(M, I, seed=4 + 10 * i, device=dev)
        act = torch.empty((M, I), dtype=torch.float16, device=dev)
        fsets.append(((gu, act), (p(gu), p(act), M, I)))
    for i in range(rotation_sets(M * 3 * I * 2, n_sets)):
        gu2 = workloads.swiglu_inputs(M, I, seed=5 + 10 * i, device=dev)
        dact = workloads.swiglu_grad(M, I, seed=5 + 10 * i, device=dev)
        bsets.append(((gu2, dact), (p(dact), p(gu2), M, I)))
    def swi_cpu(ob, backward):
        guc = workloads.swiglu_inputs(M, I, seed=4)
        if backward:
            dac = workloads.swiglu_grad(M, I, seed=5)
            return lambda: ob.swiglu_bwd(dac, guc)
        return lambda: ob.swiglu_fwd(guc)

    cases.append(Case("swiglu_fwd", "swiglu_fwd_vec_kernel", "soupk_swiglu_fwd",
                      M * 2 * I * 2 + M * I * 2, fsets, cpu=lambda ob: swi_cpu(ob, False),
                      lib=lib))
    cases.append(Case("swiglu_bwd", "swiglu_bwd_vec_kernel", "soupk_swiglu_bwd_inplace",
                      M * I * 2 + 2 * (M * 2 * I * 2), bsets, cpu=lambda ob: swi_cpu(ob, True),
                      lib=lib))

    # vocab head: one 256-row chunk of logits [256, 151936].  Timed through
    # soupk_head_stats_grad_rows (the form FusedHeadLoss calls) with the identity row map into
    # a gradient buffer of its own: the same kernel and the same bytes as the in-place
    # soupk_head_stats_grad (each labelled row read once and its gradient written once), but
    # the logits stay logits from one use of a set to the next (in place, every launch after a
    # set's first would run on the previous launch's gradient values, which are ~1e-7).
    sets = []
    rows, V = 256, workloads.VOCAB
    n_lab = 0
    for i in range(rotation_sets(rows * V * 2, n_sets)):
        z, tgt = workloads.head_logits(rows, V, seed=8 + 10 * i, device=dev)
        slot = torch.where(tgt != -100, torch.arange(rows, device=dev), -1).to(torch.int32)
        gbuf = torch.empty((rows, V), dtype=torch.float16, device=dev)
        ent = torch.empty(rows, dtype=torch.float32, device=dev)
        loss = torch.empty(rows, dtype=torch.float32, device=dev)
        cor = torch.empty(rows, dtype=torch.int32, device=dev)
        sets.append(((z, tgt, slot, gbuf, ent, loss, cor),
                     (p(z), p(tgt), p(slot), p(gbuf), rows, p(ent), p(loss), p(cor), None,
                      64.0 / 1843.0, rows, V)))
        if i == 0:
            n_lab = int((tgt != -100).sum())
    def head_cpu(ob):
        zc, tc = workloads.head_logits(rows, V, seed=8)
        return lambda: ob.head_stats_grad(zc, tc, 64.0 / 1843.0)

    cases.append(Case("head_stats_grad", "head_stats_grad_kernel", "soupk_head_stats_grad_rows",
                      rows * V * 2 + n_lab * V * 2 + 8 * rows + 4 * rows + 12 * rows, sets,
                      cpu=head_cpu, lib=lib))
    return cases


def build_extra_cases(dev, n_sets=None, lib=None):
    """HBM-bound kernels of the layer beyond the BASELINE set (reported apart, not in `value`):
    the one-launch NF4 unpack of a decoder layer's seven projections (soupk_nf4_unpack_multi,
    testt_amd.nf4.unpack_groups) and the split-K sum of the MLP's gate|up input gradient
    (soupk_sum_partials, 4 fp32 partials of [2048, 1536] -> fp16)."""
    from testt_amd import nf4

    H, I, NH, NKV, D = (workloads.HIDDEN, workloads.INTER, workloads.N_HEADS, workloads.N_KV,
                        workloads.HEAD_DIM)
    shapes = [(NH * D, H), (NKV * D, H), (NKV * D, H), (H, NH * D), (I, H), (I, H), (H, I)]
    sets, nbytes = [], 0
    elems = sum(n * k for n, k in shapes)
    for i in range(rotation_sets(elems // 2 + elems // 64, n_sets)):
        ws = [workloads.nf4_weight(n, k, seed=100 + 10 * i + j, device=dev)
              for j, (n, k) in enumerate(shapes)]
        plans = [nf4._plan(w, dev) for w in ws]
        outs = [torch.empty(n, k, dtype=torch.float16, device=dev) for n, k in shapes]
        n = len(ws)
        arrays = [(ctypes.c_void_p * n)(*[pl[0][f] for pl in plans]) for f in range(6)]
        out_a = (ctypes.c_void_p * n)(*[o.data_ptr() for o in outs])
        sizes = (ctypes.c_int64 * n)(*[pl[1] for pl in plans])
        sets.append(((ws, plans, outs, arrays, out_a, sizes),
                     (n, *[ctypes.addressof(a) for a in arrays], ctypes.addressof(out_a),
                      ctypes.addressof(sizes), 64, 256)))
        if i == 0:
            for w, pl in zip(ws, plans):
                st = w.quant_state
                nbytes += (pl[1] + st.absmax.numel() + 4 * st.state2.absmax.numel() + 4 * 256
                           + 4 * 16 + 4 + 4 * pl[1])
    cases = [Case("nf4_unpack_layer", "nf4_unpack_multi_kernel", "soupk_nf4_unpack_multi",
                  nbytes, sets, lib=lib)]
    M, n_parts = workloads.BATCH * workloads.SEQ, 4
    n = M * H
    sets = []
    for i in range(rotation_sets(4 * n_parts * n, n_sets)):
        parts = torch.randn(n_parts, n, generator=workloads.gen(200 + i)).to(dev)
        out = torch.empty(n, dtype=torch.float16, device=dev)
        sets.append(((parts, out), (parts.data_ptr(), n_parts, n, n, out.data_ptr())))
    cases.append(Case("splitk_sum", "sum_partials_kernel", "soupk_sum_partials",
                      4 * n_parts * n + 2 * n, sets, lib=lib))
    return cases


def build_floor_cases(dev, n_sets=3, lib=None):
    """The launch floor, timed exactly as the kernels are: an empty kernel of one workgroup and
    of 1024 workgroups (soupk_bench_empty), and a 4 KiB device copy (soupk_bench_copy)."""
    bufs = [(torch.empty(4096, dtype=torch.uint8, device=dev),
             torch.empty(4096, dtype=torch.uint8, device=dev)) for _ in range(n_sets)]
    return [Case("empty_kernel_1wg", "bench_empty_kernel", "soupk_bench_empty", 0,
                 [((), (1,))], lib=lib),
            Case("empty_kernel_1024wg", "bench_empty_kernel", "soupk_bench_empty", 0,
                 [((), (1024,))], lib=lib),
            Case("copy_4KiB", "bench_copy_kernel", "soupk_bench_copy", 8192,
                 [((a, b), (p(a), p(b), 4096)) for a, b in bufs], lib=lib)]


# The ragged batch of BASELINE.json's RoPE config: real lengths of the 4 rows of 512.
RAGGED_LENGTHS = (512, 152, 128, 96)


def build_shape_cases(dev, n_sets=None, lib=None):
    """Kernels of the set at the other shapes the step runs them at (reported apart, not in
    `value`): the RoPE pack forward / backward on the ragged batch RAGGED_LENGTHS (M = 888 real
    tokens of 4 x 512; the forward also writes the zeros of the 1160 pad positions, in the same
    launch, as the reference's padded layout needs); the token-major RoPE forward the layer
    runs (soupk_rope_pack_tokens: rotated q, k and v + LoRA in qkv's own row layout, no pad
    rows) on all 2048 tokens and on the ragged batch; the add + RMSNorm forward and backward on
    the ragged batch (888 rows; the forward's padded output over all 2048 positions); and the
    vocab-head kernel on a 2048-row
    chunk (head.CHUNK_ROWS, the product's chunk) through soupk_head_stats_grad_rows, the entry
    FusedHeadLoss uses (gradient rows packed into their own buffer), 90% of rows labelled."""
    H, NH, NKV, D, B, T = (workloads.HIDDEN, workloads.N_HEADS, workloads.N_KV,
                           workloads.HEAD_DIM, workloads.BATCH, workloads.SEQ)
    W = (NH + 2 * NKV) * D
    cos, sin = workloads.rope_tables(T, D, workloads.ROPE_THETA, device=dev)
    M = sum(RAGGED_LENGTHS)
    fsets, bsets = [], []
    # (the bytes read: the real positions' rows)
    n_f = rotation_sets(M * W * 2 + M * (NH + NKV) * D * 4, n_sets)
    n_b = rotation_sets(M * W * 2, n_sets)
    for i in range(max(n_f, n_b)):
        qkv, lq, lv, pos = workloads.rope_inputs(RAGGED_LENGTHS, T, NH, NKV, D, torch.float32,
                                                 seed=60 + 10 * i, device=dev)
        if i < n_f:
            inv = torch.full((B * T,), -1, dtype=torch.int32, device=dev)
            inv[pos] = torch.arange(M, dtype=torch.int32, device=dev)
            q = torch.empty((B, NH, T, D), dtype=torch.float16, device=dev)
            k = torch.empty((B, NKV, T, D), dtype=torch.float16, device=dev)
            v = torch.empty((B, NKV, T, D), dtype=torch.float16, device=dev)
            fsets.append(((qkv, lq, lv, pos, inv, q, k, v),
                          (p(qkv), p(lq), p(lv), _ext.DTYPE_F32, p(cos), p(sin), p(pos), p(inv),
                           p(q), p(k), p(v), M, B, T, NH, NKV, D)))
        if i >= n_b:
            continue
        dq, dk, dv = workloads.rope_grads(B, T, NH, NKV, D, seed=70 + 10 * i, device=dev)
        dqkv = torch.empty((M, W), dtype=torch.float16, device=dev)
        bsets.append(((dq, dk, dv, pos, dqkv),
                      (p(dq), p(dk), p(dv), p(cos), p(sin), p(pos), p(dqkv), M, B, T, NH, NKV,
                       D)))
    # cos/sin rows of the positions used (all 512 rows, read by the longest sequence)
    tab = 2 * T * D * 4
    cases = [
        Case("rope_pack_fwd_ragged888", "rope_pack_fwd_kernel", "soupk_rope_pack_fwd",
             M * W * 2 + M * (NH + NKV) * D * 4 + tab + 8 * M + 4 * B * T + B * T * W * 2,
             fsets, lib=lib),
        Case("rope_pack_bwd_ragged888", "rope_pack_bwd_kernel", "soupk_rope_pack_bwd",
             M * W * 2 + tab + 8 * M + M * W * 2, bsets, lib=lib)]
    for lengths, name in (((T,) * B, "rope_pack_tokens"),
                          (RAGGED_LENGTHS, "rope_pack_tokens_ragged888")):
        rows = sum(lengths)
        tsets = []
        for i in range(rotation_sets(rows * W * 2 + rows * (NH + NKV) * D * 4, n_sets)):
            qkv, lq, lv, pos = workloads.rope_inputs(lengths, T, NH, NKV, D, torch.float32,
                                                     seed=90 + 10 * i, device=dev)
            out = torch.empty((rows, W), dtype=torch.float16, device=dev)
            tsets.append(((qkv, lq, lv, pos, out),
                          (p(qkv), p(lq), p(lv), _ext.DTYPE_F32, p(cos), p(sin), p(pos), p(out),
                           rows, B, T, NH, NKV, D)))
        cases.append(Case(name, "rope_pack_fwd_kernel", "soupk_rope_pack_tokens",
                          rows * W * 2 + rows * (NH + NKV) * D * 4 + tab + 8 * rows
                          + rows * W * 2, tsets, lib=lib))
    # add + RMSNorm forward / backward on the ragged batch: M real rows, the forward's padded
    # output over all B * T positions (the 1160 unmapped rows zeroed in the same launch), the
    # backward's padded gradient gathered at the M mapped positions
    PT = B * T
    rfsets, rbsets = [], []
    for i in range(rotation_sets(14 * M * H, n_sets)):
        x, delta, w, pad_idx, padded = workloads.rmsnorm_inputs(M, H, PT, seed=52 + 10 * i,
                                                                device=dev)
        s_o = torch.empty_like(x)
        y = torch.empty((M, H), dtype=torch.float16, device=dev)
        ypad = torch.empty((PT, H), dtype=torch.float32, device=dev)
        rstd = torch.empty(M, dtype=torch.float32, device=dev)
        inv = torch.full((PT,), -1, dtype=torch.int32, device=dev)
        inv[pad_idx] = torch.arange(M, dtype=torch.int32, device=dev)
        rfsets.append(((x, delta, w, pad_idx, inv, s_o, y, ypad, rstd),
                       (p(x), p(delta), p(w), p(s_o), p(y), p(ypad), p(pad_idx), p(inv),
                        p(rstd), M, PT, H, 1e-6)))
        dy, dypad, ds = workloads.rmsnorm_grads(M, H, PT, seed=53 + 10 * i, device=dev)
        s_b = x + delta.float()
        rstd_b = torch.rsqrt(s_b.pow(2).mean(-1) + 1e-6)
        dx = torch.empty_like(x)
        dd = torch.empty((M, H), dtype=torch.float16, device=dev)
        rbsets.append(((s_b, rstd_b, w, dy, dypad, pad_idx, ds, dx, dd),
                       (p(s_b), p(rstd_b), p(w), p(dy), p(dypad), p(pad_idx), p(ds), p(dx),
                        p(dd), M, PT, H)))
    cases.append(Case("rmsnorm_fwd_ragged888", "rmsnorm_fwd_kernel", "soupk_rmsnorm_fwd",
                      16 * M * H + 4 * (PT - M) * H + 4 * H + 4 * M + 8 * M + 4 * PT, rfsets,
                      lib=lib))
    cases.append(Case("rmsnorm_bwd_ragged888", "rmsnorm_bwd_kernel", "soupk_rmsnorm_bwd",
                      20 * M * H + 4 * H + 4 * M + 8 * M, rbsets, lib=lib))
    rows, V = 2048, workloads.VOCAB
    sets, n_lab = [], 0
    for i in range(rotation_sets(rows * V * 2, n_sets)):
        g = torch.Generator(device=dev).manual_seed(80 + i)
        z = (0.784 * torch.randn(rows, V, generator=g, device=dev)).to(torch.float16)
        tgt = torch.randint(0, V, (rows,), generator=g, device=dev)
        tgt[torch.rand(rows, generator=g, device=dev) < 0.1] = -100
        lab = tgt != -100
        slot = torch.where(lab, torch.cumsum(lab, 0, dtype=torch.int32) - 1, -1).to(torch.int32)
        n = int(lab.sum())
        gbuf = torch.empty((n, V), dtype=torch.float16, device=dev)
        stats = [torch.empty(rows, dtype=dt, device=dev)
                 for dt in (torch.float32, torch.float32, torch.int32)]
        sets.append(((z, tgt, slot, gbuf, stats),
                     (p(z), p(tgt), p(slot), p(gbuf), n, *[p(t) for t in stats], None,
                      64.0 / 1843.0, rows, V)))
        if i == 0:
            n_lab = n
    cases.append(Case("head_stats_grad_2048rows", "head_stats_grad_kernel",
                      "soupk_head_stats_grad_rows",
                      rows * V * 2 + n_lab * V * 2 + 8 * rows + 4 * rows + 12 * rows, sets,
                      lib=lib))
    return cases


class HipEvents:
    """hipEvent_t pairs from the HIP runtime torch already loaded (RTLD_NOLOAD: the same one)."""

    def __init__(self):
        try:
            self.hip = ctypes.CDLL("libamdhip64.so.7", mode=os.RTLD_NOLOAD | os.RTLD_GLOBAL)
        except OSError:
            self.hip = ctypes.CDLL("libamdhip64.so.7")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p,
                                                 ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.events = []

    def new(self):
        ev = ctypes.c_void_p()
        if self.hip.hipEventCreate(ctypes.byref(ev)) != 0:
            raise RuntimeError("hipEventCreate failed")
        self.events.append(ev)
        return ev

    def elapsed_us(self, a, b):
        ms = ctypes.c_float()
        if self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value * 1e3

    def close(self):
        for ev in self.events:
            self.hip.hipEventDestroy(ev)
        self.events = []


class DeviceHold:
    """Keeps the current stream busy with a device-side wait (soupk_bench_hold: one wave that
    sleeps until the device's constant-rate wall clock has advanced the given time, so it
    always ends) while the host queues the launches to be timed behind it.  The GPU then runs
    them back to back, as in a training step, instead of at the host's launch rate (a ctypes
    launch with its event pair costs the host about as long as the shorter kernels run, so each
    of them would start on an idle GPU and the means would depend on the host's speed)."""

    def __init__(self, dev, lib=None):
        self.dev = dev
        self.lib = lib if lib is not None else _ext.lib()

    def hold(self, us):
        status = self.lib.soupk_bench_hold(float(min(us, 2e5)),
                                           torch.cuda.current_stream(self.dev).cuda_stream)
        if status != 0:
            raise RuntimeError(f"soupk_bench_hold failed with status {status}")


def time_gpu(cases, steps, warmup, dev, lib=None):
    """Per-launch kernel durations: soupk_time_next_launch() makes each launch record a HIP
    event pair with its own dispatch (hipExtLaunchKernelGGL), on the stream it runs on.  The
    timed launches are queued behind a DeviceHold that outlasts their enqueueing, so they run
    back to back.  Before the `warmup` steps, each case runs once on every input set."""
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    arm = (lib if lib is not None else _ext.lib()).soupk_time_next_launch
    hip = HipEvents()
    holder = DeviceHold(dev)
    # Every input set is used once before the warm-up, so that no timed launch is the first
    # access to its buffers (measured: with 5 warm-up steps and 20 timed ones, the sets first
    # used in the timed region made the kernels 3-10% slower).  A set's next use comes a whole
    # rotation later, so the Infinity Cache holds none of it by then.
    for c in cases:
        for i in range(len(c.sets)):
            c.launch(i, sh)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for w in range(warmup):
        for c in cases:
            c.launch(w, sh)
    warm_us = (time.perf_counter() - t0) * 1e6 / max(warmup, 1)
    ev = [[(hip.new(), hip.new()) for _ in cases] for _ in range(steps)]
    torch.cuda.synchronize(dev)
    # (the timed loop also arms the events: twice the warm-up's host time per step, plus 2 ms)
    holder.hold(2.0 * warm_us * steps + 2000.0)
    t0 = time.perf_counter()
    for s in range(steps):
        for j, c in enumerate(cases):
            a, b = ev[s][j]
            arm(a, b)
            c.launch(s, sh)
    host_enqueue = time.perf_counter() - t0
    torch.cuda.synchronize(dev)
    for j, c in enumerate(cases):
        c.times = [hip.elapsed_us(*ev[s][j]) for s in range(steps)]
    # GPU time from the first timed launch's start to the last one's end
    span = hip.elapsed_us(ev[0][0][0], ev[-1][-1][1]) * 1e-6
    hip.close()
    return host_enqueue, span


class GcWatch:
    """Counts Python garbage collections (and their wall time) while active: a collection
    inside a timed loop of host-driven steps shows up as a step far above the median."""

    def __init__(self):
        import gc

        self.gc = gc
        self.count, self.ms, self._t = 0, 0.0, None

    def _cb(self, phase, info):
        if phase == "start":
            self._t = time.perf_counter()
        elif self._t is not None:
            self.count += 1
            self.ms += (time.perf_counter() - self._t) * 1e3
            self._t = None

    def __enter__(self):
        self.gc.callbacks.append(self._cb)
        return self

    def __exit__(self, *exc):
        self.gc.callbacks.remove(self._cb)


def timed_steps(dev, step, steps, warmup):
    """Run `step()` warmup times, then `steps` times with a torch event pair around each step
    (the step's span on the GPU, host gaps included, as the training loop sees it).  Returns
    per-step microseconds, the span of the whole loop, and the garbage collections seen; the
    host's time to issue each step (its Python and dispatch time, microseconds) is attached to
    the GcWatch as `host_us`, so a slow step can be told apart as host- or device-side."""
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(steps)]
    host = [0.0] * steps
    torch.cuda.synchronize(dev)
    # No synchronisation between the warm-up and the timed steps: the first timed step then
    # starts behind queued work, as every step of a training loop does (after a synchronise
    # it started on an idle GPU and ran 120-300 us long in a 700 us layer step).
    for _ in range(warmup):
        step()
    with GcWatch() as gcw:
        for i, (a, b) in enumerate(evs):
            t0 = time.perf_counter()
            a.record()
            step()
            b.record()
            host[i] = (time.perf_counter() - t0) * 1e6
        torch.cuda.synchronize(dev)
    per = [a.elapsed_time(b) * 1e3 for a, b in evs]
    total = evs[0][0].elapsed_time(evs[-1][1]) * 1e3
    gcw.host_us = host
    return per, total, gcw


def step_summary(per, total, gcw, unit_scale=1.0, digits=1):
    """mean (the loop's span / steps), median, min, max of per-step times; with the host's
    issue time of the median step and of the slowest one (a slowest step whose host time
    exceeds the median host time by about its excess over the median step was held up on the
    host, not on the GPU)."""
    n = len(per)
    slowest = int(max(range(n), key=lambda i: per[i]))
    out = {"mean": round(total / n * unit_scale, digits),
           "median": round(median(per) * unit_scale, digits),
           "min": round(min(per) * unit_scale, digits),
           "max": round(max(per) * unit_scale, digits),
           "slowest_step": slowest, "steps": n,
           "gc_collections": gcw.count, "gc_ms": round(gcw.ms, 2)}
    host = getattr(gcw, "host_us", None)
    if host:
        out["host_issue_median"] = round(median(host) * unit_scale, digits)
        out["host_issue_slowest_step"] = round(host[slowest] * unit_scale, digits)
    return out


def layer_inputs(dev, lengths=None):
    """A synthetic decoder layer and its inputs at B=4 x T=512: every position real, or the
    first lengths[b] of row b (then key_valid is the key mask and pos the real positions)."""
    from testt_amd import layer

    B, T, H = workloads.BATCH, workloads.SEQ, workloads.HIDDEN
    w = layer.synthetic_layer(dev)
    if lengths is None:
        pos, key_valid = torch.arange(B * T, device=dev), None
    else:
        amask = torch.zeros(B, T, dtype=torch.int64, device=dev)
        for b, n in enumerate(lengths):
            amask[b, :n] = 1
        pos, key_valid = amask.reshape(-1).nonzero().squeeze(1), layer.key_valid_of(amask)
    M = pos.numel()
    cos, sin = (t.to(dev) for t in workloads.rope_tables(T))
    g = workloads.gen(10)
    s0 = torch.randn(M, H, generator=g).to(dev)
    d0 = (0.5 * torch.randn(M, H, generator=g)).to(torch.float16).to(dev)
    gs = (1e-2 * torch.randn(M, H, generator=g)).to(dev)
    gd = (1e-2 * torch.randn(M, H, generator=g)).to(torch.float16).to(dev)
    return w, pos, key_valid, cos, sin, s0, d0, gs, gd


def time_layer(dev, steps, warmup, reference_profile=False, lengths=None):
    """One Qwen2.5-1.5B decoder layer (testt_amd/layer.py) at B=4 x T=512 = 2048 real tokens
    (or the first `lengths` of each row): forward and forward+backward time per step of the
    eager loop (a torch event pair around each step: every kernel, GEMM and the attention).
    With reference_profile, the layer runs with the reference's memory profile: gate|up
    recomputed in backward (mlp.RECOMPUTE_GATE_UP) and the NF4 weights unpacked again in
    backward (nf4.KEEP_UNPACKED_FOR_BACKWARD = False), the work the reference's own layer
    does."""
    from testt_amd import layer, mlp, nf4

    B, T = workloads.BATCH, workloads.SEQ
    w, pos, key_valid, cos, sin, s0, d0, gs, gd = layer_inputs(dev, lengths)
    M = pos.numel()

    def step(backward):
        s_in = s0.detach().requires_grad_(True)
        d_in = d0.detach().requires_grad_(True)
        s, d = layer.decoder_layer(s_in, d_in, w, pos, B, T, cos, sin, key_valid)
        if backward:
            torch.autograd.backward([s, d], [gs, gd])

    saved = (mlp.RECOMPUTE_GATE_UP, nf4.KEEP_UNPACKED_FOR_BACKWARD)
    if reference_profile:
        mlp.RECOMPUTE_GATE_UP, nf4.KEEP_UNPACKED_FOR_BACKWARD = True, False
    out = {}
    try:
        for name, bwd in (("fwd_bwd", True), ("fwd", False)):
            per, total, gcw = timed_steps(dev, lambda: step(bwd), steps, warmup)
            st = step_summary(per, total, gcw)
            out[f"{name}_us"] = st["mean"]
            out[f"{name}_us_median"] = st["median"]
            out[f"{name}_steps"] = st
    finally:
        mlp.RECOMPUTE_GATE_UP, nf4.KEEP_UNPACKED_FOR_BACKWARD = saved
    out.update(tokens=M, batch=B, seq=T, lora_rank=16)
    if lengths is not None:
        out["lengths"] = list(lengths)
    if reference_profile:
        out["note"] = ("the reference's work profile: RECOMPUTE_GATE_UP = True (the gate|up GEMM "
                       "again in backward), KEEP_UNPACKED_FOR_BACKWARD = False (every NF4 weight "
                       "unpacked again in backward); otherwise as `layer`")
    else:
        out["note"] = ("synthetic NF4 weights, LoRA r=16 on q/v; hipBLASLt GEMMs in fp16, "
                       "every other op (attention included) a soupk kernel (testt_amd/layer.py); "
                       "*_us: mean per step of the eager loop (backward on the calling thread, "
                       "as testt_amd.apply() sets it), *_us_median the median step, *_steps the "
                       "distribution; graph_*: the same step captured once in a HIP graph and "
                       "replayed (the layer's GPU time; replays match the eager step bit for "
                       "bit, tests/test_gpu_layer_graph.py)")
    return out


def graph_layer(dev, steps, lengths=None):
    """The layer's forward+backward (and forward alone) captured in a HIP graph
    (torch.cuda.graph) and replayed `steps` times between torch events: the launches and their
    work without the Python and dispatch time of the eager loop."""
    from testt_amd import layer

    B, T = workloads.BATCH, workloads.SEQ
    w, pos, key_valid, cos, sin, s0, d0, gs, gd = layer_inputs(dev, lengths)
    s_in = s0.clone().requires_grad_(True)
    d_in = d0.clone().requires_grad_(True)
    leaves = (s_in, d_in, *w.lora_q, *w.lora_v)

    def step(backward):
        s, d = layer.decoder_layer(s_in, d_in, w, pos, B, T, cos, sin, key_valid)
        if backward:
            torch.autograd.backward([s, d], [gs, gd])
        for t in leaves:
            t.grad = None

    res = {}
    for name, bwd in (("graph_fwd_bwd_us", True), ("graph_fwd_us", False)):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            for _ in range(2):
                step(bwd)
        torch.cuda.current_stream(dev).wait_stream(side)
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step(bwd)
        graph.replay()
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(steps):
            graph.replay()
        e1.record()
        torch.cuda.synchronize(dev)
        res[name] = round(e0.elapsed_time(e1) * 1e3 / steps, 1)
        del graph
    return res


def time_attention(dev, steps, warmup, varlen_only=False):
    """The causal GQA attention kernels (testt_amd/csrc/attention.hip) at the layer's shape,
    B=4 x T=512, 12 query / 2 key-value heads of 128: forward and backward per call, torch
    events on the stream they run on.  `fwd`/`bwd`: the padded-layout kernels (every position
    real); `varlen_*`: the kernels the layer runs (token-major rows of the real tokens; the
    backward with RoPE's backward fused in); `ragged_*`: both at the BASELINE ragged batch
    (512, 152, 128, 96 real tokens), the padded ones with key flags.  Algorithmic FLOPs: 4*D
    per visible (query, key) pair forward (S and P.V), 10*D backward (recomputed S, dP, dV, dK,
    dQ), L(L+1)/2 visible pairs per real row of L tokens and head; MFMA-bound, against
    2.5 PFLOP/s dense fp16.  The timed calls are queued behind a DeviceHold, so the span
    holds the kernels' time, not the host's per-call overhead."""
    from testt_amd import attention

    B, T, NH, NKV, D = workloads.BATCH, workloads.SEQ, workloads.N_HEADS, workloads.N_KV, 128
    scale = 1.0 / math.sqrt(D)
    cos, sin = workloads.rope_tables(T, D, workloads.ROPE_THETA, device=dev)
    hold = DeviceHold(dev)

    def timed(fn):
        for _ in range(warmup):
            fn()
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        hold.hold(steps * 150 + 3000)
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize(dev)
        return e0.elapsed_time(e1) * 1e3 / steps

    def rate(us, flops):
        tflops = flops / (us * 1e-6) / 1e12
        return {"us": round(us, 2), "TFLOPs": round(tflops, 1),
                "frac_of_mfma_peak": round(tflops / PEAK_MFMA_F16_TFLOPS, 4)}

    res = {}
    for tag, lengths in (("", (T,) * B), ("ragged_", (512, 152, 128, 96))):
        g = workloads.gen(13)
        pos = workloads.ragged_positions(lengths, T).to(dev)
        M = pos.numel()
        pairs = NH * sum(n * (n + 1) / 2 for n in lengths)
        rows = torch.randn(M, (NH + 2 * NKV) * D, generator=g).to(torch.float16).to(dev)
        dout = torch.randn(M, NH * D, generator=g).to(torch.float16).to(dev)
        cu = attention.cu_seqlens_of(pos, B, T)
        out, lse = attention.attention_varlen_fwd(rows, cu, NH, NKV, scale)
        rope = (cos, sin, pos, B, T)
        res[f"{tag}varlen_fwd"] = rate(
            timed(lambda: attention.attention_varlen_fwd(rows, cu, NH, NKV, scale)),
            4 * D * pairs)
        res[f"{tag}varlen_bwd"] = rate(
            timed(lambda: attention.attention_varlen_bwd(rows, cu, out, lse, dout, scale, NH, NKV,
                                                         rope=rope)), 10 * D * pairs)
        if varlen_only:
            continue
        # the padded layout of the same tokens (key flags when rows are ragged)
        q = torch.randn(B, NH, T, D, generator=g).to(torch.float16).to(dev)
        k = torch.randn(B, NKV, T, D, generator=g).to(torch.float16).to(dev)
        v = torch.randn(B, NKV, T, D, generator=g).to(torch.float16).to(dev)
        pdout = torch.randn(B * T, NH * D, generator=g).to(torch.float16).to(dev)
        valid = None
        if M != B * T:
            valid = torch.zeros(B, T, dtype=torch.uint8, device=dev)
            for b, n in enumerate(lengths):
                valid[b, :n] = 1
        pout, plse = attention.attention_fwd(q, k, v, valid, scale)
        res[f"{tag}fwd"] = rate(timed(lambda: attention.attention_fwd(q, k, v, valid, scale)),
                                4 * D * pairs)
        res[f"{tag}bwd"] = rate(
            timed(lambda: attention.attention_bwd(q, k, v, valid, pout, plse, pdout, scale)),
            10 * D * pairs)
    res.update(shape={"batch": B, "seq": T, "q_heads": NH, "kv_heads": NKV, "head_dim": D,
                      "ragged_lengths": [512, 152, 128, 96]},
               note="causal; fwd/bwd: padded layout (bwd = D + (dQ | dK/dV-partial, one grid) + "
                    "GQA-reduce launches); varlen_*: token-major rows of the real tokens, the "
                    "layer's path (varlen_bwd writes the q|k|v GEMM output's gradient, RoPE's "
                    "backward fused into its dQ epilogue and GQA reduce); FLOPs count visible "
                    "pairs of real tokens only, so the padded kernels on the ragged batch are "
                    "charged only for the real work")
    return res


def time_nf4_gemm(dev, calls=40):
    """GPU time per call (microseconds) of the fused NF4-dequant GEMM (testt_amd/nf4_gemm.py,
    csrc/gemm_nf4.hip) against hipBLASLt on the unpacked weight, at M = 2048 for the four
    projections of a layer (q|k|v and gate|up as stacked parts): the fused kernel on fp16 and
    on NF4 weights, hipBLASLt (torch.matmul) on fp16 weights, the standalone unpack
    (nf4.unpack_concat) and unpack + hipBLASLt; and the input gradient dx = dy W fused
    (nf4_gemm.nf4_grad_input), on hipBLASLt and unpack + hipBLASLt; then the fused forward and
    input gradient against unpack + hipBLASLt at the smaller row counts SWEEP_ROWS
    (`rows_sweep`; the forward there also with its contraction split as
    nf4_gemm.split_count picks, `splits` of them).  Each variant: 5 untimed calls, then `calls`
    calls queued behind a DeviceHold and timed as one span (torch events), so host overhead is
    not in the figure.  Synthetic NF4 weights (workloads.nf4_weight), x ~ N(0, 1)."""
    from testt_amd import nf4, nf4_gemm

    hold = DeviceHold(dev)

    def span_us(fn):
        for _ in range(5):
            fn()
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        hold.hold(calls * 600 + 3000)
        e0.record()
        for _ in range(calls):
            fn()
        e1.record()
        torch.cuda.synchronize(dev)
        return round(e0.elapsed_time(e1) * 1e3 / calls, 2)

    M = 2048
    shapes = {"qkv": ((workloads.N_HEADS * workloads.HEAD_DIM, workloads.N_KV * workloads.HEAD_DIM,
                       workloads.N_KV * workloads.HEAD_DIM), workloads.HIDDEN),
              "o": ((workloads.HIDDEN,), workloads.N_HEADS * workloads.HEAD_DIM),
              "gate_up": ((workloads.INTER, workloads.INTER), workloads.HIDDEN),
              "down": ((workloads.HIDDEN,), workloads.INTER)}
    out = {}
    for name, (rows, K) in shapes.items():
        log(f"nf4 gemm: {name} ({sum(rows)} x {K}, M = {M})")
        ws = [workloads.nf4_weight(r, K, seed=50 + i, device=dev) for i, r in enumerate(rows)]
        g = workloads.gen(K)
        x = torch.randn(M, K, generator=g).to(torch.float16).to(dev)
        dy = (0.1 * torch.randn(M, sum(rows), generator=g)).to(torch.float16).to(dev)
        w16 = nf4.unpack_concat(ws, dev)
        out[name] = {
            "N": sum(rows), "K": K, "M": M,
            "fused_fp16_w_us": span_us(lambda: nf4_gemm.gemm_tn(x, w16)),
            "fused_nf4_w_us": span_us(lambda: nf4_gemm.nf4_linear(x, ws, splits=1)),
            "hipblaslt_fp16_w_us": span_us(lambda: torch.matmul(x, w16.t())),
            "unpack_us": span_us(lambda: nf4.unpack_concat(ws, dev)),
            "unpack_then_hipblaslt_us": span_us(
                lambda: torch.matmul(x, nf4.unpack_concat(ws, dev).t())),
            # the input gradient dx = dy W: fused (W dequantised in the GEMM) against
            # hipBLASLt on the fp16 weight and unpack + hipBLASLt
            "bwd_fused_nf4_w_us": span_us(lambda: nf4_gemm.nf4_grad_input(dy, ws, splits=1)),
            "bwd_hipblaslt_fp16_w_us": span_us(lambda: torch.matmul(dy, w16)),
            "bwd_unpack_then_hipblaslt_us": span_us(
                lambda: torch.matmul(dy, nf4.unpack_concat(ws, dev))),
        }
        # smaller row counts (decode- and eval-sized batches): the fused forward and input
        # gradient against unpack + hipBLASLt
        sweep = {}
        cus = torch.cuda.get_device_properties(dev).multi_processor_count
        for m in SWEEP_ROWS:
            xm, dym = x[:m].contiguous(), dy[:m].contiguous()
            splits = nf4_gemm.split_count(m, sum(rows), K, cus)
            bwd_splits = nf4_gemm.split_count(m, K, sum(rows), cus, nf4_gemm.GRAD_TILE)
            sweep[m] = {
                "splits": splits,
                "bwd_splits": bwd_splits,
                "fused_nf4_w_us": span_us(lambda: nf4_gemm.nf4_linear(xm, ws, splits=1)),
                "fused_split_nf4_w_us": span_us(
                    lambda: nf4_gemm.nf4_linear(xm, ws, splits=splits)),
                "unpack_then_hipblaslt_us": span_us(
                    lambda: torch.matmul(xm, nf4.unpack_concat(ws, dev).t())),
                "bwd_fused_nf4_w_us": span_us(lambda: nf4_gemm.nf4_grad_input(dym, ws, splits=1)),
                "bwd_fused_split_nf4_w_us": span_us(
                    lambda: nf4_gemm.nf4_grad_input(dym, ws, splits=bwd_splits)),
                "bwd_unpack_then_hipblaslt_us": span_us(
                    lambda: torch.matmul(dym, nf4.unpack_concat(ws, dev))),
            }
        out[name]["rows_sweep"] = sweep
        del ws, x, w16, dy
    return out


SWEEP_ROWS = (16, 64, 256, 512, 1024)   # row counts of the fused NF4 GEMM sweep

# token counts (B=4 rows of T=512) of the NF4-resident layer comparison
RESIDENT_LENGTHS = ((16, 0, 0, 0), (64, 0, 0, 0), (32, 32, 32, 32))
# and, with --nf4-resident-wide, the layer on NF4 weights forced at larger token counts
RESIDENT_WIDE_LENGTHS = ((64, 64, 64, 64), (128, 128, 128, 128), (192, 192, 192, 192),
                         (256, 256, 256, 256))


def trace_nf4_resident(dev, steps=5, warmup=3):
    """For a kernel trace of the layer at few tokens, NF4 weights against unpacked: for each
    token count of RESIDENT_LENGTHS and each mode, `warmup` forward+backward steps, then a
    DeviceHold, `steps` steps, a DeviceHold (summarize_nf4_resident reads the kernels between
    the holds).  Returns the segment labels in trace order."""
    from testt_amd import layer

    hold = DeviceHold(dev)
    B, T = workloads.BATCH, workloads.SEQ
    labels = []
    saved = layer.NF4_RESIDENT_SMALL_BATCHES
    try:
        for lengths in RESIDENT_LENGTHS:
            w, pos, key_valid, cos, sin, s0, d0, gs, gd = layer_inputs(dev, lengths)

            def step():
                s_in = s0.detach().requires_grad_(True)
                d_in = d0.detach().requires_grad_(True)
                s, d = layer.decoder_layer(s_in, d_in, w, pos, B, T, cos, sin, key_valid)
                torch.autograd.backward([s, d], [gs, gd])

            for resident in (True, False):
                layer.NF4_RESIDENT_SMALL_BATCHES = resident
                for _ in range(warmup):
                    step()
                torch.cuda.synchronize(dev)
                hold.hold(50)
                for _ in range(steps):
                    step()
                hold.hold(50)
                torch.cuda.synchronize(dev)
                labels.append([sum(lengths), "nf4" if resident else "unpacked", steps])
    finally:
        layer.NF4_RESIDENT_SMALL_BATCHES = saved
    return labels


def time_nf4_resident_wide(dev, steps=40, warmup=5):
    """time_nf4_resident's comparison at RESIDENT_WIDE_LENGTHS, the layer put on its NF4
    weights at every size (layer.NF4_RESIDENT_MAX_TOKENS) although single products there
    measured faster unpacked: where the layer's sum crosses over."""
    from testt_amd import layer

    saved = layer.NF4_RESIDENT_MAX_TOKENS
    try:
        layer.NF4_RESIDENT_MAX_TOKENS = max(sum(x) for x in RESIDENT_WIDE_LENGTHS)
        return time_nf4_resident(dev, steps, warmup, RESIDENT_WIDE_LENGTHS)
    finally:
        layer.NF4_RESIDENT_MAX_TOKENS = saved


def time_nf4_resident(dev, steps=40, warmup=5, lengths_list=RESIDENT_LENGTHS):
    """The decoder layer at few tokens with its products on the NF4 weights (the fused
    NF4-dequant GEMM in each direction, no fp16 weight in memory:
    layer.NF4_RESIDENT_SMALL_BATCHES) against the same layer unpacking its seven projections
    in one launch for hipBLASLt: forward+backward per step, the eager loop's median step
    (time_layer) and a captured HIP graph's replay (graph_layer, the GPU time)."""
    from testt_amd import layer

    out = {}
    saved = layer.NF4_RESIDENT_SMALL_BATCHES
    try:
        for lengths in lengths_list:
            row = {"lengths": list(lengths)}
            for resident in (True, False):
                layer.NF4_RESIDENT_SMALL_BATCHES = resident
                tag = "nf4" if resident else "unpacked"
                log(f"layer at {sum(lengths)} tokens, {tag} weights")
                t = time_layer(dev, steps, warmup, lengths=lengths)
                row[f"{tag}_eager_fwd_bwd_median_us"] = t["fwd_bwd_us_median"]
                row[f"{tag}_graph_fwd_bwd_us"] = graph_layer(dev, steps, lengths)[
                    "graph_fwd_bwd_us"]
            out[str(sum(lengths))] = row
    finally:
        layer.NF4_RESIDENT_SMALL_BATCHES = saved
    return out


def time_step(dev, steps, warmup, n_layers=28, reference_profile=False):
    """One QLoRA training step of the whole Qwen2.5-1.5B-shaped model at B=4 x T=512 = 2048
    real tokens, prompt tokens unlabelled, through the model-level drop-in the reference's
    trainer patch calls (solution/trainer_patch.py:57-63): a transformers Qwen2ForCausalLM with
    4-bit projections and LoRA r=16 on q/v (workloads.qwen2_qlora), `can_run` and then
    `fused_forward(model, input_ids, attention_mask, labels, num_items_in_batch)` under fp16
    autocast (28 decoder layers, final norm, the chunked fused head loss over the
    151,936-token vocabulary): forward and forward+backward time per step on the GPU (a torch
    event pair around each step).  With reference_profile, the reference's work profile:
    gate|up recomputed and the NF4 weights unpacked again in backward, and the head in the
    reference's 256-row chunks (head.CHUNK_ROWS = 256)."""
    from testt_amd import head, mlp, model, nf4

    B, T = workloads.BATCH, workloads.SEQ
    hf = workloads.qwen2_qlora(dev, n_layers=n_layers)
    g = workloads.gen(12)
    ids = torch.randint(0, workloads.VOCAB, (B, T), generator=g).to(dev)
    mask = torch.ones(B, T, dtype=torch.int64, device=dev)
    labels = ids.clone()
    labels[:, :T // 4] = -100                        # prompt tokens carry no label
    params = workloads.lora_parameters(hf)
    with torch.autocast("cuda", dtype=torch.float16):
        if not model.can_run(hf, ids, mask, labels, {"num_items_in_batch": None}):
            raise RuntimeError("the fused path does not take the benchmark model")

    def step(backward):
        for q in params:
            q.grad = None
        with torch.autocast("cuda", dtype=torch.float16):
            loss = model.fused_forward(hf, ids, mask, labels, None).loss
        if backward:
            loss.backward()

    saved = (mlp.RECOMPUTE_GATE_UP, nf4.KEEP_UNPACKED_FOR_BACKWARD, head.CHUNK_ROWS)
    if reference_profile:
        mlp.RECOMPUTE_GATE_UP, nf4.KEEP_UNPACKED_FOR_BACKWARD, head.CHUNK_ROWS = True, False, 256
    out = {}
    try:
        # Each mode is warmed up before it is timed: the caching allocator's pool then fits
        # that mode's allocation pattern, and no device allocation falls inside the timed steps.
        for name, bwd in (("fwd_bwd", True), ("fwd", False)):
            per, total, gcw = timed_steps(dev, lambda: step(bwd), steps, warmup)
            st = step_summary(per, total, gcw, 1e-3, 3)
            out[f"{name}_ms"] = st["mean"]
            out[f"{name}_ms_median"] = st["median"]
            out[f"{name}_steps"] = st
    finally:
        mlp.RECOMPUTE_GATE_UP, nf4.KEEP_UNPACKED_FOR_BACKWARD, head.CHUNK_ROWS = saved
    out.update(tokens=B * T, batch=B, seq=T, layers=n_layers,
               tokens_per_s=round(B * T / (out["fwd_bwd_ms"] * 1e-3), 1),
               tokens_per_s_median=round(B * T / (out["fwd_bwd_ms_median"] * 1e-3), 1))
    out["note"] = ("model.fused_forward on a transformers Qwen2ForCausalLM under fp16 autocast "
                   "(synthetic NF4 weights and fp16 tied embedding, LoRA r=16 on q/v); "
                   "hipBLASLt GEMMs in fp16, every other op (attention included) a soupk "
                   "kernel; backward "
                   "on the calling thread (testt_amd.configure_backward, as apply() sets it)"
                   + ("; the reference's work profile: RECOMPUTE_GATE_UP = True, "
                      "KEEP_UNPACKED_FOR_BACKWARD = False, CHUNK_ROWS = 256"
                      if reference_profile else ""))
    del hf
    return out


def copy_reference(cases, dev, reps=60, pool_mib=768):
    """Mean duration of a plain streaming device copy (soupk_bench_copy) moving each kernel's
    algorithmic byte count (half read, half written), timed like the kernels (back to back,
    behind a DeviceHold).  Every launch
    copies a different slice of two pool_mib pools, so more than 600 MB of other traffic lies
    between two uses of one slice and the Infinity Cache cannot serve them.  Returns
    {case name: us}."""
    lib = _ext.lib()
    pool = pool_mib << 20
    src = torch.empty(pool, dtype=torch.uint8, device=dev)
    dst = torch.empty(pool, dtype=torch.uint8, device=dev)
    sh = torch.cuda.current_stream(dev).cuda_stream
    hip = HipEvents()
    holder = DeviceHold(dev)
    out = {}
    for c in cases:
        size = (c.nbytes // 2) // 4096 * 4096
        slots = max(1, pool // size)
        evs = [(hip.new(), hip.new()) for _ in range(reps)]
        torch.cuda.synchronize(dev)
        holder.hold(60.0 * (reps + 10) + 2000.0)   # (launches run back to back, as the kernels')
        for r in range(reps + 10):
            off = (r % slots) * size
            if r >= 10:
                lib.soupk_time_next_launch(*evs[r - 10])
            st = lib.soupk_bench_copy(src.data_ptr() + off, dst.data_ptr() + off, size, sh)
            if st:
                raise _ext.SoupkError(f"soupk_bench_copy failed with status {st}")
        torch.cuda.synchronize(dev)
        ts = [hip.elapsed_us(a, b) for a, b in evs]
        out[c.name] = sum(ts) / len(ts) * (c.nbytes / (2 * size))
        hip.close()
    del src, dst
    return out


def copy_peak(dev, mib=1024, reps=12):
    """Read+write GB/s of the fastest plain streaming copy measured on this GPU
    (soupk_bench_copy: one 16-byte chunk per thread, non-temporal load, nt sc1 store) moving
    `mib` MiB, timed like the kernels (dispatch-recorded events, back to back behind a device
    wait); the median of `reps` launches."""
    lib = _ext.lib()
    size = mib << 20
    src = torch.empty(size, dtype=torch.uint8, device=dev)
    dst = torch.empty(size, dtype=torch.uint8, device=dev)
    src.fill_(1)
    sh = torch.cuda.current_stream(dev).cuda_stream
    hip = HipEvents()
    holder = DeviceHold(dev)
    evs = [(hip.new(), hip.new()) for _ in range(reps)]
    for _ in range(2):
        lib.soupk_bench_copy(src.data_ptr(), dst.data_ptr(), size, sh)
    torch.cuda.synchronize(dev)
    holder.hold(500.0 * reps + 2000.0)
    for a, b in evs:
        lib.soupk_time_next_launch(a, b)
        st = lib.soupk_bench_copy(src.data_ptr(), dst.data_ptr(), size, sh)
        if st:
            raise _ext.SoupkError(f"soupk_bench_copy failed with status {st}")
    torch.cuda.synchronize(dev)
    us = median([hip.elapsed_us(a, b) for a, b in evs])
    hip.close()
    del src, dst
    return round(2 * size / (us * 1e-6) / 1e9, 1)


def torch_copy_GBps(dev, mib=1024, reps=6):
    """Read+write GB/s of torch's device copy (copy_, __amd_rocclr_copyBuffer) of `mib` MiB;
    the 1 GiB copy whose PMC counters scale the traffic table (summarize_pmc)."""
    n = mib * (1 << 20) // 4
    a = torch.ones(n, device=dev)
    b = torch.empty(n, device=dev)
    b.copy_(a)
    torch.cuda.synchronize(dev)
    ts = []
    for _ in range(reps):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        b.copy_(a)
        e1.record()
        torch.cuda.synchronize(dev)
        ts.append(e0.elapsed_time(e1) * 1e-3)
    del a, b
    return round(2 * n * 4 / median(ts) / 1e9, 1)


def cpu_baseline(cases, seconds):
    from oracle import baseline as ob     # the CPU leg is the only user of oracle/ here

    threads = max(1, len(os.sched_getaffinity(0)))      # every core this process may run on
    torch.set_num_threads(threads)
    runs = [c.cpu(ob) for c in cases]
    for run in runs:                      # warm-up pass (page faults, thread pool)
        run()
    passes, t0 = 0, time.perf_counter()
    while True:
        for run in runs:
            run()
        passes += 1
        if time.perf_counter() - t0 >= seconds:
            break
    elapsed = time.perf_counter() - t0
    total = sum(c.nbytes for c in cases) * passes
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f if ln.startswith("model name")),
                         "")
    except OSError:
        pass
    return {"value": round(total / elapsed / 1e9, 3), "unit": "GB/s", "cores": threads,
            "cpu_model": model, "kind": "port",
            "sample": (f"{passes} full pass(es) of the kernel set at the step shape (all 8 "
                       f"kernels, BASELINE configs) through the reference's eager PyTorch path "
                       f"on the CPU (oracle/baseline.py), {elapsed:.1f} s, {model}")}


def pmc_traffic(entry, path=TRAFFIC_TABLE):
    """Measured HBM bytes per launch of bench entry `entry` (e.g. "swiglu_bwd") from the
    committed PMC table, or None."""
    try:
        with open(path) as f:
            for ln in f:
                cells = [c.strip().strip("`") for c in ln.strip().strip("|").split("|")]
                if len(cells) >= 10 and cells[0] == entry:
                    return int(cells[7])
    except (OSError, ValueError):
        pass
    return None


def _kernel_base(name):
    # A name the profiler left mangled (it does not demangle _Float16 parameters): the
    # length-prefixed function name after the namespaces.
    m = re.match(r"_ZN5soupk12_GLOBAL__N_1(\d+)", name)
    if m:
        return name[m.end():m.end() + int(m.group(1))]
    return name.replace("soupk::(anonymous namespace)::", "").replace("void ", "").split("(")[0]


def _read_csv(path):
    import csv
    with open(path) as f:
        return list(csv.DictReader(f))


def _launch_groups(rows, name_col="Kernel_Name"):
    """soupk launches of a rocprofv3 CSV grouped by (kernel, grid, workgroup), in the order of
    each group's first dispatch: {key: [rows]}."""
    groups = {}
    for r in rows:
        if "soupk" not in r[name_col]:
            continue
        grid = r.get("Grid_Size_X", r.get("Grid_Size"))
        wg = r.get("Workgroup_Size_X", r.get("Workgroup_Size"))
        key = (_kernel_base(r[name_col]), int(grid), int(wg))
        groups.setdefault(key, []).append(r)
    return dict(sorted(groups.items(), key=lambda kv: int(kv[1][0]["Dispatch_Id"])))


def _unnamed(kernel):
    """Label of a launch group that no bench entry claims."""
    return {"bench_copy_kernel": "(copy reference)",
            "bench_hold_kernel": "(device-side wait)"}.get(kernel, "-")


def _bench_entries(bench, keys):
    """{group key: (bench entry name, entry)}: bench.py times the set, then the kernels beyond
    it, then the other shapes, then the launch floor, so each entry takes the earliest unused
    group of its kernel; the floor's groups are matched by grid."""
    out, used = {}, set()
    for sect in ("kernels", "kernels_beyond_set", "kernels_other_shapes"):
        for name, v in bench.get(sect, {}).items():
            key = next((k for k in keys if k[0].split("<")[0] == v["kernel"] and k not in used),
                       None)
            if key is not None:
                used.add(key)
                out[key] = (name, v)
    for name, kern, grid in (("empty_kernel_1wg", "bench_empty_kernel", 256),
                             ("empty_kernel_1024wg", "bench_empty_kernel", 1024 * 256),
                             ("copy_4KiB", "bench_copy_kernel", 4096 // 16)):
        key = next((k for k in keys if k[0] == kern and k[1] == grid and k not in used), None)
        if key is not None and name in bench.get("launch_floor_us", {}):
            used.add(key)
            out[key] = ("launch floor: " + name, {"us_median": bench["launch_floor_us"][name]})
    return out


def summarize_stats(trace_csv, bench_json, command):
    """Markdown summary of a rocprofv3 --kernel-trace run of bench.py, launches grouped by
    kernel and grid, beside bench.py's own timing of the same launches (an unprofiled run)."""
    bench = json.loads(open(bench_json).read().strip().splitlines()[-1])
    groups = _launch_groups(_read_csv(trace_csv))
    ns = {k: [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in rs]
          for k, rs in groups.items()}
    names = _bench_entries(bench, list(groups))
    out = ["# rocprofv3 kernel trace: kernel set at the 2048-token step (bench.py)", "",
           "Command (run from /tmp on the MI355X box, TMPDIR=/tmp):", "", "```", command, "```",
           "", "Every soupk launch of the run by kernel and grid (threads / workgroup size), "
           "beside `python bench.py`'s timing of the same launches in an unprofiled run "
           "(dispatch-recorded HIP events; the mean, the median for the launch floor):", "",
           "| bench entry | kernel | grid / WG | calls | rocprof avg us | rocprof median us | "
           "min us | max us | bench us | rocprof / bench | bench GB/s | % of 8 TB/s |",
           "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for key, d in ns.items():
        entry, v = names.get(key, (_unnamed(key[0]), None))
        avg, med = sum(d) / len(d) / 1e3, median(d) / 1e3
        if v is None:
            tail = "- | - | - | -"
        elif "us_mean" in v:
            tail = (f"{v['us_mean']:.2f} | {avg / v['us_mean']:.3f} | {v['GBps']:.0f} | "
                    f"{100 * v['frac_of_peak']:.1f}")
        else:
            tail = f"{v['us_median']:.2f} | {med / v['us_median']:.3f} (median) | - | -"
        out.append(f"| {entry} | `{key[0]}` | {key[1]} / {key[2]} | {len(d)} | {avg:.2f} | "
                   f"{med:.2f} | {min(d) / 1e3:.2f} | {max(d) / 1e3:.2f} | {tail} |")
    return "\n".join(out) + "\n"


def summarize_kernels(stats_csv, title, command, top=30):
    """Markdown table of every kernel of a rocprofv3 --kernel-trace --stats run, by total time
    (hipBLASLt, torch and soupk kernels alike)."""
    rows = sorted(_read_csv(stats_csv), key=lambda r: -float(r["TotalDurationNs"]))
    # DeviceHold's waits (bench_hold_kernel) are not work: listed apart
    holds = [r for r in rows if "bench_hold_kernel" in r["Name"]]
    rows = [r for r in rows if "bench_hold_kernel" not in r["Name"]]
    total = sum(float(r["TotalDurationNs"]) for r in rows)
    out = [f"# {title}", "", "Command (run from /tmp on the MI355X box, TMPDIR=/tmp):", "", "```",
           command, "```", "", f"All kernels: {total / 1e6:.2f} ms in "
           f"{sum(int(r['Calls']) for r in rows)} launches"
           + (f", besides {sum(int(r['Calls']) for r in holds)} device-side waits "
              f"(DeviceHold, {sum(float(r['TotalDurationNs']) for r in holds) / 1e6:.1f} ms)"
              if holds else "") + ".", "",
           "| kernel | calls | avg us | total ms | share |", "|---|---:|---:|---:|---:|"]
    for r in rows[:top]:
        name = r["Name"]
        short = _kernel_base(name) if "soupk" in name else name.split("(")[0][:90]
        out.append(f"| `{short}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                   f"{float(r['TotalDurationNs']) / 1e6:.3f} | "
                   f"{100 * float(r['TotalDurationNs']) / total:.1f}% |")
    return "\n".join(out) + "\n"


def summarize_trace(trace_csv, title, command):
    """Markdown table of every launch group of a rocprofv3 --kernel-trace run, in the order of
    each group's first dispatch: calls, mean and median duration (hipBLASLt, torch and soupk
    kernels alike).  A group is one (kernel, grid, workgroup) between two DeviceHold waits, so
    launches of equal grids timed apart (two GEMMs with one output shape) stay apart; the
    waits themselves are left out."""
    groups, span = {}, 0
    for r in sorted(_read_csv(trace_csv), key=lambda r: int(r["Dispatch_Id"])):
        name = r["Kernel_Name"]
        if "bench_hold_kernel" in name:
            span += 1
            continue
        short = _kernel_base(name) if "soupk" in name else name.split("(")[0][:90]
        grid = r.get("Grid_Size_X", r.get("Grid_Size"))
        wg = r.get("Workgroup_Size_X", r.get("Workgroup_Size"))
        groups.setdefault((short, int(grid), int(wg), span), []).append(r)
    order = sorted(groups.items(), key=lambda kv: int(kv[1][0]["Dispatch_Id"]))
    out = [f"# {title}", "", "Command (run from /tmp on the MI355X box, TMPDIR=/tmp):", "", "```",
           command, "```", "", "Launches grouped by kernel and grid (threads / workgroup size) "
           "between two device-side waits, in the order of their first dispatch:", "",
           "| kernel | grid / WG | calls | avg us | median us |", "|---|---:|---:|---:|---:|"]
    for (short, grid, wg, _), rs in order:
        d = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in rs]
        out.append(f"| `{short}` | {grid} / {wg} | {len(d)} | {sum(d) / len(d):.2f} | "
                   f"{median(d):.2f} |")
    return "\n".join(out) + "\n"


def summarize_nf4_resident(trace_csv, bench_json, command):
    """Per token count and mode (trace_nf4_resident's segments): each kernel's launches and
    GPU time per forward+backward step of the layer, and the total."""
    with open(bench_json) as f:
        labels = json.loads(f.read().strip().splitlines()[-1])["nf4_resident_trace"]
    spans, cur, held = [], None, 0
    for r in sorted(_read_csv(trace_csv), key=lambda r: int(r["Dispatch_Id"])):
        name = r["Kernel_Name"]
        if "bench_hold_kernel" in name:
            held += 1
            cur = {} if held % 2 == 1 else None      # odd holds open a measured span
            if cur is not None:
                spans.append(cur)
            continue
        if cur is None:
            continue
        short = _kernel_base(name) if "soupk" in name else name.split("(")[0][:80]
        d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        n, t = cur.get(short, (0, 0.0))
        cur[short] = (n + 1, t + d)
    out = [f"# rocprofv3 kernel trace: the decoder layer at few tokens, NF4 weights (fused "
           "NF4-dequant GEMMs) against unpacked weights + hipBLASLt", "",
           "Command (run from /tmp on the MI355X box, TMPDIR=/tmp):", "", "```", command, "```",
           "", "Kernel launches and GPU time per forward+backward step of one Qwen2.5-1.5B "
           "decoder layer (synthetic NF4 weights, LoRA r=16 on q/v), averaged over the measured "
           "steps of each segment (bench.py trace_nf4_resident).", ""]
    for (tokens, mode, steps), span in zip(labels, spans):
        total = sum(t for _, t in span.values()) / steps
        out += [f"## {tokens} tokens, {mode} weights: {total:.1f} us of kernels per step", "",
                "| kernel | launches per step | us per step |", "|---|---:|---:|"]
        for short, (n, t) in sorted(span.items(), key=lambda kv: -kv[1][1]):
            out.append(f"| `{short}` | {n / steps:g} | {t / steps:.1f} |")
        out.append("")
    return "\n".join(out)


NF4_GEMM_VARIANTS = ("fused_fp16_w_us", "fused_nf4_w_us", "hipblaslt_fp16_w_us", "unpack_us",
                     "unpack_then_hipblaslt_us", "bwd_fused_nf4_w_us", "bwd_hipblaslt_fp16_w_us",
                     "bwd_unpack_then_hipblaslt_us")
NF4_GEMM_SWEEP_VARIANTS = ("fused_nf4_w_us", "fused_split_nf4_w_us", "unpack_then_hipblaslt_us",
                           "bwd_fused_nf4_w_us", "bwd_fused_split_nf4_w_us",
                           "bwd_unpack_then_hipblaslt_us")
# sweep variant -> the key of its split count
_SPLIT_KEY = {"fused_split_nf4_w_us": "splits", "bwd_fused_split_nf4_w_us": "bwd_splits"}


def nf4_gemm_spans(trace_csv, bench, calls=40):
    """Mean kernel time per call of each timed group of a `bench.py --nf4-gemm` kernel trace.
    Every group is `calls` calls queued behind one device-side wait, so the dispatches between
    two waits are one group's timed calls followed by the next group's untimed ones; a call is
    one kernel, or two for the unpack + hipBLASLt groups and the split kernels with more than
    one split (their means are added).  Returns
    {(shape, rows, variant): (kernel names, microseconds)} in the order time_nf4_gemm runs them."""
    spans, cur = [], None
    for r in sorted(_read_csv(trace_csv), key=lambda r: int(r["Dispatch_Id"])):
        name = r["Kernel_Name"]
        if "bench_hold_kernel" in name:
            cur = []
            spans.append(cur)
        elif cur is not None:
            cur.append(r)
    order = []   # (key, kernels per call)
    two = lambda k: 2 if k.endswith("unpack_then_hipblaslt_us") else 1
    for shape, v in bench.items():
        order += [((shape, v["M"], k), two(k)) for k in NF4_GEMM_VARIANTS]
        for m, sv in v.get("rows_sweep", {}).items():
            order += [((shape, int(m), k), 2 if sv.get(_SPLIT_KEY.get(k), 1) > 1 else two(k))
                      for k in NF4_GEMM_SWEEP_VARIANTS]
    if len(spans) != len(order):
        raise ValueError(f"{len(spans)} timed spans in the trace, {len(order)} groups expected")
    out = {}
    for (key, per_call), rs in zip(order, spans):
        timed = rs[:calls * per_call]
        by = {}
        for r in timed:
            n = r["Kernel_Name"]
            short = _kernel_base(n) if "soupk" in n else n.split("(")[0][:60]
            by.setdefault(short, []).append(
                (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        out[key] = (sorted(by), sum(sum(d) / len(d) for d in by.values()))
    return out


def summarize_nf4_gemm(trace_csv, bench_json, command):
    """Markdown tables of a rocprofv3 --kernel-trace run of `bench.py --nf4-gemm`: per
    projection the fused NF4-dequant GEMM (forward, input gradient) against hipBLASLt and
    unpack + hipBLASLt at 2048 rows, then the fused kernels against unpack + hipBLASLt over
    the smaller row counts, each figure the mean kernel time of its 40 timed calls."""
    bench = json.loads(open(bench_json).read().strip().splitlines()[-1])["nf4_gemm"]
    spans = nf4_gemm_spans(trace_csv, bench)
    t = lambda shape, m, k: spans[(shape, m, k)][1]
    label = {"qkv": "q\\|k\\|v", "o": "o", "gate_up": "gate\\|up", "down": "down"}
    out = [f"# rocprofv3 kernel trace: fused NF4-dequant GEMM (forward and input gradient) "
           "against hipBLASLt and unpack + hipBLASLt (bench.py --nf4-gemm)", "",
           "Command (run from /tmp on the MI355X box, TMPDIR=/tmp):", "", "```", command, "```",
           "", "Per projection shape (q|k|v: N 2048 as 1536 + 256 + 256, K 1536; o: N 1536, "
           "K 1536; gate|up: N 17920 as 8960 + 8960, K 1536; down: N 1536, K 8960) bench.py "
           "times each variant as 5 untimed calls and then 40 calls queued behind a device-side "
           "wait; every figure below is the mean kernel duration of those 40 calls in this "
           "trace (unpack + hipBLASLt: the two kernels' means added).  Fused: this build's "
           "`gemm_tn_kernel` (forward, y = x W^T) and `gemm_nn_nf4_kernel` (input gradient, "
           "dx = dy W) with W read as NF4 and dequantised in the tile loads.", "",
           "At 2048 rows (microseconds; **bold**: the faster of fused and unpack + hipBLASLt):",
           "", "| shape | fused, fp16 W | fused, NF4 W | hipBLASLt, fp16 W | unpack alone | "
           "unpack + hipBLASLt | fused dx, NF4 W | hipBLASLt dx, fp16 W | unpack + hipBLASLt dx |",
           "|---|---:|---:|---:|---:|---:|---:|---:|---:|"]
    b = lambda x, y: (f"**{x:.2f}**", f"{y:.2f}") if x <= y else (f"{x:.2f}", f"**{y:.2f}**")
    bold = lambda *xs: [f"**{x:.2f}**" if x == min(xs) else f"{x:.2f}" for x in xs]
    for shape, v in bench.items():
        m = v["M"]
        f, u = b(t(shape, m, "fused_nf4_w_us"), t(shape, m, "unpack_then_hipblaslt_us"))
        fd, ud = b(t(shape, m, "bwd_fused_nf4_w_us"), t(shape, m, "bwd_unpack_then_hipblaslt_us"))
        out.append(f"| {label.get(shape, shape)} | {t(shape, m, 'fused_fp16_w_us'):.2f} | {f} | "
                   f"{t(shape, m, 'hipblaslt_fp16_w_us'):.2f} | {t(shape, m, 'unpack_us'):.2f} | "
                   f"{u} | {fd} | {t(shape, m, 'bwd_hipblaslt_fp16_w_us'):.2f} | {ud} |")
    out += ["", "Smaller row counts (decode- and eval-sized batches), microseconds; `*`: the path "
            "FrozenNF4Linear takes (testt_amd/nf4_gemm.py prefer_fused, "
            "prefer_fused_grad_input); fused, K split: soupk_gemm_tn_nf4_split with the split "
            "count nf4_gemm.split_count picks (in parentheses; 1: the unsplit kernel), its "
            "figure the sum of its two kernels' means:", "",
            "| shape | rows | fused | fused, K split (splits) | unpack + hipBLASLt | fused dx | "
            "fused dx, split (splits) | unpack + hipBLASLt dx |",
            "|---|---:|---:|---:|---:|---:|---:|---:|"]
    from testt_amd import nf4_gemm
    cus = 256
    dims = {"qkv": (2048, 1536), "o": (1536, 1536), "gate_up": (17920, 1536),
            "down": (1536, 8960)}
    for shape, v in bench.items():
        n, k = dims.get(shape, (v["N"], v["K"]))
        sweep = {int(a): c for a, c in v.get("rows_sweep", {}).items()}
        for m in sorted(sweep):
            f, fs, u = bold(t(shape, m, "fused_nf4_w_us"), t(shape, m, "fused_split_nf4_w_us"),
                            t(shape, m, "unpack_then_hipblaslt_us"))
            fs += f" ({sweep[m].get('splits', 1)})"
            fd, fds, ud = bold(t(shape, m, "bwd_fused_nf4_w_us"),
                               t(shape, m, "bwd_fused_split_nf4_w_us"),
                               t(shape, m, "bwd_unpack_then_hipblaslt_us"))
            fds += f" ({sweep[m].get('bwd_splits', 1)})"
            if not nf4_gemm.fused_fits(m, n, k, nf4_gemm.FWD_TILE, cus,
                                       nf4_gemm.forward_split_tiles(k, cus)):
                u += " *"
            elif sweep[m].get("splits", 1) > 1:
                fs += " *"
            else:
                f += " *"
            if not nf4_gemm.fused_fits(m, k, n, nf4_gemm.GRAD_TILE, cus,
                                       nf4_gemm.grad_split_tiles(n, cus)):
                ud += " *"
            elif sweep[m].get("bwd_splits", 1) > 1:
                fds += " *"
            else:
                fd += " *"
            out.append(f"| {label.get(shape, shape)} | {m} | {f} | {fs} | {u} | {fd} | {fds} | "
                       f"{ud} |")
    return "\n".join(out) + "\n"


def summarize_step(trace_csv, title, command, n_layers=28, top=32):
    """Markdown breakdown of one training step from a rocprofv3 --kernel-trace run of bench.py:
    the launches between the first attention forward of one step and that of the next (steps
    with a backward: those holding attn_bwd launches), per kernel, for the step whose GPU busy
    time is the median among the steps of the first work profile timed (bench.py's
    reference-profile steps, which follow, launch more kernels)."""
    rows = sorted(_read_csv(trace_csv), key=lambda r: int(r["Start_Timestamp"]))
    names = [_kernel_base(r["Kernel_Name"]) if "soupk" in r["Kernel_Name"]
             else r["Kernel_Name"].split("(")[0][:90] for r in rows]
    dur = [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in rows]
    firsts = [i for i, n in enumerate(names)
              if n.split("<")[0] == "attn_fwd_kernel"][::n_layers]
    steps = []
    for a, b in zip(firsts, firsts[1:]):
        if any(names[i].startswith("attn_bwd") for i in range(a, b)):
            steps.append((sum(dur[a:b]), a, b))
    if not steps:
        raise ValueError("no forward+backward step in the trace")
    # the work profile: the earliest launch count shared by 3 or more steps (a first step
    # launches a few one-time kernels more)
    counts = [s[2] - s[1] for s in steps]
    launches = next((n for n in counts if counts.count(n) >= 3), counts[0])
    steps = sorted(s for s in steps if s[2] - s[1] == launches)
    busy, a, b = steps[len(steps) // 2]
    per, calls = {}, {}
    for i in range(a, b):
        per[names[i]] = per.get(names[i], 0) + dur[i]
        calls[names[i]] = calls.get(names[i], 0) + 1
    out = [f"# {title}", "", "Command (run from /tmp on the MI355X box, TMPDIR=/tmp):", "", "```",
           command, "```", "",
           f"One forward+backward step (the median of {len(steps)} by GPU busy time): "
           f"{busy / 1e6:.2f} ms of kernel time in {b - a} launches "
           f"({busy / 1e3 / n_layers:.0f} us per layer).", "",
           "| kernel | calls | us per call | us per step | share |", "|---|---:|---:|---:|---:|"]
    for name, t in sorted(per.items(), key=lambda kv: -kv[1])[:top]:
        out.append(f"| `{name}` | {calls[name]} | {t / 1e3 / calls[name]:.1f} | {t / 1e3:.0f} | "
                   f"{100 * t / busy:.1f}% |")
    return "\n".join(out) + "\n"


def summarize_pmc(fetch_csv, write_csv, bench_json, commands):
    """Markdown table of HBM bytes per launch from two rocprofv3 --pmc runs (FETCH_SIZE, then
    WRITE_SIZE; KiB per dispatch), each scaled by what the counter reads for the 1 GiB device
    copy that bench.py's torch_copy_GBps() makes (torch's copy_ -> __amd_rocclr_copyBuffer).  Launches
    are grouped by kernel and grid and named by the bench entry they belong to."""
    bench = json.loads(open(bench_json).read().strip().splitlines()[-1])
    fetch, write = _read_csv(fetch_csv), _read_csv(write_csv)
    gib_kib = float(1 << 20)
    copies = {r["Dispatch_Id"] for r in write if "copyBuffer" in r["Kernel_Name"]
              and float(r["Counter_Value"]) > 0.9 * gib_kib}
    if not copies:
        raise SystemExit("no 1 GiB copy dispatch in the WRITE_SIZE run")
    mean = lambda xs: sum(xs) / len(xs)
    f_copy = mean([float(r["Counter_Value"]) for r in fetch if r["Dispatch_Id"] in copies])
    w_copy = mean([float(r["Counter_Value"]) for r in write if r["Dispatch_Id"] in copies])
    f_scale, w_scale = gib_kib / f_copy, gib_kib / w_copy
    fg, wg = _launch_groups(fetch), _launch_groups(write)
    names = _bench_entries(bench, list(fg))
    out = ["# HBM traffic per launch (rocprofv3 PMC): kernel set at the 2048-token step", "",
           "Commands (run from /tmp on the MI355X box, TMPDIR=/tmp), one counter per pass:", "",
           "```", *commands, "```", "",
           f"Scale factors from the 1 GiB device copy of `bench.py` (`torch_copy_GBps`, "
           f"`__amd_rocclr_copyBuffer`, {len(copies)} dispatches): FETCH_SIZE reads "
           f"{f_copy:.0f} KiB for 1048576 KiB read -> x{f_scale:.4f}; WRITE_SIZE reads "
           f"{w_copy:.0f} KiB for 1048576 KiB written -> x{w_scale:.4f}.", "",
           "traffic = (FETCH_SIZE x fetch scale + WRITE_SIZE x write scale) x 1024 bytes, mean "
           "over dispatches; algorithmic = the compulsory bytes bench.py prices the launch at.  "
           "Launches grouped by kernel and grid (threads / workgroup size).", "",
           "| bench entry | kernel | grid / WG | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | "
           "scaled MB | traffic bytes | algorithmic bytes | traffic / algorithmic |",
           "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for key, rows in fg.items():
        f = [float(r["Counter_Value"]) for r in rows]
        w = [float(r["Counter_Value"]) for r in wg.get(key, [])]
        if not w:
            continue
        t = int(round((mean(f) * f_scale + mean(w) * w_scale) * 1024))
        entry, v = names.get(key, (_unnamed(key[0]), None))
        a = v.get("bytes") if v else None
        ratio = f"{t / a:.3f}" if a else "-"
        out.append(f"| {entry} | `{key[0]}` | {key[1]} / {key[2]} | {len(f)} | {mean(f):.1f} | "
                   f"{mean(w):.1f} | {t / 1e6:.2f} | {t} | {a if a else '-'} | {ratio} |")
    return "\n".join(out) + "\n"


VALU_COUNTERS = ("SQ_WAVES", "SQ_INSTS_VALU", "SQ_WAVE_CYCLES", "SQ_ACTIVE_INST_VALU",
                 "SQ_ACTIVE_INST_ANY", "SQ_WAIT_INST_ANY", "SQ_BUSY_CYCLES", "GRBM_GUI_ACTIVE")


def summarize_valu(raw_csv, busy_csv, bench_json, commands):
    """Markdown table of VALU activity per soupk launch group (kernel, grid) from two rocprofv3
    --pmc runs: the raw SQ counters of VALU_COUNTERS (one pass) and the derived VALUBusy (its
    own pass).  The wave counters are wave-cycle sums (quad-cycles), so their ratios are the
    share of the waves' lifetime spent issuing VALU work, issuing anything, or waiting."""
    bench = json.loads(open(bench_json).read().strip().splitlines()[-1])
    raw, busy = _launch_groups(_read_csv(raw_csv)), _launch_groups(_read_csv(busy_csv))
    names = _bench_entries(bench, list(raw))
    mean = lambda xs: sum(xs) / len(xs) if xs else float("nan")
    out = ["# VALU activity per launch (rocprofv3 PMC): kernel set at the 2048-token step", "",
           "Commands (run from /tmp on the MI355X box, TMPDIR=/tmp), raw counters and the "
           "derived VALUBusy in passes of their own:", "", "```", *commands, "```", "",
           "VALUBusy = 100 x SQ_ACTIVE_INST_VALU / CU_NUM / GRBM_GUI_ACTIVE (rocprofv3's gfx950 "
           "definition).  VALU insts / wave = SQ_INSTS_VALU / SQ_WAVES.  VALU share, issue share "
           "and wait share = SQ_ACTIVE_INST_VALU, SQ_ACTIVE_INST_ANY and SQ_WAIT_INST_ANY over "
           "SQ_WAVE_CYCLES.  Launches grouped by kernel and grid (threads / workgroup size).", "",
           "| bench entry | kernel | grid / WG | dispatches | waves | VALU insts / wave | "
           "VALUBusy % | VALU share of wave cycles | issue share | wait share |",
           "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for key, rows in raw.items():
        c = {}
        for r in rows:
            c.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
        vb = [float(r["Counter_Value"]) for r in busy.get(key, [])
              if r["Counter_Name"] == "VALUBusy"]
        waves, cyc = mean(c.get("SQ_WAVES")), mean(c.get("SQ_WAVE_CYCLES"))
        share = lambda k: f"{mean(c.get(k)) / cyc:.3f}" if cyc else "-"
        entry = names.get(key, (_unnamed(key[0]), None))[0]
        out.append(f"| {entry} | `{key[0]}` | {key[1]} / {key[2]} | "
                   f"{len(c.get('SQ_WAVES', []))} | {waves:.0f} | "
                   f"{mean(c.get('SQ_INSTS_VALU')) / waves:.0f} | {mean(vb):.1f} | "
                   f"{share('SQ_ACTIVE_INST_VALU')} | {share('SQ_ACTIVE_INST_ANY')} | "
                   f"{share('SQ_WAIT_INST_ANY')} |")
    return "\n".join(out) + "\n"


# Counter passes of the attention profile (each within one pass's hardware limits: at most 8
# SQ counters, derived counters counted by the raw counters they read).
ATTN_PMC_PASSES = (
    "SQ_WAVES SQ_WAVE_CYCLES SQ_INSTS_VALU SQ_INSTS_MFMA SQ_INSTS_LDS SQ_INSTS_SALU "
    "SQ_INSTS_VMEM SQ_INSTS_VALU_TRANS_F32",
    "MfmaUtil LdsUtil LdsBankConflict VALUBusy SQ_ACTIVE_INST_LDS SQ_WAIT_INST_LDS "
    "SQ_ACTIVE_INST_ANY SQ_WAIT_INST_ANY",
    "MeanOccupancyPerActiveCU OccupancyPercent SQ_VALU_MFMA_COEXEC_CYCLES "
    "SQ_INSTS_LDS_LOAD_BANDWIDTH SQ_INSTS_LDS_STORE_BANDWIDTH",
)


def attn_block_steps(lengths, n_heads, block=64):
    """(forward, backward) key-block steps of the varlen attention over sequences of the given
    lengths: a forward workgroup of query block i walks key blocks 0..i, so a sequence of nb
    blocks takes nb(nb+1)/2 per head; the backward's dQ workgroups walk the same pairs and its
    dK/dV workgroups (key block j over query blocks j..nb-1) as many again."""
    per_head = sum((n + block - 1) // block * ((n + block - 1) // block + 1) // 2
                   for n in lengths)
    return n_heads * per_head, 2 * n_heads * per_head


def summarize_attn_pmc(a_csv, b_csv, c_csv, bench_json, commands):
    """Markdown table of the varlen attention kernels' counters (three rocprofv3 --pmc runs of
    `bench.py --attention`): per launch group (kernel, grid), the instruction mix per key-block
    step of a wavefront, the pipes' utilisation and the occupancy.  A kernel's groups are taken
    in dispatch order: the 2048-token case, then the ragged batch (bench.py times them so)."""
    bench = json.loads(open(bench_json).read().strip().splitlines()[-1])["attention"]
    shape = bench["shape"]
    NH, B, T = shape["q_heads"], shape["batch"], shape["seq"]
    cases = (("2048 tokens", [T] * B, ""), ("ragged", shape["ragged_lengths"], "ragged_"))
    passes = [_launch_groups(_read_csv(f)) for f in (a_csv, b_csv, c_csv)]
    mean = lambda xs: sum(xs) / len(xs) if xs else float("nan")
    seen = {}
    out = ["# Varlen attention counters (rocprofv3 PMC): the layer's kernels at 2048 tokens and "
           "the ragged batch", "",
           "Commands (run from /tmp on the MI355X box, TMPDIR=/tmp), one pass each:", "", "```",
           *commands, "```", "",
           "Per launch group (kernel, grid = threads / workgroup size), means over dispatches.  "
           "Per-step figures divide a wave counter by 4 wavefronts x the key-block steps the "
           "launch performs (forward: a query block of nb blocks walks its causal key blocks, "
           "nb(nb+1)/2 per sequence and head; backward: as many dQ steps again as dK/dV steps); "
           "they include each workgroup's set-up and epilogue and the idle slots of the grid.  "
           "MfmaUtil = MFMA busy cycles / (GPU cycles x SIMDs); LdsUtil = LDS indexed-active "
           "cycles / (GPU cycles x CUs); LdsBankConflict = conflict cycles per active cycle; "
           "VALUBusy as rocprofv3 defines it; LDS issue / wait share = SQ_ACTIVE_INST_LDS / "
           "SQ_WAIT_INST_LDS over SQ_ACTIVE_INST_ANY + SQ_WAIT_INST_ANY; occupancy: "
           "MeanOccupancyPerActiveCU (waves per busy CU) and OccupancyPercent; LDS KB per step: "
           "SQ_INSTS_LDS_LOAD_BANDWIDTH / _STORE_BANDWIDTH (64-byte units).", "",
           "| case | kernel | grid / WG | µs (bench) | waves | key-block steps | VALU / step | "
           "MFMA / step | LDS instr / step | LDS KB read / step | LDS KB written / step | "
           "exp / step | VALUBusy % | MfmaUtil % | LdsUtil % | LdsBankConflict | "
           "LDS issue / wait share | waves per busy CU | occupancy % |",
           "|---|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"
           "---:|---:|"]
    for key, rows in passes[0].items():
        kern = key[0].split("<")[0]
        i = seen.get(kern, 0)
        seen[kern] = i + 1
        if i >= len(cases) or not kern.startswith("attn_"):
            continue
        label, lengths, tag = cases[i]
        fwd_steps, bwd_steps = attn_block_steps(lengths, NH)
        steps = fwd_steps if kern == "attn_fwd_kernel" else bwd_steps
        us = (bench.get(f"{tag}varlen_fwd", {}).get("us") if kern == "attn_fwd_kernel" else
              bench.get(f"{tag}varlen_bwd", {}).get("us") if kern == "attn_bwd_kernel" else None)
        c = {}
        for p_ in passes:
            for r in p_.get(key, []):
                c.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
        m = {k: mean(v) for k, v in c.items()}
        per = lambda k: f"{m[k] / (4 * steps):.0f}" if k in m and kern != "attn_bwd_delta_kernel" \
            and kern != "attn_bwd_reduce_varlen_kernel" else "-"
        kb = lambda k: (f"{m[k] * 64 / 1024 / (4 * steps):.1f}" if k in m and per(k) != "-"
                        else "-")
        busy = m.get("SQ_ACTIVE_INST_ANY", 0) + m.get("SQ_WAIT_INST_ANY", 0)
        share = (f"{m.get('SQ_ACTIVE_INST_LDS', 0) / busy:.3f} / "
                 f"{m.get('SQ_WAIT_INST_LDS', 0) / busy:.3f}") if busy else "-"
        f = lambda k, d=1: f"{m[k]:.{d}f}" if k in m else "-"
        out.append(
            f"| {label} | `{key[0]}` | {key[1]} / {key[2]} | {us if us is not None else '-'} | "
            f"{f('SQ_WAVES', 0)} | {steps if per('SQ_INSTS_VALU') != '-' else '-'} | "
            f"{per('SQ_INSTS_VALU')} | {per('SQ_INSTS_MFMA')} | {per('SQ_INSTS_LDS')} | "
            f"{kb('SQ_INSTS_LDS_LOAD_BANDWIDTH')} | {kb('SQ_INSTS_LDS_STORE_BANDWIDTH')} | "
            f"{per('SQ_INSTS_VALU_TRANS_F32')} | {f('VALUBusy')} | {f('MfmaUtil')} | "
            f"{f('LdsUtil')} | {f('LdsBankConflict', 3)} | {share} | "
            f"{f('MeanOccupancyPerActiveCU', 2)} | {f('OccupancyPercent')} |")
    return "\n".join(out) + "\n"


def median(xs):
    s = sorted(xs)
    n = len(s)
    return s[n // 2] if n % 2 else 0.5 * (s[n // 2 - 1] + s[n // 2])


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-layer", action="store_true", help="skip the whole-layer timing")
    ap.add_argument("--no-step", action="store_true",
                    help="skip the whole-model training-step timing")
    ap.add_argument("--heuristic-gemms", action="store_true",
                    help="keep hipBLASLt's heuristic choice for every GEMM (no tuned table)")
    ap.add_argument("--summarize-stats", nargs=3, metavar=("TRACE_CSV", "BENCH_JSON", "CMD"),
                    help="print a markdown summary of a rocprofv3 --kernel-trace run beside "
                         "bench.py's timing and exit (CPU)")
    ap.add_argument("--summarize-pmc", nargs=5,
                    metavar=("FETCH_CSV", "WRITE_CSV", "BENCH_JSON", "CMD1", "CMD2"),
                    help="print the HBM traffic table of two rocprofv3 --pmc runs and exit (CPU)")
    ap.add_argument("--summarize-valu", nargs=5,
                    metavar=("RAW_CSV", "BUSY_CSV", "BENCH_JSON", "CMD1", "CMD2"),
                    help="print the VALU activity table of two rocprofv3 --pmc runs and exit "
                         "(CPU)")
    ap.add_argument("--summarize-kernels", nargs=3, metavar=("STATS_CSV", "TITLE", "CMD"),
                    help="print every kernel of a rocprofv3 --stats run by total time (CPU)")
    ap.add_argument("--attention", action="store_true",
                    help="time only the layer's varlen attention kernels (forward, backward; "
                         "2048 real tokens and the ragged batch), print one JSON line and exit")
    ap.add_argument("--summarize-attn-pmc", nargs=7,
                    metavar=("A_CSV", "B_CSV", "C_CSV", "BENCH_JSON", "CMD1", "CMD2", "CMD3"),
                    help="print the attention counter table of three rocprofv3 --pmc runs of "
                         "bench.py --attention and exit (CPU)")
    ap.add_argument("--nf4-gemm", action="store_true",
                    help="time the fused NF4-dequant GEMM against hipBLASLt and unpack + "
                         "hipBLASLt at M = 2048, print one JSON line and exit")
    ap.add_argument("--nf4-resident", action="store_true",
                    help="time the decoder layer at few tokens on its NF4 weights (the fused "
                         "NF4-dequant GEMM) against unpacked weights + hipBLASLt, then exit")
    ap.add_argument("--nf4-resident-wide", action="store_true",
                    help="the --nf4-resident comparison at 256-1024 tokens, the layer forced "
                         "onto its NF4 weights")
    ap.add_argument("--summarize-nf4-resident", nargs=3,
                    metavar=("TRACE_CSV", "BENCH_JSON", "CMD"),
                    help="print the per-step kernel table of a kernel trace of --nf4-resident")
    ap.add_argument("--summarize-nf4-gemm", nargs=3, metavar=("TRACE_CSV", "BENCH_JSON", "CMD"),
                    help="print the fused NF4 GEMM tables of a rocprofv3 --kernel-trace run of "
                         "bench.py --nf4-gemm and exit (CPU)")
    ap.add_argument("--summarize-trace", nargs=3, metavar=("TRACE_CSV", "TITLE", "CMD"),
                    help="print every launch group (kernel, grid) of a rocprofv3 "
                         "--kernel-trace run (CPU)")
    ap.add_argument("--summarize-step", nargs=3, metavar=("TRACE_CSV", "TITLE", "CMD"),
                    help="print the per-kernel breakdown of one training step of a rocprofv3 "
                         "--kernel-trace run (CPU)")
    args = ap.parse_args()
    if args.summarize_nf4_resident:
        a = args.summarize_nf4_resident
        sys.stdout.write(summarize_nf4_resident(a[0], a[1], a[2]))
        return
    if args.summarize_nf4_gemm:
        a = args.summarize_nf4_gemm
        sys.stdout.write(summarize_nf4_gemm(a[0], a[1], a[2]))
        return
    if args.summarize_attn_pmc:
        a = args.summarize_attn_pmc
        sys.stdout.write(summarize_attn_pmc(a[0], a[1], a[2], a[3], a[4:]))
        return
    if args.summarize_valu:
        a = args.summarize_valu
        sys.stdout.write(summarize_valu(a[0], a[1], a[2], a[3:]))
        return
    if args.summarize_step:
        sys.stdout.write(summarize_step(*args.summarize_step))
        return
    if args.summarize_trace:
        sys.stdout.write(summarize_trace(*args.summarize_trace))
        return
    if args.summarize_kernels:
        sys.stdout.write(summarize_kernels(*args.summarize_kernels))
        return
    if args.summarize_stats:
        sys.stdout.write(summarize_stats(*args.summarize_stats))
        return
    if args.summarize_pmc:
        a = args.summarize_pmc
        sys.stdout.write(summarize_pmc(a[0], a[1], a[2], a[3:]))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the kernel set has no cross-GPU exchange and this "
              "build runs no multi-GPU configuration (a data-parallel run would all-reduce the "
              "LoRA gradients once per step; it is not implemented here).",
              file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        sys.exit(1)
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    _ext.lib()
    # Backward on this thread, as testt_amd.apply() sets it for the training thread.
    testt_amd.configure_backward()
    gemm_table = None
    if not args.heuristic_gemms:
        from testt_amd import gemm_tuning

        accepted = gemm_tuning.enable()
        gemm_table = {"table": os.path.relpath(gemm_tuning.RESULTS, ROOT), "accepted": accepted}
        log(f"tuned hipBLASLt solutions ({gemm_table['table']}): "
            f"{'replayed' if accepted else 'rejected by TunableOp, heuristic choices'}")
    if args.attention:
        print(json.dumps({"attention": time_attention(dev, args.steps, args.warmup,
                                                      varlen_only=True),
                          "timing": "GPU time per call: calls queued behind a device-side "
                                    "wait and timed as one span"}), flush=True)
        return
    if args.nf4_resident_wide:
        print(json.dumps({"nf4_resident_layer_wide": time_nf4_resident_wide(dev),
                          "gemm_selection": gemm_table}), flush=True)
        return
    if args.nf4_resident:
        print(json.dumps({"nf4_resident_layer": time_nf4_resident(dev),
                          "nf4_resident_trace": trace_nf4_resident(dev),
                          "gemm_selection": gemm_table}), flush=True)
        return
    if args.nf4_gemm:
        print(json.dumps({"nf4_gemm": time_nf4_gemm(dev), "gemm_selection": gemm_table,
                          "timing": "GPU time per call: calls queued behind a device-side "
                                    "wait and timed as one span"}), flush=True)
        return
    log("building inputs")
    cases = build_cases(dev)
    torch.cuda.synchronize(dev)
    log(f"timing {len(cases)} kernels: warmup {args.warmup}, steps {args.steps}")
    host_enqueue, span = time_gpu(cases, args.steps, args.warmup, dev)
    extra = build_extra_cases(dev)
    time_gpu(extra, args.steps, args.warmup, dev)
    shapes = build_shape_cases(dev)
    log(f"timing {len(shapes)} kernels of the set at the ragged / product-chunk shapes")
    time_gpu(shapes, args.steps, args.warmup, dev)
    floor = build_floor_cases(dev)
    time_gpu(floor, args.steps, args.warmup, dev)
    copy_gbps = copy_peak(dev)
    torch_copy_gbps = torch_copy_GBps(dev)
    copy_us = copy_reference(cases, dev)
    attn_t = None
    if not args.no_layer:
        log("timing the causal GQA attention kernels at the layer's shape")
        attn_t = time_attention(dev, 50, 5)
        log(f"attention fwd {attn_t['fwd']['us']} us, bwd {attn_t['bwd']['us']} us (padded); "
            f"varlen fwd {attn_t['varlen_fwd']['us']} us, bwd {attn_t['varlen_bwd']['us']} us; "
            f"ragged varlen fwd {attn_t['ragged_varlen_fwd']['us']} / bwd "
            f"{attn_t['ragged_varlen_bwd']['us']} us against padded "
            f"{attn_t['ragged_fwd']['us']} / {attn_t['ragged_bwd']['us']} us")
    step_t = step_ref = None
    if not args.no_step:
        log("timing one training step of the 28-layer model at 2048 tokens")
        step_t = time_step(dev, 10, 3)
        log(f"step fwd {step_t['fwd_ms']} ms (median {step_t['fwd_ms_median']}), fwd+bwd "
            f"{step_t['fwd_bwd_ms']} ms (median {step_t['fwd_bwd_ms_median']}), "
            f"{step_t['tokens_per_s']} tokens/s")
        step_ref = time_step(dev, 5, 2, reference_profile=True)
        log(f"step, reference work profile: fwd+bwd {step_ref['fwd_bwd_ms']} ms (median "
            f"{step_ref['fwd_bwd_ms_median']})")
    # Last: the layer timing captures HIP graphs, and eager work of the same process measured
    # after a capture ran slower (the 28-layer step: 36 ms against 25 ms before it); the
    # reference-profile layer (no capture) runs before it.
    layer_t = layer_ref = layer_ragged = layer_nf4 = None
    if not args.no_layer:
        log("timing one decoder layer fwd+bwd at 2048 tokens")
        n_layer_steps = max(50, min(100, args.steps // 3))
        layer_ragged = time_layer(dev, n_layer_steps, 5, lengths=(512, 152, 128, 96))
        log(f"layer at the ragged batch (M = {layer_ragged['tokens']}): fwd "
            f"{layer_ragged['fwd_us']} us, fwd+bwd {layer_ragged['fwd_bwd_us']} us (median "
            f"{layer_ragged['fwd_bwd_us_median']})")
        layer_ref = time_layer(dev, n_layer_steps, 5, reference_profile=True)
        log(f"layer, reference work profile: fwd {layer_ref['fwd_us']} us, fwd+bwd "
            f"{layer_ref['fwd_bwd_us']} us (median {layer_ref['fwd_bwd_us_median']})")
        layer_t = time_layer(dev, n_layer_steps, 5)
        # the HIP-graph replays after every eager timing
        layer_t.update(graph_layer(dev, n_layer_steps))
        layer_ragged.update(graph_layer(dev, n_layer_steps, lengths=(512, 152, 128, 96)))
        log(f"layer fwd {layer_t['fwd_us']} us (median {layer_t['fwd_us_median']}), fwd+bwd "
            f"{layer_t['fwd_bwd_us']} us (median {layer_t['fwd_bwd_us_median']}) (eager); "
            f"graph-replayed fwd {layer_t['graph_fwd_us']} us, fwd+bwd "
            f"{layer_t['graph_fwd_bwd_us']} us; ragged graph-replayed fwd+bwd "
            f"{layer_ragged['graph_fwd_bwd_us']} us")
        layer_nf4 = time_nf4_resident(dev)
    kernels = {}
    total_us = 0.0
    total_bytes = 0
    for c in cases:
        mean_us = sum(c.times) / len(c.times)
        total_us += mean_us
        total_bytes += c.nbytes
        gbps = c.nbytes / (mean_us * 1e-6) / 1e9
        kernels[c.name] = {"kernel": c.kernel, "us_mean": round(mean_us, 3),
                           "us_median": round(median(c.times), 3),
                           "us_min": round(min(c.times), 3), "bytes": c.nbytes,
                           "input_sets": len(c.sets),
                           "GBps": round(gbps, 1), "frac_of_peak": round(gbps / PEAK_HBM_GBPS, 4),
                           "copy_us": round(copy_us[c.name], 3),
                           "copy_over_kernel": round(copy_us[c.name] / mean_us, 3)}
        log(f"{c.name:16s} {mean_us:8.2f} us  {gbps:8.1f} GB/s  "
            f"{100 * gbps / PEAK_HBM_GBPS:5.1f}% of 8 TB/s  (same-size copy "
            f"{copy_us[c.name]:6.2f} us)")
    beyond = {}
    for c in extra:
        mean_us = sum(c.times) / len(c.times)
        gbps = c.nbytes / (mean_us * 1e-6) / 1e9
        beyond[c.name] = {"kernel": c.kernel, "us_mean": round(mean_us, 3),
                          "us_median": round(median(c.times), 3), "bytes": c.nbytes,
                          "input_sets": len(c.sets),
                          "GBps": round(gbps, 1), "frac_of_peak": round(gbps / PEAK_HBM_GBPS, 4)}
        log(f"{c.name:16s} {mean_us:8.2f} us  {gbps:8.1f} GB/s  "
            f"{100 * gbps / PEAK_HBM_GBPS:5.1f}% of 8 TB/s  (beyond the set)")
    other_shapes = {}
    for c in shapes:
        mean_us = sum(c.times) / len(c.times)
        gbps = c.nbytes / (mean_us * 1e-6) / 1e9
        other_shapes[c.name] = {"kernel": c.kernel, "entry": c.entry,
                                "us_mean": round(mean_us, 3),
                                "us_median": round(median(c.times), 3), "bytes": c.nbytes,
                                "input_sets": len(c.sets), "GBps": round(gbps, 1),
                                "frac_of_peak": round(gbps / PEAK_HBM_GBPS, 4)}
        log(f"{c.name:24s} {mean_us:8.2f} us  {gbps:8.1f} GB/s  "
            f"{100 * gbps / PEAK_HBM_GBPS:5.1f}% of 8 TB/s")
    launch_floor = {c.name: round(median(c.times), 3) for c in floor}
    launch_floor["note"] = ("median duration of launches timed exactly as the kernels are "
                            "(dispatch-recorded events, back to back): an empty kernel of 1 and "
                            "of 1024 workgroups x 256 threads, and a 4 KiB device copy; the "
                            "fixed cost of any launch on this GPU")
    log(f"launch floor: empty 1 WG {launch_floor['empty_kernel_1wg']} us, 1024 WG "
        f"{launch_floor['empty_kernel_1024wg']} us, 4 KiB copy {launch_floor['copy_4KiB']} us")
    dom = max(cases, key=lambda c: sum(c.times))
    dom_us = sum(dom.times) / len(dom.times)
    dom_gbps = dom.nbytes / (dom_us * 1e-6) / 1e9
    roofline = {"kernel": dom.kernel, "bound": "hbm", "achieved": round(dom_gbps, 1),
                "peak": PEAK_HBM_GBPS, "unit": "GB/s", "frac": round(dom_gbps / PEAK_HBM_GBPS, 4),
                "traffic": pmc_traffic(dom.name), "algorithmic_bytes": dom.nbytes,
                "traffic_source": os.path.relpath(TRAFFIC_TABLE, ROOT)}
    cpu = None
    if not args.no_cpu:
        log(f"CPU baseline (~{args.cpu_seconds:.0f} s)")
        cpu = cpu_baseline(cases, args.cpu_seconds)
    value = total_bytes / (total_us * 1e-6) / 1e9
    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(total_us / 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic",
        "config": {"workload": "solution/ kernel set fwd+bwd at the 2048-token step of "
                               "Qwen2.5-1.5B (nf4 gate|up unpack, add+RMSNorm fwd/bwd, "
                               "LoRA+RoPE+QKV pack fwd/bwd, SwiGLU fwd/in-place bwd, vocab-head "
                               "stats+grad on one 256x151936 chunk)",
                   "tokens": 2048, "hidden": workloads.HIDDEN, "intermediate": workloads.INTER,
                   "vocab": workloads.VOCAB, "storage": "fp16/fp32, math fp32"},
        "value_definition": "sum of compulsory HBM bytes of the 8 kernels / sum of their mean "
                            "HIP-event durations",
        "kernels": kernels,
        "kernels_beyond_set": beyond,
        "kernels_other_shapes": other_shapes,
        "launch_floor_us": launch_floor,
        "layer": layer_t,
        "layer_reference_profile": layer_ref,
        "layer_ragged": layer_ragged,
        "layer_nf4_resident": layer_nf4,
        "attention": attn_t,
        "gemm_selection": gemm_table or "hipBLASLt heuristic (--heuristic-gemms)",
        "step": step_t,
        "step_reference_profile": step_ref,
        "copy_peak_GBps": copy_gbps,
        "torch_copy_GBps": torch_copy_gbps,
        "copy_reference": "kernels[*].copy_us: a plain 16-byte streaming device copy "
                          "(one chunk per thread, non-temporal load, nt|sc1 store) "
                          "(soupk_bench_copy) moving the kernel's algorithmic bytes, half read "
                          "and half written, timed the same way; copy_over_kernel = copy_us / "
                          "us_mean",
        "timing": "per-launch HIP events recorded by the kernel dispatch itself "
                  "(soupk_time_next_launch / hipExtLaunchKernelGGL), mean over steps; the "
                  "launches run back to back, queued behind a device-side wait (DeviceHold)",
        "step_gpu_span_ms": round(span * 1e3 / args.steps, 4),
        "host_enqueue_ms": round(host_enqueue * 1e3 / args.steps, 4),
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
