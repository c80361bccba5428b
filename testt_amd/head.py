"""The output head and everything Soup computes from its logits, without full logits, on gfx950.
Drop-in for solution/head.py (same names, signatures, constants and outputs).

Design.  The rows (real tokens) are taken in their own order, CHUNK_ROWS at a time:
1. hipBLASLt (torch.matmul): logits = h @ W^T for the chunk, fp16;
2. testt_amd/csrc/head_stats.hip, one 1024-thread workgroup per row: the online statistics
   (running max, sum of exp, sum of exp * z and the first argmax, which give logsumexp,
   entropy = lse - sum(p z), the token loss lse - z[label] and whether the argmax is the label),
   stored straight at the row's place in the outputs, and for a labelled row the gradient
   (softmax - onehot) * scale in fp16, written to the row's slot in a buffer that holds only the
   chunk's labelled rows (the slot comes from a row map, -1 for an ignored row);
3. hipBLASLt: dh = that buffer @ W, appended to one packed [labelled, H] gradient.
The row map and the per-chunk labelled counts come from one cumulative sum over the labels and
one host synchronisation (the counts size the dh GEMMs).  No row is ever permuted: the hidden
states are read in place, the statistics need no unsort, and the backward forms the [M, H]
gradient in one gather from the packed rows (an appended zero row serves the ignored ones),
scaled by the loss scale on the way.  The gradient is taken in the forward because the head is
frozen.

CHUNK_ROWS keeps the reference's name; its value is MI355X's: the reference's 256 rows bound
the logits buffer on a 15 GB card (78 MB), while 2048 rows (622 MB, plus the labelled rows'
gradient buffer, of 288 GB) let the two chunk GEMMs run at a size hipBLASLt handles efficiently
(the head's forward + backward at 2048 tokens: 2.2 ms against 4.6 ms in 256-row chunks).
Every row's statistics and gradient are computed from that row alone, so no output depends on
the chunking.
"""

import math

import torch

from . import _ext

CHUNK_ROWS = 2048
# Vocabulary tile of the reference's Triton loop (solution/head.py:30); the HIP kernel streams
# a row in 16-byte chunks with 1024 threads instead, so this is kept only as a public name.
VOCAB_BLOCK = 4096
IGNORE_INDEX = -100


def head_stats_grad(logits, targets, entropy, token_loss, correct, grad_scale, lse=None):
    """Launch the per-row statistics + in-place gradient kernel on a [rows, V] fp16 chunk.

    entropy / token_loss (fp32), correct (int32) and lse (fp32, optional) receive one value per
    row; logits of labelled rows are overwritten with fp16((softmax - onehot) * grad_scale)."""
    _ext.require(logits, "logits", dtype=torch.float16, ndim=2)
    rows, vocab = logits.shape
    dev = logits.device
    _ext.require(targets, "targets", dtype=torch.int64, ndim=1, device=dev)
    for t, name, dt in ((entropy, "entropy", torch.float32), (token_loss, "token_loss",
                        torch.float32), (correct, "correct", torch.int32)):
        _ext.require(t, name, dtype=dt, device=dev)
        if t.numel() < rows:
            raise ValueError(f"{name} holds {t.numel()} values for {rows} rows")
    if targets.numel() < rows:
        raise ValueError(f"targets holds {targets.numel()} values for {rows} rows")
    if lse is not None:
        _ext.require(lse, "lse", dtype=torch.float32, device=dev)
        if lse.numel() < rows:
            raise ValueError(f"lse holds {lse.numel()} values for {rows} rows")
    if rows:
        _ext.call("soupk_head_stats_grad", _ext.ptr(logits), _ext.ptr(targets),
                  _ext.ptr(entropy), _ext.ptr(token_loss), _ext.ptr(correct), _ext.ptr(lse),
                  float(grad_scale), rows, vocab, _ext.stream_of(logits))


def _grad_unit(denominator):
    """A power of two G with G / denominator about 64: the fp16 head gradient is held at the
    magnitude base Soup's GradScaler gives it (65536 / tokens), and rescaling by a power of two
    is exact (solution/head.py:79-84)."""
    exponent = int(round(math.log2(max(float(denominator), 1e-6)))) + 6
    return float(2 ** max(0, min(16, exponent)))


def head_stats_grad_rows(logits, targets, grad_row, grad_out, entropy, token_loss, correct,
                         grad_scale, lse=None):
    """head_stats_grad with the gradient of labelled row r written to row grad_row[r] of
    grad_out (a [n, V] fp16 buffer; entries outside [0, n) write nothing), the logits left as
    they are.  grad_row and grad_out both None: statistics only."""
    _ext.require(logits, "logits", dtype=torch.float16, ndim=2)
    rows, vocab = logits.shape
    dev = logits.device
    _ext.require(targets, "targets", dtype=torch.int64, ndim=1, device=dev)
    outs = [(entropy, "entropy", torch.float32), (token_loss, "token_loss", torch.float32),
            (correct, "correct", torch.int32), (targets, "targets", torch.int64)]
    if lse is not None:
        outs.append((lse, "lse", torch.float32))
    for t, name, dt in outs:
        _ext.require(t, name, dtype=dt, device=dev)
        if t.numel() < rows:
            raise ValueError(f"{name} holds {t.numel()} values for {rows} rows")
    if (grad_row is None) != (grad_out is None):
        raise ValueError("grad_row and grad_out go together")
    n_out = 0
    if grad_out is not None:
        _ext.require(grad_row, "grad_row", dtype=torch.int32, ndim=1, device=dev)
        _ext.require(grad_out, "grad_out", dtype=torch.float16, ndim=2, device=dev)
        if grad_row.numel() < rows or grad_out.shape[1] != vocab:
            raise ValueError(f"grad_row ({grad_row.numel()}) / grad_out {tuple(grad_out.shape)}"
                             f" do not fit {rows} rows of {vocab}")
        n_out = grad_out.shape[0]
    if rows:
        _ext.call("soupk_head_stats_grad_rows", _ext.ptr(logits), _ext.ptr(targets),
                  _ext.ptr(grad_row), _ext.ptr(grad_out), n_out, _ext.ptr(entropy),
                  _ext.ptr(token_loss), _ext.ptr(correct), _ext.ptr(lse), float(grad_scale),
                  rows, vocab, _ext.stream_of(logits))


class _RowPlan:
    """Where each row's gradient goes, and the sizes the host needs, from one pass over the
    labels and one synchronisation.

    slot:     int32 [M], for a labelled row its index among the labelled rows of its chunk,
              -1 for an ignored row (the kernel's row map);
    gather:   int64 [M], for a labelled row its index among all labelled rows, n_labelled for
              an ignored row (the row of zeros appended in backward);
    counts:   labelled rows per chunk (host ints); n_labelled, denominator (host numbers)."""

    def __init__(self, targets, denominator, chunk):
        rows = targets.numel()
        dev = targets.device
        labelled = targets != IGNORE_INDEX
        seen = torch.cumsum(labelled, 0, dtype=torch.int32)       # labelled rows up to here
        n_chunks = -(-rows // chunk)
        ends = torch.arange(1, n_chunks + 1, device=dev) * chunk
        ends.clamp_(max=rows)
        at_end = seen.index_select(0, ends - 1).to(torch.float64)
        den = denominator.to(device=dev, dtype=torch.float64).reshape(1) \
            if torch.is_tensor(denominator) else None
        host = (torch.cat([at_end, den]) if den is not None else at_end).tolist()
        cum = [int(v) for v in host[:n_chunks]]
        self.denominator = host[n_chunks] if den is not None else float(denominator)
        self.n_labelled = cum[-1]
        starts = [0] + cum[:-1]
        self.counts = [b - a for a, b in zip(starts, cum)]
        self.lab_before = starts
        chunk_base = torch.tensor(starts, dtype=torch.int32, device=dev)
        base = chunk_base.repeat_interleave(chunk)[:rows]
        self.slot = torch.where(labelled, seen - 1 - base, -1).to(torch.int32)
        self.gather = torch.where(labelled, (seen - 1).to(torch.int64), self.n_labelled)


class FusedHeadLoss(torch.autograd.Function):
    """(loss, entropy [M], token loss [M], correct [M]) of the frozen head over `hidden`
    (solution/head.py:87-137's interface); the gradient for `hidden` is computed in forward."""

    @staticmethod
    def forward(ctx, hidden, weight, targets, denominator):
        rows, width = hidden.shape
        vocab = weight.shape[0]
        dev = hidden.device
        targets = targets.to(torch.int64).contiguous()
        entropy = torch.empty(rows, dtype=torch.float32, device=dev)
        token_loss = torch.empty(rows, dtype=torch.float32, device=dev)
        correct = torch.empty(rows, dtype=torch.int32, device=dev)
        want_grad = ctx.needs_input_grad[0]
        if rows == 0:
            denom = float(denominator.item()) if torch.is_tensor(denominator) \
                else float(denominator)
            plan = None
            unit = _grad_unit(denom)
            packed = torch.empty((0, width), dtype=torch.float16, device=dev)
        else:
            plan = _RowPlan(targets, denominator, CHUNK_ROWS)
            denom = plan.denominator
            unit = _grad_unit(denom)
            packed = torch.empty((plan.n_labelled if want_grad else 0, width),
                                 dtype=torch.float16, device=dev)
        scale = unit / max(denom, 1e-6)
        for c, start in enumerate(range(0, rows, CHUNK_ROWS)):
            stop = min(rows, start + CHUNK_ROWS)
            logits = torch.matmul(hidden[start:stop], weight.t())
            n_lab = plan.counts[c] if want_grad else 0
            if n_lab and (2 * vocab) % 16:
                # A row pitch of part of a 16-byte chunk: the kernel cannot give gradient rows
                # the logits rows' alignment, so it writes in place and the labelled rows are
                # gathered (vocabularies of a multiple of 8 entries never come here).
                head_stats_grad(logits, targets[start:stop], entropy[start:stop],
                                token_loss[start:stop], correct[start:stop], scale)
                g = logits.index_select(0, torch.nonzero(plan.slot[start:stop] >= 0)[:, 0])
            else:
                g = torch.empty((n_lab, vocab), dtype=torch.float16, device=dev) \
                    if n_lab else None
                head_stats_grad_rows(logits, targets[start:stop],
                                     plan.slot[start:stop] if n_lab else None, g,
                                     entropy[start:stop], token_loss[start:stop],
                                     correct[start:stop], scale)
            del logits
            if n_lab:
                first = plan.lab_before[c]
                torch.matmul(g, weight, out=packed[first:first + n_lab])
            del g
        total = token_loss.sum()
        loss = total / (denominator.to(dev) if torch.is_tensor(denominator) else denominator)
        ctx.unit = unit
        if want_grad:
            ctx.save_for_backward(packed, plan.gather if plan is not None else None)
        stats = (entropy, token_loss, correct.bool())
        ctx.mark_non_differentiable(*stats)
        return (loss, *stats)

    @staticmethod
    def backward(ctx, grad_loss, *_unused):
        if not ctx.needs_input_grad[0]:
            return None, None, None, None
        packed, gather = ctx.saved_tensors
        factor = grad_loss.to(torch.float32) / ctx.unit
        if gather is None:
            return packed.new_empty((0, packed.shape[1])), None, None, None
        # The packed rows scaled by the loss scale, one row of zeros appended for the ignored
        # rows, then every row of hidden takes its row: one gather forms [M, H].
        scaled = torch.cat([packed, packed.new_zeros((1, packed.shape[1]))]).to(torch.float32)
        scaled = (scaled * factor).to(torch.float16)
        return scaled.index_select(0, gather), None, None, None


def fused_head_loss(hidden16, weight16, targets, denominator):
    """(loss, token entropy [M], token loss [M], token correct [M]) for rows of `hidden16`.

    `targets[i]` is the label row i predicts (IGNORE_INDEX for none); `denominator` is what
    the summed loss is divided by (num_items_in_batch, or the labelled count)."""
    if not hidden16.is_cuda:
        raise ValueError("fused_head_loss: hidden16 must be a HIP device tensor (no CPU path)")
    return FusedHeadLoss.apply(hidden16.contiguous(), weight16, targets.contiguous(), denominator)
