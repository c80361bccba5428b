"""The output head and everything Soup computes from its logits, without full logits, on gfx950.
Drop-in for solution/head.py.

The head runs over the real (non-pad) tokens in chunks of CHUNK_ROWS rows, labelled rows first:
1. hipBLASLt (torch.matmul): logits = h @ W^T for the chunk, fp16;
2. testt_amd/csrc/head_stats.hip, one 1024-thread workgroup per row: the online statistics
   (running max, sum of exp, sum of exp * z and the first argmax, which give logsumexp,
   entropy = lse - sum(p z), the token loss lse - z[label] and whether the argmax is the label)
   and, for labelled rows, the gradient (softmax - onehot) * scale in fp16 written over the
   logits in place -- one read of the row from HBM when it fits the CU's registers;
3. hipBLASLt: dh = dlogits @ W for the labelled rows of the chunk.
The gradient is taken in forward (the head is frozen) and scaled by the loss scale in backward.

CHUNK_ROWS keeps the reference's name; its value is MI355X's: the reference's 256 rows bound
the logits buffer on a 15 GB card (78 MB), while 2048 rows (622 MB of 288 GB) let the two
chunk GEMMs run at a size hipBLASLt handles efficiently (the head's forward + backward at 2048
tokens: 2.2 ms against 4.6 ms in 256-row chunks).  Every row's result is independent of the
chunking.
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


class FusedHeadLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, hidden, weight, targets, denominator):
        rows, width = hidden.shape
        vocab = weight.shape[0]
        dev = hidden.device
        targets = targets.to(torch.int64)
        labelled = targets != IGNORE_INDEX
        order = torch.argsort((~labelled).to(torch.int8), stable=True)
        n_labelled, denom = _host_counts(labelled, denominator, dev)
        h = hidden.index_select(0, order)
        tgt = targets.index_select(0, order).contiguous()
        entropy = torch.empty(rows, dtype=torch.float32, device=dev)
        token_loss = torch.empty(rows, dtype=torch.float32, device=dev)
        correct = torch.empty(rows, dtype=torch.int32, device=dev)
        want_grad = ctx.needs_input_grad[0]
        unit = _grad_unit(denom)
        grad_sorted = torch.empty((n_labelled, width), dtype=torch.float16, device=dev) \
            if want_grad else None
        for start in range(0, rows, CHUNK_ROWS):
            stop = min(rows, start + CHUNK_ROWS)
            logits = torch.matmul(h[start:stop], weight.t())
            head_stats_grad(logits, tgt[start:stop], entropy[start:], token_loss[start:],
                            correct[start:], unit / max(denom, 1e-6))
            lab_stop = min(stop, n_labelled)
            if want_grad and lab_stop > start:
                torch.matmul(logits[:lab_stop - start], weight, out=grad_sorted[start:lab_stop])
            del logits
        total = token_loss.sum()
        if torch.is_tensor(denominator):
            loss = total / denominator.to(dev)
        else:
            loss = total / denominator
        if want_grad:
            grad = torch.zeros((rows, width), dtype=torch.float16, device=dev)
            grad.index_copy_(0, order[:n_labelled], grad_sorted)
            ctx.save_for_backward(grad)
        ctx.unit = unit
        unsort = torch.empty_like(order)
        unsort[order] = torch.arange(rows, device=dev)
        stats = (entropy[unsort], token_loss[unsort], correct[unsort].bool())
        ctx.mark_non_differentiable(*stats)
        return (loss, *stats)

    @staticmethod
    def backward(ctx, grad_loss, *_unused):
        if not ctx.needs_input_grad[0]:
            return None, None, None, None
        (grad,) = ctx.saved_tensors
        factor = grad_loss.to(torch.float32) / ctx.unit
        return (grad.to(torch.float32) * factor).to(torch.float16), None, None, None


def _host_counts(labelled, denominator, device):
    """(labelled rows, loss denominator) on the host, with one synchronisation."""
    if torch.is_tensor(denominator):
        pair = torch.stack([labelled.sum().to(torch.float64),
                            denominator.to(device=device, dtype=torch.float64).reshape(())])
        n_labelled, denom = pair.tolist()
    else:
        n_labelled, denom = labelled.sum().item(), float(denominator)
    return int(n_labelled), float(denom)


def fused_head_loss(hidden16, weight16, targets, denominator):
    """(loss, token entropy [M], token loss [M], token correct [M]) for rows of `hidden16`.

    `targets[i]` is the label row i predicts (IGNORE_INDEX for none); `denominator` is what
    the summed loss is divided by (num_items_in_batch, or the labelled count)."""
    if not hidden16.is_cuda:
        raise ValueError("fused_head_loss: hidden16 must be a HIP device tensor (no CPU path)")
    return FusedHeadLoss.apply(hidden16.contiguous(), weight16, targets.contiguous(), denominator)
