"""Vocab-head statistics and gradient of one logits chunk, in float64 on the CPU.
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Per row of fp16 logits z (solution/head.py:34-76):
  lse      = logsumexp(z)
  entropy  = lse - sum(softmax(z) * z)            (= -sum p log p)
  loss     = lse - z[target], 0 when target == -100
  correct  = argmax(z) == target (first maximum, as torch.argmax and the reference's
             tie_break_left), False when ignored
  grad     = fp16((softmax(z) - onehot(target)) * grad_scale) for labelled rows; ignored rows
             keep their logits.
The reference's own test (solution/test_kernels.py:179-196) checks its kernel against
F.cross_entropy / log_softmax / argmax of the fp32-cast logits; here the same quantities are
taken in float64 so that the oracle's own rounding is negligible.

Pinned by: torch.nn.functional.cross_entropy and log_softmax (float64), uniform logits
(entropy = ln V, lse = z + ln V), a single spike (argmax hit), ties (first index wins), rows of
the gradient summing to 0 before rounding, ignored rows (tests/test_oracle_head.py).

fused_head_loss restates FusedHeadLoss.forward/backward (solution/head.py:87-137) in float64:
loss = sum of token losses / denominator, and the gradient of hidden is
(softmax - onehot) @ W / denominator times the incoming loss gradient.
"""

import math

import torch

IGNORE_INDEX = -100


def head_stats_grad(logits, targets, grad_scale):
    """(entropy f64, loss f64, correct bool, lse f64, new_logits fp16) for one chunk."""
    z = logits.detach().double()
    targets = targets.long()
    lse = torch.logsumexp(z, dim=-1)
    p = torch.exp(z - lse[:, None])
    entropy = lse - (p * z).sum(-1)
    labelled = targets != IGNORE_INDEX
    safe = torch.where(labelled, targets, torch.zeros_like(targets))
    z_t = z.gather(1, safe[:, None]).squeeze(1)
    loss = torch.where(labelled, lse - z_t, torch.zeros_like(lse))
    arg = torch.argmax(z, dim=-1)
    correct = labelled & (arg == targets)
    onehot = torch.zeros_like(p)
    onehot[labelled, safe[labelled]] = 1.0
    grad = ((p - onehot) * grad_scale).to(torch.float32).to(torch.float16)
    new_logits = torch.where(labelled[:, None], grad, logits.detach().to(torch.float16))
    return entropy, loss, correct, lse, new_logits


def grad_unit(denominator):
    """solution/head.py:79-84: 2^clamp(round(log2(denominator)) + 6, 0, 16)."""
    exponent = int(round(math.log2(max(float(denominator), 1e-6)))) + 6
    return float(2 ** max(0, min(16, exponent)))


def fused_head_loss(hidden, weight, targets, denominator, grad_loss=1.0):
    """(loss, entropy, token_loss, correct, d hidden fp64) over all rows, unchunked."""
    w = weight.detach().double()
    logits = (hidden.detach().float() @ weight.detach().float().t()).to(torch.float16)
    entropy, loss, correct, _lse, _ = head_stats_grad(logits, targets, 1.0)
    z = logits.double()
    p = torch.softmax(z, dim=-1)
    labelled = targets != IGNORE_INDEX
    onehot = torch.zeros_like(p)
    onehot[labelled, targets[labelled]] = 1.0
    dlogits = (p - onehot) * labelled[:, None].double()
    dh = dlogits @ w * (float(grad_loss) / float(denominator))
    return loss.sum() / float(denominator), entropy, loss, correct, dh
