"""Training metrics from one fused forward: what the reference's trainer glue hands TRL and Soup
(solution/trainer_patch.py:96-174), computed from HeadStats instead of the logits.

- entropy: the mean token entropy over the positions with attention_mask == 1 (TRL's
  entropy_from_logits, masked; solution/trainer_patch.py:121-129);
- num_tokens: the attention-mask count of the batch, which TRL accumulates
  (solution/trainer_patch.py:131-134);
- mean_token_accuracy: labelled next-token positions whose argmax is the label, over the
  labelled positions, 0 when there are none (solution/trainer_patch.py:136-151);
- rewind row losses: Soup's per-row mean token loss and labelled count
  (solution/trainer_patch.py:160-174, HeadStats.row_losses).

`*_from_logits` compute the same quantities the way TRL and Soup do from full [batch, seq,
vocab] logits (the unfused path), for comparison.  `gather` stands for accelerate's
gather_for_metrics (a no-op on one process)."""

import torch

from .head import IGNORE_INDEX


def _identity(t):
    return t


def trl_metrics(stats, attention_mask, gather=_identity):
    """{"entropy", "num_tokens_in_batch", "mean_token_accuracy"} from a HeadStats."""
    with torch.no_grad():
        entropy = gather(stats.entropy_sum / attention_mask.sum()).mean().item()
        num_tokens = gather(attention_mask.sum()).sum().item()
        correct, total = gather(stats.correct), gather(stats.labelled)
        total_sum = total.sum()
        accuracy = (correct.sum() / total_sum).item() if total_sum > 0 else 0.0
    return {"entropy": entropy, "num_tokens_in_batch": int(num_tokens),
            "mean_token_accuracy": accuracy}


def token_entropy(logits):
    """TRL's per-position entropy of the softmax of `logits` [..., vocab] (computed in fp32)."""
    z = logits.float()
    return torch.logsumexp(z, -1) - (torch.softmax(z, -1) * z).sum(-1)


def trl_metrics_from_logits(logits, labels, attention_mask, gather=_identity):
    """The same metrics from full logits, as TRL's SFTTrainer.compute_loss computes them."""
    with torch.no_grad():
        ent = torch.sum(token_entropy(logits) * attention_mask) / attention_mask.sum()
        entropy = gather(ent).mean().item()
        num_tokens = gather(attention_mask.sum()).sum().item()
        pred = logits[..., :-1, :].argmax(dim=-1)
        tgt = labels[..., 1:]
        mask = tgt != IGNORE_INDEX
        correct = gather(((pred == tgt) & mask).sum())
        total = gather(mask.sum())
        total_sum = total.sum()
        accuracy = (correct.sum() / total_sum).item() if total_sum > 0 else 0.0
    return {"entropy": entropy, "num_tokens_in_batch": int(num_tokens),
            "mean_token_accuracy": accuracy}


def rewind_row_losses_from_logits(logits, labels):
    """(row_loss, row_tokens): per batch row, the mean cross-entropy of the shifted labelled
    tokens and their count, as Soup's rewind log computes them from logits."""
    with torch.no_grad():
        z = logits[..., :-1, :].float()
        tgt = labels[..., 1:]
        ce = torch.nn.functional.cross_entropy(z.reshape(-1, z.shape[-1]), tgt.reshape(-1),
                                               reduction="none", ignore_index=IGNORE_INDEX)
        ce = ce.view(tgt.shape)
        tokens = (tgt != IGNORE_INDEX).sum(-1)
        means = ce.sum(-1) / tokens.clamp(min=1).to(ce.dtype)
    return [float(m) for m in means.tolist()], [int(t) for t in tokens.tolist()]
