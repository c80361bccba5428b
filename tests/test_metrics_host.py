"""CPU: the trainer metrics from HeadStats (testt_amd/metrics.py, the reference's glue in
solution/trainer_patch.py:96-174) equal what TRL and Soup compute from full logits, for a padded
batch with prompt masking.  HeadStats is assembled here from per-token values the way
fused_forward assembles it from the head kernel's outputs (real rows only, shifted targets)."""

import torch

from testt_amd import metrics, model


def head_stats_from_logits(logits, labels, attention_mask):
    b, t, v = logits.shape
    pos = attention_mask.reshape(-1).nonzero().squeeze(1)
    z = logits.reshape(-1, v).index_select(0, pos).float()
    tgt = model.shifted_targets(labels, pos)
    lab = tgt != -100
    ent = metrics.token_entropy(z)
    lse = torch.logsumexp(z, -1)
    zt = z.gather(1, tgt.clamp(min=0)[:, None]).squeeze(1)
    tok_loss = torch.where(lab, lse - zt, torch.zeros_like(lse))
    correct = (z.argmax(-1) == tgt) & lab
    row = torch.div(pos, t, rounding_mode="floor")
    return model.HeadStats(
        entropy_sum=ent.sum(), correct=correct.sum(), labelled=lab.sum(),
        row_loss_sum=torch.zeros(b).index_add_(0, row, tok_loss),
        row_tokens=torch.zeros(b, dtype=torch.long).index_add_(0, row, lab.long()))


def batch(seed, vocab=53, lengths=(12, 7, 3, 12)):
    g = torch.Generator().manual_seed(seed)
    seq = max(lengths)
    logits = torch.randn(len(lengths), seq, vocab, generator=g) * 2
    ids = torch.randint(0, vocab, (len(lengths), seq), generator=g)
    mask = torch.zeros_like(ids)
    labels = torch.full_like(ids, -100)
    for r, n in enumerate(lengths):
        mask[r, :n] = 1
        labels[r, n // 3:n] = ids[r, n // 3:n]
    # make some argmax hits
    for r, n in enumerate(lengths):
        for p in range(n // 3, n - 1, 2):
            labels[r, p + 1] = int(logits[r, p].argmax())
    return logits, labels, mask


def test_trl_metrics_match_logit_path():
    for seed in range(4):
        logits, labels, mask = batch(seed)
        stats = head_stats_from_logits(logits, labels, mask)
        got = metrics.trl_metrics(stats, mask)
        ref = metrics.trl_metrics_from_logits(logits, labels, mask)
        assert got["num_tokens_in_batch"] == ref["num_tokens_in_batch"] == int(mask.sum())
        assert abs(got["entropy"] - ref["entropy"]) < 1e-5 * abs(ref["entropy"])
        assert got["mean_token_accuracy"] == ref["mean_token_accuracy"]
        assert 0.2 < ref["mean_token_accuracy"] < 1.0
        rows, toks = stats.row_losses()
        r_rows, r_toks = metrics.rewind_row_losses_from_logits(logits, labels)
        assert toks == r_toks
        for a, b in zip(rows, r_rows):
            assert abs(a - b) <= 1e-5 * abs(b) + 1e-7


def test_no_labelled_tokens_gives_zero_accuracy():
    logits, labels, mask = batch(9)
    labels[:] = -100
    stats = head_stats_from_logits(logits, labels, mask)
    assert metrics.trl_metrics(stats, mask)["mean_token_accuracy"] == 0.0
    assert metrics.trl_metrics_from_logits(logits, labels, mask)["mean_token_accuracy"] == 0.0
    assert stats.row_losses()[1] == [0, 0, 0, 0]
