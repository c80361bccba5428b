"""GPU: the fused training step (testt_amd/model.py, solution/model.py:209-279) against the
unpatched transformers Qwen2ForCausalLM on a small random 4-bit Qwen2 + LoRA: loss, every LoRA
gradient, TRL's entropy and accuracy, and Soup's per-row rewind losses, with the tolerances of
the reference's own step test (solution/test_model.py:115-127).

The reference builds the model with bitsandbytes + peft (solution/test_model.py:23-57); neither
is installed here, so the setup reproduces what they do: the fp16 checkpoint's projections are
quantized to NF4 double-quant (the oracle's bitsandbytes restatement), the unpatched model runs
with exactly the dequantized fp16 weights (what Linear4bit computes with under fp16 autocast),
every other parameter in fp32 (prepare_model_for_kbit_training), and LoRA r=16 on q_proj/v_proj
is a wrapper computing peft's `base(x) + B(A(dropout(x))) * scaling`, dropout drawn on the same
[batch, seq, hidden] fp32 input in the same order.  The unpatched side's metrics are computed
from its logits as TRL's entropy_from_logits and Soup's rewind row_losses define them."""

import math

import numpy as np
import pytest
import torch

from oracle.nf4 import dequant_state, quantize_nf4
from testt_amd import metrics
from testt_amd import model as fused_model
from testt_amd import workloads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
RANK, ALPHA = 16, 32


class LoraWrap(torch.nn.Module):
    """peft's LoRA Linear forward: base_layer(x) + lora_B(lora_A(dropout(x))) * scaling."""

    def __init__(self, base, a, b, scaling, p):
        super().__init__()
        self.base_layer, self.a, self.b, self.scaling, self.p = base, a, b, scaling, p

    def get_base_layer(self):
        return self.base_layer

    def forward(self, x):
        out = self.base_layer(x)
        d = torch.nn.functional.dropout(x.to(self.a.dtype), self.p, training=self.training)
        return out + torch.nn.functional.linear(torch.nn.functional.linear(d, self.a),
                                                self.b) * self.scaling


def nf4_of(w16, seed):
    """Params4bit-like NF4 double-quant weight of an fp16 [n_out, n_in] array, and its dequantized
    fp16 values."""
    code2 = workloads.dynamic_code_signed()
    packed, absmax_u8, absmax2, offset = quantize_nf4(w16, workloads.NF4_LEVELS, code2.numpy())
    p = workloads.nf4_weight(*w16.shape, seed=seed, device=DEV)
    st = p.quant_state
    p.data = torch.from_numpy(packed).reshape(-1, 1).to(DEV)
    st.absmax = torch.from_numpy(absmax_u8).to(DEV)
    st.state2.absmax = torch.from_numpy(absmax2).to(DEV)
    st.offset = torch.tensor(float(offset), dtype=torch.float32, device=DEV)
    return p, torch.from_numpy(dequant_state(p).astype(np.float16))


def build(dropout, hidden=256):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    # 4 heads: hidden 256 gives head dim 64 (torch SDPA), 512 head dim 128 (the HIP attention)
    cfg = Qwen2Config(vocab_size=1000, hidden_size=hidden, intermediate_size=512,
                      num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                      max_position_embeddings=256, tie_word_embeddings=True)
    cfg._attn_implementation = "sdpa"
    torch.manual_seed(0)
    hf = Qwen2ForCausalLM(cfg)
    with torch.no_grad():
        for lyr in hf.model.layers:
            for proj in (lyr.self_attn.q_proj, lyr.self_attn.k_proj, lyr.self_attn.v_proj):
                proj.bias.normal_(0, 0.1)
            lyr.input_layernorm.weight.uniform_(0.5, 1.5)
            lyr.post_attention_layernorm.weight.uniform_(0.5, 1.5)
    hf = hf.to(torch.float16).float()          # the fp16 checkpoint, non-4-bit params in fp32
    nf4 = []
    for i, lyr in enumerate(hf.model.layers):
        attn, mlp = lyr.self_attn, lyr.mlp
        mods = {"q": attn.q_proj, "k": attn.k_proj, "v": attn.v_proj, "o": attn.o_proj,
                "gate": mlp.gate_proj, "up": mlp.up_proj, "down": mlp.down_proj}
        weights = {}
        for j, (name, mod) in enumerate(mods.items()):
            p, deq = nf4_of(mod.weight.detach().to(torch.float16).numpy(), seed=100 * i + j)
            weights[name] = p
            mod.weight = torch.nn.Parameter(deq, requires_grad=False)   # Linear4bit's fp16 view
        nf4.append(weights)
    for p in hf.parameters():
        p.requires_grad_(False)
    hf.to(DEV)
    # LoRA tensors (plain leaf tensors shared by both sides; A as peft's kaiming-uniform range,
    # B ~ N(0, 0.05) as the reference's test sets it)
    g = torch.Generator().manual_seed(5)
    scaling = ALPHA / RANK
    lora = []
    for lyr in hf.model.layers:
        attn = lyr.self_attn
        pair = []
        for mod in (attn.q_proj, attn.v_proj):
            a = (torch.rand(RANK, mod.in_features, generator=g) - 0.5) * \
                (2 / math.sqrt(mod.in_features))
            b = 0.05 * torch.randn(mod.out_features, RANK, generator=g)
            pair.append((a.to(DEV).requires_grad_(True), b.to(DEV).requires_grad_(True)))
        lora.append(pair)
        attn.q_proj = LoraWrap(attn.q_proj, *pair[0], scaling, dropout)
        attn.v_proj = LoraWrap(attn.v_proj, *pair[1], scaling, dropout)
    hf.train()
    fused = fused_model.from_qwen2(hf, nf4, lora, scaling, dropout)
    return hf, fused, lora


def batch(vocab=1000):
    torch.manual_seed(1)
    lengths = [24, 15, 6]
    seq = max(lengths)
    ids = torch.randint(0, vocab, (len(lengths), seq))
    mask = torch.zeros_like(ids)
    labels = torch.full_like(ids, -100)
    for row, n in enumerate(lengths):
        mask[row, :n] = 1
        prompt = n // 3
        labels[row, prompt:n] = ids[row, prompt:n]
    ids[mask == 0] = 0
    return ids.to(DEV), mask.to(DEV), labels.to(DEV)


def grads_of(lora):
    out = {}
    for i, pair in enumerate(lora):
        for name, (a, b) in zip(("q", "v"), pair):
            out[f"{i}.{name}.A"] = a.grad.detach().float().clone()
            out[f"{i}.{name}.B"] = b.grad.detach().float().clone()
            a.grad = b.grad = None
    return out


def run_unpatched(hf, lora, ids, mask, labels, n_items):
    torch.manual_seed(123)
    with torch.autocast("cuda", dtype=torch.float16):
        out = hf(input_ids=ids, attention_mask=mask, labels=labels, num_items_in_batch=n_items)
    (out.loss * 1024).backward()
    loss = float(out.loss.detach())
    logits = out.logits.detach().float()
    # TRL entropy_from_logits, masked mean over attention_mask
    ent = torch.logsumexp(logits, -1) - (torch.softmax(logits, -1) * logits).sum(-1)
    entropy = float((ent * mask).sum() / mask.sum())
    pred = logits[:, :-1].argmax(-1)
    tgt = labels[:, 1:]
    accuracy = float(((pred == tgt) & (tgt != -100)).sum() / (tgt != -100).sum())
    # Soup rewind row_losses: mean shifted token loss per row, labelled count per row
    ce = torch.nn.functional.cross_entropy(logits[:, :-1].reshape(-1, logits.shape[-1]),
                                           tgt.reshape(-1), reduction="none",
                                           ignore_index=-100).view(tgt.shape)
    tokens = (tgt != -100).sum(1)
    rows = ([float(x) for x in (ce.sum(1) / tokens.clamp(min=1)).tolist()],
            [int(t) for t in tokens.tolist()])
    run_unpatched.pred = pred
    return loss, grads_of(lora), entropy, accuracy, rows


def run_fused(fused, lora, ids, mask, labels, n_items):
    torch.manual_seed(123)
    with torch.autocast("cuda", dtype=torch.float16):
        loss, stats = fused_model.fused_forward(fused, ids, mask, labels, n_items)
    (loss * 1024).backward()
    loss = loss.detach()
    assert isinstance(stats, fused_model.HeadStats)
    m = metrics.trl_metrics(stats, mask)          # the trainer glue's reduction of HeadStats
    assert m["num_tokens_in_batch"] == int(mask.sum())
    return float(loss), grads_of(lora), m["entropy"], m["mean_token_accuracy"], \
        stats.row_losses()


@pytest.mark.parametrize("dropout,hidden", [(0.0, 256), (0.05, 256), (0.0, 512), (0.05, 512)])
def test_fused_step_matches_unpatched_model(dropout, hidden):
    print(f"model step: tiny Qwen2 (hidden {hidden}) + NF4 + LoRA r=16, lora dropout {dropout}",
          flush=True)
    hf, fused, lora = build(dropout, hidden)
    ids, mask, labels = batch()
    n_items = (labels[:, 1:] != -100).sum()
    ref = run_unpatched(hf, lora, ids, mask, labels, n_items)
    got = run_fused(fused, lora, ids, mask, labels, n_items)
    worst = max(float((got[1][n] - g).norm() / g.norm().clamp(min=1e-12))
                for n, g in ref[1].items())
    print(f"  loss {got[0]:.6f} vs {ref[0]:.6f} (rel {abs(got[0] - ref[0]) / ref[0]:.1e}); "
          f"worst LoRA grad rel-norm {worst:.1e}; entropy {got[2]:.5f} vs {ref[2]:.5f}; "
          f"accuracy {got[3]:.4f} vs {ref[3]:.4f}", flush=True)
    assert abs(got[0] - ref[0]) / ref[0] < 2e-3, (got[0], ref[0])
    assert set(got[1]) == set(ref[1]) and ref[1]
    for name, grad in ref[1].items():
        rel = (got[1][name] - grad).norm() / grad.norm().clamp(min=1e-12)
        assert rel < 2e-2, (name, float(rel))
    assert abs(got[2] - ref[2]) / ref[2] < 2e-3, (got[2], ref[2])
    assert abs(got[3] - ref[3]) < 1e-6 + 0.02, (got[3], ref[3])
    assert got[4][1] == ref[4][1]
    for a, b in zip(got[4][0], ref[4][0]):
        assert abs(a - b) / b < 2e-3, (got[4][0], ref[4][0])

    # A random model never predicts its label (accuracy 0 on both sides), so score the step
    # again against labels that take the unpatched model's own prediction at every other
    # labelled position: the argmax-hit counts must then agree on a non-trivial accuracy.
    hit = labels.clone()
    tgt = hit[:, 1:]
    lab = (tgt != -100).nonzero()
    pick = lab[::2]
    tgt[pick[:, 0], pick[:, 1]] = run_unpatched.pred[pick[:, 0], pick[:, 1]]
    ref2 = run_unpatched(hf, lora, ids, mask, hit, n_items)
    got2 = run_fused(fused, lora, ids, mask, hit, n_items)
    print(f"  argmax labels: accuracy {got2[3]:.4f} vs {ref2[3]:.4f}", flush=True)
    assert ref2[3] > 0.4
    assert abs(got2[3] - ref2[3]) < 1e-6 + 0.02, (got2[3], ref2[3])
    assert abs(got2[0] - ref2[0]) / ref2[0] < 2e-3, (got2[0], ref2[0])


def test_synthetic_model_full_width_step():
    """Two Qwen2.5-1.5B-width layers and the full 151,936-token vocabulary on a ragged batch:
    the step runs, its loss is that of near-uniform logits, every LoRA gradient is finite and
    the statistics count what the batch holds."""
    m = fused_model.synthetic_model(DEV, n_layers=2)
    lengths, seq = (64, 40, 9), 64
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, workloads.VOCAB, (3, seq), generator=g)
    mask = torch.zeros_like(ids)
    labels = torch.full_like(ids, -100)
    for r, n in enumerate(lengths):
        mask[r, :n] = 1
        labels[r, n // 4:n] = ids[r, n // 4:n]
    ids, mask, labels = ids.to(DEV), mask.to(DEV), labels.to(DEV)
    loss, stats = fused_model.fused_forward(m, ids, mask, labels)
    loss.backward()
    assert abs(float(loss.detach()) - math.log(workloads.VOCAB)) < 1.0
    n_lab = int((torch.nn.functional.pad(labels, (0, 1), value=-100)[:, 1:][mask.bool()]
                 != -100).sum())
    assert int(stats.labelled) == n_lab
    assert sum(stats.row_losses()[1]) == n_lab
    for p in fused_model.lora_parameters(m):
        assert p.grad is not None and bool(torch.isfinite(p.grad).all())
