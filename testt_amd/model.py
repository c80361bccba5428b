"""The training forward of Qwen2ForCausalLM + LoRA on the real tokens, built from the drop-in ops.

Mirrors the reference's fused_forward (solution/model.py:209-279) and HeadStats
(solution/model.py:36-51).  With s the fp32 residual stream of the M real tokens (pad-free:
pos_idx = attention_mask.nonzero(), solution/model.py:220):

  s          = embedding(input_ids[real])             fp16 table -> fp32 rows
  per layer  : testt_amd.layer.decoder_layer          norm, QKV + LoRA, RoPE pack, attention, o-proj,
                                                       norm, NF4 MLP (the reference's loop body,
                                                       solution/model.py:235-255)
  y          = add_rmsnorm(s, d, final norm)           (solution/model.py:257)
  targets    = labels shifted by one, real rows        (ForCausalLMLoss's shift,
                                                        solution/model.py:261-263)
  loss, ...  = fused_head_loss(y, W16, targets, denom) chunked vocab head (solution/model.py:268)

and returns (loss, HeadStats) in place of the [batch, seq, vocab] logits: the statistics TRL's
metrics (entropy over attention_mask == 1, accuracy over labelled targets) and Soup's rewind
log (per-row mean token loss) read from them.

The reference takes its weights from a PEFT/bitsandbytes model; here they are plain tensors
(`ModelWeights`: the fp16 embedding, `layer.LayerWeights` per decoder layer, the final norm),
so the whole model runs without transformers, peft or bitsandbytes.  `from_qwen2` builds them
from a transformers Qwen2ForCausalLM whose projection weights the caller supplies in NF4.
"""

from dataclasses import dataclass, field

import torch

from . import layer as _layer
from . import workloads
from .head import IGNORE_INDEX, fused_head_loss
from .rmsnorm import add_rmsnorm


class HeadStats:
    """What TRL's metrics and Soup's rewind log need from one labelled forward, in place of the
    logits (solution/model.py:36-51)."""

    def __init__(self, entropy_sum, correct, labelled, row_loss_sum, row_tokens):
        self.entropy_sum = entropy_sum      # sum of token entropies over attention_mask == 1
        self.correct = correct              # labelled tokens whose argmax is the label
        self.labelled = labelled            # labelled tokens
        self.row_loss_sum = row_loss_sum    # [batch] summed token cross-entropy per row
        self.row_tokens = row_tokens        # [batch] labelled tokens per row

    def row_losses(self):
        """(row_loss, row_tokens): the per-row mean token loss and labelled count, as Soup's
        rewind log takes them (solution/model.py:47-51)."""
        tokens = self.row_tokens
        means = self.row_loss_sum / tokens.clamp(min=1).to(self.row_loss_sum.dtype)
        return [float(m) for m in means.tolist()], [int(t) for t in tokens.tolist()]


@dataclass
class ModelWeights:
    embed: torch.Tensor                         # fp16 [V, H] (the tied head reads it too)
    layers: list                                # layer.LayerWeights per decoder layer
    final_norm: torch.Tensor                    # fp32 [H]
    inv_freq: torch.Tensor                      # fp32 [head_dim / 2], the rotary frequencies
    eps: float = 1e-6
    head: torch.Tensor = field(default=None)    # fp16 [V, H]; None: tied to `embed`


def rotary_tables(inv_freq, seq):
    """cos, sin fp32 [seq, head_dim] for positions 0..seq-1, as transformers' default rotary
    embedding builds them (angle = position * inv_freq, emb = cat(angle, angle))."""
    pos = torch.arange(seq, device=inv_freq.device, dtype=torch.float32)
    freqs = pos[:, None] * inv_freq.float()[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos(), emb.sin()


def default_inv_freq(head_dim, theta, device):
    """1 / theta^(2j / head_dim), j = 0 .. head_dim/2 - 1 (Qwen2's default rope)."""
    exps = torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim
    return (1.0 / (theta ** exps)).to(device)


def shifted_targets(labels, pos_idx):
    """Causal-LM targets of the real tokens: position t is scored against label t + 1 (the last
    position of a row against IGNORE_INDEX), as transformers' ForCausalLMLoss shifts them."""
    targets = torch.nn.functional.pad(labels, (0, 1), value=IGNORE_INDEX)[:, 1:]
    return targets.reshape(-1).index_select(0, pos_idx)


def fused_forward(model, input_ids, attention_mask, labels, num_items_in_batch=None):
    """(loss, HeadStats) of one labelled training forward (solution/model.py:209-279).

    `loss` is differentiable with respect to the LoRA parameters of `model.layers` (and
    nothing else: the embedding, norms and NF4 projections are frozen, as in QLoRA)."""
    if input_ids.dim() != 2 or attention_mask.shape != input_ids.shape or \
            labels.shape != input_ids.shape:
        raise ValueError("input_ids, attention_mask and labels must share one [batch, seq] shape")
    batch, seq = input_ids.shape
    dev = input_ids.device
    pos_idx = attention_mask.reshape(-1).nonzero().squeeze(1)

    ids = input_ids.reshape(-1).index_select(0, pos_idx)
    s = torch.nn.functional.embedding(ids, model.embed).float()
    cos, sin = rotary_tables(model.inv_freq, seq)
    key_valid = _layer.key_valid_of(attention_mask)

    delta = None
    for w in model.layers:
        s, delta = _layer.decoder_layer(s, delta, w, pos_idx, batch, seq, cos, sin, key_valid)
    _, y, _ = add_rmsnorm(s, delta, model.final_norm, model.eps)
    del s, delta

    targets = shifted_targets(labels, pos_idx)
    labelled_mask = targets != IGNORE_INDEX
    denominator = num_items_in_batch if num_items_in_batch is not None else labelled_mask.sum()
    weight = model.head if model.head is not None else model.embed
    if weight.dtype != torch.float16:
        weight = weight.to(torch.float16)
    loss, entropy, token_loss, correct = fused_head_loss(y, weight, targets, denominator)

    with torch.no_grad():
        row = torch.div(pos_idx, seq, rounding_mode="floor")
        row_loss_sum = torch.zeros(batch, dtype=torch.float32, device=dev).index_add_(
            0, row, token_loss)
        row_tokens = torch.zeros(batch, dtype=torch.long, device=dev).index_add_(
            0, row, labelled_mask.long())
        stats = HeadStats(entropy_sum=entropy.sum(), correct=correct.sum(),
                          labelled=labelled_mask.sum(), row_loss_sum=row_loss_sum,
                          row_tokens=row_tokens)
    return loss, stats


def lora_parameters(model):
    """The trainable tensors of `model`: (A_q, B_q, A_v, B_v) per layer."""
    out = []
    for w in model.layers:
        out += [*w.lora_q, *w.lora_v]
    return out


def synthetic_model(device, n_layers=28, vocab=workloads.VOCAB, hidden=workloads.HIDDEN,
                    inter=workloads.INTER, n_heads=workloads.N_HEADS, n_kv=workloads.N_KV,
                    head_dim=workloads.HEAD_DIM, rank=16, alpha=32, dropout=0.0, seed=11):
    """A Qwen2.5-1.5B-shaped model (28 layers, tied 151,936 x 1536 embedding) with synthetic
    NF4 projections (distinct per layer) and LoRA r=16 on q/v, for measurement."""
    layers = [_layer.synthetic_layer(device, hidden, inter, n_heads, n_kv, head_dim, rank, alpha,
                                     dropout, seed=seed * 1000 + i) for i in range(n_layers)]
    g = workloads.gen(seed)
    embed = (0.02 * torch.randn(vocab, hidden, generator=g)).to(torch.float16).to(device)
    final = (1 + 0.02 * torch.randn(hidden, generator=g)).to(device)
    return ModelWeights(embed=embed, layers=layers, final_norm=final,
                        inv_freq=default_inv_freq(head_dim, workloads.ROPE_THETA, device))


def _base_layer(module):
    """The projection under a LoRA wrapper (peft's get_base_layer), else the module itself
    (solution/model.py:54-56)."""
    get = getattr(module, "get_base_layer", None)
    return get() if callable(get) else module


def from_qwen2(causal_lm, nf4_weights, lora, scaling, dropout=0.0):
    """ModelWeights of a transformers Qwen2ForCausalLM (the unquantized parts: embedding, norms,
    q/k/v biases, rotary frequencies), with the projections of layer i given in NF4 by
    `nf4_weights[i]` (dict q, k, v, o, gate, up, down of Params4bit-like weights) and its LoRA
    tensors by `lora[i]` ((A_q, B_q), (A_v, B_v)).  Checks the model is one the fused path runs
    (the conditions of solution/model.py:125-149: full attention, silu, no MLP bias, q/k/v
    biases all present or all absent, an untied or tied head without bias)."""
    cfg = causal_lm.config
    inner = causal_lm.model
    if getattr(cfg, "hidden_act", "silu") != "silu":
        raise ValueError("activation is not silu")
    if any(t != "full_attention" for t in (getattr(cfg, "layer_types", None) or [])):
        raise ValueError("sliding-window layers")
    n_heads, n_kv = cfg.num_attention_heads, cfg.num_key_value_heads
    head_dim = getattr(cfg, "head_dim", None) or cfg.hidden_size // n_heads
    layers = []
    for i, lyr in enumerate(inner.layers[:cfg.num_hidden_layers]):
        attn, mlp = lyr.self_attn, lyr.mlp
        q, k, v, o, gate, up, down = (_base_layer(m) for m in (
            attn.q_proj, attn.k_proj, attn.v_proj, attn.o_proj, mlp.gate_proj, mlp.up_proj,
            mlp.down_proj))
        if any(getattr(m, "bias", None) is not None for m in (gate, up, down)):
            raise ValueError("MLP bias")
        biases = [q.bias, k.bias, v.bias]
        if all(b is not None for b in biases):
            qkv_bias = torch.cat([b.detach().to(torch.float16) for b in biases])
        elif all(b is None for b in biases):
            qkv_bias = None
        else:
            raise ValueError("mixed q/k/v bias")
        if o.bias is not None:
            raise ValueError("o_proj bias")
        nw = nf4_weights[i]
        layers.append(_layer.LayerWeights(
            input_norm=lyr.input_layernorm.weight.detach().float(),
            post_norm=lyr.post_attention_layernorm.weight.detach().float(),
            q=nw["q"], k=nw["k"], v=nw["v"], o=nw["o"], gate=nw["gate"], up=nw["up"],
            down=nw["down"], qkv_bias=qkv_bias, lora_q=tuple(lora[i][0]),
            lora_v=tuple(lora[i][1]), scaling=scaling, n_heads=n_heads, n_kv=n_kv,
            head_dim=head_dim, eps=lyr.input_layernorm.variance_epsilon, dropout=dropout))
    head = causal_lm.lm_head.weight
    embed = inner.embed_tokens.weight.detach().to(torch.float16)
    tied = head.data_ptr() == inner.embed_tokens.weight.data_ptr()
    rot = getattr(inner, "rotary_emb", None)
    inv_freq = rot.inv_freq.detach().float() if rot is not None else \
        default_inv_freq(head_dim, getattr(cfg, "rope_theta", 10000.0), embed.device)
    return ModelWeights(embed=embed, layers=layers,
                        final_norm=inner.norm.weight.detach().float(), inv_freq=inv_freq,
                        eps=inner.norm.variance_epsilon,
                        head=None if tied else head.detach().to(torch.float16))
