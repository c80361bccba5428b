"""The training forward of a 4-bit Qwen2ForCausalLM + LoRA on the real tokens, built from the
drop-in ops: the model-level entry the reference's trainer patch binds
(`from .model import HeadStats, can_run, fused_forward, model_plan`,
solution/trainer_patch.py:23, called at solution/trainer_patch.py:57-63).

    model_plan(causal_lm)                      the checked layout of the model (cached on it),
                                               None when the fused path does not take the model
    can_run(causal_lm, input_ids, attention_mask, labels, extra)
                                               True for a labelled training step under fp16
                                               autocast on a HIP device that the plan covers
    fused_forward(causal_lm, input_ids, attention_mask, labels, num_items_in_batch)
                                               CausalLMOutputWithPast(loss, logits=HeadStats)

Same names, arguments, conditions and results as solution/model.py:36-51,152-279.  With s the
fp32 residual stream of the M real tokens (pos_idx = attention_mask.nonzero(), the pad-free
layout of solution/model.py:220):

  s          = embedding(input_ids[real])             (the table as the model holds it) -> fp32
  per layer  : testt_amd.layer.decoder_layer          norm, q|k|v GEMM + LoRA (HIP kernels),
                                                       RoPE + varlen causal GQA attention over
                                                       each row's real tokens (HIP), o GEMM,
                                                       norm, NF4 MLP (solution/model.py:235-255)
  y          = add_rmsnorm(s, d, final norm)           (solution/model.py:257)
  targets    = labels shifted by one, real rows        (solution/model.py:260-263)
  loss, ...  = fused_head_loss(y, W16, targets, denom) (solution/model.py:264-268)

Where the reference runs torch SDPA on the padded layout, peft's LoRA modules and one unpack per
projection, this runs the layer's own path: one NF4 unpack launch per layer (the LoRA
parameters' fp16 staging in the same launch), the rank-16 LoRA kernels, and attention over the
real tokens only with RoPE's backward inside the attention backward.  LoRA with dropout, other
ranks, or a LoRA adapter on only one of q/v run the reference's LoRA formulation
(layer.lora_branch: peft's own dropout modules on the padded fp32 norm output, so the dropout
draws are the unpatched model's); head dims other than 128 run torch SDPA on the padded layout.

The 4-bit projections are recognised by their weight's `quant_state` (bitsandbytes' Params4bit
carries it; bitsandbytes itself is not needed to run the kernels), the LoRA adapters by peft's
LoraLayer attributes (lora_A / lora_B / lora_dropout ModuleDicts, scaling, active_adapters).
`ModelWeights` + `forward_weights` run the same path on plain tensors.
"""

from dataclasses import dataclass, field

import torch

from . import layer as _layer
from ._common import kernels_ok
from .head import IGNORE_INDEX, fused_head_loss
from .rmsnorm import add_rmsnorm

# Keyword arguments of Qwen2ForCausalLM.forward that the fused path accepts
# (solution/model.py:32-33): num_items_in_batch and return_dict with any value, the two output
# flags only when false.
_ALLOWED_KWARGS = frozenset(("num_items_in_batch", "output_attentions", "output_hidden_states",
                             "return_dict"))
_ANY_VALUE_KWARGS = frozenset(("num_items_in_batch", "return_dict"))

# Where model_plan keeps its result on the model (solution/model.py:154 uses the same key).
_PLAN_KEY = "_soup_kernel_plan"


class HeadStats:
    """What TRL's metrics and Soup's rewind log need from one labelled forward, in place of the
    [batch, seq, vocab] logits (solution/model.py:36-51).  Lives in `outputs.logits`."""

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


# --------------------------------------------------------------------------------------------
# Recognising the model's modules


def _base_layer(module):
    """The projection under a LoRA wrapper (peft's get_base_layer), else the module itself
    (solution/model.py:54-56)."""
    get = getattr(module, "get_base_layer", None)
    return get() if callable(get) else module


def _is_4bit(module):
    """A 4-bit linear: its weight carries a bitsandbytes quant state (Linear4bit's Params4bit;
    solution/model.py:59-65 asks the same of a bitsandbytes.nn.Linear4bit)."""
    return getattr(getattr(module, "weight", None), "quant_state", None) is not None


class LoraParts:
    """The one active vanilla LoRA adapter of a peft LoraLayer: its dropout module, A and B
    linears and scaling (what solution/model.py:68-91 returns as a tuple)."""

    __slots__ = ("dropout", "lora_a", "lora_b", "scaling")

    def __init__(self, dropout, lora_a, lora_b, scaling):
        self.dropout, self.lora_a, self.lora_b, self.scaling = dropout, lora_a, lora_b, scaling

    def __iter__(self):
        return iter((self.dropout, self.lora_a, self.lora_b, self.scaling))


def _adapter_flag(module, attr, name):
    table = getattr(module, attr, None)
    return bool(table.get(name, False)) if isinstance(table, dict) else False


def _lora_parts(module):
    """None: no LoRA on `module` (or no active adapter of it); LoraParts: exactly one active
    vanilla adapter; False: any other LoRA state the fused path does not reproduce (merged or
    disabled adapters, several active adapters, DoRA, LoRA bias, a variant, a dropout that is
    neither Dropout nor Identity).  The rules of solution/model.py:68-91."""
    if not hasattr(module, "lora_A"):
        return None
    try:
        if getattr(module, "merged", False) or getattr(module, "disable_adapters", False):
            return False
        names = [n for n in module.active_adapters if n in module.lora_A.keys()]
        if not names:
            return None
        if len(names) > 1:
            return False
        name = names[0]
        variants = getattr(module, "lora_variant", None) or {}
        if name in variants or _adapter_flag(module, "use_dora", name) or \
                _adapter_flag(module, "lora_bias", name):
            return False
        dropout = module.lora_dropout[name]
        if not isinstance(dropout, (torch.nn.Dropout, torch.nn.Identity)):
            return False
        return LoraParts(dropout, module.lora_A[name], module.lora_B[name],
                         float(module.scaling[name]))
    except Exception:  # noqa: BLE001 - a peft layout this path does not know: not ours to run
        return False


def _norm_weight(weight):
    """A norm's weight as the RMSNorm kernels take it: fp32 (prepare_model_for_kbit_training
    leaves the norms in fp32; a model with fp16 norms gets an fp32 copy per forward)."""
    w = weight.detach()
    return w if w.dtype == torch.float32 else w.float()


def _dropout_p(dropout):
    """The probability the dropout module applies now (0 for Identity or in eval mode)."""
    if isinstance(dropout, torch.nn.Dropout) and dropout.training:
        return float(dropout.p)
    return 0.0


# --------------------------------------------------------------------------------------------
# The plan


class LayerPlan:
    """One decoder layer's frozen parts, checked once (solution/model.py:94-122): the seven
    4-bit projections, the q|k|v and o biases in fp16, the two norms, and the q/v modules whose
    LoRA state is read on every forward."""

    __slots__ = ("layer", "attn", "q", "k", "v", "o", "gate", "up", "down", "qkv_bias",
                 "o_bias", "lora_modules")

    def __init__(self, layer):
        self.layer = layer
        attn, mlp = layer.self_attn, layer.mlp
        self.attn = attn
        self.lora_modules = (attn.q_proj, attn.v_proj)
        mods = (attn.q_proj, attn.k_proj, attn.v_proj, attn.o_proj, mlp.gate_proj, mlp.up_proj,
                mlp.down_proj)
        bases = [_base_layer(m) for m in mods]
        if not all(_is_4bit(b) for b in bases):
            raise ValueError("not a bitsandbytes 4-bit layer")
        q, k, v, o, gate, up, down = bases
        self.q, self.k, self.v, self.o = q.weight, k.weight, v.weight, o.weight
        self.gate, self.up, self.down = gate.weight, up.weight, down.weight
        if any(getattr(b, "bias", None) is not None for b in (gate, up, down)):
            raise ValueError("MLP bias")
        qkv_b = [getattr(b, "bias", None) for b in (q, k, v)]
        present = sum(b is not None for b in qkv_b)
        if present not in (0, 3):
            raise ValueError("mixed q/k/v bias")
        self.qkv_bias = torch.cat([b.detach().to(torch.float16) for b in qkv_b]) \
            if present else None
        o_b = getattr(o, "bias", None)
        self.o_bias = o_b.detach().to(torch.float16) if o_b is not None else None
        for m in (attn.k_proj, attn.o_proj, mlp.gate_proj, mlp.up_proj, mlp.down_proj):
            if _lora_parts(m) is not None:
                raise ValueError("LoRA outside q_proj/v_proj")


class ModelPlan:
    """The model-level checks and parts (solution/model.py:125-149): SDPA attention, full
    attention in every layer, SiLU, an even head dim, a frozen unbiased embedding and head with
    one row per vocabulary entry, and a LayerPlan per decoder layer."""

    def __init__(self, causal_lm):
        cfg = causal_lm.config
        inner = causal_lm.model
        if getattr(cfg, "_attn_implementation", None) != "sdpa":
            raise ValueError("attention is not sdpa")
        if getattr(inner, "has_sliding_layers", False) or \
                any(t != "full_attention" for t in (getattr(cfg, "layer_types", None) or [])):
            raise ValueError("sliding-window layers")
        if getattr(cfg, "hidden_act", "silu") != "silu":
            raise ValueError("activation is not silu")
        self.n_heads = cfg.num_attention_heads
        self.n_kv = cfg.num_key_value_heads
        self.hidden = cfg.hidden_size
        self.head_dim = getattr(cfg, "head_dim", None) or self.hidden // self.n_heads
        if self.head_dim % 2:
            raise ValueError("odd head_dim")
        self.layers = [LayerPlan(lyr) for lyr in inner.layers[:cfg.num_hidden_layers]]
        self.embed = inner.embed_tokens
        self.head = causal_lm.lm_head
        self.norm = inner.norm
        self.rotary = inner.rotary_emb
        if self.embed.weight.requires_grad or self.head.weight.requires_grad or \
                getattr(self.head, "bias", None) is not None:
            raise ValueError("trainable or biased embedding/head")
        if self.head.weight.shape[0] != cfg.vocab_size:
            raise ValueError("vocab size")

    def layer_weights(self, lp):
        """layer.LayerWeights of one layer with its LoRA state as it is now (adapters can be
        switched between steps, as peft allows)."""
        lyr = lp.layer
        parts = [_lora_parts(m) for m in lp.lora_modules]
        lora = [None if p is None else (p.lora_a.weight, p.lora_b.weight) for p in parts]
        scal = [None if p is None else p.scaling for p in parts]
        drop = [None if p is None else p.dropout for p in parts]
        eps_in = lyr.input_layernorm.variance_epsilon
        if lyr.post_attention_layernorm.variance_epsilon != eps_in:
            raise ValueError("the two norms of a layer have different eps")
        return _layer.LayerWeights(
            input_norm=_norm_weight(lyr.input_layernorm.weight),
            post_norm=_norm_weight(lyr.post_attention_layernorm.weight),
            q=lp.q, k=lp.k, v=lp.v, o=lp.o, gate=lp.gate, up=lp.up, down=lp.down,
            qkv_bias=lp.qkv_bias, o_bias=lp.o_bias, lora_q=lora[0], lora_v=lora[1],
            scaling=scal[0] if scal[0] is not None else 1.0, scaling_v=scal[1],
            n_heads=self.n_heads, n_kv=self.n_kv, head_dim=self.head_dim, eps=eps_in,
            dropout=max(_dropout_p(d) for d in drop if d is not None) if any(
                d is not None for d in drop) else 0.0,
            lora_dropout=tuple(drop), attn_scale=getattr(lp.attn, "scaling", None))


def model_plan(causal_lm):
    """The checked plan of this model, built once and kept on it; None when the fused path does
    not take the model (the reason printed once, as solution/model.py:152-162 does)."""
    plan = causal_lm.__dict__.get(_PLAN_KEY)
    if plan is None:
        try:
            plan = ModelPlan(causal_lm)
        except Exception as exc:  # noqa: BLE001 - any unexpected layout: not ours to run
            plan = False
            print(f"[testt_amd] fused path off for this model: {exc}", flush=True)
        causal_lm.__dict__[_PLAN_KEY] = plan
    return plan or None


def can_run(causal_lm, input_ids, attention_mask, labels, extra):
    """Whether fused_forward takes this call (solution/model.py:165-192): a labelled training
    forward with grad enabled, [batch, seq] input_ids / attention_mask / labels on a HIP device,
    only the allowed keyword arguments, fp16 autocast, a model the plan covers, and LoRA only
    on q/v in a form the plan reproduces."""
    if not (causal_lm.training and torch.is_grad_enabled() and labels is not None):
        return False
    if input_ids is None or attention_mask is None or input_ids.dim() != 2:
        return False
    if attention_mask.shape != input_ids.shape or labels.shape != input_ids.shape:
        return False
    if not kernels_ok(input_ids):
        return False
    for key, value in extra.items():
        if key not in _ALLOWED_KWARGS or (key not in _ANY_VALUE_KWARGS and value):
            return False
    dev = input_ids.device.type
    if not torch.is_autocast_enabled(dev) or torch.get_autocast_dtype(dev) != torch.float16:
        return False
    plan = model_plan(causal_lm)
    if plan is None:
        return False
    for lp in plan.layers:
        if _lora_parts(lp.attn.k_proj) is not None:
            return False
        if any(_lora_parts(m) is False for m in lp.lora_modules):
            return False
    return True


def fused_forward(causal_lm, input_ids, attention_mask, labels, num_items_in_batch):
    """CausalLMOutputWithPast(loss=loss, logits=HeadStats) of one labelled training forward of
    `causal_lm` (solution/model.py:209-279); call it where can_run holds.  The loss is
    differentiable with respect to the LoRA parameters."""
    from transformers.modeling_outputs import CausalLMOutputWithPast

    plan = model_plan(causal_lm)
    if plan is None:
        raise ValueError("fused_forward: the fused path does not take this model")
    batch, seq = input_ids.shape
    # The model's own rotary embedding at positions 0 .. seq-1 (any rope scaling it has),
    # fp32 [seq, head_dim], as the reference takes them (solution/model.py:227-232).
    shape_ref = torch.empty((1, 1, 1), dtype=torch.float32, device=input_ids.device).expand(
        batch, seq, plan.hidden)
    position_ids = torch.arange(seq, device=input_ids.device).unsqueeze(0)
    cos, sin = plan.rotary(shape_ref, position_ids)
    cos, sin = cos[0].float(), sin[0].float()
    layers = [plan.layer_weights(lp) for lp in plan.layers]
    head = plan.head.weight
    tied = head is plan.embed.weight
    weights = ModelWeights(embed=plan.embed.weight, layers=layers,
                           final_norm=_norm_weight(plan.norm.weight),
                           inv_freq=None, eps=plan.norm.variance_epsilon,
                           head=None if tied else head)
    loss, stats = _forward(weights, cos, sin, input_ids, attention_mask, labels,
                           num_items_in_batch)
    return CausalLMOutputWithPast(loss=loss, logits=stats)


# --------------------------------------------------------------------------------------------
# The path on plain tensors


@dataclass
class ModelWeights:
    embed: torch.Tensor                         # [V, H], fp16 or fp32 (the tied head reads it)
    layers: list                                # layer.LayerWeights per decoder layer
    final_norm: torch.Tensor                    # fp32 [H]
    inv_freq: torch.Tensor                      # fp32 [head_dim / 2] rotary frequencies, or None
    eps: float = 1e-6
    head: torch.Tensor = field(default=None)    # [V, H]; None: tied to `embed`


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


def forward_weights(model, input_ids, attention_mask, labels, num_items_in_batch=None):
    """(loss, HeadStats) of one labelled training forward of the plain-tensor `model`
    (ModelWeights with `inv_freq`): the path of fused_forward without a transformers model."""
    if input_ids.dim() != 2 or attention_mask.shape != input_ids.shape or \
            labels.shape != input_ids.shape:
        raise ValueError("input_ids, attention_mask and labels must share one [batch, seq] shape")
    cos, sin = rotary_tables(model.inv_freq, input_ids.shape[1])
    return _forward(model, cos, sin, input_ids, attention_mask, labels, num_items_in_batch)


def _forward(model, cos, sin, input_ids, attention_mask, labels, num_items_in_batch):
    batch, seq = input_ids.shape
    dev = input_ids.device
    pos_idx = attention_mask.reshape(-1).nonzero().squeeze(1)

    ids = input_ids.reshape(-1).index_select(0, pos_idx)
    s = torch.nn.functional.embedding(ids, model.embed).float()
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
    """The trainable tensors of a ModelWeights: (A_q, B_q, A_v, B_v) per layer."""
    out = []
    for w in model.layers:
        for pair in (w.lora_q, w.lora_v):
            if pair is not None:
                out += list(pair)
    return out
