"""Seeded synthetic inputs at the shapes of the QLoRA step of Qwen2.5-1.5B.

Used by bench.py, the smoke test and the parity tests, so that every consumer draws the same
tensors.  Everything is generated on the CPU with torch.Generator(seed) (deterministic across
machines) and then moved to the requested device.

Shapes (Qwen2.5-1.5B): hidden H=1536, intermediate I=8960, 12 query heads, 2 key/value heads,
head_dim 128, vocab 151936; the step is batch 4 x seq 512, i.e. M=2048 real tokens.
"""

from types import SimpleNamespace

import numpy as np
import torch

HIDDEN = 1536
INTER = 8960
N_HEADS = 12
N_KV = 2
HEAD_DIM = 128
VOCAB = 151936
BATCH = 4
SEQ = 512
ROPE_THETA = 1e6
RMS_EPS = 1e-6

# The 16 NormalFloat4 levels (QLoRA, Dettmers et al. 2023, arXiv:2305.14314, appendix E), as
# fp32 values.
NF4_LEVELS = (
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
)


def gen(seed):
    return torch.Generator().manual_seed(int(seed))


def dynamic_code_signed():
    """256-entry signed dynamic 8-bit code (the table bitsandbytes' double quant indexes).

    Dynamic tree quantization (Dettmers et al. 2021, "8-bit Optimizers via Block-wise
    Quantization"): after the sign, exponent level i (0..6) carries 2^i linearly spaced
    fractions -- the midpoints of linspace(0.1, 1, 2^i + 1) -- scaled by 10^(i - 6); the table
    also holds 0 and 1, and is sorted ascending.  254 + 2 = 256 values."""
    vals = [0.0, 1.0]
    for level in range(7):
        edges = np.linspace(0.1, 1.0, 2 ** level + 1)
        mids = (edges[:-1] + edges[1:]) / 2.0 * (10.0 ** (level - 6))
        vals.extend(mids.tolist())
        vals.extend((-mids).tolist())
    assert len(vals) == 256
    return torch.tensor(sorted(vals), dtype=torch.float32)


class Params4bit(SimpleNamespace):
    """What a bitsandbytes Params4bit exposes to the kernels: `.data` and `.quant_state`."""


def nf4_weight(n_out, n_in, seed, device="cpu", absmax2_range=(0.01, 0.1), offset=0.03):
    """A synthetic NF4 double-quant weight [n_out, n_in]: uniform codes, uniform absmax codes.

    Layout of bitsandbytes' 4-bit storage: data uint8 [n_out*n_in/2, 1], two codes per byte with
    the element of lower index in the high nibble; per 64 values one absmax stored as a uint8
    code into `state2.code`, scaled per 256 absmax blocks by `state2.absmax` and shifted by
    `offset`."""
    if (n_out * n_in) % 64:
        raise ValueError("n_out * n_in must be a multiple of the 64-value block")
    g = gen(seed)
    n_bytes = n_out * n_in // 2
    n_blocks = n_out * n_in // 64
    packed = torch.randint(0, 256, (n_bytes, 1), generator=g, dtype=torch.int32).to(torch.uint8)
    absmax_u8 = torch.randint(0, 256, (n_blocks,), generator=g, dtype=torch.int32).to(torch.uint8)
    lo, hi = absmax2_range
    absmax2 = lo + (hi - lo) * torch.rand((n_blocks + 255) // 256, generator=g)
    state2 = SimpleNamespace(code=dynamic_code_signed().to(device), absmax=absmax2.to(device),
                             blocksize=256)
    state = SimpleNamespace(quant_type="nf4", nested=True, state2=state2, blocksize=64,
                            shape=(n_out, n_in), absmax=absmax_u8.to(device),
                            offset=torch.tensor(offset, dtype=torch.float32).to(device),
                            code=torch.tensor(NF4_LEVELS, dtype=torch.float32).to(device),
                            dtype=torch.float16)
    return Params4bit(data=packed.to(device), quant_state=state)


def rmsnorm_inputs(rows=2048, hidden=HIDDEN, padded=None, seed=2, device="cpu"):
    """x fp32 ~N(0,1), delta fp16 ~N(0,0.5), weight fp32 ~1+N(0,0.02), pad_idx = distinct
    positions in [0, padded) (a permutation when padded == rows)."""
    g = gen(seed)
    padded = rows if padded is None else padded
    x = torch.randn(rows, hidden, generator=g)
    delta = (0.5 * torch.randn(rows, hidden, generator=g)).to(torch.float16)
    w = 1.0 + 0.02 * torch.randn(hidden, generator=g)
    pad_idx = torch.randperm(padded, generator=g)[:rows]
    return tuple(t.to(device) for t in (x, delta, w, pad_idx)) + (padded,)


def rmsnorm_grads(rows=2048, hidden=HIDDEN, padded=None, seed=3, device="cpu"):
    """dy fp16 ~N(0,1e-2), dypad fp32 [padded, H] ~N(0,1e-2), ds fp32 ~N(0,1e-2)."""
    g = gen(seed)
    padded = rows if padded is None else padded
    dy = (1e-2 * torch.randn(rows, hidden, generator=g)).to(torch.float16)
    dypad = 1e-2 * torch.randn(padded, hidden, generator=g)
    ds = 1e-2 * torch.randn(rows, hidden, generator=g)
    return tuple(t.to(device) for t in (dy, dypad, ds))


def swiglu_inputs(rows=2048, inter=INTER, seed=4, device="cpu", scale=1.0):
    g = gen(seed)
    return (scale * torch.randn(rows, 2 * inter, generator=g)).to(torch.float16).to(device)


def swiglu_grad(rows=2048, inter=INTER, seed=5, device="cpu"):
    g = gen(seed)
    return (1e-2 * torch.randn(rows, inter, generator=g)).to(torch.float16).to(device)


def rope_tables(seq=SEQ, head_dim=HEAD_DIM, theta=ROPE_THETA, device="cpu"):
    """cos, sin fp32 [seq, head_dim] as transformers' default rotary embedding builds them:
    inv_freq = 1/theta^(2j/d), angle = t * inv_freq, emb = cat(angle, angle)."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
    freqs = torch.arange(seq).float()[:, None] * inv[None, :]
    emb = torch.cat([freqs, freqs], dim=-1)
    return emb.cos().to(device), emb.sin().to(device)


def ragged_positions(lengths, seq):
    """pos_idx of right-padded rows with the given real lengths (attention_mask.nonzero())."""
    return torch.cat([b * seq + torch.arange(n) for b, n in enumerate(lengths)]).to(torch.int64)


def rope_inputs(lengths=(SEQ,) * BATCH, seq=SEQ, n_heads=N_HEADS, n_kv=N_KV, head_dim=HEAD_DIM,
                lora_dtype=torch.float32, seed=6, device="cpu"):
    """qkv fp16 ~N(0,1) [M, (NH+2NKV)*D]; LoRA q/v deltas ~N(0,1e-2); pos_idx for `lengths`."""
    g = gen(seed)
    pos = ragged_positions(lengths, seq)
    m = pos.numel()
    width = (n_heads + 2 * n_kv) * head_dim
    qkv = torch.randn(m, width, generator=g).to(torch.float16)
    lq = (1e-2 * torch.randn(m, n_heads * head_dim, generator=g)).to(lora_dtype)
    lv = (1e-2 * torch.randn(m, n_kv * head_dim, generator=g)).to(lora_dtype)
    return tuple(t.to(device) for t in (qkv, lq, lv, pos))


def rope_grads(batch=BATCH, seq=SEQ, n_heads=N_HEADS, n_kv=N_KV, head_dim=HEAD_DIM, seed=7,
               device="cpu"):
    g = gen(seed)
    dq = (1e-2 * torch.randn(batch, n_heads, seq, head_dim, generator=g)).to(torch.float16)
    dk = (1e-2 * torch.randn(batch, n_kv, seq, head_dim, generator=g)).to(torch.float16)
    dv = (1e-2 * torch.randn(batch, n_kv, seq, head_dim, generator=g)).to(torch.float16)
    return tuple(t.to(device) for t in (dq, dk, dv))


def head_inputs(rows=256, hidden=HIDDEN, vocab=VOCAB, ignore_frac=0.1, seed=8, device="cpu"):
    """h fp16 ~N(0,1) [rows, H], tied W fp16 ~N(0,0.02) [V, H], labels uniform in [0, V) with
    `ignore_frac` of them set to -100."""
    g = gen(seed)
    h = torch.randn(rows, hidden, generator=g).to(torch.float16)
    w = (0.02 * torch.randn(vocab, hidden, generator=g)).to(torch.float16)
    targets = torch.randint(0, vocab, (rows,), generator=g, dtype=torch.int64)
    targets[torch.rand(rows, generator=g) < ignore_frac] = -100
    return h.to(device), w.to(device), targets.to(device)


def head_logits(rows=256, vocab=VOCAB, seed=8, device="cpu", scale=1.0):
    """fp16 logits with the spread of h @ W^T for h ~N(0,1), W ~N(0,0.02), H=1536 (std ~0.78),
    drawn directly (for kernel-level tests that skip the GEMM), plus labels as head_inputs."""
    g = gen(seed)
    z = (scale * 0.784 * torch.randn(rows, vocab, generator=g)).to(torch.float16)
    targets = torch.randint(0, vocab, (rows,), generator=g, dtype=torch.int64)
    targets[torch.rand(rows, generator=g) < 0.1] = -100
    return z.to(device), targets.to(device)
