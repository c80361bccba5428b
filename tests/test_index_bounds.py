"""CPU regression test: the RoPE pack kernels' per-thread index arithmetic stays in bounds.

testt_amd/csrc/rope_pack.hip maps workgroups of 512 (forward) and 256 (backward) threads onto
(token, head, 8-dim chunk) items.  When the item count is not a multiple of the workgroup size,
the last workgroup holds threads past the last item; they must form only in-bounds addresses
(they take the last item's indices).  This test replays that arithmetic for every thread of the
launch grid with numpy, at both workgroup sizes, and checks each global and LDS index against
its buffer, for the GPU tests' shapes (including 53 tokens, a fraction of a workgroup) and head
counts other than Qwen2.5-1.5B's.  No GPU is needed.
"""

import numpy as np
import pytest

def max_tok(threads):
    """rope_max_tok<THREADS>(): tokens whose cos/sin rows one workgroup stages in LDS."""
    return threads // 18 + 2


def _fwd_bwd_addresses(rows, B, T, NH, NKV, D, with_inv, THREADS):
    """Largest index each buffer is touched at, for the forward and backward vector kernels."""
    HALF = D // 2
    heads = NH + 2 * NKV
    items = heads * (HALF // 8)
    assert HALF == 64 and items >= 18           # the host's condition for the vector kernels
    slots = B * T
    total = rows * items
    tok_blocks = -(-total // THREADS)
    tid = np.arange(THREADS)
    worst = {"qkv": -1, "lq": -1, "lv": -1, "grad_q": -1, "grad_kv": -1, "out_q": -1,
             "out_kv": -1, "lds": -1, "pos": -1, "tab": -1, "ntok": 0}
    pos = np.arange(rows) % slots                # any in-range positions
    for b in range(tok_blocks):
        g0 = b * THREADS
        tok0 = g0 // items
        ntok = (min(g0 + THREADS, total) - 1) // items - tok0 + 1
        worst["ntok"] = max(worst["ntok"], ntok)
        active = g0 + tid < total
        g = np.where(active, g0 + tid, total - 1)
        tok = g // items
        it = g - tok * items
        h, c = it // (HALF // 8), it % (HALF // 8)
        worst["qkv"] = max(worst["qkv"], int((tok * heads * D + h * D + 8 * c + HALF + 7).max()))
        q = h < NH
        v = h >= NH + NKV
        if q.any():
            worst["lq"] = max(worst["lq"], int((tok * NH * D + h * D + 8 * c + HALF + 7)[q].max()))
        if v.any():
            lv = tok * NKV * D + (h - NH - NKV) * D + 8 * c + HALF + 7
            worst["lv"] = max(worst["lv"], int(lv[v].max()))
        # table staging: i = tid, tid + THREADS, ... < ntok * D/2 float4; entry i is float4
        # i % (D/2) of token tok0 + i // (D/2)'s row (cos, then sin), at t = pos % T
        stage = np.arange(0, ntok * (D // 2))
        worst["pos"] = max(worst["pos"], int(tok0 + stage.max() // (D // 2)), int(tok.max()))
        worst["lds"] = max(worst["lds"], int(stage.max()))
        t_st = pos[tok0 + stage // (D // 2)] % T
        q4 = stage % (D // 2)
        worst["tab"] = max(worst["tab"], int((t_st * D + 4 * (q4 % (D // 4)) + 3).max()))
        # after the barrier (active threads only)
        per = D // 2
        lds = (tok - tok0) * per + D // 4 + HALF // 4 + 2 * c + 1
        worst["lds"] = max(worst["lds"], int(lds[active].max()))
        p = pos[tok]
        bb, t = p // T, p % T
        oq = ((bb * NH + h) * T + t) * D + HALF + 8 * c + 7
        okv = ((bb * NKV + np.where(v, h - NH - NKV, h - NH)) * T + t) * D + HALF + 8 * c + 7
        if (active & q).any():
            worst["out_q"] = max(worst["out_q"], int(oq[active & q].max()))
            worst["grad_q"] = worst["out_q"]
        if (active & ~q).any():
            worst["out_kv"] = max(worst["out_kv"], int(okv[active & ~q].max()))
        if (~q).any():
            worst["grad_kv"] = max(worst["grad_kv"], int(okv[~q].max()))
    if with_inv:
        zero_items = slots * items
        for b in range(-(-zero_items // THREADS)):
            g = b * THREADS + tid
            p = g // items
            ok = p < slots
            it = g - p * items
            h, c = it // (HALF // 8), it % (HALF // 8)
            bb, t = p // T, p % T
            q = h < NH
            oq = ((bb * NH + h) * T + t) * D + HALF + 8 * c + 7
            okv = ((bb * NKV + np.where(h >= NH + NKV, h - NH - NKV, h - NH)) * T + t) * D \
                + HALF + 8 * c + 7
            if (ok & q).any():
                worst["out_q"] = max(worst["out_q"], int(oq[ok & q].max()))
            if (ok & ~q).any():
                worst["out_kv"] = max(worst["out_kv"], int(okv[ok & ~q].max()))
    return worst


@pytest.mark.parametrize("threads", [512, 256])
@pytest.mark.parametrize("heads", [(12, 2), (1, 1), (3, 0), (28, 4)])
@pytest.mark.parametrize("lengths,seq", [((512,) * 4, 512), ((512, 152, 128, 96), 512),
                                         ((77, 75), 77), ((40, 0, 13), 64), ((30, 20), 32),
                                         ((1,), 1), ((3, 0, 0), 4)])
def test_rope_vector_kernels_stay_in_bounds(lengths, seq, heads, threads):
    NH, NKV = heads
    D = 128
    B = len(lengths)
    rows = sum(lengths)
    w = _fwd_bwd_addresses(rows, B, seq, NH, NKV, D, rows != B * seq, threads)
    MAX_TOK = max_tok(threads)
    assert w["ntok"] <= MAX_TOK
    assert w["qkv"] < rows * (NH + 2 * NKV) * D
    assert w["lq"] < rows * NH * D and w["lv"] < rows * NKV * D
    assert w["pos"] < rows
    assert w["tab"] < seq * D
    assert w["lds"] < MAX_TOK * D // 2
    assert w["out_q"] < B * NH * seq * D
    assert w["out_kv"] < B * NKV * seq * D
    assert w["grad_kv"] < B * NKV * seq * D
