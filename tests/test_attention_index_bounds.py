"""CPU regression test: the varlen attention kernels' index arithmetic stays in bounds.

testt_amd/csrc/attention.hip launches the varlen forward on a (heads, sequences, ceil(M/64))
grid, the backward on (heads, sequences, 2 ceil(M/64)) (even z: dK/dV of a key block, odd z:
dQ of a query block), the delta kernel on (heads, 1, ceil(M/64)) and the reduce on M*NKV*16
items.  Workgroups past a sequence's blocks exit; rows are clamped to the sequence's last row
before every load; sequence bounds come from device memory (cu_seqlens) and a bound outside
[0, M] empties the sequence.  This test replays that arithmetic with numpy for every workgroup
and lane and checks each global index against its buffer, for ragged batches, an empty
sequence, T = 77, single tokens and malformed bounds.  No GPU is needed.
"""

import numpy as np
import pytest

BQ = BK = 64
D = 128


def _lanes():
    """(wave, lane) -> (w, l%16, l/16) for the 256 threads of a workgroup."""
    t = np.arange(256)
    return t // 64, (t % 64) & 15, (t % 64) >> 4


def _tile_rows():
    """Rows (2rp, 2rp+1) and 8-dim chunk dc each thread stages (tile_item, items 0 and 1)."""
    t = np.arange(256)
    lane, wv = t & 63, t >> 6
    out = []
    for it in range(2):
        wi = wv + 4 * it
        rp = 16 * (wi & 1) + ((lane >> 1) & 7) + 8 * (lane >> 5)
        dc = 4 * (wi >> 1) + (lane & 1) + 2 * ((lane >> 4) & 1)
        out.append((rp, dc))
    return out


def _seq(cu, b, M):
    s0, s1 = int(cu[b]), int(cu[b + 1])
    ok = 0 <= s0 <= s1 <= M
    return (s1 - s0 if ok else 0), (s0 if ok else 0)


def _check_tile(r0, length, base, W, col0, limit):
    for rp, dc in _tile_rows():
        for r in (2 * rp, 2 * rp + 1):
            row = np.minimum(r0 + r, length - 1)
            idx = (base + row) * W + col0 + 8 * dc + 7
            assert idx.min() >= 0 and idx.max() < limit, (r0, length, idx.max(), limit)


def replay(cu, M, NH, NKV, T_rope=None):
    """Every index of the forward, backward, delta and reduce launches for bounds cu."""
    B = len(cu) - 1
    W = (NH + 2 * NKV) * D
    HD = NH * D
    rep = NH // NKV
    slots = -(-M // BQ)
    w, ql, gr = _lanes()
    qkv_n, out_n, lse_n, part_n = M * W, M * HD, NH * M, NH * M * D
    for h in range(NH):
        g = h // rep
        for b in range(B):
            length, base = _seq(cu, b, M)
            nb = -(-length // BQ)
            # forward: z -> query block nb - 1 - z
            for z in range(slots):
                qb = nb - 1 - z
                if qb < 0:
                    continue
                q_abs = qb * BQ + 16 * w + ql
                qrow = np.minimum(q_abs, length - 1)
                assert ((base + qrow) * W + h * D + 32 * 3 + 8 * gr + 7).max() < qkv_n
                for kb in range(qb + 2):                    # block qb + 1: the clamped prefetch
                    _check_tile(kb * BK, length, base, W, (NH + g) * D, qkv_n)
                    _check_tile(kb * BK, length, base, W, (NH + NKV + g) * D, qkv_n)
                st = q_abs < length
                if st.any():
                    assert ((base + q_abs[st]) * HD + h * D + 16 * 7 + 4 * gr[st] + 3).max() < out_n
                    assert (h * M + base + q_abs[st]).max() < lse_n
            # backward: even z -> dK/dV of key block z/2, odd z -> dQ of query block nb-1-z/2
            for z in range(2 * slots):
                if z % 2 == 0:
                    kb = z // 2
                    if kb >= nb:
                        continue
                    key = kb * BK + 16 * w + ql
                    kc = np.minimum(key, length - 1)
                    assert ((base + kc) * W + (NH + NKV + g) * D + 32 * 3 + 8 * gr + 7).max() < qkv_n
                    for qb in range(kb, nb + 1):                 # + the clamped prefetch
                        _check_tile(qb * BQ, length, base, W, h * D, qkv_n)      # Q
                        _check_tile(qb * BQ, length, base, HD, h * D, out_n)     # dO
                        t = np.minimum(qb * BQ + (np.arange(256) & 63), length - 1)
                        assert (h * M + base + t).max() < lse_n               # lse, D
                    st = key < length
                    if st.any():
                        assert ((h * M + base + key[st]) * D + 16 * 7 + 4 * gr[st] + 3).max() < part_n
                else:
                    qb = nb - 1 - z // 2
                    if qb < 0:
                        continue
                    q_abs = qb * BQ + 16 * w + ql
                    qc = np.minimum(q_abs, length - 1)
                    assert ((base + qc) * W + h * D + 32 * 3 + 8 * gr + 7).max() < qkv_n
                    assert ((base + qc) * HD + h * D + 32 * 3 + 8 * gr + 7).max() < out_n
                    assert (h * M + base + qc).max() < lse_n
                    for kb in range(qb + 2):
                        _check_tile(kb * BK, length, base, W, (NH + g) * D, qkv_n)
                        _check_tile(kb * BK, length, base, W, (NH + NKV + g) * D, qkv_n)
                    st = q_abs < length
                    if st.any():
                        tok = base + q_abs[st]
                        assert tok.max() < M
                        # dQ row, first and second half (RoPE's transposed rotation)
                        assert (tok * W + h * D + 16 * 3 + 4 * gr[st] + 64 + 3).max() < qkv_n
                        if T_rope is not None:
                            # table row t < T_rope, dims d .. d+3 and d+64 .. d+67, d <= 60
                            assert 60 + 64 + 3 < D
    # delta: the padded kernel over one row of M positions (b = 0, T = M)
    for h in range(NH):
        for qb in range(slots):
            q_abs = qb * BQ + 16 * w + ql
            qc = np.minimum(q_abs, M - 1)
            assert (qc * HD + h * D + 32 * 3 + 8 * gr + 7).max() < out_n
            st = q_abs < M
            assert (h * M + q_abs[st]).max() < lse_n
    # reduce: item -> (token, key/value head, 4-dim slice of the first half)
    it = np.arange(M * NKV * 16)
    j = it & 15
    tg = it >> 4
    tok = tg // NKV
    gg = tg - tok * NKV
    d = 4 * j
    for r in range(rep):
        row = ((gg * rep + r) * M + tok) * D
        assert (row + d + 64 + 3).max() < part_n
    assert (tok * W + (NH + NKV + gg) * D + d + 64 + 3).max() < qkv_n


CASES = [
    ((512, 152, 128, 96), 12, 2),
    ((512, 512, 512, 512), 12, 2),
    ((512, 0, 77, 1), 12, 2),
    ((77,), 12, 2),
    ((1, 1, 1), 4, 4),
    ((130, 64, 63, 65), 8, 2),
]


@pytest.mark.parametrize("lengths,NH,NKV", CASES)
def test_varlen_attention_indices_in_bounds(lengths, NH, NKV):
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int64)
    replay(cu, int(cu[-1]), NH, NKV, T_rope=512)


@pytest.mark.parametrize("cu", [[0, 5, 3, 10], [0, 12, 10], [-4, 6, 10], [0, 4, 99]])
def test_malformed_bounds_empty_the_sequence(cu):
    """A bound outside [0, M] or a decreasing pair makes that sequence empty; the others stay
    in bounds."""
    cu = np.array(cu, dtype=np.int64)
    M = 10
    replay(cu, M, 4, 2)
    for b in range(len(cu) - 1):
        length, base = _seq(cu, b, M)
        assert 0 <= base and base + length <= M
