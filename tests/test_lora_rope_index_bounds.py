"""CPU regression test: the index arithmetic of the fused LoRA + RoPE forward
(lora_fwd_kernel<true>, soupk_lora_rope_fwd in testt_amd/csrc/lora.hip) stays in bounds and
writes every output element exactly once.

The kernel takes 16 rows per workgroup (grid.x) and splits the (NQ + NV + NK) / 16 column tiles
over grid.y parts at whole heads (8 tiles); wavefront w of a part takes tiles
t_begin + w + 32 i + 4 u (u < 4), pairing tile j (dims 16j..16j+15 of a head) with tile j + 4
(the rotation partners).  This test replays, with numpy, the grid and the per-lane addresses of
every load (qkv, B16 rows, cos / sin entries, positions) and store (the output rows) for the
GPU tests' shapes, and checks that the pairs are partners, the indices lie inside their buffers,
and the stores cover the [M, W] output exactly once.  No GPU is needed."""

import numpy as np
import pytest

KR, KBATCH, KROWS = 16, 4, 16


def column_parts(M, n_tiles, target=256):
    """column_parts() of lora.hip (soupk_lora_rope_fwd then caps it at the head count)."""
    row_blocks = -(-M // KROWS)
    parts = -(-target // row_blocks)
    parts = min(parts, max(1, n_tiles // (4 * KBATCH)))
    return max(parts, 1)


def tile_part(n, part, parts):
    return (n * part) // parts


@pytest.mark.parametrize("M,NH,NKV,T", [(2048, 12, 2, 512), (888, 12, 2, 512), (1, 12, 2, 1),
                                        (17, 4, 2, 40), (130, 4, 4, 130), (53, 2, 1, 64)])
def test_lora_rope_fwd_indices(M, NH, NKV, T):
    D = 128
    NQ, NV, NK = NH * D, NKV * D, NKV * D
    W = NQ + NK + NV
    nq16, nlora = NQ // 16, NQ // 16 + NV // 16
    n_tiles = nlora + NK // 16
    heads = n_tiles // 8
    parts = min(column_parts(M, nlora), W // 128)
    grid_x = -(-M // KROWS)
    written = np.zeros((M, W), dtype=np.int32)
    lane = np.arange(64)
    ql, gr = lane & 15, lane >> 4
    slots = 4 * T
    for by in range(parts):
        t_begin = 8 * tile_part(heads, by, parts)
        n16 = 8 * tile_part(heads, by + 1, parts)
        assert t_begin % 8 == 0 and n16 % 8 == 0 and n16 <= n_tiles
        for w in range(4):
            # cos / sin entries of the lane's dims (t < T): e .. e + 3 and e + 64 .. e + 67
            e_max = (T - 1) * 128 + 16 * w + 4 * gr.max() + 64 + 3
            assert e_max < T * 128
            t0 = t_begin + w
            while t0 < n16:
                for half in (0, 1):
                    tb = t0 + 4 * KBATCH * half
                    if half and not (t0 + 4 * KBATCH < n16):
                        break
                    # loads of the batch (tile clamped to n16 - 1; B16 rows clamped to nlora - 1)
                    for u in range(KBATCH):
                        tile = min(tb + 4 * u, max(n16 - 1, 0))
                        bt = min(tile, nlora - 1)
                        assert 0 <= (16 * bt + ql.max()) * KR + 4 * gr.max() + 3 < (NQ + NV) * KR
                        col = 16 * tile if tile < nq16 else (
                            NQ + NK + 16 * (tile - nq16) if tile < nlora
                            else NQ + 16 * (tile - nlora))
                        assert 0 <= col and col + 4 * gr.max() + 3 < W
                    for pr in range(KBATCH // 2):
                        ta = tb + 8 * pr
                        if ta >= n16:
                            break
                        tbp = ta + 4
                        assert tbp < n16 and ta % 8 == w and tbp % 8 == w + 4
                        col = 16 * ta if ta < nq16 else (
                            NQ + NK + 16 * (ta - nq16) if ta < nlora else NQ + 16 * (ta - nlora))
                        for bx in range(grid_x):
                            m = bx * KROWS + ql
                            ok = m < M
                            for i in range(4):
                                np.add.at(written, (m[ok], col + 4 * gr[ok] + i), 1)
                                np.add.at(written, (m[ok], col + 64 + 4 * gr[ok] + i), 1)
                t0 += 8 * KBATCH
    assert (written == 1).all(), (int((written == 0).sum()), int((written > 1).sum()))
    # every workgroup's rows read the positions at clamped rows; 32-bit store offsets
    assert M * W * 2 < 2 ** 32 and slots < 2 ** 31
