"""CPU: the window in which FrozenNF4Linear takes the fused NF4-dequant GEMM
(testt_amd/nf4_gemm.py fused_fits, forward_split_tiles, grad_split_tiles) and the split count
of the kernels that cut the contraction (split_count), checked against what `bench.py
--nf4-gemm` measured on MI355X (256 CUs, kernel trace of 40 queued calls) at Qwen2.5-1.5B's
projections, 16 to 2048 rows: the rule takes the faster path wherever the two differ by more
than 4%; the two wins it leaves to unpack + hipBLASLt (256 rows, 280 tiles, just past one wave)
are listed as such."""

import pytest

from testt_amd import nf4_gemm

CUS = 256
QKV, O, GU, DOWN = (2048, 1536), (1536, 1536), (17920, 1536), (1536, 8960)   # (W rows, cols)
LEVEL = 0.04

# (projection, rows, fused us (split as split_count picks), unpack + hipBLASLt us)
FWD = [(QKV, 16, 9.36, 14.09), (QKV, 64, 11.79, 14.66), (QKV, 256, 16.23, 17.70),
       (QKV, 512, 19.27, 18.82), (QKV, 1024, 24.67, 25.09), (QKV, 2048, 27.64, 28.03),
       (O, 16, 9.36, 13.66), (O, 64, 10.97, 14.30), (O, 256, 14.85, 14.45),
       (O, 512, 17.81, 17.16), (O, 1024, 24.63, 22.90), (O, 2048, 25.55, 25.54),
       (GU, 16, 18.37, 57.39), (GU, 64, 24.15, 37.63), (GU, 512, 63.69, 55.27),
       (GU, 1024, 116.14, 94.18), (GU, 2048, 222.58, 139.78),
       (DOWN, 16, 12.71, 38.46), (DOWN, 64, 17.66, 40.45), (DOWN, 256, 23.90, 42.16),
       (DOWN, 512, 37.17, 53.16), (DOWN, 1024, 64.37, 59.81), (DOWN, 2048, 135.95, 88.57)]
# input gradient dx = dy W
GRAD = [(QKV, 16, 10.68, 17.38), (QKV, 64, 13.08, 21.23), (QKV, 256, 17.71, 20.80),
        (QKV, 512, 23.05, 22.15), (QKV, 1024, 30.66, 32.76), (QKV, 2048, 41.40, 34.36),
        (O, 16, 9.51, 14.70), (O, 64, 11.11, 17.92), (O, 256, 14.58, 17.43),
        (O, 512, 18.42, 18.48), (O, 1024, 20.02, 25.34), (O, 2048, 29.09, 28.33),
        (GU, 16, 22.42, 75.14), (GU, 64, 26.47, 99.31), (GU, 256, 43.96, 131.56),
        (GU, 512, 77.97, 162.57), (GU, 1024, 158.09, 221.39), (GU, 2048, 313.20, 195.79),
        (DOWN, 16, 19.02, 24.70), (DOWN, 64, 19.50, 26.50), (DOWN, 512, 46.02, 40.98),
        (DOWN, 1024, 77.95, 47.08), (DOWN, 2048, 146.22, 85.43)]


def fwd_fused(rows, w):
    n, k = w
    return nf4_gemm.fused_fits(rows, n, k, nf4_gemm.FWD_TILE, CUS,
                               nf4_gemm.forward_split_tiles(k, CUS))


def grad_fused(rows, w):
    n, k = w
    return nf4_gemm.fused_fits(rows, k, n, nf4_gemm.GRAD_TILE, CUS,
                               nf4_gemm.grad_split_tiles(n, CUS))


def check(takes_fused, fused_us, unpack_us):
    if abs(fused_us - unpack_us) <= LEVEL * min(fused_us, unpack_us):
        return                                   # level: either path
    assert takes_fused == (fused_us < unpack_us)


@pytest.mark.parametrize("w,rows,fused_us,unpack_us", FWD)
def test_forward_window_matches_measurements(w, rows, fused_us, unpack_us):
    check(fwd_fused(rows, w), fused_us, unpack_us)


@pytest.mark.parametrize("w,rows,fused_us,unpack_us", GRAD)
def test_grad_input_window_matches_measurements(w, rows, fused_us, unpack_us):
    check(grad_fused(rows, w), fused_us, unpack_us)


def test_window_edges():
    # half a wave is in, one tile less is out; a full wave is in, one tile more is out
    assert nf4_gemm.fused_fits(128, 128 * 128, 64, (128, 128), 256)
    assert not nf4_gemm.fused_fits(128, 127 * 128, 64, (128, 128), 256)
    assert nf4_gemm.fused_fits(256, 128 * 128, 64, (128, 128), 256)
    assert not nf4_gemm.fused_fits(256, 129 * 128, 64, (128, 128), 256)
    assert not nf4_gemm.fused_fits(256, 128 * 128, nf4_gemm.FUSED_MAX_CONTRACTION + 64,
                                   (128, 128), 256)
    # below half a wave only where the split kernels take it
    assert not nf4_gemm.fused_fits(128, 32 * 128, 64, (128, 128), 256)
    assert nf4_gemm.fused_fits(128, 32 * 128, 64, (128, 128), 256, split_tiles=32)
    assert not nf4_gemm.fused_fits(128, 33 * 128, 64, (128, 128), 256, split_tiles=32)


def test_wins_left_outside_the_window():
    """gate|up forward at 256 rows (fused 40.2 against 48.8 us) and down's input gradient at 256
    rows (27.9 against 35.7 us) fall just past one wave (280 tiles); the rule leaves them to
    unpack + hipBLASLt rather than widen the window past q|k|v at 2560 rows (320 tiles, fused
    26-34% behind)."""
    assert not fwd_fused(256, GU)
    assert not grad_fused(256, DOWN)
    assert not fwd_fused(2560, QKV)


# (projection, rows, split count split_count picks: the best of the sweep or within 4% of it)
@pytest.mark.parametrize("w,rows,splits", [
    (QKV, 16, 12), (QKV, 64, 8), (QKV, 128, 6), (QKV, 256, 4), (QKV, 512, 3), (QKV, 1024, 1),
    (O, 16, 12), (O, 64, 12), (O, 256, 6), (O, 512, 4), (DOWN, 16, 20), (DOWN, 64, 20),
    (DOWN, 128, 20), (DOWN, 256, 10), (DOWN, 512, 5), (GU, 16, 1)])
def test_forward_split_count(w, rows, splits):
    """Splits of the forward's contraction (q|k|v at 16 rows: 7.9 us with 12 splits, 21.8 with
    none; down at 16 rows: 13.3 with 20, 109.0 with none)."""
    n, k = w
    assert nf4_gemm.split_count(rows, n, k, CUS) == splits


@pytest.mark.parametrize("w,rows,splits", [
    (QKV, 16, 16), (QKV, 64, 8), (QKV, 512, 4), (QKV, 1024, 1), (O, 16, 8), (O, 64, 8),
    (O, 512, 2), (GU, 256, 10), (GU, 1024, 8), (DOWN, 16, 1)])
def test_grad_split_count(w, rows, splits):
    """Splits of the input gradient's contraction over W's rows (gate|up at 1024 rows: 152 us
    with 8 splits, 220 with none, though its 192 tiles fill most of a wave)."""
    n, k = w
    assert nf4_gemm.split_count(rows, k, n, CUS, nf4_gemm.GRAD_TILE) == splits


def test_split_count_small_contraction():
    assert nf4_gemm.split_count(16, 128, 64, CUS) == 1       # one K tile: nothing to split
    # four K tiles: two splits would save two steps (1.4 us) for a summing launch (2.5 us)
    assert nf4_gemm.split_count(16, 128, 256, CUS) == 1
    assert nf4_gemm.split_count(16, 128, 64 * 2000, CUS) <= nf4_gemm.MAX_SPLITS
    assert nf4_gemm.split_count(16, 128 * 200, 1536, CUS) == 1   # 200 tiles, a short contraction


@pytest.mark.parametrize("rows,gate_up,down", [
    (256, 8, 2), (888, 8, 2), (1024, 8, 2), (1536, 4, 2), (2048, 4, 2), (3072, 2, 1),
    (8192, 1, 1), (0, 1, 1)])
def test_mlp_split_parts(rows, gate_up, down):
    """The K slices of the MLP's split products by row count (testt_amd/mlp.py split_parts),
    at Qwen2.5-1.5B's shapes: the gate|up input gradient [rows, 17920] @ [17920, 1536] and the
    down projection's forward [rows, 8960] @ [8960, 1536]."""
    from testt_amd import mlp
    assert mlp.split_parts(rows, 1536, 17920, "gate_up") == gate_up
    assert mlp.split_parts(rows, 1536, 8960, "down") == down
