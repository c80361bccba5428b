"""CPU: the window in which FrozenNF4Linear takes the fused NF4-dequant GEMM
(testt_amd/nf4_gemm.py fused_fits), checked against every comparison of the fused kernels with
unpack + hipBLASLt that `bench.py --nf4-gemm` measured on MI355X (256 CUs) at Qwen2.5-1.5B's
projections: the rule picks the faster path in each, and the two wins it leaves to unpack +
hipBLASLt (256 rows, 280 tiles, just past one wave) are listed as such."""

import pytest

from testt_amd import nf4_gemm

CUS = 256
QKV, O, GU, DOWN = (2048, 1536), (1536, 1536), (17920, 1536), (1536, 8960)   # (W rows, cols)

# (projection, rows, fused faster?) from the sweep: forward y = x W^T
FWD = [(QKV, 16, False), (QKV, 64, False), (QKV, 256, False), (QKV, 512, False),
       (QKV, 1024, True), (QKV, 2048, True),
       (O, 16, False), (O, 512, False), (O, 2048, True),
       (GU, 16, True), (GU, 64, True), (GU, 512, False), (GU, 1024, False), (GU, 2048, False),
       (DOWN, 16, False), (DOWN, 1024, False), (DOWN, 2048, False)]
# input gradient dx = dy W
GRAD = [(QKV, 16, False), (QKV, 512, False), (QKV, 1024, True), (QKV, 2048, False),
        (O, 64, False), (O, 512, False), (O, 1024, True), (O, 2048, False),
        (GU, 64, False), (GU, 512, False), (GU, 2048, False),
        (DOWN, 16, True), (DOWN, 64, True), (DOWN, 512, False), (DOWN, 2048, False)]


@pytest.mark.parametrize("w,rows,faster", FWD)
def test_forward_window_matches_measurements(w, rows, faster):
    n, k = w
    assert nf4_gemm.fused_fits(rows, n, k, nf4_gemm.FWD_TILE, CUS) == faster


@pytest.mark.parametrize("w,rows,faster", GRAD)
def test_grad_input_window_matches_measurements(w, rows, faster):
    n, k = w
    assert nf4_gemm.fused_fits(rows, k, n, nf4_gemm.GRAD_TILE, CUS) == faster


def test_window_edges():
    # half a wave is in, one tile less is out; a full wave is in, one tile more is out
    assert nf4_gemm.fused_fits(128, 128 * 128, 64, (128, 128), 256)
    assert not nf4_gemm.fused_fits(128, 127 * 128, 64, (128, 128), 256)
    assert nf4_gemm.fused_fits(256, 128 * 128, 64, (128, 128), 256)
    assert not nf4_gemm.fused_fits(256, 129 * 128, 64, (128, 128), 256)
    assert not nf4_gemm.fused_fits(256, 128 * 128, nf4_gemm.FUSED_MAX_CONTRACTION + 64,
                                   (128, 128), 256)


def test_wins_left_outside_the_window():
    """gate|up forward at 256 rows (fused 39.4 against 49.1 us) and down's input gradient at 256
    rows (27.7 against 35.7 us) fall just past one wave (280 tiles); the rule leaves them to
    unpack + hipBLASLt rather than widen the window past q|k|v at 2560 rows (320 tiles, fused
    26-34% behind)."""
    assert not nf4_gemm.fused_fits(256, GU[0], GU[1], nf4_gemm.FWD_TILE, CUS)
    assert not nf4_gemm.fused_fits(256, DOWN[1], DOWN[0], nf4_gemm.GRAD_TILE, CUS)
    assert not nf4_gemm.fused_fits(2560, QKV[0], QKV[1], nf4_gemm.FWD_TILE, CUS)
