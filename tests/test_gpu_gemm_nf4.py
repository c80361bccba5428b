"""GPU: the MFMA GEMM of testt_amd/csrc/gemm_nf4.hip.  The fp16 path against float64 sums of the
same fp16 products (one fp16 rounding of an fp32 accumulation: within 1 ulp plus
32 * 2^-24 * sum|terms|); the NF4 path bit-exact against unpack (the oracle-pinned unpack
kernel) followed by the fp16 path, and against float64 on the oracle's dequantised weights."""

import numpy as np
import pytest
import torch

from oracle.nf4 import dequant_state
from testt_amd import nf4, nf4_gemm, workloads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def within(got, exact, terms):
    h = exact.to(torch.float16)
    inf = torch.tensor(float("inf"), dtype=torch.float16, device=h.device)
    ulp = (torch.nextafter(h.abs(), inf) - h.abs()).double()
    err = (got.double() - exact).abs()
    bad = err > ulp + 32 * 2.0 ** -24 * terms
    assert not bool(bad.any()), f"{int(bad.sum())} of {bad.numel()} beyond, max err {float(err.max()):.3g}"


@pytest.mark.parametrize("M,N,K,with_bias", [(2048, 2048, 1536, True), (300, 256, 128, False),
                                             (1, 128, 64, True), (131, 384, 1536, False)])
def test_gemm_tn_fp16(M, N, K, with_bias):
    print(f"gemm_tn M={M} N={N} K={K} bias={with_bias}", flush=True)
    g = torch.Generator().manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g).to(torch.float16).to(DEV)
    w = (torch.randn(N, K, generator=g) / K ** 0.5).to(torch.float16).to(DEV)
    b = (0.1 * torch.randn(N, generator=g)).to(torch.float16).to(DEV) if with_bias else None
    y = nf4_gemm.gemm_tn(x, w, b)
    exact = x.double() @ w.double().t()
    terms = x.double().abs() @ w.double().abs().t()
    if b is not None:
        exact = exact + b.double()
        terms = terms + b.double().abs()
    within(y, exact, terms)


@pytest.mark.parametrize("rows,K,M", [((256,), 1536, 2048), ((256, 128, 128), 512, 77),
                                      ((128, 128), 64, 5)])
def test_gemm_tn_nf4(rows, K, M):
    print(f"gemm_tn_nf4 parts={rows} K={K} M={M}", flush=True)
    ws = [workloads.nf4_weight(r, K, seed=50 + i, device=DEV, absmax2_range=(0.005, 0.02),
                               offset=0.01) for i, r in enumerate(rows)]
    assert nf4_gemm.supported(torch.empty(M, K, dtype=torch.float16, device=DEV), ws)
    g = torch.Generator().manual_seed(M + K)
    x = torch.randn(M, K, generator=g).to(torch.float16).to(DEV)
    b = (0.1 * torch.randn(sum(rows), generator=g)).to(torch.float16).to(DEV)
    y = nf4_gemm.nf4_linear(x, ws, b, splits=1)
    w16 = nf4.unpack_concat(ws, DEV)
    assert torch.equal(y, nf4_gemm.gemm_tn(x, w16, b))        # same values, same sums
    wd = torch.from_numpy(np.concatenate([dequant_state(w) for w in ws]).astype(np.float64)).to(DEV)
    within(y, x.double() @ wd.t() + b.double(), x.double().abs() @ wd.abs().t() + b.double().abs())


@pytest.mark.parametrize("rows,K,M,splits", [
    ((256,), 1536, 16, 8), ((256, 128, 128), 320, 77, 4),   # 5 K tiles in 4 ways: 3 splits used
    ((128,), 8960, 16, 32), ((1536, 256, 256), 1536, 2048, 2), ((128,), 256, 3, 4),
    ((256,), 1536, 1, None)])                                # the split count split_count picks
def test_gemm_tn_nf4_split(rows, K, M, splits):
    """The contraction split: fp32 partials added in split order, bias added, one fp16 rounding.
    Against float64 sums over the oracle's dequantised weights (within 1 ulp plus
    32 * 2^-24 * sum|terms|, as the unsplit kernel), within twice that of the unsplit kernel
    (the same rounding of another order of fp32 sums), and the same bits on a second call."""
    print(f"gemm_tn_nf4_split parts={rows} K={K} M={M} splits={splits}", flush=True)
    ws = [workloads.nf4_weight(r, K, seed=70 + i, device=DEV, absmax2_range=(0.005, 0.02),
                               offset=0.01) for i, r in enumerate(rows)]
    g = torch.Generator().manual_seed(M + K + 7)
    x = torch.randn(M, K, generator=g).to(torch.float16).to(DEV)
    b = (0.1 * torch.randn(sum(rows), generator=g)).to(torch.float16).to(DEV)
    y = nf4_gemm.nf4_linear(x, ws, b, splits=splits)
    wd = torch.from_numpy(np.concatenate([dequant_state(w) for w in ws]).astype(np.float64)).to(DEV)
    terms = x.double().abs() @ wd.abs().t() + b.double().abs()
    within(y, x.double() @ wd.t() + b.double(), terms)
    one = nf4_gemm.nf4_linear(x, ws, b, splits=1)
    inf = torch.tensor(float("inf"), dtype=torch.float16, device=DEV)
    ulp = (torch.nextafter(one.abs(), inf) - one.abs()).double()
    assert bool(((y.double() - one.double()).abs() <= 2 * ulp + 64 * 2.0 ** -24 * terms).all())
    assert torch.equal(nf4_gemm.nf4_linear(x, ws, b, splits=splits), y)
    assert torch.equal(nf4_gemm.nf4_linear(x, ws, None, splits=splits),
                       nf4_gemm.nf4_linear(x, ws, torch.zeros_like(b), splits=splits))


@pytest.mark.parametrize("rows,K,M", [((1536, 256, 256), 1536, 2048), ((1536,), 1536, 2048),
                                      ((256, 128, 128), 512, 77), ((128,), 128, 1)])
def test_gemm_nn_nf4_grad_input(rows, K, M):
    """dx = dy @ W with W dequantised in the GEMM (the backward of nf4_linear): against float64
    sums over the oracle's dequantised weights (one fp16 rounding of fp32 sums: within 1 ulp
    plus 32 * 2^-24 * sum|terms|), and a contraction spanning the parts (q|k|v)."""
    print(f"gemm_nn_nf4 parts={rows} K={K} M={M}", flush=True)
    ws = [workloads.nf4_weight(r, K, seed=90 + i, device=DEV, absmax2_range=(0.005, 0.02),
                               offset=0.01) for i, r in enumerate(rows)]
    g = torch.Generator().manual_seed(M + K + len(rows))
    dy = (0.1 * torch.randn(M, sum(rows), generator=g)).to(torch.float16).to(DEV)
    assert nf4_gemm.grad_input_supported(dy, ws)
    dx = nf4_gemm.nf4_grad_input(dy, ws)
    wd = torch.from_numpy(np.concatenate([dequant_state(w) for w in ws]).astype(np.float64)).to(DEV)
    within(dx, dy.double() @ wd, dy.double().abs() @ wd.abs())
    # a strided dy (rows of a wider buffer) gives the same result
    wide = torch.zeros(M, sum(rows) + 64, dtype=torch.float16, device=DEV)
    wide[:, :sum(rows)] = dy
    assert torch.equal(nf4_gemm.nf4_grad_input(wide[:, :sum(rows)], ws), dx)


@pytest.mark.parametrize("rows,K,M,splits", [
    ((1536, 256, 256), 1536, 16, 8), ((256, 128, 128), 512, 77, 3),   # 8 steps in 3: 3 used
    ((8960, 8960), 1536, 16, 10), ((1536,), 1536, 300, 2), ((128,), 128, 1, None)])
def test_gemm_nn_nf4_split(rows, K, M, splits):
    """The input gradient with its contraction (W's rows, across the parts) split: against
    float64 sums over the oracle's dequantised weights (within 1 ulp plus 32 * 2^-24 *
    sum|terms|), within twice that of the unsplit kernel, and the same bits on a second call."""
    print(f"gemm_nn_nf4_split parts={rows} K={K} M={M} splits={splits}", flush=True)
    ws = [workloads.nf4_weight(r, K, seed=110 + i, device=DEV, absmax2_range=(0.005, 0.02),
                               offset=0.01) for i, r in enumerate(rows)]
    g = torch.Generator().manual_seed(M + K + 11)
    dy = (0.1 * torch.randn(M, sum(rows), generator=g)).to(torch.float16).to(DEV)
    dx = nf4_gemm.nf4_grad_input(dy, ws, splits=splits)
    wd = torch.from_numpy(np.concatenate([dequant_state(w) for w in ws]).astype(np.float64)).to(DEV)
    terms = dy.double().abs() @ wd.abs()
    within(dx, dy.double() @ wd, terms)
    one = nf4_gemm.nf4_grad_input(dy, ws, splits=1)
    inf = torch.tensor(float("inf"), dtype=torch.float16, device=DEV)
    ulp = (torch.nextafter(one.abs(), inf) - one.abs()).double()
    assert bool(((dx.double() - one.double()).abs() <= 2 * ulp + 64 * 2.0 ** -24 * terms).all())
    assert torch.equal(nf4_gemm.nf4_grad_input(dy, ws, splits=splits), dx)


@pytest.mark.parametrize("rows,K,splits", [((1536, 256, 256), 1536, 1), ((1536, 256, 256), 1536, 8),
                                           ((8960, 8960), 1536, 1), ((1536,), 8960, 20)])
def test_few_row_tiles_match_the_128_row_tiles(rows, K, splits):
    """Up to 32 rows the forward (and the split input gradient) run 32-row tiles: the same
    products in the same order, so the rows of a 16-row call equal the same rows computed
    inside a 40-row call (128-row tiles), bit for bit."""
    print(f"few-row tiles parts={rows} K={K} splits={splits}", flush=True)
    ws = [workloads.nf4_weight(r, K, seed=130 + i, device=DEV) for i, r in enumerate(rows)]
    g = torch.Generator().manual_seed(K + 5)
    x = torch.randn(40, K, generator=g).to(torch.float16).to(DEV)
    assert torch.equal(nf4_gemm.nf4_linear(x[:16].contiguous(), ws, splits=splits),
                       nf4_gemm.nf4_linear(x, ws, splits=splits)[:16])
    dy = (0.1 * torch.randn(40, sum(rows), generator=g)).to(torch.float16).to(DEV)
    if sum(rows) // 64 >= splits:
        assert torch.equal(nf4_gemm.nf4_grad_input(dy[:16].contiguous(), ws, splits=splits),
                           nf4_gemm.nf4_grad_input(dy, ws, splits=splits)[:16])


def test_rejects_shapes():
    x = torch.randn(8, 64, device=DEV).to(torch.float16)
    with pytest.raises(Exception):
        nf4_gemm.gemm_tn(x, torch.randn(100, 64, device=DEV).to(torch.float16))   # N % 128
    with pytest.raises(Exception):
        nf4_gemm.gemm_tn(torch.randn(8, 96, device=DEV).to(torch.float16),
                         torch.randn(128, 96, device=DEV).to(torch.float16))       # K % 64
    w = workloads.nf4_weight(192, 64, seed=3, device=DEV)                           # 192 rows
    assert not nf4_gemm.supported(x, [w])


def test_frozen_linear_fused_switch(monkeypatch):
    """FrozenNF4Linear with the fused NF4 GEMM forward and input gradient (forced on for this
    shape) against its unpack + hipBLASLt path: the same fp16 weights, sums in another order
    (relative L2 < 1e-3 for the output and the input gradient)."""
    from testt_amd import nf4_gemm
    ws = [workloads.nf4_weight(r, 512, seed=70 + i, device=DEV, absmax2_range=(0.005, 0.02),
                               offset=0.01) for i, r in enumerate((256, 128))]
    g = torch.Generator().manual_seed(6)
    x0 = torch.randn(200, 512, generator=g).to(torch.float16).to(DEV)
    b = (0.1 * torch.randn(384, generator=g)).to(torch.float16).to(DEV)
    gout = (1e-2 * torch.randn(200, 384, generator=g)).to(torch.float16).to(DEV)
    res = []
    calls = []
    grad = nf4_gemm.nf4_grad_input
    monkeypatch.setattr(nf4_gemm, "prefer_fused", lambda x, w: True)
    monkeypatch.setattr(nf4_gemm, "prefer_fused_grad_input", lambda dy, w: True)
    monkeypatch.setattr(nf4_gemm, "nf4_grad_input",
                        lambda dy, w: calls.append(dy.shape) or grad(dy, w))
    for fused in (False, True):
        monkeypatch.setattr(nf4, "USE_FUSED_NF4_GEMM", fused)
        x = x0.clone().requires_grad_(True)
        out = nf4.frozen_linear(x, ws, b)
        out.backward(gout)
        res.append((out.detach(), x.grad))
    assert calls == [(200, 384)]          # the fused input gradient ran in the fused pass only
    for i in (0, 1):
        ref = res[0][i].double()
        rel = float((res[1][i].double() - ref).norm() / ref.norm())
        assert rel < 1e-3, (i, rel)
