"""GPU: the split-K products of the MLP, the gate|up input gradient and the down projection's
forward (testt_amd/mlp.py matmul_split_k: batched hipBLASLt GEMMs with fp32 partials +
soupk_sum_partials).

soupk_sum_partials is checked bit for bit against the same fp32 additions in the same order
(torch elementwise adds) and one fp16 rounding.  The split product is checked against the exact
(float64) product of the fp16 operands: one fp16 rounding of an fp32 sum lies within 1 fp16 ulp
of the exact value plus the fp32 summation error, bounded by 64 * 2^-24 * sum|terms| for these
depths (the reference's single fp16 GEMM, solution/mlp.py:105-113, obeys the same bound)."""

import pytest
import torch

from testt_amd import _ext, mlp, workloads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


@pytest.mark.parametrize("parts,n,shift", [(1, 4096, 0), (2, 1001, 0), (4, 2048 * 1536, 0),
                                           (5, 333, 1), (8, 4097, 0), (9, 100, 0),
                                           (16, 77, 2)])
def test_sum_partials_bit_exact(parts, n, shift):
    print(f"sum_partials parts={parts} n={n} shift={shift}", flush=True)
    g = torch.Generator().manual_seed(parts * 1000 + n)
    stride = n + 3 * (parts > 1)
    flat = (torch.randn(parts * stride, generator=g) * 10.0 ** torch.randint(
        -3, 3, (parts * stride,), generator=g)).to(DEV)
    buf = torch.full((n + shift + 4,), float("nan"), dtype=torch.float16, device=DEV)
    out = buf[shift:shift + n]
    _ext.call("soupk_sum_partials", flat.data_ptr(), parts, stride, n, out.data_ptr(),
              _ext.stream_of(out))
    acc = flat[:n].clone()
    for p in range(1, parts):
        acc = acc + flat[p * stride:p * stride + n]
    assert torch.equal(out.view(torch.int16), acc.to(torch.float16).view(torch.int16))
    assert bool(torch.isnan(buf[:shift]).all()) and bool(torch.isnan(buf[shift + n:]).all())


def within_bound(got, a, b):
    ad, bd = a.double(), b.double()
    exact = ad @ bd
    terms = ad.abs() @ bd.abs()
    h = exact.to(torch.float16)
    inf = torch.tensor(float("inf"), dtype=torch.float16, device=DEV)
    ulp = (torch.nextafter(h.abs(), inf) - h.abs()).double()
    err = (got.double() - exact).abs()
    bad = err > ulp + 64 * 2.0 ** -24 * terms
    assert not bool(bad.any()), f"{int(bad.sum())} beyond the bound, max err {float(err.max())}"


@pytest.mark.parametrize("M,K,N,parts", [(2048, 17920, 1536, 4), (300, 1024, 256, 4),
                                         (7, 512, 64, 2), (64, 2048, 1536, 8)])
def test_matmul_split_k(M, K, N, parts):
    print(f"matmul_split_k M={M} K={K} N={N} parts={parts}", flush=True)
    g = torch.Generator().manual_seed(M + K)
    a = (0.05 * torch.randn(M, K, generator=g)).to(torch.float16).to(DEV)
    b = (0.05 * torch.randn(K, N, generator=g)).to(torch.float16).to(DEV)
    out = mlp.matmul_split_k(a, b, parts)
    assert out.dtype == torch.float16 and out.shape == (M, N)
    within_bound(out, a, b)
    # b as the transpose of a row-major [N, K] (the down projection's forward, act @ W^T)
    w = b.t().contiguous()
    out_t = mlp.matmul_split_k(a, w.t(), parts)
    within_bound(out_t, a, b)
    assert torch.equal(out_t, mlp.matmul_split_k(a, w.t(), parts))   # deterministic
    within_bound(torch.matmul(a, b), a, b)          # the single GEMM obeys the same bound
    with pytest.raises(ValueError):
        mlp.matmul_split_k(a, b, 3 if K % 3 else 5)


def test_fused_mlp_split_k_matches_single_gemm(monkeypatch):
    """FusedNF4MLP's input gradient through the split product or one GEMM: the same forward
    bits, input gradients equal to fp16 rounding (relative L2 < 2e-3)."""
    gate = workloads.nf4_weight(512, 256, seed=21, device=DEV)
    up = workloads.nf4_weight(512, 256, seed=22, device=DEV)
    down = workloads.nf4_weight(256, 512, seed=23, device=DEV)
    g = torch.Generator().manual_seed(6)
    x0 = torch.randn(129, 256, generator=g).to(torch.float16).to(DEV)
    grad = torch.randn(129, 256, generator=g).to(torch.float16).to(DEV)
    results = []
    for parts in (4, 1):
        monkeypatch.setattr(mlp, "SPLIT_K_GATE_UP", parts)
        x = x0.clone().requires_grad_(True)
        out = mlp.fused_mlp(x, gate, up, down)
        out.backward(grad)
        results.append((out.detach(), x.grad.clone()))
    assert torch.equal(results[0][0], results[1][0])
    a, b = results[0][1].double(), results[1][1].double()
    assert float((a - b).norm() / b.norm()) < 2e-3
