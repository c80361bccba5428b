"""GPU parity: the causal GQA attention kernels (testt_amd/csrc/attention.hip) against float32
attention with the same mask (torch on the CPU in float32: scores, causal + key-padding mask,
softmax, weighted sum).  The kernel rounds the probabilities to fp16 for the P.V product, as
torch's fp16 flash kernels do, and its output to fp16: outputs within 2e-3 absolute (values are
O(1)), log-sum-exp within 1e-4 relative."""

import math

import pytest
import torch

from testt_amd import attention

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")


def reference(q, k, v, valid, scale):
    """float32 attention; returns out [B, T, NH*D] and lse [B, NH, T] (+inf: no visible key)."""
    B, NH, T, D = q.shape
    rep = NH // k.shape[1]
    qf, kf, vf = q.float(), k.float().repeat_interleave(rep, 1), v.float().repeat_interleave(rep, 1)
    s = (qf @ kf.transpose(-1, -2)) * scale
    allowed = torch.ones(T, T, dtype=torch.bool).tril()[None, None]
    if valid is not None:
        allowed = allowed & valid.bool()[:, None, None, :]
    s = s.masked_fill(~allowed, float("-inf"))
    lse = torch.logsumexp(s, -1)
    p = torch.exp(s - lse[..., None]).nan_to_num(0.0)
    out = (p @ vf).transpose(1, 2).reshape(B, T, NH * D)
    return out, lse.masked_fill(torch.isinf(lse), float("inf"))


CASES = [  # B, T, NH, NKV, lengths (None: every key real)
    (4, 512, 12, 2, None),
    (3, 77, 12, 2, (77, 40, 5)),
    (2, 130, 4, 4, (130, 64)),
    (2, 64, 6, 3, (0, 64)),        # a row with no real key: output 0, lse = +inf
    (1, 1, 2, 1, None),
]


@pytest.mark.parametrize("B,T,NH,NKV,lengths", CASES)
def test_attention_forward(B, T, NH, NKV, lengths):
    print(f"attention fwd B={B} T={T} NH={NH} NKV={NKV} lengths={lengths}", flush=True)
    g = torch.Generator().manual_seed(T + NH)
    q = torch.randn(B, NH, T, 128, generator=g).to(torch.float16)
    k = torch.randn(B, NKV, T, 128, generator=g).to(torch.float16)
    v = torch.randn(B, NKV, T, 128, generator=g).to(torch.float16)
    valid = None
    if lengths is not None:
        valid = torch.zeros(B, T, dtype=torch.uint8)
        for b, n in enumerate(lengths):
            valid[b, :n] = 1
    scale = 1.0 / math.sqrt(128)
    out, lse = attention.attention_fwd(q.to(DEV), k.to(DEV), v.to(DEV),
                                       None if valid is None else valid.to(DEV), scale)
    r_out, r_lse = reference(q, k, v, valid, scale)
    got = out.cpu().float().view(B, T, -1)
    err = (got - r_out).abs().max().item()
    print(f"  max |out - ref| = {err:.2e}", flush=True)
    assert err < 2e-3
    l = lse.cpu()
    fin = torch.isfinite(r_lse)
    assert torch.equal(torch.isinf(l), ~fin)
    assert ((l[fin] - r_lse[fin]).abs() <= 1e-4 * r_lse[fin].abs() + 1e-5).all()


BWD_CASES = [
    (4, 512, 12, 2, None),
    (3, 77, 12, 2, (77, 40, 5)),
    (2, 130, 4, 4, (130, 64)),
    (2, 64, 6, 3, (0, 64)),
    (1, 1, 2, 1, None),
]


@pytest.mark.parametrize("B,T,NH,NKV,lengths", BWD_CASES)
def test_attention_backward(B, T, NH, NKV, lengths):
    """Gradients of sum(out * dO) against float32 autograd through the same masked attention.
    The kernels round P and dS to fp16 for their MFMA products (as torch's fp16 flash backward
    does): dq, dk, dv within 2e-3 of the reference relative to its largest entry."""
    print(f"attention bwd B={B} T={T} NH={NH} NKV={NKV} lengths={lengths}", flush=True)
    g = torch.Generator().manual_seed(3 * T + NH)
    q = torch.randn(B, NH, T, 128, generator=g).to(torch.float16)
    k = torch.randn(B, NKV, T, 128, generator=g).to(torch.float16)
    v = torch.randn(B, NKV, T, 128, generator=g).to(torch.float16)
    dout = torch.randn(B * T, NH * 128, generator=g).to(torch.float16)
    valid = None
    if lengths is not None:
        valid = torch.zeros(B, T, dtype=torch.uint8)
        for b, n in enumerate(lengths):
            valid[b, :n] = 1
    scale = 1.0 / math.sqrt(128)

    qd, kd, vd = (t.to(DEV).requires_grad_() for t in (q, k, v))
    out = attention.causal_attention(qd, kd, vd, None if valid is None else valid.to(DEV), scale)
    out.backward(dout.to(DEV))

    qf, kf, vf = (t.float().requires_grad_() for t in (q, k, v))
    r_out, _ = reference(qf, kf, vf, valid, scale)
    r_out.reshape(B * T, -1).backward(dout.float())
    for name, got, ref in (("dq", qd.grad, qf.grad), ("dk", kd.grad, kf.grad),
                           ("dv", vd.grad, vf.grad)):
        got = got.cpu().float()
        assert torch.isfinite(got).all(), name
        top = ref.abs().max().item()
        err = (got - ref).abs().max().item()
        print(f"  {name}: max |err| = {err:.2e}  (max |ref| = {top:.2e})", flush=True)
        assert err <= 2e-3 * max(top, 1.0), name
