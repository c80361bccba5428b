"""Pins oracle/rmsnorm.py (CPU only) against transformers' Qwen2RMSNorm (the eager module the
reference replaces), float64 closed forms of the forward and backward, and invariants."""

import os

import numpy as np
import torch

from oracle.rmsnorm import rmsnorm_fwd, rmsnorm_fwd_bwd
from testt_amd import workloads

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "rmsnorm_qwen2.npz")


def test_matches_golden_qwen2rmsnorm_fixture():
    fx = np.load(GOLDEN)
    s, y16, ypad, rstd = rmsnorm_fwd(torch.from_numpy(fx["x"]), torch.from_numpy(fx["delta"]),
                                     torch.from_numpy(fx["w"]), float(fx["eps"]),
                                     torch.from_numpy(fx["pad_idx"]), int(fx["padded"]))
    assert torch.equal(y16, torch.from_numpy(fx["y16"]))
    assert torch.equal(ypad[fx["pad_idx"]], torch.from_numpy(fx["y32"]))
    torch.testing.assert_close(rstd.double(), torch.from_numpy(fx["rstd64"]), rtol=1e-6, atol=0)


def test_bitwise_equal_to_live_qwen2rmsnorm():
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm

    x, delta, w, _, _ = workloads.rmsnorm_inputs(64, 1536, seed=31)
    norm = Qwen2RMSNorm(1536, eps=1e-6)
    with torch.no_grad():
        norm.weight.copy_(w)
        ref = norm(x + delta.float())
    _, y16, _, _ = rmsnorm_fwd(x, delta, w, 1e-6)
    assert torch.equal(y16, ref.to(torch.float16))


def test_forward_float64_closed_form():
    x, delta, w, pad_idx, padded = workloads.rmsnorm_inputs(40, 1536, 64, seed=32)
    s, y16, ypad, rstd = rmsnorm_fwd(x, delta, w, 1e-6, pad_idx, padded)
    s64 = x.double() + delta.double()
    r64 = 1.0 / torch.sqrt((s64 * s64).mean(-1) + 1e-6)
    torch.testing.assert_close(rstd.double(), r64, rtol=1e-6, atol=0)
    torch.testing.assert_close(ypad[pad_idx].double(), w.double() * s64 * r64[:, None],
                               rtol=1e-5, atol=1e-6)
    unused = torch.ones(padded, dtype=torch.bool)
    unused[pad_idx] = False
    assert torch.all(ypad[unused] == 0)


def test_backward_float64_closed_form():
    """dx = (g - n * mean(g * n)) * rstd + ds, g = (dy + dypad[pad]) * w, n = s * rstd."""
    x, delta, w, pad_idx, padded = workloads.rmsnorm_inputs(32, 1536, 48, seed=33)
    dy, dypad, ds = workloads.rmsnorm_grads(32, 1536, 48, seed=34)
    dx, ddelta = rmsnorm_fwd_bwd(x, delta, w, 1e-6, pad_idx, padded, dy, dypad, ds)
    s = x.double() + delta.double()
    rstd = 1.0 / torch.sqrt((s * s).mean(-1, keepdim=True) + 1e-6)
    n = s * rstd
    g = (dy.double() + dypad.double()[pad_idx]) * w.double()
    ref = (g - n * (g * n).mean(-1, keepdim=True)) * rstd + ds.double()
    torch.testing.assert_close(dx.double(), ref, rtol=1e-5, atol=1e-5 * float(ref.abs().max()))
    assert torch.equal(ddelta, dx.to(torch.float16))
    # a plausible mistake -- dropping the projection term -- is far outside that tolerance
    wrong = g * rstd + ds.double()
    assert float((wrong - ref).abs().max()) > 100 * 1e-5 * float(ref.abs().max())


def test_invariants():
    h = 256
    w = torch.ones(h)
    for c in (3.0, -0.5):                          # constant row: y = c / sqrt(c^2 + eps)
        x = torch.full((1, h), c)
        _, y16, _, _ = rmsnorm_fwd(x, None, w, 1e-6)
        expect = np.float32(c) / np.sqrt(np.float32(c) ** 2 + np.float32(1e-6))
        assert torch.all(y16 == torch.tensor(expect).to(torch.float16))
    x, delta, wv, _, _ = workloads.rmsnorm_inputs(8, h, seed=35)
    zero = torch.zeros_like(delta)
    a = rmsnorm_fwd(x, zero, wv, 1e-6)[1]
    b = rmsnorm_fwd(x, None, wv, 1e-6)[1]
    assert torch.equal(a, b)                       # zero delta == the no-add variant
    _, y16, _, _ = rmsnorm_fwd(x, None, w, 1e-6)   # w = 1: mean(y^2) = 1/(1 + eps/mean(s^2))
    ms = (x.double() ** 2).mean(-1)
    torch.testing.assert_close((y16.double() ** 2).mean(-1), 1 / (1 + 1e-6 / ms), rtol=2e-3,
                               atol=0)
