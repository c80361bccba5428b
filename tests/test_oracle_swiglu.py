"""Pins oracle/swiglu.py (CPU only) against float64 closed forms and special values."""

import os

import numpy as np
import torch

from oracle.swiglu import swiglu_bwd, swiglu_fwd
from tests._util import assert_f16_ulp
from testt_amd import workloads

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "swiglu_f64.npz")


def test_matches_golden_float64_fixture():
    fx = np.load(GOLDEN)
    gu = torch.from_numpy(fx["gu"])
    assert_f16_ulp(swiglu_fwd(gu), torch.from_numpy(fx["act"]), 1, "act")
    out = swiglu_bwd(torch.from_numpy(fx["dact"]), gu)
    assert_f16_ulp(out, torch.from_numpy(fx["dgu"]), 1, "d gate | d up")


def test_special_values():
    g = torch.tensor([0.0, 30.0, -30.0, 1.0])
    u = torch.tensor([2.0, 1.0, 1.0, 3.0])
    gu = torch.cat([g, u])[None].to(torch.float16)
    act = swiglu_fwd(gu).float()[0]
    assert act[0] == 0 and act[1] == 30.0 and abs(float(act[2])) < 1e-10
    out = swiglu_bwd(torch.ones(1, 4, dtype=torch.float16), gu).float()[0]
    assert out[0] == 1.0                 # d gate at g = 0: dact * u / 2
    assert out[4] == 0.0                 # d up at g = 0: silu(0) = 0
    assert out[1] == 1.0                 # d gate for large g: dact * u
    assert abs(float(out[2])) < 1e-9     # d gate for very negative g: 0


def test_random_float64_closed_form():
    gu = workloads.swiglu_inputs(16, 512, seed=51, scale=3.0)
    dact = workloads.swiglu_grad(16, 512, seed=52)
    g, u = gu[:, :512].double(), gu[:, 512:].double()
    sig = 1 / (1 + torch.exp(-g))
    assert_f16_ulp(swiglu_fwd(gu), (g * sig * u).to(torch.float16), 1, "act")
    d = dact.double()
    ref = torch.cat([d * u * sig * (1 + g * (1 - sig)), d * g * sig], 1)
    out = swiglu_bwd(dact, gu)
    # d up: 1 ulp; d gate: 1 ulp or the cancellation bound of 1 + g(1 - sig) (see the GPU test)
    assert_f16_ulp(out[:, 512:], ref[:, 512:].to(torch.float16), 1, "d up")
    err = (out[:, :512].double() - ref[:, :512]).abs()
    mag = (d * u * sig).abs() * (1 + g.abs() * (1 - sig))
    assert bool((err <= mag * 2.0**-10 + 6e-8).all())
