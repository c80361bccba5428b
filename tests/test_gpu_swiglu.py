"""GPU parity: gated-SiLU forward and in-place backward vs the oracle (F.silu(g) * u and its
autograd on the CPU).

Tolerance: fp16 outputs within 1 ulp.  One documented widening: d gate contains the factor
1 + g(1 - sig), which crosses zero at g ~ -1.2785; there both fp32 computations (kernel and
oracle) carry ~1e-7 absolute error in that factor, so for d gate the test also accepts an error
up to 2^-21 times the magnitude of the uncancelled terms |dact * u * sig| * (1 + |g| (1 - sig)).
"""

import os

import numpy as np
import pytest
import torch

from oracle.swiglu import swiglu_bwd, swiglu_fwd
from tests._util import assert_f16_ulp, ulp_diff_f16
from testt_amd import mlp, workloads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "swiglu_f64.npz")


def check_dgate(got, ref, gu, dact):
    inter = gu.shape[1] // 2
    g = gu[:, :inter].double()
    u = gu[:, inter:].double()
    sig = torch.sigmoid(g)
    mag = (dact.double() * u * sig).abs() * (1 + g.abs() * (1 - sig))
    d = torch.from_numpy(ulp_diff_f16(got, ref).astype(np.int64))
    err = (got.double() - ref.double()).abs()
    ok = (d <= 1) | (err <= mag * 2.0**-21)
    assert bool(ok.all()), f"d gate: {int((~ok).sum())} values beyond tolerance"


@pytest.mark.parametrize("rows,inter,scale", [(2048, 8960, 1.0), (333, 8960, 3.0),
                                              (5, 1500, 3.0), (3, 7, 3.0), (1, 8, 20.0)])
def test_gated_silu_fwd_bwd(rows, inter, scale):
    print(f"swiglu rows={rows} inter={inter} scale={scale}", flush=True)
    gu = workloads.swiglu_inputs(rows, inter, seed=rows + inter, scale=scale)
    dact = workloads.swiglu_grad(rows, inter, seed=rows + inter + 1)
    act = mlp.gated_silu(gu.to(DEV))
    assert_f16_ulp(act.cpu(), swiglu_fwd(gu), 1, "act")
    buf = gu.to(DEV)
    out = mlp.gated_silu_backward_(dact.to(DEV), buf)
    assert out is buf                                # in place
    ref = swiglu_bwd(dact, gu)
    got = out.cpu()
    assert_f16_ulp(got[:, inter:], ref[:, inter:], 1, "d up")
    check_dgate(got[:, :inter], ref[:, :inter], gu, dact)


def test_golden_f64_fixture():
    fx = np.load(GOLDEN)
    gu = torch.from_numpy(fx["gu"])
    act = mlp.gated_silu(gu.to(DEV))
    assert_f16_ulp(act.cpu(), torch.from_numpy(fx["act"]), 1, "act vs float64")
    out = mlp.gated_silu_backward_(torch.from_numpy(fx["dact"]).to(DEV), gu.to(DEV)).cpu()
    inter = gu.shape[1] // 2
    ref = torch.from_numpy(fx["dgu"])
    assert_f16_ulp(out[:, inter:], ref[:, inter:], 1, "d up vs float64")
    check_dgate(out[:, :inter], ref[:, :inter], gu, torch.from_numpy(fx["dact"]))


def test_special_values():
    inter = 8
    g = torch.tensor([0.0, -0.0, 30.0, -30.0, 65504.0, -65504.0, 1.0, -1.0])
    u = torch.tensor([1.0, 2.0, 1.0, 1.0, 1.0, 1.0, 0.0, 3.0])
    gu = torch.cat([g, u])[None].to(torch.float16)
    act = mlp.gated_silu(gu.to(DEV)).cpu().float()[0]
    assert act[0] == 0 and act[1] == 0
    assert act[2] == 30.0 and act[4] == 65504.0 and act[5] == 0 and act[6] == 0
    dact = torch.ones(1, inter, dtype=torch.float16)
    out = mlp.gated_silu_backward_(dact.to(DEV), gu.to(DEV)).cpu().float()[0]
    assert out[0] == 0.5 and out[1] == 1.0       # d gate at g = 0 is dact * u / 2
    assert out[inter] == 0 and out[inter + 1] == 0  # d up at g = 0 is silu(0) = 0
