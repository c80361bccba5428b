"""GPU parity: add+RMSNorm forward/backward vs the oracle (eager Qwen2RMSNorm + autograd).

Tolerances (north star): fp16 outputs within 1 ulp; fp32 reductions (rstd, and everything
derived from them) within 1e-5 relative.  dx carries the cancellation of g - n*mean(g*n), so its
absolute tolerance is 1e-5 of the largest |dx| of the tensor; ddelta must equal fp16(dx) of the
kernel's own dx exactly, and y16 must equal fp16(ypad row) exactly.
"""

import os

import numpy as np
import pytest
import torch

from oracle.rmsnorm import rmsnorm_fwd, rmsnorm_fwd_bwd
from tests._util import assert_f16_ulp, assert_rel
from testt_amd import rmsnorm, workloads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "rmsnorm_qwen2.npz")

CASES = [  # rows, hidden, padded, with_delta, with_pad
    (2048, 1536, 2048, True, True),     # the step's shape: every padded row holds a token
    (888, 1536, 2048, True, True),      # ragged batch: pad rows zeroed by the same launch
    (1500, 1536, 2048, True, True),     # 4 rows per workgroup (2048 and up: 8; under 1024: 2)
    (2051, 1536, 2051, True, True),     # 8 rows per workgroup with a partial last workgroup
    (300, 1536, 512, True, False),
    (300, 1536, 512, False, True),
    (7, 96, 10, True, True),
    (5, 98, 9, True, True),             # hidden % 4 != 0: generic kernel
    (3, 8192, 4, True, True),           # hidden > 4096: generic kernel
    (0, 1536, 16, True, True),          # no tokens: ypad all zero
]


@pytest.mark.parametrize("rows,hidden,padded,with_delta,with_pad", CASES)
def test_add_rmsnorm_fwd_bwd(rows, hidden, padded, with_delta, with_pad):
    print(f"rmsnorm rows={rows} hidden={hidden} padded={padded} delta={with_delta} "
          f"pad={with_pad}", flush=True)
    x, delta, w, pad_idx, padded = workloads.rmsnorm_inputs(rows, hidden, padded, seed=rows + 1)
    dy, dypad, ds = workloads.rmsnorm_grads(rows, hidden, padded, seed=rows + 2)
    if not with_delta:
        delta, ds = None, None
    if not with_pad:
        pad_idx, dypad = None, None

    xg = x.to(DEV).requires_grad_(True)
    dg = delta.to(DEV).requires_grad_(True) if delta is not None else None
    pg = pad_idx.to(DEV) if pad_idx is not None else None
    s, y, ypad = rmsnorm.add_rmsnorm(xg, dg, w.to(DEV), 1e-6, pg, padded if with_pad else 0)
    _, _, _, rstd = rmsnorm._launch_fwd(x.to(DEV), delta.to(DEV) if delta is not None else None,
                                        w.to(DEV), 1e-6, pg, padded if with_pad else 0)
    rs, ry, rypad, rrstd = rmsnorm_fwd(x, delta, w, 1e-6, pad_idx, padded if with_pad else 0)

    if with_delta:
        assert torch.equal(s.detach().cpu(), rs)             # one fp32 add: exact
    assert_f16_ulp(y.cpu(), ry, 1, "y16")
    assert_rel(rstd.cpu(), rrstd, 1e-5, what="rstd")
    if with_pad:
        assert ypad.shape == (padded, hidden)
        assert_rel(ypad.detach().cpu(), rypad, 1e-5, atol=1e-6, what="ypad")
        got = ypad.detach().cpu()
        assert torch.equal(got[pad_idx].to(torch.float16), y.cpu())
        unused = torch.ones(padded, dtype=torch.bool)
        unused[pad_idx] = False
        assert torch.all(got[unused] == 0)

    if rows == 0:
        return
    outs, grads = [y], [dy.to(DEV)]
    if with_pad:
        outs.append(ypad)
        grads.append(dypad.to(DEV))
    if with_delta:
        outs.append(s)
        grads.append(ds.to(DEV))
    torch.autograd.backward(outs, grads)
    rdx, rdd = rmsnorm_fwd_bwd(x, delta, w, 1e-6, pad_idx, padded, dy, dypad, ds)
    gdx = xg.grad.cpu()
    assert_rel(gdx, rdx, 1e-5, atol=1e-5 * float(rdx.abs().max()), what="dx")
    if with_delta:
        assert torch.equal(dg.grad.cpu(), gdx.to(torch.float16))


def test_golden_qwen2rmsnorm_fixture():
    fx = np.load(GOLDEN)
    x = torch.from_numpy(fx["x"]).to(DEV)
    delta = torch.from_numpy(fx["delta"]).to(DEV)
    w = torch.from_numpy(fx["w"]).to(DEV)
    pad_idx = torch.from_numpy(fx["pad_idx"]).to(DEV)
    s, y, ypad, rstd = rmsnorm._launch_fwd(x, delta, w, float(fx["eps"]), pad_idx,
                                           int(fx["padded"]))
    assert_f16_ulp(y.cpu(), torch.from_numpy(fx["y16"]), 1, "y16 vs Qwen2RMSNorm")
    assert_rel(ypad.cpu()[fx["pad_idx"]], torch.from_numpy(fx["y32"]), 1e-5, what="ypad")
    assert_rel(rstd.cpu(), torch.from_numpy(fx["rstd64"]), 1e-5, what="rstd vs float64")


def test_weight_dtype_and_errors():
    x, delta, w, pad_idx, padded = workloads.rmsnorm_inputs(16, 256, 16, seed=9)
    s, y, _, _ = rmsnorm._launch_fwd(x.to(DEV), delta.to(DEV), w.to(DEV).half(), 1e-6, None, 0)
    _, ry, _, _ = rmsnorm_fwd(x, delta, w.half().float(), 1e-6)
    assert_f16_ulp(y.cpu(), ry, 1, "y16 with fp16 weight")
    with pytest.raises(TypeError):
        rmsnorm._launch_fwd(x.to(DEV).half(), None, w.to(DEV), 1e-6, None, 0)
    with pytest.raises(ValueError):
        rmsnorm._launch_fwd(x, None, w, 1e-6, None, 0)           # CPU tensors: no CPU path
