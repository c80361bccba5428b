"""Pins oracle/head.py (CPU only) against torch's cross_entropy / log_softmax / argmax in
float64, closed forms on special rows, and the reference's grad-unit rule."""

import math
import os

import numpy as np
import torch

from oracle import head as ohead
from testt_amd import head, workloads

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "head_f64.npz")


def test_matches_golden_fixture():
    fx = np.load(GOLDEN)
    ent, loss, cor, lse, new = ohead.head_stats_grad(torch.from_numpy(fx["z"]),
                                                      torch.from_numpy(fx["targets"]),
                                                      float(fx["grad_scale"]))
    torch.testing.assert_close(ent, torch.from_numpy(fx["entropy"]), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(loss, torch.from_numpy(fx["loss"]), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(lse, torch.from_numpy(fx["lse"]), rtol=1e-12, atol=1e-12)
    assert torch.equal(cor, torch.from_numpy(fx["correct"]))
    d = (new.view(torch.int16).int() - torch.from_numpy(fx["new_logits"]).view(torch.int16).int())
    assert int(d.abs().max()) <= 1


def test_against_torch_float64():
    z, t = workloads.head_logits(16, 3001, seed=61)
    ent, loss, cor, lse, new = ohead.head_stats_grad(z, t, 0.5)
    zd = z.double()
    logp = torch.log_softmax(zd, -1)
    lab = t != -100
    ce = torch.nn.functional.cross_entropy(zd, t, ignore_index=-100, reduction="none")
    torch.testing.assert_close(loss, ce, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(ent, -(logp.exp() * logp).sum(-1), rtol=1e-12, atol=1e-12)
    assert torch.equal(cor, (zd.argmax(-1) == t) & lab)
    p = torch.softmax(zd, -1)
    grad = p.clone()
    grad[lab, t[lab]] -= 1
    assert torch.all(grad[lab].sum(-1).abs() < 1e-12)            # rows sum to zero
    torch.testing.assert_close(new[lab].double(), (grad[lab] * 0.5).to(torch.float16).double(),
                               rtol=0, atol=0)
    assert torch.equal(new[~lab], z[~lab])                          # ignored rows untouched


def test_special_rows():
    V = 1000
    z = torch.zeros(3, V, dtype=torch.float16)
    z[0] = -2.0                                          # uniform
    z[1, 7] = z[1, 900] = 5.0                            # tie: first index wins
    z[2, 42] = 20.0                                      # spike
    t = torch.tensor([0, 7, 42])
    ent, loss, cor, lse, _ = ohead.head_stats_grad(z, t, 1.0)
    assert abs(float(ent[0]) - math.log(V)) < 1e-12
    assert abs(float(lse[0]) - (-2.0 + math.log(V))) < 1e-12
    assert cor.tolist() == [True, True, True]
    assert float(loss[2]) < 1e-5


def test_grad_unit_rule():
    # 2^clamp(round(log2 d) + 6, 0, 16): the fp16 gradient sits near 64/d in magnitude
    for d, unit in ((1, 64.0), (3, 256.0), (1843, 65536.0), (1e-9, 1.0), (0.01, 1.0)):
        assert head._grad_unit(d) == unit == ohead.grad_unit(d)
