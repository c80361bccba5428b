"""Gated SiLU forward and backward, eager PyTorch on the CPU.
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

Forward: act = fp16(F.silu(g) * u) with g, u the fp32 halves of the fused [gate | up] fp16
row (solution/mlp.py:31-40; reference test solution/test_kernels.py:94-97).  Backward: autograd
of the same product for the incoming fp16 dact, then fp16 (solution/mlp.py:43-58; reference
test solution/test_kernels.py:98-102): d gate = dact * u * sig * (1 + g * (1 - sig)),
d up = dact * silu(g).

Pinned by: a float64 recomputation from the closed forms, g = 0 (act = 0, d up = 0,
d gate = dact * u / 2), and the large-|g| limits (tests/test_oracle_swiglu.py).
"""

import torch


def swiglu_fwd(gu):
    inter = gu.shape[1] // 2
    g, u = gu[:, :inter].float(), gu[:, inter:].float()
    return (torch.nn.functional.silu(g) * u).to(torch.float16)


def swiglu_bwd(dact, gu):
    """fp16 [rows, 2I]: [d gate | d up], what the in-place kernel leaves in gu."""
    inter = gu.shape[1] // 2
    g = gu[:, :inter].float().clone().requires_grad_(True)
    u = gu[:, inter:].float().clone().requires_grad_(True)
    out = torch.nn.functional.silu(g) * u
    out.backward(dact.float())
    return torch.cat([g.grad, u.grad], dim=1).to(torch.float16)
