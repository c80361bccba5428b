"""Comparison helpers for the parity tests (tolerances are stated where they are used)."""

import numpy as np
import torch


def _ordered(h16):
    """fp16 bit patterns mapped to integers that increase with the value (+0 and -0 -> 0)."""
    b = np.asarray(h16, dtype=np.float16).view(np.uint16).astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def ulp_diff_f16(a, b):
    """Elementwise distance in fp16 ulps between two fp16 arrays/tensors."""
    if torch.is_tensor(a):
        a = a.detach().cpu().numpy()
    if torch.is_tensor(b):
        b = b.detach().cpu().numpy()
    return np.abs(_ordered(a) - _ordered(b))


def assert_f16_ulp(actual, expected, max_ulp=1, what="fp16"):
    d = ulp_diff_f16(actual, expected)
    worst = int(d.max()) if d.size else 0
    assert worst <= max_ulp, (f"{what}: {int((d > max_ulp).sum())} of {d.size} values differ by "
                              f"more than {max_ulp} ulp (worst {worst})")
    return d


def assert_rel(actual, expected, rtol, atol=0.0, what="value"):
    a = torch.as_tensor(actual).detach().cpu().double()
    e = torch.as_tensor(expected).detach().cpu().double()
    err = (a - e).abs()
    bound = atol + rtol * e.abs()
    bad = ~(err <= bound) & ~(torch.isnan(a) & torch.isnan(e))   # NaN where e is not: bad
    assert not bool(bad.any()), (f"{what}: {int(bad.sum())} of {bad.numel()} exceed "
                                 f"rtol={rtol} atol={atol}; worst rel "
                                 f"{float((err / e.abs().clamp_min(1e-30)).max()):.3e}")
