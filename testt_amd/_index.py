"""Inverse of a token -> padded-position scatter index, shared by the pad-layout writers.

`pos_idx` (solution/model.py:220, `attention_mask.nonzero()`) sends token row i to padded row
pos_idx[i].  The reference writes its padded outputs into `torch.zeros` buffers
(solution/rmsnorm.py:82, solution/rope.py:141-143): a full memset, then the scatter.  Here the
scatter kernels zero the rows no token maps to in the same launch, and they learn which rows
those are from inv[p] (= i if pos_idx[i] == p, else -1), built by one small kernel.  The model
uses one pos_idx for every layer, so the map is cached on the index tensor itself and rebuilt
only when the tensor changes (its version counter moves) or another slot count is asked for.
"""

import torch

from . import _ext

_ATTR = "_soupk_inverse"


def inverse_map(idx, n_slots):
    """int32 [n_slots] device tensor: inv[p] = i where idx[i] == p, else -1."""
    _ext.require(idx, "pos_idx", dtype=torch.int64, ndim=1)
    key = (int(n_slots), idx._version, idx.data_ptr(), idx.numel())
    cached = getattr(idx, _ATTR, None)
    if cached is not None and cached[0] == key:
        return cached[1]
    inv = torch.empty(int(n_slots), dtype=torch.int32, device=idx.device)
    _ext.call("soupk_index_inverse", _ext.ptr(idx), idx.numel(), _ext.ptr(inv), int(n_slots),
              _ext.stream_of(idx))
    try:
        setattr(idx, _ATTR, (key, inv))
    except (AttributeError, RuntimeError):  # e.g. a tensor subclass with __slots__
        pass
    return inv


def as_index(t):
    """int64 contiguous view of an index tensor (pos_idx / pad_idx may arrive as int32)."""
    if t.dtype != torch.int64:
        t = t.to(torch.int64)
    return t.contiguous()
