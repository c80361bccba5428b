"""GPU: no kernel of the set stores outside its output tensors.

The vector kernels write through buffer descriptors whose hardware range check drops the stores
of lanes past a row's or a tile's end (no store predicate; testt_amd/csrc/soupk_common.hpp,
StreamOut).  Each output here lies in the middle of a buffer filled with a byte pattern, at
sizes whose last tile or row is partial; after the launch the bytes on both sides must still
hold the pattern, and the output must equal the same launch into a plain tensor.  The calls go
through the C ABI (include/soupk.h)."""

import math

import pytest
import torch

from testt_amd import _ext, nf4, workloads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
GUARD = 4096          # bytes on each side (keeps 16-byte alignment)
FILL = 0xA5


class Guarded:
    """A tensor of `shape` and `dtype` at byte GUARD of a pattern-filled buffer."""

    def __init__(self, shape, dtype, init=None):
        self.nbytes = math.prod(shape) * torch.empty((), dtype=dtype).element_size()
        self.buf = torch.full((2 * GUARD + self.nbytes,), FILL, dtype=torch.uint8, device=DEV)
        self.t = self.buf[GUARD:GUARD + self.nbytes].view(dtype).view(shape)
        if init is not None:
            self.t.copy_(init)

    def check(self, name):
        torch.cuda.synchronize()
        lo, hi = self.buf[:GUARD], self.buf[GUARD + self.nbytes:]
        bad = int((lo != FILL).sum()) + int((hi != FILL).sum())
        assert bad == 0, f"{name}: {bad} guard bytes overwritten"


def p(t):
    return None if t is None else t.data_ptr()


def stream():
    return torch.cuda.current_stream().cuda_stream


def run(name, *args):
    status = getattr(_ext.lib(), name)(*args, stream())
    assert status == 0, f"{name} returned {status}"


def test_nf4_unpack_guards():
    print("guards: nf4 unpack [37, 64] (partial tile)", flush=True)
    w = workloads.nf4_weight(37, 64, seed=31, device=DEV)
    out = Guarded((37, 64), torch.float16)
    nf4.unpack_into(w, out.t)
    out.check("nf4 out")
    ref = torch.empty((37, 64), dtype=torch.float16, device=DEV)
    nf4.unpack_into(w, ref)
    assert torch.equal(out.t, ref)


def test_nf4_unpack_multi_guards():
    """Two weights unpacked by one launch into adjacent views of one guarded buffer."""
    print("guards: nf4 unpack_multi [37, 64] + [24, 64]", flush=True)
    ws = [workloads.nf4_weight(37, 64, seed=32, device=DEV),
          workloads.nf4_weight(24, 64, seed=33, device=DEV)]
    out = Guarded((61, 64), torch.float16)
    nf4.unpack_many(ws, [out.t[:37], out.t[37:]])
    out.check("nf4 multi out")
    for w, view in zip(ws, (out.t[:37], out.t[37:])):
        ref = torch.empty(tuple(view.shape), dtype=torch.float16, device=DEV)
        nf4.unpack_into(w, ref)
        assert torch.equal(view, ref)


@pytest.mark.parametrize("rows,hidden", [(3, 1000), (5, 1536)])
def test_rmsnorm_guards(rows, hidden):
    print(f"guards: rmsnorm rows={rows} H={hidden}", flush=True)
    padded = rows + 2
    x, delta, w, pad_idx, _ = workloads.rmsnorm_inputs(rows, hidden, padded, seed=34, device=DEV)
    inv = torch.full((padded,), -1, dtype=torch.int32, device=DEV)
    inv[pad_idx] = torch.arange(rows, dtype=torch.int32, device=DEV)
    s = Guarded((rows, hidden), torch.float32)
    y = Guarded((rows, hidden), torch.float16)
    ypad = Guarded((padded, hidden), torch.float32)
    rstd = Guarded((rows,), torch.float32)
    run("soupk_rmsnorm_fwd", p(x), p(delta), p(w), p(s.t), p(y.t), p(ypad.t), p(pad_idx),
        p(inv), p(rstd.t), rows, padded, hidden, 1e-6)
    for g, name in ((s, "s"), (y, "y"), (ypad, "ypad"), (rstd, "rstd")):
        g.check(name)
    refs = [torch.empty_like(g.t) for g in (s, y, ypad, rstd)]
    run("soupk_rmsnorm_fwd", p(x), p(delta), p(w), p(refs[0]), p(refs[1]), p(refs[2]),
        p(pad_idx), p(inv), p(refs[3]), rows, padded, hidden, 1e-6)
    for g, r in zip((s, y, ypad, rstd), refs):
        assert torch.equal(g.t, r)

    dy, dypad, ds = workloads.rmsnorm_grads(rows, hidden, padded, seed=35, device=DEV)
    dx = Guarded((rows, hidden), torch.float32)
    dd = Guarded((rows, hidden), torch.float16)
    run("soupk_rmsnorm_bwd", p(s.t), p(rstd.t), p(w), p(dy), p(dypad), p(pad_idx), p(ds), p(dx.t),
        p(dd.t), rows, padded, hidden)
    dx.check("dx")
    dd.check("ddelta")
    rdx, rdd = torch.empty_like(dx.t), torch.empty_like(dd.t)
    run("soupk_rmsnorm_bwd", p(s.t), p(rstd.t), p(w), p(dy), p(dypad), p(pad_idx), p(ds), p(rdx),
        p(rdd), rows, padded, hidden)
    assert torch.equal(dx.t, rdx) and torch.equal(dd.t, rdd)


def test_rope_pack_guards():
    lengths, seq, nh, nkv, d = (5, 3), 8, 12, 2, 128
    print(f"guards: rope pack lengths={lengths} T={seq}", flush=True)
    b = len(lengths)
    qkv, lq, lv, pos = workloads.rope_inputs(lengths, seq, nh, nkv, d, torch.float32, seed=36,
                                             device=DEV)
    cos, sin = workloads.rope_tables(seq, d, device=DEV)
    rows = pos.numel()
    inv = torch.full((b * seq,), -1, dtype=torch.int32, device=DEV)
    inv[pos] = torch.arange(rows, dtype=torch.int32, device=DEV)
    outs = [Guarded((b, h, seq, d), torch.float16) for h in (nh, nkv, nkv)]
    run("soupk_rope_pack_fwd", p(qkv), p(lq), p(lv), _ext.DTYPE_F32, p(cos), p(sin), p(pos),
        p(inv), *[p(o.t) for o in outs], rows, b, seq, nh, nkv, d)
    for o, name in zip(outs, "qkv"):
        o.check(name)
    refs = [torch.empty_like(o.t) for o in outs]
    run("soupk_rope_pack_fwd", p(qkv), p(lq), p(lv), _ext.DTYPE_F32, p(cos), p(sin), p(pos),
        p(inv), *[p(r) for r in refs], rows, b, seq, nh, nkv, d)
    for o, r in zip(outs, refs):
        assert torch.equal(o.t, r)

    dq, dk, dv = workloads.rope_grads(b, seq, nh, nkv, d, seed=37, device=DEV)
    dqkv = Guarded((rows, (nh + 2 * nkv) * d), torch.float16)
    run("soupk_rope_pack_bwd", p(dq), p(dk), p(dv), p(cos), p(sin), p(pos), p(dqkv.t), rows, b,
        seq, nh, nkv, d)
    dqkv.check("dqkv")
    ref = torch.empty_like(dqkv.t)
    run("soupk_rope_pack_bwd", p(dq), p(dk), p(dv), p(cos), p(sin), p(pos), p(ref), rows, b, seq,
        nh, nkv, d)
    assert torch.equal(dqkv.t, ref)


@pytest.mark.parametrize("rows,inter", [(5, 1504), (3, 8)])
def test_swiglu_guards(rows, inter):
    print(f"guards: swiglu rows={rows} I={inter}", flush=True)
    gu = workloads.swiglu_inputs(rows, inter, seed=38, device=DEV)
    act = Guarded((rows, inter), torch.float16)
    run("soupk_swiglu_fwd", p(gu), p(act.t), rows, inter)
    act.check("act")
    ref = torch.empty_like(act.t)
    run("soupk_swiglu_fwd", p(gu), p(ref), rows, inter)
    assert torch.equal(act.t, ref)

    dact = workloads.swiglu_grad(rows, inter, seed=39, device=DEV)
    g = Guarded((rows, 2 * inter), torch.float16, init=gu)
    run("soupk_swiglu_bwd_inplace", p(dact), p(g.t), rows, inter)
    g.check("gu (in place)")
    ref = gu.clone()
    run("soupk_swiglu_bwd_inplace", p(dact), p(ref), rows, inter)
    assert torch.equal(g.t, ref)


@pytest.mark.parametrize("vocab", [1003, 151936])
def test_head_guards(vocab):
    rows = 3
    print(f"guards: head rows={rows} V={vocab}", flush=True)
    z, tgt = workloads.head_logits(rows, vocab, seed=40, device=DEV)
    tgt[1] = -100
    logits = Guarded((rows, vocab), torch.float16, init=z)
    stats = [Guarded((rows,), dt) for dt in (torch.float32, torch.float32, torch.int32,
                                             torch.float32)]
    run("soupk_head_stats_grad", p(logits.t), p(tgt), *[p(s.t) for s in stats], 0.25, rows,
        vocab)
    logits.check("logits (in place)")
    for s, name in zip(stats, ("entropy", "loss", "correct", "lse")):
        s.check(name)
    ref = z.clone()
    rstats = [torch.empty_like(s.t) for s in stats]
    run("soupk_head_stats_grad", p(ref), p(tgt), *[p(s) for s in rstats], 0.25, rows, vocab)
    assert torch.equal(logits.t, ref)
    for s, r in zip(stats, rstats):
        assert torch.equal(s.t, r)


def test_sum_partials_guards():
    n_parts, n = 4, 1000
    print(f"guards: split-K sum parts={n_parts} n={n}", flush=True)
    parts = torch.randn(n_parts, n, generator=workloads.gen(41)).to(DEV)
    out = Guarded((n,), torch.float16)
    run("soupk_sum_partials", p(parts), n_parts, n, n, p(out.t))
    out.check("out")
    ref = torch.empty_like(out.t)
    run("soupk_sum_partials", p(parts), n_parts, n, n, p(ref))
    assert torch.equal(out.t, ref)
