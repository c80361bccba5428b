"""GPU parity: LoRA-add + RoPE + QKV pack forward/backward vs the oracle (index_copy +
apply_rotary_pos_emb + autograd on the CPU).  Tolerance: fp16 outputs within 1 ulp (the fp32
arithmetic is the same sequence of separately rounded operations, so they are expected equal);
padded positions without a token must be exactly zero."""

import os

import numpy as np
import pytest
import torch

from oracle.rope import rope_pack_bwd, rope_pack_fwd
from tests._util import assert_f16_ulp
from testt_amd import rope, workloads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "rope_hf.npz")

CASES = [  # lengths, seq, nh, nkv, d, theta, lora dtype (None: no LoRA)
    ((512,) * 4, 512, 12, 2, 128, 1e6, torch.float32),      # M = 2048, every position real
    ((512, 152, 128, 96), 512, 12, 2, 128, 1e6, torch.float32),   # ragged, M = 888
    ((512, 152, 128, 96), 512, 12, 2, 128, 1e6, torch.float16),
    ((77, 75), 77, 12, 2, 128, 1e4, torch.float16),          # the reference's test shape
    ((40, 0, 13), 64, 12, 2, 128, 1e6, None),
    ((37, 20), 40, 1, 1, 128, 1e4, torch.float32),            # 24 items/token: ~21 tokens per
    ((53,), 64, 2, 1, 128, 1e6, torch.float16),               # forward workgroup, partial tail
    ((5, 3), 5, 3, 1, 8, 1e4, torch.float16),                 # head_dim 8: generic kernel
    ((6, 2), 7, 2, 1, 6, 1e4, torch.float32),                 # head_dim 6: generic kernel
]


@pytest.mark.parametrize("lengths,seq,nh,nkv,d,theta,ldt", CASES)
def test_rope_pack_fwd_bwd(lengths, seq, nh, nkv, d, theta, ldt):
    print(f"rope lengths={lengths} seq={seq} nh={nh} nkv={nkv} d={d} lora={ldt}", flush=True)
    batch = len(lengths)
    qkv, lq, lv, pos = workloads.rope_inputs(lengths, seq, nh, nkv, d,
                                             lora_dtype=ldt or torch.float32, seed=sum(lengths))
    if ldt is None:
        lq = lv = None
    cos, sin = workloads.rope_tables(seq, d, theta)
    qkv_g = qkv.to(DEV).requires_grad_(True)
    lq_g = lq.to(DEV).requires_grad_(True) if lq is not None else None
    lv_g = lv.to(DEV).requires_grad_(True) if lv is not None else None
    q, k, v = rope.rope_pack(qkv_g, lq_g, lv_g, cos.to(DEV), sin.to(DEV), pos.to(DEV), batch, seq,
                             nh, nkv, d)
    rq, rk, rv = rope_pack_fwd(qkv, lq, lv, cos, sin, pos, batch, seq, nh, nkv, d)
    for got, ref, name in ((q, rq, "q"), (k, rk, "k"), (v, rv, "v")):
        assert got.shape == ref.shape
        assert_f16_ulp(got.detach().cpu(), ref, 1, name)
    real = torch.zeros(batch * seq, dtype=torch.bool)
    real[pos] = True
    pads = ~real.view(batch, seq)
    for got in (q, k, v):
        assert torch.all(got.detach().cpu().permute(0, 2, 1, 3)[pads] == 0)

    dq, dk, dv = workloads.rope_grads(batch, seq, nh, nkv, d, seed=7 + sum(lengths))
    torch.autograd.backward([q, k, v], [dq.to(DEV), dk.to(DEV), dv.to(DEV)])
    ref = rope_pack_bwd(qkv, None, None, cos, sin, pos, batch, seq, nh, nkv, d, dq, dk, dv)
    assert_f16_ulp(qkv_g.grad.cpu(), ref, 1, "dqkv")
    if lq_g is not None:
        assert_f16_ulp(lq_g.grad.cpu().to(torch.float16), ref[:, :nh * d], 1, "dlora_q")
        assert_f16_ulp(lv_g.grad.cpu().to(torch.float16), ref[:, (nh + nkv) * d:], 1, "dlora_v")


def test_backward_with_missing_grads():
    lengths, seq, nh, nkv, d = (30, 20), 32, 12, 2, 128
    qkv, lq, lv, pos = workloads.rope_inputs(lengths, seq, nh, nkv, d, seed=77)
    cos, sin = workloads.rope_tables(seq, d)
    qkv_g = qkv.to(DEV).requires_grad_(True)
    q, k, v = rope.rope_pack(qkv_g, None, None, cos.to(DEV), sin.to(DEV), pos.to(DEV), 2, seq,
                             nh, nkv, d)
    dq, _, _ = workloads.rope_grads(2, seq, nh, nkv, d, seed=78)
    q.backward(dq.to(DEV))                         # no gradient reaches k or v
    ref = rope_pack_bwd(qkv, None, None, cos, sin, pos, 2, seq, nh, nkv, d, dq, None, None)
    assert_f16_ulp(qkv_g.grad.cpu(), ref, 1, "dqkv (q only)")
    assert torch.all(qkv_g.grad[:, nh * d:] == 0)


def test_golden_hf_fixture():
    fx = np.load(GOLDEN)
    batch, seq, nh, nkv, d = (int(x) for x in fx["dims"])
    t = {k: torch.from_numpy(fx[k]).to(DEV) for k in ("qkv", "lq", "lv", "pos", "cos", "sin")}
    q, k, v = rope.rope_pack(t["qkv"], t["lq"], t["lv"], t["cos"], t["sin"], t["pos"], batch,
                             seq, nh, nkv, d)
    for got, name in ((q, "q"), (k, "k"), (v, "v")):
        assert_f16_ulp(got.cpu(), torch.from_numpy(fx[name]), 1, f"{name} vs transformers")


def test_inverse_map_is_cached_and_rebuilt():
    pos = workloads.ragged_positions((5, 3), 8).to(DEV)
    from testt_amd._index import inverse_map

    inv = inverse_map(pos, 16)
    assert inverse_map(pos, 16) is inv
    expect = torch.full((16,), -1, dtype=torch.int32)
    expect[pos.cpu()] = torch.arange(pos.numel(), dtype=torch.int32)
    assert torch.equal(inv.cpu(), expect)
    pos[0] = 7                                      # in-place change: the map is rebuilt
    inv2 = inverse_map(pos, 16)
    assert inv2 is not inv and int(inv2[7]) == 0 and int(inv2[0]) == -1


def test_out_of_range_positions_are_skipped():
    """Positions outside [0, B*T) are skipped by the forward pass (nothing written for that
    token) and give zero gradient rows in the backward pass (the C ABI's bounds contract);
    with B*T = 0 the forward pass writes nothing and the backward pass writes zeros."""
    from testt_amd import _ext

    lengths, seq, nh, nkv, d = (20, 12), 32, 12, 2, 128
    qkv, lq, lv, pos = workloads.rope_inputs(lengths, seq, nh, nkv, d, seed=91)
    cos, sin = workloads.rope_tables(seq, d)
    m, w = pos.numel(), (nh + 2 * nkv) * d
    bad = pos.clone()
    bad[3], bad[17] = -1, 2 * seq + 5
    keep = torch.ones(m, dtype=torch.bool)
    keep[[3, 17]] = False
    g = {n: t.to(DEV) for n, t in (("qkv", qkv), ("lq", lq), ("lv", lv), ("cos", cos),
                                   ("sin", sin), ("bad", bad))}
    sentinel = 0x3C00  # fp16 1.0: slots of the skipped tokens keep it
    outs = [torch.full((2, h, seq, d), 1.0, dtype=torch.float16, device=DEV)
            for h in (nh, nkv, nkv)]
    st = torch.cuda.current_stream().cuda_stream
    _ext.call("soupk_rope_pack_fwd", g["qkv"].data_ptr(), g["lq"].data_ptr(), g["lv"].data_ptr(),
              _ext.DTYPE_F32, g["cos"].data_ptr(), g["sin"].data_ptr(), g["bad"].data_ptr(), None,
              outs[0].data_ptr(), outs[1].data_ptr(), outs[2].data_ptr(), m, 2, seq, nh, nkv, d,
              st)
    ref = rope_pack_fwd(qkv[keep], lq[keep], lv[keep], cos, sin, pos[keep], 2, seq, nh, nkv, d)
    for got, r, name in zip(outs, ref, "qkv"):
        got = got.cpu().permute(0, 2, 1, 3).reshape(2 * seq, -1, d)
        r = r.permute(0, 2, 1, 3).reshape(2 * seq, -1, d)
        assert_f16_ulp(got[pos[keep]], r[pos[keep]], 1, name)
        skipped = got[pos[[3, 17]]].contiguous().view(torch.int16)
        assert torch.all(skipped == sentinel), name

    dq, dk, dv = (t.to(DEV) for t in workloads.rope_grads(2, seq, nh, nkv, d, seed=92))
    dqkv = torch.full((m, w), 1.0, dtype=torch.float16, device=DEV)
    _ext.call("soupk_rope_pack_bwd", dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
              g["cos"].data_ptr(), g["sin"].data_ptr(), g["bad"].data_ptr(), dqkv.data_ptr(), m, 2,
              seq, nh, nkv, d, st)
    ref = rope_pack_bwd(qkv, None, None, cos, sin, pos, 2, seq, nh, nkv, d, dq.cpu(), dk.cpu(),
                        dv.cpu())
    got = dqkv.cpu()
    assert_f16_ulp(got[keep], ref[keep], 1, "dqkv (valid rows)")
    assert torch.all(got[~keep] == 0)

    # B*T = 0: empty outputs and tables (null data pointers are allowed for them)
    zpos = torch.tensor([0, 1], dtype=torch.int64, device=DEV)
    _ext.call("soupk_rope_pack_fwd", g["qkv"].data_ptr(), None, None, _ext.DTYPE_F32, None,
              None, zpos.data_ptr(), None, None, None, None, 2, 2, 0, nh, nkv, d, st)
    dz = torch.full((2, w), 1.0, dtype=torch.float16, device=DEV)
    _ext.call("soupk_rope_pack_bwd", None, None, None, None, None, zpos.data_ptr(),
              dz.data_ptr(), 2, 2, 0, nh, nkv, d, st)
    assert torch.all(dz.cpu() == 0)
