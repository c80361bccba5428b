"""GPU parity: soupk_nf4_unpack vs the oracle, bit-exact (fp16 bit patterns compared)."""

import os

import numpy as np
import pytest
import torch

from oracle.nf4 import dequant_nf4, dequant_state, quantize_nf4
from testt_amd import _ext, nf4, workloads

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda")
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "nf4_kat.npz")


def bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy()


@pytest.mark.parametrize("shape,seed", [((17920, 1536), 1), ((128, 192), 31), ((96, 640), 32),
                                        ((1536, 8960), 33)])
def test_unpack_synthetic_bit_exact(shape, seed):
    print(f"nf4 synthetic shape={shape} seed={seed}", flush=True)
    w = workloads.nf4_weight(*shape, seed=seed, device=DEV)
    assert nf4.supports_fast_unpack(w)
    out = torch.empty(shape, dtype=torch.float16, device=DEV)
    nf4.unpack_into(w, out)
    ref = dequant_state(w)
    assert np.array_equal(bits(out), ref.view(np.int16))


def _quantized(n_out, n_in, seed):
    g = np.random.default_rng(seed)
    w = (g.standard_normal((n_out, n_in)) * 0.05).astype(np.float16)
    code2 = workloads.dynamic_code_signed()
    packed, absmax_u8, absmax2, offset = quantize_nf4(w, workloads.NF4_LEVELS, code2.numpy())
    p = workloads.nf4_weight(n_out, n_in, seed=0, device=DEV)
    st = p.quant_state
    p.data = torch.from_numpy(packed).reshape(-1, 1).to(DEV)
    st.absmax = torch.from_numpy(absmax_u8).to(DEV)
    st.state2.absmax = torch.from_numpy(absmax2).to(DEV)
    st.offset = torch.tensor(float(offset), dtype=torch.float32, device=DEV)
    return p


def test_unpack_concat_quantized_weights():
    a, b = _quantized(128, 192, 41), _quantized(64, 192, 42)
    out = nf4.unpack_concat((a, b), DEV)
    ref = np.concatenate([dequant_state(a), dequant_state(b)])
    assert np.array_equal(bits(out), ref.view(np.int16))


def test_cached_plan_follows_replaced_state():
    """unpack_into caches each weight's checked kernel arguments; replacing a state tensor
    (new absmax codes, a new offset) must be seen by the next unpack."""
    w = workloads.nf4_weight(64, 256, seed=43, device=DEV)
    out = torch.empty(64, 256, dtype=torch.float16, device=DEV)
    nf4.unpack_into(w, out)
    assert np.array_equal(bits(out), dequant_state(w).view(np.int16))
    st = w.quant_state
    st.absmax = torch.flip(st.absmax, [0]).contiguous()
    st.offset = 0.25
    nf4.unpack_into(w, out)
    assert np.array_equal(bits(out), dequant_state(w).view(np.int16))


def test_golden_fixture_through_abi():
    fx = np.load(GOLDEN)
    t = {k: torch.from_numpy(np.ascontiguousarray(fx[k])).to(DEV)
         for k in ("packed", "absmax_u8", "code2", "absmax2", "offset", "nf4")}
    n_bytes = t["packed"].numel()
    out = torch.empty(2 * n_bytes, dtype=torch.float16, device=DEV)
    _ext.call("soupk_nf4_unpack", _ext.ptr(t["packed"]), _ext.ptr(t["absmax_u8"]),
              _ext.ptr(t["code2"]), _ext.ptr(t["absmax2"]), _ext.ptr(t["offset"]),
              _ext.ptr(t["nf4"]), _ext.ptr(out), n_bytes, int(fx["qblock"]), int(fx["qblock2"]),
              _ext.stream_of(out))
    assert np.array_equal(bits(out), fx["expected"].view(np.int16))


@pytest.mark.parametrize("n_bytes,out_shift", [(16 * 1000 + 5, 0), (4096, 1), (31, 0), (1, 0)])
def test_tail_and_unaligned_output(n_bytes, out_shift):
    """Bytes after the last 16-byte chunk, and an output pointer off the 16-byte grid (the
    per-byte kernel), both through the C ABI."""
    g = torch.Generator().manual_seed(n_bytes)
    packed = torch.randint(0, 256, (n_bytes,), generator=g, dtype=torch.int32).to(torch.uint8)
    n_blocks = -(-n_bytes // 32)
    absmax_u8 = torch.randint(0, 256, (n_blocks,), generator=g, dtype=torch.int32).to(torch.uint8)
    absmax2 = 0.01 + 0.09 * torch.rand(-(-n_blocks // 256), generator=g)
    code2 = workloads.dynamic_code_signed()
    nf4_t = torch.tensor(workloads.NF4_LEVELS, dtype=torch.float32)
    offset = torch.tensor([0.0277], dtype=torch.float32)
    dev = [x.to(DEV) for x in (packed, absmax_u8, code2, absmax2, offset, nf4_t)]
    buf = torch.empty(2 * n_bytes + out_shift, dtype=torch.float16, device=DEV)
    out = buf[out_shift:]
    _ext.call("soupk_nf4_unpack", *[_ext.ptr(x) for x in dev], _ext.ptr(out), n_bytes, 64, 256,
              _ext.stream_of(out))
    ref = dequant_nf4(packed.numpy(), absmax_u8.numpy(), code2.numpy(), absmax2.numpy(),
                      offset.numpy(), nf4_t.numpy())
    assert np.array_equal(bits(out), ref.view(np.int16))


def test_rejects_invalid_arguments():
    x = torch.zeros(64, dtype=torch.uint8, device=DEV)
    out = torch.empty(128, dtype=torch.float16, device=DEV)
    with pytest.raises(_ext.SoupkError):
        _ext.call("soupk_nf4_unpack", _ext.ptr(x), _ext.ptr(x), _ext.ptr(out), _ext.ptr(out),
                  _ext.ptr(out), _ext.ptr(out), _ext.ptr(out), 64, 63, 256, _ext.stream_of(out))
    w = workloads.nf4_weight(16, 64, seed=5, device=DEV)
    with pytest.raises(ValueError):
        nf4.unpack_into(w, torch.empty((16, 64), dtype=torch.float16))   # CPU output


def _raw_part(n_bytes, seed):
    """A packed NF4 stream of n_bytes with random codes and scales (host tensors)."""
    g = torch.Generator().manual_seed(seed)
    packed = torch.randint(0, 256, (n_bytes,), generator=g, dtype=torch.int32).to(torch.uint8)
    n_blocks = -(-n_bytes // 32)
    absmax_u8 = torch.randint(0, 256, (max(n_blocks, 1),), generator=g,
                              dtype=torch.int32).to(torch.uint8)
    absmax2 = 0.01 + 0.09 * torch.rand(max(-(-n_blocks // 256), 1), generator=g)
    offset = torch.tensor([0.01 * (seed % 7)], dtype=torch.float32)
    return packed, absmax_u8, absmax2, offset


def test_unpack_multi_through_abi():
    """soupk_nf4_unpack_multi against the oracle, part by part: whole tiles, a part ending
    mid-tile, a byte tail (n_bytes % 4), an output off the 16-byte grid (both on the per-part
    fallback) and an empty part, in one call."""
    import ctypes

    specs = [(16384 * 3, 0), (5000 * 4, 0), (16 * 100 + 3, 0), (4096, 1), (0, 0), (64, 0)]
    code2 = workloads.dynamic_code_signed().to(DEV)
    nf4_t = torch.tensor(workloads.NF4_LEVELS, dtype=torch.float32, device=DEV)
    parts, outs, refs = [], [], []
    for i, (n_bytes, shift) in enumerate(specs):
        packed, absmax_u8, absmax2, offset = _raw_part(n_bytes, 70 + i)
        dev = [x.to(DEV) for x in (packed, absmax_u8, absmax2, offset)]
        buf = torch.full((2 * n_bytes + shift + 8,), float("nan"), dtype=torch.float16,
                         device=DEV)
        parts.append(dev)
        outs.append((buf, buf[shift:shift + 2 * n_bytes]))
        refs.append(dequant_nf4(packed.numpy(), absmax_u8.numpy(), code2.cpu().numpy(),
                                absmax2.numpy(), offset.numpy(), nf4_t.cpu().numpy())
                    if n_bytes else np.zeros(0, np.float16))
    n = len(specs)

    def arr(values):
        return (ctypes.c_void_p * n)(*values)

    keep = [arr([p[0].data_ptr() for p in parts]), arr([p[1].data_ptr() for p in parts]),
            arr([code2.data_ptr()] * n), arr([p[2].data_ptr() for p in parts]),
            arr([p[3].data_ptr() for p in parts]), arr([nf4_t.data_ptr()] * n),
            arr([o.data_ptr() for _, o in outs])]
    sizes = (ctypes.c_int64 * n)(*[s for s, _ in specs])
    _ext.call("soupk_nf4_unpack_multi", n, *[ctypes.addressof(a) for a in keep],
              ctypes.addressof(sizes), 64, 256, _ext.stream_of(code2))
    for (n_bytes, shift), (buf, out), ref in zip(specs, outs, refs):
        assert np.array_equal(bits(out), ref.view(np.int16)), n_bytes
        rest = torch.cat([buf[:shift], buf[shift + 2 * n_bytes:]])
        assert bool(torch.isnan(rest).all()), "wrote outside its part"


def test_unpack_groups_one_buffer():
    """unpack_groups: the row stacks of a layer (here 11 weights in 4 groups, more than one
    launch's 8 parts) bit-identical to the oracle, stacked and aligned as unpack_concat's."""
    groups = (((96, 640), (32, 640), (32, 640)), ((640, 64),), ((128, 640), (128, 640)),
              ((640, 128),), ((64, 640), (64, 640), (64, 640), (64, 640)))
    weights = [tuple(workloads.nf4_weight(*shape, seed=80 + 10 * gi + wi, device=DEV)
                     for wi, shape in enumerate(group)) for gi, group in enumerate(groups)]
    stacks = nf4.unpack_groups(weights, DEV)
    base = stacks[0].data_ptr()
    for group, stack in zip(weights, stacks):
        assert stack.is_contiguous() and (stack.data_ptr() - base) % 512 == 0
        ref = np.concatenate([dequant_state(w) for w in group])
        assert np.array_equal(bits(stack), ref.view(np.int16))
        assert torch.equal(stack, nf4.unpack_concat(group, DEV))
    # the second call runs the prepared launches; a replaced state must be seen by the next
    again = nf4.unpack_groups(weights, DEV)
    assert all(torch.equal(a, b) for a, b in zip(again, stacks))
    st = weights[2][1].quant_state
    st.absmax = torch.flip(st.absmax, [0]).contiguous()
    st.offset = 0.25
    third = nf4.unpack_groups(weights, DEV)
    ref = np.concatenate([dequant_state(w) for w in weights[2]])
    assert np.array_equal(bits(third[2]), ref.view(np.int16))
    assert not torch.equal(third[2], stacks[2])


def test_unpack_groups_lora_stages_in_the_same_launch():
    """unpack_groups_lora: the stacks bit-identical to unpack_groups', and the LoRA staging
    (extra workgroups of the last launch) bit-identical to lora.stage; over more than one
    launch (11 weights) and over one."""
    from testt_amd import lora

    H, NQ, NV = 640, 384, 128
    g = torch.Generator().manual_seed(5)
    params = ((torch.randn(16, H, generator=g) / 25).to(DEV),
              (torch.randn(16, H, generator=g) / 25).to(DEV),
              (torch.randn(NQ, 16, generator=g) / 20).to(DEV),
              (torch.randn(NV, 16, generator=g) / 20).to(DEV))
    for groups in ((((96, 640), (32, 640), (32, 640)), ((640, 64),), ((128, 640), (128, 640)),
                    ((640, 128),), ((64, 640), (64, 640), (64, 640), (64, 640))),
                   (((128, 640), (64, 640)), ((640, 128),))):
        weights = [tuple(workloads.nf4_weight(*shape, seed=90 + 10 * gi + wi, device=DEV)
                         for wi, shape in enumerate(group)) for gi, group in enumerate(groups)]
        print(f"unpack_groups_lora: {sum(len(gr) for gr in groups)} weights", flush=True)
        stacks, staged = nf4.unpack_groups_lora(weights, DEV, params)
        want = nf4.unpack_groups(weights, DEV)
        assert all(torch.equal(a, b) for a, b in zip(stacks, want))
        assert staged.data_ptr() % 16 == 0
        assert torch.equal(staged, lora.stage(*params))


def test_unpack_multi_rejects_invalid_arguments():
    import ctypes

    one = (ctypes.c_void_p * 9)()
    sizes = (ctypes.c_int64 * 9)()
    for n_parts, qblock in ((9, 64), (-1, 64), (1, 63)):
        with pytest.raises(_ext.SoupkError):
            _ext.call("soupk_nf4_unpack_multi", n_parts, *[ctypes.addressof(one)] * 7,
                      ctypes.addressof(sizes), qblock, 256, None)
    sizes[0] = 64                      # a non-empty part with null pointers
    with pytest.raises(_ext.SoupkError):
        _ext.call("soupk_nf4_unpack_multi", 1, *[ctypes.addressof(one)] * 7,
                  ctypes.addressof(sizes), 64, 256, None)
