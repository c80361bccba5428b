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
