"""NF4 double-quant dequantization (the closed form) and a bitsandbytes-style quantizer.
TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).

dequant_nf4 restates solution/nf4.py:8-9 with the operation order of solution/nf4.py:36-45
and the separate rounding of solution/nf4.py:84 (enable_fp_fusion=False):

    prod      = fp32(code2[absmax_u8[b]] * absmax2[b // qblock2])
    absmax[b] = fp32(prod + offset)
    w[2i]     = fp16_rn(fp32(nf4[packed[i] >> 4] * absmax[i // (qblock/2)]))
    w[2i+1]   = fp16_rn(fp32(nf4[packed[i] & 15] * absmax[i // (qblock/2)]))

bitsandbytes 0.50.2 (pinned by the reference, README.md:171-172; not installed here) computes
the same values in two launches (blockwise 8-bit dequant of the absmax, then the 4-bit
dequant); its `dequantize_4bit` equality with the reference kernel is the reference's own GPU
test (solution/test_kernels.py:43-51), which cannot run without bitsandbytes.  Pinned here by:
the float64 route (products of fp32 values are exact in float64, so rounding them to fp32 gives
the correctly rounded fp32 product; for sums the 53-bit double rounding is also correct), by
the codebook special cases (code 7 -> 0, code 15 -> fp16(scale)), by a hand-built known-answer
vector for the nibble order and the block indices, and by the quantize -> dequantize round trip
(tests/test_oracle_nf4.py).

quantize_nf4 restates bitsandbytes' published quantize_4bit(..., quant_type="nf4",
compress_statistics=True) algorithm: per 64-value block absmax, nearest NF4 level of w/absmax,
two codes per byte with the lower index in the high nibble; then double quant: offset =
mean(absmax), and (absmax - offset) blockwise-quantized to the nearest entry of the signed
dynamic 8-bit code, per 256 absmax values scaled by their max magnitude.
"""

import numpy as np


def dequant_nf4(packed, absmax_u8, code2, absmax2, offset, nf4, qblock=64, qblock2=256):
    """fp16 numpy array [2 * n_bytes] (the row-major weight)."""
    packed = np.ascontiguousarray(packed, dtype=np.uint8).reshape(-1)
    absmax_u8 = np.asarray(absmax_u8, dtype=np.uint8).reshape(-1)
    code2 = np.asarray(code2, dtype=np.float32).reshape(-1)
    absmax2 = np.asarray(absmax2, dtype=np.float32).reshape(-1)
    nf4 = np.asarray(nf4, dtype=np.float32).reshape(-1)
    off = np.float32(np.asarray(offset, dtype=np.float32).reshape(-1)[0])
    n = packed.size
    blk = np.arange(n, dtype=np.int64) // (qblock // 2)
    prod = code2[absmax_u8[blk]] * absmax2[blk // qblock2]          # fp32 * fp32 -> fp32
    scale = (prod + off).astype(np.float32)                          # fp32 + fp32 -> fp32
    first = (nf4[packed >> 4] * scale).astype(np.float32)
    second = (nf4[packed & 15] * scale).astype(np.float32)
    out = np.empty(2 * n, dtype=np.float16)
    out[0::2] = first.astype(np.float16)                             # round to nearest even
    out[1::2] = second.astype(np.float16)
    return out


def dequant_state(weight):
    """dequant_nf4 of a Params4bit-like object (.data, .quant_state), as [N, K] fp16 numpy."""
    st = weight.quant_state

    def host(t):
        return t.detach().cpu().numpy() if hasattr(t, "detach") else np.asarray(t)

    out = dequant_nf4(host(weight.data), host(st.absmax), host(st.state2.code),
                      host(st.state2.absmax), host(st.offset), host(st.code), st.blocksize,
                      st.state2.blocksize)
    return out.reshape(tuple(st.shape))


def _nearest(levels, values):
    """Index of the nearest entry of the ascending table `levels` for each value."""
    idx = np.searchsorted(levels, values)
    idx = np.clip(idx, 1, len(levels) - 1)
    left, right = levels[idx - 1], levels[idx]
    return np.where(np.abs(values - left) <= np.abs(right - values), idx - 1, idx)


def quantize_nf4(w16, nf4_levels, code2, qblock=64, qblock2=256):
    """(packed uint8 [n/2], absmax_u8 uint8 [n/qblock], absmax2 fp32, offset fp32) for an fp16
    weight, following bitsandbytes' quantize_4bit with compress_statistics=True."""
    w = np.asarray(w16, dtype=np.float16).astype(np.float32).reshape(-1)
    if w.size % qblock:
        raise ValueError("weight size must be a multiple of the block size")
    levels = np.asarray(nf4_levels, dtype=np.float32)
    blocks = w.reshape(-1, qblock)
    absmax = np.abs(blocks).max(axis=1).astype(np.float32)
    safe = np.where(absmax == 0, np.float32(1), absmax)
    codes = _nearest(levels, (blocks / safe[:, None]).reshape(-1)).astype(np.uint8)
    packed = ((codes[0::2] << 4) | codes[1::2]).astype(np.uint8)
    offset = np.float32(absmax.mean(dtype=np.float64))
    centred = (absmax - offset).astype(np.float32)
    pad = (-centred.size) % qblock2
    groups = np.concatenate([centred, np.zeros(pad, np.float32)]).reshape(-1, qblock2)
    absmax2 = np.abs(groups).max(axis=1).astype(np.float32)
    safe2 = np.where(absmax2 == 0, np.float32(1), absmax2)
    table = np.asarray(code2, dtype=np.float32)
    q = _nearest(table, (groups / safe2[:, None]).reshape(-1))[: centred.size].astype(np.uint8)
    return packed, q, absmax2, offset
