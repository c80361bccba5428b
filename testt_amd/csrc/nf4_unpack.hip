// NF4 double-quant unpack: bitsandbytes 4-bit codes -> fp16 weights, one pass over HBM.
//
// Reference: solution/nf4.py:27-45 (nf4_unpack_kernel) and its launch in unpack_into,
// solution/nf4.py:72-89.  The arithmetic is the bitsandbytes closed form restated at
// solution/nf4.py:8-9 with each product and sum rounded on its own (solution/nf4.py:84).
//
// Layout and mapping (gfx950):
//   * one thread handles one 16-byte chunk of packed codes per step = 32 weights = 64 bytes of
//     fp16 output (four 16-byte stores); a workgroup step covers 256 consecutive chunks, so each
//     load instruction of a wave reads 1 KiB of contiguous HBM;
//   * a 16-byte chunk never straddles an absmax block when qblock is a multiple of 32 (every
//     bitsandbytes block size), so each chunk needs one scale: code2[absmax_u8[b]] *
//     absmax2[b >> log2(qblock2)] + offset, three cache-resident loads per 32 weights;
//   * the 16-entry NF4 codebook is expanded in LDS into a 256-entry table of (high, low) nibble
//     value pairs, so one ds_read_b64 per packed byte yields both codes' fp32 values;
//   * grid-stride over steps with a grid sized to the device's compute units.
// Other layouts (qblock or qblock2 not a power of two, unaligned pointers) take a one-byte-per-
// thread kernel with the same arithmetic.

#include "soupk_common.hpp"

namespace soupk {
namespace {

constexpr int kNf4Threads = 256;
constexpr int kNf4Unroll = 4;  // chunks per thread per grid-stride step (loads issued together)

__device__ __forceinline__ uint32_t nf4_pair_word(uint32_t byte, float scale,
                                                  const float2* __restrict__ pair) {
  const float2 t = pair[byte];
  return pack_h2(t.x * scale, t.y * scale);
}

// 4 packed bytes (lowest address first) -> 8 fp16 weights (high nibble first within a byte).
__device__ __forceinline__ u32x4 nf4_expand_dword(uint32_t w, float scale,
                                                  const float2* __restrict__ pair) {
  u32x4 r;
  r.x = nf4_pair_word(w & 0xffu, scale, pair);
  r.y = nf4_pair_word((w >> 8) & 0xffu, scale, pair);
  r.z = nf4_pair_word((w >> 16) & 0xffu, scale, pair);
  r.w = nf4_pair_word(w >> 24, scale, pair);
  return r;
}

__global__ __launch_bounds__(kNf4Threads) void nf4_unpack_vec_kernel(
    const u32x4* __restrict__ packed, const uint8_t* __restrict__ absmax_u8,
    const float* __restrict__ code2, const float* __restrict__ absmax2,
    const float* __restrict__ offset, const float* __restrict__ nf4, u32x4* __restrict__ out,
    int64_t n_chunks, int chunk_block_shift, int block2_shift) {
  __shared__ float2 pair[256];
  pair[threadIdx.x] = make_float2(nf4[threadIdx.x >> 4], nf4[threadIdx.x & 15]);
  __syncthreads();
  const float off = offset[0];
  const int64_t step_chunks = static_cast<int64_t>(kNf4Threads) * kNf4Unroll;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * step_chunks; base < n_chunks;
       base += static_cast<int64_t>(gridDim.x) * step_chunks) {
    u32x4 v[kNf4Unroll];
    float prod[kNf4Unroll];
#pragma unroll
    for (int u = 0; u < kNf4Unroll; ++u) {
      const int64_t c = base + u * kNf4Threads + threadIdx.x;
      if (c < n_chunks) {
        v[u] = __builtin_nontemporal_load(packed + c);
        const int64_t blk = c >> chunk_block_shift;
        prod[u] = code2[absmax_u8[blk]] * absmax2[blk >> block2_shift];
      }
    }
#pragma unroll
    for (int u = 0; u < kNf4Unroll; ++u) {
      const int64_t c = base + u * kNf4Threads + threadIdx.x;
      if (c < n_chunks) {
        const float scale = prod[u] + off;
        u32x4* dst = out + 4 * c;
        dst[0] = nf4_expand_dword(v[u].x, scale, pair);
        dst[1] = nf4_expand_dword(v[u].y, scale, pair);
        dst[2] = nf4_expand_dword(v[u].z, scale, pair);
        dst[3] = nf4_expand_dword(v[u].w, scale, pair);
      }
    }
  }
}

// One packed byte per thread; any even qblock, any qblock2, any alignment.  Also used for the
// bytes after the last whole 16-byte chunk of the vector kernel.
__global__ __launch_bounds__(kNf4Threads) void nf4_unpack_byte_kernel(
    const uint8_t* __restrict__ packed, const uint8_t* __restrict__ absmax_u8,
    const float* __restrict__ code2, const float* __restrict__ absmax2,
    const float* __restrict__ offset, const float* __restrict__ nf4, uint16_t* __restrict__ out,
    int64_t first_byte, int64_t n_bytes, int64_t bytes_per_block, int64_t qblock2) {
  const int64_t i = first_byte + static_cast<int64_t>(blockIdx.x) * kNf4Threads + threadIdx.x;
  if (i >= n_bytes) return;
  const uint32_t p = packed[i];
  const int64_t blk = i / bytes_per_block;
  const float prod = code2[absmax_u8[blk]] * absmax2[blk / qblock2];
  const float scale = prod + offset[0];
  const uint32_t w = pack_h2(nf4[p >> 4] * scale, nf4[p & 15u] * scale);
  out[2 * i] = static_cast<uint16_t>(w & 0xffffu);
  out[2 * i + 1] = static_cast<uint16_t>(w >> 16);
}

inline bool is_pow2(int64_t v) { return v > 0 && (v & (v - 1)) == 0; }
inline int log2_exact(int64_t v) {
  int s = 0;
  while ((int64_t{1} << s) < v) ++s;
  return s;
}
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace
}  // namespace soupk

using namespace soupk;

extern "C" __attribute__((visibility("default"))) int soupk_nf4_unpack(
    const uint8_t* packed, const uint8_t* absmax_u8, const float* code2, const float* absmax2,
    const float* offset, const float* nf4, uint16_t* out_f16, int64_t n_bytes, int32_t qblock,
    int32_t qblock2, void* stream) {
  if (n_bytes < 0 || qblock <= 0 || (qblock & 1) || qblock2 <= 0) return kInvalid;
  if (n_bytes == 0) return kOk;
  if (!packed || !absmax_u8 || !code2 || !absmax2 || !offset || !nf4 || !out_f16) return kInvalid;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t bytes_per_block = qblock / 2;
  int64_t vec_bytes = 0;
  if (qblock % 32 == 0 && is_pow2(qblock) && is_pow2(qblock2) && aligned16(packed) &&
      aligned16(out_f16)) {
    const int64_t n_chunks = n_bytes / 16;
    vec_bytes = n_chunks * 16;
    if (n_chunks > 0) {
      const int64_t step_chunks = static_cast<int64_t>(kNf4Threads) * kNf4Unroll;
      const int64_t steps = (n_chunks + step_chunks - 1) / step_chunks;
      const int64_t cap = static_cast<int64_t>(device_cu_count()) * 8;
      const int grid = static_cast<int>(steps < cap ? steps : cap);
      nf4_unpack_vec_kernel<<<grid, kNf4Threads, 0, s>>>(
          reinterpret_cast<const u32x4*>(packed), absmax_u8, code2, absmax2, offset, nf4,
          reinterpret_cast<u32x4*>(out_f16), n_chunks, log2_exact(qblock / 32),
          log2_exact(qblock2));
      const int st = launch_status();
      if (st != kOk) return st;
    }
  }
  const int64_t rest = n_bytes - vec_bytes;
  if (rest > 0) {
    const int64_t grid = (rest + kNf4Threads - 1) / kNf4Threads;
    if (grid > 0x7fffffff) return kInvalid;
    nf4_unpack_byte_kernel<<<static_cast<int>(grid), kNf4Threads, 0, s>>>(
        packed, absmax_u8, code2, absmax2, offset, nf4, out_f16, vec_bytes, n_bytes,
        bytes_per_block, qblock2);
    return launch_status();
  }
  return kOk;
}
