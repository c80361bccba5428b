// NF4 double-quant unpack: bitsandbytes 4-bit codes -> fp16 weights, one pass over HBM.
//
// Reference: solution/nf4.py:27-45 (nf4_unpack_kernel) and its launch in unpack_into,
// solution/nf4.py:72-89.  The arithmetic is the bitsandbytes closed form restated at
// solution/nf4.py:8-9 with each product and sum rounded on its own (solution/nf4.py:84).
//
// Layout and mapping (gfx950):
//   * the unit of work is one packed dword (4 bytes = 8 codes) -> one 16-byte fp16 store; lane l
//     of a wavefront takes dword l, l+64, ... of the wave's slice, so every load instruction of
//     a wave reads 256 contiguous bytes and every store instruction writes 1 KiB contiguous;
//   * a workgroup tile is 256 threads x kNf4Dwords dwords; the block scales of the tile
//     (code2[absmax_u8[b]] * absmax2[b >> log2(qblock2)] + offset, the double-quantised absmax)
//     are computed once per block by the first threads into LDS, instead of once per lane;
//   * the 16-entry NF4 codebook is expanded in LDS into a 256-entry table of (high, low) nibble
//     value pairs, so one ds_read_b64 per packed byte yields both codes' fp32 values;
//   * one tile per workgroup (1,680 workgroups for a [17920, 1536] weight).
// Other layouts (qblock or qblock2 not a power of two, qblock < 8, unaligned pointers) take a
// one-byte-per-thread kernel with the same arithmetic, which also handles the last n_bytes % 4.

#include "lora_stage.hpp"
#include "soupk_common.hpp"

namespace soupk {
namespace {

constexpr int kNf4Threads = 256;
#ifndef SOUPK_NF4_DWORDS
#define SOUPK_NF4_DWORDS 8
#endif
constexpr int kNf4Dwords = SOUPK_NF4_DWORDS;                 // dwords per thread per tile
constexpr int kNf4TileDwords = kNf4Threads * kNf4Dwords;     // 8 KiB of packed codes

// 4 packed bytes (lowest address first) -> 8 fp16 weights (high nibble first within a byte).
__device__ __forceinline__ u32x4 nf4_expand_dword(uint32_t w, float scale,
                                                  const float2* __restrict__ pair) {
  const float2 t0 = pair[w & 0xffu];
  const float2 t1 = pair[(w >> 8) & 0xffu];
  const float2 t2 = pair[(w >> 16) & 0xffu];
  const float2 t3 = pair[w >> 24];
  return u32x4{pack_h2(t0.x * scale, t0.y * scale), pack_h2(t1.x * scale, t1.y * scale),
               pack_h2(t2.x * scale, t2.y * scale), pack_h2(t3.x * scale, t3.y * scale)};
}

// dword_block_shift = log2(dwords per absmax block) = log2(qblock / 8); block2_shift =
// log2(qblock2).  Requires qblock a power of two in [8, 8 * kNf4TileDwords] (a dword never
// straddles two blocks, and a tile spans whole blocks).  One tile per workgroup; the packed loads are issued
// unconditionally (indices past the end clamped to the last dword, results dropped), because a
// predicated load makes the compiler wait on it before issuing the next.
// Cache policy of the packed codes (1 = non-temporal: touched once); the fp16 output is written
// with streaming stores (StreamOut: nt | sc1).
#ifndef SOUPK_NF4_NT_LD
#define SOUPK_NF4_NT_LD 1
#endif
constexpr bool kNf4NtLd = SOUPK_NF4_NT_LD != 0;

// One tile (256 threads x kNf4Dwords dwords, from dword d0) of one weight.
__device__ __forceinline__ void nf4_unpack_tile(
    const uint32_t* __restrict__ packed, const uint8_t* __restrict__ absmax_u8,
    const float* __restrict__ code2, const float* __restrict__ absmax2,
    const float* __restrict__ offset, const float* __restrict__ nf4, u32x4* __restrict__ out,
    int64_t d0, int64_t n_dwords, int64_t n_blocks, int dword_block_shift, int block2_shift,
    float2* pair, float* scale) {
  uint32_t w[kNf4Dwords];
#pragma unroll
  for (int k = 0; k < kNf4Dwords; ++k) {
    const int64_t d = d0 + k * kNf4Threads + threadIdx.x;
    w[k] = ld<kNf4NtLd>(packed + (d < n_dwords ? d : n_dwords - 1));
  }
  pair[threadIdx.x] = make_float2(nf4[threadIdx.x >> 4], nf4[threadIdx.x & 15]);
  const float off = offset[0];
  const int tile_blocks = kNf4TileDwords >> dword_block_shift;
  const int64_t b0 = d0 >> dword_block_shift;
  for (int i = threadIdx.x; i < tile_blocks; i += kNf4Threads) {
    const int64_t b = b0 + i;
    if (b < n_blocks) {
      const float prod = code2[absmax_u8[b]] * absmax2[b >> block2_shift];
      scale[i] = prod + off;
    }
  }
  __syncthreads();
  // The tile's stores: dword d at byte 16 (d - d0) of a descriptor from d0 to the end of the
  // output (dwords past the end fall outside it and are dropped).
  const StreamOut dst(out + d0, static_cast<uint64_t>(n_dwords - d0) * 16u);
#pragma unroll
  for (int k = 0; k < kNf4Dwords; ++k) {
    const int i = k * kNf4Threads + threadIdx.x;
    const u32x4 v = nf4_expand_dword(w[k], scale[i >> dword_block_shift], pair);
    dst.store(static_cast<uint32_t>(i) * 16u, v);
  }
}

__global__ __launch_bounds__(kNf4Threads) void nf4_unpack_vec_kernel(
    const uint32_t* __restrict__ packed, const uint8_t* __restrict__ absmax_u8,
    const float* __restrict__ code2, const float* __restrict__ absmax2,
    const float* __restrict__ offset, const float* __restrict__ nf4, u32x4* __restrict__ out,
    int64_t n_dwords, int64_t n_blocks, int dword_block_shift, int block2_shift) {
  __shared__ float2 pair[256];
  __shared__ float scale[kNf4TileDwords];  // enough for qblock >= 8 (1 block per dword)
  nf4_unpack_tile(packed, absmax_u8, code2, absmax2, offset, nf4, out,
                  static_cast<int64_t>(blockIdx.x) * kNf4TileDwords, n_dwords, n_blocks,
                  dword_block_shift, block2_shift, pair, scale);
}

// Several weights in one launch (the projections of a decoder layer): workgroup x unpacks tile
// x - first_tile[p] of part p, first_tile[p] <= x < first_tile[p + 1].  The part table is a
// kernel argument (read through the scalar unit); every part takes the vector path.
constexpr int kNf4MaxParts = 8;
struct Nf4Parts {
  const uint32_t* packed[kNf4MaxParts];
  const uint8_t* absmax_u8[kNf4MaxParts];
  const float* code2[kNf4MaxParts];
  const float* absmax2[kNf4MaxParts];
  const float* offset[kNf4MaxParts];
  const float* nf4[kNf4MaxParts];
  u32x4* out[kNf4MaxParts];
  int64_t n_dwords[kNf4MaxParts];
  int64_t n_blocks[kNf4MaxParts];
  int first_tile[kNf4MaxParts + 1];
  int n_parts;
};

__global__ __launch_bounds__(kNf4Threads) void nf4_unpack_multi_kernel(Nf4Parts parts,
                                                                       int dword_block_shift,
                                                                       int block2_shift) {
  __shared__ float2 pair[256];
  __shared__ float scale[kNf4TileDwords];
  const int x = static_cast<int>(blockIdx.x);
  // p = the number of parts 1..n_parts-1 whose first tile is <= x (first_tile is non-decreasing).
  // Unrolled over constant offsets, the table arrives in one batch of scalar loads; a search
  // loop waits on one scalar load per part passed before the tile's first packed load.
  int p = 0;
#pragma unroll
  for (int q = 1; q < kNf4MaxParts; ++q)
    p += (q < parts.n_parts && x >= parts.first_tile[q]) ? 1 : 0;
  nf4_unpack_tile(parts.packed[p], parts.absmax_u8[p], parts.code2[p], parts.absmax2[p],
                  parts.offset[p], parts.nf4[p], parts.out[p],
                  static_cast<int64_t>(x - parts.first_tile[p]) * kNf4TileDwords,
                  parts.n_dwords[p], parts.n_blocks[p], dword_block_shift, block2_shift, pair,
                  scale);
}

// The same launch with extra workgroups after the NF4 tiles that stage a decoder layer's LoRA
// parameters in fp16 (lora_stage.hpp), so that preparing the layer's weights takes one launch.
__global__ __launch_bounds__(kNf4Threads) void nf4_unpack_multi_lora_kernel(
    Nf4Parts parts, int dword_block_shift, int block2_shift, LoraStageArgs lora, int nf4_tiles) {
  __shared__ float2 pair[256];
  __shared__ float scale[kNf4TileDwords];
  const int x = static_cast<int>(blockIdx.x);
  if (x >= nf4_tiles) {   // a whole workgroup: no barrier below is reached by part of one
    lora_stage_value(lora, static_cast<int64_t>(x - nf4_tiles) * kNf4Threads + threadIdx.x);
    return;
  }
  int p = 0;
#pragma unroll
  for (int q = 1; q < kNf4MaxParts; ++q)
    p += (q < parts.n_parts && x >= parts.first_tile[q]) ? 1 : 0;
  nf4_unpack_tile(parts.packed[p], parts.absmax_u8[p], parts.code2[p], parts.absmax2[p],
                  parts.offset[p], parts.nf4[p], parts.out[p],
                  static_cast<int64_t>(x - parts.first_tile[p]) * kNf4TileDwords,
                  parts.n_dwords[p], parts.n_blocks[p], dword_block_shift, block2_shift, pair,
                  scale);
}

// One packed byte per thread; any even qblock, any qblock2, any alignment.  Also used for the
// bytes after the last whole dword of the vector kernel.
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
inline bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

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
  const int64_t n_blocks = (n_bytes + bytes_per_block - 1) / bytes_per_block;
  int64_t vec_bytes = 0;
  // (qblock / 8 <= kNf4TileDwords: a tile spans whole absmax blocks)
  if (qblock >= 8 && qblock / 8 <= kNf4TileDwords && is_pow2(qblock) && is_pow2(qblock2) &&
      aligned(packed, 4) && aligned(out_f16, 16)) {
    const int64_t n_dwords = n_bytes / 4;
    vec_bytes = n_dwords * 4;
    if (n_dwords > 0) {
      const int64_t tiles = (n_dwords + kNf4TileDwords - 1) / kNf4TileDwords;
      if (tiles > 0x7fffffff) return kInvalid;
      const int st = launch_kernel(
          nf4_unpack_vec_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kNf4Threads), s,
          reinterpret_cast<const uint32_t*>(packed), absmax_u8, code2, absmax2, offset, nf4,
          reinterpret_cast<u32x4*>(out_f16), n_dwords, n_blocks, log2_exact(qblock / 8),
          log2_exact(qblock2));
      if (st != kOk) return st;
    }
  }
  const int64_t rest = n_bytes - vec_bytes;
  if (rest > 0) {
    const int64_t grid = (rest + kNf4Threads - 1) / kNf4Threads;
    if (grid > 0x7fffffff) return kInvalid;
    return launch_kernel(nf4_unpack_byte_kernel, dim3(static_cast<unsigned>(grid)),
                         dim3(kNf4Threads), s, packed, absmax_u8, code2, absmax2, offset, nf4,
                         out_f16, vec_bytes, n_bytes, bytes_per_block,
                         static_cast<int64_t>(qblock2));
  }
  return kOk;
}

namespace soupk {
namespace {

// The vector-path parts of a multi-part unpack as one tile table; parts the tiles do not take
// are unpacked at once by their own launches (soupk_nf4_unpack).
int nf4_multi_parts(int32_t n_parts, const uint8_t* const* packed,
                    const uint8_t* const* absmax_u8, const float* const* code2,
                    const float* const* absmax2, const float* const* offset,
                    const float* const* nf4, uint16_t* const* out_f16, const int64_t* n_bytes,
                    int32_t qblock, int32_t qblock2, void* stream, Nf4Parts* parts,
                    int64_t* tiles_out) {
  if (n_parts < 0 || n_parts > kNf4MaxParts || qblock <= 0 || (qblock & 1) || qblock2 <= 0)
    return kInvalid;
  *tiles_out = 0;
  if (n_parts == 0) return kOk;
  if (!packed || !absmax_u8 || !code2 || !absmax2 || !offset || !nf4 || !out_f16 || !n_bytes)
    return kInvalid;
  for (int i = 0; i < n_parts; ++i) {
    if (n_bytes[i] < 0) return kInvalid;
    if (n_bytes[i] > 0 && (!packed[i] || !absmax_u8[i] || !code2[i] || !absmax2[i] ||
                           !offset[i] || !nf4[i] || !out_f16[i]))
      return kInvalid;
  }
  const bool vec_layout = qblock >= 8 && qblock / 8 <= kNf4TileDwords && is_pow2(qblock) &&
                          is_pow2(qblock2);
  const int64_t bytes_per_block = qblock / 2;
  *parts = Nf4Parts{};
  int64_t tiles = 0;
  for (int i = 0; i < n_parts; ++i) {
    if (n_bytes[i] == 0) continue;
    const bool vec = vec_layout && n_bytes[i] % 4 == 0 && aligned(packed[i], 4) &&
                     aligned(out_f16[i], 16);
    if (!vec) {   // a layout the tiles do not take: its own launches, as soupk_nf4_unpack
      const int st = soupk_nf4_unpack(packed[i], absmax_u8[i], code2[i], absmax2[i], offset[i],
                                      nf4[i], out_f16[i], n_bytes[i], qblock, qblock2, stream);
      if (st != kOk) return st;
      continue;
    }
    const int j = parts->n_parts++;
    parts->packed[j] = reinterpret_cast<const uint32_t*>(packed[i]);
    parts->absmax_u8[j] = absmax_u8[i];
    parts->code2[j] = code2[i];
    parts->absmax2[j] = absmax2[i];
    parts->offset[j] = offset[i];
    parts->nf4[j] = nf4[i];
    parts->out[j] = reinterpret_cast<u32x4*>(out_f16[i]);
    parts->n_dwords[j] = n_bytes[i] / 4;
    parts->n_blocks[j] = (n_bytes[i] + bytes_per_block - 1) / bytes_per_block;
    parts->first_tile[j] = static_cast<int>(tiles);
    tiles += (parts->n_dwords[j] + kNf4TileDwords - 1) / kNf4TileDwords;
    if (tiles > 0x7fffffff) return kInvalid;
  }
  for (int j = parts->n_parts; j <= kNf4MaxParts; ++j)
    parts->first_tile[j] = static_cast<int>(tiles);
  *tiles_out = tiles;
  return kOk;
}

}  // namespace
}  // namespace soupk

extern "C" __attribute__((visibility("default"))) int soupk_nf4_unpack_multi(
    int32_t n_parts, const uint8_t* const* packed, const uint8_t* const* absmax_u8,
    const float* const* code2, const float* const* absmax2, const float* const* offset,
    const float* const* nf4, uint16_t* const* out_f16, const int64_t* n_bytes, int32_t qblock,
    int32_t qblock2, void* stream) {
  Nf4Parts parts;
  int64_t tiles = 0;
  const int rc = nf4_multi_parts(n_parts, packed, absmax_u8, code2, absmax2, offset, nf4,
                                 out_f16, n_bytes, qblock, qblock2, stream, &parts, &tiles);
  if (rc != kOk || tiles == 0) return rc;
  return launch_kernel(nf4_unpack_multi_kernel, dim3(static_cast<unsigned>(tiles)),
                       dim3(kNf4Threads), static_cast<hipStream_t>(stream), parts,
                       log2_exact(qblock / 8), log2_exact(qblock2));
}

extern "C" __attribute__((visibility("default"))) int soupk_nf4_unpack_multi_lora(
    int32_t n_parts, const uint8_t* const* packed, const uint8_t* const* absmax_u8,
    const float* const* code2, const float* const* absmax2, const float* const* offset,
    const float* const* nf4, uint16_t* const* out_f16, const int64_t* n_bytes, int32_t qblock,
    int32_t qblock2, const float* a_q, const float* a_v, const float* b_q, const float* b_v,
    uint16_t* staged, int64_t staged_elems, int32_t H, int32_t NQ, int32_t NV, int32_t r,
    void* stream) {
  // The LoRA arguments first (nothing launched if they are rejected): soupk_lora_stage's rules.
  if (r != kLoraRank || H <= 0 || NQ <= 0 || NV <= 0 || H % 128 || NQ % 128 || NV % 128)
    return kInvalid;
  if (!a_q || !a_v || !b_q || !b_v || !staged || !aligned(staged, 16)) return kInvalid;
  if (staged_elems < staged_layout(H, NQ, NV).total) return kInvalid;
  if (n_parts < 0 || n_parts > kNf4MaxParts) return kInvalid;
  Nf4Parts parts;
  int64_t tiles = 0;
  const int rc = nf4_multi_parts(n_parts, packed, absmax_u8, code2, absmax2, offset, nf4,
                                 out_f16, n_bytes, qblock, qblock2, stream, &parts, &tiles);
  if (rc != kOk) return rc;
  const int64_t stage_groups = (staged_values(H, NQ, NV) + kNf4Threads - 1) / kNf4Threads;
  if (tiles + stage_groups > 0x7fffffff) return kInvalid;
  const LoraStageArgs lora{a_q, a_v, b_q, b_v, reinterpret_cast<_Float16*>(staged), H, NQ, NV};
  const int qshift = tiles > 0 ? log2_exact(qblock / 8) : 0;
  const int q2shift = tiles > 0 ? log2_exact(qblock2) : 0;
  return launch_kernel(nf4_unpack_multi_lora_kernel,
                       dim3(static_cast<unsigned>(tiles + stage_groups)), dim3(kNf4Threads),
                       static_cast<hipStream_t>(stream), parts, qshift, q2shift, lora,
                       static_cast<int>(tiles));
}
