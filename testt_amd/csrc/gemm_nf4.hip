// y = x W^T (+ bias) with the frozen weight W read in NF4 (bitsandbytes double quant) and
// dequantised inside the GEMM, on gfx950 MFMA (v_mfma_f32_32x32x16_f16): the fused NF4-dequant
// GEMM the reference names as its next step (README.md:190-192, SUBMISSION.md:54-58), in place
// of unpacking W to fp16 in HBM (testt_amd/csrc/nf4_unpack.hip) and a hipBLASLt GEMM
// (solution/nf4.py:108-127).  The same kernel also takes an fp16 W (the plain GEMM), which is
// how its GEMM core is checked against hipBLASLt.
//
// Tiling: a workgroup computes a BM x BN tile of y (BM rows of x, BN rows of W) with WM x WN
// wavefronts, each a grid of 32 x 32 MFMA tiles (16 fp32 accumulators each); the shipped shape is
// 128 x 128 on 8 wavefronts (4 x 2, two per SIMD) of 32 x 64.  K advances in tiles of 64: x and
// W tiles are staged in LDS ([BM][72] / [BN][72] halves, double-buffered; the 72-half row stride
// makes the 16-byte fragment reads of 8 consecutive lanes hit 8 distinct 4-bank groups), the
// global loads run two tiles ahead of the MFMAs, and one barrier per K tile separates the LDS
// writes from the reads.
//
// NF4 weights: a 64-wide K tile of one W row is exactly one 64-value quantisation block, so a
// thread dequantises 32 codes of one row with one block scale:
//   scale = fp32(fp32(code2[absmax_u8[b]] * absmax2[b / 256]) + offset)
//   w     = fp16(nf4[code] * scale)          (the unpack kernel's arithmetic, bit for bit)
// code2 and nf4 staged in LDS.  W may be up to 4 row parts with their own quantisation states
// (q | k | v, gate | up), each a multiple of 128 rows.
//
// MFMA 32x32x16 layouts (checked on the device): A[32 x 16]: lane l holds row l%32,
// k = 8(l/32)..+7; B[16 x 32]: lane l holds column l%32, same k; C: element i of lane l is row
// 8(i/4) + 4(l/32) + i%4, column l%32.

#include "soupk_common.hpp"

namespace soupk {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16v __attribute__((ext_vector_type(16)));

constexpr int kQBlock = 64;            // NF4 quantisation block (values)
constexpr int kMaxParts = 4;

struct Nf4Part {
  const uint8_t* packed;     // [rows * K / 2] bytes, high nibble = even element
  const uint8_t* absmax_u8;  // [rows * K / 64]
  const float* code2;        // [256]
  const float* absmax2;      // [ceil(rows * K / 64 / 256)]
  const float* offset;       // [1]
  const float* nf4;          // [16]
  int rows;
};

struct Nf4Weights {
  Nf4Part part[kMaxParts];
  int n_parts;
};

__device__ __forceinline__ f16v mfma32x32(h8 a, h8 b, f16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void issue_here() { __asm__ volatile("" ::: "memory"); }

// Workgroups are dispatched to the 8 XCDs of the chip in turn (workgroup i to XCD i % 8), and
// each XCD has its own L2.  Tile order: XCD j takes the j-th eighth of the tiles in row-major
// (m-block, n-block) order, so the workgroups sharing an L2 work on few m-blocks -- their rows
// of x stay in that L2 while the XCD walks the n-blocks -- instead of every XCD reading all of
// x.  (With a tile count not divisible by 8 the plain order is kept.)
constexpr int kXcds = 8;
__device__ __forceinline__ void tile_of(int wg, int n_blocks, int m_blocks, int& nb, int& mb) {
  const int tiles = n_blocks * m_blocks;
  int t = wg;
  if (tiles % kXcds == 0) t = (wg % kXcds) * (tiles / kXcds) + wg / kXcds;
  mb = t / n_blocks;
  nb = t - mb * n_blocks;
}

// Tile shape of one launch: a BM x BN block of y per workgroup, WM x WN wavefronts, each a
// (BM/WM) x (BN/WN) tile of 32 x 32 MFMA tiles.
template <int BM_, int BN_, int WM_, int WN_, int BK_ = 64>
struct GemmShape {
  static constexpr int BM = BM_, BN = BN_, WM = WM_, WN = WN_, BK = BK_;
  static constexpr int kThreads = 64 * WM * WN;
  static constexpr int kLds = BK + 8;                // LDS row stride (halves)
  static constexpr int CPR = BK / 8;                 // 16-byte chunks per row of a K tile
  static constexpr int IPR = BK / 16;                // NF4 16-code items per row of a K tile
  static constexpr int TM = BM / WM, TN = BN / WN;   // wave tile
  static constexpr int FM = TM / 32, FN = TN / 32;   // 32 x 32 MFMA tiles per wave
  static constexpr int XC = BM * CPR / kThreads;     // 16-byte x chunks per thread per K tile
  static constexpr int WC = BN * CPR / kThreads;     // fp16 W chunks
  static constexpr int NI = (BN * IPR + kThreads - 1) / kThreads;   // NF4: 16-code items
  static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tiles are whole 32 x 32 MFMA tiles");
  static_assert(XC * kThreads == BM * CPR && WC * kThreads == BN * CPR, "whole chunks");
  static_assert(BK % kQBlock == 0, "a K tile holds whole quantisation blocks");
};

// Registers of one K tile for one thread: XC x 16 bytes of x (chunk c = tid + threads*j: row
// c / 8, 8 halves at 8 * (c % 8)); for W either WC x 16 bytes of fp16 (same mapping) or NI items
// of 16 NF4 codes (8 bytes; item i: row i / 4, codes 16 (i % 4) .. +15 of the row's 64-code
// block) with the block's scale inputs.
template <class S>
struct TileRegs {
  u32x4 x[S::XC];
  u32x4 w[S::WC];
  u32x2 c[S::NI];
  uint32_t ablk[S::NI];   // NF4: absmax_u8 of the block
  float a2[S::NI];        // NF4: absmax2 of the block's group
};

#ifndef SOUPK_GEMM_WPE
#define SOUPK_GEMM_WPE 0
#endif
template <class S, bool NF4>
__global__ __launch_bounds__(S::kThreads)
#if SOUPK_GEMM_WPE
__attribute__((amdgpu_waves_per_eu(SOUPK_GEMM_WPE, SOUPK_GEMM_WPE)))
#endif
void gemm_tn_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* w16, Nf4Weights nw,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int M, int N, int K,
    float* __restrict__ partial, int split_tiles) {
  constexpr int BM = S::BM, BN = S::BN, T = S::kThreads, kBK = S::BK, kLds = S::kLds;
  constexpr int CPR = S::CPR, IPR = S::IPR;
  // Two LDS stages as separate arrays, so that the compiler sees the staging of one and the
  // MFMA reads of the other as independent and interleaves them.
  __shared__ __align__(16) _Float16 Xs0[BM * kLds];
  __shared__ __align__(16) _Float16 Ws0[BN * kLds];
  __shared__ __align__(16) _Float16 Xs1[BM * kLds];
  __shared__ __align__(16) _Float16 Ws1[BN * kLds];
  __shared__ float code2_s[256];
  __shared__ float2 pair_s[256];   // NF4: (nf4[b >> 4], nf4[b & 15]) of byte value b
  const int tid = threadIdx.x;
  int nb, mb;
  tile_of(blockIdx.x, N / BN, (M + BM - 1) / BM, nb, mb);
  const int n0 = nb * BN, m0 = mb * BM;
  const int lane = tid % kWave, wv = tid / kWave;
  const int wm = wv / S::WN, wn = wv % S::WN;

  // the weight part holding rows n0 .. n0 + BN - 1, and the row of that part
  int part = 0, prow0 = n0;
  if constexpr (NF4) {
    while (part + 1 < nw.n_parts && prow0 >= nw.part[part].rows) {
      prow0 -= nw.part[part].rows;
      ++part;
    }
  }
  const Nf4Part P = nw.part[part];
  float offset = 0.f;
  if constexpr (NF4) {
    for (int i = tid; i < 256; i += T) {
      code2_s[i] = P.code2[i];
      pair_s[i] = float2{P.nf4[i >> 4], P.nf4[i & 15]};
    }
    offset = P.offset[0];
  }

  // Split of the contraction (partial != null): workgroup row blockIdx.y takes K tiles
  // kt_base .. kt_base + split_tiles - 1 and writes an fp32 partial of its output tile.
  const int kt_base = static_cast<int>(blockIdx.y) * split_tiles;
  const int KT = min(split_tiles, K / kBK - kt_base);
  auto load = [&](TileRegs<S>& r, int kt) {
    const int k0 = (kt_base + kt) * kBK;
#pragma unroll
    for (int j = 0; j < S::XC; ++j) {
      const int c = tid + T * j, row = c / CPR, ch = c % CPR;
      const int64_t xr = min(m0 + row, M - 1);
      r.x[j] = *reinterpret_cast<const u32x4*>(x + xr * ldx + k0 + 8 * ch);
    }
    if constexpr (!NF4) {
#pragma unroll
      for (int j = 0; j < S::WC; ++j) {
        const int c = tid + T * j, row = c / CPR, ch = c % CPR;
        r.w[j] = *reinterpret_cast<const u32x4*>(w16 + static_cast<int64_t>(n0 + row) * K + k0 +
                                                 8 * ch);
      }
    } else {
#pragma unroll
      for (int j = 0; j < S::NI; ++j) {
        const int it = min(tid + T * j, BN * IPR - 1), row = it / IPR, q = it % IPR;
        // first element of the item
        const int64_t e0 = static_cast<int64_t>(prow0 + row) * K + k0 + 16 * q;
        r.c[j] = *reinterpret_cast<const u32x2*>(P.packed + e0 / 2);
        const int64_t blk = e0 / kQBlock;
        r.ablk[j] = P.absmax_u8[blk];
        r.a2[j] = P.absmax2[blk / 256];
      }
    }
  };
  auto store = [&](const TileRegs<S>& r, _Float16* Xs, _Float16* Ws) {
#pragma unroll
    for (int j = 0; j < S::XC; ++j) {
      const int c = tid + T * j, row = c / CPR, ch = c % CPR;
      *reinterpret_cast<u32x4*>(&Xs[row * kLds + 8 * ch]) = r.x[j];
    }
    if constexpr (!NF4) {
#pragma unroll
      for (int j = 0; j < S::WC; ++j) {
        const int c = tid + T * j, row = c / CPR, ch = c % CPR;
        *reinterpret_cast<u32x4*>(&Ws[row * kLds + 8 * ch]) = r.w[j];
      }
    } else {
#pragma unroll
      for (int j = 0; j < S::NI; ++j) {
        const int it = tid + T * j;
        if (S::NI * T > BN * IPR && it >= BN * IPR) break;
        const int row = it / IPR, q = it % IPR;
        const uint32_t words[2] = {r.c[j].x, r.c[j].y};
        // All eight (nf4[hi], nf4[lo]) lookups and the scale's code2 lookup are issued before
        // any is used: left to itself the compiler issued them one at a time, each waiting for
        // its own LDS round trip.
        float2 v[8];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int b = 0; b < 4; ++b) v[h * 4 + b] = pair_s[(words[h] >> (8 * b)) & 0xffu];
        const float c2 = code2_s[r.ablk[j]];
        __builtin_amdgcn_sched_barrier(0);
        const float scale = c2 * r.a2[j] + offset;   // two roundings (no FMA)
        uint32_t out[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) out[k] = pack_h2(v[k].x * scale, v[k].y * scale);
        _Float16* dst = &Ws[row * kLds + 16 * q];
        *reinterpret_cast<u32x4*>(dst) = u32x4{out[0], out[1], out[2], out[3]};
        *reinterpret_cast<u32x4*>(dst + 8) = u32x4{out[4], out[5], out[6], out[7]};
      }
    }
  };

  f16v acc[S::FM][S::FN];
#pragma unroll
  for (int i = 0; i < S::FM; ++i)
#pragma unroll
    for (int j = 0; j < S::FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  auto compute = [&](const _Float16* Xs, const _Float16* Ws) {
    const _Float16* xa = &Xs[(S::TM * wm + (lane % 32)) * kLds + 8 * (lane / 32)];
    const _Float16* wb = &Ws[(S::TN * wn + (lane % 32)) * kLds + 8 * (lane / 32)];
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      h8 a[S::FM], b[S::FN];
#pragma unroll
      for (int i = 0; i < S::FM; ++i)
        a[i] = *reinterpret_cast<const h8*>(xa + 32 * i * kLds + 16 * ks);
#pragma unroll
      for (int j = 0; j < S::FN; ++j)
        b[j] = *reinterpret_cast<const h8*>(wb + 32 * j * kLds + 16 * ks);
#pragma unroll
      for (int i = 0; i < S::FM; ++i)
#pragma unroll
        for (int j = 0; j < S::FN; ++j) acc[i][j] = mfma32x32(a[i], b[j], acc[i][j]);
    }
  };

  // Software pipeline: at step kt the MFMAs read stage kt % 2 while the registers of tile
  // kt + 1 (loaded a step earlier) are dequantised / written into the other stage and the
  // global loads of tile kt + 2 are issued; one barrier per step.
  TileRegs<S> ra, rb;
  load(ra, 0);
  if constexpr (NF4) __syncthreads();   // code2_s / pair_s written before the first store
  store(ra, Xs0, Ws0);
  if (KT > 1) load(ra, 1);
  auto step = [&](int kt, TileRegs<S>& staged, TileRegs<S>& next, const _Float16* cx,
                  const _Float16* cw, _Float16* sx, _Float16* sw) {
    __syncthreads();
    if (kt + 2 < KT) load(next, kt + 2);
    issue_here();
    compute(cx, cw);
    if (kt + 1 < KT) store(staged, sx, sw);
  };
  // Steady state with every load and store unconditional: with the loads and stores under
  // tests inside the loop, the compiler's wait-count analysis merged the paths and waited for
  // all outstanding loads before issuing the next tile's (one tile of prefetch instead of two).
  int kt = 0;
  for (; kt + 3 < KT; kt += 2) {
    __syncthreads();
    load(rb, kt + 2);
    issue_here();
    compute(Xs0, Ws0);
    store(ra, Xs1, Ws1);
    __syncthreads();
    load(ra, kt + 3);
    issue_here();
    compute(Xs1, Ws1);
    store(rb, Xs0, Ws0);
  }
  for (; kt < KT; kt += 2) {      // the last (up to three) steps
    step(kt, ra, rb, Xs0, Ws0, Xs1, Ws1);
    if (kt + 1 < KT) step(kt + 1, rb, ra, Xs1, Ws1, Xs0, Ws0);
  }

  // epilogue: element e of acc[i][j] is row TM wm + 32i + 8(e/4) + 4(lane/32) + e%4,
  // column TN wn + 32j + lane%32
  if (partial != nullptr) {   // the split's fp32 partial, no bias
    float* pz = partial + static_cast<int64_t>(blockIdx.y) * M * N;
#pragma unroll
    for (int j = 0; j < S::FN; ++j) {
      const int n = n0 + S::TN * wn + 32 * j + lane % 32;
#pragma unroll
      for (int i = 0; i < S::FM; ++i) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m0 + S::TM * wm + 32 * i + 8 * (e / 4) + 4 * (lane / 32) + e % 4;
          if (m < M) pz[static_cast<int64_t>(m) * N + n] = acc[i][j][e];
        }
      }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < S::FN; ++j) {
    const int n = n0 + S::TN * wn + 32 * j + lane % 32;
    const float bv = bias != nullptr ? h2f(bias[n]) : 0.f;
#pragma unroll
    for (int i = 0; i < S::FM; ++i) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + S::TM * wm + 32 * i + 8 * (e / 4) + 4 * (lane / 32) + e % 4;
        if (m < M)
          y[static_cast<int64_t>(m) * N + n] =
              __builtin_bit_cast(uint16_t, static_cast<_Float16>(acc[i][j][e] + bv));
      }
    }
  }
}

// ---- the input gradient: dX = dY W with W read as NF4 --------------------------------------
// dX [M, Kw] = dY [M, Nw] W [Nw, Kw] for y = x W^T: the contraction runs over W's rows (Nw).  A
// contraction step stages 64 rows of W x BN output columns in LDS in W's own layout (row n,
// columns contiguous), dequantised as in the forward -- a thread's item is 16 consecutive
// columns of one row (8 code bytes, 8 lanes reading a row's 64 contiguous bytes; one 64-value
// block), written as two 16-byte stores -- and the MFMA B fragments (column c, 8 consecutive
// rows) are read with two ds_read_b64_tr_b16 each: in a 16-lane group, lane k reads 4 columns
// of row r0 + k/4 and receives column c0 + k of rows r0 .. r0 + 3.  (Staged transposed with
// 4-byte stores instead, the dequantised tile took 8-way LDS bank conflicts: 60.8 us against
// 34.3 us for unpack + hipBLASLt at the q|k|v shape.)  W may be up to 4 row parts (q|k|v); a
// 64-row step lies in one part, whose tables (code2, nf4 pairs) are all staged at the start.
template <class S>
struct TileRegsNN {
  static constexpr int IPR = S::BN / 16;   // 16-column items per W row of a step
  static constexpr int NI = (64 * IPR + S::kThreads - 1) / S::kThreads;
  u32x4 x[S::XC];
  u32x2 c[NI];
  uint32_t ablk[NI];
  float a2[NI];
};

typedef short s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4 lds_s4;
typedef __attribute__((address_space(3))) _Float16 lds_h;
typedef _Float16 h4 __attribute__((ext_vector_type(4)));

template <class S>
__global__ __launch_bounds__(S::kThreads) void gemm_nn_nf4_kernel(
    const uint16_t* __restrict__ dy, int64_t lddy, Nf4Weights nw, uint16_t* __restrict__ dx,
    int M, int N /* W columns: dx columns */, int K /* W rows: the contraction */,
    float* __restrict__ partial, int split_tiles) {
  constexpr int BM = S::BM, BN = S::BN, T = S::kThreads, kBK = 64, kLds = kBK + 8;
  constexpr int kLdw = BN + 8;                   // W tile row stride (halves)
  constexpr int CPR = kBK / 8;
  constexpr int IPR = TileRegsNN<S>::IPR;
  constexpr int NI = TileRegsNN<S>::NI;
  static_assert(S::BK == 64, "64-row contraction steps");
  __shared__ __align__(16) _Float16 Xs0[BM * kLds];
  __shared__ __align__(16) _Float16 Ws0[kBK * kLdw];
  __shared__ __align__(16) _Float16 Xs1[BM * kLds];
  __shared__ __align__(16) _Float16 Ws1[kBK * kLdw];
  __shared__ float code2_s[kMaxParts][256];
  __shared__ float2 pair_s[kMaxParts][256];
  const int tid = threadIdx.x;
  int nb, mb;
  tile_of(blockIdx.x, N / BN, (M + BM - 1) / BM, nb, mb);
  const int n0 = nb * BN, m0 = mb * BM;
  const int lane = tid % kWave, wv = tid / kWave;
  const int wm = wv / S::WN, wn = wv % S::WN;
  for (int p = 0; p < nw.n_parts; ++p)
    for (int i = tid; i < 256; i += T) {
      code2_s[p][i] = nw.part[p].code2[i];
      pair_s[p][i] = float2{nw.part[p].nf4[i >> 4], nw.part[p].nf4[i & 15]};
    }

  // Split of the contraction (partial != null): workgroup row blockIdx.y takes contraction
  // steps kt_base .. kt_base + split_tiles - 1 and writes an fp32 partial of its output tile.
  const int kt_base = static_cast<int>(blockIdx.y) * split_tiles;
  const int KT = min(split_tiles, K / kBK - kt_base);
  // the part holding W rows k0 .. k0 + 63, and the row of that part (wave-uniform)
  auto part_of = [&](int k0, int& prow) {
    int part = 0;
    prow = k0;
    while (part + 1 < nw.n_parts && prow >= nw.part[part].rows) {
      prow -= nw.part[part].rows;
      ++part;
    }
    return part;
  };
  auto load = [&](TileRegsNN<S>& r, int kt) {
    const int k0 = (kt_base + kt) * kBK;
#pragma unroll
    for (int j = 0; j < S::XC; ++j) {
      const int c = tid + T * j, row = c / CPR, ch = c % CPR;
      const int64_t xr = min(m0 + row, M - 1);
      r.x[j] = *reinterpret_cast<const u32x4*>(dy + xr * lddy + k0 + 8 * ch);
    }
    int prow0;
    const Nf4Part P = nw.part[part_of(k0, prow0)];
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int it = min(tid + T * j, 64 * IPR - 1), row = it / IPR, q = it % IPR;
      const int64_t e0 = static_cast<int64_t>(prow0 + row) * N + n0 + 16 * q;
      r.c[j] = *reinterpret_cast<const u32x2*>(P.packed + e0 / 2);
      const int64_t blk = e0 / kQBlock;
      r.ablk[j] = P.absmax_u8[blk];
      r.a2[j] = P.absmax2[blk / 256];
    }
  };
  auto store = [&](const TileRegsNN<S>& r, int kt, _Float16* Xs, _Float16* Ws) {
#pragma unroll
    for (int j = 0; j < S::XC; ++j) {
      const int c = tid + T * j, row = c / CPR, ch = c % CPR;
      *reinterpret_cast<u32x4*>(&Xs[row * kLds + 8 * ch]) = r.x[j];
    }
    int prow0;
    const int part = part_of((kt_base + kt) * kBK, prow0);
    const float offset = nw.part[part].offset[0];
#pragma unroll
    for (int j = 0; j < NI; ++j) {
      const int it = tid + T * j;
      if (NI * T > 64 * IPR && it >= 64 * IPR) break;
      const int row = it / IPR, q = it % IPR;
      const uint32_t words[2] = {r.c[j].x, r.c[j].y};
      float2 v[8];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int b = 0; b < 4; ++b) v[h * 4 + b] = pair_s[part][(words[h] >> (8 * b)) & 0xffu];
      const float c2 = code2_s[part][r.ablk[j]];
      __builtin_amdgcn_sched_barrier(0);
      const float scale = c2 * r.a2[j] + offset;   // two roundings (no FMA)
      uint32_t out[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) out[k] = pack_h2(v[k].x * scale, v[k].y * scale);
      _Float16* dst = &Ws[row * kLdw + 16 * q];
      *reinterpret_cast<u32x4*>(dst) = u32x4{out[0], out[1], out[2], out[3]};
      *reinterpret_cast<u32x4*>(dst + 8) = u32x4{out[4], out[5], out[6], out[7]};
    }
  };

  f16v acc[S::FM][S::FN];
#pragma unroll
  for (int i = 0; i < S::FM; ++i)
#pragma unroll
    for (int j = 0; j < S::FN; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
  // B fragment of output columns c0 + lane%32 at contraction rows 16ks + 8(lane/32) .. +7
  const int gk = lane & 15, grp = lane >> 4;
  auto compute = [&](const _Float16* Xs, const _Float16* Ws) {
    const _Float16* xa = &Xs[(S::TM * wm + (lane % 32)) * kLds + 8 * (lane / 32)];
    const lds_h* wbase = (const lds_h*)(Ws);
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      h8 a[S::FM], b[S::FN];
#pragma unroll
      for (int i = 0; i < S::FM; ++i)
        a[i] = *reinterpret_cast<const h8*>(xa + 32 * i * kLds + 16 * ks);
#pragma unroll
      for (int j = 0; j < S::FN; ++j) {
        const int row = 16 * ks + 8 * (grp >> 1) + (gk >> 2);
        const int col = S::TN * wn + 32 * j + 16 * (grp & 1) + 4 * (gk & 3);
        const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s4*)(wbase + row * kLdw + col));
        const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_s4*)(wbase + (row + 4) * kLdw + col));
        b[j] = __builtin_shufflevector(__builtin_bit_cast(h4, lo), __builtin_bit_cast(h4, hi),
                                       0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int i = 0; i < S::FM; ++i)
#pragma unroll
        for (int j = 0; j < S::FN; ++j) acc[i][j] = mfma32x32(a[i], b[j], acc[i][j]);
    }
  };
  TileRegsNN<S> ra, rb;
  load(ra, 0);
  __syncthreads();   // the tables written before the first store
  store(ra, 0, Xs0, Ws0);
  if (KT > 1) load(ra, 1);
  auto step = [&](int kt, TileRegsNN<S>& staged, TileRegsNN<S>& next, const _Float16* cx,
                  const _Float16* cw, _Float16* sx, _Float16* sw) {
    __syncthreads();
    if (kt + 2 < KT) load(next, kt + 2);
    issue_here();
    compute(cx, cw);
    if (kt + 1 < KT) store(staged, kt + 1, sx, sw);
  };
  int kt = 0;
  for (; kt + 3 < KT; kt += 2) {   // steady state: every load and store unconditional
    __syncthreads();
    load(rb, kt + 2);
    issue_here();
    compute(Xs0, Ws0);
    store(ra, kt + 1, Xs1, Ws1);
    __syncthreads();
    load(ra, kt + 3);
    issue_here();
    compute(Xs1, Ws1);
    store(rb, kt + 2, Xs0, Ws0);
  }
  for (; kt < KT; kt += 2) {
    step(kt, ra, rb, Xs0, Ws0, Xs1, Ws1);
    if (kt + 1 < KT) step(kt + 1, rb, ra, Xs1, Ws1, Xs0, Ws0);
  }
  if (partial != nullptr) {   // the split's fp32 partial
    float* pz = partial + static_cast<int64_t>(blockIdx.y) * M * N;
#pragma unroll
    for (int j = 0; j < S::FN; ++j) {
      const int n = n0 + S::TN * wn + 32 * j + lane % 32;
#pragma unroll
      for (int i = 0; i < S::FM; ++i) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m0 + S::TM * wm + 32 * i + 8 * (e / 4) + 4 * (lane / 32) + e % 4;
          if (m < M) pz[static_cast<int64_t>(m) * N + n] = acc[i][j][e];
        }
      }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < S::FN; ++j) {
    const int n = n0 + S::TN * wn + 32 * j + lane % 32;
#pragma unroll
    for (int i = 0; i < S::FM; ++i) {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int m = m0 + S::TM * wm + 32 * i + 8 * (e / 4) + 4 * (lane / 32) + e % 4;
        if (m < M)
          dx[static_cast<int64_t>(m) * N + n] =
              __builtin_bit_cast(uint16_t, static_cast<_Float16>(acc[i][j][e]));
      }
    }
  }
}

// The tile shape of both entry points (SOUPK_GEMM_SHAPE selects another for measurement):
//   0: 128 x 128, 2 x 2 waves of 64 x 64      1: 128 x 128, 4 x 2 waves of 32 x 64
//   2: 128 x 128, 2 x 4 waves of 64 x 32      3: 128 x 64, 2 x 2 waves of 64 x 32
//   4: 64 x 128, 2 x 2 waves of 32 x 64       5: 256 x 128, 4 x 2 waves of 64 x 64
//   6: as 1 with K tiles of 128               7: 256 x 256, 2 x 4 waves of 128 x 64
//   8: 256 x 256, 4 x 2 waves of 64 x 128     9: 256 x 128, 2 x 2 waves of 128 x 64
//  10: 32 x 128, 1 x 4 waves of 32 x 32
#ifndef SOUPK_GEMM_SHAPE
#define SOUPK_GEMM_SHAPE 1
#endif
#if SOUPK_GEMM_SHAPE == 0
using Shape = GemmShape<128, 128, 2, 2>;
#elif SOUPK_GEMM_SHAPE == 1
using Shape = GemmShape<128, 128, 4, 2>;
#elif SOUPK_GEMM_SHAPE == 2
using Shape = GemmShape<128, 128, 2, 4>;
#elif SOUPK_GEMM_SHAPE == 3
using Shape = GemmShape<128, 64, 2, 2>;
#elif SOUPK_GEMM_SHAPE == 4
using Shape = GemmShape<64, 128, 2, 2>;
#elif SOUPK_GEMM_SHAPE == 5
using Shape = GemmShape<256, 128, 4, 2>;
#elif SOUPK_GEMM_SHAPE == 7
using Shape = GemmShape<256, 256, 2, 4>;
#elif SOUPK_GEMM_SHAPE == 8
using Shape = GemmShape<256, 256, 4, 2>;
#elif SOUPK_GEMM_SHAPE == 9
using Shape = GemmShape<256, 128, 2, 2>;
#elif SOUPK_GEMM_SHAPE == 10
using Shape = GemmShape<32, 128, 1, 4>;
#else
using Shape = GemmShape<128, 128, 4, 2, 128>;
#endif
constexpr int kBK = Shape::BK;
constexpr int kBM = Shape::BM, kBN = Shape::BN;
// Up to 32 rows of x the forward runs 32-row tiles on 4 wavefronts of 32 x 32: the 128-row
// tile computed three quarters clamped copies of the last row there.  Measured (MI355X, NF4 W,
// the split counts split_count picks): at 16 rows q|k|v 8.02 -> 7.55 us, o 7.63 -> 7.18,
// gate|up 23.58 -> 18.38, down 12.77 -> 11.07; slower from 64 rows (gate|up 24.07 -> 26.25).
// Same products in the same order: identical results.
using SmallShape = GemmShape<32, 128, 1, 4>;
constexpr int kSmallRows = 32;
static_assert(SmallShape::BN == kBN && SmallShape::BK == kBK, "one column tiling for both");

int check_gemm(int64_t M, int32_t N, int32_t K, int64_t ldx) {
  if (M < 0 || N <= 0 || K <= 0 || N % kBN || K % kBK || ldx < K || ldx % 8) return kInvalid;
  if ((M + kBM - 1) / kBM * static_cast<int64_t>(N / kBN) > 0x7fffffff) return kInvalid;
  if (M * static_cast<int64_t>(N) >= (int64_t{1} << 40)) return kInvalid;
  return kOk;
}

bool bad_ptr(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15); }

// The NF4 parts of W (up to kMaxParts stacked by rows, each a multiple of 128 rows), checked.
int nf4_parts(int32_t n_parts, const uint8_t* const* packed, const uint8_t* const* absmax_u8,
              const float* const* code2, const float* const* absmax2,
              const float* const* offset, const float* const* nf4, const int32_t* part_rows,
              int32_t qblock, int32_t qblock2, int64_t total_rows, Nf4Weights& nw) {
  if (qblock != kQBlock || qblock2 != 256) return kInvalid;
  if (n_parts < 1 || n_parts > kMaxParts || !packed || !absmax_u8 || !code2 || !absmax2 ||
      !offset || !nf4 || !part_rows)
    return kInvalid;
  nw = Nf4Weights{};
  int64_t rows = 0;
  for (int i = 0; i < n_parts; ++i) {
    if (part_rows[i] <= 0 || part_rows[i] % 128 || bad_ptr(packed[i]) || !absmax_u8[i] ||
        !code2[i] || !absmax2[i] || !offset[i] || !nf4[i])
      return kInvalid;
    nw.part[i] = Nf4Part{packed[i], absmax_u8[i], code2[i], absmax2[i], offset[i], nf4[i],
                         part_rows[i]};
    rows += part_rows[i];
  }
  nw.n_parts = n_parts;
  return rows == total_rows ? kOk : kInvalid;
}

}  // namespace
}  // namespace soupk

namespace soupk {
namespace {

constexpr int kMaxSplits = 32;

// y = fp16(((p[0] + p[1]) + ...) + bias) over the splits' fp32 partials [splits, M, N], four
// consecutive outputs per thread (N is a multiple of 64), partials added in split order.  All
// of a thread's loads are issued before the first add (unrolled to kMaxSplits under a uniform
// test), so the kernel waits on memory once, not once per split.
__global__ __launch_bounds__(256) void split_sum_kernel(
    const f32x4* __restrict__ parts, int splits, int64_t stride4, int64_t n4, int n_cols4,
    const uint16_t* __restrict__ bias, u32x2* __restrict__ y) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n4) return;
  f32x4 v[kMaxSplits];
#pragma unroll
  for (int p = 0; p < kMaxSplits; ++p)
    if (p < splits) v[p] = parts[p * stride4 + i];
  f32x4 s = v[0];
#pragma unroll
  for (int p = 1; p < kMaxSplits; ++p)
    if (p < splits) s = s + v[p];
  if (bias != nullptr) {
    const int c = static_cast<int>(i % n_cols4) * 4;
    const u32x2 bw = *reinterpret_cast<const u32x2*>(bias + c);
    s = s + f32x4{lo_h(bw.x), hi_h(bw.x), lo_h(bw.y), hi_h(bw.y)};
  }
  y[i] = u32x2{pack_h2(s[0], s[1]), pack_h2(s[2], s[3])};
}

// Contraction steps per split and the splits that leaves non-empty, for `kt` 64-wide steps cut
// `splits` ways (kInvalid unless 1 <= splits <= min(kMaxSplits, kt)).
int split_plan(int kt, int32_t splits, int& per, int& used) {
  if (splits < 1 || splits > kMaxSplits || splits > kt) return kInvalid;
  per = (kt + splits - 1) / splits;
  used = (kt + per - 1) / per;
  return kOk;
}

}  // namespace
}  // namespace soupk

using namespace soupk;

extern "C" __attribute__((visibility("default"))) int soupk_gemm_tn(
    const uint16_t* x, int64_t ldx, const uint16_t* w, const uint16_t* bias, uint16_t* y,
    int64_t M, int32_t N, int32_t K, void* stream) {
  const int rc = check_gemm(M, N, K, ldx);
  if (rc != kOk) return rc;
  if (M == 0) return kOk;
  if (bad_ptr(x) || bad_ptr(w) || bad_ptr(y)) return kInvalid;
  Nf4Weights none{};
  if (M <= kSmallRows)
    return launch_kernel(gemm_tn_kernel<SmallShape, false>,
                         dim3(static_cast<unsigned>(N / kBN)), dim3(SmallShape::kThreads),
                         static_cast<hipStream_t>(stream), x, ldx, w, none, bias, y,
                         static_cast<int>(M), N, K, nullptr, K / kBK);
  const dim3 grid(static_cast<unsigned>((N / kBN) * ((M + kBM - 1) / kBM)));
  return launch_kernel(gemm_tn_kernel<Shape, false>, grid, dim3(Shape::kThreads),
                       static_cast<hipStream_t>(stream), x, ldx, w, none, bias, y,
                       static_cast<int>(M), N, K, nullptr, K / kBK);
}

extern "C" __attribute__((visibility("default"))) int soupk_gemm_tn_nf4(
    const uint16_t* x, int64_t ldx, int32_t n_parts, const uint8_t* const* packed,
    const uint8_t* const* absmax_u8, const float* const* code2, const float* const* absmax2,
    const float* const* offset, const float* const* nf4, const int32_t* part_rows,
    int32_t qblock, int32_t qblock2, const uint16_t* bias, uint16_t* y, int64_t M, int32_t N,
    int32_t K, void* stream) {
  const int rc = check_gemm(M, N, K, ldx);
  if (rc != kOk) return rc;
  Nf4Weights nw;
  const int rp = nf4_parts(n_parts, packed, absmax_u8, code2, absmax2, offset, nf4, part_rows,
                           qblock, qblock2, N, nw);
  if (rp != kOk) return rp;
  for (int i = 0; i < n_parts; ++i)
    if (part_rows[i] % kBN) return kInvalid;
  if (M == 0) return kOk;
  if (bad_ptr(x) || bad_ptr(y)) return kInvalid;
  if (M <= kSmallRows)
    return launch_kernel(gemm_tn_kernel<SmallShape, true>,
                         dim3(static_cast<unsigned>(N / kBN)), dim3(SmallShape::kThreads),
                         static_cast<hipStream_t>(stream), x, ldx, nullptr, nw, bias, y,
                         static_cast<int>(M), N, K, nullptr, K / kBK);
  const dim3 grid(static_cast<unsigned>((N / kBN) * ((M + kBM - 1) / kBM)));
  return launch_kernel(gemm_tn_kernel<Shape, true>, grid, dim3(Shape::kThreads),
                       static_cast<hipStream_t>(stream), x, ldx, nullptr, nw, bias, y,
                       static_cast<int>(M), N, K, nullptr, K / kBK);
}

extern "C" __attribute__((visibility("default"))) int soupk_gemm_tn_nf4_split(
    const uint16_t* x, int64_t ldx, int32_t n_parts, const uint8_t* const* packed,
    const uint8_t* const* absmax_u8, const float* const* code2, const float* const* absmax2,
    const float* const* offset, const float* const* nf4, const int32_t* part_rows,
    int32_t qblock, int32_t qblock2, const uint16_t* bias, uint16_t* y, int64_t M, int32_t N,
    int32_t K, int32_t splits, float* workspace, int64_t workspace_floats, void* stream) {
  const int rc = check_gemm(M, N, K, ldx);
  if (rc != kOk) return rc;
  Nf4Weights nw;
  const int rp = nf4_parts(n_parts, packed, absmax_u8, code2, absmax2, offset, nf4, part_rows,
                           qblock, qblock2, N, nw);
  if (rp != kOk) return rp;
  for (int i = 0; i < n_parts; ++i)
    if (part_rows[i] % kBN) return kInvalid;
  int per, used;
  if (split_plan(K / kBK, splits, per, used) != kOk) return kInvalid;
  if (workspace_floats < static_cast<int64_t>(used) * M * N) return kInvalid;
  if (M == 0) return kOk;
  if (bad_ptr(x) || bad_ptr(y) || bad_ptr(workspace)) return kInvalid;
  if (reinterpret_cast<uintptr_t>(bias) & 7) return kInvalid;   // read 4 halves at a time
  hipStream_t st = static_cast<hipStream_t>(stream);
  int r;
  if (M <= kSmallRows)
    r = launch_kernel(gemm_tn_kernel<SmallShape, true>,
                      dim3(static_cast<unsigned>(N / kBN), static_cast<unsigned>(used)),
                      dim3(SmallShape::kThreads), st, x, ldx, nullptr, nw, bias, y,
                      static_cast<int>(M), N, K, workspace, per);
  else
    r = launch_kernel(gemm_tn_kernel<Shape, true>,
                      dim3(static_cast<unsigned>((N / kBN) * ((M + kBM - 1) / kBM)),
                           static_cast<unsigned>(used)),
                      dim3(Shape::kThreads), st, x, ldx, nullptr, nw, bias, y,
                      static_cast<int>(M), N, K, workspace, per);
  if (r != kOk) return r;
  const int64_t n4 = M * static_cast<int64_t>(N) / 4;
  return launch_kernel(split_sum_kernel, dim3(static_cast<unsigned>((n4 + 255) / 256)),
                       dim3(256), st, reinterpret_cast<const f32x4*>(workspace), used,
                       M * static_cast<int64_t>(N) / 4, n4, N / 4, bias,
                       reinterpret_cast<u32x2*>(y));
}

namespace {
// Tile shape of the input gradient (measured at M = 2048 on MI355X: 128 x 64 on 4 wavefronts
// 40.9 / 28.8 us at the q|k|v / o shapes; 128 x 128 on 8, 44.9 / 32.2 us, fills only 192 of the
// 256 CUs there; 64 x 128, 54.1 / 39.6 us).
#ifndef SOUPK_GEMM_NN_SHAPE
#define SOUPK_GEMM_NN_SHAPE 1
#endif
#if SOUPK_GEMM_NN_SHAPE == 0
using NS = GemmShape<128, 128, 4, 2>;
#elif SOUPK_GEMM_NN_SHAPE == 1
using NS = GemmShape<128, 64, 2, 2>;
#elif SOUPK_GEMM_NN_SHAPE == 2
using NS = GemmShape<64, 128, 2, 2>;
#else
using NS = GemmShape<128, 64, 4, 2>;
#endif
// The split form up to 32 rows of dy: 32-row tiles on 2 wavefronts of 32 x 32 (the column
// tiling unchanged).  Measured (MI355X, the split counts split_count picks): at 16 rows q|k|v
// 9.71 -> 9.13 us, o 8.34 -> 7.68, gate|up 23.46 -> 20.70; the unsplit kernel (down's input
// gradient, 140 tiles walking the whole contraction) was 3% slower on 2 wavefronts and keeps
// NS.  Same products in the same order: identical results.
#ifndef SOUPK_GEMM_NN_SMALL
#define SOUPK_GEMM_NN_SMALL 1
#endif
using NSmall = GemmShape<32, 64, 1, 2>;
static_assert(NSmall::BN == NS::BN, "one column tiling for both");
constexpr int kNnSmallRows = SOUPK_GEMM_NN_SMALL ? 32 : 0;

// The input gradient's arguments, checked; N: W's columns (dx's), K: W's rows (the
// contraction, dy's columns).
int check_nn(const uint16_t* dy, int64_t lddy, int32_t n_parts, const uint8_t* const* packed,
             const uint8_t* const* absmax_u8, const float* const* code2,
             const float* const* absmax2, const float* const* offset, const float* const* nf4,
             const int32_t* part_rows, int32_t qblock, int32_t qblock2, int64_t M, int32_t N,
             int32_t K, Nf4Weights& nw) {
  if (M < 0 || N <= 0 || K <= 0 || N % NS::BN || K % 64 || lddy < K || lddy % 8) return kInvalid;
  if ((M + NS::BM - 1) / NS::BM * static_cast<int64_t>(N / NS::BN) > 0x7fffffff) return kInvalid;
  if (M * static_cast<int64_t>(N) >= (int64_t{1} << 40)) return kInvalid;
  return nf4_parts(n_parts, packed, absmax_u8, code2, absmax2, offset, nf4, part_rows, qblock,
                   qblock2, K, nw);
}
}  // namespace

extern "C" __attribute__((visibility("default"))) int soupk_gemm_nn_nf4(
    const uint16_t* dy, int64_t lddy, int32_t n_parts, const uint8_t* const* packed,
    const uint8_t* const* absmax_u8, const float* const* code2, const float* const* absmax2,
    const float* const* offset, const float* const* nf4, const int32_t* part_rows,
    int32_t qblock, int32_t qblock2, uint16_t* dx, int64_t M, int32_t N, int32_t K,
    void* stream) {
  Nf4Weights nw;
  const int rc = check_nn(dy, lddy, n_parts, packed, absmax_u8, code2, absmax2, offset, nf4,
                          part_rows, qblock, qblock2, M, N, K, nw);
  if (rc != kOk) return rc;
  if (M == 0) return kOk;
  if (bad_ptr(dy) || bad_ptr(dx)) return kInvalid;
  const dim3 grid(static_cast<unsigned>((N / NS::BN) * ((M + NS::BM - 1) / NS::BM)));
  return launch_kernel(gemm_nn_nf4_kernel<NS>, grid, dim3(NS::kThreads),
                       static_cast<hipStream_t>(stream), dy, lddy, nw, dx, static_cast<int>(M),
                       N, K, nullptr, K / 64);
}

extern "C" __attribute__((visibility("default"))) int soupk_gemm_nn_nf4_split(
    const uint16_t* dy, int64_t lddy, int32_t n_parts, const uint8_t* const* packed,
    const uint8_t* const* absmax_u8, const float* const* code2, const float* const* absmax2,
    const float* const* offset, const float* const* nf4, const int32_t* part_rows,
    int32_t qblock, int32_t qblock2, uint16_t* dx, int64_t M, int32_t N, int32_t K,
    int32_t splits, float* workspace, int64_t workspace_floats, void* stream) {
  Nf4Weights nw;
  const int rc = check_nn(dy, lddy, n_parts, packed, absmax_u8, code2, absmax2, offset, nf4,
                          part_rows, qblock, qblock2, M, N, K, nw);
  if (rc != kOk) return rc;
  int per, used;
  if (split_plan(K / 64, splits, per, used) != kOk) return kInvalid;
  if (workspace_floats < static_cast<int64_t>(used) * M * N) return kInvalid;
  if (M == 0) return kOk;
  if (bad_ptr(dy) || bad_ptr(dx) || bad_ptr(workspace)) return kInvalid;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int r;
  if (M <= kNnSmallRows)
    r = launch_kernel(gemm_nn_nf4_kernel<NSmall>,
                      dim3(static_cast<unsigned>(N / NS::BN), static_cast<unsigned>(used)),
                      dim3(NSmall::kThreads), st, dy, lddy, nw, dx, static_cast<int>(M), N, K,
                      workspace, per);
  else
    r = launch_kernel(gemm_nn_nf4_kernel<NS>,
                      dim3(static_cast<unsigned>((N / NS::BN) * ((M + NS::BM - 1) / NS::BM)),
                           static_cast<unsigned>(used)),
                      dim3(NS::kThreads), st, dy, lddy, nw, dx, static_cast<int>(M), N, K,
                      workspace, per);
  if (r != kOk) return r;
  const int64_t n4 = M * static_cast<int64_t>(N) / 4;
  return launch_kernel(split_sum_kernel, dim3(static_cast<unsigned>((n4 + 255) / 256)),
                       dim3(256), st, reinterpret_cast<const f32x4*>(workspace), used, n4, n4,
                       N / 4, nullptr, reinterpret_cast<u32x2*>(dx));
}
