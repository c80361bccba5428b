// The LoRA branch of the q and v projections (peft's lora_B(lora_A(x)) * scaling under fp16
// autocast, solution/model.py:195-206 with dropout 0), for rank 16, in two launches per
// direction instead of a dozen small GEMMs, casts and scalings:
//
//   soupk_lora_fwd:       t  = fp16(y A^T)                        [M, 2r]  (A = A_q | A_v)
//                         lq = fp16(fp16(t_q B_q^T) * scaling)    [M, NQ]
//                         lv = fp16(fp16(t_v B_v^T) * scaling)    [M, NV]
//   soupk_lora_bwd_rows:  gs_x = fp16(g_x * scaling)              (g_x: the gradients of lq, lv;
//                                                                 in registers, not stored)
//                         dt   = fp16(gs_q B_q | gs_v B_v)        [M, 2r]
//                         dy   = fp16(dt A16)                     [M, H]
// with fp16(.) the rounding of an fp16 GEMM (fp32 sums, one rounding) and A16, B16 the fp16
// casts of the fp32 LoRA parameters, rounded as .to(torch.float16) rounds them.  The casts are
// made once per forward by soupk_lora_stage, into one buffer that holds each in the layouts the
// kernels read with 8- and 16-byte loads:
//   A16  [2r, H]   (A_q rows, then A_v rows)   t's contraction over H
//   A16T [H, 2r]                               dy's contraction over the ranks
//   B16  [NQ + NV, r]                          lq / lv's contraction over the ranks
//   B16T [r, NQ], then [r, NV]                 dt's contraction over NQ / NV
// (with the fp32 parameters read and cast in the kernels themselves, every workgroup of the
// forward reads 196 KB of A: the forward took 13.3 us at 2048 rows against 10.0 us with the
// staged fp16 A, identical bits; the row backward takes 11.1 us either way, and the staging
// launch 2.2 us).  The caller then adds the frozen projection's input gradient into dy in
// place and forms the parameter gradients (B_x: gs_x^T t_x, A: dt^T y) from g, t and dt: the
// parameter kernel forms gs from g again as it stages g's rows, so gs never goes to memory (its
// stores took 2.1 of the row kernel's 11.2 us at 2048 rows).
//
// A workgroup is 4 wavefronts and kRowTiles 16-row MFMA tiles (which share every A / B fragment a
// wavefront loads), and the workgroups of a row block split the wide output (lq|lv, or dy) by
// 16-column tiles (grid.y parts), each recomputing the block's rank-2r product (the rank-2r
// product, t or dt, and gs are written by part 0).  Measured on MI355X at 2048 rows: one row tile
// and about 256 workgroups (two column parts) is fastest (13.3 / 11.2 us against 16.4 / 13.8 us
// with one part; four row tiles, or more parts, are slower).  The long contractions (over H for t,
// over NQ / NV for dt) run on v_mfma_f32_16x16x32_f16 with the contraction split over the 4
// wavefronts and the partial sums added in wavefront order (deterministic).  The short ones (over r
// for lq/lv, on v_mfma_f32_16x16x16f16; over 2r for dy, on 16x16x32) are computed transposed, one
// 16-column tile at a time: (out tile)^T = W16 x^T, so that a lane's four results are four
// consecutive columns of one row (one 8-byte store).  MFMA layouts: A lane l holds row l%16, B lane
// l column l%16, each with k = 8(l/16)..+7 (16x16x32) or 4(l/16)..+3 (16x16x16); C lane l holds
// column l%16, rows 4(l/16)..+3.

#include <algorithm>
#include <mutex>

#include "fastdiv.hpp"
#include "lora_stage.hpp"
#include "soupk_common.hpp"

namespace soupk {
namespace {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kR = kLoraRank;    // LoRA rank
#ifndef SOUPK_LORA_ROW_TILES
#define SOUPK_LORA_ROW_TILES 1
#endif
constexpr int kRowTiles = SOUPK_LORA_ROW_TILES;   // 16-row MFMA tiles per workgroup
constexpr int kRows = 16 * kRowTiles;              // rows per workgroup
constexpr int kThreads = 256;

__device__ __forceinline__ f4 mfma32(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float r16(float x) {
  return static_cast<float>(static_cast<_Float16>(x));
}

__device__ __forceinline__ uint16_t h_bits(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }

// Loop steps and tiles are processed kBatch at a time: the loads of a batch (at clamped
// indices, so unconditional) are all issued before its first MFMA, and the MFMAs and stores
// past the end of the range are skipped (a wavefront-uniform test).  One step at a time, each
// MFMA waited for its own loads; batches of 6 measured the same as 4 on MI355X at the step
// shape, and of 8 slower (forward 16.9 against 15.3 us); 12 spills.
#ifndef SOUPK_LORA_BATCH
#define SOUPK_LORA_BATCH 4
#endif
constexpr int kBatch = SOUPK_LORA_BATCH;

// Split of the output tiles over the workgroups of one row block (grid.y column parts): each
// part recomputes the row block's rank-r product (cheap: 2r columns) and writes its share of
// the wide output, so that a small M still fills the GPU.
__device__ __forceinline__ int tile_part(int n_tiles, int part, int parts) {
  return static_cast<int>((static_cast<int64_t>(n_tiles) * part) / parts);
}

// A compiler-only barrier (no instruction): the prefetch loads issued above it stay above it
// instead of being moved down to their first use.
__device__ __forceinline__ void issue_here() { __asm__ volatile("" ::: "memory"); }

// One thread per parameter value: the fp16 cast written in both layouts of its section.
__global__ __launch_bounds__(256) void lora_stage_kernel(LoraStageArgs a) {
  lora_stage_value(a, static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x);
}

// The parameter and activation pointers of the row kernels are not __restrict__: loads through
// restrict pointers are taken as invariant and moved to their use, which would undo the
// prefetch of the next batch.
// The fused LoRA + RoPE form of the forward (ROPE = true): instead of lq and lv it writes the
// rows the varlen attention reads, out = [rotated q + lq | rotated k | v + lv] in the q|k|v
// GEMM's own layout [M, NQ + NK + NV] (head dim 128), with the arithmetic of
// soupk_rope_pack_tokens: x = fp32(qkv) + fp32(fp16 LoRA delta), then
// (x1*c1 - x2*s1, x2*c2 + x1*s2) with each product rounded, then fp16.  The LoRA tiles of a
// head's dims d..d+15 and d+64..d+79 (the rotation partners) are tiles j and j + 4 of the head's
// eight, which the same wavefront computes as items u and u + 1 of a batch (a wavefront takes
// every fourth tile, and the column parts split the tiles at whole heads), so a lane holds
// both partners of its four dims.  The k columns are extra tiles with no LoRA product.
struct LoraRope {
  const uint16_t* qkv;   // [M, W] q|k|v GEMM output, W = NQ + NK + NV
  uint16_t* out;         // [M, W]
  const float* cos_t;    // [T, 128]
  const float* sin_t;    // [T, 128]
  const int64_t* pos;    // [M] padded position of each row, b * T + t
  int NK;                // key columns (NKV * 128): rotation only
  int T;
  int64_t slots;         // B * T (< 2^31)
  FastDiv per_seq;       // divides by T
};

template <bool ROPE>
__global__ __launch_bounds__(kThreads) void lora_fwd_kernel(
    const uint16_t* y, const _Float16* staged, float scaling, uint16_t* __restrict__ t_out,
    uint16_t* __restrict__ lq, uint16_t* __restrict__ lv, int M, int H, int NQ, int NV,
    LoraRope ra) {
  const StagedLayout L = staged_layout(H, NQ, NV);
  const _Float16* a16 = staged + L.a16;
  const _Float16* b16 = staged + L.b16;
  __shared__ float part[4][kRows][2 * kR + 1];
  __shared__ float tt[kRows][2 * kR];
  const int m0 = blockIdx.x * kRows;
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int ql = lane & 15, gr = lane >> 4;
  // Output tiles of this wavefront (phase 2): their B16 fragments do not depend on t, so the
  // first batch is loaded now and arrives while t is computed.
  const int nq16 = NQ / 16;
  const int nlora = NQ / 16 + NV / 16;
  int t_begin, n16;
  if constexpr (ROPE) {   // whole heads (8 tiles) per column part
    const int heads = (nlora + ra.NK / 16) / 8;
    t_begin = 8 * tile_part(heads, blockIdx.y, gridDim.y);
    n16 = 8 * tile_part(heads, blockIdx.y + 1, gridDim.y);
  } else {
    t_begin = tile_part(nlora, blockIdx.y, gridDim.y);
    n16 = tile_part(nlora, blockIdx.y + 1, gridDim.y);
  }
  const int W = NQ + ra.NK + NV;
  // (ROPE) the output column of tile `tile`: q tiles, then v tiles, then k tiles
  auto tile_col = [&](int tile) {
    return tile < nq16 ? 16 * tile
                       : (tile < nlora ? NQ + ra.NK + 16 * (tile - nq16) : NQ + 16 * (tile - nlora));
  };
  typedef uint32_t u32x2v __attribute__((ext_vector_type(2)));
  auto load_b = [&](h4* bw, u32x2v (*xq)[kRowTiles], int t0) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      // B16 row of output tile column ql (the v rows follow the q rows)
      const int tile = min(t0 + 4 * u, max(n16 - 1, 0));
      const int bt = ROPE ? min(tile, nlora - 1) : tile;
      bw[u] = *reinterpret_cast<const h4*>(b16 + static_cast<int64_t>(16 * bt + ql) * kR +
                                           4 * gr);
      if constexpr (ROPE) {   // this lane's four columns of the GEMM output
#pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt) {
          const int64_t m = min(m0 + 16 * rt + ql, M - 1);
          xq[u][rt] = *reinterpret_cast<const u32x2v*>(ra.qkv + m * W + tile_col(tile) + 4 * gr);
        }
      }
    }
  };
  h4 bw_next[kBatch];
  u32x2v xq_next[kBatch][kRowTiles];
  if (t_begin + w < n16) load_b(bw_next, xq_next, t_begin + w);
  // t = y A^T: A operand = y rows (row 16rt + ql of row tile rt, k = k0 + 8gr..+7); B operand =
  // A_q / A_v rows (column = feature ql), loaded once per step for the kRowTiles row tiles.
  // The contraction over H is split over the 4 wavefronts; batches of kBatch steps, the next
  // batch's loads issued before the current batch's MFMAs.
  const int kw = H / 4;
  const uint16_t* yrow[kRowTiles];
  f4 acc_q[kRowTiles], acc_v[kRowTiles];
#pragma unroll
  for (int rt = 0; rt < kRowTiles; ++rt) {
    yrow[rt] = y + static_cast<int64_t>(min(m0 + 16 * rt + ql, M - 1)) * H;
    acc_q[rt] = f4{0.f, 0.f, 0.f, 0.f};
    acc_v[rt] = f4{0.f, 0.f, 0.f, 0.f};
  }
  const int steps = kw / 32;
  const _Float16* aqrow = a16 + static_cast<int64_t>(ql) * H + 8 * gr;
  const _Float16* avrow = a16 + static_cast<int64_t>(kR + ql) * H + 8 * gr;
  struct Batch {
    h8 ya[kBatch][kRowTiles];
    h8 qa[kBatch], va[kBatch];
  };
  auto load_t = [&](Batch& r, int s0) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int k0 = w * kw + 32 * min(s0 + u, steps - 1);
#pragma unroll
      for (int rt = 0; rt < kRowTiles; ++rt)
        r.ya[u][rt] = *reinterpret_cast<const h8*>(yrow[rt] + k0 + 8 * gr);
      r.qa[u] = *reinterpret_cast<const h8*>(aqrow + k0);
      r.va[u] = *reinterpret_cast<const h8*>(avrow + k0);
    }
  };
  auto mma_t = [&](const Batch& r, int s0) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (s0 + u < steps) {
        const h8 bq8 = r.qa[u], bv8 = r.va[u];
#pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt) {
          acc_q[rt] = mfma32(r.ya[u][rt], bq8, acc_q[rt]);
          acc_v[rt] = mfma32(r.ya[u][rt], bv8, acc_v[rt]);
        }
      }
    }
  };
  {
    Batch r0, r1;
    load_t(r0, 0);
    for (int s0 = 0; s0 < steps; s0 += 2 * kBatch) {
      if (s0 + kBatch < steps) load_t(r1, s0 + kBatch);
      issue_here();
      mma_t(r0, s0);
      if (s0 + kBatch < steps) {
        if (s0 + 2 * kBatch < steps) load_t(r0, s0 + 2 * kBatch);
        issue_here();
        mma_t(r1, s0 + kBatch);
      }
    }
  }
  // C: column = feature ql, rows 16rt + 4gr .. +3
#pragma unroll
  for (int rt = 0; rt < kRowTiles; ++rt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      part[w][16 * rt + 4 * gr + i][ql] = acc_q[rt][i];
      part[w][16 * rt + 4 * gr + i][kR + ql] = acc_v[rt][i];
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < kRows * 2 * kR; e += kThreads) {
    const int m = e / (2 * kR), f = e % (2 * kR);
    const float s = ((part[0][m][f] + part[1][m][f]) + part[2][m][f]) + part[3][m][f];
    const _Float16 h = static_cast<_Float16>(s);
    tt[m][f] = static_cast<float>(h);
    if (blockIdx.y == 0 && m0 + m < M)
      t_out[static_cast<int64_t>(m0 + m) * (2 * kR) + f] = h_bits(h);
  }
  __syncthreads();
  // lq, lv: tile f0..f0+15 of the output columns, transposed: A = B16 rows (feature f0 + ql,
  // k = rank 4gr..+3), B = t rows (column = row ql of a row tile, same k).  Column part
  // blockIdx.y of gridDim.y takes tiles [t_begin, t_end) of the NQ/16 + NV/16; each batch's
  // B16 fragments were loaded a batch ahead (the first before the t phase).
  h4 tq4[kRowTiles], tv4[kRowTiles];
  bool row_ok[kRowTiles];
#pragma unroll
  for (int rt = 0; rt < kRowTiles; ++rt) {
    const float* tq = &tt[16 * rt + ql][4 * gr];
    const float* tv = &tt[16 * rt + ql][kR + 4 * gr];
    tq4[rt] = h4{static_cast<_Float16>(tq[0]), static_cast<_Float16>(tq[1]),
                 static_cast<_Float16>(tq[2]), static_cast<_Float16>(tq[3])};
    tv4[rt] = h4{static_cast<_Float16>(tv[0]), static_cast<_Float16>(tv[1]),
                 static_cast<_Float16>(tv[2]), static_cast<_Float16>(tv[3])};
    row_ok[rt] = m0 + 16 * rt + ql < M;
  }
  // (ROPE) per lane: the position of its rows and the table entries of its dims d .. d+3 and
  // d+64 .. d+67, d = 16w + 4gr (every tile pair this wavefront takes is j = w, j + 4 of a head)
  f4 cs1[kRowTiles], cs2[kRowTiles], sn1[kRowTiles], sn2[kRowTiles];
  bool pos_ok[kRowTiles];
  if constexpr (ROPE) {
#pragma unroll
    for (int rt = 0; rt < kRowTiles; ++rt) {
      const int64_t p = ra.pos[min(m0 + 16 * rt + ql, M - 1)];
      pos_ok[rt] = p >= 0 && p < ra.slots;
      const uint32_t pu = pos_ok[rt] ? static_cast<uint32_t>(p) : 0u;
      const uint32_t t = pu - ra.per_seq.div(pu) * static_cast<uint32_t>(ra.T);
      const int64_t e = static_cast<int64_t>(t) * 128 + 16 * w + 4 * gr;
      cs1[rt] = *reinterpret_cast<const f4*>(ra.cos_t + e);
      cs2[rt] = *reinterpret_cast<const f4*>(ra.cos_t + e + 64);
      sn1[rt] = *reinterpret_cast<const f4*>(ra.sin_t + e);
      sn2[rt] = *reinterpret_cast<const f4*>(ra.sin_t + e + 64);
    }
  }
  // fp16(fp16(c) * scaling), the LoRA delta as peft's fp16 matmul and scaling round it (the
  // empty asm keeps the multiply and the fp16 conversion from fusing into one rounding)
  auto delta = [&](float c) {
    float v = r16(c) * scaling;
    asm("" : "+v"(v));
    return r16(v);
  };
  auto out_tiles = [&](const h4* bw, u32x2v (*xq)[kRowTiles], int t0) {
    if constexpr (ROPE) {
      const StreamOut out(ra.out, static_cast<uint64_t>(M) * W * 2u);
#pragma unroll
      for (int pr = 0; pr < kBatch / 2; ++pr) {
        const int tile = t0 + 8 * pr;          // dims d of a head; tile + 4: dims d + 64
        if (tile >= n16) break;
        const bool is_q = tile < nq16, is_k = tile >= nlora;
        const int col = tile_col(tile);
#pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt) {
          const u32x2v a2 = xq[2 * pr][rt], b2 = xq[2 * pr + 1][rt];
          float x1[4] = {lo_h(a2.x), hi_h(a2.x), lo_h(a2.y), hi_h(a2.y)};
          float x2[4] = {lo_h(b2.x), hi_h(b2.x), lo_h(b2.y), hi_h(b2.y)};
          if (!is_k) {
            const h4 tr = is_q ? tq4[rt] : tv4[rt];
            const f4 c1 = mfma16(bw[2 * pr], tr, f4{0.f, 0.f, 0.f, 0.f});
            const f4 c2 = mfma16(bw[2 * pr + 1], tr, f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              x1[i] = x1[i] + delta(c1[i]);
              x2[i] = x2[i] + delta(c2[i]);
            }
          }
          if (is_q || is_k) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float r1 = x1[i] * cs1[rt][i] - x2[i] * sn1[rt][i];
              const float r2 = x2[i] * cs2[rt][i] + x1[i] * sn2[rt][i];
              x1[i] = r1;
              x2[i] = r2;
            }
          }
          if (!pos_ok[rt]) {     // a row with no place: zeros, as soupk_rope_pack_tokens
#pragma unroll
            for (int i = 0; i < 4; ++i) x1[i] = x2[i] = 0.f;
          }
          if (row_ok[rt]) {
            const uint32_t off =
                (static_cast<uint32_t>(m0 + 16 * rt + ql) * W + col + 4 * gr) * 2u;
            out.store(off, u32x2{pack_h2(x1[0], x1[1]), pack_h2(x1[2], x1[3])});
            out.store(off + 128u, u32x2{pack_h2(x2[0], x2[1]), pack_h2(x2[2], x2[3])});
          }
        }
      }
    } else {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int tile = t0 + 4 * u;
        if (tile >= n16) break;
        const bool is_q = tile < nq16;
        const int f0 = 16 * (is_q ? tile : tile - nq16);
        const int N = is_q ? NQ : NV;
        const h4 a = bw[u];
#pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt) {
          const f4 c = mfma16(a, is_q ? tq4[rt] : tv4[rt], f4{0.f, 0.f, 0.f, 0.f});
          // C: column = row 16rt + ql, rows = features f0 + 4gr .. +3
          if (row_ok[rt]) {
            uint16_t* dst = (is_q ? lq : lv) + static_cast<int64_t>(m0 + 16 * rt + ql) * N +
                            f0 + 4 * gr;
            *reinterpret_cast<u32x2*>(dst) =
                u32x2{pack_h2(r16(c[0]) * scaling, r16(c[1]) * scaling),
                      pack_h2(r16(c[2]) * scaling, r16(c[3]) * scaling)};
          }
        }
      }
    }
  };
  h4 bw_cur[kBatch];
  u32x2v xq_cur[kBatch][kRowTiles];
  auto take = [&]() {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      bw_cur[u] = bw_next[u];
      if constexpr (ROPE) {
#pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt) xq_cur[u][rt] = xq_next[u][rt];
      }
    }
  };
  for (int t0 = t_begin + w; t0 < n16; t0 += 8 * kBatch) {
    take();
    if (t0 + 4 * kBatch < n16) load_b(bw_next, xq_next, t0 + 4 * kBatch);
    issue_here();
    out_tiles(bw_cur, xq_cur, t0);
    if (t0 + 4 * kBatch < n16) {
      take();
      if (t0 + 8 * kBatch < n16) load_b(bw_next, xq_next, t0 + 8 * kBatch);
      issue_here();
      out_tiles(bw_cur, xq_cur, t0 + 4 * kBatch);
    }
  }
}

__global__ __launch_bounds__(kThreads) void lora_bwd_rows_kernel(
    const uint16_t* gq, int64_t ldq, const uint16_t* gv, int64_t ldv, const _Float16* staged,
    float scaling, uint16_t* __restrict__ dt_out, uint16_t* __restrict__ dy, int M, int H,
    int NQ, int NV) {
  const StagedLayout L = staged_layout(H, NQ, NV);
  __shared__ float part[4][kRows][2 * kR + 1];
  __shared__ float dts[kRows][2 * kR];
  const int m0 = blockIdx.x * kRows;
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int ql = lane & 15, gr = lane >> 4;
  int64_t row[kRowTiles];
  bool row_ok[kRowTiles];
#pragma unroll
  for (int rt = 0; rt < kRowTiles; ++rt) {
    row[rt] = min(m0 + 16 * rt + ql, M - 1);
    row_ok[rt] = m0 + 16 * rt + ql < M;
  }
  // dt_x = gs_x B16_x: A operand = gs rows (row 16rt + ql, k = j0 + 8gr..+7); B operand =
  // B16_x (column = rank index ql, k = j: 8
  // consecutive entries of row ql of B16T_x, one 16-byte load), loaded once per step for the
  // kRowTiles row tiles.
  f4 acc_q[kRowTiles], acc_v[kRowTiles];
#pragma unroll
  for (int rt = 0; rt < kRowTiles; ++rt) {
    acc_q[rt] = f4{0.f, 0.f, 0.f, 0.f};
    acc_v[rt] = f4{0.f, 0.f, 0.f, 0.f};
  }
  // steps of 32 columns of g over this wavefront's quarter of N, in batches of kBatch steps,
  // the next batch's loads issued before the current batch's MFMAs
  struct Batch {
    h8 graw[kBatch][kRowTiles];
    h8 b[kBatch];
  };
  auto run = [&](const uint16_t* g, int64_t ldg, int N, const _Float16* bt, f4* acc) {
    const int kn = N / 4, steps = kn / 32;
    const _Float16* brow = bt + static_cast<int64_t>(ql) * N + w * kn + 8 * gr;
    auto load = [&](Batch& r, int s0) {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const int j = 32 * min(s0 + u, steps - 1);
#pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt)
          r.graw[u][rt] = *reinterpret_cast<const h8*>(g + row[rt] * ldg + w * kn + 8 * gr + j);
        r.b[u] = *reinterpret_cast<const h8*>(brow + j);
      }
    };
    auto mma = [&](const Batch& r, int s0) {
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        if (s0 + u >= steps) break;
        const h8 ba = r.b[u];
#pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt) {
          h8 ga;
#pragma unroll
          for (int i = 0; i < 8; ++i)
            ga[i] = static_cast<_Float16>(static_cast<float>(r.graw[u][rt][i]) * scaling);
          acc[rt] = mfma32(ga, ba, acc[rt]);
        }
      }
    };
    if (steps <= 0) return;
    Batch r0, r1;
    load(r0, 0);
    for (int s0 = 0; s0 < steps; s0 += 2 * kBatch) {
      if (s0 + kBatch < steps) load(r1, s0 + kBatch);
      issue_here();
      mma(r0, s0);
      if (s0 + kBatch < steps) {
        if (s0 + 2 * kBatch < steps) load(r0, s0 + 2 * kBatch);
        issue_here();
        mma(r1, s0 + kBatch);
      }
    }
  };
  run(gq, ldq, NQ, staged + L.b16t_q, acc_q);
  run(gv, ldv, NV, staged + L.b16t_v, acc_v);
#pragma unroll
  for (int rt = 0; rt < kRowTiles; ++rt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      part[w][16 * rt + 4 * gr + i][ql] = acc_q[rt][i];
      part[w][16 * rt + 4 * gr + i][kR + ql] = acc_v[rt][i];
    }
  }
  __syncthreads();
  for (int e = threadIdx.x; e < kRows * 2 * kR; e += kThreads) {
    const int m = e / (2 * kR), f = e % (2 * kR);
    const float s = ((part[0][m][f] + part[1][m][f]) + part[2][m][f]) + part[3][m][f];
    const _Float16 h = static_cast<_Float16>(s);
    dts[m][f] = static_cast<float>(h);
    if (blockIdx.y == 0 && m0 + m < M)
      dt_out[static_cast<int64_t>(m0 + m) * (2 * kR) + f] = h_bits(h);
  }
  __syncthreads();
  // dy = dt A16 (contraction over the 2r rank indices; A = A_q rows then A_v rows), one
  // 16-column tile of H at a time, transposed: A operand = A16 columns (row h0 + ql, k = rank
  // 8gr..+7: 8 consecutive entries of row h0 + ql of A16T, one 16-byte load), B = dt rows
  // (column = row ql of a row tile)
  h8 dtb[kRowTiles];
#pragma unroll
  for (int rt = 0; rt < kRowTiles; ++rt) {
#pragma unroll
    for (int i = 0; i < 8; ++i) dtb[rt][i] = static_cast<_Float16>(dts[16 * rt + ql][8 * gr + i]);
  }
  const _Float16* abase = staged + L.a16t + static_cast<int64_t>(ql) * (2 * kR) + 8 * gr;
  const int t_begin = tile_part(H / 16, blockIdx.y, gridDim.y);
  const int n16 = tile_part(H / 16, blockIdx.y + 1, gridDim.y);
  auto load_a = [&](h8* araw, int t0) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int h0 = 16 * min(t0 + 4 * u, n16 - 1);
      araw[u] = *reinterpret_cast<const h8*>(abase + static_cast<int64_t>(h0) * (2 * kR));
    }
  };
  auto out_tiles = [&](const h8* araw, int t0) {
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int tile = t0 + 4 * u;
      if (tile >= n16) break;
      const h8 a = araw[u];
#pragma unroll
      for (int rt = 0; rt < kRowTiles; ++rt) {
        const f4 c = mfma32(a, dtb[rt], f4{0.f, 0.f, 0.f, 0.f});
        if (row_ok[rt])
          *reinterpret_cast<u32x2*>(dy + (m0 + 16 * rt + ql) * static_cast<int64_t>(H) +
                                    16 * tile + 4 * gr) =
              u32x2{pack_h2(c[0], c[1]), pack_h2(c[2], c[3])};
      }
    }
  };
  if (t_begin + w < n16) {
    h8 a0[kBatch], a1[kBatch];
    load_a(a0, t_begin + w);
    for (int t0 = t_begin + w; t0 < n16; t0 += 8 * kBatch) {
      if (t0 + 4 * kBatch < n16) load_a(a1, t0 + 4 * kBatch);
      issue_here();
      out_tiles(a0, t0);
      if (t0 + 4 * kBatch < n16) {
        if (t0 + 8 * kBatch < n16) load_a(a0, t0 + 8 * kBatch);
        issue_here();
        out_tiles(a1, t0 + 4 * kBatch);
      }
    }
  }
}

// ---- parameter gradients: reductions over the rows ---------------------------------------
//   dA[i][k]  = fp16(sum_m dt[m][i] y[m][k])          i < 2r, k < H  (A_q rows, then A_v rows)
//   dBq[j][i] = fp16(sum_m gs_q[m][j] t[m][i])        j < NQ, i < r,  gs_x = fp16(g_x * s)
//   dBv[j][i] = fp16(sum_m gs_v[m][j] t[m][r + i])    j < NV, i < r
// each cast to fp32 (the fp16 GEMM result cast to the fp32 parameter, as autocast's backward
// gives it).  lora_params_partial_kernel: workgroup (column block of 64, slice of kSlice rows)
// stages 64-row chunks of X (y, or g_q / g_v scaled and rounded to gs as they are staged: its
// 64 columns) and Z (dt or t) through LDS,
// transposed so that each MFMA operand is 8 consecutive rows of one column, and writes fp32
// partial sums per slice; lora_params_reduce_kernel adds the slices in order and rounds.
// With the next chunk's loads issued before the current chunk's MFMAs and the reduce's loads
// issued eight slices at a time, the pair took 10.5 us against 13.2 us at 2048 rows on
// MI355X (identical bits); 256-row slices were faster at 2048 rows (9.4 us) but slower at 888
// (8.0 against 7.3 us), 64-row slices slower at both.
constexpr int kSlice = 128;        // rows per slice
constexpr int kChunk = 64;         // rows per LDS chunk
constexpr int kPStride = kChunk + 8;   // transposed tile row (halves): 144 B, 16-B aligned

// Rows (2rp, 2rp+1) x 8 columns, loaded at clamped rows and zeroed past `rows` ...
__device__ __forceinline__ void load_pair(const uint16_t* src, int64_t ld, int r0, int rows,
                                          int rp, int c8, u32x4& a, u32x4& b) {
  const int t0 = r0 + 2 * rp, t1 = t0 + 1;
  a = *reinterpret_cast<const u32x4*>(src + static_cast<int64_t>(min(t0, rows - 1)) * ld + 8 * c8);
  b = *reinterpret_cast<const u32x4*>(src + static_cast<int64_t>(min(t1, rows - 1)) * ld + 8 * c8);
  if (t0 >= rows) a = u32x4{0u, 0u, 0u, 0u};
  if (t1 >= rows) b = u32x4{0u, 0u, 0u, 0u};
}

// Eight fp16 values times s, each rounded to fp16.
__device__ __forceinline__ u32x4 scale_h8(u32x4 v, float s) {
  return u32x4{pack_h2(lo_h(v.x) * s, hi_h(v.x) * s), pack_h2(lo_h(v.y) * s, hi_h(v.y) * s),
               pack_h2(lo_h(v.z) * s, hi_h(v.z) * s), pack_h2(lo_h(v.w) * s, hi_h(v.w) * s)};
}

// ... and written transposed into tr[col][row] (stride kPStride) as 4-byte pairs.
__device__ __forceinline__ void store_pair_t(_Float16* tr, u32x4 a, u32x4 b, int rp, int c8) {
  const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
  uint32_t* col = reinterpret_cast<uint32_t*>(tr + (8 * c8) * kPStride + 2 * rp);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    col[(2 * j) * (kPStride / 2)] = (aw[j] & 0xffffu) | (bw[j] << 16);
    col[(2 * j + 1) * (kPStride / 2)] = (aw[j] >> 16) | (bw[j] & 0xffff0000u);
  }
}

__global__ __launch_bounds__(kThreads) void lora_params_partial_kernel(
    const uint16_t* __restrict__ y, const uint16_t* __restrict__ t,
    const uint16_t* __restrict__ dt, const uint16_t* __restrict__ gq, int64_t ldq,
    const uint16_t* __restrict__ gv, int64_t ldv, float scaling, float* __restrict__ part, int M,
    int H, int NQ, int NV, int64_t n_out) {
  __shared__ __align__(16) _Float16 XT[64 * kPStride];       // [64 columns][64 rows]
  __shared__ __align__(16) _Float16 ZT[2 * kR * kPStride];   // [32 columns][64 rows]
  const int nba = H / 64, nbq = NQ / 64;
  const int blk = blockIdx.x, slice = blockIdx.y;
  // kind 0: dA (X = y, Z = dt, 32 Z columns), 1: dBq (X = gs_q, Z = t[:, :r]), 2: dBv
  const int kind = blk < nba ? 0 : (blk < nba + nbq ? 1 : 2);
  const int col0 = 64 * (kind == 0 ? blk : (kind == 1 ? blk - nba : blk - nba - nbq));
  const uint16_t* X = kind == 0 ? y : (kind == 1 ? gq : gv);
  const int64_t ldx = kind == 0 ? H : (kind == 1 ? ldq : ldv);
  const int zc = kind == 0 ? 2 * kR : kR;                   // Z columns
  const uint16_t* Z = (kind == 0 ? dt : t) + (kind == 2 ? kR : 0);
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int ql = lane & 15, gr = lane >> 4;
  const int r_begin = slice * kSlice, r_end = min(M, r_begin + kSlice);
  // dA: C = X^T Z tiles (row = X column, column = Z column): wave w owns X columns 16w..+15
  //     and both Z tiles; dB: C = Z^T X (row = Z column, column = X column): wave w owns X
  //     columns 16w..+15.  Either way a lane's 4 results are 4 consecutive partial entries.
  f4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  // Staging: 32 row pairs x 8 column chunks of X, and of Z for the first zc / 8 chunks (whole
  // wavefronts).  The next chunk's loads are issued before the current chunk's MFMAs.
  const int rp = threadIdx.x & 31, c8 = threadIdx.x >> 5;
  const bool has_z = c8 < zc / 8;
  u32x4 xa, xb, za = {0u, 0u, 0u, 0u}, zb = za;
  load_pair(X + col0, ldx, r_begin, r_end, rp, c8, xa, xb);
  if (has_z) load_pair(Z, 2 * kR, r_begin, r_end, rp, c8, za, zb);
  for (int r0 = r_begin; r0 < r_end; r0 += kChunk) {
    __syncthreads();
    if (kind != 0) {   // gs = fp16(g * scaling), the value the fp16 GEMM it replaces reads
      xa = scale_h8(xa, scaling);
      xb = scale_h8(xb, scaling);
    }
    store_pair_t(XT, xa, xb, rp, c8);
    if (has_z) store_pair_t(ZT, za, zb, rp, c8);
    __syncthreads();
    if (r0 + kChunk < r_end) {
      load_pair(X + col0, ldx, r0 + kChunk, r_end, rp, c8, xa, xb);
      if (has_z) load_pair(Z, 2 * kR, r0 + kChunk, r_end, rp, c8, za, zb);
    }
    __asm__ volatile("" ::: "memory");   // keep the prefetch above the MFMAs
#pragma unroll
    for (int s = 0; s < kChunk / 32; ++s) {
      const h8 xf = *reinterpret_cast<const h8*>(XT + (16 * w + ql) * kPStride + 32 * s + 8 * gr);
      const h8 z0 = *reinterpret_cast<const h8*>(ZT + ql * kPStride + 32 * s + 8 * gr);
      if (kind == 0) {
        const h8 z1 =
            *reinterpret_cast<const h8*>(ZT + (kR + ql) * kPStride + 32 * s + 8 * gr);
        acc0 = mfma32(xf, z0, acc0);   // rows = X columns, column = Z column ql
        acc1 = mfma32(xf, z1, acc1);
      } else {
        acc0 = mfma32(z0, xf, acc0);   // rows = Z columns, column = X column
      }
    }
  }
  float* out = part + static_cast<int64_t>(slice) * n_out;
  if (kind == 0) {
    // dA[i][k]: i = Z column (ql, or r + ql), k = col0 + 16w + 4gr .. +3
    const int k = col0 + 16 * w + 4 * gr;
    *reinterpret_cast<f4*>(out + static_cast<int64_t>(ql) * H + k) = acc0;
    *reinterpret_cast<f4*>(out + static_cast<int64_t>(kR + ql) * H + k) = acc1;
  } else {
    // dB[j][i]: j = col0 + 16w + ql (X column), i = 4gr .. +3
    const int64_t base = 2 * kR * static_cast<int64_t>(H) + (kind == 2 ? kR * NQ : 0);
    *reinterpret_cast<f4*>(out + base + static_cast<int64_t>(col0 + 16 * w + ql) * kR + 4 * gr) =
        acc0;
  }
}

// Sum of the slices in slice order, one fp16 rounding, then fp32: dA_q, dA_v [r, H], dB_q
// [NQ, r], dB_v [NV, r] (the partial layout: dA rows, then dB_q, then dB_v).
__global__ __launch_bounds__(256) void lora_params_reduce_kernel(
    const float* __restrict__ part, int slices, int64_t n_out, int H, int NQ,
    float* __restrict__ daq, float* __restrict__ dav, float* __restrict__ dbq,
    float* __restrict__ dbv) {
  const int64_t o = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (o >= n_out) return;
  // Eight slices' loads issued together (clamped, so unconditional), then added in slice order.
  float s = 0.f;
  for (int i0 = 0; i0 < slices; i0 += 8) {
    float v8[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      v8[j] = part[static_cast<int64_t>(min(i0 + j, slices - 1)) * n_out + o];
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (i0 + j < slices) s += v8[j];
  }
  const float v = r16(s);
  const int64_t na = static_cast<int64_t>(kR) * H;
  if (o < na) daq[o] = v;
  else if (o < 2 * na) dav[o - na] = v;
  else if (o < 2 * na + static_cast<int64_t>(kR) * NQ) dbq[o - 2 * na] = v;
  else dbv[o - 2 * na - static_cast<int64_t>(kR) * NQ] = v;
}

int check_dims(int64_t M, int32_t H, int32_t NQ, int32_t NV, int32_t r) {
  if (M < 0 || r != kR || H <= 0 || NQ <= 0 || NV <= 0) return kInvalid;
  if (H % 128 || NQ % 128 || NV % 128) return kInvalid;   // 4-way split of 32-wide steps
  if ((M + kRows - 1) / kRows > 0x7fffffff || M * static_cast<int64_t>(H) >= (int64_t{1} << 40))
    return kInvalid;
  return kOk;
}

bool misaligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) != 0; }

// Column parts per row block: about kTargetGroups workgroups in all, each part at least
// 4 * kBatch output tiles (one batch per wavefront).
#ifndef SOUPK_LORA_TARGET_GROUPS
#define SOUPK_LORA_TARGET_GROUPS 256
#endif
constexpr int64_t kTargetGroups = SOUPK_LORA_TARGET_GROUPS;
unsigned column_parts(int64_t M, int n_tiles) {
  const int64_t row_blocks = (M + kRows - 1) / kRows;
  int64_t parts = (kTargetGroups + row_blocks - 1) / row_blocks;
  parts = std::min<int64_t>(parts, std::max(1, n_tiles / (4 * kBatch)));
  return static_cast<unsigned>(std::max<int64_t>(parts, 1));
}

}  // namespace
}  // namespace soupk

using namespace soupk;

extern "C" __attribute__((visibility("default"))) int soupk_lora_stage(
    const float* a_q, const float* a_v, const float* b_q, const float* b_v, uint16_t* staged,
    int64_t staged_elems, int32_t H, int32_t NQ, int32_t NV, int32_t r, void* stream) {
  const int rc = check_dims(0, H, NQ, NV, r);
  if (rc != kOk) return rc;
  if (!a_q || !a_v || !b_q || !b_v || !staged) return kInvalid;
  if (misaligned(staged)) return kInvalid;
  if (staged_elems < staged_layout(H, NQ, NV).total) return kInvalid;
  const int64_t n = staged_values(H, NQ, NV);
  const LoraStageArgs a{a_q, a_v, b_q, b_v, reinterpret_cast<_Float16*>(staged), H, NQ, NV};
  return launch_kernel(lora_stage_kernel, dim3(static_cast<unsigned>((n + 255) / 256)),
                       dim3(256), static_cast<hipStream_t>(stream), a);
}

extern "C" __attribute__((visibility("default"))) int soupk_lora_fwd(
    const uint16_t* y, const uint16_t* staged, float scaling, uint16_t* t, uint16_t* lq,
    uint16_t* lv, int64_t M, int32_t H, int32_t NQ, int32_t NV, int32_t r, void* stream) {
  const int rc = check_dims(M, H, NQ, NV, r);
  if (rc != kOk) return rc;
  if (M == 0) return kOk;
  if (!y || !staged || !t || !lq || !lv) return kInvalid;
  for (const void* p : {static_cast<const void*>(y), static_cast<const void*>(staged),
                        static_cast<const void*>(lq), static_cast<const void*>(lv)})
    if (misaligned(p)) return kInvalid;
  const unsigned grid = static_cast<unsigned>((M + kRows - 1) / kRows);
  return launch_kernel(lora_fwd_kernel<false>, dim3(grid, column_parts(M, NQ / 16 + NV / 16)),
                       dim3(kThreads), static_cast<hipStream_t>(stream), y,
                       reinterpret_cast<const _Float16*>(staged), scaling, t, lq, lv,
                       static_cast<int>(M), H, NQ, NV, LoraRope{});
}

extern "C" __attribute__((visibility("default"))) int soupk_lora_rope_fwd(
    const uint16_t* y, const uint16_t* staged, float scaling, const uint16_t* qkv,
    const float* cos, const float* sin, const int64_t* pos, uint16_t* t, uint16_t* out,
    int64_t M, int32_t H, int32_t NH, int32_t NKV, int32_t D, int32_t r, int32_t B, int32_t T,
    void* stream) {
  if (D != 128 || NH <= 0 || NKV <= 0 || B < 0 || T < 1) return kInvalid;
  const int32_t NQ = NH * D, NV = NKV * D;
  const int rc = check_dims(M, H, NQ, NV, r);
  if (rc != kOk) return rc;
  const int64_t W = static_cast<int64_t>(NQ) + 2 * NV;
  const int64_t slots = static_cast<int64_t>(B) * T;
  // (32-bit store offsets into `out`; positions split with a 31-bit divider)
  if (M * W * 2 >= (int64_t{1} << 32) || slots >= (int64_t{1} << 31)) return kInvalid;
  if (M == 0) return kOk;
  if (!y || !staged || !qkv || !cos || !sin || !pos || !t || !out) return kInvalid;
  for (const void* p : {static_cast<const void*>(y), static_cast<const void*>(staged),
                        static_cast<const void*>(qkv), static_cast<const void*>(cos),
                        static_cast<const void*>(sin), static_cast<const void*>(out)})
    if (misaligned(p)) return kInvalid;
  LoraRope ra{qkv, out, cos, sin, pos, NV, T, slots, FastDiv(static_cast<uint32_t>(T))};
  // whole heads per column part (one part per head at most)
  const int heads = static_cast<int>((W / 128));
  const unsigned parts = std::min<unsigned>(column_parts(M, NQ / 16 + NV / 16),
                                            static_cast<unsigned>(heads));
  const unsigned grid = static_cast<unsigned>((M + kRows - 1) / kRows);
  return launch_kernel(lora_fwd_kernel<true>, dim3(grid, parts), dim3(kThreads),
                       static_cast<hipStream_t>(stream), y,
                       reinterpret_cast<const _Float16*>(staged), scaling, t,
                       static_cast<uint16_t*>(nullptr), static_cast<uint16_t*>(nullptr),
                       static_cast<int>(M), H, NQ, NV, ra);
}

extern "C" __attribute__((visibility("default"))) int soupk_lora_bwd_rows(
    const uint16_t* g_q, int64_t ld_q, const uint16_t* g_v, int64_t ld_v,
    const uint16_t* staged, float scaling, uint16_t* dt, uint16_t* dy, int64_t M, int32_t H,
    int32_t NQ, int32_t NV, int32_t r, void* stream) {
  const int rc = check_dims(M, H, NQ, NV, r);
  if (rc != kOk) return rc;
  if (ld_q < NQ || ld_v < NV || ld_q % 8 || ld_v % 8) return kInvalid;
  if (M == 0) return kOk;
  if (!g_q || !g_v || !staged || !dt || !dy) return kInvalid;
  for (const void* p : {static_cast<const void*>(g_q), static_cast<const void*>(g_v),
                        static_cast<const void*>(staged), static_cast<const void*>(dy)})
    if (misaligned(p)) return kInvalid;
  const unsigned grid = static_cast<unsigned>((M + kRows - 1) / kRows);
  return launch_kernel(lora_bwd_rows_kernel, dim3(grid, column_parts(M, H / 16)),
                       dim3(kThreads), static_cast<hipStream_t>(stream), g_q, ld_q, g_v, ld_v,
                       reinterpret_cast<const _Float16*>(staged), scaling, dt, dy,
                       static_cast<int>(M), H, NQ, NV);
}

// Workspace of soupk_lora_bwd_params, in floats: ceil(M / 128) slices of partial sums.
static int64_t lora_params_workspace(int64_t M, int32_t H, int32_t NQ, int32_t NV) {
  const int64_t slices = (M + kSlice - 1) / kSlice;
  return slices * (2 * kR * static_cast<int64_t>(H) + kR * static_cast<int64_t>(NQ + NV));
}

namespace {

// The two launches of the parameter gradients over a caller-given partial-sum buffer `part`
// (at least lora_params_workspace(M, H, NQ, NV) floats).  The partial kernel writes every
// entry of every slice, so `part` needs no clearing and its old contents never leak into a
// result.
int lora_params_launch(const uint16_t* y, const uint16_t* t, const uint16_t* dt,
                       const uint16_t* g_q, int64_t ld_q, const uint16_t* g_v, int64_t ld_v,
                       float scaling, float* part, float* d_aq, float* d_av, float* d_bq,
                       float* d_bv, int64_t M, int32_t H, int32_t NQ, int32_t NV,
                       hipStream_t st) {
  const int64_t n_out = 2 * kR * static_cast<int64_t>(H) + kR * static_cast<int64_t>(NQ + NV);
  const unsigned reduce_grid = static_cast<unsigned>((n_out + 255) / 256);
  if (M == 0)   // no rows: zero gradients (the reduction over no slices)
    return launch_kernel(lora_params_reduce_kernel, dim3(reduce_grid), dim3(256), st,
                         static_cast<const float*>(nullptr), 0, n_out, H, NQ, d_aq, d_av,
                         d_bq, d_bv);
  const int slices = static_cast<int>((M + kSlice - 1) / kSlice);
  const dim3 grid(static_cast<unsigned>(H / 64 + NQ / 64 + NV / 64),
                  static_cast<unsigned>(slices));
  int rc2 = launch_kernel(lora_params_partial_kernel, grid, dim3(kThreads), st, y, t, dt, g_q,
                          ld_q, g_v, ld_v, scaling, part, static_cast<int>(M), H, NQ, NV, n_out);
  if (rc2 != kOk) return rc2;
  return launch_kernel(lora_params_reduce_kernel, dim3(reduce_grid), dim3(256), st, part,
                       slices, n_out, H, NQ, d_aq, d_av, d_bq, d_bv);
}

// Argument checks shared by both entry points (before any HIP call).
int lora_params_check(const uint16_t* y, const uint16_t* t, const uint16_t* dt,
                      const uint16_t* g_q, int64_t ld_q, const uint16_t* g_v, int64_t ld_v,
                      float* d_aq, float* d_av, float* d_bq, float* d_bv, int64_t M, int32_t H,
                      int32_t NQ, int32_t NV, int32_t r) {
  const int rc = check_dims(M, H, NQ, NV, r);
  if (rc != kOk) return rc;
  if (H % 64 || NQ % 64 || NV % 64) return kInvalid;
  if (ld_q < NQ || ld_v < NV || ld_q % 8 || ld_v % 8) return kInvalid;
  if (!d_aq || !d_av || !d_bq || !d_bv) return kInvalid;
  if (M == 0) return kOk;
  if (!y || !t || !dt || !g_q || !g_v) return kInvalid;
  for (const void* p : {static_cast<const void*>(y), static_cast<const void*>(t),
                        static_cast<const void*>(dt), static_cast<const void*>(g_q),
                        static_cast<const void*>(g_v)})
    if (misaligned(p)) return kInvalid;
  if ((M + kSlice - 1) / kSlice > 65535) return kInvalid;
  return kOk;
}

// ---- the allocation-free variant's scratch ----------------------------------------------------
// One fixed partial-sum buffer per GPU, in the library's code object: it exists on every device
// the library's kernels are loaded on, from module load to process exit.  Host code never
// passes `lora_scratch` itself to a kernel (on the host the name is only a stand-in for the
// symbol); each device's address is looked up once, with that device current, and kept.
constexpr int64_t kLoraScratchFloats = SOUPK_LORA_SCRATCH_FLOATS;
__device__ __align__(256) float lora_scratch[kLoraScratchFloats];

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kScratchDevices];   // device address of lora_scratch per ordinal (or null)

// The device address of the current device's lora_scratch (looked up on its first use).
int scratch_on_current_device(float** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return static_cast<int>(e);
  if (dev < 0 || dev >= kScratchDevices) return kInvalid;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(lora_scratch));
    if (e != hipSuccess) return static_cast<int>(e);
    if (p == nullptr) return static_cast<int>(hipErrorInvalidSymbol);
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *out = g_scratch_ptr[dev];
  return kOk;
}

}  // namespace

extern "C" __attribute__((visibility("default"))) int soupk_lora_bwd_params(
    const uint16_t* y, const uint16_t* t, const uint16_t* dt, const uint16_t* g_q, int64_t ld_q,
    const uint16_t* g_v, int64_t ld_v, float scaling, float* workspace, int64_t workspace_floats,
    float* d_aq, float* d_av, float* d_bq, float* d_bv, int64_t M, int32_t H, int32_t NQ,
    int32_t NV, int32_t r, void* stream) {
  const int rc = lora_params_check(y, t, dt, g_q, ld_q, g_v, ld_v, d_aq, d_av, d_bq, d_bv, M, H,
                                   NQ, NV, r);
  if (rc != kOk) return rc;
  if (workspace_floats < lora_params_workspace(M, H, NQ, NV)) return kInvalid;
  if (M > 0 && (!workspace || misaligned(workspace))) return kInvalid;
  return lora_params_launch(y, t, dt, g_q, ld_q, g_v, ld_v, scaling, workspace, d_aq, d_av, d_bq,
                            d_bv, M, H, NQ, NV, static_cast<hipStream_t>(stream));
}

extern "C" __attribute__((visibility("default"))) int soupk_lora_bwd_params_noalloc(
    const uint16_t* y, const uint16_t* t, const uint16_t* dt, const uint16_t* g_q, int64_t ld_q,
    const uint16_t* g_v, int64_t ld_v, float scaling, float* d_aq, float* d_av, float* d_bq,
    float* d_bv, int64_t M, int32_t H, int32_t NQ, int32_t NV, int32_t r, void* stream) {
  const int rc = lora_params_check(y, t, dt, g_q, ld_q, g_v, ld_v, d_aq, d_av, d_bq, d_bv, M, H,
                                   NQ, NV, r);
  if (rc != kOk) return rc;
  if (lora_params_workspace(M, H, NQ, NV) > kLoraScratchFloats) return SOUPK_STATUS_SCRATCH_LIMIT;
  float* part = nullptr;
  if (M > 0) {
    // Under stream capture the address must already be known (soupk_init_device, which the
    // Python binding calls when it loads the library): the lookup is not a call to make while
    // a graph is being captured.
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices) return kInvalid;
    float* known = nullptr;
    {
      std::lock_guard<std::mutex> lock(g_scratch_mu);
      known = g_scratch_ptr[dev];
    }
    if (known == nullptr) {
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      if (hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cs) != hipSuccess)
        return kInvalid;
      if (cs != hipStreamCaptureStatusNone)
        return static_cast<int>(hipErrorStreamCaptureUnsupported);
    }
    const int rs = scratch_on_current_device(&part);
    if (rs != kOk) return rs;
  }
  return lora_params_launch(y, t, dt, g_q, ld_q, g_v, ld_v, scaling, part, d_aq, d_av, d_bq,
                            d_bv, M, H, NQ, NV, static_cast<hipStream_t>(stream));
}

extern "C" __attribute__((visibility("default"))) int soupk_init_device(void) {
  float* part = nullptr;
  return scratch_on_current_device(&part);
}
