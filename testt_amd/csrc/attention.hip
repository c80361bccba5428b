// Causal grouped-query attention over the padded [B, heads, T, D] layout, forward and backward,
// for head_dim 128 on gfx950 MFMA (v_mfma_f32_16x16x32_f16).
//
// Replaces torch's scaled_dot_product_attention in the layer loop of the reference's
// fused_forward (solution/model.py:246-247, transformers' sdpa_attention_forward with the causal
// + key-padding mask of create_causal_mask): query i of a row attends to key j iff j <= i and
// key j is a real token (key_valid[b, j] != 0, or every key when key_valid is NULL).
//
// MFMA operand layouts (16x16x32 f16, checked on the device): A[16 x 32]: lane l holds row
// l%16, k = 8(l/16)..+7; B[32 x 16]: lane l holds column l%16, k = 8(l/16)..+7; C[16 x 16]:
// lane l holds column l%16, rows 4(l/16)..+3.  Below, a lane's "group" is l/16 and its
// "column" l%16.
//
// Forward (flash attention, online softmax): a workgroup is 4 wavefronts and 64 queries of one
// (batch, head); wavefront w owns queries 16w..16w+15.  Key blocks of 64 rows are staged in LDS
// -- K and V row-major -- and each wavefront computes
//   S^T (64 keys x 16 queries) = K Q^T        (A = K rows from LDS, B = Q^T from registers)
// so that, in the C layout, lane l holds the scores of query l%16 for keys 16n + 4(l/16) + i
// of key tile n.  Two C tiles (n = 2m, 2m+1) together are the B operand of
//   O^T (128 x 16) += V^T P^T                  (A = V^T from LDS, B = P^T from registers)
// when the contraction index j of group gr stands for key 32m + 4gr + j (j < 4) or
// 32m + 16 + 4gr + (j - 4): the A operand is read in the same order, with LDS transpose reads
// of the row-major V tile (lds_runs_tr).  The online-softmax state of a query is local to its four lanes (l%16 + 16r), which
// combine block maxima and final sums with v_permlane16_swap / v_permlane32_swap (no LDS).
// Scores are kept in base 2: x = s * scale * log2(e), p = 2^(x - m).  The reference value m of
// a query is raised only when a block maximum exceeds it by more than 8 (p <= 2^8 otherwise,
// exact in fp16 and fp32), so the accumulators are rarely rescaled.  The output is written
// token-major, out[(b*T + t), h*D + d], the layout the o-projection GEMM reads, and the
// per-query log-sum-exp (natural log) for the backward pass; a query with no visible key gets
// output 0 and lse = +inf (so its backward probabilities are 0).
//
// LDS: row-major tiles [64][144] halves (see kRStride: conflict-free 16-byte and transpose
// reads).

#include "fastdiv.hpp"
#include "soupk_common.hpp"

namespace soupk {
namespace {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;               // head dim
constexpr int kBQ = 64;               // queries per workgroup (4 wavefronts x 16)
constexpr int kBK = 64;               // keys per block
constexpr int kAttnThreads = 256;
// Row-major tile row stride (halves), 288 B.  gfx950's LDS serves 256 B per clock to reads:
// with a 144-half stride the 16-byte fragment reads (lanes 0..7 and 16..23 of a wavefront
// together: 8 rows x 2 column chunks) and the transpose reads (32 lanes: 8 rows x 4 column
// runs) each land on 64 distinct banks.  A 136-half stride gave both 2-way bank conflicts
// (measured with the SQ_LDS_BANK_CONFLICT counter on a probe: 7.77 against 3.92 cycles per
// 16-byte read, 3.96 against 2.00 per transpose read); the varlen backward took 46.2 -> 44.8 us
// with the wider stride, the ragged backward 32.1 -> 31.0 us.
constexpr int kRStride = kD + 16;
constexpr float kRescaleMargin = 8.f;  // log2 of the largest unnormalised probability kept

__device__ __forceinline__ f4 mfma32(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ h8 lds_h8(const _Float16* p) {
  return *reinterpret_cast<const h8*>(p);
}

// The A operand of a product contracted over keys (or queries), read transposed from a
// row-major tile rm (row stride ld halves): lane l gets column col0 + l%16 at rows
// 32m + 4gr .. +3, then 32m + 16 + 4gr .. +3 (the order of the two C tiles 2m, 2m+1 it meets).
// Two ds_read_b64_tr_b16: within each 16-lane group, result lane i element j is element i%4
// of the 8-byte read of lane 4j + i/4, so lane k of group gr reads row r0 + k/4 at columns
// col0 + 4(k%4) (r0 = 32m + 4gr, then + 16); result lane i then holds rows r0..r0+3 of column
// col0 + i.  (Layout checked on the device.)  Against a transposed copy of the tile built
// with 4-byte LDS stores: forward 16.1 -> 15.4 us, backward 47.5 -> 46.0 us, identical bits.
typedef short s4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s4 lds_s4;
typedef __attribute__((address_space(3))) _Float16 lds_h;
__device__ __forceinline__ h8 lds_runs_tr(const _Float16* rm, int ld, int col0, int m, int gr) {
  const int k = threadIdx.x & 15;
  const int row = 32 * m + 4 * gr + (k >> 2), col = col0 + 4 * (k & 3);
  const lds_h* base = (const lds_h*)(rm);   // (an address-space cast: rm points into LDS)
  const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(base + row * ld + col));
  const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(base + (row + 16) * ld + col));
  const h4 l4 = __builtin_bit_cast(h4, lo), h4v = __builtin_bit_cast(h4, hi);
  return __builtin_shufflevector(l4, h4v, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Max / sum over the four lanes of a column (l%16 + 16r, r = 0..3): rows 0<->1 and 2<->3 are
// exchanged, then the two halves.  Every lane of the column gets the same bits (the operands
// are combined in lane order on all four).
__device__ __forceinline__ float column_max(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float column_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// A [64 x 128] fp16 tile (64 rows of one head) is staged through registers: thread item
// it (0, 1) covers rows 2rp, 2rp+1 at dims 8dc..8dc+7 (tile_item), one pair of 16-byte row
// loads and two 16-byte LDS stores.  The loads of block i+1 are issued before block i is
// computed and written to LDS after the next barrier, so their latency overlaps the MFMAs.
// Row indices past the end clamp to the last row (a finite value): the callers give such rows
// zero weight (key flags, query bounds), so no branch guards the loads.  The pointers these
// loads go through are not __restrict__: that keeps the compiler from moving them past the
// barriers (it would otherwise issue them just before their LDS stores, hiding nothing).
struct TileRegs {
  u32x4 a[2], b[2];
};

// Which row pair rp (0..31) and 8-dim chunk dc (0..15) thread item `it` covers: a
// wavefront's item covers 16 row pairs x 4 chunks, lane bits (dc0, rp0, rp1, rp2, dc1, rp3).
// Each 16-lane group of a 16-byte row-major store then writes 8 row pairs x 2 chunks on
// distinct LDS banks, and the global loads read 64 contiguous bytes per row.  (With the
// transposed tile copies this layout replaced, it took the forward from 20.0 to 18.3 us and
// the backward from 39.8 to 36.7 us at the 2048-token shape.)
__device__ __forceinline__ void tile_item(int it, int& rp, int& dc) {
  const int lane = threadIdx.x & 63, wi = (threadIdx.x >> 6) + 4 * it;
  rp = 16 * (wi & 1) + ((lane >> 1) & 7) + 8 * (lane >> 5);
  dc = 4 * (wi >> 1) + (lane & 1) + 2 * ((lane >> 4) & 1);
}

// Row t of a tile source with row stride `ld` elements.  The entry points keep every row offset
// of a sequence below 2^31 elements, so it is formed with one 32-bit multiply.
__device__ __forceinline__ const uint16_t* row_at(const uint16_t* base, int t, int64_t ld) {
  return base + static_cast<uint32_t>(t) * static_cast<uint32_t>(ld);
}

__device__ __forceinline__ void load_tile(TileRegs& r, const uint16_t* src, int64_t stride,
                                          int r0, int nrows) {
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    int rp, dc;
    tile_item(it, rp, dc);
    const int t0 = min(r0 + 2 * rp, nrows - 1), t1 = min(r0 + 2 * rp + 1, nrows - 1);
    r.a[it] = *reinterpret_cast<const u32x4*>(row_at(src, t0, stride) + 8 * dc);
    r.b[it] = *reinterpret_cast<const u32x4*>(row_at(src, t1, stride) + 8 * dc);
  }
}

// A compiler-only barrier (no instruction, no wait): the prefetch loads above it stay above it
// instead of being moved down to their use in the next iteration.
__device__ __forceinline__ void issue_here() { __asm__ volatile("" ::: "memory"); }

// Rows (2rp, 2rp+1) x 8 dims, row-major into `rm` ([64][kRStride]).
__device__ __forceinline__ void stage_pair(_Float16* rm, u32x4 a, u32x4 b, int rp, int dc) {
  *reinterpret_cast<u32x4*>(rm + (2 * rp) * kRStride + 8 * dc) = a;
  *reinterpret_cast<u32x4*>(rm + (2 * rp + 1) * kRStride + 8 * dc) = b;
}

__device__ __forceinline__ void store_tile(_Float16* rm, const TileRegs& r) {
#pragma unroll
  for (int it = 0; it < 2; ++it) {
    int rp, dc;
    tile_item(it, rp, dc);
    stage_pair(rm, r.a[it], r.b[it], rp, dc);
  }
}

// The key-valid byte of key key0 + threadIdx.x % 64, loaded unconditionally (from `any`, a
// readable address, when there is no flag array) and tested only when stored, so that the
// test does not wait for the tile loads issued with it.
__device__ __forceinline__ uint8_t load_flag_raw(const uint8_t* valid, const void* any, int key0,
                                                 int T) {
  const int t = min(key0 + (threadIdx.x & (kBK - 1)), T - 1);
  return *(valid != nullptr ? valid + t : static_cast<const uint8_t*>(any));
}

__device__ __forceinline__ uint8_t key_flag(uint8_t raw, bool has_valid, int key0, int T) {
  const int t = key0 + (threadIdx.x & (kBK - 1));
  return (t < T && (!has_valid || raw != 0)) ? 1 : 0;
}

// Flags of keys 16n + 4gr .. +3 of the staged block, one byte each.
__device__ __forceinline__ uint32_t flag_word(const uint8_t* kflag, int n, int gr) {
  return *reinterpret_cast<const uint32_t*>(kflag + 16 * n + 4 * gr);
}

// ---- the rows of one (sequence, head) ----------------------------------------------------------
// Both layouts reduce to: a sequence of `len` rows; row t of Q at q + t*ld_q, of K / V at
// k / v + t*ld_kv, of O and dO at out / dout + t*ld_o (token-major); its lse and D at lse[t],
// delta[t]; its dK / dV partials at row `plane + t` of the partial buffers; key flags (padded
// layout only) at valid[t].
//   padded [B, heads, T, D]: a sequence is a batch row (len = T, flags from key_valid);
//   varlen: a sequence is tokens [cu[b], cu[b+1]) of the token-major q|k|v rows [M, W] that
//           soupk_rope_pack_tokens writes (every token real, no flags; lse, D and the
//           partials are [NH, M] planes).
struct AttnParams {
  const uint16_t* q;        // padded q, or the varlen q|k|v rows
  const uint16_t* k;
  const uint16_t* v;
  const uint8_t* key_valid;
  const int32_t* cu;        // varlen: [B + 1] sequence starts
  uint16_t* out;
  const uint16_t* dout;
  float* lse;
  float* delta;
  uint16_t* dq;             // padded dq [B, NH, T, D]; varlen dq|dk|dv rows [M, W]
  uint16_t* dk;             // padded dk, dv (the reduce kernel's outputs)
  uint16_t* dv;
  float* dk_part;
  float* dv_part;
  const float* cos;         // varlen backward: the RoPE tables [rope_T, D] (null: no rotation)
  const float* sin;
  const int64_t* pos;       // varlen backward: padded position of each token
  int64_t pos_slots;        // positions at or past this have no table row
  FastDiv rope_div;         // divides by rope_T
  int T, NH, NKV;
  int64_t M, W;             // varlen: tokens, q|k|v row stride
  float scale, scale_log2;
};

struct SeqHead {
  int len;
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t ld_q, ld_kv, ld_o;
  const uint8_t* valid;
  uint16_t* out;
  const uint16_t* dout;
  float* lse;
  const float* delta;
  int64_t tok0;             // token index of row 0 (varlen)
  int64_t plane;            // partial-buffer row of row 0
};

template <bool VARLEN>
__device__ __forceinline__ SeqHead seq_head(const AttnParams& p, int b, int h) {
  const int g = h / (p.NH / p.NKV);
  const int64_t HD = static_cast<int64_t>(p.NH) * kD;
  SeqHead s;
  if constexpr (VARLEN) {
    // Sequence bounds come from device memory: a bound outside [0, M], or an end before its
    // start, makes the sequence empty (nothing read, nothing written).
    const int64_t s0 = p.cu[b], s1 = p.cu[b + 1];
    const bool ok = s0 >= 0 && s1 >= s0 && s1 <= p.M;
    s.len = ok ? static_cast<int>(s1 - s0) : 0;
    const int64_t base = ok ? s0 : 0;
    s.q = p.q + base * p.W + h * kD;
    s.k = p.q + base * p.W + (p.NH + g) * kD;
    s.v = p.q + base * p.W + (p.NH + p.NKV + g) * kD;
    s.ld_q = s.ld_kv = p.W;
    s.valid = nullptr;
    s.out = p.out + base * HD + h * kD;
    s.dout = p.dout + base * HD + h * kD;
    s.ld_o = HD;
    s.lse = p.lse + h * p.M + base;
    s.delta = p.delta + h * p.M + base;
    s.tok0 = base;
    s.plane = h * p.M + base;
  } else {
    const int64_t T = p.T;
    s.len = p.T;
    s.q = p.q + (static_cast<int64_t>(b) * p.NH + h) * T * kD;
    s.k = p.k + (static_cast<int64_t>(b) * p.NKV + g) * T * kD;
    s.v = p.v + (static_cast<int64_t>(b) * p.NKV + g) * T * kD;
    s.ld_q = s.ld_kv = kD;
    s.valid = p.key_valid != nullptr ? p.key_valid + b * T : nullptr;
    s.out = p.out + b * T * HD + h * kD;
    s.dout = p.dout + b * T * HD + h * kD;
    s.ld_o = HD;
    s.lse = p.lse + (static_cast<int64_t>(b) * p.NH + h) * T;
    s.delta = p.delta + (static_cast<int64_t>(b) * p.NH + h) * T;
    s.tok0 = b * T;
    s.plane = (static_cast<int64_t>(b) * p.NH + h) * T;
  }
  return s;
}

// One query block of one (sequence, head): flash-attention forward.
__device__ __forceinline__ void attn_fwd_block(const AttnParams& p, const SeqHead& sh, int qb,
                                               _Float16* Ks, _Float16* Vs, uint8_t* kflag) {
  const int T = sh.len;
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int ql = lane & 15, gr = lane >> 4;
  const int q_abs = qb * kBQ + 16 * w + ql;
  const uint16_t* qrow = row_at(sh.q, min(q_abs, T - 1), sh.ld_q);
  const uint16_t* kbase = sh.k;
  const uint16_t* vbase = sh.v;
  const uint8_t* valid = sh.valid;
  const bool has_valid = valid != nullptr;
  const float scale_log2 = p.scale_log2;

  // Q^T operand: 4 k-steps of 32 dims, lane holds Q[q][32s + 8gr .. +7]
  h8 qf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) qf[s] = *reinterpret_cast<const h8*>(qrow + 32 * s + 8 * gr);
  f4 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
  float m_ref = -INFINITY, lsum = 0.f;

  TileRegs kr, vr;
  load_tile(kr, kbase, sh.ld_kv, 0, T);
  load_tile(vr, vbase, sh.ld_kv, 0, T);
  uint8_t fl_raw = load_flag_raw(valid, kbase, 0, T);
  for (int kb = 0; kb <= qb; ++kb) {
    __syncthreads();
    store_tile(Ks, kr);
    store_tile(Vs, vr);   // V row-major too: its V^T fragments are read transposed
    if (threadIdx.x < kBK) kflag[threadIdx.x] = key_flag(fl_raw, has_valid, kb * kBK, T);
    __syncthreads();
    load_tile(kr, kbase, sh.ld_kv, (kb + 1) * kBK, T);   // the next block (clamped past the end)
    load_tile(vr, vbase, sh.ld_kv, (kb + 1) * kBK, T);
    fl_raw = load_flag_raw(valid, kbase, (kb + 1) * kBK, T);
    issue_here();
    // S^T for the 4 key tiles: the 16 K fragments read first, then the MFMAs k-step by k-step
    // over the 4 independent accumulators (a wavefront is alone on its SIMD, so four chains in
    // flight instead of one keep the MFMA pipe busy; pinned with scheduling-group barriers,
    // since the compiler otherwise reads each fragment just before its use and runs one tile's
    // chain after another: 15.52 -> 15.22 us at 2048 tokens, 12.83 -> 12.21 us ragged).
    f4 sc[4];
    {
      h8 kf[4][4];
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int s = 0; s < 4; ++s)
          kf[n][s] = lds_h8(Ks + (16 * n + ql) * kRStride + 32 * s + 8 * gr);
#pragma unroll
      for (int n = 0; n < 4; ++n) sc[n] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int n = 0; n < 4; ++n) sc[n] = mfma32(kf[n][s], qf[s], sc[n]);
      __builtin_amdgcn_sched_group_barrier(0x100, 16, 0);   // the 16 LDS reads
      __builtin_amdgcn_sched_group_barrier(0x008, 16, 0);   // then the 16 MFMAs
    }
    // scale, mask (the diagonal block, or keys with flags), block max.  Keys of an interior
    // block (kb < qb) precede every query of this workgroup and lie below T.
    float x[4][4];
    float mx = -INFINITY;
    if (kb == qb || has_valid) {
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const uint32_t fl = flag_word(kflag, n, gr);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = kb * kBK + 16 * n + 4 * gr + i;
          const bool vis = key <= q_abs && ((fl >> (8 * i)) & 0xffu) != 0;
          x[n][i] = vis ? sc[n][i] * scale_log2 : -INFINITY;
          mx = fmaxf(mx, x[n][i]);
        }
      }
    } else {
#pragma unroll
      for (int n = 0; n < 4; ++n) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[n][i] = sc[n][i] * scale_log2;
          mx = fmaxf(mx, x[n][i]);
        }
      }
    }
    mx = column_max(mx);
    if (__any(mx > m_ref + kRescaleMargin)) {   // (m_ref = -inf: any visible key)
      const float m_new = fmaxf(m_ref, mx);
      const float alpha = m_ref == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m_ref - m_new);
      lsum *= alpha;
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[t] = acc[t] * alpha;
      m_ref = m_new;
    }
    const float m_use = m_ref == -INFINITY ? 0.f : m_ref;
    float ps = 0.f;
    h8 pb[2];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float pr = __builtin_amdgcn_exp2f(x[n][i] - m_use);  // 2^-inf = 0
        ps += pr;
        pb[n >> 1][4 * (n & 1) + i] = static_cast<_Float16>(pr);
      }
    }
    lsum += ps;
    // O^T += V^T P^T
#pragma unroll
    for (int t = 0; t < 8; ++t) {
#pragma unroll
      for (int m = 0; m < 2; ++m)
        acc[t] = mfma32(lds_runs_tr(Vs, kRStride, 16 * t, m, gr), pb[m], acc[t]);
    }
  }
  const float l_tot = column_sum(lsum);
  if (q_abs >= T) return;
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  uint16_t* orow = sh.out + static_cast<uint32_t>(q_abs) * static_cast<uint32_t>(sh.ld_o);
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const f4 o = acc[t] * inv;
    *reinterpret_cast<u32x2*>(orow + 16 * t + 4 * gr) = u32x2{pack_h2(o[0], o[1]),
                                                                pack_h2(o[2], o[3])};
  }
  if (gr == 0) sh.lse[q_abs] = l_tot > 0.f ? (m_ref + log2f(l_tot)) * kLn2 : INFINITY;
}

// Grid: x = head, y = sequence (batch row), z = query-block slot: slot z is query block
// nqb-1-z of its sequence, so the heaviest blocks (the most key blocks) are dispatched first.
// The host gives z at least as many slots as the longest possible sequence has blocks (T for
// the padded layout, ceil(M/64) for varlen, since no sequence holds more than M tokens): slots
// past a sequence's blocks exit at once.  (A loop over several blocks per workgroup cost
// 0.5 us forward and backward at the step's shape; the idle workgroups measured nothing.)
// One forward workgroup per CU: the K tile array is padded so that a workgroup's LDS exceeds
// half of a CU's 160 KB.  The dispatcher then never places a second workgroup beside one that
// walks a long causal key range (the heaviest are dispatched first), and the lighter ones start
// on whichever CU frees first.  At 2048 tokens (4 x 512) 15.24 -> 15.04 us, on rows of 512,
// 512, 256 and 128 tokens 14.48 -> 13.04 us, no case slower.
constexpr int kFwdLdsPad = 24576;   // halves
static_assert((2 * kBK * kRStride + kFwdLdsPad) * 2 > 80 * 1024, "one workgroup per CU");

template <bool VARLEN>
__global__ __launch_bounds__(kAttnThreads) void attn_fwd_kernel(AttnParams p) {
  __shared__ __align__(16) _Float16 Ks[kBK * kRStride + kFwdLdsPad];
  __shared__ __align__(16) _Float16 Vs[kBK * kRStride];
  __shared__ __align__(16) uint8_t kflag[kBK];
  const SeqHead sh = seq_head<VARLEN>(p, blockIdx.y, blockIdx.x);
  const int qb = (sh.len + kBQ - 1) / kBQ - 1 - static_cast<int>(blockIdx.z);
  if (qb >= 0) attn_fwd_block(p, sh, qb, Ks, Vs, kflag);
}

// ---- backward ------------------------------------------------------------------------------
// With P = softmax of the scaled scores (recomputed from the saved log-sum-exp), dO the output
// gradient and D = rowsum(dO * O):  dP = dO V^T,  dS = P * (dP - D),  dQ = scale * dS K,
// dK = scale * dS^T Q,  dV = P^T dO.  Three launches:
//   attn_bwd_delta_kernel (b, head, 64 queries): D;
//   attn_bwd_kernel       two kinds of workgroup in one grid, so that they run side by side
//                         (z even: dK/dV of 64 keys, z odd: dQ of 64 queries, the heaviest
//                         causal blocks of both kinds dispatched first):
//     dQ   (b, head, 64 queries): over its key blocks S^T = K Q^T, dP^T = V dO^T (the
//          forward's orientation: query = lane column), dQ^T += K^T dS^T;
//     dKdV (b, head, 64 keys): over the query blocks that see them, S = Q K^T, dP = dO V^T
//          (key = lane column), dV^T += dO^T P, dK^T += Q^T dS, into fp32 partials per query
//          head;
//   attn_bwd_reduce_kernel: dK, dV of a key/value head = the sum of its query heads' partials
//                         (a fixed order: deterministic), fp16.
// Every tile is staged row-major.  Operands contracted over the head dim are read with
// 16-byte LDS reads; operands contracted over keys or queries with LDS transpose reads of
// the same tiles, in the order of the C tiles they meet (lds_runs_tr).

// D = rowsum(dO * O) of 64 queries: lane (row l%16 of wavefront w's 16, group l/16) sums dims
// 32s + 8gr .. +7 (s = 0..3) in order, then the four groups are combined by column_sum.
__global__ __launch_bounds__(kAttnThreads) void attn_bwd_delta_kernel(
    const uint16_t* __restrict__ out, const uint16_t* __restrict__ dout, float* __restrict__ delta,
    int T, int NH) {
  const int qb = static_cast<int>(blockIdx.z);
  const int h = blockIdx.x, b = blockIdx.y;
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int ql = lane & 15, gr = lane >> 4;
  const int q_abs = qb * kBQ + 16 * w + ql;
  const int qc = min(q_abs, T - 1);
  const int64_t HD = static_cast<int64_t>(NH) * kD;
  const uint16_t* orow = out + (static_cast<int64_t>(b) * T + qc) * HD + h * kD;
  const uint16_t* dorow = dout + (static_cast<int64_t>(b) * T + qc) * HD + h * kD;
  h8 of[4], dof[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    of[s] = *reinterpret_cast<const h8*>(orow + 32 * s + 8 * gr);
    dof[s] = *reinterpret_cast<const h8*>(dorow + 32 * s + 8 * gr);
  }
  float dsum = 0.f;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      dsum = dsum + static_cast<float>(dof[s][i]) * static_cast<float>(of[s][i]);
  }
  dsum = column_sum(dsum);
  if (gr == 0 && q_abs < T) delta[(static_cast<int64_t>(b) * NH + h) * T + q_abs] = dsum;
}

// LDS of the backward workgroups (the larger of the two kinds: dKdV's Q and dO tiles and the
// block's lse / D values).
constexpr int kBwdLdsBytes = 2 * kBQ * kRStride * 2 + 2 * kBQ * 4;

// fp32 -> fp16 -> fp32: the value a kernel that stores fp16 hands to the next one.
__device__ __forceinline__ float round_h(float x) { return lo_h(pack_h2(x, 0.f)); }

// Table rows (cos, sin) of the token's position for the transposed rotation, or null when the
// token has none (no tables, or a position outside [0, pos_slots)).
__device__ __forceinline__ bool rope_rows(const AttnParams& p, int64_t tok, const float** c,
                                          const float** sn) {
  if (p.cos == nullptr) return false;
  const int64_t ps = p.pos[tok];
  if (ps < 0 || ps >= p.pos_slots) return false;
  const uint32_t pu = static_cast<uint32_t>(ps);
  const uint32_t t = pu - p.rope_div.div(pu) * p.rope_div.d;
  *c = p.cos + static_cast<int64_t>(t) * kD;
  *sn = p.sin + static_cast<int64_t>(t) * kD;
  return true;
}

// The transposed rotation of RoPE's backward (solution/rope.py:78-128) on fp16-rounded
// gradients g1 (dims d..d+3 of the first half) and g2 (the same dims of the second half):
// (g1*c1 + g2*s2, g2*c2 - g1*s1), each product rounded.
__device__ __forceinline__ void rope_bwd4(const f4& c1, const f4& c2, const f4& s1, const f4& s2,
                                          const f4& g1, const f4& g2, f4& o1, f4& o2) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o1[i] = g1[i] * c1[i] + g2[i] * s2[i];
    o2[i] = g2[i] * c2[i] - g1[i] * s1[i];
  }
}

__device__ __forceinline__ void rope_bwd4(const float* c, const float* sn, int d, const f4& g1,
                                          const f4& g2, f4& o1, f4& o2) {
  const f4 c1 = *reinterpret_cast<const f4*>(c + d), c2 = *reinterpret_cast<const f4*>(c + d + 64);
  const f4 s1 = *reinterpret_cast<const f4*>(sn + d);
  const f4 s2 = *reinterpret_cast<const f4*>(sn + d + 64);
  rope_bwd4(c1, c2, s1, s2, g1, g2, o1, o2);
}

template <bool VARLEN>
__device__ __forceinline__ void attn_bwd_dq(const AttnParams& p, const SeqHead& sh, int h, int b,
                                            int qb, unsigned char* smem) {
  _Float16* Ks = reinterpret_cast<_Float16*>(smem);
  _Float16* Vs = Ks + kBK * kRStride;
  uint8_t* kflag = reinterpret_cast<uint8_t*>(Vs + kBK * kRStride);
  const int T = sh.len;
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int ql = lane & 15, gr = lane >> 4;
  const int q_abs = qb * kBQ + 16 * w + ql;
  const int qc = min(q_abs, T - 1);
  const uint16_t* qrow = row_at(sh.q, qc, sh.ld_q);
  const uint16_t* dorow = row_at(sh.dout, qc, sh.ld_o);
  const uint16_t* kbase = sh.k;
  const uint16_t* vbase = sh.v;
  const uint8_t* valid = sh.valid;
  const bool has_valid = valid != nullptr;
  const float scale_log2 = p.scale_log2;

  h8 qf[4], dof[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    qf[s] = *reinterpret_cast<const h8*>(qrow + 32 * s + 8 * gr);
    dof[s] = *reinterpret_cast<const h8*>(dorow + 32 * s + 8 * gr);
  }
  const float dsum = sh.delta[qc];
  const float lse2 = sh.lse[qc] * kLog2e;  // +inf: no visible key, every p = 0

  f4 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
  TileRegs kr, vr;
  load_tile(kr, kbase, sh.ld_kv, 0, T);
  load_tile(vr, vbase, sh.ld_kv, 0, T);
  uint8_t fl_raw = load_flag_raw(valid, kbase, 0, T);
  for (int kb = 0; kb <= qb; ++kb) {
    __syncthreads();
    store_tile(Ks, kr);   // K^T fragments read transposed from Ks
    store_tile(Vs, vr);
    if (threadIdx.x < kBK) kflag[threadIdx.x] = key_flag(fl_raw, has_valid, kb * kBK, T);
    __syncthreads();
    load_tile(kr, kbase, sh.ld_kv, (kb + 1) * kBK, T);   // the next block (clamped past the end)
    load_tile(vr, vbase, sh.ld_kv, (kb + 1) * kBK, T);
    fl_raw = load_flag_raw(valid, kbase, (kb + 1) * kBK, T);
    issue_here();
    const bool masked = kb == qb || has_valid;
    h8 dsb[2];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      h8 kf[4], vf[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        kf[s] = lds_h8(Ks + (16 * n + ql) * kRStride + 32 * s + 8 * gr);
        vf[s] = lds_h8(Vs + (16 * n + ql) * kRStride + 32 * s + 8 * gr);
      }
      f4 sc = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        sc = mfma32(kf[s], qf[s], sc);
        dp = mfma32(vf[s], dof[s], dp);
      }
      const uint32_t fl = masked ? flag_word(kflag, n, gr) : 0x01010101u;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kb * kBK + 16 * n + 4 * gr + i;
        const bool vis = !masked || (key <= q_abs && ((fl >> (8 * i)) & 0xffu) != 0);
        const float pr = vis ? __builtin_amdgcn_exp2f(sc[i] * scale_log2 - lse2) : 0.f;
        dsb[n >> 1][4 * (n & 1) + i] = static_cast<_Float16>(pr * (dp[i] - dsum));
      }
    }
    // dQ^T += K^T dS^T
#pragma unroll
    for (int t = 0; t < 8; ++t) {
#pragma unroll
      for (int m = 0; m < 2; ++m)
        acc[t] = mfma32(lds_runs_tr(Ks, kRStride, 16 * t, m, gr), dsb[m], acc[t]);
    }
  }
  if (q_abs >= T) return;
  const float scale = p.scale;
  if constexpr (VARLEN) {
    // dq|dk|dv row of the token; with tables, dQ is rounded to fp16 (the value an attention
    // backward would store) and rotated back (RoPE's backward) before its store.
    const int64_t tok = sh.tok0 + q_abs;
    uint16_t* dqrow = p.dq + tok * p.W + h * kD;
    const float* c = nullptr;
    const float* sn = nullptr;
    if (rope_rows(p, tok, &c, &sn)) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        f4 g1, g2, o1, o2;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          g1[i] = round_h(acc[t][i] * scale);
          g2[i] = round_h(acc[t + 4][i] * scale);
        }
        const int d = 16 * t + 4 * gr;
        rope_bwd4(c, sn, d, g1, g2, o1, o2);
        *reinterpret_cast<u32x2*>(dqrow + d) = u32x2{pack_h2(o1[0], o1[1]), pack_h2(o1[2], o1[3])};
        *reinterpret_cast<u32x2*>(dqrow + d + 64) =
            u32x2{pack_h2(o2[0], o2[1]), pack_h2(o2[2], o2[3])};
      }
      return;
    }
    if (p.cos != nullptr) {   // a token without a table row: no gradient reaches its input
#pragma unroll
      for (int t = 0; t < 8; ++t)
        *reinterpret_cast<u32x2*>(dqrow + 16 * t + 4 * gr) = u32x2{0u, 0u};
      return;
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const f4 o = acc[t] * scale;
      *reinterpret_cast<u32x2*>(dqrow + 16 * t + 4 * gr) = u32x2{pack_h2(o[0], o[1]),
                                                                   pack_h2(o[2], o[3])};
    }
  } else {
    uint16_t* dqrow = p.dq + ((static_cast<int64_t>(b) * p.NH + h) * p.T + q_abs) * kD;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const f4 o = acc[t] * scale;
      *reinterpret_cast<u32x2*>(dqrow + 16 * t + 4 * gr) = u32x2{pack_h2(o[0], o[1]),
                                                                   pack_h2(o[2], o[3])};
    }
  }
}

__device__ __forceinline__ void attn_bwd_dkdv(const AttnParams& p, const SeqHead& sh, int kb,
                                              unsigned char* smem) {
  _Float16* Qs = reinterpret_cast<_Float16*>(smem);
  _Float16* Ds = Qs + kBQ * kRStride;   // dO row-major
  float* lse2_s = reinterpret_cast<float*>(Ds + kBQ * kRStride);
  float* delta_s = lse2_s + kBQ;
  const int T = sh.len;
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int kl = lane & 15, gr = lane >> 4;
  const int key_abs = kb * kBK + 16 * w + kl;
  const int kc = min(key_abs, T - 1);
  const bool key_vis = key_abs < T && (sh.valid == nullptr || sh.valid[key_abs] != 0);
  const bool has_valid = sh.valid != nullptr;
  const uint16_t* krow = row_at(sh.k, kc, sh.ld_kv);
  const uint16_t* vrow = row_at(sh.v, kc, sh.ld_kv);
  const uint16_t* qbase = sh.q;
  const uint16_t* dobase = sh.dout;
  const float* lse_bh = sh.lse;
  const float* del_bh = sh.delta;
  const float scale_log2 = p.scale_log2;

  // K^T and V^T operands (B of S = Q K^T and of dP = dO V^T): lane holds row key of K / V,
  // dims 32s + 8gr .. +7
  h8 kf[4], vf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    kf[s] = *reinterpret_cast<const h8*>(krow + 32 * s + 8 * gr);
    vf[s] = *reinterpret_cast<const h8*>(vrow + 32 * s + 8 * gr);
  }
  f4 dk[8], dv[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) dk[t] = dv[t] = f4{0.f, 0.f, 0.f, 0.f};
  const int nqb = (T + kBQ - 1) / kBQ;
  TileRegs qr, dr;
  float lse_raw, del_raw;   // tested against T only when stored (see load_flag_raw)
  auto load_block = [&](int q0) {
    load_tile(qr, qbase, sh.ld_q, q0, T);
    load_tile(dr, dobase, sh.ld_o, q0, T);
    const int t = min(q0 + (static_cast<int>(threadIdx.x) & (kBQ - 1)), T - 1);
    lse_raw = lse_bh[t];
    del_raw = del_bh[t];
  };
  load_block(kb * kBQ);
  for (int qb = kb; qb < nqb; ++qb) {
    __syncthreads();
    store_tile(Qs, qr);   // Q^T, dO^T fragments read transposed
    store_tile(Ds, dr);
    if (threadIdx.x < kBQ) {
      const bool in = qb * kBQ + static_cast<int>(threadIdx.x) < T;
      lse2_s[threadIdx.x] = in ? lse_raw * kLog2e : INFINITY;
      delta_s[threadIdx.x] = in ? del_raw : 0.f;
    }
    __syncthreads();
    load_block((qb + 1) * kBQ);   // the next block (clamped past the end)
    issue_here();
    // Every (query, key) pair of an interior block is visible: the queries follow the keys,
    // lie below T, and no flags apply.
    const bool masked = qb == kb || has_valid || (qb + 1) * kBQ > T;
    h8 pb[2], dsb[2];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      h8 qa[4], da[4];
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        qa[s] = lds_h8(Qs + (16 * n + kl) * kRStride + 32 * s + 8 * gr);
        da[s] = lds_h8(Ds + (16 * n + kl) * kRStride + 32 * s + 8 * gr);
      }
      f4 sc = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        sc = mfma32(qa[s], kf[s], sc);
        dp = mfma32(da[s], vf[s], dp);
      }
      // C: rows = queries 16n + 4gr + i, column = this lane's key.  The per-query values are
      // read and every exponential computed unconditionally, the mask applied as a select:
      // a conditional LDS read would put each of them behind its own branch and wait.
      const f4 l2 = *reinterpret_cast<const f4*>(lse2_s + 16 * n + 4 * gr);
      const f4 dl = *reinterpret_cast<const f4*>(delta_s + 16 * n + 4 * gr);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int q_abs = qb * kBQ + 16 * n + 4 * gr + i;
        // (bitwise, not short-circuit: no per-lane branch)
        const bool vis = !masked | (key_vis & (key_abs <= q_abs) & (q_abs < T));
        const float e = __builtin_amdgcn_exp2f(sc[i] * scale_log2 - l2[i]);
        const float pr = vis ? e : 0.f;
        pb[n >> 1][4 * (n & 1) + i] = static_cast<_Float16>(pr);
        dsb[n >> 1][4 * (n & 1) + i] = static_cast<_Float16>(pr * (dp[i] - dl[i]));
      }
    }
    // dV^T += dO^T P, dK^T += Q^T dS  (contraction over the block's queries)
#pragma unroll
    for (int t = 0; t < 8; ++t) {
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        dv[t] = mfma32(lds_runs_tr(Ds, kRStride, 16 * t, m, gr), pb[m], dv[t]);
        dk[t] = mfma32(lds_runs_tr(Qs, kRStride, 16 * t, m, gr), dsb[m], dk[t]);
      }
    }
  }
  if (key_abs >= T) return;
  // C: rows = dims 16t + 4gr + i, column = this lane's key
  float* dkp = p.dk_part + (sh.plane + key_abs) * kD;
  float* dvp = p.dv_part + (sh.plane + key_abs) * kD;
  const float scale = p.scale;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    *reinterpret_cast<f4*>(dkp + 16 * t + 4 * gr) = dk[t] * scale;
    *reinterpret_cast<f4*>(dvp + 16 * t + 4 * gr) = dv[t];
  }
}

// Grid z = 2 * slots (as the forward's): z even -> dKdV of key block z/2 (block 0 sees the
// most query blocks), z odd -> dQ of query block nqb-1-z/2 (the last sees the most key blocks).
template <bool VARLEN>
__global__ __launch_bounds__(kAttnThreads) void attn_bwd_kernel(AttnParams p) {
  __shared__ __align__(16) unsigned char smem[kBwdLdsBytes];
  const int h = blockIdx.x, b = blockIdx.y;
  const SeqHead sh = seq_head<VARLEN>(p, b, h);
  const int nb = (sh.len + kBQ - 1) / kBQ;
  const int z = static_cast<int>(blockIdx.z);
  if ((z & 1) == 0) {
    if ((z >> 1) < nb) attn_bwd_dkdv(p, sh, z >> 1, smem);
  } else if (nb - 1 - (z >> 1) >= 0) {
    attn_bwd_dq<VARLEN>(p, sh, h, b, nb - 1 - (z >> 1), smem);
  }
}

// dK, dV of each key/value head: the sum of its NH/NKV query heads' partials, in head order.
__global__ __launch_bounds__(256) void attn_bwd_reduce_kernel(
    const float* __restrict__ dk_part, const float* __restrict__ dv_part,
    uint16_t* __restrict__ dk, uint16_t* __restrict__ dv, int64_t per_head, int NH, int NKV,
    int64_t n4) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // float4 index
  if (i >= n4) return;
  const int rep = NH / NKV;
  const int64_t heads4 = per_head / 4;              // float4 per head plane
  const int64_t bg = i / heads4, off = i % heads4;  // (b * NKV + g), offset in the plane
  const int64_t b = bg / NKV, g = bg % NKV;
  f4 sk = {0.f, 0.f, 0.f, 0.f}, sv = {0.f, 0.f, 0.f, 0.f};
  for (int r = 0; r < rep; ++r) {
    const int64_t src = (b * NH + g * rep + r) * heads4 + off;
    sk = sk + reinterpret_cast<const f4*>(dk_part)[src];
    sv = sv + reinterpret_cast<const f4*>(dv_part)[src];
  }
  reinterpret_cast<u32x2*>(dk)[i] = u32x2{pack_h2(sk[0], sk[1]), pack_h2(sk[2], sk[3])};
  reinterpret_cast<u32x2*>(dv)[i] = u32x2{pack_h2(sv[0], sv[1]), pack_h2(sv[2], sv[3])};
}

// Query heads per key/value head whose partials the reduce kernels load all at once (more take
// a loop that waits on each head's loads in turn).
constexpr int kMaxRep = 8;

// The varlen form of the reduce: item (token, key/value head g, 4-dim slice j of the first half)
// sums dims 4j..4j+3 and 4j+64..+67 of the dK and dV partials of the group's query heads (head
// order, as above), rounds to fp16 and writes them into the token's dq|dk|dv row, dK rotated
// back (RoPE's backward) when tables are given.
__global__ __launch_bounds__(256) void attn_bwd_reduce_varlen_kernel(AttnParams p,
                                                                      int64_t items) {
  const int64_t it = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (it >= items) return;
  const int j = static_cast<int>(it & 15);
  const int64_t tg = it >> 4;
  const int64_t tok = tg / p.NKV;
  const int g = static_cast<int>(tg - tok * p.NKV);
  const int rep = p.NH / p.NKV;
  const int d = 4 * j;
  // The table rows first, so that the position load and then the rows' go out beside the
  // partials' instead of after their sums (a token without a row reads row 0 and discards it).
  const float* c = p.cos;
  const float* sn = p.sin;
  const bool rope = p.cos != nullptr;
  const bool rope_row = rope && rope_rows(p, tok, &c, &sn);
  f4 c1 = {0.f, 0.f, 0.f, 0.f}, c2 = c1, s1 = c1, s2 = c1;
  if (rope) {
    c1 = *reinterpret_cast<const f4*>(c + d);
    c2 = *reinterpret_cast<const f4*>(c + d + 64);
    s1 = *reinterpret_cast<const f4*>(sn + d);
    s2 = *reinterpret_cast<const f4*>(sn + d + 64);
  }
  f4 k1 = {0.f, 0.f, 0.f, 0.f}, k2 = k1, v1 = k1, v2 = k1;
  if (rep <= kMaxRep) {
    // every partial's loads issued before the first add (a loop of loads and adds waited on
    // memory once per query head), unconditionally at a clamped head (loads under a test
    // were issued one test at a time), the adds then in head order as in the loop
    f4 a[kMaxRep][4];
#pragma unroll
    for (int r = 0; r < kMaxRep; ++r) {
      const int rr = r < rep ? r : rep - 1;
      const int64_t row = (static_cast<int64_t>(g * rep + rr) * p.M + tok) * kD;
      a[r][0] = *reinterpret_cast<const f4*>(p.dk_part + row + d);
      a[r][1] = *reinterpret_cast<const f4*>(p.dk_part + row + d + 64);
      a[r][2] = *reinterpret_cast<const f4*>(p.dv_part + row + d);
      a[r][3] = *reinterpret_cast<const f4*>(p.dv_part + row + d + 64);
    }
#pragma unroll
    for (int r = 0; r < kMaxRep; ++r) {
      if (r < rep) {
        k1 = k1 + a[r][0];
        k2 = k2 + a[r][1];
        v1 = v1 + a[r][2];
        v2 = v2 + a[r][3];
      }
    }
  } else {
    for (int r = 0; r < rep; ++r) {
      const int64_t row = (static_cast<int64_t>(g * rep + r) * p.M + tok) * kD;
      k1 = k1 + *reinterpret_cast<const f4*>(p.dk_part + row + d);
      k2 = k2 + *reinterpret_cast<const f4*>(p.dk_part + row + d + 64);
      v1 = v1 + *reinterpret_cast<const f4*>(p.dv_part + row + d);
      v2 = v2 + *reinterpret_cast<const f4*>(p.dv_part + row + d + 64);
    }
  }
  uint16_t* krow = p.dq + tok * p.W + (p.NH + g) * kD;
  uint16_t* vrow = p.dq + tok * p.W + (p.NH + p.NKV + g) * kD;
  if (rope) {
    if (rope_row) {
      f4 g1, g2;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        g1[i] = round_h(k1[i]);
        g2[i] = round_h(k2[i]);
      }
      rope_bwd4(c1, c2, s1, s2, g1, g2, k1, k2);
    } else {
      k1 = k2 = f4{0.f, 0.f, 0.f, 0.f};   // no table row: no gradient reaches the input
    }
  }
  *reinterpret_cast<u32x2*>(krow + d) = u32x2{pack_h2(k1[0], k1[1]), pack_h2(k1[2], k1[3])};
  *reinterpret_cast<u32x2*>(krow + d + 64) = u32x2{pack_h2(k2[0], k2[1]), pack_h2(k2[2], k2[3])};
  *reinterpret_cast<u32x2*>(vrow + d) = u32x2{pack_h2(v1[0], v1[1]), pack_h2(v1[2], v1[3])};
  *reinterpret_cast<u32x2*>(vrow + d + 64) = u32x2{pack_h2(v2[0], v2[1]), pack_h2(v2[2], v2[3])};
}

// Shape checks shared by the padded entry points.
int check_shape(int32_t B, int32_t T, int32_t NH, int32_t NKV, int32_t D, float scale) {
  if (B < 0 || T < 0 || NH <= 0 || NKV <= 0 || NH % NKV != 0 || D != kD) return kInvalid;
  if (!(scale > 0.f)) return kInvalid;
  if (B > 65535 || 2 * ((T + kBQ - 1) / kBQ) > 65535) return kInvalid;   // grid y, z limits
  if (static_cast<int64_t>(B) * NH * T * kD >= (int64_t{1} << 40)) return kInvalid;
  if (static_cast<int64_t>(T) * NH * kD >= (int64_t{1} << 31)) return kInvalid;  // row offsets
  return kOk;
}

// ... and by the varlen ones (the grid's z covers ceil(M/64) block slots, twice backward).
int check_varlen(int32_t B, int64_t M, int32_t NH, int32_t NKV, int32_t D, float scale) {
  if (B < 0 || M < 0 || NH <= 0 || NKV <= 0 || NH % NKV != 0 || D != kD) return kInvalid;
  if (!(scale > 0.f)) return kInvalid;
  if (B > 65535 || 2 * ((M + kBQ - 1) / kBQ) > 65535) return kInvalid;
  if (M * (NH + 2 * NKV) * kD >= (int64_t{1} << 31)) return kInvalid;   // 32-bit row offsets
  return kOk;
}

bool misaligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) != 0; }

AttnParams base_params(int32_t NH, int32_t NKV, float scale) {
  AttnParams p = {};
  p.NH = NH;
  p.NKV = NKV;
  p.scale = scale;
  p.scale_log2 = scale * kLog2e;
  p.rope_div = FastDiv(1);
  return p;
}

}  // namespace
}  // namespace soupk

using namespace soupk;

extern "C" __attribute__((visibility("default"))) int soupk_attention_fwd(
    const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint8_t* key_valid,
    uint16_t* out, float* lse, int32_t B, int32_t T, int32_t NH, int32_t NKV, int32_t D,
    float scale, void* stream) {
  const int rc = check_shape(B, T, NH, NKV, D, scale);
  if (rc != kOk) return rc;
  if (B == 0 || T == 0) return kOk;
  if (!q || !k || !v || !out || !lse) return kInvalid;
  for (const void* ptr : {static_cast<const void*>(q), static_cast<const void*>(k),
                          static_cast<const void*>(v), static_cast<const void*>(out)})
    if (misaligned16(ptr)) return kInvalid;
  AttnParams p = base_params(NH, NKV, scale);
  p.q = q;
  p.k = k;
  p.v = v;
  p.key_valid = key_valid;
  p.out = out;
  p.lse = lse;
  p.T = T;
  const dim3 grid(static_cast<unsigned>(NH), static_cast<unsigned>(B),
                  static_cast<unsigned>((T + kBQ - 1) / kBQ));
  return launch_kernel(attn_fwd_kernel<false>, grid, dim3(kAttnThreads),
                       static_cast<hipStream_t>(stream), p);
}

extern "C" __attribute__((visibility("default"))) int soupk_attention_bwd(
    const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint8_t* key_valid,
    const uint16_t* out, const uint16_t* dout, const float* lse, float* workspace,
    uint16_t* dq, uint16_t* dk, uint16_t* dv, int32_t B, int32_t T, int32_t NH, int32_t NKV,
    int32_t D, float scale, void* stream) {
  const int rc0 = check_shape(B, T, NH, NKV, D, scale);
  if (rc0 != kOk) return rc0;
  if (B == 0 || T == 0) return kOk;
  if (!q || !k || !v || !out || !dout || !lse || !workspace || !dq || !dk || !dv)
    return kInvalid;
  for (const void* ptr : {static_cast<const void*>(q), static_cast<const void*>(k),
                          static_cast<const void*>(v), static_cast<const void*>(out),
                          static_cast<const void*>(dout), static_cast<const void*>(workspace),
                          static_cast<const void*>(dq), static_cast<const void*>(dk),
                          static_cast<const void*>(dv)})
    if (misaligned16(ptr)) return kInvalid;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t per_head = static_cast<int64_t>(T) * kD;
  const int64_t part = static_cast<int64_t>(B) * NH * per_head;  // floats per partial
  // workspace: delta [B*NH*T] (padded to 4 floats), then the dK and dV partials
  const int64_t delta_n = (static_cast<int64_t>(B) * NH * T + 3) / 4 * 4;
  AttnParams p = base_params(NH, NKV, scale);
  p.q = q;
  p.k = k;
  p.v = v;
  p.key_valid = key_valid;
  p.out = const_cast<uint16_t*>(out);
  p.dout = dout;
  p.lse = const_cast<float*>(lse);
  p.delta = workspace;
  p.dk_part = workspace + delta_n;
  p.dv_part = p.dk_part + part;
  p.dq = dq;
  p.T = T;
  const int nb = (T + kBQ - 1) / kBQ;
  const dim3 grid(static_cast<unsigned>(NH), static_cast<unsigned>(B), static_cast<unsigned>(nb));
  int rc = launch_kernel(attn_bwd_delta_kernel, grid, dim3(kAttnThreads), st, out, dout,
                         p.delta, T, NH);
  if (rc != kOk) return rc;
  const dim3 grid2(static_cast<unsigned>(NH), static_cast<unsigned>(B),
                   static_cast<unsigned>(2 * nb));
  rc = launch_kernel(attn_bwd_kernel<false>, grid2, dim3(kAttnThreads), st, p);
  if (rc != kOk) return rc;
  const int64_t n4 = static_cast<int64_t>(B) * NKV * per_head / 4;
  return launch_kernel(attn_bwd_reduce_kernel, dim3(static_cast<unsigned>((n4 + 255) / 256)),
                       dim3(256), st, p.dk_part, p.dv_part, dk, dv, per_head, NH, NKV, n4);
}

extern "C" __attribute__((visibility("default"))) int soupk_attention_varlen_fwd(
    const uint16_t* qkv, const int32_t* cu_seqlens, int32_t B, uint16_t* out, float* lse,
    int64_t M, int32_t NH, int32_t NKV, int32_t D, float scale, void* stream) {
  const int rc = check_varlen(B, M, NH, NKV, D, scale);
  if (rc != kOk) return rc;
  if (B == 0 || M == 0) return kOk;
  if (!qkv || !cu_seqlens || !out || !lse) return kInvalid;
  if (misaligned16(qkv) || misaligned16(out)) return kInvalid;
  AttnParams p = base_params(NH, NKV, scale);
  p.q = qkv;
  p.cu = cu_seqlens;
  p.out = out;
  p.lse = lse;
  p.M = M;
  p.W = static_cast<int64_t>(NH + 2 * NKV) * kD;
  const int slots = static_cast<int>((M + kBQ - 1) / kBQ);
  const dim3 grid(static_cast<unsigned>(NH), static_cast<unsigned>(B),
                  static_cast<unsigned>(slots));
  return launch_kernel(attn_fwd_kernel<true>, grid, dim3(kAttnThreads),
                       static_cast<hipStream_t>(stream), p);
}

extern "C" __attribute__((visibility("default"))) int soupk_attention_varlen_bwd(
    const uint16_t* qkv, const int32_t* cu_seqlens, int32_t B, const uint16_t* out,
    const uint16_t* dout, const float* lse, const float* cos, const float* sin,
    const int64_t* pos, int64_t pos_slots, int32_t T_rope, float* workspace, uint16_t* dqkv,
    int64_t M, int32_t NH, int32_t NKV, int32_t D, float scale, void* stream) {
  const int rc0 = check_varlen(B, M, NH, NKV, D, scale);
  if (rc0 != kOk) return rc0;
  const bool rope = cos != nullptr || sin != nullptr || pos != nullptr;
  if (rope && (!cos || !sin || !pos || T_rope <= 0 || pos_slots < 0 ||
               pos_slots >= (int64_t{1} << 31) || misaligned16(cos) || misaligned16(sin)))
    return kInvalid;
  if (M == 0) return kOk;
  if (!qkv || !cu_seqlens || !out || !dout || !lse || !workspace || !dqkv) return kInvalid;
  for (const void* ptr : {static_cast<const void*>(qkv), static_cast<const void*>(out),
                          static_cast<const void*>(dout), static_cast<const void*>(workspace),
                          static_cast<const void*>(dqkv)})
    if (misaligned16(ptr)) return kInvalid;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t part = M * NH * kD;
  const int64_t delta_n = (M * NH + 3) / 4 * 4;
  AttnParams p = base_params(NH, NKV, scale);
  p.q = qkv;
  p.cu = cu_seqlens;
  p.out = const_cast<uint16_t*>(out);
  p.dout = dout;
  p.lse = const_cast<float*>(lse);
  p.delta = workspace;
  p.dk_part = workspace + delta_n;
  p.dv_part = p.dk_part + part;
  p.dq = dqkv;
  p.M = M;
  p.W = static_cast<int64_t>(NH + 2 * NKV) * kD;
  if (rope) {
    p.cos = cos;
    p.sin = sin;
    p.pos = pos;
    p.pos_slots = pos_slots;
    p.rope_div = FastDiv(static_cast<uint32_t>(T_rope));
  }
  // With cu_seqlens running from 0 to M, every token row of dq|dk|dv is written: dQ by the dQ
  // workgroups of its sequence, dK and dV by the reduce over all M tokens.  (A token outside
  // every sequence gets an unspecified row; every access stays inside the buffers.)
  // D = rowsum(dO * O) over all M tokens: the padded delta kernel over one row of M "positions"
  // (its lse / D plane index (b*NH + h)*T + t is h*M + t for b = 0, T = M).
  const int nbm = static_cast<int>((M + kBQ - 1) / kBQ);   // (check_varlen: 2 * nbm <= 65535)
  int rc = launch_kernel(attn_bwd_delta_kernel,
                         dim3(static_cast<unsigned>(NH), 1u, static_cast<unsigned>(nbm)),
                         dim3(kAttnThreads), st, out, dout, p.delta, static_cast<int>(M), NH);
  if (rc != kOk) return rc;
  if (B > 0) {
    const int slots = nbm;
    const dim3 grid(static_cast<unsigned>(NH), static_cast<unsigned>(B),
                    static_cast<unsigned>(2 * slots));
    rc = launch_kernel(attn_bwd_kernel<true>, grid, dim3(kAttnThreads), st, p);
    if (rc != kOk) return rc;
  }
  const int64_t items = M * NKV * 16;
  return launch_kernel(attn_bwd_reduce_varlen_kernel,
                       dim3(static_cast<unsigned>((items + 255) / 256)), dim3(256), st, p, items);
}
