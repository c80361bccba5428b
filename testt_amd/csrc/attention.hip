// Causal grouped-query attention over the padded [B, heads, T, D] layout, forward and backward,
// for head_dim 128 on gfx950 MFMA (v_mfma_f32_16x16x16_f16).
//
// Replaces torch's scaled_dot_product_attention in the layer loop of the reference's
// fused_forward (solution/model.py:246-247, transformers' sdpa_attention_forward with the causal
// + key-padding mask of create_causal_mask): query i of a row attends to key j iff j <= i and
// key j is a real token (key_valid[b, j] != 0, or every key when key_valid is NULL).
//
// Forward (flash attention, online softmax): a workgroup is 4 wavefronts and 64 queries of one
// (batch, head); wavefront w owns queries 16w..16w+15.  Key blocks of 64 rows are staged in LDS
// -- K row-major, V transposed (key-contiguous) -- and each wavefront computes
//   S^T (64 keys x 16 queries) = K Q^T       (A = K from LDS, B = Q^T from registers)
// so that, in the MFMA output layout, lane l holds the scores of query l%16 for keys
// 16n + 4(l/16) + i: exactly the B operand of
//   O^T (128 x 16) += V^T P^T                 (A = V^T from LDS, B = P^T from registers),
// and the online-softmax rescale of O^T is local to the lane (its query is l%16 too).  The four
// lanes of a query (l%16 + 16r) combine their block maxima with two cross-row shuffles; their
// partial sums are combined once, at the end.  Scores are kept in base 2:
// x = s * scale * log2(e), p = 2^(x - m).  The output is written token-major,
// out[(b*T + t), h*D + d], the layout the o-projection GEMM reads, and the per-query
// log-sum-exp (natural log) for the backward pass; a query with no visible key gets output 0
// and lse = +inf (so its backward probabilities are 0).
//
// MFMA operand layouts (16x16x16, checked on the device): A[16 x 16]: lane l holds row l%16,
// k = 4(l/16)..+3; B[16 x 16]: lane l holds column l%16, k = 4(l/16)..+3; C: lane l holds
// column l%16, rows 4(l/16)..+3.

#include "soupk_common.hpp"

namespace soupk {
namespace {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kD = 128;               // head dim
constexpr int kBQ = 64;               // queries per workgroup (4 wavefronts x 16)
constexpr int kBK = 64;               // keys per block
constexpr int kAttnThreads = 256;
constexpr int kKStride = kD + 8;      // Ks row stride (halves): 272 B, conflict-free 8-B reads
constexpr int kVStride = kBK + 8;     // Vt row stride (halves): 144 B

__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ h4 lds_h4(const _Float16* p) {
  return *reinterpret_cast<const h4*>(p);
}

// Stage key block kb of (b, g): Ks[key][d] row-major, Vt[d][key] transposed, and the 64 key
// flags (1 = visible).  Rows past T read as zeros and are flagged invisible.
__device__ __forceinline__ void stage_kv(_Float16* Ks, _Float16* Vt, uint8_t* kflag,
                                         const uint16_t* __restrict__ kbase,
                                         const uint16_t* __restrict__ vbase,
                                         const uint8_t* __restrict__ valid, int key0, int T) {
  const int tid = threadIdx.x;
  // K: 64 keys x 16 chunks of 8 halves, 4 chunks per thread
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int c = tid + kAttnThreads * r;
    const int key = c >> 4, dc = c & 15;
    const int t = key0 + key;
    u32x4 w = {0u, 0u, 0u, 0u};
    if (t < T) w = *reinterpret_cast<const u32x4*>(kbase + static_cast<int64_t>(t) * kD + 8 * dc);
    *reinterpret_cast<u32x4*>(Ks + key * kKStride + 8 * dc) = w;
  }
  // V transposed: 32 key pairs x 16 chunks of 8 d; per item two 16-B row loads and eight
  // 4-byte LDS words (the pair's values at one d).
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int item = tid + kAttnThreads * r;
    const int kp = item & 31, dc = item >> 5;
    const int t0 = key0 + 2 * kp;
    u32x4 a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
    if (t0 < T) a = *reinterpret_cast<const u32x4*>(vbase + static_cast<int64_t>(t0) * kD + 8 * dc);
    if (t0 + 1 < T)
      b = *reinterpret_cast<const u32x4*>(vbase + static_cast<int64_t>(t0 + 1) * kD + 8 * dc);
    const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
    uint32_t* col = reinterpret_cast<uint32_t*>(Vt + (8 * dc) * kVStride + 2 * kp);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // d = 8dc + 2j (low halves) and 8dc + 2j + 1 (high halves)
      col[(2 * j) * (kVStride / 2)] = (aw[j] & 0xffffu) | (bw[j] << 16);
      col[(2 * j + 1) * (kVStride / 2)] = (aw[j] >> 16) | (bw[j] & 0xffff0000u);
    }
  }
  if (tid < kBK) {
    const int t = key0 + tid;
    kflag[tid] = (t < T && (valid == nullptr || valid[t] != 0)) ? 1 : 0;
  }
}

__global__ __launch_bounds__(kAttnThreads) void attn_fwd_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint8_t* __restrict__ key_valid,
    uint16_t* __restrict__ out, float* __restrict__ lse, int T, int NH, int NKV,
    float scale_log2) {
  __shared__ __align__(16) _Float16 Ks[kBK * kKStride];
  __shared__ __align__(16) _Float16 Vt[kD * kVStride];
  __shared__ __align__(16) uint8_t kflag[kBK];
  const int nqb = (T + kBQ - 1) / kBQ;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x);  // longest (latest) blocks first
  const int h = blockIdx.y, b = blockIdx.z;
  const int g = h / (NH / NKV);
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int ql = lane & 15, kq = lane >> 4;
  const int q_abs = qb * kBQ + 16 * w + ql;
  const uint16_t* qrow = q + ((static_cast<int64_t>(b) * NH + h) * T + min(q_abs, T - 1)) * kD;
  const uint16_t* kbase = k + (static_cast<int64_t>(b) * NKV + g) * T * kD;
  const uint16_t* vbase = v + (static_cast<int64_t>(b) * NKV + g) * T * kD;
  const uint8_t* valid = key_valid != nullptr ? key_valid + static_cast<int64_t>(b) * T : nullptr;

  // Q^T operand: 8 k-steps of 16 dims, lane holds Q[q][16s + 4kq .. +3]
  h4 qf[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    const u32x2 wq = *reinterpret_cast<const u32x2*>(qrow + 16 * s + 4 * kq);
    qf[s] = __builtin_bit_cast(h4, wq);
  }
  f4 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, lsum = 0.f;

  const int kb_last = min(qb, (T - 1) / kBK);
  for (int kb = 0; kb <= kb_last; ++kb) {
    __syncthreads();
    stage_kv(Ks, Vt, kflag, kbase, vbase, valid, kb * kBK, T);
    __syncthreads();
    // S^T for the 4 key tiles
    f4 s4[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      f4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 8; ++s)
        c = mfma16(lds_h4(Ks + (16 * n + ql) * kKStride + 16 * s + 4 * kq), qf[s], c);
      s4[n] = c;
    }
    // mask, scale, block max
    float x[4][4];
    float mx = -INFINITY;
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const uint32_t fl = *reinterpret_cast<const uint32_t*>(kflag + 16 * n + 4 * kq);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kb * kBK + 16 * n + 4 * kq + i;
        const bool vis = key <= q_abs && ((fl >> (8 * i)) & 0xffu) != 0;
        x[n][i] = vis ? s4[n][i] * scale_log2 : -INFINITY;
        mx = fmaxf(mx, x[n][i]);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, kWave));
    mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
    const float m_new = fmaxf(m, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - m_use);
    m = m_new;
    float ps = 0.f;
    h4 pb[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = __builtin_amdgcn_exp2f(x[n][i] - m_use);  // 2^-inf = 0
        ps += p;
        pb[n][i] = static_cast<_Float16>(p);
      }
    }
    lsum = lsum * alpha + ps;
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = acc[t] * alpha;
    // O^T += V^T P^T
#pragma unroll
    for (int n = 0; n < 4; ++n) {
#pragma unroll
      for (int t = 0; t < 8; ++t)
        acc[t] = mfma16(lds_h4(Vt + (16 * t + ql) * kVStride + 16 * n + 4 * kq), pb[n], acc[t]);
    }
  }
  float l_tot = lsum + __shfl_xor(lsum, 16, kWave);
  l_tot = l_tot + __shfl_xor(l_tot, 32, kWave);
  if (q_abs >= T) return;
  const float inv = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  uint16_t* orow = out + (static_cast<int64_t>(b) * T + q_abs) * (static_cast<int64_t>(NH) * kD) +
                   h * kD;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const f4 o = acc[t] * inv;
    *reinterpret_cast<u32x2*>(orow + 16 * t + 4 * kq) = u32x2{pack_h2(o[0], o[1]),
                                                                pack_h2(o[2], o[3])};
  }
  if (kq == 0)
    lse[(static_cast<int64_t>(b) * NH + h) * T + q_abs] =
        l_tot > 0.f ? (m + log2f(l_tot)) * kLn2 : INFINITY;
}

// ---- backward ------------------------------------------------------------------------------
// With P = softmax of the scaled scores (recomputed from the saved log-sum-exp), dO the output
// gradient and D = rowsum(dO * O):  dP = dO V^T,  dS = P * (dP - D),  dQ = scale * dS K,
// dK = scale * dS^T Q,  dV = P^T dO.  Three launches:
//   attn_bwd_dq_kernel   (b, head, 64 queries): D for its queries (written for the next kernel),
//                        then over its key blocks S^T = K Q^T, dP^T = V dO^T (the forward's
//                        orientation: query = lane % 16), dQ^T += K^T dS^T;
//   attn_bwd_dkdv_kernel (b, head, 64 keys): over the query blocks that see them,
//                        S = Q K^T, dP = dO V^T (key = lane % 16), dV^T += dO^T P,
//                        dK^T += Q^T dS, into fp32 partials per query head;
//   attn_bwd_reduce_kernel: dK, dV of a key/value head = the sum of its query heads' partials
//                        (a fixed order: deterministic), fp16.
// Every operand a MFMA reads from LDS is laid out so that a lane's four k-values are 8
// contiguous bytes: row-major tiles for operands contracted over the head dim, transposed
// (row-contiguous) tiles for operands contracted over queries or keys.

// Two rows (2rp, 2rp+1) x 8 dims of a [64 x 128] tile: row-major into `rm` (stride kKStride)
// and/or transposed into `tr` ([128][kVStride]), from one pair of 16-byte loads.
template <bool RM, bool TR>
__device__ __forceinline__ void stage_pair(_Float16* rm, _Float16* tr, u32x4 a, u32x4 b, int rp,
                                           int dc) {
  if constexpr (RM) {
    *reinterpret_cast<u32x4*>(rm + (2 * rp) * kKStride + 8 * dc) = a;
    *reinterpret_cast<u32x4*>(rm + (2 * rp + 1) * kKStride + 8 * dc) = b;
  }
  if constexpr (TR) {
    const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, bw[4] = {b.x, b.y, b.z, b.w};
    uint32_t* col = reinterpret_cast<uint32_t*>(tr + (8 * dc) * kVStride + 2 * rp);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      col[(2 * j) * (kVStride / 2)] = (aw[j] & 0xffffu) | (bw[j] << 16);
      col[(2 * j + 1) * (kVStride / 2)] = (aw[j] >> 16) | (bw[j] & 0xffff0000u);
    }
  }
}

// Stage 64 rows of 128 fp16 (row r at src + r*stride; rows r0+r >= nrows read as 0).
template <bool RM, bool TR>
__device__ __forceinline__ void stage_tile(_Float16* rm, _Float16* tr,
                                           const uint16_t* __restrict__ src, int64_t stride,
                                           int r0, int nrows) {
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int item = threadIdx.x + kAttnThreads * r;
    const int rp = item & 31, dc = item >> 5;
    const int t0 = r0 + 2 * rp;
    u32x4 a = {0u, 0u, 0u, 0u}, b = {0u, 0u, 0u, 0u};
    if (t0 < nrows) a = *reinterpret_cast<const u32x4*>(src + t0 * stride + 8 * dc);
    if (t0 + 1 < nrows) b = *reinterpret_cast<const u32x4*>(src + (t0 + 1) * stride + 8 * dc);
    stage_pair<RM, TR>(rm, tr, a, b, rp, dc);
  }
}

__global__ __launch_bounds__(kAttnThreads) void attn_bwd_dq_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint8_t* __restrict__ key_valid,
    const uint16_t* __restrict__ out, const uint16_t* __restrict__ dout,
    const float* __restrict__ lse, float* __restrict__ delta, uint16_t* __restrict__ dq, int T,
    int NH, int NKV, float scale, float scale_log2) {
  __shared__ __align__(16) _Float16 Ks[kBK * kKStride];
  __shared__ __align__(16) _Float16 Vs[kBK * kKStride];
  __shared__ __align__(16) _Float16 Kt[kD * kVStride];
  __shared__ __align__(16) uint8_t kflag[kBK];
  const int nqb = (T + kBQ - 1) / kBQ;
  const int qb = nqb - 1 - static_cast<int>(blockIdx.x);
  const int h = blockIdx.y, b = blockIdx.z;
  const int g = h / (NH / NKV);
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int ql = lane & 15, kq = lane >> 4;
  const int q_abs = qb * kBQ + 16 * w + ql;
  const int qc = min(q_abs, T - 1);
  const int64_t HD = static_cast<int64_t>(NH) * kD;
  const uint16_t* qrow = q + ((static_cast<int64_t>(b) * NH + h) * T + qc) * kD;
  const uint16_t* orow = out + (static_cast<int64_t>(b) * T + qc) * HD + h * kD;
  const uint16_t* dorow = dout + (static_cast<int64_t>(b) * T + qc) * HD + h * kD;
  const uint16_t* kbase = k + (static_cast<int64_t>(b) * NKV + g) * T * kD;
  const uint16_t* vbase = v + (static_cast<int64_t>(b) * NKV + g) * T * kD;
  const uint8_t* valid = key_valid != nullptr ? key_valid + static_cast<int64_t>(b) * T : nullptr;

  h4 qf[8], dof[8];
  float dsum = 0.f;
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    qf[s] = __builtin_bit_cast(h4, *reinterpret_cast<const u32x2*>(qrow + 16 * s + 4 * kq));
    dof[s] = __builtin_bit_cast(h4, *reinterpret_cast<const u32x2*>(dorow + 16 * s + 4 * kq));
    const h4 of = __builtin_bit_cast(h4, *reinterpret_cast<const u32x2*>(orow + 16 * s + 4 * kq));
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dsum = dsum + static_cast<float>(dof[s][i]) * static_cast<float>(of[i]);
  }
  dsum = dsum + __shfl_xor(dsum, 16, kWave);
  dsum = dsum + __shfl_xor(dsum, 32, kWave);
  const float lse_q = lse[(static_cast<int64_t>(b) * NH + h) * T + qc];
  const float lse2 = lse_q * kLog2e;  // +inf: no visible key, every p = 0
  if (kq == 0 && q_abs < T) delta[(static_cast<int64_t>(b) * NH + h) * T + q_abs] = dsum;

  f4 acc[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) acc[t] = f4{0.f, 0.f, 0.f, 0.f};
  const int kb_last = min(qb, (T - 1) / kBK);
  for (int kb = 0; kb <= kb_last; ++kb) {
    __syncthreads();
    stage_tile<true, true>(Ks, Kt, kbase, kD, kb * kBK, T);
    stage_tile<true, false>(Vs, nullptr, vbase, kD, kb * kBK, T);
    if (threadIdx.x < kBK) {
      const int t = kb * kBK + threadIdx.x;
      kflag[threadIdx.x] = (t < T && (valid == nullptr || valid[t] != 0)) ? 1 : 0;
    }
    __syncthreads();
    h4 dsb[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      f4 sc = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        sc = mfma16(lds_h4(Ks + (16 * n + ql) * kKStride + 16 * s + 4 * kq), qf[s], sc);
        dp = mfma16(lds_h4(Vs + (16 * n + ql) * kKStride + 16 * s + 4 * kq), dof[s], dp);
      }
      const uint32_t fl = *reinterpret_cast<const uint32_t*>(kflag + 16 * n + 4 * kq);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kb * kBK + 16 * n + 4 * kq + i;
        const bool vis = key <= q_abs && ((fl >> (8 * i)) & 0xffu) != 0;
        const float p = vis ? __builtin_amdgcn_exp2f(sc[i] * scale_log2 - lse2) : 0.f;
        dsb[n][i] = static_cast<_Float16>(p * (dp[i] - dsum));
      }
    }
#pragma unroll
    for (int n = 0; n < 4; ++n) {
#pragma unroll
      for (int t = 0; t < 8; ++t)
        acc[t] = mfma16(lds_h4(Kt + (16 * t + ql) * kVStride + 16 * n + 4 * kq), dsb[n], acc[t]);
    }
  }
  if (q_abs >= T) return;
  uint16_t* dqrow = dq + ((static_cast<int64_t>(b) * NH + h) * T + q_abs) * kD;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const f4 o = acc[t] * scale;
    *reinterpret_cast<u32x2*>(dqrow + 16 * t + 4 * kq) = u32x2{pack_h2(o[0], o[1]),
                                                                 pack_h2(o[2], o[3])};
  }
}

__global__ __launch_bounds__(kAttnThreads) void attn_bwd_dkdv_kernel(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const uint8_t* __restrict__ key_valid,
    const uint16_t* __restrict__ dout, const float* __restrict__ lse,
    const float* __restrict__ delta, float* __restrict__ dk_part, float* __restrict__ dv_part,
    int T, int NH, int NKV, float scale, float scale_log2) {
  __shared__ __align__(16) _Float16 Qs[kBQ * kKStride];
  __shared__ __align__(16) _Float16 Qt[kD * kVStride];
  __shared__ __align__(16) _Float16 Ds[kBQ * kKStride];   // dO row-major
  __shared__ __align__(16) _Float16 Dt[kD * kVStride];    // dO transposed
  __shared__ float lse2_s[kBQ], delta_s[kBQ];
  const int nkb = (T + kBK - 1) / kBK;
  const int kb = static_cast<int>(blockIdx.x);  // block 0 sees the most query blocks
  const int h = blockIdx.y, b = blockIdx.z;
  const int g = h / (NH / NKV);
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int kl = lane & 15, qq = lane >> 4;
  const int key_abs = kb * kBK + 16 * w + kl;
  const int kc = min(key_abs, T - 1);
  const bool key_vis = key_abs < T && (key_valid == nullptr ||
                                       key_valid[static_cast<int64_t>(b) * T + key_abs] != 0);
  const int64_t HD = static_cast<int64_t>(NH) * kD;
  const uint16_t* krow = k + ((static_cast<int64_t>(b) * NKV + g) * T + kc) * kD;
  const uint16_t* vrow = v + ((static_cast<int64_t>(b) * NKV + g) * T + kc) * kD;
  const uint16_t* qbase = q + (static_cast<int64_t>(b) * NH + h) * T * kD;
  const uint16_t* dobase = dout + static_cast<int64_t>(b) * T * HD + h * kD;
  const float* lse_bh = lse + (static_cast<int64_t>(b) * NH + h) * T;
  const float* del_bh = delta + (static_cast<int64_t>(b) * NH + h) * T;

  // K^T and V^T operands (B of S = Q K^T and of dP = dO V^T): lane holds row key of K / V,
  // dims 16s + 4qq .. +3
  h4 kf[8], vf[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) {
    kf[s] = __builtin_bit_cast(h4, *reinterpret_cast<const u32x2*>(krow + 16 * s + 4 * qq));
    vf[s] = __builtin_bit_cast(h4, *reinterpret_cast<const u32x2*>(vrow + 16 * s + 4 * qq));
  }
  f4 dk[8], dv[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) dk[t] = dv[t] = f4{0.f, 0.f, 0.f, 0.f};
  (void)nkb;
  const int nqb = (T + kBQ - 1) / kBQ;
  for (int qb = kb; qb < nqb; ++qb) {
    __syncthreads();
    stage_tile<true, true>(Qs, Qt, qbase, kD, qb * kBQ, T);
    stage_tile<true, true>(Ds, Dt, dobase, HD, qb * kBQ, T);
    if (threadIdx.x < kBQ) {
      const int t = qb * kBQ + threadIdx.x;
      lse2_s[threadIdx.x] = t < T ? lse_bh[t] * kLog2e : INFINITY;
      delta_s[threadIdx.x] = t < T ? del_bh[t] : 0.f;
    }
    __syncthreads();
    h4 pb[4], dsb[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      f4 sc = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        sc = mfma16(lds_h4(Qs + (16 * n + kl) * kKStride + 16 * s + 4 * qq), kf[s], sc);
        dp = mfma16(lds_h4(Ds + (16 * n + kl) * kKStride + 16 * s + 4 * qq), vf[s], dp);
      }
      // C: rows = queries 16n + 4qq + i, column = this lane's key
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int qi = 16 * n + 4 * qq + i;
        const int q_abs = qb * kBQ + qi;
        const bool vis = key_vis && key_abs <= q_abs && q_abs < T;
        const float p = vis ? __builtin_amdgcn_exp2f(sc[i] * scale_log2 - lse2_s[qi]) : 0.f;
        pb[n][i] = static_cast<_Float16>(p);
        dsb[n][i] = static_cast<_Float16>(p * (dp[i] - delta_s[qi]));
      }
    }
    // dV^T += dO^T P, dK^T += Q^T dS  (k = queries)
#pragma unroll
    for (int n = 0; n < 4; ++n) {
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        dv[t] = mfma16(lds_h4(Dt + (16 * t + kl) * kVStride + 16 * n + 4 * qq), pb[n], dv[t]);
        dk[t] = mfma16(lds_h4(Qt + (16 * t + kl) * kVStride + 16 * n + 4 * qq), dsb[n], dk[t]);
      }
    }
  }
  if (key_abs >= T) return;
  // C: rows = dims 16t + 4qq + i, column = this lane's key
  float* dkp = dk_part + ((static_cast<int64_t>(b) * NH + h) * T + key_abs) * kD;
  float* dvp = dv_part + ((static_cast<int64_t>(b) * NH + h) * T + key_abs) * kD;
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    *reinterpret_cast<f4*>(dkp + 16 * t + 4 * qq) = dk[t] * scale;
    *reinterpret_cast<f4*>(dvp + 16 * t + 4 * qq) = dv[t];
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

}  // namespace
}  // namespace soupk

using namespace soupk;

extern "C" __attribute__((visibility("default"))) int soupk_attention_fwd(
    const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint8_t* key_valid,
    uint16_t* out, float* lse, int32_t B, int32_t T, int32_t NH, int32_t NKV, int32_t D,
    float scale, void* stream) {
  if (B < 0 || T < 0 || NH <= 0 || NKV <= 0 || NH % NKV != 0 || D != kD) return kInvalid;
  if (!(scale > 0.f)) return kInvalid;
  if (B == 0 || T == 0) return kOk;
  if (!q || !k || !v || !out || !lse) return kInvalid;
  for (const void* p : {static_cast<const void*>(q), static_cast<const void*>(k),
                        static_cast<const void*>(v), static_cast<const void*>(out)})
    if (reinterpret_cast<uintptr_t>(p) & 15) return kInvalid;
  if (static_cast<int64_t>(B) * NH * T * kD >= (int64_t{1} << 40)) return kInvalid;
  const dim3 grid(static_cast<unsigned>((T + kBQ - 1) / kBQ), static_cast<unsigned>(NH),
                  static_cast<unsigned>(B));
  return launch_kernel(attn_fwd_kernel, grid, dim3(kAttnThreads),
                       static_cast<hipStream_t>(stream), q, k, v, key_valid, out, lse, T, NH,
                       NKV, scale * kLog2e);
}

extern "C" __attribute__((visibility("default"))) int soupk_attention_bwd(
    const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint8_t* key_valid,
    const uint16_t* out, const uint16_t* dout, const float* lse, float* workspace,
    uint16_t* dq, uint16_t* dk, uint16_t* dv, int32_t B, int32_t T, int32_t NH, int32_t NKV,
    int32_t D, float scale, void* stream) {
  if (B < 0 || T < 0 || NH <= 0 || NKV <= 0 || NH % NKV != 0 || D != kD) return kInvalid;
  if (!(scale > 0.f)) return kInvalid;
  if (B == 0 || T == 0) return kOk;
  if (!q || !k || !v || !out || !dout || !lse || !workspace || !dq || !dk || !dv)
    return kInvalid;
  for (const void* p : {static_cast<const void*>(q), static_cast<const void*>(k),
                        static_cast<const void*>(v), static_cast<const void*>(out),
                        static_cast<const void*>(dout), static_cast<const void*>(workspace),
                        static_cast<const void*>(dq), static_cast<const void*>(dk),
                        static_cast<const void*>(dv)})
    if (reinterpret_cast<uintptr_t>(p) & 15) return kInvalid;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int64_t per_head = static_cast<int64_t>(T) * kD;
  const int64_t part = static_cast<int64_t>(B) * NH * per_head;  // floats per partial
  // workspace: delta [B*NH*T] (padded to 4 floats), then the dK and dV partials
  const int64_t delta_n = (static_cast<int64_t>(B) * NH * T + 3) / 4 * 4;
  float* delta = workspace;
  float* dk_part = workspace + delta_n;
  float* dv_part = dk_part + part;
  const int nb = (T + kBQ - 1) / kBQ;
  const dim3 grid(static_cast<unsigned>(nb), static_cast<unsigned>(NH), static_cast<unsigned>(B));
  int rc = launch_kernel(attn_bwd_dq_kernel, grid, dim3(kAttnThreads), st, q, k, v, key_valid,
                         out, dout, lse, delta, dq, T, NH, NKV, scale, scale * kLog2e);
  if (rc != kOk) return rc;
  rc = launch_kernel(attn_bwd_dkdv_kernel, grid, dim3(kAttnThreads), st, q, k, v, key_valid,
                     dout, lse, delta, dk_part, dv_part, T, NH, NKV, scale, scale * kLog2e);
  if (rc != kOk) return rc;
  const int64_t n4 = static_cast<int64_t>(B) * NKV * per_head / 4;
  return launch_kernel(attn_bwd_reduce_kernel, dim3(static_cast<unsigned>((n4 + 255) / 256)),
                       dim3(256), st, dk_part, dv_part, dk, dv, per_head, NH, NKV, n4);
}
