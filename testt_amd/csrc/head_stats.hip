// Vocab-head online softmax: per-row lse, entropy, token loss, argmax hit, and the in-place fp16
// gradient (softmax - onehot) * grad_scale of the chunk logits.
//
// Reference: solution/head.py:34-76 (head_stats_grad_kernel), launched per 256-row chunk from
// FusedHeadLoss.forward, solution/head.py:105-114.
//
// Mapping (gfx950): one workgroup of 1024 threads (16 wavefronts, a whole CU) per logits row.
// Sweep 1 streams the row once with 16-byte loads (a wave reads 1 KiB per load instruction)
// and keeps per lane a running max m, sum(e) and sum(e*z) with e = exp(z - m), plus the first
// column where the max was reached (lanes visit their columns in increasing order, so a strict
// '>' keeps the first occurrence; the cross-lane merge breaks value ties on the smaller column,
// which is torch.argmax's first-maximum rule).  The rescale of the running sums happens once
// per 8-value chunk, only when the chunk raises the max.  The 16 wave results merge through
// LDS.  Sweep 2 (labelled rows only) re-reads the row, now resident in L2 / the Infinity Cache,
// and overwrites it with the gradient; the onehot term is applied to the one chunk holding the
// label.  exp(x) is computed as 2^(x*log2 e) with v_exp_f32.

#include <limits.h>

#include "soupk_common.hpp"

namespace soupk {
namespace {

constexpr int kHeadThreads = 1024;
constexpr int kHeadWaves = kHeadThreads / kWave;
constexpr int kHeadUnroll = 2;  // 16-byte chunks per thread per sweep step
constexpr int64_t kIgnoreIndex = -100;

struct RowStats {
  float m;    // running max (also the best value for the argmax)
  float se;   // sum exp(z - m)
  float sd;   // sum exp(z - m) * z
  int32_t ix; // first column holding m (INT_MAX: none yet)
};

__device__ __forceinline__ float scale_to(float m_old, float m_new) {
  // exp(m_old - m_new); an empty accumulator (m_old = -inf) contributes nothing.
  return m_old == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((m_old - m_new) * kLog2e);
}

// Fold N consecutive columns z[0..N) starting at column col0 into the running statistics.
template <int N>
__device__ __forceinline__ void absorb(RowStats& st, const float* z, int32_t col0) {
  float bm = z[0];
#pragma unroll
  for (int j = 1; j < N; ++j) bm = fmaxf(bm, z[j]);
  if (bm > st.m) {
    const float f = scale_to(st.m, bm);
    st.se = st.se * f;
    st.sd = st.sd * f;
    st.m = bm;
#pragma unroll
    for (int j = N - 1; j >= 0; --j)
      if (z[j] == bm) st.ix = col0 + j;
  }
  const float shift = -st.m * kLog2e;
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(z[j], kLog2e, shift));
    st.se = st.se + e;
    st.sd = __builtin_fmaf(e, z[j], st.sd);
  }
}

__device__ __forceinline__ void merge(RowStats& a, const RowStats& b) {
  const float M = fmaxf(a.m, b.m);
  const float fa = scale_to(a.m, M), fb = scale_to(b.m, M);
  if (b.m > a.m || (b.m == a.m && b.ix < a.ix)) a.ix = b.ix;
  a.se = a.se * fa + b.se * fb;
  a.sd = a.sd * fa + b.sd * fb;
  a.m = M;
}

__device__ __forceinline__ void wave_merge(RowStats& s) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    RowStats t;
    t.m = __shfl_xor(s.m, o, kWave);
    t.se = __shfl_xor(s.se, o, kWave);
    t.sd = __shfl_xor(s.sd, o, kWave);
    t.ix = __shfl_xor(s.ix, o, kWave);
    merge(s, t);
  }
}

__device__ __forceinline__ void unpack8(const u32x4 w, float* z) {
  z[0] = lo_h(w.x); z[1] = hi_h(w.x); z[2] = lo_h(w.y); z[3] = hi_h(w.y);
  z[4] = lo_h(w.z); z[5] = hi_h(w.z); z[6] = lo_h(w.w); z[7] = hi_h(w.w);
}

__global__ __launch_bounds__(kHeadThreads) void head_stats_grad_kernel(
    uint16_t* __restrict__ logits, const int64_t* __restrict__ target,
    float* __restrict__ entropy, float* __restrict__ loss, int32_t* __restrict__ correct,
    float* __restrict__ lse_out, float grad_scale, int64_t V) {
  __shared__ RowStats part[kHeadWaves];
  __shared__ float row_lse;

  const int64_t row = blockIdx.x;
  uint16_t* base = logits + row * V;
  const int64_t tgt = target[row];
  const bool labelled = tgt != kIgnoreIndex;
  const bool tgt_ok = tgt >= 0 && tgt < V;
  const int tid = threadIdx.x;

  // Columns [0, lead) precede the first 16-byte boundary; [tail0, V) follow the last whole chunk.
  int64_t lead = ((16 - static_cast<int>(reinterpret_cast<uintptr_t>(base) & 15)) & 15) >> 1;
  if (lead > V) lead = V;
  const int64_t nvec = (V - lead) >> 3;
  const int64_t tail0 = lead + nvec * 8;
  const u32x4* vb = reinterpret_cast<const u32x4*>(base + lead);
  constexpr int64_t kStep = static_cast<int64_t>(kHeadThreads) * kHeadUnroll;

  // ---- sweep 1: statistics -------------------------------------------------------------
  RowStats st = {-INFINITY, 0.f, 0.f, INT_MAX};
  if (tid < lead) {
    const float z = h2f(base[tid]);
    absorb<1>(st, &z, tid);
  }
  for (int64_t s0 = 0; s0 < nvec; s0 += kStep) {
    u32x4 w[kHeadUnroll];
#pragma unroll
    for (int u = 0; u < kHeadUnroll; ++u) {
      const int64_t c = s0 + u * kHeadThreads + tid;
      if (c < nvec) w[u] = vb[c];
    }
#pragma unroll
    for (int u = 0; u < kHeadUnroll; ++u) {
      const int64_t c = s0 + u * kHeadThreads + tid;
      if (c < nvec) {
        float z[8];
        unpack8(w[u], z);
        absorb<8>(st, z, static_cast<int32_t>(lead + 8 * c));
      }
    }
  }
  if (tail0 + tid < V) {
    const float z = h2f(base[tail0 + tid]);
    absorb<1>(st, &z, static_cast<int32_t>(tail0 + tid));
  }
  wave_merge(st);
  const int wave = tid / kWave, lane = tid % kWave;
  if (lane == 0) part[wave] = st;
  __syncthreads();
  if (wave == 0) {
    RowStats r = lane < kHeadWaves ? part[lane] : RowStats{-INFINITY, 0.f, 0.f, INT_MAX};
    wave_merge(r);
    if (lane == 0) {
      const float lse = r.m + logf(r.se);
      const int32_t arg = r.ix == INT_MAX ? 0 : r.ix;
      entropy[row] = lse - r.sd / r.se;
      float l = 0.f;
      if (labelled) l = tgt_ok ? lse - h2f(base[tgt]) : NAN;
      loss[row] = l;
      correct[row] = (labelled && tgt_ok && static_cast<int64_t>(arg) == tgt) ? 1 : 0;
      if (lse_out != nullptr) lse_out[row] = lse;
      row_lse = lse;
    }
  }
  __syncthreads();
  if (!labelled) return;

  // ---- sweep 2: gradient in place --------------------------------------------------------
  const float shift = -row_lse * kLog2e;
  const int64_t tchunk = (tgt_ok && tgt >= lead && tgt < tail0) ? (tgt - lead) >> 3 : -1;
  auto grad1 = [&](int64_t col) {
    const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(h2f(base[col]), kLog2e, shift));
    const float g = (col == tgt ? p - 1.0f : p) * grad_scale;
    base[col] = static_cast<uint16_t>(pack_h2(g, 0.f) & 0xffffu);
  };
  if (tid < lead) grad1(tid);
  u32x4* vw = reinterpret_cast<u32x4*>(base + lead);
  for (int64_t s0 = 0; s0 < nvec; s0 += kStep) {
    u32x4 w[kHeadUnroll];
#pragma unroll
    for (int u = 0; u < kHeadUnroll; ++u) {
      const int64_t c = s0 + u * kHeadThreads + tid;
      if (c < nvec) w[u] = vw[c];
    }
#pragma unroll
    for (int u = 0; u < kHeadUnroll; ++u) {
      const int64_t c = s0 + u * kHeadThreads + tid;
      if (c < nvec) {
        float z[8];
        unpack8(w[u], z);
#pragma unroll
        for (int j = 0; j < 8; ++j) z[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(z[j], kLog2e, shift));
        if (c == tchunk) {
          const int jj = static_cast<int>((tgt - lead) & 7);
#pragma unroll
          for (int j = 0; j < 8; ++j)
            if (j == jj) z[j] = z[j] - 1.0f;
        }
        u32x4 o;
        o.x = pack_h2(z[0] * grad_scale, z[1] * grad_scale);
        o.y = pack_h2(z[2] * grad_scale, z[3] * grad_scale);
        o.z = pack_h2(z[4] * grad_scale, z[5] * grad_scale);
        o.w = pack_h2(z[6] * grad_scale, z[7] * grad_scale);
        __builtin_nontemporal_store(o, vw + c);
      }
    }
  }
  if (tail0 + tid < V) grad1(tail0 + tid);
}

}  // namespace
}  // namespace soupk

using namespace soupk;

extern "C" __attribute__((visibility("default"))) int soupk_head_stats_grad(
    uint16_t* logits, const int64_t* target, float* entropy, float* loss, int32_t* correct,
    float* lse_out, float grad_scale, int64_t rows, int64_t V, void* stream) {
  if (rows < 0 || V <= 0 || V >= (int64_t{1} << 31) - 16) return kInvalid;
  if (rows == 0) return kOk;
  if (rows > 0x7fffffff) return kInvalid;
  if (!logits || !target || !entropy || !loss || !correct) return kInvalid;
  if (reinterpret_cast<uintptr_t>(logits) & 1u) return kInvalid;
  hipStream_t st = static_cast<hipStream_t>(stream);
  head_stats_grad_kernel<<<static_cast<unsigned>(rows), kHeadThreads, 0, st>>>(
      logits, target, entropy, loss, correct, lse_out, grad_scale, V);
  return launch_status();
}
