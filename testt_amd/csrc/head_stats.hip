// Vocab-head online softmax: per-row lse, entropy, token loss, argmax hit, and the in-place fp16
// gradient (softmax - onehot) * grad_scale of the chunk logits.
//
// Reference: solution/head.py:34-76 (head_stats_grad_kernel), launched per 256-row chunk from
// FusedHeadLoss.forward, solution/head.py:105-114.
//
// Mapping (gfx950): one workgroup of 1024 threads (16 wavefronts, a whole CU) per logits row.
// Register-resident form (V <= 1024 * 8 * kMaxCpt): each thread loads its share of the row --
// chunk k*1024 + tid, 16 bytes each, every wave load instruction reading 1 KiB contiguous --
// into VGPRs (a 151,936-column row is 297 KiB = 19 x 16 B per thread, loads kept 2 deep),
// computes the statistics from the registers as the loads land -- replacing each chunk by its
// exponentials -- and after the workgroup reduction writes the gradient from the same
// registers: the row crosses HBM once in and (for labelled rows) once out, the compulsory
// traffic.  Larger vocabularies use the streaming form, which reads the row
// twice (the second read served by L2 / the Infinity Cache).
//
// Statistics per lane: running max m, sum(e) and sum(e*z) with e = exp(z - m), and the first
// column where the max was reached (lanes visit their columns in increasing order, so a strict
// '>' keeps the first occurrence; merges across lanes break value ties on the smaller column,
// which is torch.argmax's first-maximum rule).  The running sums are rescaled once per 8-value
// chunk, only when the chunk raises the max.  exp(x) is computed as 2^(x*log2 e) (v_exp_f32).

#include <limits.h>

#include <type_traits>

#include "soupk_common.hpp"

namespace soupk {
namespace {

constexpr int kHeadThreads = 1024;
constexpr int kHeadWaves = kHeadThreads / kWave;
constexpr int kStreamUnroll = 2;  // 16-byte chunks per thread per step, streaming form
constexpr int kMaxCpt = 20;       // register-resident form: up to 20 chunks (80 VGPRs) / thread
#ifndef SOUPK_HEAD_PREFETCH
#define SOUPK_HEAD_PREFETCH 2
#endif

constexpr int kHeadPrefetch = SOUPK_HEAD_PREFETCH;  // resident form: chunk loads in flight per lane
constexpr int64_t kIgnoreIndex = -100;

struct RowStats {
  float m;     // running max (also the best value for the argmax)
  float se;    // sum exp(z - m)
  float sd;    // sum exp(z - m) * z
  int32_t ix;  // first column holding m (INT_MAX: none yet)
};

__device__ __forceinline__ float scale_to(float m_old, float m_new) {
  // exp(m_old - m_new); an empty accumulator (m_old = -inf) contributes nothing.
  return m_old == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((m_old - m_new) * kLog2e);
}

__device__ __forceinline__ void unpack8(const u32x4 w, float* z) {
  z[0] = lo_h(w.x); z[1] = hi_h(w.x); z[2] = lo_h(w.y); z[3] = hi_h(w.y);
  z[4] = lo_h(w.z); z[5] = hi_h(w.z); z[6] = lo_h(w.w); z[7] = hi_h(w.w);
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

// Fold one scalar column into the running statistics; with ties_win the column takes the
// argmax on an equal value too (used for a column left of everything folded in before it).
// `lift` scales the exponentials by 2^lift, as the resident form keeps its sums.
__device__ __forceinline__ void absorb_col(RowStats& st, float z, int32_t col, bool ties_win,
                                           float lift) {
  if (z > st.m || (ties_win && z == st.m)) {
    if (z > st.m) {
      const float f = scale_to(st.m, z);
      st.se = st.se * f;
      st.sd = st.sd * f;
      st.m = z;
    }
    st.ix = col;
  }
  const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(z, kLog2e, lift - st.m * kLog2e));
  st.se = st.se + e;
  st.sd = __builtin_fmaf(e, z, st.sd);
}

// Fold one 16-byte chunk (8 fp16 columns starting at col0) into the running statistics.  The
// chunk max is taken in packed fp16 (exact: a max selects one of its inputs), and the fp16
// values feed the fp32 exp/dot arithmetic directly (v_fma_mix_f32), so the chunk is never
// widened to eight fp32 registers.
__device__ __forceinline__ void absorb_chunk(RowStats& st, const u32x4 w, int32_t col0) {
  const f16x2 a = as_h2(w.x), b = as_h2(w.y), c = as_h2(w.z), d = as_h2(w.w);
  const f16x2 m2 = __builtin_elementwise_max(__builtin_elementwise_max(a, b),
                                             __builtin_elementwise_max(c, d));
  const float bm = fmaxf(static_cast<float>(m2[0]), static_cast<float>(m2[1]));
  if (bm > st.m) {
    const float f = scale_to(st.m, bm);
    st.se = st.se * f;
    st.sd = st.sd * f;
    st.m = bm;
    float z[8];
    unpack8(w, z);
#pragma unroll
    for (int j = 7; j >= 0; --j)
      if (z[j] == bm) st.ix = col0 + j;
  }
  const float shift = -st.m * kLog2e;
  const f16 h[8] = {a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float z = static_cast<float>(h[j]);
    const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(z, kLog2e, shift));
    st.se = st.se + e;
    st.sd = __builtin_fmaf(e, z, st.sd);
  }
}

// ---- row reductions -------------------------------------------------------------------------
// With the DPP row reductions of soupk_common.hpp.  The statistics are reduced as: the maximum
// first; then every lane rescales its sums to that maximum (one exponential) and the sums are
// added; the argmax is the smallest column among the lanes holding the maximum (first-maximum
// rule).  (A butterfly of full merges would need an LDS permute and two exponentials per step.)
// Statistics of 16 entries held by the 16 lanes of each row (every lane gets the result).
__device__ __forceinline__ RowStats row16_stats(const RowStats& s) {
  RowStats r;
  r.m = row16_max(s.m);
  const float f = scale_to(s.m, r.m);
  r.se = row16_sum(s.se * f);
  r.sd = row16_sum(s.sd * f);
  r.ix = row16_min(s.m == r.m ? s.ix : INT_MAX);
  return r;
}

// Statistics of the whole wavefront (uniform result).
__device__ __forceinline__ RowStats wave_stats(const RowStats& s) {
  RowStats r;
  const float rm = row16_max(s.m);
  r.m = fmaxf(fmaxf(lanef(rm, 0), lanef(rm, 16)), fmaxf(lanef(rm, 32), lanef(rm, 48)));
  const float f = scale_to(s.m, r.m);
  const float se = row16_sum(s.se * f), sd = row16_sum(s.sd * f);
  const int ix = row16_min(s.m == r.m ? s.ix : INT_MAX);
  r.se = (lanef(se, 0) + lanef(se, 16)) + (lanef(se, 32) + lanef(se, 48));
  r.sd = (lanef(sd, 0) + lanef(sd, 16)) + (lanef(sd, 32) + lanef(sd, 48));
  r.ix = min(min(__builtin_amdgcn_readlane(ix, 0), __builtin_amdgcn_readlane(ix, 16)),
             min(__builtin_amdgcn_readlane(ix, 32), __builtin_amdgcn_readlane(ix, 48)));
  return r;
}

// Row geometry: columns [0, lead) precede the first 16-byte boundary of the row, [tail0, V)
// follow its last whole 16-byte chunk; nvec chunks lie between.
struct RowSpan {
  int64_t lead, nvec, tail0;
};

__device__ __forceinline__ RowSpan row_span(const uint16_t* base, int64_t V) {
  RowSpan r;
  r.lead = ((16 - static_cast<int>(reinterpret_cast<uintptr_t>(base) & 15)) & 15) >> 1;
  if (r.lead > V) r.lead = V;
  r.nvec = (V - r.lead) >> 3;
  r.tail0 = r.lead + r.nvec * 8;
  return r;
}

// Workgroup merge of the per-thread statistics and the per-row outputs; returns the row's lse
// to every thread.  Each wavefront reduces its lanes and posts the result in LDS; after one
// barrier every wavefront reduces the 16 posted results itself (lanes l and l+16k read entry
// l), so no second barrier is needed.  zt is z[target] (0 without a valid target), read by the
// caller at the start of the kernel, before any thread overwrites the row.  The sums carry a
// factor 2^lift (lse removes it; entropy is a ratio).
__device__ float finish_row(RowStats st, RowStats* part, float zt, int64_t row, int64_t tgt,
                            bool labelled, bool tgt_ok, float* entropy, float* loss,
                            int32_t* correct, float* lse_out, float lift) {
  static_assert(kHeadWaves == 16, "one posted entry per lane of a 16-lane row");
  const RowStats w = wave_stats(st);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  if (lane == 0) part[wave] = w;
  __syncthreads();
  const RowStats r = row16_stats(part[lane % kHeadWaves]);
  const float lse = r.m + (logf(r.se) - lift * kLn2);
  if (threadIdx.x == 0) {
    const int32_t arg = r.ix == INT_MAX ? 0 : r.ix;
    entropy[row] = lse - r.sd / r.se;
    float l = 0.f;
    if (labelled) l = tgt_ok ? lse - zt : NAN;
    loss[row] = l;
    correct[row] = (labelled && tgt_ok && static_cast<int64_t>(arg) == tgt) ? 1 : 0;
    if (lse_out != nullptr) lse_out[row] = lse;
  }
  return lse;
}

// Gradient of one 8-column chunk: fp16((exp(z - lse) - [col == tgt]) * grad_scale).
__device__ __forceinline__ u32x4 grad_chunk(u32x4 w, float shift, float grad_scale,
                                            int hit /* 0..7, or -1 */) {
  float z[8];
  unpack8(w, z);
#pragma unroll
  for (int j = 0; j < 8; ++j) z[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(z[j], kLog2e, shift));
  if (hit >= 0) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j == hit) z[j] = z[j] - 1.0f;
  }
  return u32x4{pack_h2(z[0] * grad_scale, z[1] * grad_scale),
               pack_h2(z[2] * grad_scale, z[3] * grad_scale),
               pack_h2(z[4] * grad_scale, z[5] * grad_scale),
               pack_h2(z[6] * grad_scale, z[7] * grad_scale)};
}

__device__ __forceinline__ void grad_scalar(const uint16_t* src, uint16_t* dst, int64_t col,
                                            int64_t tgt, float shift, float grad_scale) {
  const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(h2f(src[col]), kLog2e, shift));
  const float g = (col == tgt ? p - 1.0f : p) * grad_scale;
  dst[col] = static_cast<uint16_t>(pack_h2(g, 0.f) & 0xffffu);
}

// Where the gradient of `row` goes: the row itself (grad_out NULL, in place), row
// grad_row[row] of grad_out, or nowhere (a row map entry outside [0, grad_rows), or no
// gradient output at all: grad_row NULL with grad_out NULL and in_place false).
struct GradDest {
  const int32_t* grad_row;  // nullable
  uint16_t* grad_out;       // nullable
  int64_t grad_rows;
  bool in_place;
};

__device__ __forceinline__ uint16_t* grad_row_base(const GradDest& gd, uint16_t* base,
                                                   int64_t row, int64_t V) {
  if (gd.in_place) return base;
  if (gd.grad_out == nullptr || gd.grad_row == nullptr) return nullptr;
  const int64_t d = gd.grad_row[row];
  return (d >= 0 && d < gd.grad_rows) ? gd.grad_out + d * V : nullptr;
}

// ---- register-resident form ------------------------------------------------------------------
// The statistics pass keeps, in place of each 16-byte chunk of logits, the chunk's eight
// exponentials e = 2^kLift * exp(z - m_k) as fp16 (m_k: the thread's running max when the chunk
// was folded in, saved per chunk in LDS as fp16 -- exact, it is one of the fp16 logits).  The
// gradient pass then needs one exponential per chunk, F_k = exp(m_k - lse) * grad_scale *
// 2^-kLift, and one multiply per column: grad = e * F_k.  The factor 2^kLift keeps e out of the
// fp16 subnormal range down to exp(z - m) = 2^-29, where the product is far below one fp16 ulp
// of any gradient the scale can produce (grad_scale <= 2^15); above it e carries a relative
// error <= 2^-11, so the product rounds to fp16 within one ulp of the exactly rounded value.
// The target column (p - 1 cancels) is recomputed from its logit in full fp32.
constexpr float kLift = 15.f;

// Per-chunk statistics step: the chunk max uses v_pk_maximum3_f16 (exact: a max selects one of
// its inputs).  When it raises the running max, the sums are rescaled and the chunk's raw
// logits are kept in `best` (with its number in kbest) for the argmax, which is resolved once at
// the end; then the chunk's registers are overwritten with its lifted exponentials.
// `shift` (kLift - m * log2 e) and `m16` (m as fp16, exact: m is one of the logits) follow the
// running max, updated only when a chunk raises it, not recomputed for every chunk.
__device__ __forceinline__ void absorb_keep(RowStats& st, float& shift, f16& m16, int& kbest,
                                            u32x4& best, u32x4& w, int k) {
  const f16x2 a = as_h2(w.x), b = as_h2(w.y), c = as_h2(w.z), d = as_h2(w.w);
  const f16x2 m2 = __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b),
                                                 __builtin_elementwise_maximum(c, d));
  // Compared in fp16 with m16 (which equals st.m exactly): the widening to fp32 is needed only
  // when the chunk raises the max.
  const f16 bm16 = __builtin_elementwise_maximum(m2[0], m2[1]);
  if (bm16 > m16) {
    const float bm = static_cast<float>(bm16);
    const float f = scale_to(st.m, bm);
    st.se = st.se * f;
    st.sd = st.sd * f;
    st.m = bm;
    shift = kLift - bm * kLog2e;
    m16 = bm16;
    kbest = k;
    best = w;
  }
  const f16 h[8] = {a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
  float e[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float z = static_cast<float>(h[j]);
    e[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(z, kLog2e, shift));
    st.se = st.se + e[j];
    st.sd = __builtin_fmaf(e[j], z, st.sd);
  }
  w = u32x4{pack_h2(e[0], e[1]), pack_h2(e[2], e[3]), pack_h2(e[4], e[5]), pack_h2(e[6], e[7])};
}

// Gradient of one chunk from its lifted exponentials: fp16(e * F); in the target's chunk the
// column `hit` (0..7) takes `gt`, computed from the logit itself.
__device__ __forceinline__ u32x4 grad_from_e(u32x4 w, float F, int hit, float gt) {
  const f16x2 a = as_h2(w.x), b = as_h2(w.y), c = as_h2(w.z), d = as_h2(w.w);
  const f16 h[8] = {a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
  float g[8];
  // e * F as one fused multiply-add with a zero addend: v_fma_mix_f32 reads the fp16 e
  // directly, and the result is the product rounded once, as a multiply would give.
#pragma unroll
  for (int j = 0; j < 8; ++j) g[j] = __builtin_fmaf(static_cast<float>(h[j]), F, 0.0f);
  if (hit >= 0) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      if (j == hit) g[j] = gt;
  }
  return u32x4{pack_h2(g[0], g[1]), pack_h2(g[2], g[3]), pack_h2(g[4], g[5]),
               pack_h2(g[6], g[7])};
}

template <int CPT>
__global__ __launch_bounds__(kHeadThreads) void head_stats_grad_kernel(
    uint16_t* __restrict__ logits, const int64_t* __restrict__ target,
    float* __restrict__ entropy, float* __restrict__ loss, int32_t* __restrict__ correct,
    float* __restrict__ lse_out, float grad_scale, int64_t V, GradDest gd) {
  constexpr int P = CPT < kHeadPrefetch ? CPT : kHeadPrefetch;  // loads kept ahead of compute
  __shared__ RowStats part[kHeadWaves];
  __shared__ f16 chunk_max[CPT * kHeadThreads];  // m_k of chunk k of thread t at [k*1024 + t]
  const int64_t row = blockIdx.x;
  uint16_t* base = logits + row * V;
  const int tid = threadIdx.x;
  const RowSpan sp = row_span(base, V);
  // The row's whole chunks as one range-checked buffer: every load is issued unconditionally
  // (chunks past the row read as 0), and each chunk needs only a 32-bit offset register.
  const __amdgpu_buffer_rsrc_t rsrc =
      buffer_rsrc(base + sp.lead, static_cast<uint32_t>(sp.nvec * 16));
  const uint32_t off0 = static_cast<uint32_t>(tid) * 16;
  constexpr uint32_t kChunkStride = kHeadThreads * 16;
  // The scalar head/tail columns are loaded first: waiting for a load waits for every load
  // issued before it, so they must not queue behind the chunk prefetch.
  // Both are unconditional, at clamped in-row columns, so that no branch forces an early wait.
  // The target's logit is read here too (every thread, one address), for the loss and the
  // gradient of the target column.
  const bool has_lead = tid < sp.lead, has_tail = sp.tail0 + tid < V;
  const float zlead = h2f(base[has_lead ? tid : 0]);
  const float ztail = h2f(base[has_tail ? sp.tail0 + tid : V - 1]);
  u32x4 w[CPT];
  // Chunk column k of this thread (at byte offset off0 + k*kChunkStride of the row's chunks).
  auto load_col = [&](int k) -> u32x4 {
    return __builtin_amdgcn_raw_buffer_load_b128(rsrc, off0 + k * kChunkStride, 0,
                                                 kAuxNonTemporal);
  };
#pragma unroll
  for (int k = 0; k < P; ++k) w[k] = load_col(k);
  __builtin_amdgcn_sched_barrier(0);
  // The target, and then its logit, are read only once the first chunk loads are in flight:
  // the logit's address needs the target's scalar load, and a wait for that load placed
  // before the chunk loads held every row's first bytes back by one memory round trip.
  const int64_t tgt = target[row];
  const bool labelled = tgt != kIgnoreIndex;
  const bool tgt_ok = tgt >= 0 && tgt < V;
  const float zt_raw = h2f(base[tgt_ok ? tgt : 0]);
  const float zt = tgt_ok ? zt_raw : 0.f;

  // 32-bit chunk indices (a row has < 2^28 chunks): 64-bit ones would cost a register pair
  // per chunk on top of the row.
  const int32_t nvec = static_cast<int32_t>(sp.nvec), lead = static_cast<int32_t>(sp.lead);
  RowStats st = {-INFINITY, 0.f, 0.f, INT_MAX};
  float run_shift = kLift - st.m * kLog2e;   // (+inf until a chunk sets the max)
  f16 m16 = static_cast<f16>(-INFINITY);
  int kbest = -1;
  u32x4 best = {0u, 0u, 0u, 0u};
  // Load k + P is issued before chunk k is folded in, so each wave keeps P chunks in flight and
  // its arithmetic follows the data as it lands; the scheduling fences keep one chunk's
  // temporaries live at a time (the row already occupies 4*CPT VGPRs).
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    if (k + P < CPT) w[k + P] = load_col(k + P);
    if (k * kHeadThreads + tid < nvec) {
      absorb_keep(st, run_shift, m16, kbest, best, w[k], k);
      chunk_max[k * kHeadThreads + tid] = m16;
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  if (kbest >= 0) {
    // First column of the max inside chunk kbest.
    float z[8];
    unpack8(best, z);
    int j0 = 7;
#pragma unroll
    for (int j = 6; j >= 0; --j)
      if (z[j] == st.m) j0 = j;
    st.ix = lead + 8 * (kbest * kHeadThreads + tid) + j0;
  }
  // The scalar columns come last (the sums do not depend on order): the head column lies left
  // of every chunk, so it takes the argmax on ties; the tail column lies right of them all.
  if (has_lead) absorb_col(st, zlead, tid, true, kLift);
  if (has_tail) absorb_col(st, ztail, static_cast<int32_t>(sp.tail0 + tid), false, kLift);

  const float lse = finish_row(st, part, zt, row, tgt, labelled, tgt_ok, entropy,
                               loss, correct, lse_out, kLift);
  uint16_t* const gbase = grad_row_base(gd, base, row, V);
  if (!labelled || gbase == nullptr) return;
  // The gradient row has the logits row's alignment (the entry point checks it), so it splits
  // into the same lead columns, whole chunks and tail columns.
  const __amdgpu_buffer_rsrc_t wrsrc =
      buffer_rsrc(gbase + sp.lead, static_cast<uint32_t>(sp.nvec * 16));
  const float shift = -lse * kLog2e;
  // F_k = 2^(m_k*log2e + fbase) = exp(m_k - lse) * grad_scale * 2^-kLift.
  const float fbase = (log2f(grad_scale) - kLift) - lse * kLog2e;
  const int32_t tc =
      (tgt_ok && tgt >= sp.lead && tgt < sp.tail0) ? static_cast<int32_t>((tgt - sp.lead) >> 3)
                                                   : -1;
  const int thit = static_cast<int>((tgt - sp.lead) & 7);
  // The target column: (exp(z_t - lse) - 1) * grad_scale in fp32 (used by one lane only).
  const float gt =
      (__builtin_amdgcn_exp2f(__builtin_fmaf(zt, kLog2e, shift)) - 1.0f) * grad_scale;
  if (has_lead) grad_scalar(base, gbase, tid, tgt, shift, grad_scale);
  // The gradient is stored non-temporal without the device-scope bit the streaming kernels' stores
  // carry (nt | sc1): with it the kernel took 26.9 us at 256 rows, without 26.5 us, the other
  // kernels of the set unchanged (one set of buffers for both builds).  Cached stores made it
  // 24.8 us but the kernels after it 1.1 us slower: their write-back only moved out of its time.
  // Store offsets are recomputed from an opaque copy of tid*16 (one add per chunk) rather than
  // kept live from the load phase: CPT offset registers on top of the row would spill.
  uint32_t lane_off = off0;
  asm volatile("" : "+v"(lane_off));
#pragma unroll
  for (int k = 0; k < CPT; ++k) {
    const int32_t c = k * kHeadThreads + tid;
    if (c < nvec) {
      const float mk = static_cast<float>(chunk_max[k * kHeadThreads + tid]);
      const float F = __builtin_amdgcn_exp2f(__builtin_fmaf(mk, kLog2e, fbase));
      __builtin_amdgcn_raw_buffer_store_b128(grad_from_e(w[k], F, c == tc ? thit : -1, gt),
                                             wrsrc, lane_off + k * kChunkStride, 0,
                                             kAuxNonTemporal);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  if (has_tail) grad_scalar(base, gbase, sp.tail0 + tid, tgt, shift, grad_scale);
}

// ---- streaming form (two reads of the row) -----------------------------------------------------
__global__ __launch_bounds__(kHeadThreads) void head_stats_grad_stream_kernel(
    uint16_t* __restrict__ logits, const int64_t* __restrict__ target,
    float* __restrict__ entropy, float* __restrict__ loss, int32_t* __restrict__ correct,
    float* __restrict__ lse_out, float grad_scale, int64_t V, GradDest gd) {
  __shared__ RowStats part[kHeadWaves];
  const int64_t row = blockIdx.x;
  uint16_t* base = logits + row * V;
  const int64_t tgt = target[row];
  const bool labelled = tgt != kIgnoreIndex;
  const bool tgt_ok = tgt >= 0 && tgt < V;
  const int tid = threadIdx.x;
  const RowSpan sp = row_span(base, V);
  u32x4* vb = reinterpret_cast<u32x4*>(base + sp.lead);
  constexpr int64_t kStep = static_cast<int64_t>(kHeadThreads) * kStreamUnroll;
  const float zt_raw = h2f(base[tgt_ok ? tgt : 0]);  // (before any write)
  const float zt = tgt_ok ? zt_raw : 0.f;

  RowStats st = {-INFINITY, 0.f, 0.f, INT_MAX};
  if (tid < sp.lead) {
    const float z = h2f(base[tid]);
    absorb<1>(st, &z, tid);
  }
  for (int64_t s0 = 0; s0 < sp.nvec; s0 += kStep) {
    u32x4 w[kStreamUnroll];
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u) {
      const int64_t c = s0 + u * kHeadThreads + tid;
      w[u] = vb[c < sp.nvec ? c : sp.nvec - 1];
    }
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u) {
      const int64_t c = s0 + u * kHeadThreads + tid;
      if (c < sp.nvec) absorb_chunk(st, w[u], static_cast<int32_t>(sp.lead + 8 * c));
    }
  }
  if (sp.tail0 + tid < V) {
    const float z = h2f(base[sp.tail0 + tid]);
    absorb<1>(st, &z, static_cast<int32_t>(sp.tail0 + tid));
  }
  const float lse = finish_row(st, part, zt, row, tgt, labelled, tgt_ok, entropy,
                               loss, correct, lse_out, 0.f);
  uint16_t* const gbase = grad_row_base(gd, base, row, V);
  if (!labelled || gbase == nullptr) return;
  u32x4* const gvb = reinterpret_cast<u32x4*>(gbase + sp.lead);
  const float shift = -lse * kLog2e;
  const int64_t tc = (tgt_ok && tgt >= sp.lead && tgt < sp.tail0) ? (tgt - sp.lead) >> 3 : -1;
  const int thit = static_cast<int>((tgt - sp.lead) & 7);
  if (tid < sp.lead) grad_scalar(base, gbase, tid, tgt, shift, grad_scale);
  for (int64_t s0 = 0; s0 < sp.nvec; s0 += kStep) {
    u32x4 w[kStreamUnroll];
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u) {
      const int64_t c = s0 + u * kHeadThreads + tid;
      w[u] = vb[c < sp.nvec ? c : sp.nvec - 1];
    }
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u) {
      const int64_t c = s0 + u * kHeadThreads + tid;
      if (c < sp.nvec)
        __builtin_nontemporal_store(grad_chunk(w[u], shift, grad_scale, c == tc ? thit : -1),
                                    gvb + c);
    }
  }
  if (sp.tail0 + tid < V) grad_scalar(base, gbase, sp.tail0 + tid, tgt, shift, grad_scale);
}

}  // namespace
}  // namespace soupk

using namespace soupk;

namespace {

int head_launch(uint16_t* logits, const int64_t* target, float* entropy, float* loss,
                int32_t* correct, float* lse_out, float grad_scale, int64_t rows, int64_t V,
                const GradDest& gd, void* stream) {
  if (rows < 0 || V <= 0 || V >= (int64_t{1} << 31) - 16) return kInvalid;
  if (rows == 0) return kOk;
  if (rows > 0x7fffffff) return kInvalid;
  if (!logits || !target || !entropy || !loss || !correct) return kInvalid;
  if (reinterpret_cast<uintptr_t>(logits) & 1u) return kInvalid;
  if (!(grad_scale >= 0.f)) return kInvalid;  // negative or NaN (log2 of it is taken)
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(rows)), block(kHeadThreads);
  // Whole 16-byte chunks per thread: at most V/8 chunks per row over 1024 threads.
  const int64_t cpt = (V / 8 + kHeadThreads - 1) / kHeadThreads;
  auto run = [&](auto tag) {
    constexpr int C = decltype(tag)::value;
    return launch_kernel(head_stats_grad_kernel<C>, grid, block, s, logits, target, entropy,
                         loss, correct, lse_out, grad_scale, V, gd);
  };
  if (cpt <= 1) return run(std::integral_constant<int, 1>{});
  if (cpt <= 2) return run(std::integral_constant<int, 2>{});
  if (cpt <= 4) return run(std::integral_constant<int, 4>{});
  if (cpt <= 8) return run(std::integral_constant<int, 8>{});
  if (cpt <= 12) return run(std::integral_constant<int, 12>{});
  if (cpt <= 16) return run(std::integral_constant<int, 16>{});
  if (cpt <= 19) return run(std::integral_constant<int, 19>{});
  if (cpt <= kMaxCpt) return run(std::integral_constant<int, kMaxCpt>{});
  return launch_kernel(head_stats_grad_stream_kernel, grid, block, s, logits, target, entropy,
                       loss, correct, lse_out, grad_scale, V, gd);
}

}  // namespace

extern "C" __attribute__((visibility("default"))) int soupk_head_stats_grad(
    uint16_t* logits, const int64_t* target, float* entropy, float* loss, int32_t* correct,
    float* lse_out, float grad_scale, int64_t rows, int64_t V, void* stream) {
  const GradDest gd{nullptr, nullptr, 0, true};
  return head_launch(logits, target, entropy, loss, correct, lse_out, grad_scale, rows, V, gd,
                     stream);
}

extern "C" __attribute__((visibility("default"))) int soupk_head_stats_grad_rows(
    const uint16_t* logits, const int64_t* target, const int32_t* grad_row, uint16_t* grad_out,
    int64_t grad_rows, float* entropy, float* loss, int32_t* correct, float* lse_out,
    float grad_scale, int64_t rows, int64_t V, void* stream) {
  if ((grad_out == nullptr) != (grad_row == nullptr) || grad_rows < 0) return kInvalid;
  if (grad_out != nullptr) {
    // Every gradient row must split into the same lead columns, 16-byte chunks and tail
    // columns as every logits row: the same address modulo 16 and a row pitch of whole chunks.
    if ((V * 2) % 16 != 0) return kInvalid;
    if ((reinterpret_cast<uintptr_t>(grad_out) - reinterpret_cast<uintptr_t>(logits)) & 15u)
      return kInvalid;
  }
  const GradDest gd{grad_row, grad_out, grad_rows, false};
  // The kernels only read the logits when the gradient goes elsewhere (or nowhere).
  return head_launch(const_cast<uint16_t*>(logits), target, entropy, loss, correct, lse_out,
                     grad_scale, rows, V, gd, stream);
}
