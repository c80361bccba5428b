// Residual add + Qwen2RMSNorm, forward and backward, one or two wavefronts per token row.
//
// Reference: solution/rmsnorm.py:24-43 (rmsnorm_fwd_kernel) and solution/rmsnorm.py:46-69
// (rmsnorm_bwd_kernel), launched from _launch_fwd / _launch_bwd, solution/rmsnorm.py:76-112.
// The normalisation is transformers' Qwen2RMSNorm (modeling_qwen2.py:247-252):
// w * (s * rsqrt(mean(s^2) + eps)), with the product (s * rstd) rounded before the weight.
//
// Mapping (gfx950): a row of H fp32 is H/4 float4 chunks, split over WPR wavefronts (2 in both
// directions) owning alternate 64-chunk slices, so every load or store instruction of a wave
// touches 1 KiB (fp32) or 512 B (fp16) of contiguous memory.  The row's values stay in registers
// between the load, the wave64 reduction (DPP steps; combined across the row's waves in LDS) and
// the stores.  In the forward pass two waves per row give 16 waves per CU at 2048 rows, which
// hides HBM latency better than one (and 2 rows per wave, 4 waves per CU, ran 40% slower).  A
// workgroup holds 2, 4 or 8 rows, by the row count.  In the forward pass extra workgroups after
// the row workgroups zero the rows of the padded fp32 output that no token maps to (the pad
// rows), so the padded tensor needs no separate memset.

#include "soupk_common.hpp"

namespace soupk {
namespace {

// Rows per workgroup, chosen at launch from the row count (fwd_rows_per_block,
// bwd_rows_per_block below).
// Wavefronts per row on the vector path (measured on MI355X at 2048 x 1536: the forward pass is
// 17% faster with two than with one; the backward pass, with streaming stores, 2% faster).
#ifndef SOUPK_NORM_WPR_FWD
#define SOUPK_NORM_WPR_FWD 2
#endif
#ifndef SOUPK_NORM_WPR_BWD
#define SOUPK_NORM_WPR_BWD 2
#endif
constexpr int kWprFwd = SOUPK_NORM_WPR_FWD;
constexpr int kWprBwd = SOUPK_NORM_WPR_BWD;
#ifndef SOUPK_NORM_NT_LD
#define SOUPK_NORM_NT_LD 1
#endif
// Row streams (x, delta, s, dy, dypad, ds in; s, y, ypad, dx, ddelta out) are touched once per
// launch: non-temporal loads (1) and streaming stores (nt | sc1 backward, nt forward).  The
// weight, read by every row, stays cached.  (Cached row loads made the backward pass 2% faster
// on MI355X but the RoPE forward kernel that follows it in a training step 10% slower.)
constexpr bool kNormNtLd = SOUPK_NORM_NT_LD != 0;
// The forward pass's stores take nt alone, without the device-scope bit: 8.54 -> 8.19 us at
// 2048 rows, the other kernels of the set unchanged (one set of buffers for both builds); the
// backward pass, like the other streaming kernels, is faster with nt | sc1.
using FwdOut = StreamOutT<kAuxNonTemporal>;

// Row streams read through range-checked buffer descriptors.  A stream the caller leaves out
// (nullable delta, dy, dypad, ds) gets a descriptor of zero bytes, whose loads return zeros, so
// every load is issued unconditionally: a load under `p != nullptr ? load : zero` compiled to a
// branch and a wait for all outstanding loads at its join, once per chunk.  Chunks past a row's
// end read zeros the same way.
constexpr int kNormLdAux = kNormNtLd ? kAuxNonTemporal : 0;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* base, uint32_t bytes) {
  return buffer_rsrc(base, base != nullptr ? bytes : 0u);
}
template <int Aux = kNormLdAux>
__device__ __forceinline__ f32x4 bload_f4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, Aux));
}
__device__ __forceinline__ f32x4 bload_h4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x2 w = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kNormLdAux);
  return f32x4{lo_h(w.x), hi_h(w.x), lo_h(w.y), hi_h(w.y)};
}
__device__ __forceinline__ u32x2 pack_h4(f32x4 v) {
  return u32x2{pack_h2(v.x, v.y), pack_h2(v.z, v.w)};
}
// A value loaded at a wave-uniform address, moved to scalar registers (a buffer descriptor
// built from it then needs no per-lane loop).
__device__ __forceinline__ int64_t uniform_i64(int64_t v) {
  const uint64_t u = static_cast<uint64_t>(v);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(u >> 32));
  return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}


// WPR wavefronts share a row: lane l of the row's wave `sub` owns the float4 chunks
// j*64*WPR + sub*64 + l, so each wave load or store instruction touches 1 KiB (fp32) or
// 512 B (fp16) of contiguous memory.  The row's sum of squares (forward) or dot product
// (backward) is combined across the row's waves through LDS, always in the same order.  All
// loads are issued before any arithmetic: in the backward through the rows' buffer descriptors
// (chunks past a row's end read zeros), in the forward at clamped chunk indices (lanes past the
// row's end zero their values with a select).
template <int CPL, int WPR, int ROWS>
__global__ __launch_bounds__(kWave * ROWS * WPR) void rmsnorm_fwd_kernel(
    const float* __restrict__ x, const uint16_t* __restrict__ delta, const float* __restrict__ w,
    float* __restrict__ s_out, uint16_t* __restrict__ y, float* __restrict__ ypad,
    const int64_t* __restrict__ pad_idx, const int32_t* __restrict__ pad_inv,
    float* __restrict__ rstd_out, int64_t rows, int64_t pad_rows, int H, float eps,
    int64_t row_blocks) {
  __shared__ float part[ROWS][WPR];
  const int lane = threadIdx.x % kWave;
  const int nch = H / 4;
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
  if (static_cast<int64_t>(blockIdx.x) >= row_blocks) {
    // Zero the padded rows that no token row is scattered to (one row per wavefront).
    const int64_t p =
        (static_cast<int64_t>(blockIdx.x) - row_blocks) * (ROWS * WPR) + wave;
    if (p >= pad_rows || pad_inv[p] >= 0) return;
    const FwdOut dst(ypad + p * H, static_cast<uint64_t>(H) * 4u);
    for (int c = lane; c < nch; c += kWave) dst.store(16u * c, zero);
    return;
  }
  const int rib = wave / WPR, sub = wave % WPR;  // row in block, wave within the row
  const int64_t row_raw = static_cast<int64_t>(blockIdx.x) * ROWS + rib;
  const bool live = row_raw < rows;  // (all waves reach the barrier below)
  const int64_t row = live ? row_raw : rows - 1;
  // (The forward keeps global loads at clamped chunk indices, with the delta loads under their
  // null test: the same loads through buffer descriptors, unconditional, ran 8.48 -> 8.97 us
  // at 2048 rows on MI355X.  The backward gained from them: 11.34 -> 11.23 us.)
  const f32x4* xr = reinterpret_cast<const f32x4*>(x + row * H);
  const f32x4* wr = reinterpret_cast<const f32x4*>(w);
  f32x4 v[CPL], wv[CPL], d[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = min((j * WPR + sub) * kWave + lane, nch - 1);
    v[j] = ld<kNormNtLd>(xr + c);
    wv[j] = wr[c];
    if (delta != nullptr) {
      const u32x2 h = ld<kNormNtLd>(reinterpret_cast<const u32x2*>(delta + row * H + 4 * c));
      d[j] = f32x4{lo_h(h.x), hi_h(h.x), lo_h(h.y), hi_h(h.y)};
    }
  }
  int64_t dest = -1;
  if (ypad != nullptr) {
    dest = uniform_i64(pad_idx[row]);  // (row is the wave's: the destination is wave-uniform)
    if (dest < 0 || dest >= pad_rows) dest = -1;
  }
#pragma unroll
  for (int j = 0; j < CPL; ++j)
    if ((j * WPR + sub) * kWave + lane >= nch) v[j] = zero;
  if (delta != nullptr) {
    // (chunks past the row's end fall outside the row's descriptor: their stores are dropped)
    const FwdOut sr(s_out + row * H, static_cast<uint64_t>(H) * 4u);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const int c = (j * WPR + sub) * kWave + lane;
      v[j] = v[j] + d[j];
      if (live) sr.store(16u * c, v[j]);
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j)
      if ((j * WPR + sub) * kWave + lane >= nch) v[j] = zero;
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j)
    ss += (v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w);
  ss = wave_sum(ss);
  if constexpr (WPR > 1) {
    if (lane == 0) part[rib][sub] = ss;
    __syncthreads();
    ss = part[rib][0];
#pragma unroll
    for (int i = 1; i < WPR; ++i) ss += part[rib][i];
  }
  if (!live) return;
  const float rstd = 1.0f / sqrtf(ss / static_cast<float>(H) + eps);
  const FwdOut yr(y + row * H, static_cast<uint64_t>(H) * 2u);
  const FwdOut pr(ypad + (dest >= 0 ? dest : 0) * H, static_cast<uint64_t>(H) * 4u);
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = (j * WPR + sub) * kWave + lane;
    const f32x4 o = (v[j] * rstd) * wv[j];
    yr.store(8u * c, pack_h4(o));
    if (dest >= 0) pr.store(16u * c, o);
  }
  if (sub == 0 && lane == 0) rstd_out[row] = rstd;
}

template <int CPL, int WPR, int ROWS>
__global__ __launch_bounds__(kWave * ROWS * WPR) void rmsnorm_bwd_kernel(
    const float* __restrict__ s, const float* __restrict__ rstd_in, const float* __restrict__ w,
    const uint16_t* __restrict__ dy, const float* __restrict__ dypad,
    const int64_t* __restrict__ pad_idx, const float* __restrict__ ds, float* __restrict__ dx,
    uint16_t* __restrict__ ddelta, int64_t rows, int64_t pad_rows, int H) {
  __shared__ float part[ROWS][WPR];
  const int lane = threadIdx.x % kWave;
  const int nch = H / 4;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
  const int rib = wave / WPR, sub = wave % WPR;
  const int64_t row_raw = static_cast<int64_t>(blockIdx.x) * ROWS + rib;
  const bool live = row_raw < rows;  // (all waves reach the barrier below)
  const int64_t row = live ? row_raw : rows - 1;
  // The padded gradient row is a gather through pad_idx.  Its index is loaded first, and the
  // four streams that do not depend on it are issued before the wait for it, so the index's
  // latency is not paid ahead of every load of the row (waiting on pad_idx before the first
  // load, as the source row's pointer was formed, serialised the two).
  // (a vector load, counted in order with the row loads issued after it: waiting for it does
  // not wait for them, as a scalar load's wait would -- scalar loads complete out of order)
  const __amdgpu_buffer_rsrc_t ir = row_rsrc(dypad != nullptr ? pad_idx + row : nullptr, 8u);
  const u32x2 src_raw = __builtin_amdgcn_raw_buffer_load_b64(ir, 0, 0, 0);
  __builtin_amdgcn_sched_barrier(0);   // (issued ahead of the row loads, not sunk past them)
  const uint32_t bytes4 = static_cast<uint32_t>(H) * 4u;
  const __amdgpu_buffer_rsrc_t sr = row_rsrc(s + row * H, bytes4);
  const __amdgpu_buffer_rsrc_t wr = row_rsrc(w, bytes4);
  const __amdgpu_buffer_rsrc_t gr =
      row_rsrc(dy != nullptr ? dy + row * H : nullptr, static_cast<uint32_t>(H) * 2u);
  const __amdgpu_buffer_rsrc_t dsr = row_rsrc(ds != nullptr ? ds + row * H : nullptr, bytes4);
  f32x4 n[CPL], g[CPL], wv[CPL], gp[CPL], dd[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const uint32_t c = static_cast<uint32_t>((j * WPR + sub) * kWave + lane);
    n[j] = bload_f4(sr, 16u * c);
    wv[j] = bload_f4<0>(wr, 16u * c);
    g[j] = bload_h4(gr, 8u * c);
    dd[j] = bload_f4(dsr, 16u * c);
  }
  // (row is the wave's: the source is wave-uniform)
  int64_t src =
      uniform_i64(static_cast<int64_t>((static_cast<uint64_t>(src_raw.y) << 32) | src_raw.x));
  if (dypad == nullptr || src < 0 || src >= pad_rows) src = -1;
  const __amdgpu_buffer_rsrc_t pr = row_rsrc(src >= 0 ? dypad + src * H : nullptr, bytes4);
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const uint32_t c = static_cast<uint32_t>((j * WPR + sub) * kWave + lane);
    gp[j] = bload_f4(pr, 16u * c);
  }
  const float rstd = rstd_in[row];
  float dot = 0.f;
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    g[j] = (g[j] + gp[j]) * wv[j];
    n[j] = n[j] * rstd;
    const f32x4 p = g[j] * n[j];
    if ((j * WPR + sub) * kWave + lane < nch) dot += (p.x + p.y) + (p.z + p.w);
  }
  dot = wave_sum(dot);
  if constexpr (WPR > 1) {
    if (lane == 0) part[rib][sub] = dot;
    __syncthreads();
    dot = part[rib][0];
#pragma unroll
    for (int i = 1; i < WPR; ++i) dot += part[rib][i];
  }
  if (!live) return;
  const float proj = dot / static_cast<float>(H);
  // (chunks past the row's end fall outside the rows' descriptors: their stores are dropped)
  const StreamOut dxr(dx + row * H, static_cast<uint64_t>(H) * 4u);
  const StreamOut ddr(ddelta != nullptr ? static_cast<const void*>(ddelta + row * H) : dx,
                      static_cast<uint64_t>(H) * 2u);
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    const int c = (j * WPR + sub) * kWave + lane;
    f32x4 o = (g[j] - n[j] * proj) * rstd;
    if (ds != nullptr) o = o + dd[j];
    dxr.store(16u * c, o);
    if (ddelta != nullptr) ddr.store(8u * c, pack_h4(o));
  }
}

// ---- generic forms: any H (one workgroup of 256 threads per row, two passes) -------------
constexpr int kGenThreads = 256;

__device__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < kGenThreads / kWave; ++i) t += red[i];
  return t;
}

__global__ __launch_bounds__(kGenThreads) void rmsnorm_fwd_generic_kernel(
    const float* __restrict__ x, const uint16_t* __restrict__ delta, const float* __restrict__ w,
    float* __restrict__ s_out, uint16_t* __restrict__ y, float* __restrict__ ypad,
    const int64_t* __restrict__ pad_idx, const int32_t* __restrict__ pad_inv,
    float* __restrict__ rstd_out, int64_t rows, int64_t pad_rows, int H, float eps) {
  __shared__ float red[kGenThreads / kWave];
  const int64_t b = blockIdx.x;
  if (b >= rows) {
    const int64_t p = b - rows;
    if (p >= pad_rows || pad_inv[p] >= 0) return;
    for (int c = threadIdx.x; c < H; c += kGenThreads) ypad[p * H + c] = 0.f;
    return;
  }
  const int64_t row = b;
  float ss = 0.f;
  for (int c = threadIdx.x; c < H; c += kGenThreads) {
    float v = x[row * H + c];
    if (delta != nullptr) {
      v = v + h2f(delta[row * H + c]);
      s_out[row * H + c] = v;
    }
    ss += v * v;
  }
  ss = block_sum(ss, red);
  const float rstd = 1.0f / sqrtf(ss / static_cast<float>(H) + eps);
  int64_t dest = -1;
  if (ypad != nullptr) {
    dest = uniform_i64(pad_idx[row]);  // (row is the wave's: the destination is wave-uniform)
    if (dest < 0 || dest >= pad_rows) dest = -1;
  }
  for (int c = threadIdx.x; c < H; c += kGenThreads) {
    const float v = delta != nullptr ? s_out[row * H + c] : x[row * H + c];
    const float o = (v * rstd) * w[c];
    y[row * H + c] = static_cast<uint16_t>(pack_h2(o, 0.f) & 0xffffu);
    if (dest >= 0) ypad[dest * H + c] = o;
  }
  if (threadIdx.x == 0) rstd_out[row] = rstd;
}

__global__ __launch_bounds__(kGenThreads) void rmsnorm_bwd_generic_kernel(
    const float* __restrict__ s, const float* __restrict__ rstd_in, const float* __restrict__ w,
    const uint16_t* __restrict__ dy, const float* __restrict__ dypad,
    const int64_t* __restrict__ pad_idx, const float* __restrict__ ds, float* __restrict__ dx,
    uint16_t* __restrict__ ddelta, int64_t rows, int64_t pad_rows, int H) {
  __shared__ float red[kGenThreads / kWave];
  const int64_t row = blockIdx.x;
  if (row >= rows) return;
  int64_t src = -1;
  if (dypad != nullptr) {
    src = uniform_i64(pad_idx[row]);  // (row is the wave's: the source is wave-uniform)
    if (src < 0 || src >= pad_rows) src = -1;
  }
  const float rstd = rstd_in[row];
  float dot = 0.f;
  for (int c = threadIdx.x; c < H; c += kGenThreads) {
    float g = 0.f;
    if (dy != nullptr) g = g + h2f(dy[row * H + c]);
    if (src >= 0) g = g + dypad[src * H + c];
    g = g * w[c];
    dot += g * (s[row * H + c] * rstd);
  }
  const float proj = block_sum(dot, red) / static_cast<float>(H);
  for (int c = threadIdx.x; c < H; c += kGenThreads) {
    float g = 0.f;
    if (dy != nullptr) g = g + h2f(dy[row * H + c]);
    if (src >= 0) g = g + dypad[src * H + c];
    g = g * w[c];
    const float n = s[row * H + c] * rstd;
    float o = (g - n * proj) * rstd;
    if (ds != nullptr) o = o + ds[row * H + c];
    dx[row * H + c] = o;
    if (ddelta != nullptr) ddelta[row * H + c] = static_cast<uint16_t>(pack_h2(o, 0.f) & 0xffffu);
  }
}

inline bool aligned(const void* p, uintptr_t a) {
  return p == nullptr || (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// Dispatch on the number of float4 chunks per lane.
template <template <int> class Launch, typename... Args>
int with_cpl(int cpl, Args... args) {
  switch (cpl) {
    case 1: return Launch<1>::run(args...);
    case 2: return Launch<2>::run(args...);
    case 3: return Launch<3>::run(args...);
    case 4: return Launch<4>::run(args...);
    case 5: case 6: return Launch<6>::run(args...);
    case 7: case 8: return Launch<8>::run(args...);
    case 9: case 10: case 11: case 12: return Launch<12>::run(args...);
    case 13: case 14: case 15: case 16: return Launch<16>::run(args...);
    default: return -1;
  }
}
constexpr int kMaxCpl = 16;  // H <= 4 * 64 * WPR * 16 on the register-resident path

// Rows per workgroup (measured on MI355X, 256 CUs, H = 1536, medians of 5 rounds in one
// process): the backward at 2048 rows takes 10.35 us with 8 rows per workgroup (one
// 1024-thread workgroup per CU), 11.23 with 4, 12.03 with 2; at the ragged batch's 888 rows 8
// rows leave most CUs idle (7.16 us) and 4 is best (5.49; 2: 6.28).  The forward: 8.20 / 8.28
// / 8.42 us at 2048 rows with 8 / 4 / 2 rows per workgroup, and 5.80 / 5.42 / 5.21 us at 888.
constexpr int64_t kFullWaveRows = 8 * 256;   // 8 rows per workgroup fill the 256 CUs once
int fwd_rows_per_block(int64_t rows) {
#ifdef SOUPK_NORM_FWD_RPB
  if (SOUPK_NORM_FWD_RPB) return SOUPK_NORM_FWD_RPB;
#endif
  return rows >= kFullWaveRows ? 8 : rows >= kFullWaveRows / 2 ? 4 : 2;
}
int bwd_rows_per_block(int64_t rows) { return rows >= kFullWaveRows ? 8 : 4; }

template <int CPL>
struct FwdLaunch {
  template <int ROWS>
  static int go(dim3 grid, hipStream_t st, const float* x, const uint16_t* delta, const float* w,
                float* s_out, uint16_t* y, float* ypad, const int64_t* pad_idx,
                const int32_t* pad_inv, float* rstd, int64_t rows, int64_t pad_rows, int H,
                float eps, int64_t row_blocks) {
    return launch_kernel(rmsnorm_fwd_kernel<CPL, kWprFwd, ROWS>, grid,
                         dim3(kWave * ROWS * kWprFwd), st, x, delta, w, s_out, y, ypad, pad_idx,
                         pad_inv, rstd, rows, pad_rows, H, eps, row_blocks);
  }
  template <typename... Args>
  static int run(int rpb, Args... args) {
    return rpb == 8 ? go<8>(args...) : rpb == 4 ? go<4>(args...) : go<2>(args...);
  }
};

template <int CPL>
struct BwdLaunch {
  template <int ROWS>
  static int go(dim3 grid, hipStream_t st, const float* s, const float* rstd, const float* w,
                const uint16_t* dy, const float* dypad, const int64_t* pad_idx, const float* ds,
                float* dx, uint16_t* ddelta, int64_t rows, int64_t pad_rows, int H) {
    return launch_kernel(rmsnorm_bwd_kernel<CPL, kWprBwd, ROWS>, grid,
                         dim3(kWave * ROWS * kWprBwd), st, s, rstd, w, dy, dypad, pad_idx, ds,
                         dx, ddelta, rows, pad_rows, H);
  }
  template <typename... Args>
  static int run(int rpb, Args... args) {
    return rpb == 8 ? go<8>(args...) : go<4>(args...);
  }
};

}  // namespace
}  // namespace soupk

using namespace soupk;

extern "C" __attribute__((visibility("default"))) int soupk_rmsnorm_fwd(
    const float* x, const uint16_t* delta, const float* w, float* s_out, uint16_t* y,
    float* ypad, const int64_t* pad_idx, const int32_t* pad_inv, float* rstd, int64_t rows,
    int64_t pad_rows, int32_t H, float eps, void* stream) {
  if (rows < 0 || H <= 0 || pad_rows < 0) return kInvalid;
  const int64_t zero_rows = pad_inv != nullptr ? pad_rows : 0;
  if (rows == 0 && zero_rows == 0) return kOk;
  if (zero_rows > 0 && ypad == nullptr) return kInvalid;
  if (rows > 0) {
    // (An empty tensor's data pointer may be null, so the pairings are checked only with rows.)
    if (!x || !w || !y || !rstd) return kInvalid;
    if ((delta == nullptr) != (s_out == nullptr)) return kInvalid;
    if ((ypad == nullptr) != (pad_idx == nullptr)) return kInvalid;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int cpl = (H / 4 + kWave * kWprFwd - 1) / (kWave * kWprFwd);
  const bool vec = H % 4 == 0 && cpl <= kMaxCpl && aligned(x, 16) && aligned(w, 16) &&
                   aligned(s_out, 16) && aligned(ypad, 16) && aligned(delta, 8) && aligned(y, 8);
  if (vec) {
    const int rpb = fwd_rows_per_block(rows);
    const int64_t row_blocks = (rows + rpb - 1) / rpb;
    const int64_t zero_per_block = rpb * kWprFwd;  // one pad row per wavefront
    const int64_t blocks = row_blocks + (zero_rows + zero_per_block - 1) / zero_per_block;
    if (blocks > 0x7fffffff) return kInvalid;
    return with_cpl<FwdLaunch>(cpl, rpb, dim3(static_cast<unsigned>(blocks)), st, x, delta, w,
                               s_out, y, ypad, pad_idx, pad_inv, rstd, rows, pad_rows,
                               static_cast<int>(H), eps, row_blocks);
  }
  const int64_t blocks = rows + zero_rows;
  if (blocks > 0x7fffffff) return kInvalid;
  return launch_kernel(rmsnorm_fwd_generic_kernel, dim3(static_cast<unsigned>(blocks)),
                       dim3(kGenThreads), st, x, delta, w, s_out, y, ypad, pad_idx, pad_inv, rstd,
                       rows, pad_rows, H, eps);
}

extern "C" __attribute__((visibility("default"))) int soupk_rmsnorm_bwd(
    const float* s, const float* rstd, const float* w, const uint16_t* dy, const float* dypad,
    const int64_t* pad_idx, const float* ds, float* dx, uint16_t* ddelta, int64_t rows,
    int64_t pad_rows, int32_t H, void* stream) {
  if (rows < 0 || H <= 0 || pad_rows < 0) return kInvalid;
  if (dypad != nullptr && pad_idx == nullptr) return kInvalid;
  if (rows == 0) return kOk;
  if (!s || !rstd || !w || !dx) return kInvalid;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int cpl = (H / 4 + kWave * kWprBwd - 1) / (kWave * kWprBwd);
  const bool vec = H % 4 == 0 && cpl <= kMaxCpl && aligned(s, 16) && aligned(w, 16) &&
                   aligned(dypad, 16) && aligned(ds, 16) && aligned(dx, 16) && aligned(dy, 8) &&
                   aligned(ddelta, 8);
  if (vec) {
    const int rpb = bwd_rows_per_block(rows);
    const int64_t blocks = (rows + rpb - 1) / rpb;
    if (blocks > 0x7fffffff) return kInvalid;
    return with_cpl<BwdLaunch>(cpl, rpb, dim3(static_cast<unsigned>(blocks)), st, s, rstd, w,
                               dy, dypad, pad_idx, ds, dx, ddelta, rows, pad_rows,
                               static_cast<int>(H));
  }
  if (rows > 0x7fffffff) return kInvalid;
  return launch_kernel(rmsnorm_bwd_generic_kernel, dim3(static_cast<unsigned>(rows)),
                       dim3(kGenThreads), st, s, rstd, w, dy, dypad, pad_idx, ds, dx, ddelta, rows,
                       pad_rows, H);
}
