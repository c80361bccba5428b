// Gated SiLU (SwiGLU) forward and in-place backward over the fused [gate | up] GEMM output.
//
// Reference: solution/mlp.py:31-40 (gated_silu_fwd_kernel), solution/mlp.py:43-58
// (gated_silu_bwd_inplace_kernel), launched from gated_silu / gated_silu_backward_,
// solution/mlp.py:61-77.
//
// Pure HBM streaming.  The flat index space is rows * I/8 chunks of 8 fp16 (16 bytes); chunk c
// lives in row r = c / (I/8), and because act is [rows, I] contiguous its chunk offset is 8c,
// while gate sits at 8c + r*I and up at 8c + r*I + I of the [rows, 2I] buffer.  Each thread
// issues all loads of its kSwiUnroll chunks back to back before any arithmetic; one chunk per
// thread (many small workgroups) measured fastest on MI355X.  Arithmetic is fp32: exp through
// v_exp_f32, the reciprocal through v_rcp_f32 (both about 1 ulp of fp32, far below the fp16
// rounding of the result).

#include "fastdiv.hpp"
#include "soupk_common.hpp"

namespace soupk {
namespace {

constexpr int kSwiThreads = 256;
#ifndef SOUPK_SWI_UNROLL
#define SOUPK_SWI_UNROLL 1
#endif
constexpr int kSwiUnroll = SOUPK_SWI_UNROLL;  // 16-byte chunks per thread per workgroup tile

__device__ __forceinline__ float sigmoid_f(float g) {
  return __builtin_amdgcn_rcpf(1.0f + fast_exp(-g));
}

__device__ __forceinline__ uint32_t silu_mul_word(uint32_t gw, uint32_t uw) {
  const float g0 = lo_h(gw), g1 = hi_h(gw);
  const float u0 = lo_h(uw), u1 = hi_h(uw);
  return pack_h2(g0 * sigmoid_f(g0) * u0, g1 * sigmoid_f(g1) * u1);
}

// Returns {d gate word, d up word} for one dword (two fp16) of dact, gate and up.
__device__ __forceinline__ u32x2 silu_bwd_word(uint32_t dw, uint32_t gw, uint32_t uw) {
  float dg[2], du[2];
  const float d[2] = {lo_h(dw), hi_h(dw)};
  const float g[2] = {lo_h(gw), hi_h(gw)};
  const float u[2] = {lo_h(uw), hi_h(uw)};
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const float sig = sigmoid_f(g[j]);
    const float d_silu = d[j] * u[j];
    dg[j] = d_silu * sig * (1.0f + g[j] * (1.0f - sig));
    du[j] = d[j] * (g[j] * sig);
  }
  return u32x2{pack_h2(dg[0], dg[1]), pack_h2(du[0], du[1])};
}

// Cache policy of the streamed loads (1 = non-temporal: each operand is touched once per
// launch; cached loads ran 15% slower on MI355X and slowed the kernels that follow).  The
// results are written with streaming stores (StreamOut: nt | sc1).
#ifndef SOUPK_SWI_NT_LD
#define SOUPK_SWI_NT_LD 1
#endif
constexpr bool kSwiNtLd = SOUPK_SWI_NT_LD != 0;

// One workgroup = one tile of kSwiThreads * kSwiUnroll chunks; chunk k*kSwiThreads + tid of the
// tile per thread, so each wave load/store instruction covers 1 KiB contiguous.  All loads are
// issued unconditionally (indices past the end are clamped to the last chunk and their results
// dropped): a predicated load would make the compiler wait on it before issuing the next.
__global__ __launch_bounds__(kSwiThreads) void swiglu_fwd_vec_kernel(
    const u32x4* __restrict__ gu, u32x4* __restrict__ act, uint32_t n_chunks, FastDiv row_of,
    uint32_t I_chunks) {
  const uint32_t c0 = blockIdx.x * (kSwiThreads * kSwiUnroll);
  const uint32_t base = c0 + threadIdx.x;
  // Stores of the tile: chunk c at byte 16 (c - c0) of a descriptor from chunk c0 to the end of
  // act (chunks past the end fall outside it and are dropped).
  const StreamOut out(act + c0, static_cast<uint64_t>(n_chunks - c0) * 16u);
  u32x4 g[kSwiUnroll], u[kSwiUnroll];
#pragma unroll
  for (int k = 0; k < kSwiUnroll; ++k) {
    const uint32_t c = min(base + k * kSwiThreads, n_chunks - 1);
    const uint64_t gi = static_cast<uint64_t>(c) + static_cast<uint64_t>(row_of.div(c)) *
                                                       I_chunks;
    g[k] = ld<kSwiNtLd>(gu + gi);
    u[k] = ld<kSwiNtLd>(gu + gi + I_chunks);
  }
#pragma unroll
  for (int k = 0; k < kSwiUnroll; ++k) {
    const uint32_t c = base + k * kSwiThreads;
    const u32x4 r = {silu_mul_word(g[k].x, u[k].x), silu_mul_word(g[k].y, u[k].y),
                     silu_mul_word(g[k].z, u[k].z), silu_mul_word(g[k].w, u[k].w)};
    out.store((c - c0) * 16u, r);
  }
}

__global__ __launch_bounds__(kSwiThreads) void swiglu_bwd_vec_kernel(
    const u32x4* __restrict__ dact, u32x4* __restrict__ gu, uint32_t n_chunks, FastDiv row_of,
    uint32_t I_chunks) {
  const uint32_t c0 = blockIdx.x * (kSwiThreads * kSwiUnroll);
  const uint32_t base = c0 + threadIdx.x;
  // Stores of the tile relative to the tile's first gate chunk g0 (the host keeps the tile's
  // span, under two rows of gate|up plus a tile, below 2^32 bytes).
  const uint64_t g0 = static_cast<uint64_t>(c0) + static_cast<uint64_t>(row_of.div(c0)) * I_chunks;
  const StreamOut out(gu + g0, (2ull * n_chunks - g0) * 16u);
  u32x4 d[kSwiUnroll], g[kSwiUnroll], u[kSwiUnroll];
  uint64_t gi[kSwiUnroll];
#pragma unroll
  for (int k = 0; k < kSwiUnroll; ++k) {
    const uint32_t c = min(base + k * kSwiThreads, n_chunks - 1);
    gi[k] = static_cast<uint64_t>(c) + static_cast<uint64_t>(row_of.div(c)) * I_chunks;
    d[k] = ld<kSwiNtLd>(dact + c);
    g[k] = ld<kSwiNtLd>(gu + gi[k]);
    u[k] = ld<kSwiNtLd>(gu + gi[k] + I_chunks);
  }
#pragma unroll
  for (int k = 0; k < kSwiUnroll; ++k) {
    const uint32_t c = base + k * kSwiThreads;
    const u32x2 r0 = silu_bwd_word(d[k].x, g[k].x, u[k].x);
    const u32x2 r1 = silu_bwd_word(d[k].y, g[k].y, u[k].y);
    const u32x2 r2 = silu_bwd_word(d[k].z, g[k].z, u[k].z);
    const u32x2 r3 = silu_bwd_word(d[k].w, g[k].w, u[k].w);
    // (a thread past the end holds the last chunk's indices: its store would overwrite that
    // chunk's result in place, so it stores nothing)
    if (c < n_chunks) {
      const uint32_t off = static_cast<uint32_t>(gi[k] - g0) * 16u;
      out.store(off, u32x4{r0.x, r1.x, r2.x, r3.x});
      out.store(off + I_chunks * 16u, u32x4{r0.y, r1.y, r2.y, r3.y});
    }
  }
}

// Element-wise forms for shapes the vector kernels do not take (I % 8 != 0, unaligned).
__global__ __launch_bounds__(kSwiThreads) void swiglu_fwd_elem_kernel(
    const uint16_t* __restrict__ gu, uint16_t* __restrict__ act, int64_t n, int64_t I) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * kSwiThreads + threadIdx.x;
  if (e >= n) return;
  const int64_t r = e / I;
  const int64_t gi = e + r * I;
  const float g = h2f(gu[gi]), u = h2f(gu[gi + I]);
  act[e] = static_cast<uint16_t>(pack_h2(g * sigmoid_f(g) * u, 0.0f) & 0xffffu);
}

__global__ __launch_bounds__(kSwiThreads) void swiglu_bwd_elem_kernel(
    const uint16_t* __restrict__ dact, uint16_t* __restrict__ gu, int64_t n, int64_t I) {
  const int64_t e = static_cast<int64_t>(blockIdx.x) * kSwiThreads + threadIdx.x;
  if (e >= n) return;
  const int64_t gi = e + (e / I) * I;
  const u32x2 r = silu_bwd_word(dact[e], gu[gi], gu[gi + I]);
  gu[gi] = static_cast<uint16_t>(r.x & 0xffffu);
  gu[gi + I] = static_cast<uint16_t>(r.y & 0xffffu);
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline unsigned vec_grid(uint32_t n_chunks) {
  const uint32_t tile = kSwiThreads * kSwiUnroll;
  return (n_chunks + tile - 1) / tile;
}

}  // namespace
}  // namespace soupk

using namespace soupk;

extern "C" __attribute__((visibility("default"))) int soupk_swiglu_fwd(const uint16_t* gu,
                                                                        uint16_t* act,
                                                                        int64_t rows, int64_t I,
                                                                        void* stream) {
  if (rows < 0 || I < 0) return kInvalid;
  const int64_t n = rows * I;
  if (n == 0) return kOk;
  if (!gu || !act) return kInvalid;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (I % 8 == 0 && n / 8 < (int64_t{1} << 31) && aligned16(gu) && aligned16(act)) {
    const uint32_t n_chunks = static_cast<uint32_t>(n / 8);
    const uint32_t I_chunks = static_cast<uint32_t>(I / 8);
    return launch_kernel(swiglu_fwd_vec_kernel, dim3(vec_grid(n_chunks)), dim3(kSwiThreads), s,
                         reinterpret_cast<const u32x4*>(gu), reinterpret_cast<u32x4*>(act),
                         n_chunks, FastDiv(I_chunks), I_chunks);
  }
  const int64_t grid = (n + kSwiThreads - 1) / kSwiThreads;
  if (grid > 0x7fffffff) return kInvalid;
  return launch_kernel(swiglu_fwd_elem_kernel, dim3(static_cast<unsigned>(grid)),
                       dim3(kSwiThreads), s, gu, act, n, I);
}

extern "C" __attribute__((visibility("default"))) int soupk_swiglu_bwd_inplace(
    const uint16_t* dact, uint16_t* gu, int64_t rows, int64_t I, void* stream) {
  if (rows < 0 || I < 0) return kInvalid;
  const int64_t n = rows * I;
  if (n == 0) return kOk;
  if (!gu || !dact) return kInvalid;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (I % 8 == 0 && n / 8 < (int64_t{1} << 31) && I / 8 < (int64_t{1} << 26) && aligned16(gu) &&
      aligned16(dact)) {
    const uint32_t n_chunks = static_cast<uint32_t>(n / 8);
    const uint32_t I_chunks = static_cast<uint32_t>(I / 8);
    return launch_kernel(swiglu_bwd_vec_kernel, dim3(vec_grid(n_chunks)), dim3(kSwiThreads), s,
                         reinterpret_cast<const u32x4*>(dact), reinterpret_cast<u32x4*>(gu),
                         n_chunks, FastDiv(I_chunks), I_chunks);
  }
  const int64_t grid = (n + kSwiThreads - 1) / kSwiThreads;
  if (grid > 0x7fffffff) return kInvalid;
  return launch_kernel(swiglu_bwd_elem_kernel, dim3(static_cast<unsigned>(grid)),
                       dim3(kSwiThreads), s, dact, gu, n, I);
}
