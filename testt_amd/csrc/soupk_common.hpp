// Device helpers shared by the soupk kernels.  gfx950 (CDNA4) only: wave64, 16-byte vector
// memory accesses, fp32 arithmetic with round-to-nearest-even fp16 stores.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "../../include/soupk.h"

// Products and sums are rounded one at a time everywhere in this library, as the eager PyTorch
// path and the NF4 closed form round them.  (The build also passes -ffp-contract=off.)
#pragma clang fp contract(off)

namespace soupk {

typedef _Float16 f16;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ---- status codes (hipError_t values) -------------------------------------------------------
constexpr int kOk = 0;
constexpr int kInvalid = 1;  // hipErrorInvalidValue

inline int launch_status() { return static_cast<int>(hipGetLastError()); }

// Number of compute units of the current device (256 on MI355X), cached per device ordinal.
int device_cu_count();

// Events set by soupk_time_next_launch() on the calling thread, handed to (and cleared by) the
// next kernel launch of that thread.
void take_timing_events(hipEvent_t* start, hipEvent_t* stop);

// Every kernel launch of the library goes through here: a plain launch, or, when the calling
// thread armed soupk_time_next_launch(), a launch whose dispatch itself records the two events
// (hipExtLaunchKernelGGL), so they time the kernel and nothing else.
template <typename... KArgs, typename... Args>
int launch_kernel(void (*kernel)(KArgs...), dim3 grid, dim3 block, hipStream_t stream,
                  Args... args) {
  hipEvent_t start = nullptr, stop = nullptr;
  take_timing_events(&start, &stop);
  if (start != nullptr || stop != nullptr)
    hipExtLaunchKernelGGL(kernel, grid, block, 0, stream, start, stop, 0,
                          static_cast<KArgs>(args)...);
  else
    kernel<<<grid, block, 0, stream>>>(static_cast<KArgs>(args)...);
  return launch_status();
}

// ---- fp16 <-> fp32 ---------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint32_t bits16) {
  return static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(bits16)));
}
// One dword as two fp16.  Always pass a scalar: hipcc (clang 22) lowers
// __builtin_bit_cast(f16x2, v.y) of an ext-vector element as a read of element 0.
__device__ __forceinline__ f16x2 as_h2(uint32_t w) { return __builtin_bit_cast(f16x2, w); }
__device__ __forceinline__ float lo_h(uint32_t w) { return h2f(w & 0xffffu); }
__device__ __forceinline__ float hi_h(uint32_t w) { return h2f(w >> 16); }
// Two fp32 -> one dword of two fp16 (round to nearest even), `a` at the lower address.
// The empty asm makes a and b opaque fp32 values: without it the compiler may fuse the multiply
// that produced them with the conversion into v_fma_mix*_f16, which rounds the exact product
// once to fp16 instead of rounding to fp32 first (as the eager path and the reference do); the
// two differ when the fp32 value lands on an fp16 rounding tie.
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  asm("" : "+v"(a), "+v"(b));
  f16x2 v = {static_cast<f16>(a), static_cast<f16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

// ---- buffer (MUBUF) access with hardware range checking ----------------------------------------
// A raw buffer descriptor over [base, base + bytes): loads at offsets >= bytes return 0 and
// stores there are dropped, so a kernel can issue whole-wave accesses past the end of a row
// without a predicate (which would make the compiler wait on every load) and without a fault.
// Word 3 (0x00020000) is the gfx9-family format word for raw 32-bit-addressed buffers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes),
                                           0x00020000);
}
constexpr int kAuxNonTemporal = 2;  // cache-policy bits of buffer ops: streaming (nt)

// ---- streaming stores: non-temporal at device scope ------------------------------------------
// Streams written once per launch go out through a buffer descriptor with the cache policy
// nt | sc1 (non-temporal, device scope).  Plain 16-byte copies of 17 - 183 MB on MI355X,
// timed per dispatch, ran 2 - 5% faster with it than with nt alone (the most on the shortest
// copies); loads gained nothing from the scope bits.  A vector global store cannot carry sc1
// from HIP source; a buffer store takes it in its cache-policy operand.  The descriptor is made
// from a wave-uniform base (kernel arguments, blockIdx, readfirstlane values) and covers `bytes`
// from it: the hardware drops stores at byte offsets >= bytes.
constexpr int kAuxStream = 2 | 16;  // nt | sc1
// (A kernel may take nt alone, Aux = kAuxNonTemporal, where that measured faster.)
template <int Aux>
struct StreamOutT {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ StreamOutT(const void* base, uint64_t bytes)
      : r(buffer_rsrc(base, bytes > 0xffffffffull ? 0xffffffffu
                                                  : static_cast<uint32_t>(bytes))) {}
  __device__ __forceinline__ void store(uint32_t off, u32x4 v) const {
    __builtin_amdgcn_raw_buffer_store_b128(v, r, static_cast<int>(off), 0, Aux);
  }
  __device__ __forceinline__ void store(uint32_t off, f32x4 v) const {
    store(off, __builtin_bit_cast(u32x4, v));
  }
  __device__ __forceinline__ void store(uint32_t off, u32x2 v) const {
    __builtin_amdgcn_raw_buffer_store_b64(v, r, static_cast<int>(off), 0, Aux);
  }
};
using StreamOut = StreamOutT<kAuxStream>;

// ---- streaming (non-temporal) or cached global access, chosen at compile time ---------------
// Data read or written exactly once per launch streams past the caches when NT is true.
template <bool NT, typename T>
__device__ __forceinline__ T ld(const T* p) {
  if constexpr (NT) return __builtin_nontemporal_load(p);
  else return *p;
}
template <bool NT, typename T>
__device__ __forceinline__ void st(T* p, T v) {
  if constexpr (NT) __builtin_nontemporal_store(v, p);
  else *p = v;
}

// ---- wave64 reductions (every lane ends with the result) -------------------------------------
// Four DPP steps combine the 16 lanes of each row (quad swaps, then the half-row and row
// mirrors: every lane ends with its row's result) and v_readlane_b32 brings the four rows
// together: no LDS permute round trips (a shuffle butterfly needs six, one after another).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
constexpr int kDppQuad1032 = 0xb1;     // quad_perm [1,0,3,2]
constexpr int kDppQuad2301 = 0x4e;     // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppMirror = 0x140;      // row_mirror

__device__ __forceinline__ float row16_sum(float v) {
  v = v + dpp_f<kDppQuad1032>(v);
  v = v + dpp_f<kDppQuad2301>(v);
  v = v + dpp_f<kDppHalfMirror>(v);
  return v + dpp_f<kDppMirror>(v);
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<kDppQuad1032>(v));
  v = fmaxf(v, dpp_f<kDppQuad2301>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  return fmaxf(v, dpp_f<kDppMirror>(v));
}
__device__ __forceinline__ int row16_min(int v) {
  v = min(v, dpp_i<kDppQuad1032>(v));
  v = min(v, dpp_i<kDppQuad2301>(v));
  v = min(v, dpp_i<kDppHalfMirror>(v));
  return min(v, dpp_i<kDppMirror>(v));
}
// Value of lane l (a wave-uniform constant or register) as a wave-uniform float.
__device__ __forceinline__ float lanef(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}
__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  return (lanef(v, 0) + lanef(v, 16)) + (lanef(v, 32) + lanef(v, 48));
}

// ---- exp via the hardware base-2 exponential ------------------------------------------------
// exp(x) = 2^(x*log2 e).  v_exp_f32 is accurate to about 1 ulp; the rounding of x*log2(e)
// adds |x|*2^-24 relative error, far below the fp16 output rounding these kernels feed.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

}  // namespace soupk
