// Device helpers shared by the soupk kernels.  gfx950 (CDNA4) only: wave64, 16-byte vector
// memory accesses, fp32 arithmetic with round-to-nearest-even fp16 stores.
#pragma once

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

// ---- status codes (hipError_t values) -------------------------------------------------------
constexpr int kOk = 0;
constexpr int kInvalid = 1;  // hipErrorInvalidValue

inline int launch_status() { return static_cast<int>(hipGetLastError()); }

// Number of compute units of the current device (256 on MI355X), cached per device ordinal.
int device_cu_count();

// ---- fp16 <-> fp32 ---------------------------------------------------------------------------
__device__ __forceinline__ float h2f(uint32_t bits16) {
  return static_cast<float>(__builtin_bit_cast(f16, static_cast<uint16_t>(bits16)));
}
__device__ __forceinline__ float lo_h(uint32_t w) { return h2f(w & 0xffffu); }
__device__ __forceinline__ float hi_h(uint32_t w) { return h2f(w >> 16); }
// Two fp32 -> one dword of two fp16 (round to nearest even), `a` at the lower address.
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  f16x2 v = {static_cast<f16>(a), static_cast<f16>(b)};
  return __builtin_bit_cast(uint32_t, v);
}

// ---- wave64 reductions (butterfly: every lane ends with the result) -------------------------
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
  return v;
}

// ---- exp via the hardware base-2 exponential ------------------------------------------------
// exp(x) = 2^(x*log2 e).  v_exp_f32 is accurate to about 1 ulp; the rounding of x*log2(e)
// adds |x|*2^-24 relative error, far below the fp16 output rounding these kernels feed.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }

}  // namespace soupk
