// Sum of split-K partial products: out = fp16_rn(((p[0] + p[1]) + p[2]) + ...), fp32 partials.
//
// The reference computes the gate|up input gradient of the MLP backward as one fp16 GEMM
// (grad_x = d(gate|up) @ [W_gate; W_up], solution/mlp.py:105-113, K = 2 * 8960).  Its output
// is only [2048 x 1536], too few tiles for 256 CUs, so on MI355X the product is split along K
// into batched GEMMs with fp32 outputs (hipBLASLt) and this kernel adds the partials in a
// fixed order and rounds once to fp16: one fp16 rounding of an fp32-accumulated sum, as a single
// GEMM gives, with a different (still deterministic) summation order.
//
// Pure HBM streaming: each thread reads 4 chunks of 4 consecutive floats of every partial
// (16-byte non-temporal loads, the workgroup's chunks 256 apart, all issued before the first
// add) and writes 4 x 4 fp16 (8-byte streaming stores).

#include "soupk_common.hpp"

namespace soupk {
namespace {

constexpr int kRedThreads = 256;
constexpr int kMaxPartials = 16;

// 16-byte chunks of each partial per thread, all loads issued before the first add: the
// gate|up input gradient's four [2048 x 1536] partials (56.6 MB moved) in 9.93 us with 4
// against 10.44 us with 2, 10.91 us with 1 and 10.33 us with 8 (MI355X, HBM-resident inputs).
#ifndef SOUPK_SUM_CHUNKS
#define SOUPK_SUM_CHUNKS 4
#endif
constexpr int kChunks = SOUPK_SUM_CHUNKS;

template <int P>
__global__ __launch_bounds__(kRedThreads) void sum_partials_kernel(
    const f32x4* __restrict__ parts, int64_t stride4, int64_t n4, u32x2* __restrict__ out) {
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * kRedThreads * kChunks;
  f32x4 v[kChunks][P];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    const int64_t i = min(i0 + c * kRedThreads + threadIdx.x, n4 - 1);
#pragma unroll
    for (int p = 0; p < P; ++p) v[c][p] = ld<true>(parts + p * stride4 + i);
  }
  // Streaming store through a descriptor over the workgroup's slice of out (chunks past n4
  // are dropped by its range).
  const StreamOut dst(out + i0, static_cast<uint64_t>(n4 - i0) * 8u);
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    f32x4 s = v[c][0];
#pragma unroll
    for (int p = 1; p < P; ++p) s = s + v[c][p];
    dst.store(static_cast<uint32_t>(c * kRedThreads + threadIdx.x) * 8u,
              u32x2{pack_h2(s[0], s[1]), pack_h2(s[2], s[3])});
  }
}

// Any count of partials (up to kMaxPartials) and any n: one element per thread.
__global__ __launch_bounds__(kRedThreads) void sum_partials_scalar_kernel(
    const float* __restrict__ parts, int n_parts, int64_t stride, int64_t first, int64_t n,
    uint16_t* __restrict__ out) {
  const int64_t i = first + static_cast<int64_t>(blockIdx.x) * kRedThreads + threadIdx.x;
  if (i >= n) return;
  float s = parts[i];
  for (int p = 1; p < n_parts; ++p) s = s + parts[p * stride + i];
  out[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(s));
}

template <int P>
int launch_vec(const float* parts, int64_t stride, int64_t n4, uint16_t* out, hipStream_t st) {
  const int64_t grid = (n4 + kRedThreads * kChunks - 1) / (kRedThreads * kChunks);
  if (grid > 0x7fffffff) return kInvalid;
  return launch_kernel(sum_partials_kernel<P>, dim3(static_cast<unsigned>(grid)),
                       dim3(kRedThreads), st, reinterpret_cast<const f32x4*>(parts), stride / 4,
                       n4, reinterpret_cast<u32x2*>(out));
}

}  // namespace
}  // namespace soupk

using namespace soupk;

extern "C" __attribute__((visibility("default"))) int soupk_sum_partials(
    const float* parts, int32_t n_parts, int64_t part_stride, int64_t n, uint16_t* out_f16,
    void* stream) {
  if (n_parts < 1 || n_parts > kMaxPartials || n < 0 || part_stride < n) return kInvalid;
  if (n == 0) return kOk;
  if (!parts || !out_f16) return kInvalid;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int64_t done = 0;
  const bool vec = (reinterpret_cast<uintptr_t>(parts) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(out_f16) & 7) == 0 && part_stride % 4 == 0;
  if (vec && n >= 4) {
    const int64_t n4 = n / 4;
    int rc = kInvalid;
    switch (n_parts) {
      case 1: rc = launch_vec<1>(parts, part_stride, n4, out_f16, st); break;
      case 2: rc = launch_vec<2>(parts, part_stride, n4, out_f16, st); break;
      case 3: rc = launch_vec<3>(parts, part_stride, n4, out_f16, st); break;
      case 4: rc = launch_vec<4>(parts, part_stride, n4, out_f16, st); break;
      case 5: rc = launch_vec<5>(parts, part_stride, n4, out_f16, st); break;
      case 6: rc = launch_vec<6>(parts, part_stride, n4, out_f16, st); break;
      case 7: rc = launch_vec<7>(parts, part_stride, n4, out_f16, st); break;
      case 8: rc = launch_vec<8>(parts, part_stride, n4, out_f16, st); break;
      default: rc = -1; break;     // more partials: the scalar kernel below
    }
    if (rc > 0) return rc;
    if (rc == kOk) done = n4 * 4;
  }
  if (done < n) {
    const int64_t grid = (n - done + kRedThreads - 1) / kRedThreads;
    if (grid > 0x7fffffff) return kInvalid;
    return launch_kernel(sum_partials_scalar_kernel, dim3(static_cast<unsigned>(grid)),
                         dim3(kRedThreads), st, parts, n_parts, part_stride, done, n, out_f16);
  }
  return kOk;
}
