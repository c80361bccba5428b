// The LoRA branch of the q and v projections (peft's lora_B(lora_A(x)) * scaling under fp16
// autocast, solution/model.py:195-206 with dropout 0), for rank 16, in two launches per
// direction instead of a dozen small GEMMs, casts and scalings:
//
//   soupk_lora_fwd:       t  = fp16(y A^T)                        [M, 2r]  (A = A_q | A_v)
//                         lq = fp16(fp16(t_q B_q^T) * scaling)    [M, NQ]
//                         lv = fp16(fp16(t_v B_v^T) * scaling)    [M, NV]
//   soupk_lora_bwd_rows:  gs_x = fp16(g_x * scaling)              (g_x: the gradients of lq, lv)
//                         dt   = fp16(gs_q B_q | gs_v B_v)        [M, 2r]
//                         dy   = fp16(dt A16)                     [M, H]
// with fp16(.) the rounding of an fp16 GEMM (fp32 sums, one rounding) and A16, B16 the fp16
// casts of the fp32 LoRA parameters, rounded here as .to(torch.float16) rounds them.  The
// caller then adds the frozen projection's input gradient into dy in place and forms the
// parameter gradients (B_x: gs_x^T t_x, A: dt^T y) from gs, t and dt.
//
// A workgroup is 4 wavefronts and 16 rows.  The long contractions (over H for t, over NQ / NV
// for dt) run on v_mfma_f32_16x16x32_f16 with the contraction split over the 4 wavefronts and
// the partial sums added in wavefront order (deterministic).  The short ones (over r for lq/lv,
// on v_mfma_f32_16x16x16f16; over 2r for dy, on 16x16x32) are computed transposed, one 16-column
// tile at a time: (out tile)^T = W16 x^T, so that a lane's four results are four consecutive
// columns of one row (one 8-byte store).  MFMA layouts: A lane l holds row l%16, B lane l
// column l%16, each with k = 8(l/16)..+7 (16x16x32) or 4(l/16)..+3 (16x16x16); C lane l holds
// column l%16, rows 4(l/16)..+3.

#include "soupk_common.hpp"

namespace soupk {
namespace {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kR = 16;           // LoRA rank
constexpr int kRows = 16;        // rows per workgroup
constexpr int kThreads = 256;

__device__ __forceinline__ f4 mfma32(h8 a, h8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float r16(float x) { return static_cast<float>(static_cast<_Float16>(x)); }

// Eight consecutive fp32 values rounded to fp16.
__device__ __forceinline__ h8 cast8(const float* p) {
  const f4 a = *reinterpret_cast<const f4*>(p), b = *reinterpret_cast<const f4*>(p + 4);
  h8 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    r[i] = static_cast<_Float16>(a[i]);
    r[4 + i] = static_cast<_Float16>(b[i]);
  }
  return r;
}

__device__ __forceinline__ uint16_t h_bits(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }

__global__ __launch_bounds__(kThreads) void lora_fwd_kernel(
    const uint16_t* __restrict__ y, const float* __restrict__ aq, const float* __restrict__ av,
    const float* __restrict__ bq, const float* __restrict__ bv, float scaling,
    uint16_t* __restrict__ t_out, uint16_t* __restrict__ lq, uint16_t* __restrict__ lv, int M,
    int H, int NQ, int NV) {
  __shared__ float part[4][kRows][2 * kR + 1];
  __shared__ float tt[kRows][2 * kR];
  const int m0 = blockIdx.x * kRows;
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int ql = lane & 15, gr = lane >> 4;
  const int64_t row = min(m0 + ql, M - 1);
  // t = y A^T: A operand = y rows (row ql, k = k0 + 8gr..+7); B operand = A_q / A_v rows
  // (column = feature ql).  The contraction over H is split over the 4 wavefronts.
  const int kw = H / 4;
  f4 acc_q = {0.f, 0.f, 0.f, 0.f}, acc_v = {0.f, 0.f, 0.f, 0.f};
  const uint16_t* yrow = y + row * H;

  for (int k0 = w * kw; k0 < (w + 1) * kw; k0 += 32) {
    const h8 ya = *reinterpret_cast<const h8*>(yrow + k0 + 8 * gr);
    const h8 qa = cast8(aq + static_cast<int64_t>(ql) * H + k0 + 8 * gr);
    const h8 va = cast8(av + static_cast<int64_t>(ql) * H + k0 + 8 * gr);
    acc_q = mfma32(ya, qa, acc_q);
    acc_v = mfma32(ya, va, acc_v);
  }
  // C: column = feature ql, rows 4gr .. +3
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    part[w][4 * gr + i][ql] = acc_q[i];
    part[w][4 * gr + i][kR + ql] = acc_v[i];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < kRows * 2 * kR; e += kThreads) {
    const int m = e / (2 * kR), f = e % (2 * kR);
    const float s = ((part[0][m][f] + part[1][m][f]) + part[2][m][f]) + part[3][m][f];
    const _Float16 h = static_cast<_Float16>(s);
    tt[m][f] = static_cast<float>(h);
    if (m0 + m < M) t_out[static_cast<int64_t>(m0 + m) * (2 * kR) + f] = h_bits(h);
  }
  __syncthreads();
  // lq, lv: tile f0..f0+15 of the output columns, transposed: A = B16 rows (feature f0 + ql,
  // k = rank 4gr..+3), B = t rows (column = row ql of the workgroup, same k)
  const int nq16 = NQ / 16, n16 = nq16 + NV / 16;
  for (int tile = w; tile < n16; tile += 4) {
    const bool is_q = tile < nq16;
    const int f0 = 16 * (is_q ? tile : tile - nq16);
    const int N = is_q ? NQ : NV;
    const f4 bw = *reinterpret_cast<const f4*>((is_q ? bq : bv) +
                                               static_cast<int64_t>(f0 + ql) * kR + 4 * gr);
    const h4 a = {static_cast<_Float16>(bw[0]), static_cast<_Float16>(bw[1]),
                  static_cast<_Float16>(bw[2]), static_cast<_Float16>(bw[3])};
    const float* trow = &tt[ql][(is_q ? 0 : kR) + 4 * gr];
    const h4 b = {static_cast<_Float16>(trow[0]), static_cast<_Float16>(trow[1]),
                  static_cast<_Float16>(trow[2]), static_cast<_Float16>(trow[3])};
    const f4 c = mfma16(a, b, f4{0.f, 0.f, 0.f, 0.f});
    // C: column = row ql, rows = features f0 + 4gr .. +3
    if (m0 + ql < M) {
      uint16_t* dst = (is_q ? lq : lv) + static_cast<int64_t>(m0 + ql) * N + f0 + 4 * gr;
      *reinterpret_cast<u32x2*>(dst) =
          u32x2{pack_h2(r16(c[0]) * scaling, r16(c[1]) * scaling),
                pack_h2(r16(c[2]) * scaling, r16(c[3]) * scaling)};
    }
  }
}

__global__ __launch_bounds__(kThreads) void lora_bwd_rows_kernel(
    const uint16_t* __restrict__ gq, int64_t ldq, const uint16_t* __restrict__ gv, int64_t ldv,
    const float* __restrict__ aq, const float* __restrict__ av, const float* __restrict__ bq,
    const float* __restrict__ bv, float scaling, uint16_t* __restrict__ gsq,
    uint16_t* __restrict__ gsv, uint16_t* __restrict__ dt_out, uint16_t* __restrict__ dy, int M,
    int H, int NQ, int NV) {
  __shared__ float part[4][kRows][2 * kR + 1];
  __shared__ float dts[kRows][2 * kR];
  const int m0 = blockIdx.x * kRows;
  const int lane = threadIdx.x % kWave, w = threadIdx.x / kWave;
  const int ql = lane & 15, gr = lane >> 4;
  const int mr = m0 + ql;
  const int64_t row = min(mr, M - 1);
  const bool row_ok = mr < M;
  // dt_x = gs_x B16_x: A operand = gs rows (row ql, k = j0 + 8gr..+7), stored as gs on the
  // way; B operand = B16 (column = rank index ql, k = j rows: B is [N, r] row-major, so the
  // 8 k-values of a lane are 8 rows, each read by 16 consecutive lanes as 64 contiguous bytes)
  f4 acc_q = {0.f, 0.f, 0.f, 0.f}, acc_v = {0.f, 0.f, 0.f, 0.f};
  auto step = [&](const uint16_t* g, int64_t ldg, uint16_t* gs, int N, const float* b, int j0,
                  f4& acc) {
    const h8 graw = *reinterpret_cast<const h8*>(g + row * ldg + j0 + 8 * gr);
    h8 ga;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      ga[i] = static_cast<_Float16>(static_cast<float>(graw[i]) * scaling);
    if (row_ok) *reinterpret_cast<h8*>(gs + static_cast<int64_t>(mr) * N + j0 + 8 * gr) = ga;
    h8 ba;
#pragma unroll
    for (int i = 0; i < 8; ++i)
      ba[i] = static_cast<_Float16>(b[static_cast<int64_t>(j0 + 8 * gr + i) * kR + ql]);
    acc = mfma32(ga, ba, acc);
  };
  const int kq = NQ / 4, kv = NV / 4;

  for (int j0 = w * kq; j0 < (w + 1) * kq; j0 += 32) step(gq, ldq, gsq, NQ, bq, j0, acc_q);

  for (int j0 = w * kv; j0 < (w + 1) * kv; j0 += 32) step(gv, ldv, gsv, NV, bv, j0, acc_v);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    part[w][4 * gr + i][ql] = acc_q[i];
    part[w][4 * gr + i][kR + ql] = acc_v[i];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < kRows * 2 * kR; e += kThreads) {
    const int m = e / (2 * kR), f = e % (2 * kR);
    const float s = ((part[0][m][f] + part[1][m][f]) + part[2][m][f]) + part[3][m][f];
    const _Float16 h = static_cast<_Float16>(s);
    dts[m][f] = static_cast<float>(h);
    if (m0 + m < M) dt_out[static_cast<int64_t>(m0 + m) * (2 * kR) + f] = h_bits(h);
  }
  __syncthreads();
  // dy = dt A16 (contraction over the 2r rank indices; A = A_q rows then A_v rows), one
  // 16-column tile of H at a time, transposed: A operand = A16 columns (row h0 + ql, k = rank
  // 8gr..+7: 8 rows of A, each read by 16 consecutive lanes as 64 contiguous bytes), B = dt
  // rows (column = row ql)
  for (int tile = w; tile < H / 16; tile += 4) {
    const int h0 = 16 * tile;
    const float* acol = (gr < 2 ? aq + static_cast<int64_t>(8 * gr) * H
                                : av + static_cast<int64_t>(8 * (gr - 2)) * H) + h0 + ql;
    h8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[i] = static_cast<_Float16>(acol[static_cast<int64_t>(i) * H]);
      b[i] = static_cast<_Float16>(dts[ql][8 * gr + i]);
    }
    const f4 c = mfma32(a, b, f4{0.f, 0.f, 0.f, 0.f});
    if (m0 + ql < M)
      *reinterpret_cast<u32x2*>(dy + static_cast<int64_t>(m0 + ql) * H + h0 + 4 * gr) =
          u32x2{pack_h2(c[0], c[1]), pack_h2(c[2], c[3])};
  }
}

int check_dims(int64_t M, int32_t H, int32_t NQ, int32_t NV, int32_t r) {
  if (M < 0 || r != kR || H <= 0 || NQ <= 0 || NV <= 0) return kInvalid;
  if (H % 128 || NQ % 128 || NV % 128) return kInvalid;   // 4-way split of 32-wide steps
  if ((M + kRows - 1) / kRows > 0x7fffffff || M * static_cast<int64_t>(H) >= (int64_t{1} << 40))
    return kInvalid;
  return kOk;
}

bool misaligned(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) != 0; }

}  // namespace
}  // namespace soupk

using namespace soupk;

extern "C" __attribute__((visibility("default"))) int soupk_lora_fwd(
    const uint16_t* y, const float* a_q, const float* a_v, const float* b_q, const float* b_v,
    float scaling, uint16_t* t, uint16_t* lq, uint16_t* lv, int64_t M, int32_t H, int32_t NQ,
    int32_t NV, int32_t r, void* stream) {
  const int rc = check_dims(M, H, NQ, NV, r);
  if (rc != kOk) return rc;
  if (M == 0) return kOk;
  if (!y || !a_q || !a_v || !b_q || !b_v || !t || !lq || !lv) return kInvalid;
  for (const void* p : {static_cast<const void*>(y), static_cast<const void*>(a_q),
                        static_cast<const void*>(a_v), static_cast<const void*>(b_q),
                        static_cast<const void*>(b_v), static_cast<const void*>(lq),
                        static_cast<const void*>(lv)})
    if (misaligned(p)) return kInvalid;
  const unsigned grid = static_cast<unsigned>((M + kRows - 1) / kRows);
  return launch_kernel(lora_fwd_kernel, dim3(grid), dim3(kThreads),
                       static_cast<hipStream_t>(stream), y, a_q, a_v, b_q, b_v, scaling, t, lq,
                       lv, static_cast<int>(M), H, NQ, NV);
}

extern "C" __attribute__((visibility("default"))) int soupk_lora_bwd_rows(
    const uint16_t* g_q, int64_t ld_q, const uint16_t* g_v, int64_t ld_v, const float* a_q,
    const float* a_v, const float* b_q, const float* b_v, float scaling, uint16_t* gs_q,
    uint16_t* gs_v, uint16_t* dt, uint16_t* dy, int64_t M, int32_t H, int32_t NQ, int32_t NV,
    int32_t r, void* stream) {
  const int rc = check_dims(M, H, NQ, NV, r);
  if (rc != kOk) return rc;
  if (ld_q < NQ || ld_v < NV || ld_q % 8 || ld_v % 8) return kInvalid;
  if (M == 0) return kOk;
  if (!g_q || !g_v || !a_q || !a_v || !b_q || !b_v || !gs_q || !gs_v || !dt || !dy)
    return kInvalid;
  for (const void* p : {static_cast<const void*>(g_q), static_cast<const void*>(g_v),
                        static_cast<const void*>(a_q), static_cast<const void*>(a_v),
                        static_cast<const void*>(gs_q), static_cast<const void*>(gs_v),
                        static_cast<const void*>(dy)})
    if (misaligned(p)) return kInvalid;
  const unsigned grid = static_cast<unsigned>((M + kRows - 1) / kRows);
  return launch_kernel(lora_bwd_rows_kernel, dim3(grid), dim3(kThreads),
                       static_cast<hipStream_t>(stream), g_q, ld_q, g_v, ld_v, a_q, a_v, b_q, b_v,
                       scaling, gs_q, gs_v, dt, dy, static_cast<int>(M), H, NQ, NV);
}
