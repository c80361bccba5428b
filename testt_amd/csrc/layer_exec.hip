// One decoder layer's forward and backward issued from C: the layer's kernels and hipBLASLt
// GEMMs in order, each through its own entry point with the arguments testt_amd/layer.py
// passes it, so that the values are those of the per-operation path bit for bit.  What this
// removes is the host time between the launches: issued from Python one operation at a time
// (argument checks, allocations, the autograd engine's nodes, a ctypes call each), the layer's
// ~25 launches took ~490 us of host time on the MI355X box, more than the ragged batch's GPU
// time; here they are ~25 C calls.  With the weights left in NF4 (few tokens), the products
// are the fused NF4-dequant GEMMs of gemm_nf4.hip instead.
//
// Reference: the layer the reference's solution/model.py:209-279 runs (input norm, q|k|v + LoRA,
// RoPE, attention, o, post norm, MLP) and its autograd backward.
#include "soupk_common.hpp"
#include "../../include/soupk.h"

namespace soupk {
namespace {

// y += x elementwise in fp16 (each sum in fp32, rounded once), n a multiple of 8
__global__ __launch_bounds__(256) void add_f16_kernel(u32x4* __restrict__ y,
                                                      const u32x4* __restrict__ x, int64_t n8) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n8) return;
  const u32x4 a = y[i], b = x[i];
  u32x4 out;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    out[k] = pack_h2(lo_h(a[k]) + lo_h(b[k]), hi_h(a[k]) + hi_h(b[k]));
  y[i] = out;
}

}  // namespace
}  // namespace soupk

namespace {

using soupk::u32x4;

#define SOUPK_TRY(call)        \
  do {                         \
    const int rc_ = (call);    \
    if (rc_ != 0) return rc_;  \
  } while (0)

int check_dims(const SoupkLayerDims* d) {
  if (!d) return soupk::kInvalid;
  if (d->M < 0 || d->H <= 0 || d->NH <= 0 || d->NKV <= 0 || d->D != 128 || d->I <= 0 ||
      d->r != 16 || d->batch < 0 || d->seq < 1 || d->p_down < 1 || d->p_gu < 1)
    return soupk::kInvalid;
  if (d->I % d->p_down || (2 * d->I) % d->p_gu) return soupk::kInvalid;
  if (!d->norm1 || !d->norm2 || !d->staged || !d->cos || !d->sin || !d->pos || !d->cu ||
      (d->gemm_ws_bytes > 0 && !d->gemm_ws))
    return soupk::kInvalid;
  if (d->nf4) {
    // NF4 weights: the fused GEMMs take no hipBLASLt splits; each group 1-4 parts, each split
    // count positive (the entry points check the rest: part rows, tables, partials' size)
    const SoupkLayerNf4* n = d->nf4;
    if (d->p_down != 1 || d->p_gu != 1) return soupk::kInvalid;
    for (const SoupkNf4Group* g : {&n->qkv, &n->o, &n->gu, &n->down})
      if (g->n_parts < 1 || g->n_parts > 4) return soupk::kInvalid;
    for (int i = 0; i < 4; ++i)
      if (n->split_fwd[i] < 1 || n->split_bwd[i] < 1) return soupk::kInvalid;
    return soupk::kOk;
  }
  if (!d->w_qkv || !d->w_o || !d->w_gu || !d->w_d) return soupk::kInvalid;
  return soupk::kOk;
}

// y [M, N] = x [M, K] W^T (+ bias) for an NF4 group W [N, K]: soupk_gemm_tn_nf4, or its
// contraction-split form with `splits` > 1
int nf4_fwd(const SoupkLayerNf4* n, const SoupkNf4Group& g, int splits, const uint16_t* x,
            int64_t ldx, const uint16_t* bias, uint16_t* y, int64_t M, int32_t N, int32_t K,
            void* stream) {
  if (splits > 1)
    return soupk_gemm_tn_nf4_split(x, ldx, g.n_parts, g.packed, g.absmax, g.code2, g.absmax2,
                                   g.offset, g.nf4, g.rows, 64, 256, bias, y, M, N, K, splits,
                                   n->partials, n->partials_floats, stream);
  return soupk_gemm_tn_nf4(x, ldx, g.n_parts, g.packed, g.absmax, g.code2, g.absmax2, g.offset,
                           g.nf4, g.rows, 64, 256, bias, y, M, N, K, stream);
}

// dx [M, N] = dy [M, K] W for an NF4 group W [K, N] (N: W's columns, K: its rows)
int nf4_bwd(const SoupkLayerNf4* n, const SoupkNf4Group& g, int splits, const uint16_t* dy,
            int64_t lddy, uint16_t* dx, int64_t M, int32_t N, int32_t K, void* stream) {
  if (splits > 1)
    return soupk_gemm_nn_nf4_split(dy, lddy, g.n_parts, g.packed, g.absmax, g.code2,
                                   g.absmax2, g.offset, g.nf4, g.rows, 64, 256, dx, M, N, K,
                                   splits, n->partials, n->partials_floats, stream);
  return soupk_gemm_nn_nf4(dy, lddy, g.n_parts, g.packed, g.absmax, g.code2, g.absmax2,
                           g.offset, g.nf4, g.rows, 64, 256, dx, M, N, K, stream);
}

int add_f16(uint16_t* y, const uint16_t* x, int64_t n, void* stream) {
  if (n % 8) return soupk::kInvalid;
  const int64_t n8 = n / 8;
  if (n8 == 0) return soupk::kOk;
  return soupk::launch_kernel(soupk::add_f16_kernel, dim3(static_cast<unsigned>((n8 + 255) / 256)),
                              dim3(256), static_cast<hipStream_t>(stream),
                              reinterpret_cast<u32x4*>(y), reinterpret_cast<const u32x4*>(x),
                              n8);
}

}  // namespace

extern "C" __attribute__((visibility("default"))) int soupk_layer_fwd(
    const SoupkLayerDims* dm, const SoupkLayerFwd* a, void* stream) {
  SOUPK_TRY(check_dims(dm));
  if (!a) return soupk::kInvalid;
  const int64_t M = dm->M;
  if (M == 0) return soupk::kOk;
  const int32_t H = dm->H, NQ = dm->NH * dm->D, NV = dm->NKV * dm->D, I = dm->I;
  const int64_t W = static_cast<int64_t>(NQ) + 2 * NV;
  void* const ws = dm->gemm_ws;
  const int64_t wsb = dm->gemm_ws_bytes;
  // input norm: s1 = s_in + delta, y = norm(s1) (without delta: y = norm(s_in))
  const float* s1 = a->delta ? a->s1 : a->s_in;
  SOUPK_TRY(soupk_rmsnorm_fwd(a->s_in, a->delta, dm->norm1, a->delta ? a->s1 : nullptr, a->y,
                              nullptr, nullptr, nullptr, a->rstd1, M, 0, H, dm->eps, stream));
  const SoupkLayerNf4* n4 = dm->nf4;
  // qkv = y @ W_qkv^T + b
  if (n4)
    SOUPK_TRY(nf4_fwd(n4, n4->qkv, n4->split_fwd[0], a->y, H, dm->qkv_bias, a->qkv, M, W, H,
                      stream));
  else
    SOUPK_TRY(soupk_gemm_lt(1, 0, W, M, H, dm->w_qkv, H, 0, a->y, H, 0, a->qkv, W, 0, 0, 1, 0,
                            dm->qkv_bias, a->algo_qkv, ws, wsb, stream));
  // t = y A^T, and the rotated q|k|v rows with the LoRA deltas added
  SOUPK_TRY(soupk_lora_rope_fwd(a->y, dm->staged, dm->scaling, a->qkv, dm->cos, dm->sin, dm->pos,
                                a->t, a->qkv_r, M, H, dm->NH, dm->NKV, dm->D, dm->r, dm->batch,
                                dm->seq, stream));
  SOUPK_TRY(soupk_attention_varlen_fwd(a->qkv_r, dm->cu, dm->batch, a->attn, a->lse, M, dm->NH,
                                       dm->NKV, dm->D, dm->scale, stream));
  // o = attn @ W_o^T; s2 = s1 + o, y2 = norm(s2)
  if (n4)
    SOUPK_TRY(nf4_fwd(n4, n4->o, n4->split_fwd[1], a->attn, NQ, nullptr, a->o, M, H, NQ,
                      stream));
  else
    SOUPK_TRY(soupk_gemm_lt(1, 0, H, M, NQ, dm->w_o, NQ, 0, a->attn, NQ, 0, a->o, H, 0, 0, 1,
                            0, nullptr, a->algo_o, ws, wsb, stream));
  SOUPK_TRY(soupk_rmsnorm_fwd(s1, a->o, dm->norm2, a->s2, a->y2, nullptr, nullptr, nullptr,
                              a->rstd2, M, 0, H, dm->eps, stream));
  // MLP: gu = y2 @ W_gu^T, act = silu(gate) * up, d = act @ W_d^T
  if (n4) {
    SOUPK_TRY(nf4_fwd(n4, n4->gu, n4->split_fwd[2], a->y2, H, nullptr, a->gu, M, 2 * I, H,
                      stream));
    SOUPK_TRY(soupk_swiglu_fwd(a->gu, a->act, M, I, stream));
    return nf4_fwd(n4, n4->down, n4->split_fwd[3], a->act, I, nullptr, a->d, M, H, I, stream);
  }
  SOUPK_TRY(soupk_gemm_lt(1, 0, 2 * static_cast<int64_t>(I), M, H, dm->w_gu, H, 0, a->y2, H, 0,
                          a->gu, 2 * static_cast<int64_t>(I), 0, 0, 1, 0, nullptr, a->algo_gu,
                          ws, wsb, stream));
  SOUPK_TRY(soupk_swiglu_fwd(a->gu, a->act, M, I, stream));
  if (dm->p_down > 1) {
    const int64_t c = I / dm->p_down;
    SOUPK_TRY(soupk_gemm_lt(1, 0, H, M, c, dm->w_d, I, c, a->act, I, c, a->down_part, H,
                            M * H, 1, dm->p_down, 0, nullptr, -1, ws, wsb, stream));
    return soupk_sum_partials(a->down_part, dm->p_down, M * H, M * H, a->d, stream);
  }
  return soupk_gemm_lt(1, 0, H, M, I, dm->w_d, I, 0, a->act, I, 0, a->d, H, 0, 0, 1, 0, nullptr,
                       a->algo_down, ws, wsb, stream);
}

extern "C" __attribute__((visibility("default"))) int soupk_layer_bwd(
    const SoupkLayerDims* dm, const SoupkLayerBwd* a, void* stream) {
  SOUPK_TRY(check_dims(dm));
  if (!a) return soupk::kInvalid;
  const int64_t M = dm->M;
  if (M == 0) return soupk::kOk;
  const int32_t H = dm->H, NQ = dm->NH * dm->D, NV = dm->NKV * dm->D, I = dm->I;
  const int64_t W = static_cast<int64_t>(NQ) + 2 * NV;
  const int64_t I2 = 2 * static_cast<int64_t>(I);
  void* const ws = dm->gemm_ws;
  const int64_t wsb = dm->gemm_ws_bytes;
  const SoupkLayerNf4* n4 = dm->nf4;
  // MLP: dact = g_d @ W_d; gu <- [d gate | d up]; g_y2 = gu @ W_gu
  if (n4)
    SOUPK_TRY(nf4_bwd(n4, n4->down, n4->split_bwd[3], a->g_d, H, a->dact, M, I, H, stream));
  else
    SOUPK_TRY(soupk_gemm_lt(0, 0, I, M, H, dm->w_d, I, 0, a->g_d, H, 0, a->dact, I, 0, 0, 1, 0,
                            nullptr, a->algo_down_dx, ws, wsb, stream));
  SOUPK_TRY(soupk_swiglu_bwd_inplace(a->dact, a->gu, M, I, stream));
  if (n4) {
    SOUPK_TRY(nf4_bwd(n4, n4->gu, n4->split_bwd[2], a->gu, I2, a->g_y2, M, H,
                      static_cast<int32_t>(I2), stream));
  } else if (dm->p_gu > 1) {
    const int64_t c = I2 / dm->p_gu;
    SOUPK_TRY(soupk_gemm_lt(0, 0, H, M, c, dm->w_gu, H, c * H, a->gu, I2, c, a->gu_part, H,
                            M * H, 1, dm->p_gu, 0, nullptr, -1, ws, wsb, stream));
    SOUPK_TRY(soupk_sum_partials(a->gu_part, dm->p_gu, M * H, M * H, a->g_y2, stream));
  } else {
    SOUPK_TRY(soupk_gemm_lt(0, 0, H, M, I2, dm->w_gu, H, 0, a->gu, I2, 0, a->g_y2, H, 0, 0, 1,
                            0, nullptr, a->algo_gu_dx, ws, wsb, stream));
  }
  // post-attention norm: g_s1 (residual), g_o
  SOUPK_TRY(soupk_rmsnorm_bwd(a->s2, a->rstd2, dm->norm2, a->g_y2, nullptr, nullptr, a->g_s,
                              a->g_s1, a->g_o, M, 0, H, stream));
  // o projection: g_a = g_o @ W_o
  if (n4)
    SOUPK_TRY(nf4_bwd(n4, n4->o, n4->split_bwd[1], a->g_o, H, a->g_a, M, NQ, H, stream));
  else
    SOUPK_TRY(soupk_gemm_lt(0, 0, NQ, M, H, dm->w_o, NQ, 0, a->g_o, H, 0, a->g_a, NQ, 0, 0, 1,
                            0, nullptr, a->algo_o_dx, ws, wsb, stream));
  // attention with RoPE's backward: dqkv, the gradient of the q|k|v GEMM output
  SOUPK_TRY(soupk_attention_varlen_bwd(a->qkv_r, dm->cu, dm->batch, a->attn, a->g_a, a->lse,
                                       dm->cos, dm->sin, dm->pos,
                                       static_cast<int64_t>(dm->batch) * dm->seq, dm->seq,
                                       a->attn_ws, a->dqkv, M, dm->NH, dm->NKV, dm->D, dm->scale,
                                       stream));
  // LoRA: its q and v gradients are dqkv's q and v columns
  const uint16_t* g_q = a->dqkv;
  const uint16_t* g_v = a->dqkv + NQ + NV;
  SOUPK_TRY(soupk_lora_bwd_rows(g_q, W, g_v, W, dm->staged, dm->scaling, a->dt, a->dy, M, H, NQ,
                                NV, dm->r, stream));
  SOUPK_TRY(soupk_lora_bwd_params(a->y, a->t, a->dt, g_q, W, g_v, W, dm->scaling, a->lora_ws,
                                  a->lora_ws_floats, a->d_aq, a->d_av, a->d_bq, a->d_bv, M, H, NQ,
                                  NV, dm->r, stream));
  // dy += dqkv @ W_qkv (NF4: the product into g_o's buffer, dead since the o input gradient,
  // then added)
  if (n4) {
    SOUPK_TRY(nf4_bwd(n4, n4->qkv, n4->split_bwd[0], a->dqkv, W, a->g_o, M, H,
                      static_cast<int32_t>(W), stream));
    SOUPK_TRY(add_f16(a->dy, a->g_o, M * H, stream));
  } else {
    SOUPK_TRY(soupk_gemm_lt(0, 0, H, M, W, dm->w_qkv, H, 0, a->dqkv, W, 0, a->dy, H, 0, 0, 1,
                            1, nullptr, a->algo_qkv_dx, ws, wsb, stream));
  }
  // input norm
  if (a->has_delta)
    return soupk_rmsnorm_bwd(a->s1, a->rstd1, dm->norm1, a->dy, nullptr, nullptr, a->g_s1,
                             a->g_s_in, a->g_delta, M, 0, H, stream);
  return soupk_rmsnorm_bwd(a->s_in, a->rstd1, dm->norm1, a->dy, nullptr, nullptr, nullptr,
                           a->g_s_in, nullptr, M, 0, H, stream);
}
