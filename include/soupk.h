/*
 * soupk.h - C ABI of libsoupk.so, the gfx950 (MI355X / CDNA4) kernels behind the QLoRA
 * fused-kernel set of SalReII/testt `solution/`.
 *
 * Every entry point:
 *   - takes plain device pointers, element counts and a HIP stream (`void*`, a hipStream_t;
 *     NULL is the legacy default stream), enqueues its kernels asynchronously and returns;
 *   - never allocates, never synchronises, and shares no mutable state between threads
 *     (re-entrant: PyTorch runs backward on its own worker thread); the only state is the
 *     per-thread benchmark hook of soupk_time_next_launch;
 *   - returns 0 on success, hipErrorInvalidValue (1) for arguments it rejects before
 *     launching, or the hipError_t of the launch;
 *   - bounds-checks every index it reads from device memory (positions, pad rows, labels):
 *     an out-of-range index is skipped, never dereferenced.
 * fp16 buffers are passed as uint16_t (IEEE binary16 bit patterns).
 * Nullable pointers replace the reference's dummy-tensor + has_* flag convention
 * (solution/rmsnorm.py:86-91,104-110, solution/rope.py:146-147,165-169).
 */
#ifndef SOUPK_H
#define SOUPK_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ABI version of this header; soupk_abi_version() returns the library's.  4 adds
   soupk_lora_rope_fwd, soupk_gemm_nn_nf4, soupk_gemm_tn_nf4_split, soupk_gemm_nn_nf4_split,
   soupk_gemm_lt, soupk_gemm_lt_index, soupk_layer_fwd, soupk_layer_bwd (with the layer's
   products on NF4 weights: SoupkLayerNf4) and soupk_init_device to version 3's entry
   points. */
#define SOUPK_ABI_VERSION 4

/* Status of soupk_lora_bwd_params_noalloc for a problem beyond its static scratch (no launch). */
#define SOUPK_STATUS_SCRATCH_LIMIT 20001

int soupk_abi_version(void);

/* Human-readable text of a status code returned by any soupk_* call. */
const char* soupk_status_string(int status);

/*
 * Benchmark instrumentation (no counterpart in the reference, which times its Triton kernels
 * with CUDA events around each launch, harness/_train.py:60-83): the next kernel launched by
 * the calling thread through any soupk_* entry point records `start_event` when its dispatch
 * begins and `stop_event` when it ends (hipExtLaunchKernelGGL), so the pair measures exactly
 * that kernel.  Events (hipEvent_t, nullable) are created by the caller; the setting is per
 * thread and is cleared by that launch.
 */
int soupk_time_next_launch(void* start_event, void* stop_event);

/*
 * Benchmark reference (no counterpart in the reference): a plain device-to-device copy of
 * `bytes` (a positive multiple of 16; both pointers 16-byte aligned) with 16-byte non-temporal
 * loads and stores.  bench.py times it at each kernel's byte count, so every kernel is reported
 * beside what a bare copy of the same size reaches on the same GPU.
 */
int soupk_bench_copy(const void* src, void* dst, int64_t bytes, void* stream);

/*
 * Benchmark reference (no counterpart in the reference): `workgroups` workgroups of 256
 * threads that do nothing.  bench.py times it like the kernels (the fixed cost of a launch:
 * dispatch, wave launch and completion) beside a 4 KiB soupk_bench_copy.
 */
int soupk_bench_empty(int32_t workgroups, void* stream);

/*
 * Benchmark utility (no counterpart in the reference): one wave that keeps `stream` busy for
 * `microseconds` (0 to 2e6) of the device's constant-rate wall clock, then ends.  bench.py
 * queues its timed launches behind it, so they run back to back however long the host takes
 * to enqueue them.
 */
int soupk_bench_hold(double microseconds, void* stream);

/*
 * NF4 double-quant unpack (replaces the launch of nf4_unpack_kernel, solution/nf4.py:27-45,
 * launched from unpack_into, solution/nf4.py:72-89).
 *   absmax[b] = fp32(fp32(code2[absmax_u8[b]] * absmax2[b / qblock2]) + offset[0])
 *   out[2i]   = fp16_rn(nf4[packed[i] >> 4] * absmax[i / (qblock/2)])
 *   out[2i+1] = fp16_rn(nf4[packed[i] & 15] * absmax[i / (qblock/2)])
 * Every product and sum is rounded separately (no fused multiply-add), as bitsandbytes does.
 * packed: n_bytes; absmax_u8: ceil(n_bytes / (qblock/2)); absmax2: ceil(#absmax / qblock2);
 * code2: 256; nf4: 16; offset: 1 fp32; out: 2*n_bytes fp16.  qblock even, qblock2 >= 1.
 */
int soupk_nf4_unpack(const uint8_t* packed, const uint8_t* absmax_u8, const float* code2,
                     const float* absmax2, const float* offset, const float* nf4,
                     uint16_t* out_f16, int64_t n_bytes, int32_t qblock, int32_t qblock2,
                     void* stream);

/*
 * soupk_nf4_unpack over up to 8 weights in one launch (the reference launches its unpack
 * kernel once per weight, solution/nf4.py:72-89 called per projection from
 * solution/nf4.py:125 and solution/mlp.py:105-108; here the projections of one decoder
 * layer, or the q|k|v and gate|up stacks, share a launch).  Part i is the soupk_nf4_unpack
 * call (packed[i], absmax_u8[i], code2[i], absmax2[i], offset[i], nf4[i], out_f16[i],
 * n_bytes[i]) with the common qblock, qblock2; results are bit-identical to those calls.
 * Parts of zero bytes are skipped; a part the tiled kernel does not take (n_bytes % 4,
 * alignment, qblock not a power of two) gets its own soupk_nf4_unpack launches.
 */
int soupk_nf4_unpack_multi(int32_t n_parts, const uint8_t* const* packed,
                           const uint8_t* const* absmax_u8, const float* const* code2,
                           const float* const* absmax2, const float* const* offset,
                           const float* const* nf4, uint16_t* const* out_f16,
                           const int64_t* n_bytes, int32_t qblock, int32_t qblock2,
                           void* stream);

/*
 * soupk_nf4_unpack_multi and soupk_lora_stage in one launch: the NF4 parts as there, and the
 * rank-16 LoRA parameters a_q, a_v, b_q, b_v of the same layer cast to fp16 into `staged` by
 * extra workgroups (the same values and layout as soupk_lora_stage).  A decoder layer then
 * prepares all of its weights, frozen and trainable, with one launch before its forward.  The
 * LoRA arguments follow soupk_lora_stage's rules and are checked before anything is launched.
 */
int soupk_nf4_unpack_multi_lora(int32_t n_parts, const uint8_t* const* packed,
                                const uint8_t* const* absmax_u8, const float* const* code2,
                                const float* const* absmax2, const float* const* offset,
                                const float* const* nf4, uint16_t* const* out_f16,
                                const int64_t* n_bytes, int32_t qblock, int32_t qblock2,
                                const float* a_q, const float* a_v, const float* b_q,
                                const float* b_v, uint16_t* staged, int64_t staged_elems,
                                int32_t H, int32_t NQ, int32_t NV, int32_t r, void* stream);

/*
 * Inverse of a scatter index (no counterpart kernel in the reference: it lets the pad-layout
 * writers of rmsnorm_fwd and rope_pack_fwd zero the unused rows in the same launch instead of
 * a separate torch.zeros, solution/rmsnorm.py:82, solution/rope.py:141-143).
 *   inv[p] = i if idx[i] == p, else -1, for p in [0, n_slots).  idx entries must be distinct;
 *   entries outside [0, n_slots) are ignored.
 */
int soupk_index_inverse(const int64_t* idx, int64_t n, int32_t* inv, int64_t n_slots,
                        void* stream);

/*
 * Split-K reduction (no counterpart kernel in the reference: the reference computes the MLP's
 * gate|up input gradient as one fp16 GEMM, solution/mlp.py:105-113; here that GEMM runs as
 * n_parts batched GEMMs over slices of K with fp32 outputs, and this sums them).
 *   out_f16[i] = fp16_rn(((parts[i] + parts[stride + i]) + parts[2 stride + i]) + ...)
 * for i < n, partials added in index order.  1 <= n_parts <= 16, part_stride >= n.
 */
int soupk_sum_partials(const float* parts, int32_t n_parts, int64_t part_stride, int64_t n,
                       uint16_t* out_f16, void* stream);

/*
 * Residual add + Qwen2RMSNorm forward (replaces rmsnorm_fwd_kernel, solution/rmsnorm.py:24-43,
 * launched from _launch_fwd, solution/rmsnorm.py:76-92).  Per row r of [rows, H]:
 *   s = x + fp32(delta)            (stored to s_out when delta != NULL)
 *   rstd = 1 / sqrt(sum(s*s) / H + eps)
 *   y = fp16_rn((s * rstd) * w);   ypad[pad_idx[r]] = (s * rstd) * w  (fp32)
 * delta, s_out: both NULL or both set.  ypad/pad_idx: both NULL or both set; ypad has
 * pad_rows rows.  pad_inv (nullable, from soupk_index_inverse over pad_idx): rows p of ypad
 * with pad_inv[p] < 0 are written with zeros in the same launch; with pad_inv NULL the caller
 * owns the rows that no pad_idx entry names.
 */
int soupk_rmsnorm_fwd(const float* x, const uint16_t* delta, const float* w, float* s_out,
                      uint16_t* y, float* ypad, const int64_t* pad_idx, const int32_t* pad_inv,
                      float* rstd, int64_t rows, int64_t pad_rows, int32_t H, float eps,
                      void* stream);

/*
 * Residual add + RMSNorm backward (replaces rmsnorm_bwd_kernel, solution/rmsnorm.py:46-69,
 * launched from _launch_bwd, solution/rmsnorm.py:95-112).  Per row r:
 *   g = (fp32(dy) + dypad[pad_idx[r]]) * w          (absent terms are 0)
 *   n = s * rstd;  proj = sum(g * n) / H
 *   dx = (g - n * proj) * rstd + ds;  ddelta = fp16_rn(dx)
 * dy, dypad (with pad_idx, pad_rows rows), ds and ddelta are nullable.
 */
int soupk_rmsnorm_bwd(const float* s, const float* rstd, const float* w, const uint16_t* dy,
                      const float* dypad, const int64_t* pad_idx, const float* ds, float* dx,
                      uint16_t* ddelta, int64_t rows, int64_t pad_rows, int32_t H, void* stream);

/* LoRA-delta element types for soupk_rope_pack_fwd. */
#define SOUPK_DTYPE_F16 0
#define SOUPK_DTYPE_F32 1

/*
 * LoRA add + RoPE + QKV pack forward (replaces rope_pack_fwd_kernel, solution/rope.py:24-75,
 * launched from RopePack.forward, solution/rope.py:137-151).
 * qkv: [rows, (NH + 2*NKV) * D] fp16 (q heads, then k heads, then v heads);
 * lora_q: [rows, NH*D], lora_v: [rows, NKV*D] (nullable, element type lora_dtype);
 * cos, sin: [T, D] fp32; pos: [rows] int64 padded positions b*T + t.
 * Writes q [B, NH, T, D], k, v [B, NKV, T, D] fp16 at (b, h, t):
 *   q = rot(qkv_q + lora_q), k = rot(qkv_k), v = qkv_v + lora_v, with
 *   rot(x1, x2) = (x1*c1 - x2*s1, x2*c2 + x1*s2) in fp32 (x1, x2 the two halves of a head).
 * pos_inv (nullable, soupk_index_inverse over pos with B*T slots): positions with
 * pos_inv[p] < 0 are written with zeros in the same launch.  D even.
 */
int soupk_rope_pack_fwd(const uint16_t* qkv, const void* lora_q, const void* lora_v,
                        int32_t lora_dtype, const float* cos, const float* sin,
                        const int64_t* pos, const int32_t* pos_inv, uint16_t* q, uint16_t* k,
                        uint16_t* v, int64_t rows, int32_t B, int32_t T, int32_t NH,
                        int32_t NKV, int32_t D, void* stream);

/*
 * RoPE pack backward (replaces rope_pack_bwd_kernel, solution/rope.py:78-128, launched from
 * RopePack.backward, solution/rope.py:153-176).  Gathers dq/dk/dv (each nullable = zero) at
 * (b, h, t) of every token and writes dqkv [rows, (NH + 2*NKV) * D] fp16:
 *   q, k: (g1*c1 + g2*s2, g2*c2 - g1*s1);  v: passthrough.
 */
int soupk_rope_pack_bwd(const uint16_t* dq, const uint16_t* dk, const uint16_t* dv,
                        const float* cos, const float* sin, const int64_t* pos, uint16_t* dqkv,
                        int64_t rows, int32_t B, int32_t T, int32_t NH, int32_t NKV, int32_t D,
                        void* stream);

/*
 * Gated SiLU forward (replaces gated_silu_fwd_kernel, solution/mlp.py:31-40, launched from
 * gated_silu, solution/mlp.py:61-68).  gu: [rows, 2I] fp16 = [gate | up];
 *   act[r, c] = fp16_rn(gate / (1 + exp(-gate)) * up), in fp32.
 */
int soupk_swiglu_fwd(const uint16_t* gu, uint16_t* act, int64_t rows, int64_t I, void* stream);

/*
 * Gated SiLU backward, in place (replaces gated_silu_bwd_inplace_kernel, solution/mlp.py:43-58,
 * launched from gated_silu_backward_, solution/mlp.py:71-77).  sig = 1/(1+exp(-gate)):
 *   gu[:, :I] <- fp16_rn(dact * up * sig * (1 + gate * (1 - sig)))
 *   gu[:, I:] <- fp16_rn(dact * (gate * sig))
 */
int soupk_swiglu_bwd_inplace(const uint16_t* dact, uint16_t* gu, int64_t rows, int64_t I,
                             void* stream);

/*
 * Vocab-head statistics + in-place gradient (replaces head_stats_grad_kernel,
 * solution/head.py:34-76, launched from FusedHeadLoss.forward, solution/head.py:108-110).
 * logits: [rows, V] fp16, overwritten for labelled rows.  Per row, over z = fp32(logits):
 *   lse = max + log(sum exp(z - max));  entropy = lse - sum(exp(z - max) * z) / sum(exp(z - max))
 *   loss = lse - z[target] (0 when target == -100);  correct = argmax(z) == target (first max)
 *   labelled rows: logits <- fp16_rn((exp(z - lse) - onehot(target)) * grad_scale)
 * lse_out is nullable (an extra output the reference kernel does not store).  A target outside
 * [0, V) other than -100 gives loss = NaN, correct = 0 and no onehot term.
 */
int soupk_head_stats_grad(uint16_t* logits, const int64_t* target, float* entropy, float* loss,
                          int32_t* correct, float* lse_out, float grad_scale, int64_t rows,
                          int64_t V, void* stream);

/*
 * soupk_head_stats_grad with the gradient written away from the logits (the kernel of
 * solution/head.py:34-76 as FusedHeadLoss.forward, solution/head.py:87-137, uses it; no
 * counterpart entry in the reference).  Statistics as soupk_head_stats_grad, at row r of
 * entropy / loss / correct / lse_out.  logits are only read.  The gradient of a labelled row r
 * goes to row grad_row[r] of grad_out ([grad_rows, V] fp16), so the labelled rows of a chunk
 * land packed in their own buffer for the dh GEMM; a row whose grad_row entry lies outside
 * [0, grad_rows) gets none.  grad_row and grad_out are both NULL (statistics only, no gradient
 * written) or both set; then (2V) % 16 == 0 and grad_out has logits' address modulo 16.
 */
int soupk_head_stats_grad_rows(const uint16_t* logits, const int64_t* target,
                               const int32_t* grad_row, uint16_t* grad_out, int64_t grad_rows,
                               float* entropy, float* loss, int32_t* correct, float* lse_out,
                               float grad_scale, int64_t rows, int64_t V, void* stream);

/*
 * Causal grouped-query attention, forward (widening beyond the reference's kernel set: it
 * replaces torch's scaled_dot_product_attention in the layer loop of fused_forward,
 * solution/model.py:246-247).  q [B, NH, T, D], k and v [B, NKV, T, D] fp16 (NH a multiple of
 * NKV; D = 128); query i of row b attends to key j iff j <= i and key_valid[b*T + j] != 0
 * (every key when key_valid is NULL).  Writes out[(b*T + t)*NH*D + h*D + d] fp16 (token-major,
 * the layout the o-projection reads) and lse[(b*NH + h)*T + t] (natural log-sum-exp of the
 * scaled scores; +inf for a query with no visible key, whose output is 0).  All fp16 pointers
 * 16-byte aligned.
 */
int soupk_attention_fwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                        const uint8_t* key_valid, uint16_t* out, float* lse, int32_t B,
                        int32_t T, int32_t NH, int32_t NKV, int32_t D, float scale,
                        void* stream);

/*
 * Causal grouped-query attention, backward (the gradient half of the same replacement).  Inputs
 * as soupk_attention_fwd, plus its out and lse and dout (the output gradient, token-major like
 * out).  Writes dq [B, NH, T, D] and dk, dv [B, NKV, T, D] fp16 (dk, dv summed over each
 * key/value head's NH/NKV query heads in a fixed order: deterministic).  workspace: fp32 device
 * memory of  round_up(B*NH*T, 4) + 2*B*NH*T*D  floats, 16-byte aligned (D and the partial dK,
 * dV of every query head).
 */
int soupk_attention_bwd(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                        const uint8_t* key_valid, const uint16_t* out, const uint16_t* dout,
                        const float* lse, float* workspace, uint16_t* dq, uint16_t* dk,
                        uint16_t* dv, int32_t B, int32_t T, int32_t NH, int32_t NKV, int32_t D,
                        float scale, void* stream);

/*
 * The RoPE pack forward into the token-major layout (the varlen attention's input; the padded
 * layout of soupk_rope_pack_fwd, solution/rope.py:24-75, is what it replaces in the layer):
 * out [rows, (NH + 2*NKV) * 128] fp16 in qkv's layout holds q = rot(qkv_q + lora_q),
 * k = rot(qkv_k), v = qkv_v + lora_v, bit-identical to what soupk_rope_pack_fwd writes at the
 * token's padded position; no scatter, no zero rows.  A token whose pos lies outside
 * [0, B*T) gets a row of zeros.  D must be 128; T >= 1; pointers 16-byte aligned.
 */
int soupk_rope_pack_tokens(const uint16_t* qkv, const void* lora_q, const void* lora_v,
                           int32_t lora_dtype, const float* cos, const float* sin,
                           const int64_t* pos, uint16_t* out, int64_t rows, int32_t B, int32_t T,
                           int32_t NH, int32_t NKV, int32_t D, void* stream);

/*
 * Causal GQA attention over variable-length sequences of real tokens (the reference's stated
 * next step, "flash-attention with GQA and varlen without padding", README.md:187-189; it
 * replaces soupk_attention_fwd on the padded layout in the layer).  qkv: [M, (NH+2*NKV)*128]
 * fp16 token-major rows (soupk_rope_pack_tokens' output).  Sequence b is tokens
 * cu_seqlens[b] .. cu_seqlens[b+1]-1 (int32 [B+1], non-decreasing from 0 to M; a sequence
 * whose bounds leave [0, M] is skipped); query i of a sequence attends to its keys j <= i.
 * Writes out [M, NH*128] fp16 (token-major) and lse [NH, M] (natural log).  16-byte aligned
 * qkv and out; M * (NH + 2*NKV) * 128 < 2^31.
 */
int soupk_attention_varlen_fwd(const uint16_t* qkv, const int32_t* cu_seqlens, int32_t B,
                               uint16_t* out, float* lse, int64_t M, int32_t NH, int32_t NKV,
                               int32_t D, float scale, void* stream);

/*
 * Its backward, with RoPE's backward (solution/rope.py:78-128) fused in: writes dqkv
 * [M, (NH+2*NKV)*128] fp16, the gradient of the token-major q|k|v rows.  With cos, sin
 * ([T_rope, 128] fp32) and pos (int64 [M], padded positions; t = pos % T_rope) given, the q and
 * k gradients are rounded to fp16 and rotated back, (g1*c1 + g2*s2, g2*c2 - g1*s1), exactly as
 * soupk_attention_bwd followed by soupk_rope_pack_bwd would give them, so dqkv is the gradient
 * of the rows before rotation (of the q|k|v GEMM output); a token with pos outside
 * [0, pos_slots) gets zero q and k gradients.  cos, sin, pos all NULL: dqkv is the gradient of
 * qkv itself.  dK and dV are summed over each key/value head's query heads in a fixed order
 * (deterministic).  workspace: fp32, round_up(NH*M, 4) + 2*NH*M*128 floats, 16-byte aligned.
 */
int soupk_attention_varlen_bwd(const uint16_t* qkv, const int32_t* cu_seqlens, int32_t B,
                               const uint16_t* out, const uint16_t* dout, const float* lse,
                               const float* cos, const float* sin, const int64_t* pos,
                               int64_t pos_slots, int32_t T_rope, float* workspace,
                               uint16_t* dqkv, int64_t M, int32_t NH, int32_t NKV, int32_t D,
                               float scale, void* stream);

/*
 * LoRA branch of the q and v projections for rank 16 (peft's lora_B(lora_A(x)) * scaling under
 * fp16 autocast, solution/model.py:195-206 with dropout 0; widening: the reference runs it as
 * separate fp16 GEMMs, casts and a scaling).
 *
 * soupk_lora_stage casts the fp32 LoRA parameters a_q, a_v [16, H] and b_q [NQ, 16],
 * b_v [NV, 16] to fp16 (as .to(float16) rounds) into `staged`, once per forward, in the layouts
 * soupk_lora_fwd and soupk_lora_bwd_rows read: [a_q; a_v] [32, H], its transpose [H, 32],
 * [b_q; b_v] [NQ + NV, 16], b_q^T [16, NQ], b_v^T [16, NV], in that order:
 * staged_elems >= 128*H + 32*(NQ + NV) halves, 16-byte aligned.
 */
int soupk_lora_stage(const float* a_q, const float* a_v, const float* b_q, const float* b_v,
                     uint16_t* staged, int64_t staged_elems, int32_t H, int32_t NQ, int32_t NV,
                     int32_t r, void* stream);

/*
 * The forward: y [M, H] fp16, `staged` from soupk_lora_stage.  Writes
 * t = fp16(y [a_q; a_v]^T) [M, 32] fp16 (kept for the backward),
 * lq = fp16(fp16(t[:, :16] b_q^T) * scaling) [M, NQ], lv likewise from t[:, 16:] and b_v.
 * H, NQ, NV multiples of 128; r must be 16; pointers 16-byte aligned (t: 2-byte).
 */
int soupk_lora_fwd(const uint16_t* y, const uint16_t* staged, float scaling, uint16_t* t,
                   uint16_t* lq, uint16_t* lv, int64_t M, int32_t H, int32_t NQ, int32_t NV,
                   int32_t r, void* stream);

/*
 * The forward fused with the RoPE pack of the varlen attention (replaces soupk_lora_fwd followed
 * by soupk_rope_pack_tokens on the layer's path; the reference's rope_pack_fwd_kernel,
 * solution/rope.py:24-75, in the token-major layout of soupk_rope_pack_tokens).  qkv
 * [M, (NH + 2*NKV)*128] fp16 is the q|k|v GEMM output, cos/sin [>= T, 128] fp32, pos int64 [M]
 * (padded positions b*T + t).  Writes t as soupk_lora_fwd does and
 * out [M, (NH + 2*NKV)*128] fp16 = rotated(q + lq) | rotated(k) | v + lv, with lq, lv the deltas
 * soupk_lora_fwd would write (NQ = NH*128, NV = NKV*128) and the rotation of
 * soupk_rope_pack_tokens: the same bits as that pair of launches, without lq / lv in memory.  A
 * row whose position lies outside [0, B*T) gets zeros.  D must be 128, r 16, H a multiple of 128;
 * pointers 16-byte aligned (t, pos: element-aligned); M*(NH + 2*NKV)*256 < 2^32 bytes.
 */
int soupk_lora_rope_fwd(const uint16_t* y, const uint16_t* staged, float scaling,
                        const uint16_t* qkv, const float* cos, const float* sin,
                        const int64_t* pos, uint16_t* t, uint16_t* out, int64_t M, int32_t H,
                        int32_t NH, int32_t NKV, int32_t D, int32_t r, int32_t B, int32_t T,
                        void* stream);

/*
 * Its backward, the row-local part: with g_q [M, NQ] (row stride ld_q) and g_v [M, NV] (ld_v)
 * the fp16 gradients of lq and lv, and the forward's `staged` parameters, writes
 * dt = fp16([gs_q b_q16 | gs_v b_v16]) [M, 32], gs_x = fp16(g_x * scaling) (formed in
 * registers, not stored), and dy = fp16(dt [a_q16; a_v16]) [M, H] (the LoRA part of the
 * gradient of y; the caller adds the frozen projection's part in place).  Same shape rules;
 * ld_q, ld_v multiples of 8.
 */
int soupk_lora_bwd_rows(const uint16_t* g_q, int64_t ld_q, const uint16_t* g_v, int64_t ld_v,
                        const uint16_t* staged, float scaling, uint16_t* dt, uint16_t* dy,
                        int64_t M, int32_t H, int32_t NQ, int32_t NV, int32_t r, void* stream);

/*
 * Its backward, the parameter gradients (reductions over the M rows), each the fp16 GEMM result
 * cast to fp32: d_aq = fp16(dt[:, :16]^T y), d_av = fp16(dt[:, 16:]^T y) [16, H];
 * d_bq = fp16(gs_q^T t[:, :16]) [NQ, 16], d_bv = fp16(gs_v^T t[:, 16:]) [NV, 16], with
 * gs_x = fp16(g_x * scaling) formed from g_q (row stride ld_q) and g_v (ld_v) as they are read.
 * workspace: fp32 device memory of ceil(M/128) * (32*H + 16*(NQ + NV)) floats (per-slice
 * partial sums, added in slice order: deterministic).  Same shape rules (H, NQ, NV multiples
 * of 128; ld_q, ld_v multiples of 8).
 */
int soupk_lora_bwd_params(const uint16_t* y, const uint16_t* t, const uint16_t* dt,
                          const uint16_t* g_q, int64_t ld_q, const uint16_t* g_v, int64_t ld_v,
                          float scaling, float* workspace, int64_t workspace_floats, float* d_aq,
                          float* d_av, float* d_bq, float* d_bv, int64_t M, int32_t H,
                          int32_t NQ, int32_t NV, int32_t r, void* stream);

/*
 * soupk_lora_bwd_params without the workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  Same arguments, results and rounding as
 * soupk_lora_bwd_params (the same kernels), but the per-slice partial sums live in a static
 * buffer of SOUPK_LORA_SCRATCH_FLOATS floats (16 MiB) that the library holds on each GPU it
 * runs on until the process ends; it calls no allocator.  A problem needing more than that,
 * ceil(M/128) * (32*H + 16*(NQ + NV)) > SOUPK_LORA_SCRATCH_FLOATS (M > 6784 rows at H = 1536,
 * NQ = 1536, NV = 256), returns SOUPK_STATUS_SCRATCH_LIMIT before any launch.  Every call on one
 * GPU shares that GPU's buffer: calls that overlap on one GPU (concurrent streams, threads)
 * race and must be serialised by the caller.  The buffer needs no clearing between calls (every
 * entry a call reads is written by that call first).
 */
#define SOUPK_LORA_SCRATCH_FLOATS (4 << 20)
/*
 * Per-device set-up of the library (no counterpart in the reference): looks up, with the
 * calling thread's current device, the device address of that device's no-alloc scratch
 * buffer and keeps it.  The Python binding calls it when it loads the library.  A caller that
 * captures soupk_lora_bwd_params_noalloc into a HIP graph calls it once per device before the
 * capture: under capture, that entry point does not make the lookup itself and returns
 * hipErrorStreamCaptureUnsupported if it has not been made.  Returns 0 or a hipError_t value.
 */
int soupk_init_device(void);
int soupk_lora_bwd_params_noalloc(const uint16_t* y, const uint16_t* t, const uint16_t* dt,
                                  const uint16_t* g_q, int64_t ld_q, const uint16_t* g_v,
                                  int64_t ld_v, float scaling, float* d_aq, float* d_av,
                                  float* d_bq, float* d_bv, int64_t M, int32_t H, int32_t NQ,
                                  int32_t NV, int32_t r, void* stream);

/*
 * y = x W^T (+ bias), fp16, on MFMA with 128 x 128 tiles (the GEMM core of soupk_gemm_tn_nf4;
 * widening: the reference's torch.matmul).  x [M, K] (row stride ldx, a multiple of 8), W
 * [N, K] row-major, bias nullable fp16 [N], y [M, N]; N a multiple of 128, K of 64.
 */
int soupk_gemm_tn(const uint16_t* x, int64_t ldx, const uint16_t* w, const uint16_t* bias,
                  uint16_t* y, int64_t M, int32_t N, int32_t K, void* stream);

/*
 * The fused NF4-dequant GEMM (the reference's stated next step, README.md:190-192, in place of
 * nf4_unpack + torch.matmul in FrozenNF4Linear, solution/nf4.py:108-127): y = x W^T (+ bias)
 * with W the row stack of n_parts (1..4) NF4 weights, part i given by host arrays of device
 * pointers packed[i], absmax_u8[i], code2[i], absmax2[i], offset[i], nf4[i] (the
 * soupk_nf4_unpack operands) and part_rows[i] (a multiple of 128; the sum is N).  qblock must
 * be 64 and qblock2 256.  The dequantised values are soupk_nf4_unpack's bit for bit.
 */
int soupk_gemm_tn_nf4(const uint16_t* x, int64_t ldx, int32_t n_parts,
                      const uint8_t* const* packed, const uint8_t* const* absmax_u8,
                      const float* const* code2, const float* const* absmax2,
                      const float* const* offset, const float* const* nf4,
                      const int32_t* part_rows, int32_t qblock, int32_t qblock2,
                      const uint16_t* bias, uint16_t* y, int64_t M, int32_t N, int32_t K,
                      void* stream);

/*
 * soupk_gemm_tn_nf4 with the contraction split (widening, for grids of few tiles: few rows of x
 * against a small W, or a long K): the K tiles are cut into `splits` (1..32, at most K/64)
 * consecutive ranges, each workgroup writes the fp32 product of its range into `workspace`
 * ([used splits, M, N] floats, used = ceil(K/64 / ceil(K/64 / splits)) <= splits), and a second
 * launch writes y = fp16(((p[0] + p[1]) + ...) + bias) in split order (deterministic; one
 * rounding, as the unsplit kernel, with another order of the fp32 sums).  workspace: 16-byte
 * aligned, at least used * M * N floats; y 16-byte aligned; bias (optional) 8-byte aligned.
 */
int soupk_gemm_tn_nf4_split(const uint16_t* x, int64_t ldx, int32_t n_parts,
                            const uint8_t* const* packed, const uint8_t* const* absmax_u8,
                            const float* const* code2, const float* const* absmax2,
                            const float* const* offset, const float* const* nf4,
                            const int32_t* part_rows, int32_t qblock, int32_t qblock2,
                            const uint16_t* bias, uint16_t* y, int64_t M, int32_t N, int32_t K,
                            int32_t splits, float* workspace, int64_t workspace_floats,
                            void* stream);

/*
 * Its input gradient (the backward of the same projection): dx = dy W, dy [M, K] fp16 (row
 * pitch lddy), W [K, N] the NF4 row stack (n_parts parts of part_rows[i] rows, K in all, each a
 * multiple of 128; N, W's columns, a multiple of 128; K a multiple of 64) dequantised as it is
 * staged (the same values as soupk_nf4_unpack), dx [M, N] fp16.  One fp16 rounding of fp32 MFMA
 * sums.  No counterpart kernel in the reference, which unpacks W again and calls cuBLAS
 * (solution/nf4.py:122-127); the fused form its README names as the next step
 * (README.md:190-192).
 */
int soupk_gemm_nn_nf4(const uint16_t* dy, int64_t lddy, int32_t n_parts,
                      const uint8_t* const* packed, const uint8_t* const* absmax_u8,
                      const float* const* code2, const float* const* absmax2,
                      const float* const* offset, const float* const* nf4,
                      const int32_t* part_rows, int32_t qblock, int32_t qblock2, uint16_t* dx,
                      int64_t M, int32_t N, int32_t K, void* stream);

/*
 * soupk_gemm_nn_nf4 with the contraction (W's rows) split, as soupk_gemm_tn_nf4_split: each
 * workgroup writes the fp32 product of its range of 64-row steps into `workspace`
 * ([used splits, M, N] floats), and a second launch writes dx = fp16((p[0] + p[1]) + ...) in
 * split order.  splits 1..32, at most K/64; workspace 16-byte aligned, at least used * M * N
 * floats (used = ceil(K/64 / ceil(K/64 / splits))).  No counterpart in the reference beyond its
 * stated next step (README.md:190-192); the widening for batches of few rows.
 */
int soupk_gemm_nn_nf4_split(const uint16_t* dy, int64_t lddy, int32_t n_parts,
                            const uint8_t* const* packed, const uint8_t* const* absmax_u8,
                            const float* const* code2, const float* const* absmax2,
                            const float* const* offset, const float* const* nf4,
                            const int32_t* part_rows, int32_t qblock, int32_t qblock2,
                            uint16_t* dx, int64_t M, int32_t N, int32_t K, int32_t splits,
                            float* workspace, int64_t workspace_floats, void* stream);

/*
 * D = op(A) op(B) (+ D with accumulate = 1) (+ bias[m] along D's columns), column-major as BLAS,
 * fp16 A and B, fp16 D or fp32 D (d_f32 = 1), fp32 accumulation, `batch` problems strided by
 * stride_a / stride_b / stride_d elements, on hipBLASLt: the library that runs the step's dense
 * GEMMs, called without its per-call setup.  A problem's descriptor, layouts and algorithm are
 * made on its first call and kept (per device); the algorithm is hipBLASLt solution
 * `algo_index` when it supports the problem within `workspace_bytes`, else the heuristic's
 * first choice (algo_index -1: always).  Replaces the per-call setup of torch.matmul, through
 * which the reference runs these GEMMs (solution/nf4.py:108-127, solution/mlp.py:80-113).
 * bias: fp16, one problem, fp16 D.  Returns hipErrorLaunchFailure when hipBLASLt fails.
 */
int soupk_gemm_lt(int32_t trans_a, int32_t trans_b, int64_t m, int64_t n, int64_t k,
                  const uint16_t* A, int64_t lda, int64_t stride_a, const uint16_t* B,
                  int64_t ldb, int64_t stride_b, void* D, int64_t ldd, int64_t stride_d,
                  int32_t d_f32, int32_t batch, int32_t accumulate, const uint16_t* bias,
                  int32_t algo_index, void* workspace, int64_t workspace_bytes, void* stream);

/* The hipBLASLt solution index a soupk_gemm_lt problem runs with, -1 before its first call
   (the same arguments, without the pointers and the stream; has_bias for the bias). */
int soupk_gemm_lt_index(int32_t trans_a, int32_t trans_b, int64_t m, int64_t n, int64_t k,
                        int64_t lda, int64_t stride_a, int64_t ldb, int64_t stride_b,
                        int64_t ldd, int64_t stride_d, int32_t d_f32, int32_t batch,
                        int32_t has_bias, int32_t accumulate, int32_t algo_index,
                        int64_t workspace_bytes);

/*
 * One Qwen2 decoder layer of the QLoRA step, forward and backward, each as one call that issues
 * the layer's kernels and hipBLASLt GEMMs in order on `stream` (widening: the reference's
 * layer, solution/model.py:209-279, runs them from Python one operation at a time).  The layer
 * is the fused path of testt_amd/layer.py: input RMSNorm (with the residual add unless delta is
 * NULL), q|k|v GEMM + bias, the rank-16 LoRA forward fused with RoPE, varlen causal GQA
 * attention, o GEMM, residual add + post-attention RMSNorm, gate|up GEMM, gated SiLU, down GEMM
 * (split over K into p_down slices when p_down > 1); the backward mirrors it (the gate|up input
 * gradient split into p_gu slices; the attention backward with RoPE's backward fused in; the
 * LoRA backward).  Every value is the one the same kernels give when called one by one: the
 * calls are the entry points above with the arguments testt_amd/layer.py passes them.  The
 * caller owns every buffer; the unpacked weights (row stacks q|k|v [W, H], o [H, NH*D],
 * gate|up [2I, H], down [H, I], W = (NH + 2 NKV) * D) and the staged LoRA parameters are the
 * layer's soupk_nf4_unpack_multi_lora output.  algo_*: hipBLASLt solution indices (-1: the
 * heuristic's) of the GEMMs as soupk_gemm_lt takes them.  Returns the first failing call's
 * status; nothing is launched after it.
 *
 * With dims->nf4 set, the weights stay in NF4 (w_* unused, may be NULL; p_down = p_gu = 1):
 * each product is the fused NF4-dequant GEMM, soupk_gemm_tn_nf4 forward and soupk_gemm_nn_nf4
 * for the input gradients, or their contraction-split forms where split_fwd / split_bwd > 1
 * (partials in nf4->partials); the q|k|v input gradient is formed in g_o's buffer and added to
 * the LoRA part of dy (fp16 + fp16 in fp32, rounded once more), as testt_amd/layer.py's
 * per-operation path does on NF4 weights.
 */
typedef struct SoupkNf4Group {                 /* one product's weight: 1-4 row parts */
  int32_t n_parts;
  int32_t rows[4];
  const uint8_t* packed[4];                    /* as soupk_gemm_tn_nf4 takes them */
  const uint8_t* absmax[4];
  const float* code2[4];
  const float* absmax2[4];
  const float* offset[4];
  const float* nf4[4];
} SoupkNf4Group;

typedef struct SoupkLayerNf4 {
  SoupkNf4Group qkv, o, gu, down;              /* [Wq;Wk;Wv], Wo, [Wgate;Wup], Wdown */
  int32_t split_fwd[4];                        /* contraction splits (1: none), same order */
  int32_t split_bwd[4];
  float* partials;                             /* fp32 scratch of the split products */
  int64_t partials_floats;
} SoupkLayerNf4;

typedef struct SoupkLayerDims {
  int64_t M;                                   /* tokens (rows) */
  int32_t H, NH, NKV, D, I, r, batch, seq;     /* D = 128, r = 16 */
  int32_t p_down, p_gu;                        /* K slices of the split products (1: none) */
  float eps, scaling, scale;
  const float* norm1;                          /* fp32 [H] RMSNorm weights */
  const float* norm2;
  const uint16_t* qkv_bias;                    /* fp16 [W] or NULL */
  const uint16_t* w_qkv;
  const uint16_t* w_o;
  const uint16_t* w_gu;
  const uint16_t* w_d;
  const uint16_t* staged;
  const float* cos;                            /* fp32 [>= seq, D] */
  const float* sin;
  const int64_t* pos;                          /* int64 [M]: padded positions b * seq + t */
  const int32_t* cu;                           /* int32 [batch + 1] */
  void* gemm_ws;                               /* hipBLASLt workspace */
  int64_t gemm_ws_bytes;
  const SoupkLayerNf4* nf4;                    /* NULL: w_* are the unpacked fp16 stacks */
} SoupkLayerDims;

typedef struct SoupkLayerFwd {
  const float* s_in;                           /* fp32 [M, H] residual stream */
  const uint16_t* delta;                       /* fp16 [M, H], or NULL (the first layer) */
  int32_t algo_qkv, algo_o, algo_gu, algo_down;
  /* saved for the backward */
  float* s1;                                   /* fp32 [M, H] (unused when delta is NULL) */
  uint16_t* y;                                 /* fp16 [M, H] */
  float* rstd1;                                /* fp32 [M] */
  uint16_t* t;                                 /* fp16 [M, 2r] */
  uint16_t* qkv_r;                             /* fp16 [M, W] */
  uint16_t* attn;                              /* fp16 [M, NH*D] */
  float* lse;                                  /* fp32 [NH, M] */
  float* s2;                                   /* fp32 [M, H] (output) */
  uint16_t* y2;                                /* fp16 [M, H] */
  float* rstd2;                                /* fp32 [M] */
  uint16_t* gu;                                /* fp16 [M, 2I] */
  /* transient */
  uint16_t* qkv;                               /* fp16 [M, W] */
  uint16_t* o;                                 /* fp16 [M, H] */
  uint16_t* act;                               /* fp16 [M, I] */
  float* down_part;                            /* fp32 [p_down, M, H] when p_down > 1 */
  uint16_t* d;                                 /* fp16 [M, H] (output) */
} SoupkLayerFwd;

typedef struct SoupkLayerBwd {
  const float* s_in;                           /* the forward's input, and its saved tensors */
  const float* s1;
  const float* rstd1;
  const uint16_t* y;
  const uint16_t* t;
  const uint16_t* qkv_r;
  const uint16_t* attn;
  const float* lse;
  const float* s2;
  const float* rstd2;
  const uint16_t* y2;
  uint16_t* gu;                                /* overwritten with its gradient */
  int32_t has_delta;                           /* 0: the forward's delta was NULL */
  int32_t algo_down_dx, algo_gu_dx, algo_o_dx, algo_qkv_dx;
  const float* g_s;                            /* fp32 [M, H] gradient of s2 */
  const uint16_t* g_d;                         /* fp16 [M, H] gradient of d */
  /* scratch */
  uint16_t* dact;                              /* fp16 [M, I] */
  float* gu_part;                              /* fp32 [p_gu, M, H] when p_gu > 1 */
  uint16_t* g_y2;                              /* fp16 [M, H] */
  float* g_s1;                                 /* fp32 [M, H] */
  uint16_t* g_o;                               /* fp16 [M, H] */
  uint16_t* g_a;                               /* fp16 [M, NH*D] */
  float* attn_ws;                              /* soupk_attention_varlen_bwd's workspace */
  uint16_t* dqkv;                              /* fp16 [M, W] */
  uint16_t* dt;                                /* fp16 [M, 2r] */
  uint16_t* dy;                                /* fp16 [M, H] */
  float* lora_ws;                              /* soupk_lora_bwd_params' workspace */
  int64_t lora_ws_floats;
  /* outputs */
  float* g_s_in;                               /* fp32 [M, H]; without delta, the norm's part
                                                  only (the caller adds g_s1) */
  uint16_t* g_delta;                           /* fp16 [M, H], or NULL without delta */
  float* d_aq;                                 /* fp32 [r, H] */
  float* d_av;
  float* d_bq;                                 /* fp32 [NH*D, r] */
  float* d_bv;                                 /* fp32 [NKV*D, r] */
} SoupkLayerBwd;

int soupk_layer_fwd(const SoupkLayerDims* dims, const SoupkLayerFwd* a, void* stream);
int soupk_layer_bwd(const SoupkLayerDims* dims, const SoupkLayerBwd* a, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SOUPK_H */
