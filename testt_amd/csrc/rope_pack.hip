// LoRA add + rotary embedding + scatter of q/k/v into the padded [B, heads, T, D] layout, and
// its backward (gather + transposed rotation).
//
// Reference: solution/rope.py:24-75 (rope_pack_fwd_kernel), solution/rope.py:78-128
// (rope_pack_bwd_kernel), launched from RopePack, solution/rope.py:136-176.  The rotation is
// transformers' apply_rotary_pos_emb / rotate_half (modeling_qwen2.py:105-135):
// q*cos + rotate_half(q)*sin, i.e. (x1*c1 - x2*s1, x2*c2 + x1*s2) with each product rounded.
//
// Mapping (gfx950): a work item is one 8-dim slice of one head of one token, together with the
// matching 8 dims of the head's other half (the rotation partner), so a thread does two 16-byte
// fp16 loads of qkv, up to four 16-byte loads of fp32 LoRA delta, two 16-byte stores, and reads
// its cos/sin slices from LDS, where the workgroup staged the rows of its tokens once (one
// 16-byte load per thread; eight per thread straight from the tables would make the vector
// memory unit, not HBM, set the pace).  Items are numbered token-major, so a wavefront reads a
// token's 4 KiB qkv row in full.  The token's position is loaded before the streaming loads
// (its latency then overlaps theirs), and b = p / T, t = p % T use a 32-bit multiply-high
// divider (a 64-bit division is a long instruction sequence on the path to the stores).  In the forward pass the workgroups
// after the token workgroups write zeros at the padded positions that no token maps to
// (pos_inv[p] < 0), replacing the three torch.zeros memsets of the reference.

#include <type_traits>

#include "soupk_common.hpp"
#include "fastdiv.hpp"

namespace soupk {
namespace {

// Workgroup sizes: the vector forward kernels take 512 items (4 tokens of Qwen2.5-1.5B's 16
// heads x 8 chunks) per workgroup, the backward and generic kernels 256.  Measured on MI355X
// with HBM-resident inputs at 2048 tokens / the ragged 888: the padded forward 6.58 -> 6.45 us,
// ragged 5.84 -> 5.65 us, the token-major forward 6.4-6.6 -> 6.34 us, ragged 4.2 -> 4.06 us;
// 256 or 1024 were slower (1024 badly so on the ragged batch: 7.05 us), and the backward kept
// 256 (4.25 against 4.28 us with 512).
constexpr int kRopeThreads = 256;
constexpr int kRopeFwdThreads = 512;
// Cache policy of the loads per direction (1 = non-temporal), chosen by measurement on MI355X
// at 2048 tokens: every input is read once, and non-temporal loads are used both ways.  With
// inputs read from HBM, the forward pass takes as long with cached loads (6.62 us against 6.65),
// and the 23 MB they leave in the caches slowed the kernels launched after it (the NF4 unpack
// 11.7 us against 11.2, the add+RMSNorm forward 8.6 against 8.2); cached loads only looked
// faster (5.6 us) when the same inputs were re-read out of the Infinity Cache.  Results are
// written with streaming stores (StreamOut: nt | sc1).  The cos/sin tables, shared by every
// token at a position, are always read cached.
#ifndef SOUPK_ROPE_NT_FWD_LD
#define SOUPK_ROPE_NT_FWD_LD 1
#endif
#ifndef SOUPK_ROPE_NT_FWD_LORA_LD
#define SOUPK_ROPE_NT_FWD_LORA_LD SOUPK_ROPE_NT_FWD_LD
#endif
#ifndef SOUPK_ROPE_NT_BWD_LD
#define SOUPK_ROPE_NT_BWD_LD 1
#endif
constexpr bool kFwdNtLd = SOUPK_ROPE_NT_FWD_LD != 0;          // the qkv rows
constexpr bool kFwdLoraNtLd = SOUPK_ROPE_NT_FWD_LORA_LD != 0;  // the LoRA deltas
constexpr bool kBwdNtLd = SOUPK_ROPE_NT_BWD_LD != 0;

struct RopeDims {
  int B, T, NH, NKV;
  uint32_t items;   // (NH + 2*NKV) * HALF/8 items per token or position
  FastDiv per_tok;  // divides by items
  FastDiv per_seq;  // divides by T (positions are < B*T < 2^31, checked by the host)
};

// Position -> (b, t) for 0 <= p < B*T.
__device__ __forceinline__ void split_pos(int64_t p, const RopeDims& dm, int& b, int& t) {
  const uint32_t pu = static_cast<uint32_t>(p);
  const uint32_t q = dm.per_seq.div(pu);
  b = static_cast<int>(q);
  t = static_cast<int>(pu - q * static_cast<uint32_t>(dm.T));
}

template <bool NT>
__device__ __forceinline__ void load8_f32(const float* p, float* v) {
  const f32x4 a = ld<NT>(reinterpret_cast<const f32x4*>(p));
  const f32x4 b = ld<NT>(reinterpret_cast<const f32x4*>(p + 4));
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
template <bool NT>
__device__ __forceinline__ void load8_h(const uint16_t* p, float* v) {
  const u32x4 w = ld<NT>(reinterpret_cast<const u32x4*>(p));
  v[0] = lo_h(w.x); v[1] = hi_h(w.x); v[2] = lo_h(w.y); v[3] = hi_h(w.y);
  v[4] = lo_h(w.z); v[5] = hi_h(w.z); v[6] = lo_h(w.w); v[7] = hi_h(w.w);
}
__device__ __forceinline__ u32x4 pack8_h(const float* v) {
  return u32x4{pack_h2(v[0], v[1]), pack_h2(v[2], v[3]), pack_h2(v[4], v[5]),
               pack_h2(v[6], v[7])};
}
// Streaming stores into q, k, v ([B, heads, T, D] fp16 each) through one descriptor per tensor
// over the whole tensor (the host keeps each below 2^32 bytes).  A lane picks its tensor with a
// branch, never a per-lane choice of descriptor (that would not be wave-uniform).
struct PackedOut {
  StreamOut q, k, v;
  int NH, NKV, T;
  template <int D>
  __device__ __forceinline__ PackedOut(uint16_t* q_, uint16_t* k_, uint16_t* v_,
                                       const RopeDims& dm, std::integral_constant<int, D>)
      : q(q_, static_cast<uint64_t>(dm.B) * dm.NH * dm.T * D * 2u),
        k(k_, static_cast<uint64_t>(dm.B) * dm.NKV * dm.T * D * 2u),
        v(v_, static_cast<uint64_t>(dm.B) * dm.NKV * dm.T * D * 2u),
        NH(dm.NH), NKV(dm.NKV), T(dm.T) {}
  // Stores a (first half) and bh (second half) of the 8-dim slice c of head h at (b, t).
  template <int D>
  __device__ __forceinline__ void store(int h, int b, int t, int c, u32x4 a, u32x4 bh) const {
    constexpr uint32_t kHalfBytes = D;  // D/2 fp16
    if (h < NH) {
      const uint32_t off = ((static_cast<uint32_t>(b) * NH + h) * T + t) * (2u * D) + 16u * c;
      q.store(off, a);
      q.store(off + kHalfBytes, bh);
    } else if (h < NH + NKV) {
      const uint32_t off =
          ((static_cast<uint32_t>(b) * NKV + (h - NH)) * T + t) * (2u * D) + 16u * c;
      k.store(off, a);
      k.store(off + kHalfBytes, bh);
    } else {
      const uint32_t off =
          ((static_cast<uint32_t>(b) * NKV + (h - NH - NKV)) * T + t) * (2u * D) + 16u * c;
      v.store(off, a);
      v.store(off + kHalfBytes, bh);
    }
  }
};
// The cos/sin rows of the tokens a workgroup touches are staged once in LDS (per token 2*D fp32:
// cos then sin), instead of every thread reading its 4 x 32 bytes of them from L1/L2.  With at
// least 18 items per token (the host's condition) a workgroup of THREADS consecutive items
// spans at most ceil((THREADS - 1) / 18) + 1 <= THREADS / 18 + 2 tokens.
template <int THREADS>
constexpr int rope_max_tok() {
  return THREADS / 18 + 2;
}

template <int HALF, int THREADS>
__device__ __forceinline__ int stage_tables(f32x4* tab, const float* __restrict__ cos_t,
                                            const float* __restrict__ sin_t,
                                            const int64_t* __restrict__ pos, uint32_t tok0,
                                            uint32_t ntok, const RopeDims& dm) {
  constexpr int D = 2 * HALF;
  constexpr int Q = D / 4;  // float4 per table row
  const int64_t slots = static_cast<int64_t>(dm.B) * dm.T;
  for (int i = threadIdx.x; i < static_cast<int>(ntok) * 2 * Q; i += THREADS) {
    const int j = i / (2 * Q), q = i % (2 * Q);
    const int64_t p = pos[tok0 + j];
    int b = 0, t = 0;  // (row 0 for an invalid position: the host guarantees T >= 1)
    if (p >= 0 && p < slots) split_pos(p, dm, b, t);
    const float* src = q < Q ? cos_t + static_cast<int64_t>(t) * D + 4 * q
                             : sin_t + static_cast<int64_t>(t) * D + 4 * (q - Q);
    tab[i] = *reinterpret_cast<const f32x4*>(src);
  }
  return 2 * Q;  // f32x4 per staged token
}

__device__ __forceinline__ void lds8(const f32x4* p, float* v) {
  const f32x4 a = p[0], b = p[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// TOKENS = false: q, k, v in the padded [B, heads, T, D] layout (the reference's), pad
// positions zeroed by the workgroups after the token ones.  TOKENS = true: one token-major
// output, q = [rows, (NH + 2*NKV) * D] in qkv's own layout (rotated q, rotated k, v + LoRA),
// the form the varlen attention reads; k and v are unused and a token whose position has no
// place (outside [0, B*T)) gets a row of zeros.
template <int HALF, bool TOKENS>
__global__ __launch_bounds__(kRopeFwdThreads) void rope_pack_fwd_kernel(
    const uint16_t* __restrict__ qkv, const void* __restrict__ lora_q,
    const void* __restrict__ lora_v, int lora_f32, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, const int64_t* __restrict__ pos,
    const int32_t* __restrict__ pos_inv, uint16_t* __restrict__ q, uint16_t* __restrict__ k,
    uint16_t* __restrict__ v, int64_t rows, RopeDims dm, int64_t tok_blocks) {
  constexpr int D = 2 * HALF;
  constexpr int CPH = HALF / 8;  // items per head
  __shared__ f32x4 tab[rope_max_tok<kRopeFwdThreads>() * D / 2];
  const int heads = dm.NH + 2 * dm.NKV;
  const int64_t slots = static_cast<int64_t>(dm.B) * dm.T;
  if (!TOKENS && static_cast<int64_t>(blockIdx.x) >= tok_blocks) {
    // Zero the padded positions with no token.
    const uint32_t g = (blockIdx.x - static_cast<uint32_t>(tok_blocks)) * kRopeFwdThreads +
                       threadIdx.x;
    const uint32_t p = dm.per_tok.div(g);
    if (p >= slots || pos_inv[p] >= 0) return;
    const int it = static_cast<int>(g - p * dm.items);
    const int h = it / CPH, c = it % CPH;
    int b, t;
    split_pos(p, dm, b, t);
    const u32x4 z = {0u, 0u, 0u, 0u};
    PackedOut(q, k, v, dm, std::integral_constant<int, D>()).store<D>(h, b, t, c, z, z);
    return;
  }
  const uint32_t g0 = blockIdx.x * kRopeFwdThreads;
  const uint32_t total = static_cast<uint32_t>(rows) * dm.items;
  const uint32_t tok0 = dm.per_tok.div(g0);
  const uint32_t ntok = dm.per_tok.div(min(g0 + kRopeFwdThreads, total) - 1) - tok0 + 1;
  // Threads past the last item take the last item's indices (so every address they form is in
  // bounds), help stage the tables, and leave after the barrier.
  const bool active = g0 + threadIdx.x < total;
  const uint32_t g = active ? g0 + threadIdx.x : total - 1;
  const uint32_t tok = dm.per_tok.div(g);
  const int it = static_cast<int>(g - tok * dm.items);
  const int h = it / CPH, c = it % CPH;
  const bool is_q = h < dm.NH, is_v = h >= dm.NH + dm.NKV;

  const int64_t p = pos[tok];
  // Issue this thread's qkv and LoRA loads, then stage the tables while they are in flight.
  float x1[8], x2[8], l1[8], l2[8];
  const uint16_t* row = qkv + static_cast<int64_t>(tok) * heads * D + h * D + 8 * c;
  load8_h<kFwdNtLd>(row, x1);
  load8_h<kFwdNtLd>(row + HALF, x2);
  const void* lora = is_q ? lora_q : (is_v ? lora_v : nullptr);
  const bool has_lora = lora != nullptr;
  if (has_lora) {
    const int64_t off = is_q ? static_cast<int64_t>(tok) * dm.NH * D + h * D + 8 * c
                             : static_cast<int64_t>(tok) * dm.NKV * D +
                                   (h - dm.NH - dm.NKV) * D + 8 * c;
    if (lora_f32) {
      load8_f32<kFwdLoraNtLd>(static_cast<const float*>(lora) + off, l1);
      load8_f32<kFwdLoraNtLd>(static_cast<const float*>(lora) + off + HALF, l2);
    } else {
      load8_h<kFwdLoraNtLd>(static_cast<const uint16_t*>(lora) + off, l1);
      load8_h<kFwdLoraNtLd>(static_cast<const uint16_t*>(lora) + off + HALF, l2);
    }
  }
  const int per = stage_tables<HALF, kRopeFwdThreads>(tab, cos_t, sin_t, pos, tok0, ntok, dm);
  __syncthreads();
  if (!active) return;
  // (token-major rows: one descriptor over the whole output; the host keeps it < 2^32 bytes)
  const uint32_t tok_off = (tok * static_cast<uint32_t>(heads) + h) * (2u * D) + 16u * c;
  if (p < 0 || p >= slots) {
    if constexpr (TOKENS) {
      const StreamOut out(q, static_cast<uint64_t>(rows) * heads * D * 2u);
      const u32x4 z = {0u, 0u, 0u, 0u};
      out.store(tok_off, z);
      out.store(tok_off + 2u * HALF, z);
    }
    return;
  }
  int b, t;
  split_pos(p, dm, b, t);
  if (has_lora) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x1[i] = x1[i] + l1[i];
      x2[i] = x2[i] + l2[i];
    }
  }
  if (!is_v) {
    const f32x4* tr = tab + (tok - tok0) * per;
    float c1[8], c2[8], s1[8], s2[8];
    lds8(tr + 2 * c, c1);
    lds8(tr + HALF / 4 + 2 * c, c2);
    lds8(tr + D / 4 + 2 * c, s1);
    lds8(tr + D / 4 + HALF / 4 + 2 * c, s2);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float r1 = x1[i] * c1[i] - x2[i] * s1[i];
      const float r2 = x2[i] * c2[i] + x1[i] * s2[i];
      x1[i] = r1;
      x2[i] = r2;
    }
  }
  if constexpr (TOKENS) {
    const StreamOut out(q, static_cast<uint64_t>(rows) * heads * D * 2u);
    out.store(tok_off, pack8_h(x1));
    out.store(tok_off + 2u * HALF, pack8_h(x2));
  } else {
    PackedOut(q, k, v, dm, std::integral_constant<int, D>())
        .store<D>(h, b, t, c, pack8_h(x1), pack8_h(x2));
  }
}

template <int HALF>
__global__ __launch_bounds__(kRopeThreads) void rope_pack_bwd_kernel(
    const uint16_t* __restrict__ dq, const uint16_t* __restrict__ dk,
    const uint16_t* __restrict__ dv, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, const int64_t* __restrict__ pos,
    uint16_t* __restrict__ dqkv, int64_t rows, RopeDims dm) {
  constexpr int D = 2 * HALF;
  constexpr int CPH = HALF / 8;
  __shared__ f32x4 tab[rope_max_tok<kRopeThreads>() * D / 2];
  const int heads = dm.NH + 2 * dm.NKV;
  const int64_t slots = static_cast<int64_t>(dm.B) * dm.T;
  const uint32_t g0 = blockIdx.x * kRopeThreads;
  const uint32_t total = static_cast<uint32_t>(rows) * dm.items;
  const uint32_t tok0 = dm.per_tok.div(g0);
  const uint32_t ntok = dm.per_tok.div(min(g0 + kRopeThreads, total) - 1) - tok0 + 1;
  // Threads past the last item take the last item's indices (every address they form is in
  // bounds), help stage the tables, and leave after the barrier.
  const bool active = g0 + threadIdx.x < total;
  const uint32_t g = active ? g0 + threadIdx.x : total - 1;
  const uint32_t tok = dm.per_tok.div(g);
  const int it = static_cast<int>(g - tok * dm.items);
  const int h = it / CPH, c = it % CPH;
  const bool is_q = h < dm.NH, is_v = h >= dm.NH + dm.NKV;
  const int64_t p = pos[tok];
  const bool valid = p >= 0 && p < slots;
  int b = 0, t = 0;
  if (valid) split_pos(p, dm, b, t);
  float g1[8], g2[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) g1[i] = g2[i] = 0.f;
  const uint16_t* src = is_q ? dq : (is_v ? dv : dk);
  if (valid && src != nullptr) {
    const int64_t base =
        is_q ? ((static_cast<int64_t>(b) * dm.NH + h) * dm.T + t) * D
             : (is_v ? ((static_cast<int64_t>(b) * dm.NKV + (h - dm.NH - dm.NKV)) * dm.T + t) * D
                     : ((static_cast<int64_t>(b) * dm.NKV + (h - dm.NH)) * dm.T + t) * D);
    load8_h<kBwdNtLd>(src + base + 8 * c, g1);
    load8_h<kBwdNtLd>(src + base + HALF + 8 * c, g2);
  }
  const int per = stage_tables<HALF, kRopeThreads>(tab, cos_t, sin_t, pos, tok0, ntok, dm);
  __syncthreads();
  if (!active) return;
  // Streaming stores through one descriptor over dqkv (the host keeps it below 2^32 bytes).
  const StreamOut out(dqkv, static_cast<uint64_t>(rows) * heads * D * 2u);
  const uint32_t off = (tok * static_cast<uint32_t>(heads) + h) * (2u * D) + 16u * c;
  if (!is_v) {
    const f32x4* tr = tab + (tok - tok0) * per;
    float c1[8], c2[8], s1[8], s2[8];
    lds8(tr + 2 * c, c1);
    lds8(tr + HALF / 4 + 2 * c, c2);
    lds8(tr + D / 4 + 2 * c, s1);
    lds8(tr + D / 4 + HALF / 4 + 2 * c, s2);
    float o1[8], o2[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      o1[i] = g1[i] * c1[i] + g2[i] * s2[i];
      o2[i] = g2[i] * c2[i] - g1[i] * s1[i];
    }
    out.store(off, pack8_h(o1));
    out.store(off + 2u * HALF, pack8_h(o2));
  } else {
    out.store(off, pack8_h(g1));
    out.store(off + 2u * HALF, pack8_h(g2));
  }
}

// ---- generic forms: any even D, one thread per (token or position, head, dim of first half)
__global__ __launch_bounds__(kRopeThreads) void rope_pack_fwd_generic_kernel(
    const uint16_t* __restrict__ qkv, const void* __restrict__ lora_q,
    const void* __restrict__ lora_v, int lora_f32, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, const int64_t* __restrict__ pos,
    const int32_t* __restrict__ pos_inv, uint16_t* __restrict__ q, uint16_t* __restrict__ k,
    uint16_t* __restrict__ v, int64_t rows, int B, int T, int NH, int NKV, int D,
    int64_t tok_items) {
  const int half = D / 2;
  const int heads = NH + 2 * NKV;
  const int64_t per = static_cast<int64_t>(heads) * half;
  const int64_t slots = static_cast<int64_t>(B) * T;
  const int64_t g = static_cast<int64_t>(blockIdx.x) * kRopeThreads + threadIdx.x;
  auto lora = [&](const void* l, int64_t off) -> float {
    return lora_f32 ? static_cast<const float*>(l)[off] : h2f(static_cast<const uint16_t*>(l)[off]);
  };
  auto put = [&](uint16_t* base, int i, float a, float bv) {
    base[i] = static_cast<uint16_t>(pack_h2(a, 0.f) & 0xffffu);
    base[i + half] = static_cast<uint16_t>(pack_h2(bv, 0.f) & 0xffffu);
  };
  int64_t p, tok = -1;
  int64_t it;
  if (g < tok_items) {
    tok = g / per;
    it = g % per;
    p = pos[tok];
    if (p < 0 || p >= slots) return;
  } else {
    const int64_t z = g - tok_items;
    p = z / per;
    it = z % per;
    if (p >= slots || pos_inv == nullptr || pos_inv[p] >= 0) return;
  }
  const int h = static_cast<int>(it / half), i = static_cast<int>(it % half);
  const int b = static_cast<int>(p / T), t = static_cast<int>(p % T);
  uint16_t* base;
  if (h < NH)
    base = q + ((static_cast<int64_t>(b) * NH + h) * T + t) * D;
  else if (h < NH + NKV)
    base = k + ((static_cast<int64_t>(b) * NKV + (h - NH)) * T + t) * D;
  else
    base = v + ((static_cast<int64_t>(b) * NKV + (h - NH - NKV)) * T + t) * D;
  if (tok < 0) {
    put(base, i, 0.f, 0.f);
    return;
  }
  const uint16_t* row = qkv + tok * heads * D + h * D;
  float x1 = h2f(row[i]), x2 = h2f(row[i + half]);
  if (h < NH && lora_q != nullptr) {
    const int64_t off = tok * NH * D + h * D + i;
    x1 = x1 + lora(lora_q, off);
    x2 = x2 + lora(lora_q, off + half);
  }
  if (h >= NH + NKV) {
    if (lora_v != nullptr) {
      const int64_t off = tok * NKV * D + (h - NH - NKV) * D + i;
      x1 = x1 + lora(lora_v, off);
      x2 = x2 + lora(lora_v, off + half);
    }
    put(base, i, x1, x2);
    return;
  }
  const float* cr = cos_t + static_cast<int64_t>(t) * D;
  const float* sr = sin_t + static_cast<int64_t>(t) * D;
  put(base, i, x1 * cr[i] - x2 * sr[i], x2 * cr[i + half] + x1 * sr[i + half]);
}

__global__ __launch_bounds__(kRopeThreads) void rope_pack_bwd_generic_kernel(
    const uint16_t* __restrict__ dq, const uint16_t* __restrict__ dk,
    const uint16_t* __restrict__ dv, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, const int64_t* __restrict__ pos,
    uint16_t* __restrict__ dqkv, int64_t rows, int B, int T, int NH, int NKV, int D) {
  const int half = D / 2;
  const int heads = NH + 2 * NKV;
  const int64_t per = static_cast<int64_t>(heads) * half;
  const int64_t slots = static_cast<int64_t>(B) * T;
  const int64_t g = static_cast<int64_t>(blockIdx.x) * kRopeThreads + threadIdx.x;
  if (g >= rows * per) return;
  const int64_t tok = g / per;
  const int h = static_cast<int>((g % per) / half), i = static_cast<int>(g % half);
  const int64_t p = pos[tok];
  const bool valid = p >= 0 && p < slots;
  const int b = valid ? static_cast<int>(p / T) : 0, t = valid ? static_cast<int>(p % T) : 0;
  float g1 = 0.f, g2 = 0.f;
  const uint16_t* src;
  int64_t base;
  if (h < NH) {
    src = dq;
    base = ((static_cast<int64_t>(b) * NH + h) * T + t) * D;
  } else if (h < NH + NKV) {
    src = dk;
    base = ((static_cast<int64_t>(b) * NKV + (h - NH)) * T + t) * D;
  } else {
    src = dv;
    base = ((static_cast<int64_t>(b) * NKV + (h - NH - NKV)) * T + t) * D;
  }
  if (valid && src != nullptr) {
    g1 = h2f(src[base + i]);
    g2 = h2f(src[base + i + half]);
  }
  float o1 = g1, o2 = g2;
  if (valid && h < NH + NKV) {  // (an invalid position reads no table row; T may be 0)
    const float* cr = cos_t + static_cast<int64_t>(t) * D;
    const float* sr = sin_t + static_cast<int64_t>(t) * D;
    o1 = g1 * cr[i] + g2 * sr[i + half];
    o2 = g2 * cr[i + half] - g1 * sr[i];
  }
  uint16_t* out = dqkv + tok * heads * D + h * D;
  out[i] = static_cast<uint16_t>(pack_h2(o1, 0.f) & 0xffffu);
  out[i + half] = static_cast<uint16_t>(pack_h2(o2, 0.f) & 0xffffu);
}

inline bool aligned(const void* p, uintptr_t a) {
  return p == nullptr || (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

}  // namespace
}  // namespace soupk

using namespace soupk;

extern "C" __attribute__((visibility("default"))) int soupk_rope_pack_fwd(
    const uint16_t* qkv, const void* lora_q, const void* lora_v, int32_t lora_dtype,
    const float* cos, const float* sin, const int64_t* pos, const int32_t* pos_inv, uint16_t* q,
    uint16_t* k, uint16_t* v, int64_t rows, int32_t B, int32_t T, int32_t NH, int32_t NKV,
    int32_t D, void* stream) {
  if (rows < 0 || B < 0 || T < 0 || NH < 0 || NKV < 0 || D <= 0 || (D & 1)) return kInvalid;
  if (lora_dtype != SOUPK_DTYPE_F16 && lora_dtype != SOUPK_DTYPE_F32) return kInvalid;
  const int64_t slots = static_cast<int64_t>(B) * T;
  const int64_t zero_slots = pos_inv != nullptr ? slots : 0;
  // No position exists (B*T = 0): no token has a destination, nothing to write.
  if ((rows == 0 && zero_slots == 0) || NH + 2 * NKV == 0 || slots == 0) return kOk;
  if (!q || !k || !v || !cos || !sin || (rows > 0 && (!qkv || !pos))) return kInvalid;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int half = D / 2;
  const int heads = NH + 2 * NKV;
  const int lora_align = 16;
  // (items per token >= 18: a workgroup's items span at most rope_max_tok() tokens)
  // (the stores address q, k and v with 32-bit byte offsets)
  const bool vec = half == 64 && heads * (half / 8) >= 18 && slots < (int64_t{1} << 31) &&
                   slots * (NH > NKV ? NH : NKV) * D * 2 < (int64_t{1} << 32) &&
                   aligned(qkv, 16) &&
                   aligned(cos, 16) && aligned(sin, 16) && aligned(q, 16) && aligned(k, 16) &&
                   aligned(v, 16) && aligned(lora_q, lora_align) && aligned(lora_v, lora_align);
  if (vec) {
    RopeDims dm;
    dm.B = B; dm.T = T; dm.NH = NH; dm.NKV = NKV;
    dm.items = static_cast<uint32_t>(heads * (half / 8));
    dm.per_tok = FastDiv(dm.items);
    dm.per_seq = FastDiv(static_cast<uint32_t>(T));
    const int64_t tok_items = rows * dm.items;
    const int64_t zero_items = zero_slots * dm.items;
    if (tok_items + zero_items >= (int64_t{1} << 31)) return kInvalid;
    const int64_t tok_blocks = (tok_items + kRopeFwdThreads - 1) / kRopeFwdThreads;
    const int64_t blocks = tok_blocks + (zero_items + kRopeFwdThreads - 1) / kRopeFwdThreads;
    return launch_kernel(rope_pack_fwd_kernel<64, false>, dim3(static_cast<unsigned>(blocks)),
                         dim3(kRopeFwdThreads), st, qkv, lora_q, lora_v,
                         static_cast<int>(lora_dtype == SOUPK_DTYPE_F32), cos, sin, pos, pos_inv,
                         q, k, v, rows, dm, tok_blocks);
  }
  const int64_t per = static_cast<int64_t>(heads) * half;
  const int64_t tok_items = rows * per;
  const int64_t total = tok_items + zero_slots * per;
  const int64_t blocks = (total + kRopeThreads - 1) / kRopeThreads;
  if (blocks > 0x7fffffff) return kInvalid;
  return launch_kernel(rope_pack_fwd_generic_kernel, dim3(static_cast<unsigned>(blocks)),
                       dim3(kRopeThreads), st, qkv, lora_q, lora_v,
                       static_cast<int>(lora_dtype == SOUPK_DTYPE_F32), cos, sin, pos, pos_inv, q,
                       k, v, rows, B, T, NH, NKV, D, tok_items);
}

extern "C" __attribute__((visibility("default"))) int soupk_rope_pack_bwd(
    const uint16_t* dq, const uint16_t* dk, const uint16_t* dv, const float* cos,
    const float* sin, const int64_t* pos, uint16_t* dqkv, int64_t rows, int32_t B, int32_t T,
    int32_t NH, int32_t NKV, int32_t D, void* stream) {
  if (rows < 0 || B < 0 || T < 0 || NH < 0 || NKV < 0 || D <= 0 || (D & 1)) return kInvalid;
  if (rows == 0 || NH + 2 * NKV == 0) return kOk;
  // With B*T = 0 every position is out of range: the gradient rows are zeros and the (empty)
  // tables are not read.
  const bool no_slots = static_cast<int64_t>(B) * T == 0;
  if (!dqkv || !pos || (!no_slots && (!cos || !sin))) return kInvalid;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int half = D / 2;
  const int heads = NH + 2 * NKV;
  // (the vector kernel stages table row 0 for invalid positions, so it needs T >= 1)
  const int64_t slots = static_cast<int64_t>(B) * T;
  // (the stores address dqkv with 32-bit byte offsets)
  const bool vec = half == 64 && heads * (half / 8) >= 18 && slots > 0 &&
                   slots < (int64_t{1} << 31) && rows * heads * D * 2 < (int64_t{1} << 32) &&
                   aligned(dq, 16) &&
                   aligned(dk, 16) && aligned(dv, 16) && aligned(cos, 16) && aligned(sin, 16) &&
                   aligned(dqkv, 16);
  if (vec) {
    RopeDims dm;
    dm.B = B; dm.T = T; dm.NH = NH; dm.NKV = NKV;
    dm.items = static_cast<uint32_t>(heads * (half / 8));
    dm.per_tok = FastDiv(dm.items);
    dm.per_seq = FastDiv(static_cast<uint32_t>(T));
    const int64_t items = rows * dm.items;
    if (items >= (int64_t{1} << 31)) return kInvalid;
    return launch_kernel(rope_pack_bwd_kernel<64>,
                         dim3(static_cast<unsigned>((items + kRopeThreads - 1) / kRopeThreads)),
                         dim3(kRopeThreads), st, dq, dk, dv, cos, sin, pos, dqkv, rows, dm);
  }
  const int64_t total = rows * heads * half;
  const int64_t blocks = (total + kRopeThreads - 1) / kRopeThreads;
  if (blocks > 0x7fffffff) return kInvalid;
  return launch_kernel(rope_pack_bwd_generic_kernel, dim3(static_cast<unsigned>(blocks)),
                       dim3(kRopeThreads), st, dq, dk, dv, cos, sin, pos, dqkv, rows, B, T, NH,
                       NKV, D);
}

extern "C" __attribute__((visibility("default"))) int soupk_rope_pack_tokens(
    const uint16_t* qkv, const void* lora_q, const void* lora_v, int32_t lora_dtype,
    const float* cos, const float* sin, const int64_t* pos, uint16_t* out, int64_t rows,
    int32_t B, int32_t T, int32_t NH, int32_t NKV, int32_t D, void* stream) {
  if (rows < 0 || B < 0 || T < 0 || NH < 0 || NKV < 0 || D != 128) return kInvalid;
  if (lora_dtype != SOUPK_DTYPE_F16 && lora_dtype != SOUPK_DTYPE_F32) return kInvalid;
  const int heads = NH + 2 * NKV;
  if (rows == 0 || heads == 0) return kOk;
  const int64_t slots = static_cast<int64_t>(B) * T;
  if (!qkv || !pos || !out || !cos || !sin || T < 1) return kInvalid;
  // (items per token >= 18: a workgroup's items span at most rope_max_tok() tokens; the
  // stores address `out` with 32-bit byte offsets)
  if (heads * 8 < 18 || slots >= (int64_t{1} << 31) || rows * heads * D * 2 >= (int64_t{1} << 32))
    return kInvalid;
  if (!aligned(qkv, 16) || !aligned(cos, 16) || !aligned(sin, 16) || !aligned(out, 16) ||
      !aligned(lora_q, 16) || !aligned(lora_v, 16))
    return kInvalid;
  RopeDims dm;
  dm.B = B; dm.T = T; dm.NH = NH; dm.NKV = NKV;
  dm.items = static_cast<uint32_t>(heads * 8);
  dm.per_tok = FastDiv(dm.items);
  dm.per_seq = FastDiv(static_cast<uint32_t>(T));
  const int64_t items = rows * dm.items;
  if (items >= (int64_t{1} << 31)) return kInvalid;
  const int64_t blocks = (items + kRopeFwdThreads - 1) / kRopeFwdThreads;
  return launch_kernel(rope_pack_fwd_kernel<64, true>, dim3(static_cast<unsigned>(blocks)),
                       dim3(kRopeFwdThreads), static_cast<hipStream_t>(stream), qkv, lora_q, lora_v,
                       static_cast<int>(lora_dtype == SOUPK_DTYPE_F32), cos, sin, pos,
                       static_cast<const int32_t*>(nullptr), out, static_cast<uint16_t*>(nullptr),
                       static_cast<uint16_t*>(nullptr), rows, dm, blocks);
}
