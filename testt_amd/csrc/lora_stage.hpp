// The fp16 staging of the rank-16 LoRA parameters, shared by the LoRA kernels (lora.hip: the
// standalone staging launch) and the per-layer weight launch (nf4_unpack.hip: the staging done
// by extra workgroups of the NF4 unpack of the layer's projections).
//
// The staged buffer holds the fp16 casts of the fp32 parameters (rounded as .to(torch.float16)
// rounds them) in the layouts the row kernels read with 8- and 16-byte loads:
//   A16  [2r, H]   (A_q rows, then A_v rows)   t's contraction over H
//   A16T [H, 2r]                               dy's contraction over the ranks
//   B16  [NQ + NV, r]                          lq / lv's contraction over the ranks
//   B16T [r, NQ], then [r, NV]                 dt's contraction over NQ / NV
#pragma once

#include "soupk_common.hpp"

namespace soupk {

constexpr int kLoraRank = 16;

// Offsets (halves) of the sections of the staged parameter buffer.
struct StagedLayout {
  int64_t a16, a16t, b16, b16t_q, b16t_v, total;
};

__host__ __device__ inline StagedLayout staged_layout(int64_t H, int64_t NQ, int64_t NV) {
  constexpr int r = kLoraRank;
  StagedLayout L;
  L.a16 = 0;
  L.a16t = 2 * r * H;
  L.b16 = 4 * r * H;
  L.b16t_q = L.b16 + (NQ + NV) * r;
  L.b16t_v = L.b16t_q + r * NQ;
  L.total = L.b16t_v + r * NV;
  return L;
}

// Parameter values to stage: 2r*H of A, then (NQ + NV)*r of B.
__host__ __device__ inline int64_t staged_values(int64_t H, int64_t NQ, int64_t NV) {
  return 2 * kLoraRank * H + (NQ + NV) * kLoraRank;
}

struct LoraStageArgs {
  const float* aq;
  const float* av;
  const float* bq;
  const float* bv;
  _Float16* st;
  int H, NQ, NV;
};

// Parameter value e (< staged_values): its fp16 cast written in both layouts of its section.
__device__ __forceinline__ void lora_stage_value(const LoraStageArgs& a, int64_t e) {
  constexpr int r = kLoraRank;
  const StagedLayout L = staged_layout(a.H, a.NQ, a.NV);
  const int64_t na = 2 * r * static_cast<int64_t>(a.H);
  if (e < na) {
    const int i = static_cast<int>(e / a.H), k = static_cast<int>(e % a.H);
    const _Float16 v =
        static_cast<_Float16>(i < r ? a.aq[e] : a.av[e - r * static_cast<int64_t>(a.H)]);
    a.st[L.a16 + e] = v;
    a.st[L.a16t + static_cast<int64_t>(k) * (2 * r) + i] = v;
  } else if (e < na + static_cast<int64_t>(a.NQ + a.NV) * r) {
    const int64_t e2 = e - na;
    const int j = static_cast<int>(e2 / r), i = static_cast<int>(e2 % r);
    const bool q = j < a.NQ;
    const _Float16 v =
        static_cast<_Float16>(q ? a.bq[e2] : a.bv[e2 - static_cast<int64_t>(a.NQ) * r]);
    a.st[L.b16 + e2] = v;
    if (q) a.st[L.b16t_q + static_cast<int64_t>(i) * a.NQ + j] = v;
    else a.st[L.b16t_v + static_cast<int64_t>(i) * a.NV + (j - a.NQ)] = v;
  }
}

}  // namespace soupk
