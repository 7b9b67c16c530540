// Small-T (T <= 64) plan of the expert GEMMs, rebuilt in LDS by every workgroup of the
// first GEMM from the routing outputs: the stable token -> local-expert permutation of
// main.py:216-226 (for each local expert in ascending order, its tokens in ascending order,
// as torch.nonzero gives them), the 16-row m-tile table and the K-splits of both GEMMs.
// With at most 512 pairs this takes one round of L2 reads and a few LDS passes, less than
// a separate launch; workgroup 0 also writes the global tables the second GEMM and the
// caller's debug outputs read.
#pragma once

#include "moefp8_device.h"
#include "moefp8_launch.h"

namespace moefp8 {

constexpr int kSmallT = 64;
static_assert(kSmallT <= 256, "pair tokens are stored as bytes");
constexpr int kSmallTile = 16;
constexpr int kSmallPairs = kSmallT * kTopK;
constexpr int kSmallMaxMtiles = kSmallPairs / kSmallTile + kEGlobal;
constexpr int kPlanThreads = 256;   // threads of a workgroup that builds the plan

// What the GEMM reads while it runs ...
struct DecodePlanLds {
  int4 mt[kSmallMaxMtiles];             // {expert, first pair row, rows, OR of pair flags}
  // token of each pair row (T <= 64), as bytes: with ints the workgroup's LDS (32,024 B) no
  // longer let five workgroups share a CU (an empty GEMM1 launch 1 us slower, measured)
  uint8_t tok[kSmallPairs];
  float w[kSmallPairs];                 // routing weight of each pair row
  int n_mt, P, S1, S2;
};
// ... and what only the build uses (free for other use once it returns).
struct DecodePlanScratch {
  unsigned long long tmask[kEGlobal];   // tokens (bit t) that picked each local expert
  int base[kEGlobal];                   // first pair row of each local expert
  int mtb[kEGlobal];                    // first m-tile of each local expert
  int ids[kSmallPairs];                 // local expert of each (token, k) pair, -1 if none
  float w[kSmallPairs];                 // routing weight of each (token, k) pair
  float a2[kSmallT];                    // squared hidden norm of each token
  float esig[2 * kEGlobal];             // weight-scale estimates of each local expert
};

// K-split of a decode GEMM.  Few m-tiles (their groups leave room for at least two splits within
// `budget` units, two per CU): the most splits <= kDecFewSplit within the budget.  Otherwise the
// largest S <= kDecMaxSplit whose units still fit one resident round of the grid
// (n_mt * ncb * S <= slots).  Always S * P <= rows_cap (the partial rows) and S >= ceil(kb / 64) (a
// unit holds the weight scales of its <= 64 K-blocks one per lane).  More splits fill more of the
// grid but lengthen the reduction each group's last unit does; about two units per CU was the best
// count for both GEMMs at T = 1 and 4 (one and two local pairs: GEMM1 S = 8 / 4, GEMM2 S = 4 / 2;
// per call 29.6 -> 29.2 and 37.3 -> 36.5 us against S <= 4 everywhere; S <= 8 everywhere had cost
// 34.3 / 44.4 against 31.6 / 38.9, up to 20 splits 35.4 / 41.4).
// `s_floor`: the fewest splits whose K ranges fit the staged path's LDS rows (kPreMaxKB /
// kPre2MaxKB K-blocks), kept even where one resident round would hold fewer units: GEMM1 at
// T = 64 (19 m-tiles, S = 1 by the round) with S = 2 runs its m-tiles of <= 4 rows on the staged
// path, 187.8 -> 183.9 us per call (GEMM2 with S = 2 there: +15 us, so its floor stays 1).
constexpr int kDecMaxSplit = 4;
constexpr int kDecFewSplit = 8;
constexpr int kPreMaxKB = 28;    // K-blocks a GEMM1 unit can stage (staged path)
constexpr int kPre2MaxKB = 16;   // the same for GEMM2
__device__ __forceinline__ int pick_split(int n_mt, int ncb, int kb, int slots, int P, int rows_cap, int budget,
                                          int s_floor) {
  const int s_min = (kb + kWave - 1) / kWave;
  const int per = n_mt * ncb;   // units per split
  int S = min(kb, kDecMaxSplit);
  if (per > 0 && 2 * per <= budget) S = min(kb, min(kDecFewSplit, budget / per));
  else if (per > 0) S = min(S, max(s_floor, slots / per));
  if (P > 0) S = min(S, rows_cap / P);
  return max(S, s_min);
}

// Builds the plan in `L` using `X` (every thread of a workgroup of kPlanThreads takes part;
// ends with a barrier).
// With `global`, also writes expert_offsets, active, mtile_offsets, info {P, active experts,
// m-tiles, S1, S2}, perm_token, perm_w, tok_slot (each token's pair rows in ascending local
// expert order, -1 past its last) and the m-tile table.
__device__ void build_decode_plan(const DecodePlanArgs& a, DecodePlanLds& L, DecodePlanScratch& X, bool global) {
  const int tid = threadIdx.x, nth = blockDim.x, lane = lane_id(), wave = tid >> 6;
  const int T = a.T, E = a.E_local, NP = T * kTopK;
  // every global input in one round of loads: each thread loads its (at most two) ids and
  // weights, one token norm and its (at most two) expert estimates at clamped indices, with no
  // branch between the loads (loads in bounded loops were each waited for before the next loop's),
  // then stores those in range
  static_assert(2 * kPlanThreads >= kSmallPairs && 2 * kPlanThreads >= 2 * kEGlobal && kPlanThreads >= kSmallT,
                "two loads per thread cover every input");
  int idv[2];
  float wv[2], ev[2];
#pragma unroll
  for (int q = 0; q < 2; q++) {
    const int i = min(tid + q * kPlanThreads, NP - 1), k = min(tid + q * kPlanThreads, 2 * E - 1);
    idv[q] = a.topk_ids[i];
    wv[q] = a.topk_w[i];
    ev[q] = a.esig[k];
  }
  const float av = a.tok_a2[min(tid, T - 1)];
  for (int e = tid; e < E; e += nth) X.tmask[e] = 0ull;
#pragma unroll
  for (int q = 0; q < 2; q++) {
    const int i = tid + q * kPlanThreads;
    if (i < NP) {
      const int le = idv[q] - a.offset;
      X.ids[i] = le >= 0 && le < E ? le : -1;
      X.w[i] = wv[q];
    }
    if (i < 2 * E) X.esig[i] = ev[q];
  }
  if (tid < T) X.a2[tid] = av;
  __syncthreads();
  for (int i = tid; i < NP; i += nth)
    if (X.ids[i] >= 0) atomicOr(&X.tmask[X.ids[i]], 1ull << (i >> 3));
  __syncthreads();

  // per-expert counts -> pair offsets, m-tile offsets, active list (wave 0, ballot prefix sums)
  if (wave == 0) {
    int carry_p = 0, carry_mt = 0, carry_a = 0;
    for (int e0 = 0; e0 < E; e0 += kWave) {
      const int e = e0 + lane;
      const int c = e < E ? __popcll(X.tmask[e]) : 0;
      const int mt = (c + kSmallTile - 1) / kSmallTile;
      int pc = 0, pm = 0;
#pragma unroll
      for (int bit = 0; bit < 7; bit++) {
        pc += lanes_below(__ballot((c >> bit) & 1)) << bit;
        pm += lanes_below(__ballot((mt >> bit) & 1)) << bit;
      }
      const uint64_t act = __ballot(c > 0);
      if (e < E) {
        X.base[e] = carry_p + pc;
        X.mtb[e] = carry_mt + pm;
        for (int j = 0; j < mt; j++)
          L.mt[carry_mt + pm + j] = int4{e, carry_p + pc + kSmallTile * j, min(kSmallTile, c - kSmallTile * j), 0};
        if (global) {
          a.expert_offsets[e] = carry_p + pc;
          a.mtile_offsets[e] = carry_mt + pm;
          if (c > 0) a.active[carry_a + lanes_below(act)] = e;
        }
      }
      carry_p += __builtin_amdgcn_readlane(pc + c, kWave - 1);
      carry_mt += __builtin_amdgcn_readlane(pm + mt, kWave - 1);
      carry_a += (int)__popcll(act);
    }
    if (lane == 0) {
      L.P = carry_p;
      L.n_mt = carry_mt;
      L.S1 = pick_split(carry_mt, a.sp.ncb1, a.sp.kb1, a.sp.slots1, carry_p, a.sp.rows_cap1, a.sp.budget,
                        (a.sp.kb1 + kPreMaxKB - 1) / kPreMaxKB);
      L.S2 = pick_split(carry_mt, a.sp.ncb2, a.sp.kb2, a.sp.slots2, carry_p, a.sp.rows_cap2, a.sp.budget, 1);
      if (global) {
        a.expert_offsets[E] = carry_p;
        a.mtile_offsets[E] = carry_mt;
        a.info[0] = carry_p;
        a.info[1] = carry_a;
        a.info[2] = carry_mt;
        a.info[3] = L.S1;
        a.info[4] = L.S2;
      }
    }
  }
  __syncthreads();

  // pair rows: rank of the token inside its expert (popcount of the lower tokens); the
  // m-tile flags are the OR of its pairs' predicted precision flags
  for (int i0 = 0; i0 < NP; i0 += nth) {
    const int i = i0 + tid;
    const int t = i >> 3, j = i & 7;
    const int le = i < NP ? X.ids[i] : -1;
    // k = rank of this pair's local expert among its token's local experts (8 consecutive
    // lanes hold one token): the combine adds a token's rows in ascending expert order
    int k = 0, n_loc = 0;
#pragma unroll
    for (int q = 0; q < kTopK; q++) {
      const int le_q = __shfl(le >= 0 ? le : kEGlobal, (lane & ~7) + q, kWave);
      k += le_q < le ? 1 : 0;
      n_loc += le_q < kEGlobal ? 1 : 0;
    }
    if (le >= 0) {
      const int pos = X.base[le] + (int)__popcll(X.tmask[le] & ((1ull << t) - 1ull));
      L.tok[pos] = t;
      const float w = X.w[i];
      L.w[pos] = w;
      const float pred = predicted_output_rms(X.a2[t], w, X.esig[2 * le], X.esig[2 * le + 1], a.sqrt_i);
      const int flags = (pred > kPreciseRms ? kFlagExactProducts : 0) | (pred > kOneTermRms ? kFlagTwoTermC : 0);
      if (flags) atomicOr(&L.mt[X.mtb[le] + (pos - X.base[le]) / kSmallTile].w, flags);
      if (global) {
        a.perm_token[pos] = t;
        a.perm_w[pos] = w;
        a.tok_slot[t * kTopK + k] = pos;
      }
    }
    if (global && i < NP && j >= n_loc) a.tok_slot[t * kTopK + j] = -1;
  }
  __syncthreads();
  if (global)
    for (int g = tid; g < L.n_mt; g += nth) a.mtiles[g] = L.mt[g];
}

}  // namespace moefp8
