// Host-side launchers of the gfx950 MoE kernels (one per kernel family).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moefp8 {

// Inputs and outputs of the magnitude estimates behind the exact-product decision.
struct MagInputs {
  const uint8_t* hidden;
  const float* hscale;
  const float* s13;
  const float* s2;
  int H, I, E_local;
  float* tok_a2;   // [T]   squared norm of each dequantised hidden row
  float* esig;     // [E, 2] rms estimates of W13 and W2 entries
};

// K-split choice of the small-T GEMMs: the largest S in {8, 4, 2, 1} with
// m_tiles * ncb * S <= slots, S * P <= rows_cap and S <= kb.
struct SplitPolicy {
  int slots1, ncb1, kb1, rows_cap1;   // GEMM1: grid workgroups, column blocks per m-tile, K-blocks (H/128)
  int slots2, ncb2, kb2, rows_cap2;   // GEMM2: the same for H columns and I/128 K-blocks
};

// Routing of every token (main.py:139-165): topk_ids [T,8] ascending, topk_w [T,8];
// with `mag`, also the magnitude estimates.
void launch_route(const void* logits, int logits_dt, const void* bias, int bias_dt, int64_t T, float rsf,
                  int* topk_ids, float* topk_w, const MagInputs* mag, hipStream_t stream);

// Stable counting sort of the local (token, expert) pairs (main.py:216-226), plus the
// per-pair exact-product flag.
void launch_permute(const int* topk_ids, const float* topk_w, int T, int E_local, int offset, int tile_m,
                    int* expert_offsets, int* perm_token, float* perm_w, int* tok_slot, int* active,
                    int* mtile_offsets, int* info, const float* tok_a2, const float* esig, int I,
                    uint8_t* perm_exact, hipStream_t stream);

// The same permutation for T <= 64 in one workgroup with no serial loop, plus the
// m-tile table (tile height 16) and the K-splits of the small-T GEMMs.
void launch_permute_small(const int* topk_ids, const float* topk_w, int T, int E_local, int offset,
                          int* expert_offsets, int* perm_token, float* perm_w, int* tok_slot, int* active,
                          int* mtile_offsets, int* info, const float* tok_a2, const float* esig, int I,
                          uint8_t* perm_exact, int4* mtiles, const SplitPolicy& sp, hipStream_t stream);

// Pointers into the caller's workspace produced by routing + permutation.
struct Plan {
  const int* expert_offsets;  // [E_local + 1]
  const int* perm_token;      // [Pmax]
  const float* perm_w;        // [Pmax]
  const int* tok_slot;        // [T * 8]
  const int* active;          // [E_local]
  const int* mtile_offsets;   // [E_local + 1]
  const int* info;            // {P, n_active, m_tiles, S1, S2}: S1/S2 = K-splits of the small-T GEMMs
  const uint8_t* exact;       // [Pmax] 1 = pair runs on the exact-product (f16 MFMA) path
  const int4* mtiles;         // small T: per m-tile {expert, first pair, rows, 0}
};

struct Problem {
  const uint8_t* hidden;  // [T, H]
  const float* hscale;    // [H/128, T]
  const uint8_t* w13;     // [E, 2I, H]
  const float* s13;       // [E, 2I/128, H/128]
  const uint8_t* w2;      // [E, H, I]
  const float* s2;        // [E, H/128, I/128]
  int T, E_local, H, I;
};

// Small-T path: GEMM1 partials -> activation (f16 hi/lo C) -> GEMM2 partials.
struct CHalf {
  _Float16* hi;   // [Pmax][I]
  _Float16* lo;   // [Pmax][I]
  float* scale;   // [Pmax][I/128]
};
int decode_grid();
int decode_unit_groups();
void launch_gemm1_decode(const Problem& pb, const Plan& pl, float* gbuf, hipStream_t stream);
void launch_activation_decode(const Problem& pb, const Plan& pl, const float* gbuf, const CHalf& ch, int pmax,
                              hipStream_t stream);
void launch_gemm2_decode(const Problem& pb, const Plan& pl, const CHalf& ch, float* obuf, hipStream_t stream);

// GEMM1 -> GEMM2 activations of the large-T path: up to kMaxTerms e4m3 planes of C,
// one fp32 scale per (pair, 128 columns) and the term count of every 16-row sub-tile.
struct CSplit {
  uint8_t* q;       // [kMaxTerms][plane] bytes, plane = pmax * I
  size_t plane;
  float* scale;     // [pmax][I/128]
  uint8_t* kmax;    // [max_mtiles][tile_m/16][I/128]: e4m3 term count, or kExactTerms
  _Float16* c16;    // [2][pmax][I] two-term f16 split of C for exact-product sub-tiles
};

// kmax marker of a sub-tile that runs GEMM2 on the exact-product path.
constexpr int kExactTerms = 16;

// Large-T path: LDS-staged grouped GEMM1 (+SwiGLU + multi-term split of C) and GEMM2.
void launch_gemm1_prefill(const Problem& pb, const Plan& pl, int tile_m, const CSplit& cs, int max_mtiles,
                          hipStream_t stream);
void launch_gemm2_prefill(const Problem& pb, const Plan& pl, int tile_m, const CSplit& cs, float* obuf,
                          int max_mtiles, hipStream_t stream);

// out[t] = bf16(sum over t's local pairs in ascending expert order of obuf[pair]) (main.py:240-243).
void launch_combine(const Plan& pl, const float* obuf, uint16_t* out, int T, int H, hipStream_t stream);

int num_compute_units();

}  // namespace moefp8
