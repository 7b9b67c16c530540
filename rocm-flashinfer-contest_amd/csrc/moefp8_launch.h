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

// Inputs of the small-T GEMMs' K-split choice (pick_split).
struct SplitPolicy {
  int slots1, ncb1, kb1, rows_cap1;   // GEMM1: grid workgroups, column blocks per m-tile, K-blocks (H/128)
  int slots2, ncb2, kb2, rows_cap2;   // GEMM2: the same for H columns and I/128 K-blocks
  int budget;                         // units that few m-tiles split into: two per CU
};

// Routing of every token (main.py:139-165): topk_ids [T,8] ascending, topk_w [T,8];
// with `mag`, also the magnitude estimates; zeroes zero[i * kCounterStride] for i < n_zero
// (arrival counters and flags of the small-T GEMMs) on the way.
void launch_route(const void* logits, int logits_dt, const void* bias, int bias_dt, int64_t T, float rsf,
                  int* topk_ids, float* topk_w, const MagInputs* mag, int* zero, int n_zero, hipStream_t stream);

// Inputs and global outputs of the small-T plan (permutation of main.py:216-226, m-tiles
// of height 16, K-splits) that the first small-T GEMM builds.
struct DecodePlanArgs {
  const int* topk_ids;
  const float* topk_w;
  const float* tok_a2;
  const float* esig;
  int T, E_local, offset;
  float sqrt_i;
  SplitPolicy sp;
  int* expert_offsets;  // [E_local + 1]
  int* mtile_offsets;   // [E_local + 1]
  int* active;          // [E_local]
  int* info;
  int* perm_token;      // [Pmax]
  float* perm_w;        // [Pmax]
  int* tok_slot;        // [T * 8]
  int4* mtiles;         // m-tile table
};

// Pointers into the caller's workspace produced by routing + permutation.
struct Plan {
  const int* expert_offsets;  // [E_local + 1]
  const int* perm_token;      // [Pmax]
  const float* perm_w;        // [Pmax]
  const int* tok_slot;        // [T * 8]
  const int* active;          // [E_local]
  const int* mtile_offsets;   // [E_local + 1]
  const int* info;            // {P, n_active, GEMM1 m-blocks|m-tiles, S1, S2, GEMM2 m-blocks, m-tiles}
  const int4* mtiles;         // small T: per m-tile {expert, first pair, rows, OR of pair flags}
  const int4* mblocks;        // large T, both GEMMs: m-blocks {expert, first row, rows, flags}, expert by
                              // expert: its class 0 and 1 rows together (two-term C where a block
                              // holds class 1 rows), then its exact-product rows; info[2] (= info[5])
                              // blocks in all
  const int2* mbgroup;        // large T: per m-block {first m-block of its expert, the expert's m-blocks}
  int* queues;                // large T: per-XCD unit queues of GEMM1 (0..7) and GEMM2 (8..15), kQueueStride apart
  const int* canon_token;     // token of each pair in canonical (expert, token) order
  int* counters;              // small T: arrivals per (m-tile, 128 C columns), zeroed by the routing
  int* counters2;             // small T: arrivals per 64 output columns, zeroed by the routing
                              // (small-T counters and flags: kCounterStride ints apart)
  const float* esig;          // [E, 2] W13 and W2 entry scale estimates of each local expert (routing)
  int* two_term;              // GEMM2's precision flags from measured C (needs_two_terms): per m-tile
                              // at small T (zeroed by the routing, set by GEMM1), per m-block at large T
                              // (written by the flags launch between the GEMMs)
  const void* shared;         // optional [T, H] rows added before the bf16 rounding (NULL: none)
  int shared_dt;              // 0 fp32, 1 bf16
  int out_f32;                // output in fp32 (the sum before its bf16 rounding) instead of bf16
  int pair_rows;              // pair rows the workspace holds (perm_token, C, O): pair indices read
                              // from the tables are clamped below it where they become addresses
  // 128-row path, GEMM2's own row table (built by the g2 plan launch from the C GEMM1 wrote): per
  // expert its one-term rows, then its two-term rows (GEMM2 takes them in blocks of up to 128)
  const int* g2_pair;         // [Pmax] GEMM2 row -> pair row
  int* g2_ctl;                // [2 E_local] one- / two-term row counts per expert (zeroed by the
                              // permutation)
  const int* xrow;            // [E_local] first exact-product row of each local expert (permutation)
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

// Small-T path: GEMM1 partials (+ SwiGLU into f16 hi/lo C by the last unit of each group)
// -> GEMM2 partials (+ the combine into the bf16 output by the last unit of each column block).
struct CHalf {
  _Float16* hi;   // [Pmax][I]
  _Float16* lo;   // [Pmax][I]
  float* scale;   // [Pmax][I/128]
};
int decode_grid1();
int decode_grid2();
int decode_unit_groups();
void launch_gemm1_decode(const Problem& pb, const Plan& pl, const DecodePlanArgs& da, float* gbuf, const CHalf& ch,
                         hipStream_t stream);
void launch_gemm2_decode(const Problem& pb, const Plan& pl, const CHalf& ch, float* obuf, void* out,
                        hipStream_t stream);

constexpr int kUnitQueues = 24;   // GEMM1 (0..7), GEMM2 by output-column pass (8..15, 16..23)
constexpr int kQueueStride = 64;   // ints between queue counters: one 256-byte line each
// Small-T arrival counters and GEMM2 precision flags sit kCounterStride ints apart (one 128-byte
// line each): device-scope atomics from many workgroups on one line serialise (measured at T = 1:
// GEMM1 29 -> 18 us with 80 arrivals on each of 16 counters of one line).
constexpr int kCounterStride = 32;

// Large-T path (T > 64).  Permutation arguments: pair counts per (block of 256 tokens,
// bucket = local expert x magnitude class) and the outputs of its two launches.
struct LargePermArgs {
  const int* topk_ids;
  const float* topk_w;
  const float* tok_a2;
  const float* esig;
  int T, E_local, offset;
  float sqrt_i;
  int nblk;
  int* bcnt;            // [nblk][E_local * 3] pairs per block and bucket
  int* expert_offsets;  // [E_local + 1]
  int* mtile_offsets;   // [E_local + 1]
  int* active;          // [E_local]
  int* info;
  int* perm_token;      // [Pmax] internal row order (class-grouped inside each expert)
  float* perm_w;        // [Pmax]
  int* canon_token;     // [Pmax] canonical order
  int* tok_slot;        // [T * 8] internal rows of each token's pairs, ascending expert
  int4* mblocks;        // m-blocks of both GEMMs {expert, first row, rows, flags}
  int2* mbgroup;        // per m-block: {first m-block of its expert, the expert's m-blocks}
  int* queues;          // [kUnitQueues * kQueueStride] unit queues of the grouped GEMMs, zeroed here
  int* g2_ctl;          // [2 E_local] GEMM2 row-table counters, zeroed here (NULL: none)
  int* xrow;            // [E_local] first exact-product (class 2) row of each local expert
  int mixed;            // fold <= 32 exact-product rows into the expert's last class 0/1 block
  int rows_a;           // block height over an expert's class 0 and 1 rows
  int rows_b;           // block height over its class 2 (exact-product) rows
};
void launch_permute_large(const LargePermArgs& args, hipStream_t stream);
int permute_large_blocks(int64_t T);

// C between the large-T GEMMs: hi = f16(C/s), lo16 = f16(C/s - hi), s = max |C| / 448 per
// (pair, 128 columns).  GEMM2 reads lo16 only in m-blocks flagged two_term.
struct CHalf8 {
  _Float16* hi;     // [Pmax][I]
  _Float16* lo16;   // [Pmax][I]
  float* scale;     // [Pmax][I/128]
};
int large_grid();
// GEMM1 over its blocks [0, info[2]), 16 * mt rows per block
void launch_gemm1_large(const Problem& pb, const Plan& pl, const CHalf8& ch, int mt, int max_units,
                        hipStream_t stream);
// GEMM1 over the whole table (kBigRows-row class 0/1 blocks, 32-row exact-product blocks), one
// workgroup per CU
constexpr int kBigRows = 128;
constexpr int kBigMaxKB = 64;   // H <= 8192
void launch_gemm1_big(const Problem& pb, const Plan& pl, const CHalf8& ch, int max_units, hipStream_t stream);
// GEMM2's precision flags (Plan::two_term) of the blocks [0, info[2]) from GEMM1's output
void launch_c_flags(const Plan& pl, const CHalf8& ch, int I, int max_blocks, hipStream_t stream);
// GEMM2 over the blocks [0, info[2]), taken 16 * mt rows at a time
void launch_gemm2_large(const Problem& pb, const Plan& pl, const CHalf8& ch, float* obuf, int mt, int max_units,
                        hipStream_t stream);
// GEMM2's row table for the 128-row path (Plan::g2_*): every pair whose C needs both f16 terms
// (its magnitude class, or needs_two_terms on the C scales GEMM1 wrote) goes to its expert's
// two-term blocks, the others to its one-term blocks.  Pmax bounds the launch's pair rows.
void launch_g2_plan(const Problem& pb, const Plan& pl, const CHalf8& ch, int pmax, hipStream_t stream);
// Output-column pass `pass` (0 or 1) of a call whose O buffer holds o_rows rows of H floats: with at
// most o_rows pairs, pass 0 covers all H columns (rows of H floats) and pass 1 nothing; with more,
// each pass covers half of the column blocks of 256 (rows of H / 2 floats, rounded up to 256).
struct OutPass {
  int c0, c1, ocols, rows_cap;
};
__device__ __forceinline__ OutPass out_pass(int P, int H, int o_rows, int pass, int pair_rows) {
  if (P <= o_rows) return pass == 0 ? OutPass{0, H, H, o_rows} : OutPass{H, H, H, o_rows};
  const int half = (H / 256 + 1) / 2 * 256;
  return pass == 0 ? OutPass{0, half, half, pair_rows} : OutPass{half, H, half, pair_rows};
}
// GEMM2 over its row table (Plan::g2_*), 256 output columns per unit, over the columns of output
// pass `pass` (out_pass)
void launch_gemm2_big(const Problem& pb, const Plan& pl, const CHalf8& ch, float* obuf, int max_units, int o_rows,
                      int pass, hipStream_t stream);

void launch_combine(const Plan& pl, const float* obuf, void* out, int T, int H, hipStream_t stream);
// The combine of output pass `pass` (out_pass) of the 128-row path.
void launch_combine_pass(const Plan& pl, const float* obuf, void* out, int T, int H, int o_rows, int pass,
                         hipStream_t stream);

// Per-token 1x128 e4m3 quantization of bf16 (x_dt 1) or fp32 (0) activations [T, H] into
// q [T, H] and scale [H/128, T].
void launch_quantize_hidden(const void* x, int x_dt, int64_t T, int H, uint8_t* q, float* scale, hipStream_t stream);

int num_compute_units();

}  // namespace moefp8
