// Combine (main.py:241-243): each token's pair rows, summed in ascending expert order
// starting from zero (the order of index_add_ in the reference), rounded once to bf16.
// Tokens without a local expert get exact zero rows.  Pair rows may come split over K
// (small-T GEMM2); the splits of a pair are added first, in ascending order.  An optional
// shared row (the shared expert's output) is added last, before the rounding.
#include "moefp8_device.h"
#include "moefp8_launch.h"

namespace moefp8 {

// Workgroup = (token, 512 columns), 4 columns per thread (measured at T = 8192: 65 µs, against 67
// with 1024 columns, 72 with 256, and 81 with 4 tokens x 1024 columns of 16 per lane).
constexpr int kCombineCols = 512;
constexpr int kCombineThreads = kCombineCols / 4;
// Workgroups of the second output pass, which has nothing to do unless the call's pairs outnumber
// its O rows.
constexpr int kCombineSpareGrid = 256;

// Token t's pair rows (tok_slot: ascending local expert, -1 past the last).
__device__ __forceinline__ void load_slots(const int* __restrict__ tok_slot, int t, int (&slots)[kTopK]) {
#pragma unroll
  for (int k = 0; k < kTopK; k++) slots[k] = tok_slot[(size_t)t * kTopK + k];
}

// Token t's output columns [c, c + 4) (c inside [op.c0, op.c1)), from O rows [op.rows_cap][op.ocols]
// holding the pass's columns from column 0.
__device__ __forceinline__ void combine_quad(const int (&slots)[kTopK], const float* __restrict__ obuf,
                                             void* __restrict__ out, int t, int c, int H, int S, const OutPass& op,
                                             const void* shared, int shared_dt, int out_f32) {
  const int oc = c - op.c0;
  float4 acc = {0.f, 0.f, 0.f, 0.f};
  if (S == 1) {
    // O is read once, each row by whole lines (a wavefront's 64 lanes load 1 KB of it), so the loads
    // carry the non-temporal hint (streamed through L2): 67.7 -> 61.5 us at T = 8192, measured
    v4f v[kTopK];
#pragma unroll
    for (int k = 0; k < kTopK; k++)
      v[k] = slots[k] >= 0 ? __builtin_nontemporal_load(reinterpret_cast<const v4f*>(
                                 obuf + (size_t)clamp_index(slots[k], op.rows_cap) * op.ocols + oc))
                           : v4f{0.f, 0.f, 0.f, 0.f};
    // every row's load issued before the first add (without this the compiler adds row 0 inside its
    // load's branch and waits for it there, a second round trip for a token with several rows)
    asm volatile("" : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7]));
    // slots past the token's last add +0.0, which changes no bit of a sum that starts at +0.0 (it is
    // never -0.0)
#pragma unroll
    for (int k = 0; k < kTopK; k++) {
      const bool on = slots[k] >= 0;
      acc.x += on ? v[k][0] : 0.f;
      acc.y += on ? v[k][1] : 0.f;
      acc.z += on ? v[k][2] : 0.f;
      acc.w += on ? v[k][3] : 0.f;
    }
  } else {
    // K-split partials of each pair row, added split by split, then pair by pair
    for (int k = 0; k < kTopK; k++) {
      if (slots[k] < 0) break;
      const float* row = obuf + (size_t)clamp_index(slots[k], op.rows_cap) * S * op.ocols + oc;
      float4 o = *reinterpret_cast<const float4*>(row);
      for (int s = 1; s < S; s++) {
        const float4 v = *reinterpret_cast<const float4*>(row + (size_t)s * op.ocols);
        o.x += v.x;
        o.y += v.y;
        o.z += v.z;
        o.w += v.w;
      }
      acc.x += o.x;
      acc.y += o.y;
      acc.z += o.z;
      acc.w += o.w;
    }
  }
  if (shared) add_shared4(acc, shared, shared_dt, (size_t)t * H + c);
  store_out4(out, (size_t)t * H + c, acc, out_f32);
}

// Workgroup (token blockIdx.x, 512 columns blockIdx.y from the pass's first column): with pass < 0
// all H columns from O rows [pair_rows][H], else the columns of output pass `pass` (out_pass).
__global__ __launch_bounds__(kCombineThreads) void combine_kernel(const int* __restrict__ tok_slot,
                                                      const int* __restrict__ info,
                                                      const float* __restrict__ obuf,
                                                      void* __restrict__ out, int H, int o_rows, int pass,
                                                      const void* shared, int shared_dt, int out_f32,
                                                      int pair_rows) {
  // the token's slots with the pair count and K-split, one round of loads (the slots do not depend
  // on the pass)
  int slots[kTopK];
  load_slots(tok_slot, blockIdx.x, slots);
  const int P = info[0], S = info[4];
  asm volatile("" ::"s"(slots[0]), "s"(slots[1]), "s"(slots[2]), "s"(slots[3]), "s"(slots[4]), "s"(slots[5]),
               "s"(slots[6]), "s"(slots[7]), "s"(P), "s"(S));
  OutPass op{0, H, H, pair_rows};
  if (pass >= 0) op = out_pass(P, H, o_rows, pass, pair_rows);
  const int c = op.c0 + blockIdx.y * kCombineCols + 4 * threadIdx.x;
  if (c >= op.c1) return;
  combine_quad(slots, obuf, out, blockIdx.x, c, H, S, op, shared, shared_dt, out_f32);
}

// The same over a fixed grid (items (token, 512 columns), tokens fastest), for an output pass that
// has columns only when the call's pairs outnumber O's rows: its workgroups exit at once otherwise.
__global__ __launch_bounds__(kCombineThreads) void combine_spare_kernel(const int* __restrict__ tok_slot,
                                                            const int* __restrict__ info,
                                                            const float* __restrict__ obuf,
                                                            void* __restrict__ out, int T, int H, int o_rows,
                                                            int pass, const void* shared, int shared_dt,
                                                            int out_f32, int pair_rows) {
  const OutPass op = out_pass(info[0], H, o_rows, pass, pair_rows);
  const int n_chunks = (op.c1 - op.c0 + kCombineCols - 1) / kCombineCols, S = info[4];
  for (int64_t item = blockIdx.x; item < (int64_t)T * n_chunks; item += gridDim.x) {
    const int t = (int)(item % T), chunk = (int)(item / T);
    const int c = op.c0 + chunk * kCombineCols + 4 * threadIdx.x;
    if (c < op.c1) {
      int slots[kTopK];
      load_slots(tok_slot, t, slots);
      combine_quad(slots, obuf, out, t, c, H, S, op, shared, shared_dt, out_f32);
    }
  }
}

void launch_combine(const Plan& pl, const float* obuf, void* out, int T, int H, hipStream_t stream) {
  if (T <= 0) return;
  hipLaunchKernelGGL(combine_kernel, dim3(T, (H + kCombineCols - 1) / kCombineCols), dim3(kCombineThreads), 0, stream,
                     pl.tok_slot, pl.info, obuf, out, H, 0, -1, pl.shared, pl.shared_dt, pl.out_f32, pl.pair_rows);
}

// Pass 0 (the single pass of nearly every call) takes one workgroup per (token, 512 columns) of
// all H columns; pass 1 a fixed grid that exits at once unless the call's pairs outnumber O's rows.
void launch_combine_pass(const Plan& pl, const float* obuf, void* out, int T, int H, int o_rows, int pass,
                         hipStream_t stream) {
  if (T <= 0) return;
  if (pass == 0) {
    hipLaunchKernelGGL(combine_kernel, dim3(T, (H + kCombineCols - 1) / kCombineCols), dim3(kCombineThreads), 0,
                       stream, pl.tok_slot, pl.info, obuf, out, H, o_rows, 0, pl.shared, pl.shared_dt, pl.out_f32,
                       pl.pair_rows);
  } else {
    hipLaunchKernelGGL(combine_spare_kernel, dim3(kCombineSpareGrid), dim3(kCombineThreads), 0, stream, pl.tok_slot,
                       pl.info, obuf, out, T, H, o_rows, pass, pl.shared, pl.shared_dt, pl.out_f32, pl.pair_rows);
  }
}

}  // namespace moefp8
