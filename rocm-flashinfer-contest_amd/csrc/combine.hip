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

__global__ __launch_bounds__(kCombineThreads) void combine_kernel(const int* __restrict__ tok_slot,
                                                      const int* __restrict__ info,
                                                      const float* __restrict__ obuf,
                                                      void* __restrict__ out, int H, const void* shared,
                                                      int shared_dt, int out_f32, int pair_rows) {
  const int t = blockIdx.x;
  const int c = blockIdx.y * kCombineCols + 4 * threadIdx.x;
  const int S = info[4];
  int slots[kTopK];
#pragma unroll
  for (int k = 0; k < kTopK; k++) slots[k] = tok_slot[(size_t)t * kTopK + k];
  if (c >= H) return;
  float4 acc = {0.f, 0.f, 0.f, 0.f};
  if (S == 1) {
    float4 v[kTopK];
#pragma unroll
    for (int k = 0; k < kTopK; k++)
      v[k] = slots[k] >= 0 ? *reinterpret_cast<const float4*>(obuf + (size_t)clamp_index(slots[k], pair_rows) * H + c)
                           : float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < kTopK; k++) {
      if (slots[k] < 0) break;
      acc.x += v[k].x;
      acc.y += v[k].y;
      acc.z += v[k].z;
      acc.w += v[k].w;
    }
  } else {
    // K-split partials of each pair row, added split by split, then pair by pair
    for (int k = 0; k < kTopK; k++) {
      if (slots[k] < 0) break;
      const float* row = obuf + (size_t)clamp_index(slots[k], pair_rows) * S * H + c;
      float4 o = *reinterpret_cast<const float4*>(row);
      for (int s = 1; s < S; s++) {
        const float4 v = *reinterpret_cast<const float4*>(row + (size_t)s * H);
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


void launch_combine(const Plan& pl, const float* obuf, void* out, int T, int H, hipStream_t stream) {
  if (T <= 0) return;
  hipLaunchKernelGGL(combine_kernel, dim3(T, (H + kCombineCols - 1) / kCombineCols), dim3(kCombineThreads), 0, stream,
                     pl.tok_slot, pl.info, obuf, out, H, pl.shared, pl.shared_dt, pl.out_f32, pl.pair_rows);
}

}  // namespace moefp8
