// Per-token 1x128 e4m3 quantization of the hidden states: the step before the operator.
//
// The operator consumes hidden_states as e4m3fn [T, H] with fp32 scales stored transposed
// [H/128, T] (A[t, h] = e4m3(hs[t, h]) * scale[h / 128, t], solutions/moe_fp8/main.py:129-136).
// This kernel produces that pair from bf16 (or fp32) activations [T, H] with the DeepSeek-V3
// per-token, per-128-column convention: scale = amax / 448 (1 when the block is all zero),
// q = e4m3(x / scale) with an IEEE fp32 division and round-to-nearest-even; inputs are
// finite.  Codes and scales are bit-exact with that arithmetic (the division is done as a
// correctly rounded reciprocal multiply with an exact-residual correction, see div_by_scale).
//
// HBM-bound (2 + 1 bytes per value for bf16 in, plus 4 / 128 for the scales).  A workgroup
// covers 8 tokens x 512 columns: each wavefront handles 2 tokens, a lane 8 consecutive values
// (one 16-byte bf16 load), so 16 lanes hold one 128-column block and its amax is a DPP
// reduction inside the 16-lane row.  The 4 x 8 block scales go through LDS so that the
// transposed [H/128, T] rows are written as 32-byte runs instead of 4-byte strided stores.
// The grid is (512-column piece, token group): consecutive workgroups take consecutive pieces
// of the same tokens, so the grid walks memory in order.  Measured at T = 8192: 32.4 us, against
// 37.3 for 16 tokens with the token group fastest; 4 or 32 tokens 36.9 / 41.3; the same order as
// a 1-D grid, whose workgroup index needs a division by the piece count, 35.6; non-temporal
// loads and loads issued ahead of their bounds checks, no gain.
#include "moefp8_device.h"
#include "moefp8_launch.h"

namespace moefp8 {

constexpr int kQTokens = 8;         // tokens per workgroup
constexpr int kQRows = kQTokens / 4;  // tokens per wavefront
constexpr int kQMaxGroups = 65535;  // grid rows (token groups) per launch; more stride over them
constexpr int kQCols = 512;         // columns per workgroup (4 blocks of 128)
constexpr int kQThreads = 256;
constexpr float kMinFastScale = 0x1p-100f;   // below it, reciprocal and quotient leave the normal range

// x / s rounded to nearest, given y = 1/s rounded to nearest (Markstein): q = x y, the
// residual x - q s is exact in one fma, and q + y r rounds to the correctly rounded quotient.
// Three operations per value instead of the ~10 of a general division (the scale is shared
// by its 128 values); the sign is taken from x so that -0 and negative underflows keep it.
__device__ __forceinline__ float div_by_scale(float x, float s, float y) {
  const float q = x * y;
  const float r = __builtin_fmaf(-q, s, x);
  return __builtin_copysignf(__builtin_fmaf(r, y, q), x);
}
// 1/s rounded to nearest: hardware reciprocal (1 ulp) plus one Newton step.
__device__ __forceinline__ float recip_rn(float s) {
  const float y0 = __builtin_amdgcn_rcpf(s);
  const float e = __builtin_fmaf(-s, y0, 1.0f);
  return __builtin_fmaf(e, y0, y0);
}

// Largest value of the 16-lane row (every lane of the row gets it).
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f32<kDppXor1>(v));
  v = fmaxf(v, dpp_f32<kDppXor2>(v));
  v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f32<kDppRowMirror>(v));
  return v;
}

// 8 consecutive input values as fp32 (bf16: one 16-byte load; fp32: two)
template <int kDt>
__device__ __forceinline__ void load8(const void* x, size_t i, float (&v)[8]) {
  if constexpr (kDt == 1) {
    const v4i w = *reinterpret_cast<const v4i*>(reinterpret_cast<const uint16_t*>(x) + i);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      v[2 * j] = __uint_as_float((uint32_t)w[j] << 16);
      v[2 * j + 1] = __uint_as_float((uint32_t)w[j] & 0xffff0000u);
    }
  } else {
    const float4 a = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(x) + i);
    const float4 b = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(x) + i + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
}

template <int kDt>
__global__ __launch_bounds__(kQThreads) void quantize_hidden_kernel(const void* __restrict__ x, int T, int H,
                                                                    uint8_t* __restrict__ q,
                                                                    float* __restrict__ scale) {
  __shared__ float sc_s[kQCols / kBlock][kQTokens];
  const int wave = threadIdx.x >> 6, lane = lane_id();
  const int c0 = blockIdx.x * kQCols;
  const int col = c0 + 8 * lane;                 // this lane's 8 columns
  const bool in_cols = col < H;                  // H is a multiple of 128: whole 16-lane rows
  for (int t0 = blockIdx.y * kQTokens; t0 < T; t0 += gridDim.y * kQTokens) {
    float v[kQRows][8];
#pragma unroll
    for (int r = 0; r < kQRows; r++) {
      const int t = t0 + kQRows * wave + r;
      if (t < T && in_cols) load8<kDt>(x, (size_t)t * H + col, v[r]);
      else
#pragma unroll
        for (int j = 0; j < 8; j++) v[r][j] = 0.f;
    }
#pragma unroll
    for (int r = 0; r < kQRows; r++) {
      const int t = t0 + kQRows * wave + r;
      float a = 0.f;
#pragma unroll
      for (int j = 0; j < 8; j++) a = fmaxf(a, fabsf(v[r][j]));
      const float amax = row16_max(a);
      const float s = amax > 0.f ? amax / 448.0f : 1.0f;
      uint32_t lo = 0, hi = 0;
      if (s >= kMinFastScale) {
        const float y = recip_rn(s);
#pragma unroll
        for (int j = 0; j < 4; j++) {
          lo |= f32_to_e4m3(div_by_scale(v[r][j], s, y)) << (8 * j);
          hi |= f32_to_e4m3(div_by_scale(v[r][4 + j], s, y)) << (8 * j);
        }
      } else {
        // scales near the bottom of the fp32 range (1/s would overflow): IEEE division
#pragma unroll
        for (int j = 0; j < 4; j++) {
          lo |= f32_to_e4m3(v[r][j] / s) << (8 * j);
          hi |= f32_to_e4m3(v[r][4 + j] / s) << (8 * j);
        }
      }
      if (t < T && in_cols) *reinterpret_cast<uint2*>(q + (size_t)t * H + col) = uint2{lo, hi};
      if ((lane & 15) == 0) sc_s[lane >> 4][kQRows * wave + r] = s;
    }
    __syncthreads();
    // scale rows: 4 blocks x 8 consecutive tokens
    if (threadIdx.x < (kQCols / kBlock) * kQTokens) {
      const int b = threadIdx.x / kQTokens, i = threadIdx.x % kQTokens;
      const int kbw = c0 / kBlock + b, t = t0 + i;
      if (t < T && kbw < H / kBlock) scale[(size_t)kbw * T + t] = sc_s[b][i];
    }
    // the scales are read before the next group writes them
    __syncthreads();
  }
}

void launch_quantize_hidden(const void* x, int x_dt, int64_t T, int H, uint8_t* q, float* scale, hipStream_t stream) {
  if (T <= 0) return;
  const int64_t groups = (T + kQTokens - 1) / kQTokens;
  const dim3 grid((unsigned)((H + kQCols - 1) / kQCols), (unsigned)(groups < kQMaxGroups ? groups : kQMaxGroups));
  if (x_dt == 1)
    hipLaunchKernelGGL(quantize_hidden_kernel<1>, grid, dim3(kQThreads), 0, stream, x, (int)T, H, q, scale);
  else
    hipLaunchKernelGGL(quantize_hidden_kernel<0>, grid, dim3(kQThreads), 0, stream, x, (int)T, H, q, scale);
}

}  // namespace moefp8
