// Device-side helpers shared by the gfx950 MoE kernels: operand vector types,
// the fp8 MFMA, wavefront shuffles, OCP e4m3 encode/decode and bf16 rounding.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moefp8 {

constexpr int kEGlobal = 256;
constexpr int kTopK = 8;
constexpr int kNGroup = 8;
constexpr int kTopKGroup = 4;
constexpr int kGroupSize = kEGlobal / kNGroup;
constexpr int kBlock = 128;
constexpr int kWave = 64;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

// D = A(16x128 e4m3) * B(128x16 e4m3) + C.  Lane l holds A row l%16 and B column
// l%16, 32 consecutive k of the k-group l/16 (any k order works as long as A and
// B agree).  D: lane l, element r -> row 4*(l/16)+r, column l%16.
__device__ __forceinline__ v4f mfma16x16x128(const v8i& a, const v8i& b, const v4f& c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// Exact-product path.  The fp8 MFMA sums its 128 products with a truncating
// adder (measured on gfx950: mean error 2^-19.4 of sum|products|, worst 2.4e-5),
// while the f16 MFMA sums e4m3 products (exact in f16) with fp32-exact accuracy
// (2^-32).  Sub-tiles whose outputs are large enough for the fp8 error to show
// against the operator's absolute tolerance run on the f16 MFMA: the same fp8
// operand registers are widened to f16 (e4m3 -> f16 is exact) and one 128-K
// block becomes four chained v_mfma_f32_16x16x32_f16.  k-values stay in the
// same lane/slot order, so A and B still agree on k.
__device__ __forceinline__ void widen_fp8_operand(const v8i& x, v8h (&y)[4]) {
#pragma unroll
  for (int s = 0; s < 4; s++) {
#pragma unroll
    for (int w = 0; w < 2; w++) {
      const uint32_t word = (uint32_t)x[2 * s + w];
      const v2h lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(word, 1.0f, false);
      const v2h hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(word, 1.0f, true);
      y[s][4 * w + 0] = lo[0];
      y[s][4 * w + 1] = lo[1];
      y[s][4 * w + 2] = hi[0];
      y[s][4 * w + 3] = hi[1];
    }
  }
}

__device__ __forceinline__ v4f mfma_f16_block(const v8h (&a)[4], const v8h (&b)[4], v4f c) {
#pragma unroll
  for (int s = 0; s < 4; s++) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[s], b[s], c, 0, 0, 0);
  return c;
}

// Two-term f16 split of v = x * inv (|v| <= 448): v ~ hi + lo, ~2^-22 relative.
__device__ __forceinline__ void split_f16(float x, float inv, _Float16& hi, _Float16& lo) {
  const float v = fminf(fmaxf(x * inv, -448.0f), 448.0f);
  hi = (_Float16)v;
  lo = (_Float16)(v - (float)hi);
}

// Predicted size of a pair's output row (rms of routing-weighted GEMM2 output) from
// the token's squared hidden-state norm and the expert's weight-magnitude estimates:
// rms(G1) ~ ||A|| s13, rms(C) ~ 0.7 rms(G1)^2, rms(O) ~ rms(C) s2 sqrt(I) (it over-estimates
// the measured rms ~7x).  Used before GEMM1, where only the inputs are known: pairs above
// kPreciseRms take GEMM1's exact-product path (the fp8 MFMA's adder error is relative to
// sum |a w|, which this estimate tracks), and pairs above kOneTermRms are grouped together inside
// their expert and take two terms of C in GEMM2 (kFlagTwoTermC) on the small-T and grouped paths
// (the 128-row path decides each row's terms from its measured C alone, g2_plan_kernel).
constexpr float kPreciseRms = 96.0f;
constexpr float kOneTermRms = 8.0f;
constexpr uint8_t kFlagExactProducts = 1;
constexpr uint8_t kFlagTwoTermC = 2;
// Large-T m-block flags only: the block also holds its expert's <= 32 exact-product rows, their
// count in the bits from kMixedShift up.
constexpr int kFlagMixed = 4;
constexpr int kMixedShift = 8;

// GEMM2's precision of C, also checked on C itself, so that inputs the estimate above misjudges
// (hidden rows aligned with an expert's W13 rows, where G1 is ~sqrt(H) times the estimate) still
// get two terms.  GEMM1 knows, per pair and 128-column block cb, amax_cb = max |C| over the block
// (it scales C's split by it); the test is
//   q = |w| * sigma2 * sqrt(I) * amax_cb > kOneTermQ,
// sigma2 the expert's W2 entry scale (448 * largest block scale / 3).  Since
// ||C||_2^2 <= sum_cb 128 amax_cb^2 <= I max_cb amax_cb^2, the largest q over the blocks bounds
// |w| ||C||_2 sigma2, the rms of the pair's routing-weighted output row for W2 entries of rms
// sigma2.  C's f16 hi term rounds each element by at most 2^-11 relative (a block's largest
// element, scaled to 448, exactly), so one term leaves an output error of rms at most
// 2^-11 / sqrt(3) * q (C flat across its elements); on the lognormal T = 8192 benchmark
// workload the one-term error of a pair measures at most 2.1e-5 * q in rms and 9.1e-5 * q at its
// worst column.  There every pair the estimate keeps at one term has q <= 37 (99% <= 23), so
// kOneTermQ sits above them: the measured test only adds two-term blocks where the estimate
// fails.  An m-block (m-tile at small T) holding a pair with q > kOneTermQ takes C's f16 lo term
// (22 significant bits in all); the flag is set, never cleared, by whichever unit finds such a
// pair, so it does not depend on the order in which units finish.
constexpr float kOneTermQ = 32.0f;

__device__ __forceinline__ bool needs_two_terms(float w, float sigma2, float amax, float sqrt_i) {
  return fabsf(w) * sigma2 * sqrt_i * amax > kOneTermQ;
}

__device__ __forceinline__ float predicted_output_rms(float a2, float w, float s13, float s2, float sqrt_i) {
  return fabsf(w) * 0.7f * a2 * s13 * s13 * s2 * sqrt_i;
}

__device__ __forceinline__ bool needs_exact_products(float a2, float w, float s13, float s2, float sqrt_i) {
  return predicted_output_rms(a2, w, s13, s2, sqrt_i) > kPreciseRms;
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

// An index read from the permutation tables (a token, or a pair row), clamped to [0, n) where it
// becomes a load or DMA address (one VALU op; negative values clamp to n - 1): a wrong table
// entry then shows as a parity failure instead of a memory fault.
__device__ __forceinline__ int clamp_index(int i, int n) { return (int)min((uint32_t)i, (uint32_t)(n - 1)); }

// LDS slot swizzles of 16-byte chunks: chunk c of row r sits in slot c ^ key(r).  The keys are
// linear in the row bits and were chosen so that the MFMA operand reads (lanes = 16 rows x chunk
// groups) and the row-order writes of the stages below are conflict-free whether the LDS serves
// a 16-byte access 8, 16 or 32 lanes at a time (over 128, 256 or 512 bytes of banks).
// 128-byte rows (8 slots):
__device__ __forceinline__ int slot_key8(int row) { return (row & 7) ^ ((row >> 3) & 1); }
// 256-byte rows (16 slots):
__device__ __forceinline__ int slot_key16(int row) { return (row & 11) ^ (((row >> 2) & 1) * 5); }

// A value the caller knows to be equal on every lane, moved to a scalar register.
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }
// Wavefront index inside the workgroup, as a wave-uniform (scalar) value.
__device__ __forceinline__ int wave_index() { return __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)); }

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, kWave); }
__device__ __forceinline__ int shfl_xor_i(int v, int m) { return __shfl_xor(v, m, kWave); }
__device__ __forceinline__ float shfl_f(float v, int src) { return __shfl(v, src, kWave); }
__device__ __forceinline__ int shfl_i(int v, int src) { return __shfl(v, src, kWave); }

// Cross-lane moves inside a row of 16 lanes through DPP (no LDS round trip).
// quad_perm [1,0,3,2] and [2,3,0,1] pair lanes at distance 1 and 2; the half-row
// mirror pairs lane i with 7-i and the row mirror i with 15-i.
constexpr int kDppXor1 = 0xB1;
constexpr int kDppXor2 = 0x4E;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, kCtrl, 0xF, 0xF, false);
}
template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), kCtrl, 0xF, 0xF, false));
}

__device__ __forceinline__ uint32_t readlane_u32(uint32_t v, int lane) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, lane);
}
__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Largest value over the wavefront (uniform result).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, dpp_u32<kDppXor1>(v));
  v = max(v, dpp_u32<kDppXor2>(v));
  v = max(v, dpp_u32<kDppHalfMirror>(v));
  v = max(v, dpp_u32<kDppRowMirror>(v));
  return max(max(readlane_u32(v, 0), readlane_u32(v, 16)), max(readlane_u32(v, 32), readlane_u32(v, 48)));
}
__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, dpp_f32<kDppXor1>(v));
  v = fmaxf(v, dpp_f32<kDppXor2>(v));
  v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f32<kDppRowMirror>(v));
  return fmaxf(fmaxf(readlane_f32(v, 0), readlane_f32(v, 16)), fmaxf(readlane_f32(v, 32), readlane_f32(v, 48)));
}

// Sum over the wavefront (uniform result; fixed summation order).
__device__ __forceinline__ float wave_sum_f32(float v) {
  v += dpp_f32<kDppXor1>(v);
  v += dpp_f32<kDppXor2>(v);
  v += dpp_f32<kDppHalfMirror>(v);
  v += dpp_f32<kDppRowMirror>(v);
  return (readlane_f32(v, 0) + readlane_f32(v, 16)) + (readlane_f32(v, 32) + readlane_f32(v, 48));
}

// Exclusive prefix sum over the wavefront (Hillis-Steele on shuffles).
__device__ __forceinline__ int wave_exclusive_sum(int v) {
  const int lane = lane_id();
  int x = v;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) {
    const int y = __shfl_up(x, off, kWave);
    if (lane >= off) x += y;
  }
  return x - v;
}

// Number of set bits of m in lanes below this one.
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// Order-preserving map of a float onto uint32 (larger float -> larger key; -0 == +0).
// 0 is never produced for a non-NaN input, so it can mark "no candidate".
__device__ __forceinline__ uint32_t order_key(float v) {
  const uint32_t u = __float_as_uint(v + 0.0f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// OCP e4m3fn byte -> fp32 (exact; v_cvt_f32_fp8).
__device__ __forceinline__ float e4m3_to_f32(uint32_t byte) {
  return __builtin_amdgcn_cvt_f32_fp8((int)byte, 0);
}

// fp32 -> OCP e4m3fn, round to nearest even; |x| must be <= 448 (callers clamp).
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(x, 0.0f, 0, false) & 0xffu;
}

// Per-block scale of the split: amax -> (inv = 448/amax, scale = amax/448).
__device__ __forceinline__ void split_scale(float amax, float& inv, float& scale) {
  if (amax > 0.0f) {
    inv = __fdiv_rn(448.0f, amax);
    scale = __fdiv_rn(amax, 448.0f);
  } else {
    inv = 0.0f;
    scale = 0.0f;
  }
}

// fp32 -> bf16 bits, round to nearest even (NaN -> quiet NaN), as torch's .to(bfloat16).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Stores output elements i .. i + 3 (i a multiple of 4): rounded to bf16 (nearest even), or
// as fp32 when out_f32.
__device__ __forceinline__ void store_out4(void* out, size_t i, float4 v, int out_f32) {
  if (out_f32) {
    *reinterpret_cast<float4*>(static_cast<float*>(out) + i) = v;
    return;
  }
  uint2 o;
  o.x = (uint32_t)f32_to_bf16_rne(v.x) | ((uint32_t)f32_to_bf16_rne(v.y) << 16);
  o.y = (uint32_t)f32_to_bf16_rne(v.z) | ((uint32_t)f32_to_bf16_rne(v.w) << 16);
  *reinterpret_cast<uint2*>(static_cast<uint16_t*>(out) + i) = o;
}

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(((uint32_t)b) << 16); }

__device__ __forceinline__ float half_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// Load element i of a routing input of dtype code dt (0 f32, 1 bf16, 2 f16) as fp32.
__device__ __forceinline__ float load_as_f32(const void* p, int dt, int64_t i) {
  if (dt == 0) return reinterpret_cast<const float*>(p)[i];
  uint16_t h = reinterpret_cast<const uint16_t*>(p)[i];
  return dt == 1 ? bf16_to_f32(h) : half_to_f32(h);
}

// acc += the 4 consecutive elements [i, i + 4) of a shared row of dtype dt (0 f32, 1 bf16),
// the last term of a token's combine.
__device__ __forceinline__ void add_shared4(float4& acc, const void* shared, int dt, size_t i) {
  if (dt == 0) {
    const float4 v = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(shared) + i);
    acc.x += v.x;
    acc.y += v.y;
    acc.z += v.z;
    acc.w += v.w;
  } else {
    const uint2 v = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint16_t*>(shared) + i);
    acc.x += __uint_as_float(v.x << 16);
    acc.y += __uint_as_float(v.x & 0xffff0000u);
    acc.z += __uint_as_float(v.y << 16);
    acc.w += __uint_as_float(v.y & 0xffff0000u);
  }
}

__device__ __forceinline__ float silu_f32(float x) {
  return __fdiv_rn(x, 1.0f + __expf(-x));
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)p; }

// DMA and its completion wait as inline asm, for kernels whose LDS operand reads are ordinary
// loads: the compiler then neither knows of the DMAs nor drains them before every LDS read, and
// schedules the reads with exact lgkmcnt waits.  The writer of M0 must precede the DMA by one
// wait state.
__device__ __forceinline__ void dma_lds16(const void* g, uint32_t lds_uniform) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "s"(lds_uniform)
               : "memory", "m0");
}
__device__ __forceinline__ void dma_lds4(const void* g, uint32_t lds_uniform) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dword %0, off" : : "v"(g), "s"(lds_uniform)
               : "memory", "m0");
}
// The same with a wave-uniform 64-bit base in SGPRs and a 32-bit per-lane byte offset.
__device__ __forceinline__ void dma_lds16_s(uint32_t voff, const void* sbase, uint32_t lds_uniform) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" : : "v"(voff), "s"(sbase),
               "s"(lds_uniform) : "memory", "m0");
}
// The same with the non-temporal hint (streamed through L2), for lines read once per call.
__device__ __forceinline__ void dma_lds16_s_nt(uint32_t voff, const void* sbase, uint32_t lds_uniform) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" : : "v"(voff), "s"(sbase),
               "s"(lds_uniform) : "memory", "m0");
}
__device__ __forceinline__ void dma_lds4_s(uint32_t voff, const void* sbase, uint32_t lds_uniform) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" : : "v"(voff), "s"(sbase),
               "s"(lds_uniform) : "memory", "m0");
}

}  // namespace moefp8
