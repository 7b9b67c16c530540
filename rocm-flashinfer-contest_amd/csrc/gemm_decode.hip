// Small-T expert GEMMs: weight streaming on fp8 MFMA (v_mfma_f32_16x16x128_f8f6f4).
//
// With a few tokens per expert the work is reading each active expert's weights
// once (HBM bound).  Every workgroup owns one (active expert, column slice) and
// its waves split K, so even one active expert spreads over hundreds of
// wavefronts.  Weights and activations go straight from global memory into the
// MFMA operand registers; the only LDS use is the fixed-order cross-wave sum.
//
// GEMM1  G1 = A_e W13_e^T, C = silu(G1[:, I:]) * G1[:, :I]   (main.py:229-233), C in fp32.
// GEMM2  O = C W2_e^T times the pair's routing weight, summed per token in ascending
//        expert order and written as bf16 (main.py:234-243); see gemm2_decode_kernel.
#include "moefp8_device.h"
#include "moefp8_launch.h"

namespace moefp8 {

constexpr int kDecWaves = 8;             // waves per workgroup (split K)
constexpr int kDec1Cols = 32;            // C columns per GEMM1 workgroup (32 up + 32 gate rows of W13)
constexpr int kDec1Unroll = 2;           // GEMM1 K blocks in flight per wave

__device__ __forceinline__ v8i load_v8i(const uint8_t* p) {
  const v4i* q = reinterpret_cast<const v4i*>(p);
  const v4i x = q[0], y = q[1];
  return __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7);
}

__global__ __launch_bounds__(64 * kDecWaves) void gemm1_decode_kernel(Problem pb, Plan pl,
                                                                      float* __restrict__ cbuf) {
  const int slot = blockIdx.y;
  if (slot >= pl.info[1]) return;
  const int e = pl.active[slot];
  const int row0 = pl.expert_offsets[e];
  const int M = pl.expert_offsets[e + 1] - row0;
  const int H = pb.H, I = pb.I, T = pb.T;
  const int KB = H / kBlock;
  const int c0 = blockIdx.x * kDec1Cols;
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int lr = lane & 15, kg = lane >> 4;

  // B rows: subtiles 0,1 = up rows c0+16j+lr, subtiles 2,3 = gate rows I+c0+16(j-2)+lr
  const uint8_t* wexp = pb.w13 + (size_t)e * 2 * I * H;
  const uint8_t* brow[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int n = (j < 2 ? c0 + 16 * j : I + c0 + 16 * (j - 2)) + lr;
    brow[j] = wexp + (size_t)n * H + kg * 32;
  }
  const float* s_up = pb.s13 + ((size_t)e * (2 * I / kBlock) + c0 / kBlock) * KB;
  const float* s_gate = pb.s13 + ((size_t)e * (2 * I / kBlock) + (I + c0) / kBlock) * KB;

  __shared__ float red[kDecWaves][4][4][64];

  for (int m0 = 0; m0 < M; m0 += 16) {
    const int ar = m0 + lr;
    const bool a_ok = ar < M;
    const uint8_t* arow = pb.hidden + (size_t)pl.perm_token[row0 + (a_ok ? ar : 0)] * H + kg * 32;
    int tok_d[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int dr = m0 + kg * 4 + r;
      tok_d[r] = pl.perm_token[row0 + (dr < M ? dr : 0)];
    }
    // exact-product sub-tile if any of its 16 pairs is flagged
    const bool exact = __ballot(lane < 16 && a_ok && pl.exact[row0 + ar]) != 0;
    v4f acc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};

    for (int kb0 = wave; kb0 < KB; kb0 += kDecWaves * kDec1Unroll) {
      v8i a[kDec1Unroll], b[kDec1Unroll][4];
      float sa[kDec1Unroll][4], su[kDec1Unroll], sg[kDec1Unroll];
#pragma unroll
      for (int u = 0; u < kDec1Unroll; u++) {
        const int kb = kb0 + u * kDecWaves;
        if (kb < KB) {
          a[u] = a_ok ? load_v8i(arow + kb * kBlock) : v8i{0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
          for (int j = 0; j < 4; j++) b[u][j] = load_v8i(brow[j] + kb * kBlock);
#pragma unroll
          for (int r = 0; r < 4; r++) sa[u][r] = pb.hscale[(size_t)kb * T + tok_d[r]];
          su[u] = s_up[kb];
          sg[u] = s_gate[kb];
        }
      }
#pragma unroll
      for (int u = 0; u < kDec1Unroll; u++) {
        const int kb = kb0 + u * kDecWaves;
        if (kb < KB) {
          v8h a16[4];
          if (exact) widen_fp8_operand(a[u], a16);
#pragma unroll
          for (int j = 0; j < 4; j++) {
            v4f p;
            if (exact) {
              v8h b16[4];
              widen_fp8_operand(b[u][j], b16);
              p = mfma_f16_block(a16, b16, v4f{0.f, 0.f, 0.f, 0.f});
            } else {
              p = mfma16x16x128(a[u], b[u][j], v4f{0.f, 0.f, 0.f, 0.f});
            }
            const float sw = j < 2 ? su[u] : sg[u];
#pragma unroll
            for (int r = 0; r < 4; r++) acc[j][r] += p[r] * (sa[u][r] * sw);
          }
        }
      }
    }

#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) red[wave][j][r][lane] = acc[j][r];
    __syncthreads();
    // 16 rows x 32 C columns; thread -> (lane', half q, r)
    for (int idx = threadIdx.x; idx < 16 * kDec1Cols; idx += 64 * kDecWaves) {
      const int ln = idx & 63, q = (idx >> 6) & 1, r = idx >> 7;
      float up = 0.f, gate = 0.f;
#pragma unroll
      for (int w = 0; w < kDecWaves; w++) {
        up += red[w][q][r][ln];
        gate += red[w][q + 2][r][ln];
      }
      const int row = m0 + (ln >> 4) * 4 + r;
      if (row < M) cbuf[(size_t)(row0 + row) * I + c0 + q * 16 + (ln & 15)] = silu_f32(gate) * up;
    }
    __syncthreads();
  }
}

// GEMM2 for small T (main.py:234-241).  Workgroup = (active expert, 64 H
// columns); its 8 waves split K and a fixed-order LDS sum gives O for each of the expert's
// pairs, stored routing-weighted in fp32.  C (fp32 from GEMM1) is split on load into two f16
// terms per 128-block with one fp32 scale and multiplied with W2 widened to f16: exact
// products, ~2^-22 relative error on C.  The combine kernel then sums each token's pair rows.
__global__ __launch_bounds__(64 * kDecWaves) void gemm2_decode_kernel(Problem pb, Plan pl,
                                                                              const float* __restrict__ cbuf,
                                                                              float* __restrict__ obuf) {
  const int slot = blockIdx.y;
  const int n_act = pl.info[1];
  const int H = pb.H, I = pb.I, T = pb.T;
  const int h0 = blockIdx.x * kDec2Cols;
  if (slot >= n_act) return;
  const int e = pl.active[slot];
  const int row0 = pl.expert_offsets[e];
  const int M = pl.expert_offsets[e + 1] - row0;
  const int KB = I / kBlock;
  const int HB = H / kBlock;
  const int lane = lane_id(), wave = threadIdx.x >> 6;
  const int lr = lane & 15, kg = lane >> 4;

  const uint8_t* wexp = pb.w2 + (size_t)e * H * I;
  const uint8_t* brow[4];
#pragma unroll
  for (int j = 0; j < 4; j++) brow[j] = wexp + (size_t)(h0 + 16 * j + lr) * I + kg * 32;
  const float* s_row = pb.s2 + ((size_t)e * HB + h0 / kBlock) * KB;

  __shared__ float red[kDecWaves][4][4][64];

  for (int m0 = 0; m0 < M; m0 += 16) {
    const int ar = m0 + lr;
    const bool a_ok = ar < M;
    const float* crow = cbuf + (size_t)(row0 + (a_ok ? ar : 0)) * I + kg * 32;
    v4f acc[4];
#pragma unroll
    for (int j = 0; j < 4; j++) acc[j] = v4f{0.f, 0.f, 0.f, 0.f};

    for (int kb0 = wave; kb0 < KB; kb0 += 2 * kDecWaves) {
      v8i b[2][4];
      float cv[2][32];
      float sw[2];
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int kb = kb0 + u * kDecWaves;
        if (kb < KB) {
#pragma unroll
          for (int j = 0; j < 4; j++) b[u][j] = load_v8i(brow[j] + kb * kBlock);
          const float4* cp = reinterpret_cast<const float4*>(crow + kb * kBlock);
#pragma unroll
          for (int c4 = 0; c4 < 8; c4++) {
            const float4 v = a_ok ? cp[c4] : float4{0.f, 0.f, 0.f, 0.f};
            cv[u][4 * c4 + 0] = v.x;
            cv[u][4 * c4 + 1] = v.y;
            cv[u][4 * c4 + 2] = v.z;
            cv[u][4 * c4 + 3] = v.w;
          }
          sw[u] = s_row[kb];
        }
      }
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int kb = kb0 + u * kDecWaves;
        if (kb < KB) {
          float amax = 0.f;
#pragma unroll
          for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(cv[u][i]));
          amax = fmaxf(amax, shfl_xor_f(amax, 16));
          amax = fmaxf(amax, shfl_xor_f(amax, 32));
          float inv, scale;
          split_scale(amax, inv, scale);
          float sa[4];
#pragma unroll
          for (int r = 0; r < 4; r++) sa[r] = shfl_f(scale, kg * 4 + r);
          v8h ch[4], cl[4];
#pragma unroll
          for (int i = 0; i < 32; i++) {
            _Float16 hv, lv;
            split_f16(cv[u][i], inv, hv, lv);
            ch[i >> 3][i & 7] = hv;
            cl[i >> 3][i & 7] = lv;
          }
#pragma unroll
          for (int j = 0; j < 4; j++) {
            v8h b16[4];
            widen_fp8_operand(b[u][j], b16);
            v4f p = mfma_f16_block(ch, b16, v4f{0.f, 0.f, 0.f, 0.f});
            p = mfma_f16_block(cl, b16, p);
#pragma unroll
            for (int r = 0; r < 4; r++) acc[j][r] += p[r] * (sa[r] * sw[u]);
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int r = 0; r < 4; r++) red[wave][j][r][lane] = acc[j][r];
    __syncthreads();
    for (int idx = threadIdx.x; idx < 16 * kDec2Cols; idx += 64 * kDecWaves) {
      const int ln = idx & 63, j = (idx >> 6) & 3, r = idx >> 8;
      float o = 0.f;
#pragma unroll
      for (int w = 0; w < kDecWaves; w++) o += red[w][j][r][ln];
      const int row = m0 + (ln >> 4) * 4 + r;
      if (row < M) {
        const int p = row0 + row;
        obuf[(size_t)p * H + h0 + 16 * j + (ln & 15)] = o * pl.perm_w[p];
      }
    }
    __syncthreads();
  }

}

void launch_gemm1_decode(const Problem& pb, const Plan& pl, float* cbuf, int n_slots, hipStream_t stream) {
  if (n_slots <= 0) return;
  hipLaunchKernelGGL(gemm1_decode_kernel, dim3(pb.I / kDec1Cols, n_slots), dim3(64 * kDecWaves), 0, stream,
                     pb, pl, cbuf);
}

void launch_gemm2_decode(const Problem& pb, const Plan& pl, const float* cbuf, float* obuf, int n_slots,
                         hipStream_t stream) {
  if (n_slots <= 0) return;
  hipLaunchKernelGGL(gemm2_decode_kernel, dim3(pb.H / kDec2Cols, n_slots), dim3(64 * kDecWaves), 0, stream, pb, pl,
                     cbuf, obuf);
}

}  // namespace moefp8
