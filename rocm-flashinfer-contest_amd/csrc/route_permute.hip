// DeepSeek-V3 no-aux grouped routing for gfx950 wave64.
//
// route_kernel   restates solutions/moe_fp8/main.py:139-165 (_route) in the
//                canonical arithmetic of the oracle: fp64-evaluated sigmoid rounded
//                once to fp32, (value desc, index asc) ranking for groups and
//                experts, ascending-id output, sequential fp32 normaliser.
// The token -> local-expert permutation that follows (main.py:216-226) is rebuilt by the
// first small-T GEMM itself (decode_plan.h) or by permute_large.hip.
#include "moefp8_device.h"
#include "moefp8_launch.h"

#pragma clang fp contract(off)

namespace moefp8 {

// Is (va, ia) ranked before (vb, ib)?  Larger value first, lower index on ties.
__device__ __forceinline__ bool ranks_before(float va, int ia, float vb, int ib) {
  return va > vb || (va == vb && ia < ib);
}

// Magnitude inputs of the exact-product decision (optional): per token the squared
// L2 norm of its dequantised hidden row, per local expert an rms estimate of its
// W13 and W2 entries (448 * largest block scale / 3).
struct MagArgs {
  const uint8_t* hidden;   // [T, H] e4m3; NULL = skip
  const float* hscale;     // [H/128, T]
  const float* s13;        // [E, 2I/128, H/128]
  const float* s2;         // [E, H/128, I/128]
  int H, I, E_local;
  float* tok_a2;           // [T]
  float* esig;             // [E, 2]
};

// Scale estimates of local expert e by one workgroup of 256 threads.  W13 has exactly
// twice as many scale blocks as W2 (2I/128 x H/128 against H/128 x I/128), so one
// predicated batch of 8 + 4 loads per thread covers both tensors of the full-size
// expert (1792 + 896 scales) in a single memory round trip.
constexpr int kSigmaThreads = 256;

__device__ void expert_sigma_block(const MagArgs& mg, int e) {
  __shared__ float red[2][kSigmaThreads / kWave];
  const int n2 = (mg.H / kBlock) * (mg.I / kBlock), n13 = 2 * n2;
  const float* p13 = mg.s13 + (size_t)e * n13;
  const float* p2 = mg.s2 + (size_t)e * n2;
  const int tid = threadIdx.x, wave = tid >> 6;
  float m13 = 0.f, m2 = 0.f;
  for (int i0 = 0; i0 < n2; i0 += 4 * kSigmaThreads) {
    float v13[8], v2[4];
#pragma unroll
    for (int it = 0; it < 8; it++) {
      const int i = 2 * i0 + it * kSigmaThreads + tid;
      v13[it] = i < n13 ? p13[i] : 0.f;
    }
#pragma unroll
    for (int it = 0; it < 4; it++) {
      const int i = i0 + it * kSigmaThreads + tid;
      v2[it] = i < n2 ? p2[i] : 0.f;
    }
#pragma unroll
    for (int it = 0; it < 8; it++) m13 = fmaxf(m13, v13[it]);
#pragma unroll
    for (int it = 0; it < 4; it++) m2 = fmaxf(m2, v2[it]);
  }
  m13 = wave_max_f32(m13);
  m2 = wave_max_f32(m2);
  if (lane_id() == 0) {
    red[0][wave] = m13;
    red[1][wave] = m2;
  }
  __syncthreads();
  if (tid == 0) {
    float a = red[0][0], b = red[1][0];
#pragma unroll
    for (int w = 1; w < kSigmaThreads / kWave; w++) {
      a = fmaxf(a, red[0][w]);
      b = fmaxf(b, red[1][w]);
    }
    mg.esig[2 * e] = a * (448.0f / 3.0f);
    mg.esig[2 * e + 1] = b * (448.0f / 3.0f);
  }
}

// Squared L2 norm of token t's dequantised hidden row (one wavefront):
// ||A_t||^2 = sum_kb scale[kb,t]^2 * sum_{k in kb} e4m3(hs[t,k])^2.
__device__ float token_sq_norm(const uint8_t* hidden, const float* hscale, int H, int64_t T, int64_t t) {
  const int lane = lane_id();
  const int nch = H / 16;                       // 16-byte chunks of the row
  const uint8_t* row = hidden + t * H;
  float a2 = 0.f;
  for (int c0 = 0; c0 < nch; c0 += 8 * kWave) {
    // one predicated batch of loads per wave (no serialised round trips)
    v4i q[8];
    float sc[8];
#pragma unroll
    for (int it = 0; it < 8; it++) {
      const int c = c0 + it * kWave + lane;
      const bool ok = c < nch;
      q[it] = ok ? *reinterpret_cast<const v4i*>(row + (size_t)c * 16) : v4i{0, 0, 0, 0};
      sc[it] = ok ? hscale[(size_t)(c >> 3) * T + t] : 0.f;
    }
#pragma unroll
    for (int it = 0; it < 8; it++) {
      // e4m3 -> f16 is exact, and so are the f16 squares inside the fp32 dot products
      float ss = 0.f;
#pragma unroll
      for (int w4 = 0; w4 < 4; w4++) {
        const uint32_t word = (uint32_t)q[it][w4];
        const v2h lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(word, 1.0f, false);
        const v2h hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(word, 1.0f, true);
        ss = __builtin_amdgcn_fdot2(lo, lo, ss, false);
        ss = __builtin_amdgcn_fdot2(hi, hi, ss, false);
      }
      a2 += ss * sc[it] * sc[it];
    }
  }
  return wave_sum_f32(a2);
}

// Elements [i, i + 4) of a tensor of dtype dt (0 f32, 1 bf16, 2 f16; i a multiple of 4, the
// tensor 16-byte aligned) as fp32: two 8-byte loads (a 16-bit type loads its 8 bytes twice) and
// selects instead of branches, so that the loads of the bias and of a token's logits leave
// together (a load under a dtype branch is waited for before the next one is issued).
__device__ __forceinline__ void load4_as_f32(const void* p, int dt, int64_t i, float (&x)[4]) {
  const uint8_t* b = reinterpret_cast<const uint8_t*>(p) + i * (dt == 0 ? 4 : 2);
  const uint2 u = *reinterpret_cast<const uint2*>(b);
  const uint2 v = *reinterpret_cast<const uint2*>(b + (dt == 0 ? 8 : 0));
  const uint32_t w[4] = {u.x, u.y, v.x, v.y};
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint16_t h = (uint16_t)((k & 1) ? (w[k >> 1] >> 16) : (w[k >> 1] & 0xffffu));
    const float f16v = dt == 1 ? bf16_to_f32(h) : half_to_f32(h);
    x[k] = dt == 0 ? __uint_as_float(w[k]) : f16v;
  }
}

// The 4 logits of lane l (experts 4l..4l+3) of token t, as fp32.
__device__ __forceinline__ void load_logits(const void* logits, int logits_dt, int64_t t, float (&x)[4]) {
  load4_as_f32(logits, logits_dt, t * kEGlobal + 4 * lane_id(), x);
}

// Merge of two (largest, second largest) pairs.
__device__ __forceinline__ void merge_top2(float& m1, float& m2, float o1, float o2) {
  const float n2 = fmaxf(fminf(m1, o1), fmaxf(m2, o2));
  m1 = fmaxf(m1, o1);
  m2 = n2;
}

// Routing of one token by one wavefront (main.py:139-165); lane l owns experts 4l..4l+3
// (logits x, bias b), so lanes 8g..8g+7 own group g.  Lanes 0..7 return the j-th selected
// id (ascending) and its weight in *id / *w; other lanes return -1.  Cross-lane steps use
// DPP inside rows of 16 lanes and readlane / ballot across rows, so every selected expert
// is a wave-uniform value and no step waits on an LDS round trip.
__device__ void route_token(const float (&x)[4], const float (&b)[4], float rsf, int* id_out, float* w_out) {
  const int lane = lane_id();
  float s[4], sb[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    s[i] = (float)(1.0 / (1.0 + exp(-(double)x[i])));   // main.py:147
    sb[i] = s[i] + b[i];                                  // main.py:148
  }

  // per-group sum of the two largest sb (main.py:151-153): lane top-2, then merged with the
  // partners at distance 1 and 2 and the mirror lane of the 8-lane group
  float m1 = fmaxf(sb[0], sb[1]), m2 = fminf(sb[0], sb[1]);
#pragma unroll
  for (int i = 2; i < 4; i++) merge_top2(m1, m2, sb[i], -INFINITY);
  merge_top2(m1, m2, dpp_f32<kDppXor1>(m1), dpp_f32<kDppXor1>(m2));
  merge_top2(m1, m2, dpp_f32<kDppXor2>(m1), dpp_f32<kDppXor2>(m2));
  merge_top2(m1, m2, dpp_f32<kDppHalfMirror>(m1), dpp_f32<kDppHalfMirror>(m2));
  const float gscore = m1 + m2;

  // top-4 of 8 groups (main.py:154-156): rank of this lane's group against all 8
  const int my_group = lane >> 3;
  int beaten_by = 0;
#pragma unroll
  for (int g = 0; g < kNGroup; g++) beaten_by += ranks_before(readlane_f32(gscore, 8 * g), g, gscore, my_group);
  const bool group_kept = beaten_by < kTopKGroup;

  // top-8 experts inside the kept groups (main.py:158-160): per round the largest key
  // over the wave; ties go to the lowest lane (= lowest expert id) via the ballot and to
  // the lowest slot inside the lane via the strict comparison
  uint32_t key[4];
#pragma unroll
  for (int i = 0; i < 4; i++) key[i] = group_kept ? order_key(sb[i]) : 0u;
  int sel[kTopK];
#pragma unroll
  for (int r = 0; r < kTopK; r++) {
    uint32_t lk = key[0];
    int li = 0;
#pragma unroll
    for (int i = 1; i < 4; i++)
      if (key[i] > lk) {
        lk = key[i];
        li = i;
      }
    const uint32_t wk = wave_max_u32(lk);
    const int owner = (int)__builtin_ctzll(__ballot(lk == wk));
    const int slot = __builtin_amdgcn_readlane(li, owner);
    sel[r] = 4 * owner + slot;
#pragma unroll
    for (int i = 0; i < 4; i++)
      if (lane == owner && i == slot) key[i] = 0u;
  }

  // ascending id order (odd-even transposition network on wave-uniform values)
#pragma unroll
  for (int pass = 0; pass < kTopK; pass++) {
#pragma unroll
    for (int j = pass & 1; j + 1 < kTopK; j += 2) {
      const int lo = min(sel[j], sel[j + 1]), hi = max(sel[j], sel[j + 1]);
      sel[j] = lo;
      sel[j + 1] = hi;
    }
  }

  // weights from the unbiased s, normalised in ascending id order (main.py:162-164)
  float s_sel[kTopK];
#pragma unroll
  for (int j = 0; j < kTopK; j++) {
    const int owner = sel[j] >> 2, slot = sel[j] & 3;
    const float mine = slot == 0 ? s[0] : slot == 1 ? s[1] : slot == 2 ? s[2] : s[3];
    s_sel[j] = readlane_f32(mine, owner);
  }
  float acc = s_sel[0];
#pragma unroll
  for (int j = 1; j < kTopK; j++) acc = acc + s_sel[j];
  const float denom = acc + 1e-20f;
  *id_out = -1;
  *w_out = 0.f;
  if (lane < kTopK) {
    float sv = s_sel[0];
    int id = sel[0];
#pragma unroll
    for (int j = 1; j < kTopK; j++)
      if (lane == j) {
        sv = s_sel[j];
        id = sel[j];
      }
    *id_out = id;
    *w_out = __fdiv_rn(sv, denom) * rsf;
  }
}

// Blocks in order: one per local expert for the weight-scale estimates, then, with the magnitude
// inputs, the hidden-row norm blocks, then the routing blocks (the two leading kinds first, so
// that they run beside the routing blocks instead of after them; at T <= 64 the dispatch order is
// rotated to put the routing blocks first).  Norm and routing blocks take
// one token per wavefront (kSigmaThreads / 64 tokens per block): the norm streams the hidden
// rows while the routing arithmetic runs on other wavefronts.
__global__ __launch_bounds__(kSigmaThreads) void route_kernel(const void* __restrict__ logits, int logits_dt,
                                                              const void* __restrict__ bias, int bias_dt, int64_t T,
                                                              float rsf, int* __restrict__ topk_ids,
                                                              float* __restrict__ topk_w, int token_blocks,
                                                              int norm_blocks, MagArgs mg, int* __restrict__ zero,
                                                              int n_zero) {
  const int sigma_blocks = (int)gridDim.x - token_blocks - norm_blocks;
  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  constexpr int kWavesPerBlock = kSigmaThreads / kWave;
  // At T <= 64 every block is resident at once and the few routing blocks are the launch's
  // critical path, so they are dispatched first (route stage -0.2-0.3 us, measured); at large T
  // the leading sigma and norm blocks must not wait behind thousands of routing blocks.
  const int bid = T <= 64 ? ((int)blockIdx.x + sigma_blocks + norm_blocks) % (int)gridDim.x : (int)blockIdx.x;
  if (bid < sigma_blocks) {
    expert_sigma_block(mg, bid);
    return;
  }
  if (bid < sigma_blocks + norm_blocks) {
    const int nb = bid - sigma_blocks;
    for (int64_t t = (int64_t)nb * kWavesPerBlock + wave; t < T; t += (int64_t)norm_blocks * kWavesPerBlock) {
      const float a2 = token_sq_norm(mg.hidden, mg.hscale, mg.H, T, t);
      if (lane == 0) mg.tok_a2[t] = a2;
    }
    return;
  }
  const int tb = bid - sigma_blocks - norm_blocks;   // routing block
  for (int i = tb * kSigmaThreads + threadIdx.x; i < n_zero; i += token_blocks * kSigmaThreads)
    zero[(size_t)i * kCounterStride] = 0;
  // the first token's logits (a clamped row: no branch) leave with the bias, one round trip
  // for both; each later token's logits are loaded while the current one is routed
  const int64_t t0 = (int64_t)tb * kWavesPerBlock + wave, stride = (int64_t)token_blocks * kWavesPerBlock;
  float x[4], b[4];
  load_logits(logits, logits_dt, t0 < T ? t0 : T - 1, x);
  load4_as_f32(bias, bias_dt, 4 * lane, b);
  for (int64_t t = t0; t < T; t += stride) {
    int id;
    float w;
    route_token(x, b, rsf, &id, &w);
    if (t + stride < T) load_logits(logits, logits_dt, t + stride, x);
    if (lane < kTopK) {
      topk_ids[t * kTopK + lane] = id;
      topk_w[t * kTopK + lane] = w;
    }
  }
}

void launch_route(const void* logits, int logits_dt, const void* bias, int bias_dt, int64_t T, float rsf,
                  int* topk_ids, float* topk_w, const MagInputs* mag, int* zero, int n_zero, hipStream_t stream) {
  if (T <= 0) return;
  const int64_t tokens_per_block = kSigmaThreads / kWave;
  int64_t blocks = (T + tokens_per_block - 1) / tokens_per_block;
  if (blocks > 4096) blocks = 4096;
  MagArgs mg = {};
  int extra = 0;
  if (mag) {
    mg.hidden = mag->hidden;
    mg.hscale = mag->hscale;
    mg.s13 = mag->s13;
    mg.s2 = mag->s2;
    mg.H = mag->H;
    mg.I = mag->I;
    mg.E_local = mag->E_local;
    mg.tok_a2 = mag->tok_a2;
    mg.esig = mag->esig;
    extra = mag->E_local;
  }
  // the norm blocks stream the hidden rows (bandwidth-bound): 256 of them (each wavefront then
  // takes T / 1024 rows in turn) leave the CUs' slots to the routing blocks at large T
  const int norm_blocks = mag ? (int)(blocks < 256 ? blocks : 256) : 0;
  hipLaunchKernelGGL(route_kernel, dim3((unsigned)(blocks + norm_blocks + extra)), dim3(kSigmaThreads), 0, stream,
                     logits, logits_dt, bias, bias_dt, T, rsf, topk_ids, topk_w, (int)blocks, norm_blocks, mg, zero,
                     n_zero);
}


}  // namespace moefp8
