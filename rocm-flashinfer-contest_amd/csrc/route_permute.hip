// DeepSeek-V3 no-aux grouped routing and the deterministic token -> local-expert
// permutation, for gfx950 wave64.
//
// route_kernel   restates solutions/moe_fp8/main.py:139-165 (_route) in the
//                canonical arithmetic of the oracle: fp64-evaluated sigmoid rounded
//                once to fp32, (value desc, index asc) ranking for groups and
//                experts, ascending-id output, sequential fp32 normaliser.
// permute_kernel restates the selection of main.py:216-226: for each local
//                expert in ascending order, the tokens that picked it in ascending
//                token order (torch.nonzero), as one stable counting sort.
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

__device__ float wave_max_batched(const float* p, int n);

__device__ void expert_sigma_block(const MagArgs& mg, int e) {
  __shared__ float red[2][4];
  const int n13 = (2 * mg.I / kBlock) * (mg.H / kBlock), n2 = (mg.H / kBlock) * (mg.I / kBlock);
  const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  // wave w reduces the w-th quarter of each scale tensor
  const int q13 = (n13 + nw - 1) / nw, q2 = (n2 + nw - 1) / nw;
  const int b13 = min(n13, wave * q13), b2 = min(n2, wave * q2);
  const float m13 = wave_max_batched(mg.s13 + (size_t)e * n13 + b13, min(n13, b13 + q13) - b13);
  const float m2 = wave_max_batched(mg.s2 + (size_t)e * n2 + b2, min(n2, b2 + q2) - b2);
  if (lane_id() == 0) {
    red[0][wave] = m13;
    red[1][wave] = m2;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float a = red[0][0], b = red[1][0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++) {
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
      float ss = 0.f;
#pragma unroll
      for (int w4 = 0; w4 < 4; w4++)
#pragma unroll
        for (int bb = 0; bb < 4; bb++) {
          const float v = e4m3_to_f32(((uint32_t)q[it][w4] >> (8 * bb)) & 0xffu);
          ss += v * v;
        }
      a2 += ss * sc[it] * sc[it];
    }
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) a2 += shfl_xor_f(a2, off);
  return a2;
}

// Largest of n floats (one wavefront, loads in predicated batches of 16 per lane).
__device__ float wave_max_batched(const float* p, int n) {
  const int lane = lane_id();
  float m = 0.f;
  for (int i0 = 0; i0 < n; i0 += 16 * kWave) {
    float v[16];
#pragma unroll
    for (int it = 0; it < 16; it++) {
      const int i = i0 + it * kWave + lane;
      v[it] = i < n ? p[i] : 0.f;
    }
#pragma unroll
    for (int it = 0; it < 16; it++) m = fmaxf(m, v[it]);
  }
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) m = fmaxf(m, shfl_xor_f(m, off));
  return m;
}

// Routing of token t by one wavefront (main.py:139-165); lane l owns experts 4l..4l+3, so
// lanes 8g..8g+7 own group g.  Lanes 0..7 return the j-th selected id (ascending) and its
// weight in *id / *w; other lanes return -1.
__device__ void route_token(const void* logits, int logits_dt, const float (&b)[4], int64_t t, float rsf, int* id_out,
                            float* w_out) {
  const int lane = lane_id();
  float x[4];
  if (logits_dt == 0) {
    const float4 v = reinterpret_cast<const float4*>(logits)[t * (kEGlobal / 4) + lane];
    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) x[i] = load_as_f32(logits, logits_dt, t * kEGlobal + 4 * lane + i);
  }
  float s[4], sb[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    s[i] = (float)(1.0 / (1.0 + exp(-(double)x[i])));   // main.py:147
    sb[i] = s[i] + b[i];                                  // main.py:148
  }

  // per-group sum of the two largest sb (main.py:151-153): lane top-2, then merge over 8 lanes
  float m1 = fmaxf(sb[0], sb[1]), m2 = fminf(sb[0], sb[1]);
#pragma unroll
  for (int i = 2; i < 4; i++) {
    const float v = sb[i];
    const float n2 = fmaxf(fminf(m1, v), m2);
    m1 = fmaxf(m1, v);
    m2 = n2;
  }
#pragma unroll
  for (int off = 1; off < 8; off <<= 1) {
    const float o1 = shfl_xor_f(m1, off), o2 = shfl_xor_f(m2, off);
    const float n2 = fmaxf(fminf(m1, o1), fmaxf(m2, o2));
    m1 = fmaxf(m1, o1);
    m2 = n2;
  }
  const float gscore = m1 + m2;

  // top-4 of 8 groups (main.py:154-156)
  const int my_group = lane >> 3;
  int beaten_by = 0;
#pragma unroll
  for (int g = 0; g < kNGroup; g++) {
    const float gs = shfl_f(gscore, 8 * g);
    beaten_by += ranks_before(gs, g, gscore, my_group) ? 1 : 0;
  }
  const bool group_kept = beaten_by < kTopKGroup;

  // top-8 experts inside the kept groups (main.py:158-160), one arg-max per round
  bool alive[4];
#pragma unroll
  for (int i = 0; i < 4; i++) alive[i] = group_kept;
  int sel[kTopK];
#pragma unroll
  for (int r = 0; r < kTopK; r++) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      if (alive[i] && ranks_before(sb[i], 4 * lane + i, bv, bi)) {
        bv = sb[i];
        bi = 4 * lane + i;
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = shfl_xor_f(bv, off);
      const int oi = shfl_xor_i(bi, off);
      if (ranks_before(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    sel[r] = bi;
#pragma unroll
    for (int i = 0; i < 4; i++)
      if (bi == 4 * lane + i) alive[i] = false;
  }

  // ascending id order (odd-even transposition network, 8 elements)
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
    s_sel[j] = __shfl(mine, owner, kWave);
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

// One wavefront per token.
__global__ __launch_bounds__(256) void route_kernel(const void* __restrict__ logits, int logits_dt,
                                                    const void* __restrict__ bias, int bias_dt, int64_t T,
                                                    float rsf, int* __restrict__ topk_ids,
                                                    float* __restrict__ topk_w, int token_blocks, MagArgs mg) {
  if ((int)blockIdx.x >= token_blocks) {                 // trailing blocks: one per local expert
    expert_sigma_block(mg, blockIdx.x - token_blocks);
    return;
  }
  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  const int waves_per_block = blockDim.x >> 6;
  float b[4];
#pragma unroll
  for (int i = 0; i < 4; i++) b[i] = load_as_f32(bias, bias_dt, 4 * lane + i);

  for (int64_t t = (int64_t)blockIdx.x * waves_per_block + wave; t < T;
       t += (int64_t)token_blocks * waves_per_block) {
    if (mg.hidden) {
      const float a2 = token_sq_norm(mg.hidden, mg.hscale, mg.H, T, t);
      if (lane == 0) mg.tok_a2[t] = a2;
    }
    int id;
    float w;
    route_token(logits, logits_dt, b, t, rsf, &id, &w);
    if (lane < kTopK) {
      topk_ids[t * kTopK + lane] = id;
      topk_w[t * kTopK + lane] = w;
    }
  }
}

// Single-workgroup stable counting sort of (token, local expert) pairs.
//   counts/offsets  per local expert (main.py:222, 225)
//   perm_token[p]   token of pair p, expert-major, token-ascending
//   perm_w[p]       routing weight of pair p (main.py:240)
//   tok_slot[t][k]  pair index of token t's k-th local expert (ascending expert), -1 padded
//   active[]        local experts with >= 1 token, ascending; info[] totals
constexpr int kPermThreads = 1024;
constexpr int kPermWaves = kPermThreads / kWave;
constexpr int kSmallT = 64;

__global__ __launch_bounds__(kPermThreads) void permute_kernel(
    const int* __restrict__ topk_ids, const float* __restrict__ topk_w, int T, int E_local, int offset,
    int tile_m, int* __restrict__ expert_offsets, int* __restrict__ perm_token, float* __restrict__ perm_w,
    int* __restrict__ tok_slot, int* __restrict__ active, int* __restrict__ mtile_offsets,
    int* __restrict__ info, const float* __restrict__ tok_a2, const float* __restrict__ esig, float sqrt_i,
    uint8_t* __restrict__ perm_exact) {
  __shared__ int cnt[kEGlobal];
  __shared__ int base[kEGlobal];
  __shared__ int wcnt[kPermWaves][kEGlobal];
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;

  for (int e = tid; e < E_local; e += kPermThreads) cnt[e] = 0;
  __syncthreads();
  for (int i = tid; i < T * kTopK; i += kPermThreads) {
    const int le = topk_ids[i] - offset;
    if (le >= 0 && le < E_local) atomicAdd(&cnt[le], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0, n_act = 0, mt = 0;
    for (int e = 0; e < E_local; e++) {
      expert_offsets[e] = run;
      mtile_offsets[e] = mt;
      base[e] = run;
      run += cnt[e];
      mt += (cnt[e] + tile_m - 1) / tile_m;
      if (cnt[e] > 0) active[n_act++] = e;
    }
    expert_offsets[E_local] = run;
    mtile_offsets[E_local] = mt;
    info[0] = run;    // P
    info[1] = n_act;  // active experts
    info[2] = mt;     // m-tiles of height tile_m
  }
  __syncthreads();

  for (int c0 = 0; c0 < T; c0 += kPermThreads) {
    const int t = c0 + tid;
    int les[kTopK], slots[kTopK], rank[kTopK];
    int n = 0;
    if (t < T) {
#pragma unroll
      for (int j = 0; j < kTopK; j++) {
        const int le = topk_ids[t * kTopK + j] - offset;
        if (le >= 0 && le < E_local) {
#pragma unroll
          for (int k = 0; k < kTopK; k++)
            if (k == n) {
              les[k] = le;
              slots[k] = j;
            }
          n++;
        }
      }
    }
    int ptr = 0;
    for (int e = 0; e < E_local; e++) {
      int cur = -1;
#pragma unroll
      for (int k = 0; k < kTopK; k++)
        if (k == ptr) cur = les[k];
      const bool pick = ptr < n && cur == e;
      const uint64_t m = __ballot(pick);
      if (lane == 0) wcnt[wave][e] = __popcll(m);
      if (pick) {
        const int r = __popcll(m & ((1ull << lane) - 1ull));
#pragma unroll
        for (int k = 0; k < kTopK; k++)
          if (k == ptr) rank[k] = r;
        ptr++;
      }
    }
    __syncthreads();
    for (int e = tid; e < E_local; e += kPermThreads) {
      int run = base[e];
      for (int w = 0; w < kPermWaves; w++) {
        const int c = wcnt[w][e];
        wcnt[w][e] = run;
        run += c;
      }
      base[e] = run;
    }
    __syncthreads();
    if (t < T) {
#pragma unroll
      for (int k = 0; k < kTopK; k++) {
        int pos = -1;
        if (k < n) {
          pos = wcnt[wave][les[k]] + rank[k];
          const float w = topk_w[t * kTopK + slots[k]];
          perm_token[pos] = t;
          perm_w[pos] = w;
          perm_exact[pos] = needs_exact_products(tok_a2[t], w, esig[2 * les[k]], esig[2 * les[k] + 1], sqrt_i);
        }
        tok_slot[t * kTopK + k] = pos;
      }
    }
    __syncthreads();
  }
}

// Small-T front end (T <= kSmallT): routing, token norms, expert weight-scale estimates,
// exact-product flags and the stable permutation in ONE workgroup (one launch instead of
// two).  Wave w routes tokens w, w+16, ...; wave 0 then ranks all (<= 64) tokens with
// ballots, so pairs come out expert-major and token-ascending as in main.py:218-225.
__global__ __launch_bounds__(kPermThreads) void route_permute_small_kernel(
    const void* __restrict__ logits, int logits_dt, const void* __restrict__ bias, int bias_dt, int T, float rsf,
    MagArgs mg, int offset, int tile_m, int* __restrict__ topk_ids, float* __restrict__ topk_w,
    int* __restrict__ expert_offsets, int* __restrict__ perm_token, float* __restrict__ perm_w,
    int* __restrict__ tok_slot, int* __restrict__ active, int* __restrict__ mtile_offsets, int* __restrict__ info,
    uint8_t* __restrict__ perm_exact) {
  __shared__ int ids_s[kSmallT][kTopK];
  __shared__ float w_s[kSmallT][kTopK];
  __shared__ float a2_s[kSmallT];
  __shared__ int cnt[kEGlobal];
  __shared__ int base[kEGlobal];
  __shared__ int act_s[kEGlobal];
  __shared__ int n_act_s;
  __shared__ float sig_s[kEGlobal][2];
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  const int E_local = mg.E_local;

  // weight-scale estimates of every local expert (independent of the routing, so their loads
  // overlap it): wave w takes experts w, w+16, ...
  const int n13 = (2 * mg.I / kBlock) * (mg.H / kBlock), n2 = (mg.H / kBlock) * (mg.I / kBlock);
  for (int e = wave; e < E_local; e += kPermWaves) {
    const float m13 = wave_max_batched(mg.s13 + (size_t)e * n13, n13);
    const float m2 = wave_max_batched(mg.s2 + (size_t)e * n2, n2);
    if (lane == 0) {
      sig_s[e][0] = m13 * (448.0f / 3.0f);
      sig_s[e][1] = m2 * (448.0f / 3.0f);
    }
  }
  float b[4];
#pragma unroll
  for (int i = 0; i < 4; i++) b[i] = load_as_f32(bias, bias_dt, 4 * lane + i);
  for (int t = wave; t < T; t += kPermWaves) {
    const float a2 = token_sq_norm(mg.hidden, mg.hscale, mg.H, T, t);
    int id;
    float w;
    route_token(logits, logits_dt, b, t, rsf, &id, &w);
    if (lane < kTopK) {
      ids_s[t][lane] = id;
      w_s[t][lane] = w;
      topk_ids[t * kTopK + lane] = id;
      topk_w[t * kTopK + lane] = w;
    }
    if (lane == 0) a2_s[t] = a2;
  }
  for (int e = tid; e < E_local; e += kPermThreads) cnt[e] = 0;
  __syncthreads();
  if (tid < T * kTopK) {
    const int le = ids_s[tid >> 3][tid & 7] - offset;
    if (le >= 0 && le < E_local) atomicAdd(&cnt[le], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0, n_act = 0, mt = 0;
    for (int e = 0; e < E_local; e++) {
      expert_offsets[e] = run;
      mtile_offsets[e] = mt;
      base[e] = run;
      run += cnt[e];
      mt += (cnt[e] + tile_m - 1) / tile_m;
      if (cnt[e] > 0) {
        active[n_act] = e;
        act_s[n_act++] = e;
      }
    }
    expert_offsets[E_local] = run;
    mtile_offsets[E_local] = mt;
    info[0] = run;
    info[1] = n_act;
    info[2] = mt;
    n_act_s = n_act;
  }
  __syncthreads();
  if (wave == 0) {
    const int t = lane;
    int les[kTopK], slots[kTopK];
    int n = 0;
#pragma unroll
    for (int k = 0; k < kTopK; k++) {
      les[k] = -1;
      slots[k] = 0;
    }
    if (t < T) {
#pragma unroll
      for (int j = 0; j < kTopK; j++) {
        const int le = ids_s[t][j] - offset;
        if (le >= 0 && le < E_local) {
#pragma unroll
          for (int k = 0; k < kTopK; k++)
            if (k == n) {
              les[k] = le;
              slots[k] = j;
            }
          n++;
        }
      }
    }
    int ptr = 0;
    int pos_k[kTopK];
#pragma unroll
    for (int k = 0; k < kTopK; k++) pos_k[k] = -1;
    const float sqrt_i = sqrtf((float)mg.I);
    for (int a = 0; a < n_act_s; a++) {
      const int e = act_s[a];
      int cur = -1;
#pragma unroll
      for (int k = 0; k < kTopK; k++)
        if (k == ptr) cur = les[k];
      const bool pick = ptr < n && cur == e;
      const uint64_t m = __ballot(pick);
      if (pick) {
        const int pos = base[e] + __popcll(m & ((1ull << lane) - 1ull));
        int slot = 0;
#pragma unroll
        for (int k = 0; k < kTopK; k++)
          if (k == ptr) {
            slot = slots[k];
            pos_k[k] = pos;
          }
        const float w = w_s[t][slot];
        perm_token[pos] = t;
        perm_w[pos] = w;
        perm_exact[pos] = needs_exact_products(a2_s[t], w, sig_s[e][0], sig_s[e][1], sqrt_i);
        ptr++;
      }
    }
    if (t < T) {
#pragma unroll
      for (int k = 0; k < kTopK; k++) tok_slot[t * kTopK + k] = pos_k[k];
    }
  }
}

void launch_route_permute_small(const void* logits, int logits_dt, const void* bias, int bias_dt, int T, float rsf,
                                const MagInputs& mag, int offset, int tile_m, int* topk_ids, float* topk_w,
                                int* expert_offsets, int* perm_token, float* perm_w, int* tok_slot, int* active,
                                int* mtile_offsets, int* info, uint8_t* perm_exact, hipStream_t stream) {
  MagArgs mg = {};
  mg.hidden = mag.hidden;
  mg.hscale = mag.hscale;
  mg.s13 = mag.s13;
  mg.s2 = mag.s2;
  mg.H = mag.H;
  mg.I = mag.I;
  mg.E_local = mag.E_local;
  hipLaunchKernelGGL(route_permute_small_kernel, dim3(1), dim3(kPermThreads), 0, stream, logits, logits_dt, bias,
                     bias_dt, T, rsf, mg, offset, tile_m, topk_ids, topk_w, expert_offsets, perm_token, perm_w,
                     tok_slot, active, mtile_offsets, info, perm_exact);
}

void launch_route(const void* logits, int logits_dt, const void* bias, int bias_dt, int64_t T, float rsf,
                  int* topk_ids, float* topk_w, const MagInputs* mag, hipStream_t stream) {
  if (T <= 0) return;
  const int64_t tokens_per_block = 4;
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
  hipLaunchKernelGGL(route_kernel, dim3((unsigned)(blocks + extra)), dim3(256), 0, stream, logits, logits_dt,
                     bias, bias_dt, T, rsf, topk_ids, topk_w, (int)blocks, mg);
}

void launch_permute(const int* topk_ids, const float* topk_w, int T, int E_local, int offset, int tile_m,
                    int* expert_offsets, int* perm_token, float* perm_w, int* tok_slot, int* active,
                    int* mtile_offsets, int* info, const float* tok_a2, const float* esig, int I,
                    uint8_t* perm_exact, hipStream_t stream) {
  hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(kPermThreads), 0, stream, topk_ids, topk_w, T, E_local,
                     offset, tile_m, expert_offsets, perm_token, perm_w, tok_slot, active, mtile_offsets, info,
                     tok_a2, esig, sqrtf((float)I), perm_exact);
}

}  // namespace moefp8
