// Large-T grouped expert GEMMs on fp8 MFMA (v_mfma_f32_16x16x128_f8f6f4).
//
// A tile = (local expert e, tile_m permuted rows of e, output column block).
// Tiles are numbered expert-major, then column block, then row block, so the
// workgroups that run together share one weight block (read from HBM once,
// then from L2 / Infinity Cache).  A persistent grid walks the tile list that
// routing + permutation left on the device: no host sync, no empty launches.
//
// Operands
//   A  gathered activation rows, staged through LDS (two stages, XOR-swizzled
//      16-byte chunks so the MFMA operand reads are bank-conflict free) and
//      shared by the 4 waves of the workgroup;
//   B  weight rows, loaded by each wave straight into MFMA operand registers
//      (each weight byte feeds exactly one wave), one K block ahead.
// Every K block of 128 is one MFMA per 16x16 sub-tile; its fp32 partial is
// scaled by scale_A[row, kb] * scale_W[nb, kb] and accumulated in fp32
// (main.py:93-94, 117, 134-136 dequantisation folded into the accumulation).
//
// GEMM1 (main.py:229-233): 128 C columns = W13 rows [n0, n0+128) (up) and
//   [I+n0, I+n0+128) (gate); epilogue C = silu(gate) * up, then the multi-term
//   e4m3 split of C (2-4 terms, one fp32 scale per (row, 128 columns)) and the
//   term count each 16-row sub-tile needs for GEMM2's error budget.
// GEMM2 (main.py:234-241): 256 H columns; A = the term planes, one MFMA per
//   term into one partial (term k scaled by 2^-4k inside the MFMA); epilogue
//   multiplies by the pair's routing weight.
#include "moefp8_device.h"
#include "moefp8_launch.h"

namespace moefp8 {

constexpr int kPfThreads = 256;
constexpr int kPfWaves = kPfThreads / kWave;

__device__ __forceinline__ v8i load_v8i_g(const uint8_t* p) {
  const v4i* q = reinterpret_cast<const v4i*>(p);
  const v4i x = q[0], y = q[1];
  return __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Byte offset of 16-byte chunk c of row r inside a [rows][128] LDS tile.
__device__ __forceinline__ int swz(int r, int c) { return r * kBlock + ((c ^ (r & 7)) << 4); }

// A operand (16 rows x 128 k) of m-subtile ms from an LDS tile.
__device__ __forceinline__ v8i lds_a_operand(const uint8_t* tile, int ms, int lr, int kg) {
  const int r = ms * 16 + lr;
  const v4i x = *reinterpret_cast<const v4i*>(tile + swz(r, 2 * kg));
  const v4i y = *reinterpret_cast<const v4i*>(tile + swz(r, 2 * kg + 1));
  return __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7);
}

struct TileCoord {
  int e, nt, row0, M, mtile_global;
};

// Decode a linear tile id into (expert, column block, first row, valid rows).
__device__ __forceinline__ TileCoord locate_tile(const Plan& pl, int E_local, int NT, int tile_m, int tile) {
  int lo = 0, hi = E_local;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (pl.mtile_offsets[mid] * NT <= tile) lo = mid; else hi = mid;
  }
  const int mt0 = pl.mtile_offsets[lo];
  const int cnt = pl.mtile_offsets[lo + 1] - mt0;
  const int local = tile - mt0 * NT;
  TileCoord tc;
  tc.e = lo;
  tc.nt = local / cnt;
  const int mtile = local - tc.nt * cnt;
  tc.row0 = pl.expert_offsets[lo] + mtile * tile_m;
  tc.M = min(tile_m, pl.expert_offsets[lo + 1] - tc.row0);
  tc.mtile_global = mt0 + mtile;
  return tc;
}

template <int BM>
__global__ __launch_bounds__(kPfThreads) void gemm1_prefill_kernel(Problem pb, Plan pl, CSplit cs) {
  constexpr int MS = BM / 16;
  constexpr int ACH = BM * 8 / kPfThreads;  // 16-byte A chunks per thread per K block
  static_assert(ACH >= 1, "tile_m too small");
  // stages 0,1 hold A during the K loop; all kMaxTerms buffers stage C's terms in the epilogue
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[kMaxTerms][BM * kBlock];
  __shared__ __attribute__((aligned(16))) float sa_lds[2][BM];
  __shared__ float amax_lds[kPfWaves][BM];
  __shared__ float ssq_lds[kPfWaves][BM];
  __shared__ int kmax_lds[MS];

  const int H = pb.H, I = pb.I, T = pb.T;
  const int KB = H / kBlock;
  const int NT = I / kBlock;
  const int total = pl.info[2] * NT;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  const int lr = lane & 15, kg = lane >> 4;

  for (int tile = blockIdx.x; tile < total; tile += gridDim.x) {
    const TileCoord tc = locate_tile(pl, pb.E_local, NT, BM, tile);
    const int e = tc.e, row0 = tc.row0, M = tc.M;
    const int n0 = tc.nt * kBlock;

    // A staging sources (rows past M repeat the last valid row; never stored)
    const uint8_t* a_src[ACH];
    int a_dst[ACH];
#pragma unroll
    for (int i = 0; i < ACH; i++) {
      const int ch = tid + i * kPfThreads;
      const int r = ch >> 3, c = ch & 7;
      const int tok = pl.perm_token[row0 + min(r, M - 1)];
      a_src[i] = pb.hidden + (size_t)tok * H + c * 16;
      a_dst[i] = swz(r, c);
    }
    const float* sa_src = pb.hscale + (tid < BM ? pl.perm_token[row0 + min(tid, M - 1)] : 0);

    // B rows of this wave: sub-tiles 0,1 up rows, 2,3 gate rows
    const uint8_t* wexp = pb.w13 + (size_t)e * 2 * I * H;
    const uint8_t* brow[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int n = (j < 2 ? n0 + wave * 32 + 16 * j : I + n0 + wave * 32 + 16 * (j - 2)) + lr;
      brow[j] = wexp + (size_t)n * H + kg * 32;
    }
    const float* s_up = pb.s13 + ((size_t)e * (2 * I / kBlock) + n0 / kBlock) * KB;
    const float* s_gate = pb.s13 + ((size_t)e * (2 * I / kBlock) + (I + n0) / kBlock) * KB;

    v4f acc[MS][4];
#pragma unroll
    for (int ms = 0; ms < MS; ms++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[ms][j] = v4f{0.f, 0.f, 0.f, 0.f};
    // exact-product sub-tiles: bit ms set if any of its 16 pairs is flagged
    uint32_t exact_mask = 0;
#pragma unroll
    for (int ms = 0; ms < MS; ms++) {
      const int r = ms * 16 + lr;
      if (__ballot(lane < 16 && r < M && pl.exact[row0 + r]) != 0) exact_mask |= 1u << ms;
    }

    // prologue: K block 0 -> LDS stage 0, B block 0 -> registers
    v4i areg[ACH];
    float sareg = 0.f;
#pragma unroll
    for (int i = 0; i < ACH; i++) areg[i] = *reinterpret_cast<const v4i*>(a_src[i]);
    if (tid < BM) sareg = sa_src[0];
#pragma unroll
    for (int i = 0; i < ACH; i++) *reinterpret_cast<v4i*>(&a_lds[0][a_dst[i]]) = areg[i];
    if (tid < BM) sa_lds[0][tid] = sareg;
    v8i bcur[4];
#pragma unroll
    for (int j = 0; j < 4; j++) bcur[j] = load_v8i_g(brow[j]);
    __syncthreads();

    for (int kb = 0; kb < KB; kb++) {
      const int st = kb & 1;
      const bool more = kb + 1 < KB;
      v8i bnxt[4];
      if (more) {
        const size_t koff = (size_t)(kb + 1) * kBlock;
#pragma unroll
        for (int i = 0; i < ACH; i++) areg[i] = *reinterpret_cast<const v4i*>(a_src[i] + koff);
        if (tid < BM) sareg = sa_src[(size_t)(kb + 1) * T];
#pragma unroll
        for (int j = 0; j < 4; j++) bnxt[j] = load_v8i_g(brow[j] + koff);
      }
      const float su = s_up[kb], sg = s_gate[kb];
#pragma unroll
      for (int ms = 0; ms < MS; ms++) {
        const v8i a = lds_a_operand(a_lds[st], ms, lr, kg);
        const v4f sa = *reinterpret_cast<const v4f*>(&sa_lds[st][ms * 16 + kg * 4]);
        if (exact_mask & (1u << ms)) {
          v8h a16[4];
          widen_fp8_operand(a, a16);
#pragma unroll
          for (int j = 0; j < 4; j++) {
            v8h b16[4];
            widen_fp8_operand(bcur[j], b16);
            const v4f p = mfma_f16_block(a16, b16, v4f{0.f, 0.f, 0.f, 0.f});
            const float sw = j < 2 ? su : sg;
#pragma unroll
            for (int r = 0; r < 4; r++) acc[ms][j][r] += p[r] * (sa[r] * sw);
          }
          continue;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const v4f p = mfma16x16x128(a, bcur[j], v4f{0.f, 0.f, 0.f, 0.f});
          const float sw = j < 2 ? su : sg;
#pragma unroll
          for (int r = 0; r < 4; r++) acc[ms][j][r] += p[r] * (sa[r] * sw);
        }
      }
      if (more) {
#pragma unroll
        for (int i = 0; i < ACH; i++) *reinterpret_cast<v4i*>(&a_lds[st ^ 1][a_dst[i]]) = areg[i];
        if (tid < BM) sa_lds[st ^ 1][tid] = sareg;
#pragma unroll
        for (int j = 0; j < 4; j++) bcur[j] = bnxt[j];
      }
      __syncthreads();
    }

    // epilogue: SwiGLU (gate = second half), then the multi-term e4m3 split of C
    // with one fp32 scale per (row, 128 columns)
    float cval[MS][2][4];
#pragma unroll
    for (int ms = 0; ms < MS; ms++)
#pragma unroll
      for (int r = 0; r < 4; r++) {
        float m = 0.f, ss = 0.f;
#pragma unroll
        for (int q = 0; q < 2; q++) {
          const float v = silu_f32(acc[ms][q + 2][r]) * acc[ms][q][r];
          cval[ms][q][r] = v;
          m = fmaxf(m, fabsf(v));
          ss += v * v;
        }
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
          m = fmaxf(m, shfl_xor_f(m, off));
          ss += shfl_xor_f(ss, off);
        }
        if (lr == 0) {
          amax_lds[wave][ms * 16 + kg * 4 + r] = m;
          ssq_lds[wave][ms * 16 + kg * 4 + r] = ss;
        }
      }
    // largest |W2| in GEMM2's K block n0/128 of this expert
    const int HB = H / kBlock;
    float wm = 0.f;
    for (int hb = lane; hb < HB; hb += kWave) wm = fmaxf(wm, pb.s2[((size_t)e * HB + hb) * NT + tc.nt]);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) wm = fmaxf(wm, shfl_xor_f(wm, off));
    wm *= 448.0f;
    __syncthreads();
    int kneed[MS];
#pragma unroll
    for (int ms = 0; ms < MS; ms++) {
      kneed[ms] = 2;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int row = ms * 16 + kg * 4 + r;
        float m = amax_lds[0][row], ss = ssq_lds[0][row];
#pragma unroll
        for (int w = 1; w < kPfWaves; w++) {
          m = fmaxf(m, amax_lds[w][row]);
          ss += ssq_lds[w][row];
        }
        float inv, scale;
        split_scale(m, inv, scale);
        const float wr = row < M ? fabsf(pl.perm_w[row0 + row]) : 0.f;
        kneed[ms] = max(kneed[ms], terms_needed(sqrtf(ss) * wr * wm));
        if (wave == 0 && lr == 0 && row < M) cs.scale[(size_t)(row0 + row) * NT + tc.nt] = scale;
        if (exact_mask & (1u << ms)) {
          // exact-product sub-tile: two-term f16 split straight to global
          if (row < M) {
#pragma unroll
            for (int q = 0; q < 2; q++) {
              _Float16 h, l;
              split_f16(cval[ms][q][r], inv, h, l);
              const size_t g = (size_t)(row0 + row) * I + n0 + wave * 32 + q * 16 + lr;
              cs.c16[g] = h;
              cs.c16[cs.plane + g] = l;
            }
          }
          continue;
        }
#pragma unroll
        for (int q = 0; q < 2; q++) {
          uint32_t qv[kMaxTerms];
          split_terms(cval[ms][q][r], inv, qv);
          const int col = wave * 32 + q * 16 + lr;
          const int off = swz(row, col >> 4) + (col & 15);
#pragma unroll
          for (int k = 0; k < kMaxTerms; k++) a_lds[k][off] = (uint8_t)qv[k];
        }
      }
      kneed[ms] = max(kneed[ms], shfl_xor_i(kneed[ms], 16));
      kneed[ms] = max(kneed[ms], shfl_xor_i(kneed[ms], 32));
      if (exact_mask & (1u << ms)) kneed[ms] = kExactTerms;
    }
    if (tid == 0) {
#pragma unroll
      for (int ms = 0; ms < MS; ms++) {
        kmax_lds[ms] = kneed[ms];
        cs.kmax[((size_t)tc.mtile_global * MS + ms) * NT + tc.nt] = (uint8_t)kneed[ms];
      }
    }
    __syncthreads();
    for (int ch = tid; ch < BM * 8; ch += kPfThreads) {
      const int r = ch >> 3, c = ch & 7;
      if (r < M) {
        const size_t g = (size_t)(row0 + r) * I + n0 + c * 16;
        const int nk = kmax_lds[r >> 4] == kExactTerms ? 0 : kmax_lds[r >> 4];
#pragma unroll
        for (int k = 0; k < kMaxTerms; k++)
          if (k < nk) *reinterpret_cast<v4i*>(cs.q + (size_t)k * cs.plane + g) =
                          *reinterpret_cast<const v4i*>(&a_lds[k][swz(r, c)]);
      }
    }
    __syncthreads();
  }
}

template <int BM>
__global__ __launch_bounds__(kPfThreads) void gemm2_prefill_kernel(Problem pb, Plan pl, CSplit cs,
                                                                  float* __restrict__ obuf) {
  constexpr int MS = BM / 16;
  constexpr int BN = 256;
  constexpr int ACH = BM * 8 / kPfThreads;  // 16-byte chunks per thread per term plane
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[2][kMaxTerms][BM * kBlock];  // [stage][term]
  __shared__ __attribute__((aligned(16))) float sa_lds[2][BM];

  const int H = pb.H, I = pb.I;
  const int KB = I / kBlock;
  const int NT = (H + BN - 1) / BN;
  const int total = pl.info[2] * NT;
  const int tid = threadIdx.x, lane = lane_id(), wave = tid >> 6;
  const int lr = lane & 15, kg = lane >> 4;

  for (int tile = blockIdx.x; tile < total; tile += gridDim.x) {
    const TileCoord tc = locate_tile(pl, pb.E_local, NT, BM, tile);
    const int e = tc.e, row0 = tc.row0, M = tc.M;
    const int h0 = tc.nt * BN + wave * 64;   // this wave's 64 columns
    const bool wave_on = h0 < H;              // H % 256 == 128 leaves the last two waves idle
    const uint8_t* kmax = cs.kmax + (size_t)tc.mtile_global * MS * KB;   // [MS][KB]
    auto planes_for = [&](int kb) {
      int n = 0;
#pragma unroll
      for (int ms = 0; ms < MS; ms++) {
        const int k = kmax[ms * KB + kb];
        n = max(n, k == kExactTerms ? 0 : k);
      }
      return n;
    };

    size_t a_src[ACH];
    int a_dst[ACH];
#pragma unroll
    for (int i = 0; i < ACH; i++) {
      const int ch = tid + i * kPfThreads;
      const int r = ch >> 3, c = ch & 7;
      a_src[i] = (size_t)(row0 + min(r, M - 1)) * I + c * 16;
      a_dst[i] = swz(r, c);
    }
    const float* sa_src = cs.scale + (size_t)(row0 + min(tid, M - 1)) * KB;

    const uint8_t* wexp = pb.w2 + (size_t)e * H * I;
    const uint8_t* brow[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int h = wave_on ? h0 + 16 * j + lr : 0;
      brow[j] = wexp + (size_t)h * I + kg * 32;
    }
    const float* s_row = pb.s2 + ((size_t)e * (H / kBlock) + (wave_on ? h0 : 0) / kBlock) * KB;

    v4f acc[MS][4];
#pragma unroll
    for (int ms = 0; ms < MS; ms++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[ms][j] = v4f{0.f, 0.f, 0.f, 0.f};

    v4i qreg[kMaxTerms][ACH];
    float sareg = 0.f;
    int np = planes_for(0);
#pragma unroll
    for (int k = 0; k < kMaxTerms; k++)
      if (k < np)
#pragma unroll
        for (int i = 0; i < ACH; i++) qreg[k][i] = *reinterpret_cast<const v4i*>(cs.q + (size_t)k * cs.plane + a_src[i]);
    if (tid < BM) sareg = sa_src[0];
#pragma unroll
    for (int k = 0; k < kMaxTerms; k++)
      if (k < np)
#pragma unroll
        for (int i = 0; i < ACH; i++) *reinterpret_cast<v4i*>(&a_lds[0][k][a_dst[i]]) = qreg[k][i];
    if (tid < BM) sa_lds[0][tid] = sareg;
    v8i bcur[4];
#pragma unroll
    for (int j = 0; j < 4; j++) bcur[j] = wave_on ? load_v8i_g(brow[j]) : v8i{0, 0, 0, 0, 0, 0, 0, 0};
    __syncthreads();

    for (int kb = 0; kb < KB; kb++) {
      const int st = kb & 1;
      const bool more = kb + 1 < KB;
      v8i bnxt[4];
      int np_next = 0;
      if (more) {
        const size_t koff = (size_t)(kb + 1) * kBlock;
        np_next = planes_for(kb + 1);
#pragma unroll
        for (int k = 0; k < kMaxTerms; k++)
          if (k < np_next)
#pragma unroll
            for (int i = 0; i < ACH; i++)
              qreg[k][i] = *reinterpret_cast<const v4i*>(cs.q + (size_t)k * cs.plane + a_src[i] + koff);
        if (tid < BM) sareg = sa_src[kb + 1];
#pragma unroll
        for (int j = 0; j < 4; j++)
          bnxt[j] = wave_on ? load_v8i_g(brow[j] + koff) : v8i{0, 0, 0, 0, 0, 0, 0, 0};
      }
      const float sw = s_row[kb];
#pragma unroll
      for (int ms = 0; ms < MS; ms++) {
        const int nk = kmax[ms * KB + kb];
        const v4f sa_x = *reinterpret_cast<const v4f*>(&sa_lds[st][ms * 16 + kg * 4]);
        if (nk == kExactTerms) {
          // exact-product sub-tile: f16 hi/lo split of C from global, W2 widened to f16
          const size_t g = (size_t)(row0 + min(ms * 16 + lr, M - 1)) * I + kb * kBlock + kg * 32;
          v8h ah[4], al[4];
#pragma unroll
          for (int s4 = 0; s4 < 4; s4++) {
            ah[s4] = *reinterpret_cast<const v8h*>(cs.c16 + g + 8 * s4);
            al[s4] = *reinterpret_cast<const v8h*>(cs.c16 + cs.plane + g + 8 * s4);
          }
#pragma unroll
          for (int j = 0; j < 4; j++) {
            v8h b16[4];
            widen_fp8_operand(bcur[j], b16);
            v4f p = mfma_f16_block(ah, b16, v4f{0.f, 0.f, 0.f, 0.f});
            p = mfma_f16_block(al, b16, p);
#pragma unroll
            for (int r = 0; r < 4; r++) acc[ms][j][r] += p[r] * (sa_x[r] * sw);
          }
          continue;
        }
        v8i aq[kMaxTerms];
#pragma unroll
        for (int k = 0; k < kMaxTerms; k++)
          if (k < nk) aq[k] = lds_a_operand(a_lds[st][k], ms, lr, kg);
        const v4f sa = *reinterpret_cast<const v4f*>(&sa_lds[st][ms * 16 + kg * 4]);
#pragma unroll
        for (int j = 0; j < 4; j++) {
          v4f p = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int k = 0; k < kMaxTerms; k++)
            if (k < nk) p = mfma16x16x128_term(aq[k], bcur[j], p, k);
#pragma unroll
          for (int r = 0; r < 4; r++) acc[ms][j][r] += p[r] * (sa[r] * sw);
        }
      }
      if (more) {
#pragma unroll
        for (int k = 0; k < kMaxTerms; k++)
          if (k < np_next)
#pragma unroll
            for (int i = 0; i < ACH; i++) *reinterpret_cast<v4i*>(&a_lds[st ^ 1][k][a_dst[i]]) = qreg[k][i];
        if (tid < BM) sa_lds[st ^ 1][tid] = sareg;
#pragma unroll
        for (int j = 0; j < 4; j++) bcur[j] = bnxt[j];
      }
      __syncthreads();
    }

    if (wave_on) {
#pragma unroll
      for (int ms = 0; ms < MS; ms++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
          const int row = ms * 16 + kg * 4 + r;
          if (row < M) {
            const int p = row0 + row;
            const float w = pl.perm_w[p];
            float* dst = obuf + (size_t)p * H + h0 + lr;
#pragma unroll
            for (int j = 0; j < 4; j++) dst[16 * j] = acc[ms][j][r] * w;
          }
        }
    }
  }
}

// Workgroup = (token, 1024 columns): fixed ascending-expert sum of the token's pair rows from
// zero (the index_add_ order of main.py:241), bf16 RNE (main.py:243); zero rows for tokens
// without a local expert.
constexpr int kCombineCols = 1024;

__global__ __launch_bounds__(256) void combine_kernel(const int* __restrict__ tok_slot,
                                                      const int* __restrict__ info,
                                                      const float* __restrict__ obuf,
                                                      uint16_t* __restrict__ out, int H) {
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
      v[k] = slots[k] >= 0 ? *reinterpret_cast<const float4*>(obuf + (size_t)slots[k] * H + c)
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
      const float* row = obuf + (size_t)slots[k] * S * H + c;
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
  uint2 o;
  o.x = (uint32_t)f32_to_bf16_rne(acc.x) | ((uint32_t)f32_to_bf16_rne(acc.y) << 16);
  o.y = (uint32_t)f32_to_bf16_rne(acc.z) | ((uint32_t)f32_to_bf16_rne(acc.w) << 16);
  *reinterpret_cast<uint2*>(out + (size_t)t * H + c) = o;
}

template <int BM>
static void launch_g1(const Problem& pb, const Plan& pl, const CSplit& cs, int grid, hipStream_t stream) {
  hipLaunchKernelGGL(gemm1_prefill_kernel<BM>, dim3(grid), dim3(kPfThreads), 0, stream, pb, pl, cs);
}

template <int BM>
static void launch_g2(const Problem& pb, const Plan& pl, const CSplit& cs, float* obuf, int grid,
                      hipStream_t stream) {
  hipLaunchKernelGGL(gemm2_prefill_kernel<BM>, dim3(grid), dim3(kPfThreads), 0, stream, pb, pl, cs, obuf);
}

static int persistent_grid(int max_tiles) {
  const int cap = num_compute_units() * 2;
  return max_tiles < cap ? max_tiles : cap;
}

void launch_gemm1_prefill(const Problem& pb, const Plan& pl, int tile_m, const CSplit& cs, int max_mtiles,
                          hipStream_t stream) {
  const int grid = persistent_grid(max_mtiles * (pb.I / kBlock));
  if (grid <= 0) return;
  switch (tile_m) {
    case 32: launch_g1<32>(pb, pl, cs, grid, stream); break;
    case 64: launch_g1<64>(pb, pl, cs, grid, stream); break;
    default: launch_g1<128>(pb, pl, cs, grid, stream); break;
  }
}

void launch_gemm2_prefill(const Problem& pb, const Plan& pl, int tile_m, const CSplit& cs, float* obuf,
                          int max_mtiles, hipStream_t stream) {
  const int grid = persistent_grid(max_mtiles * ((pb.H + 255) / 256));
  if (grid <= 0) return;
  switch (tile_m) {
    case 32: launch_g2<32>(pb, pl, cs, obuf, grid, stream); break;
    case 64: launch_g2<64>(pb, pl, cs, obuf, grid, stream); break;
    default: launch_g2<128>(pb, pl, cs, obuf, grid, stream); break;
  }
}

void launch_combine(const Plan& pl, const float* obuf, uint16_t* out, int T, int H, hipStream_t stream) {
  if (T <= 0) return;
  hipLaunchKernelGGL(combine_kernel, dim3(T, (H + kCombineCols - 1) / kCombineCols), dim3(256), 0, stream,
                     pl.tok_slot, pl.info, obuf, out, H);
}

}  // namespace moefp8
