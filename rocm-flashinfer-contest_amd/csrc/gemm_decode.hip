// Small-T expert GEMMs (T <= 64): balanced weight streams on MFMA.
//
// With a few tokens per expert the work is reading each active expert's weights once
// (HBM bound), so both GEMMs are built around one balanced, fully resident round of
// weight streams.  A workgroup unit is (m-tile, K-slice, 4 consecutive 16-column groups);
// each of its 4 wavefronts streams the 16 weight rows of its column group through a
// register ring (several K-blocks of loads in flight) and keeps its 16 x 16 accumulator
// in registers.  The activation tile of the m-tile is the same for the 4 wavefronts, so
// it is loaded once per workgroup: each K step a few carrier wavefronts fetch one piece
// of the activation block and its 16 row scales and publish them through LDS.
// Per-wavefront activation loads from global memory cost the weight stream about a
// third of its bandwidth on this chip (measured); sharing them through LDS removes it.
//
// A persistent grid sized to the resident capacity walks the units.  The K-split S of
// each GEMM (chosen by the permutation kernel from the m-tile count) is the largest that
// still fits the grid, so a handful of active experts still spreads over every CU; the S
// partial sums go to separate rows and the next stage adds them in ascending order.
//
// GEMM1       G1 partials = A_e W13_e^T over a K-slice                  (main.py:229-231);
//             the last unit to finish a (m-tile, 128 C columns) group then forms
//             C = silu(sum_s G1[:, I:]) * sum_s G1[:, :I]              (main.py:232-233),
//             stored as f16 hi + lo with one fp32 scale per (pair, 128 columns)
// GEMM2       O partials = routing weight * C W2_e^T over a K-slice   (main.py:234-241),
//             exact products of C's f16 hi term (2^-11 relative) and W2 widened to f16;
//             the last unit to finish a 64-column block then sums each token's pair rows
//             and splits over those columns into the bf16 output   (main.py:241-243).
// M-tiles flagged for exact products (GEMM1) or for both f16 terms of C (GEMM2) take a
// simpler per-wavefront path.
#include "decode_plan.h"
#include "moefp8_device.h"
#include "moefp8_launch.h"

namespace moefp8 {

constexpr int kDecBlockWaves = 4;            // wavefronts per workgroup = column groups per unit
constexpr int kDec1BlocksPerCU = 5;          // GEMM1 resident workgroups per CU (<= 96 VGPRs)
constexpr int kDec2BlocksPerCU = 5;          // GEMM2 too (<= 96 VGPRs: its per-step path keeps a
                                             // shallower ring; a scratch spill there cost ~20% of
                                             // the kernel's time, measured)
constexpr int kDecDepth = 3;                 // K-blocks in flight per wavefront (register ring)
static_assert(64 * kDecBlockWaves == kPlanThreads, "the GEMM1 workgroups build the plan");

// One 16-byte chunk of a weight line.  Each weight byte is read once per call and each 128-byte
// line by one load instruction (8 lanes), so the load carries the non-temporal hint (streamed
// through L2): 5% less time per call at 16 tokens, measured.  On loads that split a line over two
// instructions (the MFMA layout, 16 rows x 64 bytes) the hint evicts it in between (16% more time
// at 64 tokens, measured), so every weight stream loads whole lines.
__device__ __forceinline__ v4i load_w_line(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const v4i*>(p));
}

__device__ __forceinline__ v8i load_v8i(const uint8_t* p) {
  const v4i* q = reinterpret_cast<const v4i*>(p);
  const v4i x = q[0], y = q[1];
  return __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ void load_v8h4(const _Float16* p, v8h (&y)[4]) {
  const v8h* q = reinterpret_cast<const v8h*>(p);
#pragma unroll
  for (int i = 0; i < 4; i++) y[i] = q[i];
}

// Unit u -> (m-tile g, K-split s, column block cb of 4 groups), column block fastest.
struct DecUnit {
  int g, s, cb;
};
__device__ __forceinline__ DecUnit decode_unit(int u, int S, int NCB) {
  const int rest = u / NCB;
  return DecUnit{rest / S, rest % S, u - rest * NCB};
}

// LDS stage of GEMM1: 16 activation rows x 128 e4m3 bytes (chunk c of row r in slot
// c ^ slot_key8(r)) and the 16 row scales.
struct alignas(16) G1Stage {
  uint8_t a[16 * kBlock];
  float sa[16];
};

// Activation rows of an m-tile with at most kPreRows rows, staged once per unit for its
// whole K-range (<= kPreMaxKB K-blocks) with their scales: the weight stream then runs
// without a barrier per K step.  In decode most m-tiles hold one or two pairs.  Rows are
// padded (GEMM1 80 bytes, GEMM2 16) so that the operand reads of the <= 4 rows (GEMM1: 32
// bytes per lane group, GEMM2: 64) fall on distinct 16-byte bank groups whether the LDS serves
// 8, 16 or 32 lanes at a time.
constexpr int kPreRows = 4;
constexpr int kPre1RowBytes = kPreMaxKB * kBlock + 80;
struct alignas(16) G1Pre {
  uint8_t a[kPreRows * kPre1RowBytes];
  float sa[kPreMaxKB][kPreRows];
};

// GEMM2's staged rows: C's f16 hi term, <= kPre2MaxKB K-blocks of 128 columns per unit.
constexpr int kPre2RowBytes = kPre2MaxKB * kBlock * 2 + 16;
struct alignas(16) G2Pre {
  uint8_t a[kPreRows * kPre2RowBytes];
  float sa[kPre2MaxKB][kPreRows];
};

// LDS stage of GEMM2: 16 rows of C's f16 hi term x 128 columns (256 bytes, chunk c of row r in
// slot c ^ slot_key16(r)) and the 16 row scales.
struct alignas(16) G2Stage {
  uint8_t a[16 * 2 * kBlock];
  float sa[16];
};

// Steady state of both GEMMs, K step j: the carrier wavefronts write the activation piece
// of step j (loaded kDecDepth steps earlier) into LDS stage j & 1, the workgroup
// barrier publishes it, every wavefront computes step j from LDS and its own weight
// registers, then loads its pieces of step j + kDecDepth.  A stage is rewritten two
// steps after it was read, i.e. after the barrier that follows every wavefront's read.

// Partial sums that another workgroup of the same launch reads (possibly on another XCD,
// whose L2 is not coherent with this one's) are stored and loaded at device scope: the
// stores write through to the device-coherent level and the loads read from it, so no
// cache-wide fence is needed (a device-scope fence writes back and invalidates the whole
// L2; one per unit multiplied GEMM1's time by 5, measured).
__device__ __forceinline__ void store_shared_f32(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 load_shared_f32x2(const float* p) {
  return __builtin_bit_cast(float2, __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT));
}
// Counts one more arrival at *counter once this workgroup's device-scope stores are
// complete; true in every thread of the workgroup that arrived last of `expected`.
__device__ __forceinline__ bool arrive_last(int* counter, int expected, int* flag_s) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0)
    *flag_s = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == expected - 1;
  __syncthreads();
  return *flag_s;
}

// SwiGLU of pair p's C columns [128 cb, 128 cb + 128) by one wavefront: sums the GEMM1
// partials of the S K-splits in split order, applies silu(gate) * up and writes C as two
// f16 terms with one scale (max |C| -> 448).  The block's max |C| against the pair's routing
// weight w and its expert's W2 scale sigma2 decides whether GEMM2 needs both terms in this m-tile
// (needs_two_terms): *two_term is then set.
__device__ __forceinline__ void swiglu_block(int I, int S, int p, int cb, const float* __restrict__ gbuf,
                                             const CHalf& ch, float w, float sigma2, int* two_term) {
  constexpr int kBatch = 8;   // partial loads issued together
  const int CB = I / kBlock, I2 = 2 * I;
  const int lane = lane_id();
  const int c = cb * kBlock + 2 * lane;
  float2 up = {0.f, 0.f}, gate = {0.f, 0.f};
  for (int s0 = 0; s0 < S; s0 += kBatch) {
    float2 u[kBatch], g[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; q++) {
      const int s = min(s0 + q, S - 1);
      const float* row = gbuf + ((size_t)p * S + s) * I2;
      u[q] = load_shared_f32x2(row + c);
      g[q] = load_shared_f32x2(row + I + c);
    }
#pragma unroll
    for (int q = 0; q < kBatch; q++) {
      if (s0 + q < S) {
        up.x += u[q].x;
        up.y += u[q].y;
        gate.x += g[q].x;
        gate.y += g[q].y;
      }
    }
  }
  const float c0 = silu_f32(gate.x) * up.x, c1 = silu_f32(gate.y) * up.y;
  const float amax = wave_max_f32(fmaxf(fabsf(c0), fabsf(c1)));
  if (lane == 0 && needs_two_terms(w, sigma2, amax, sqrtf((float)I))) atomicOr(two_term, 1);
  float inv, scale;
  split_scale(amax, inv, scale);
  _Float16 h0, l0, h1, l1;
  split_f16(c0, inv, h0, l0);
  split_f16(c1, inv, h1, l1);
  *reinterpret_cast<v2h*>(ch.hi + (size_t)p * I + c) = v2h{h0, h1};
  *reinterpret_cast<v2h*>(ch.lo + (size_t)p * I + c) = v2h{l0, l1};
  if (lane == 0) ch.scale[(size_t)p * CB + cb] = scale;
}

__global__ __launch_bounds__(64 * kDecBlockWaves, kDec1BlocksPerCU) void gemm1_decode_kernel(Problem pb, Plan pl,
                                                                                             DecodePlanArgs da,
                                                                                             float* __restrict__ gbuf,
                                                                                             CHalf ch) {
  // the plan's build scratch, the per-step ring and the staged rows are never live together
  __shared__ union {
    DecodePlanScratch plan_x;
    G1Stage ring[2];
    G1Pre pre;
  } sh;
  __shared__ DecodePlanLds plan;
  __shared__ int last_s;
  // per-wavefront weight transpose buffers of the staged path (16 rows x 128 bytes)
  __shared__ __attribute__((aligned(16))) uint8_t wtr[kDecBlockWaves][16 * kBlock];
  G1Stage* ring = sh.ring;
  build_decode_plan(da, plan, sh.plan_x, blockIdx.x == 0);
  const int n_mt = plan.n_mt, S = plan.S1;
  const int H = pb.H, I = pb.I, I2 = 2 * pb.I, T = pb.T;
  const int KB = H / kBlock, NCB = I2 / (16 * kDecBlockWaves);
  const int n_units = n_mt * S * NCB;
  const int wave = wave_index();

  for (int u = blockIdx.x; u < n_units; u += gridDim.x) {
    // lane-dependent addresses are formed per unit: hoisted in front of the loop they stay
    // live across all three paths and spill
    int lane = lane_id();
    asm volatile("" : "+v"(lane));
    const int lr = lane & 15, kg = lane >> 4;
    const DecUnit du = decode_unit(u, S, NCB);
    const int4 mt = plan.mt[du.g];
    const int e = uniform(mt.x), row0 = uniform(mt.y), M = uniform(mt.z), flags = uniform(mt.w);
    const int kb0 = du.s * KB / S, n = (du.s + 1) * KB / S - kb0;
    const int cg = du.cb * kDecBlockWaves + wave;
    // W13 row cg*16 + lr (columns [0, I) are "up", [I, 2I) "gate"); lane reads k-group kg
    const uint8_t* bp = pb.w13 + ((size_t)e * I2 + cg * 16 + lr) * H + (size_t)kb0 * kBlock + kg * 32;
    const float* swp = pb.s13 + ((size_t)e * (I2 / kBlock) + (cg * 16) / kBlock) * KB + kb0;
    // rows >= M repeat the m-tile's first pair (real data, results discarded)
    const int tok = clamp_index(plan.tok[row0 + (lr < M ? lr : 0)], T);
    v4f acc = {0.f, 0.f, 0.f, 0.f};

    if (!(flags & kFlagExactProducts) && M <= kPreRows && n <= kPreMaxKB) {
      const float swv = swp[min(lane, n - 1)];
      // weights as whole 128-byte lines: lane l loads 16-byte chunk l%8 of rows l/8 and
      // 8 + l/8 of each K-block, then the wavefront transposes the block through its LDS
      // buffer into the MFMA layout (16 rows x 64 bytes per load instruction in that layout
      // streams ~7% slower, measured).  Chunk c of row r sits at slot c ^ slot_key8(r).
      const int wr = lane >> 3, wc = lane & 7;
      const uint8_t* wsrc = pb.w13 + ((size_t)e * I2 + cg * 16 + wr) * H + (size_t)kb0 * kBlock + wc * 16;
      uint8_t* const tb = wtr[wave];
      uint8_t* const tw0 = tb + wr * kBlock + (wc ^ slot_key8(wr)) * 16;
      uint8_t* const tw1 = tb + (wr + 8) * kBlock + (wc ^ slot_key8(wr + 8)) * 16;
      const uint8_t* const trx = tb + lr * kBlock + ((2 * kg) ^ slot_key8(lr)) * 16;
      const uint8_t* const try_ = tb + lr * kBlock + ((2 * kg + 1) ^ slot_key8(lr)) * 16;
      v4i B0[kDecDepth], B1[kDecDepth];
      auto load = [&](int d, int j) {
        const uint8_t* p = wsrc + (size_t)min(j, n - 1) * kBlock;
        B0[d] = load_w_line(p);
        B1[d] = load_w_line(p + (size_t)8 * H);
      };
#pragma unroll
      for (int d = 0; d < kDecDepth; d++) load(d, d);
      {
        // rows [0, M) x K-blocks [kb0, kb0 + n) in 16-byte chunks (<= 4 per thread), then the
        // M x n scales (<= 128), all loads issued before the first store
        constexpr int kChunks = kPreRows * kPreMaxKB * (kBlock / 16);
        constexpr int kPer = (kChunks + 64 * kDecBlockWaves - 1) / (64 * kDecBlockWaves);
        static_assert(kPer * 64 * kDecBlockWaves >= kChunks, "every staged chunk has a thread");
        const int nch = M * n * (kBlock / 16);
        v4i v[kPer];
#pragma unroll
        for (int q = 0; q < kPer; q++) {
          const int i = min((int)threadIdx.x + q * 64 * kDecBlockWaves, nch - 1);
          const int r = i / (n * 8), c = i - r * n * 8;
          v[q] = *reinterpret_cast<const v4i*>(pb.hidden + (size_t)clamp_index(plan.tok[row0 + r], T) * H +
                                               (size_t)kb0 * kBlock + c * 16);
        }
        const int si = min((int)threadIdx.x, M * n - 1), sr = si / n, sj = si - sr * n;
        const float sv = pb.hscale[(size_t)(kb0 + sj) * T + clamp_index(plan.tok[row0 + sr], T)];
#pragma unroll
        for (int q = 0; q < kPer; q++) {
          const int i = threadIdx.x + q * 64 * kDecBlockWaves;
          const int r = i / (n * 8), c = i - r * n * 8;
          if (i < nch) *reinterpret_cast<v4i*>(sh.pre.a + r * kPre1RowBytes + c * 16) = v[q];
        }
        if ((int)threadIdx.x < M * n) sh.pre.sa[sj][sr] = sv;
        __syncthreads();
      }
      // rows >= M read row M - 1 (real data, results discarded)
      const uint8_t* arow = sh.pre.a + min(lr, M - 1) * kPre1RowBytes + kg * 32;
      auto step = [&](int d, int j) {
        *reinterpret_cast<v4i*>(tw0) = B0[d];
        *reinterpret_cast<v4i*>(tw1) = B1[d];
        const v4i bx = *reinterpret_cast<const v4i*>(trx);
        const v4i by = *reinterpret_cast<const v4i*>(try_);
        const v4i x = *reinterpret_cast<const v4i*>(arow + j * kBlock);
        const v4i y = *reinterpret_cast<const v4i*>(arow + j * kBlock + 16);
        const float4 sa = *reinterpret_cast<const float4*>(sh.pre.sa[j]);   // rows 0..3 (lanes kg = 0)
        const float sw = readlane_f32(swv, j);
        const v4f p = mfma16x16x128(__builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7),
                                    __builtin_shufflevector(bx, by, 0, 1, 2, 3, 4, 5, 6, 7),
                                    v4f{0.f, 0.f, 0.f, 0.f});
        acc[0] += p[0] * (sa.x * sw);
        acc[1] += p[1] * (sa.y * sw);
        acc[2] += p[2] * (sa.z * sw);
        acc[3] += p[3] * (sa.w * sw);
      };
      int j = 0;
      for (; j + kDecDepth <= n; j += kDecDepth) {
#pragma unroll
        for (int d = 0; d < kDecDepth; d++) {
          step(d, j + d);
          load(d, j + d + kDecDepth);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
#pragma unroll
      for (int d = 0; d < kDecDepth - 1; d++)
        if (j + d < n) step(d, j + d);
      // the next unit restages only after every wavefront has read this one's rows
      __syncthreads();
    } else if (!(flags & kFlagExactProducts)) {
      constexpr int kStepDepth = 2;   // (register budget shared with the staged path)
      // carriers: waves 0/1 load rows 8q .. 8q + 7 of the activation block as whole 128-byte
      // lines (lane l: row 8q + l/8, 16-byte chunk l%8) and publish them to the stage; wave 0's
      // lanes < 16 publish the scale of row lane.  Waves 2/3 issue as many loads, from one
      // fixed line (loads under a branch would make the compiler's wait counting fall back to
      // draining all of them).  Activation loads in the MFMA layout by every wavefront (16
      // rows x 64 bytes per instruction) cost the weight stream ~20% (measured).
      const int ar = 8 * (wave & 1) + (lane >> 3);
      const int atok = clamp_index(plan.tok[row0 + (ar < M ? ar : 0)], T);
      const uint8_t* asrc =
          wave < 2 ? pb.hidden + (size_t)atok * H + (size_t)kb0 * kBlock + (lane & 7) * 16 : pb.hidden;
      const int astep = wave < 2 ? kBlock : 0;
      const float* ssrc = pb.hscale + (size_t)kb0 * T + tok;
      // weight scale of K-block kb0 + l in lane l (n <= 64), read per step with readlane
      const float swv = swp[min(lane, n - 1)];
      // weights as whole lines with the non-temporal hint, transposed per wavefront through its LDS
      // buffer tb as on the staged path (MFMA-layout loads instead: 184.8 against 173.9 us per call
      // at T = 64, both GEMMs, measured).  Chunk c of row r sits at r * 128 + (c ^ slot_key8(r)) * 16,
      // so row wr + 8's chunk is at (tw0o ^ 16) + 1024 and chunk 2kg + 1 of row lr at trxo ^ 16
      // (slot_key8(r + 8) = slot_key8(r) ^ 1 for r < 8): two offsets kept instead of four
      const int wr = lane >> 3, wc = lane & 7;
      const uint8_t* wsrc = pb.w13 + ((size_t)e * I2 + cg * 16 + wr) * H + (size_t)kb0 * kBlock + wc * 16;
      uint8_t* const tb = wtr[wave];
      const int tw0o = wr * kBlock + (wc ^ slot_key8(wr)) * 16;
      const int trxo = lr * kBlock + ((2 * kg) ^ slot_key8(lr)) * 16;
      v4i B0[kStepDepth], B1[kStepDepth];
      v4i AR[kStepDepth];
      float SR[kStepDepth];
      auto load = [&](int d, int j) {
        const int jj = min(j, n - 1);
        B0[d] = load_w_line(wsrc + (size_t)jj * kBlock);
        B1[d] = load_w_line(wsrc + (size_t)jj * kBlock + (size_t)8 * H);
        AR[d] = *reinterpret_cast<const v4i*>(asrc + (size_t)jj * astep);
        SR[d] = ssrc[(size_t)jj * T];
      };
      auto step = [&](int d, int j) {
        G1Stage& st = ring[j & 1];
        if (wave < 2) *reinterpret_cast<v4i*>(st.a + ar * kBlock + ((lane & 7) ^ slot_key8(ar)) * 16) = AR[d];
        if (wave == 0 && lane < 16) st.sa[lane] = SR[d];
        // (formed per step: four live offsets spilled at the 96-VGPR budget)
        int t0 = tw0o, t1 = trxo;
        asm volatile("" : "+v"(t0), "+v"(t1));
        *reinterpret_cast<v4i*>(tb + t0) = B0[d];
        *reinterpret_cast<v4i*>(tb + ((t0 ^ 16) + 1024)) = B1[d];
        __syncthreads();
        const v4i bx = *reinterpret_cast<const v4i*>(tb + t1);
        const v4i by = *reinterpret_cast<const v4i*>(tb + (t1 ^ 16));
        const v4i x = *reinterpret_cast<const v4i*>(st.a + lr * kBlock + ((2 * kg) ^ slot_key8(lr)) * 16);
        const v4i y = *reinterpret_cast<const v4i*>(st.a + lr * kBlock + ((2 * kg + 1) ^ slot_key8(lr)) * 16);
        const float4 sa = *reinterpret_cast<const float4*>(st.sa + 4 * kg);
        const float sw = readlane_f32(swv, j);
        const v4f p = mfma16x16x128(__builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7),
                                    __builtin_shufflevector(bx, by, 0, 1, 2, 3, 4, 5, 6, 7),
                                    v4f{0.f, 0.f, 0.f, 0.f});
        acc[0] += p[0] * (sa.x * sw);
        acc[1] += p[1] * (sa.y * sw);
        acc[2] += p[2] * (sa.z * sw);
        acc[3] += p[3] * (sa.w * sw);
      };
#pragma unroll
      for (int d = 0; d < kStepDepth; d++) load(d, d);
      // full groups of kStepDepth steps (no early exit, so every prefetch stays where it is
      // written), then the remaining < kStepDepth steps from the ring without new loads
      int j = 0;
      for (; j + kStepDepth <= n; j += kStepDepth) {
#pragma unroll
        for (int d = 0; d < kStepDepth; d++) {
          step(d, j + d);
          load(d, j + d + kStepDepth);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
#pragma unroll
      for (int d = 0; d < kStepDepth - 1; d++)
        if (j + d < n) step(d, j + d);
      // the next unit writes stage 0 only after every wavefront has read this unit's last stage
      __syncthreads();
    } else {
      int tok_d[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int dr = 4 * kg + r;
        tok_d[r] = clamp_index(plan.tok[row0 + (dr < M ? dr : 0)], T);
      }
      const uint8_t* ap = pb.hidden + (size_t)tok * H + (size_t)kb0 * kBlock + kg * 32;
      for (int j = 0; j < n; j++) {
        const v8i b = load_v8i(bp + (size_t)j * kBlock);
        const v8i a = load_v8i(ap + (size_t)j * kBlock);
        float sa[4];
#pragma unroll
        for (int r = 0; r < 4; r++) sa[r] = pb.hscale[(size_t)(kb0 + j) * T + tok_d[r]];
        const float sw = swp[j];
        v8h a16[4], b16[4];
        widen_fp8_operand(a, a16);
        widen_fp8_operand(b, b16);
        const v4f p = mfma_f16_block(a16, b16, v4f{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int r = 0; r < 4; r++) acc[r] += p[r] * (sa[r] * sw);
      }
    }
    // D layout: lane holds rows 4*kg + r of column lr
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int row = 4 * kg + r;
      if (row < M) store_shared_f32(gbuf + ((size_t)(row0 + row) * S + du.s) * I2 + cg * 16 + lr, acc[r]);
    }
    // C columns [128 j, 128 j + 128) of the m-tile need the partials of 4 S units: column
    // blocks 2j, 2j + 1 ("up") and NCB/2 + 2j, NCB/2 + 2j + 1 ("gate"), S K-splits each.
    // Every unit publishes its partials and counts itself in; the last one forms C.  The pairs'
    // routing weights come from the plan in LDS, so after the arrival the last unit's one round
    // trip to memory is the partials (with the expert's W2 estimate, needed only at the end):
    // -0.6 / -1.0 / -0.35 / -1.5 us per call at T = 1 / 4 / 16 / 64 against reading them from
    // the routing outputs (measured).
    const int j = (du.cb % (NCB / 2)) / 2;
    if (arrive_last(pl.counters + (du.g * (I / kBlock) + j) * kCounterStride, 4 * S, &last_s)) {
      const float sigma2 = da.esig[2 * e + 1];
      for (int r = wave; r < M; r += kDecBlockWaves)
        swiglu_block(I, S, row0 + r, j, gbuf, ch, plan.w[row0 + r], sigma2, pl.two_term + du.g * kCounterStride);
    }
  }
}

// Combine of output columns [c0, c0 + 64) for every token by one workgroup (main.py:241-243):
// each token's pair rows in ascending local-expert order (tok_slot, here its copy in LDS), the
// K-split partials of a row first, summed from zero in fp32 and rounded once to bf16; tokens
// without a local expert get zeros.  Thread = (token, 4 columns).  Pair indices read from
// tok_slot are clamped below pair_rows (the call's pair count: rows pair_rows * S of the partials
// are written).
__device__ void combine_columns(const int* tok_slot_lds, const float* __restrict__ obuf,
                                void* __restrict__ out, int T, int H, int S, int c0, const void* shared,
                                int shared_dt, int out_f32, int pair_rows) {
  constexpr int kQuads = 16;                            // 4-column groups of the 64 columns
  const int c = c0 + 4 * (threadIdx.x % kQuads);
  for (int t = threadIdx.x / kQuads; t < T; t += blockDim.x / kQuads) {
    int slots[kTopK];
#pragma unroll
    for (int k = 0; k < kTopK; k++) slots[k] = tok_slot_lds[t * kTopK + k];
    float4 acc = {0.f, 0.f, 0.f, 0.f};
    if (S == 1) {
      // the token's (at most 8) rows loaded together; a token's unused slots are -1 and last
      float2 lo[kTopK], hi[kTopK];
#pragma unroll
      for (int k = 0; k < kTopK; k++) {
        const float* r = obuf + (size_t)clamp_index(max(slots[k], 0), pair_rows) * H + c;
        lo[k] = load_shared_f32x2(r);
        hi[k] = load_shared_f32x2(r + 2);
      }
#pragma unroll
      for (int k = 0; k < kTopK; k++) {
        if (slots[k] >= 0) {
          acc.x += lo[k].x;
          acc.y += lo[k].y;
          acc.z += hi[k].x;
          acc.w += hi[k].y;
        }
      }
    }
    for (int k = 0; S > 1 && k < kTopK; k++) {
      if (slots[k] < 0) break;
      const float* row = obuf + (size_t)clamp_index(slots[k], pair_rows) * S * H + c;
      float4 o = {0.f, 0.f, 0.f, 0.f};                 // the row's splits, in order
      for (int s0 = 0; s0 < S; s0 += kTopK) {
        float2 lo[kTopK], hi[kTopK];                    // up to 8 splits loaded together
#pragma unroll
        for (int q = 0; q < kTopK; q++) {
          const float* r = row + (size_t)min(s0 + q, S - 1) * H;
          lo[q] = load_shared_f32x2(r);
          hi[q] = load_shared_f32x2(r + 2);
        }
#pragma unroll
        for (int q = 0; q < kTopK; q++) {
          if (s0 + q == 0) {
            o = float4{lo[q].x, lo[q].y, hi[q].x, hi[q].y};
          } else if (s0 + q < S) {
            o.x += lo[q].x;
            o.y += lo[q].y;
            o.z += hi[q].x;
            o.w += hi[q].y;
          }
        }
      }
      acc.x += o.x;
      acc.y += o.y;
      acc.z += o.z;
      acc.w += o.w;
    }
    if (shared) add_shared4(acc, shared, shared_dt, (size_t)t * H + c);
    store_out4(out, (size_t)t * H + c, acc, out_f32);
  }
}

__global__ __launch_bounds__(64 * kDecBlockWaves, kDec2BlocksPerCU) void gemm2_decode_kernel(Problem pb, Plan pl,
                                                                                             CHalf ch,
                                                                                             float* __restrict__ obuf,
                                                                                             void* __restrict__ out) {
  __shared__ union {
    G2Stage ring[2];
    G2Pre pre;
  } sh;
  __shared__ int last_s;
  // per-wavefront weight transpose buffers of the staged path (16 rows x 128 bytes)
  __shared__ __attribute__((aligned(16))) uint8_t wtr[kDecBlockWaves][16 * kBlock];
  // every token's pair rows (tok_slot) for the combine
  __shared__ __attribute__((aligned(16))) int slot_s[kSmallT * kTopK];
  G2Stage* ring = sh.ring;
  const int n_mt = pl.info[2], S = pl.info[4];
  const int H = pb.H, I = pb.I, T = pb.T;
  const int KB = I / kBlock, HB = H / kBlock, NCB = H / (16 * kDecBlockWaves);
  const int n_units = n_mt * S * NCB;
  const int wave = wave_index();
  if (n_units == 0) {
    // no local pairs: every output row is zero (plus the shared row)
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < (size_t)T * H / 4;
         i += (size_t)gridDim.x * blockDim.x) {
      float4 acc = {0.f, 0.f, 0.f, 0.f};
      if (pl.shared) add_shared4(acc, pl.shared, pl.shared_dt, 4 * i);
      store_out4(out, 4 * i, acc, pl.out_f32);
    }
    return;
  }

  // tok_slot (T x 8 ints, <= 2 KB) copied into LDS by DMA (waves 0 and 1, 1 KB each), issued
  // before the first unit: nothing waits for it until a combine, which follows the arrival's wait
  // for all of the workgroup's memory operations and a barrier, so the last unit of a column
  // block goes straight to the pair rows (one round trip less per combine pass).  The oldest
  // operation in flight, it only makes the waits of the compiler's own loads more conservative
  // until it lands.
  if ((int)blockIdx.x < n_units && wave * kWave * 4 < T * kTopK) {
    const uint32_t bytes = (uint32_t)(T * kTopK * 4);
    const uint32_t off = min((uint32_t)(wave * kWave + lane_id()) * 16u, bytes - 16u);
    dma_lds16_s(off, pl.tok_slot, uniform((int)lds_addr(slot_s)) + (uint32_t)(wave * kWave * 16));
  }

  for (int u = blockIdx.x; u < n_units; u += gridDim.x) {
    // lane-dependent addresses are formed per unit (hoisted, they stay live across all paths)
    int lane = lane_id();
    asm volatile("" : "+v"(lane));
    const int lr = lane & 15, kg = lane >> 4;
    const DecUnit du = decode_unit(u, S, NCB);
    // the m-tile and GEMM1's measured flag loaded together (not the flag behind the tile's test)
    const int measured = pl.two_term[du.g * kCounterStride];
    const int4 mt = pl.mtiles[du.g];
    const int e = uniform(mt.x), row0 = uniform(mt.y), M = uniform(mt.z);
    // both f16 terms of C: predicted (the plan), or measured by GEMM1
    const bool two = ((uniform(mt.w) & kFlagTwoTermC) | uniform(measured)) != 0;
    const int kb0 = du.s * KB / S, n = (du.s + 1) * KB / S - kb0;
    const int cg = du.cb * kDecBlockWaves + wave;
    const uint8_t* bp = pb.w2 + ((size_t)e * H + cg * 16 + lr) * I + (size_t)kb0 * kBlock + kg * 32;
    const float* swp = pb.s2 + ((size_t)e * HB + (cg * 16) / kBlock) * KB + kb0;
    const int prow = row0 + (lr < M ? lr : 0);
    v4f acc = {0.f, 0.f, 0.f, 0.f};

    if (!two && M <= kPreRows && n <= kPre2MaxKB) {
      const float swv = swp[min(lane, n - 1)];
      // weights as whole lines, transposed per wavefront through LDS (as in GEMM1)
      const int wr = lane >> 3, wc = lane & 7;
      const uint8_t* wsrc = pb.w2 + ((size_t)e * H + cg * 16 + wr) * I + (size_t)kb0 * kBlock + wc * 16;
      uint8_t* const tb = wtr[wave];
      uint8_t* const tw0 = tb + wr * kBlock + (wc ^ slot_key8(wr)) * 16;
      uint8_t* const tw1 = tb + (wr + 8) * kBlock + (wc ^ slot_key8(wr + 8)) * 16;
      const uint8_t* const trx = tb + lr * kBlock + ((2 * kg) ^ slot_key8(lr)) * 16;
      const uint8_t* const try_ = tb + lr * kBlock + ((2 * kg + 1) ^ slot_key8(lr)) * 16;
      v4i B0[kDecDepth], B1[kDecDepth];
      auto load = [&](int d, int j) {
        const uint8_t* p = wsrc + (size_t)min(j, n - 1) * kBlock;
        B0[d] = load_w_line(p);
        B1[d] = load_w_line(p + (size_t)8 * I);
      };
#pragma unroll
      for (int d = 0; d < kDecDepth; d++) load(d, d);
      {
        // rows [0, M) x K-blocks [kb0, kb0 + n) of C's hi term in 16-byte chunks (<= 4 per
        // thread), then the M x n scales, all loads issued before the first store
        constexpr int kChunksPerKB = kBlock * 2 / 16;
        constexpr int kChunks = kPreRows * kPre2MaxKB * kChunksPerKB;
        constexpr int kPer = (kChunks + 64 * kDecBlockWaves - 1) / (64 * kDecBlockWaves);
        static_assert(kPer * 64 * kDecBlockWaves >= kChunks, "every staged chunk has a thread");
        const int nch = M * n * kChunksPerKB;
        v4i v[kPer];
#pragma unroll
        for (int q = 0; q < kPer; q++) {
          const int i = min((int)threadIdx.x + q * 64 * kDecBlockWaves, nch - 1);
          const int r = i / (n * kChunksPerKB), c = i - r * n * kChunksPerKB;
          v[q] = *reinterpret_cast<const v4i*>(ch.hi + (size_t)(row0 + r) * I + (size_t)kb0 * kBlock + c * 8);
        }
        const int si = min((int)threadIdx.x, M * n - 1), sr = si / n, sj = si - sr * n;
        const float sv = ch.scale[(size_t)(row0 + sr) * KB + kb0 + sj];
#pragma unroll
        for (int q = 0; q < kPer; q++) {
          const int i = threadIdx.x + q * 64 * kDecBlockWaves;
          const int r = i / (n * kChunksPerKB), c = i - r * n * kChunksPerKB;
          if (i < nch) *reinterpret_cast<v4i*>(sh.pre.a + r * kPre2RowBytes + c * 16) = v[q];
        }
        if ((int)threadIdx.x < M * n) sh.pre.sa[sj][sr] = sv;
        __syncthreads();
      }
      // rows >= M read row M - 1 (real data, results discarded)
      const uint8_t* arow = sh.pre.a + min(lr, M - 1) * kPre2RowBytes + kg * 64;
      auto step = [&](int d, int j) {
        *reinterpret_cast<v4i*>(tw0) = B0[d];
        *reinterpret_cast<v4i*>(tw1) = B1[d];
        const v4i bx = *reinterpret_cast<const v4i*>(trx);
        const v4i by = *reinterpret_cast<const v4i*>(try_);
        v8h ah[4];
#pragma unroll
        for (int t = 0; t < 4; t++) ah[t] = *reinterpret_cast<const v8h*>(arow + j * (2 * kBlock) + t * 16);
        const float4 sa = *reinterpret_cast<const float4*>(sh.pre.sa[j]);   // rows 0..3 (lanes kg = 0)
        const float sw = readlane_f32(swv, j);
        v8h b16[4];
        widen_fp8_operand(__builtin_shufflevector(bx, by, 0, 1, 2, 3, 4, 5, 6, 7), b16);
        const v4f p = mfma_f16_block(ah, b16, v4f{0.f, 0.f, 0.f, 0.f});
        acc[0] += p[0] * (sa.x * sw);
        acc[1] += p[1] * (sa.y * sw);
        acc[2] += p[2] * (sa.z * sw);
        acc[3] += p[3] * (sa.w * sw);
      };
      int j = 0;
      for (; j + kDecDepth <= n; j += kDecDepth) {
#pragma unroll
        for (int d = 0; d < kDecDepth; d++) {
          step(d, j + d);
          load(d, j + d + kDecDepth);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
#pragma unroll
      for (int d = 0; d < kDecDepth - 1; d++)
        if (j + d < n) step(d, j + d);
      __syncthreads();
    } else if (!two) {
      constexpr int kStepDepth2 = 2;   // (register budget shared with the staged path)
      // carriers: wave q loads rows 4q .. 4q + 3 of C's hi term as whole lines (lane l: row
      // 4q + l/16, 16-byte chunk l%16) and publishes them to the stage; wave 0's lanes < 16 the
      // scale of row lane (all lanes load it: no loads under a branch)
      const int ar = 4 * wave + (lane >> 4);
      const _Float16* asrc = ch.hi + (size_t)(row0 + (ar < M ? ar : 0)) * I + (size_t)kb0 * kBlock + (lane & 15) * 8;
      const float* ssrc = ch.scale + (size_t)prow * KB + kb0;
      const float swv = swp[min(lane, n - 1)];
      // weights as whole lines with the non-temporal hint, transposed per wavefront through its LDS
      // buffer tb as on the staged path (MFMA-layout loads instead: 184.8 against 173.9 us per call
      // at T = 64, both GEMMs, measured).  Chunk c of row r sits at r * 128 + (c ^ slot_key8(r)) * 16,
      // so row wr + 8's chunk is at (tw0o ^ 16) + 1024 and chunk 2kg + 1 of row lr at trxo ^ 16
      // (slot_key8(r + 8) = slot_key8(r) ^ 1 for r < 8): two offsets kept instead of four
      const int wr = lane >> 3, wc = lane & 7;
      const uint8_t* wsrc = pb.w2 + ((size_t)e * H + cg * 16 + wr) * I + (size_t)kb0 * kBlock + wc * 16;
      uint8_t* const tb = wtr[wave];
      const int tw0o = wr * kBlock + (wc ^ slot_key8(wr)) * 16;
      const int trxo = lr * kBlock + ((2 * kg) ^ slot_key8(lr)) * 16;
      v4i B0[kStepDepth2], B1[kStepDepth2];
      v4i AR[kStepDepth2];
      float SR[kStepDepth2];
      auto load = [&](int d, int j) {
        const int jj = min(j, n - 1);
        B0[d] = load_w_line(wsrc + (size_t)jj * kBlock);
        B1[d] = load_w_line(wsrc + (size_t)jj * kBlock + (size_t)8 * I);
        AR[d] = *reinterpret_cast<const v4i*>(asrc + (size_t)jj * kBlock);
        SR[d] = ssrc[jj];
      };
      auto step = [&](int d, int j) {
        G2Stage& st = ring[j & 1];
        *reinterpret_cast<v4i*>(st.a + ar * (2 * kBlock) + ((lane & 15) ^ slot_key16(ar)) * 16) = AR[d];
        if (wave == 0 && lane < 16) st.sa[lane] = SR[d];
        // (formed per step: four live offsets spilled at the 96-VGPR budget)
        int t0 = tw0o, t1 = trxo;
        asm volatile("" : "+v"(t0), "+v"(t1));
        *reinterpret_cast<v4i*>(tb + t0) = B0[d];
        *reinterpret_cast<v4i*>(tb + ((t0 ^ 16) + 1024)) = B1[d];
        __syncthreads();
        const v4i bx = *reinterpret_cast<const v4i*>(tb + t1);
        const v4i by = *reinterpret_cast<const v4i*>(tb + (t1 ^ 16));
        // chunk 4 kg + t sits at byte (4 kg ^ key) * 16 ^ 16 t of the row: one base register,
        // formed here (hoisted, the four addresses stay live across the loop and spill)
        int rb = lr * (2 * kBlock) + ((4 * kg) ^ slot_key16(lr)) * 16;
        asm volatile("" : "+v"(rb));
        const float4 sa = *reinterpret_cast<const float4*>(st.sa + 4 * kg);
        const float sw = readlane_f32(swv, j);
        // one 32-K piece at a time (C's hi chunk, the W2 chunk widened exactly, their MFMA), in
        // the order of widen_fp8_operand + mfma_f16_block: all four pieces widened at once
        // spilled 4 VGPRs
        v4f p = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; t++) {
          const v8h ah = *reinterpret_cast<const v8h*>(st.a + (rb ^ (16 * t)));
          const uint32_t w0 = (uint32_t)(t < 2 ? bx[2 * t] : by[2 * t - 4]);
          const uint32_t w1 = (uint32_t)(t < 2 ? bx[2 * t + 1] : by[2 * t - 3]);
          const v2h l0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false);
          const v2h h0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true);
          const v2h l1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false);
          const v2h h1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true);
          const v8h b = {l0[0], l0[1], h0[0], h0[1], l1[0], l1[1], h1[0], h1[1]};
          p = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, b, p, 0, 0, 0);
        }
        acc[0] += p[0] * (sa.x * sw);
        acc[1] += p[1] * (sa.y * sw);
        acc[2] += p[2] * (sa.z * sw);
        acc[3] += p[3] * (sa.w * sw);
      };
#pragma unroll
      for (int d = 0; d < kStepDepth2; d++) load(d, d);
      int j = 0;
      for (; j + kStepDepth2 <= n; j += kStepDepth2) {
#pragma unroll
        for (int d = 0; d < kStepDepth2; d++) {
          step(d, j + d);
          load(d, j + d + kStepDepth2);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
#pragma unroll
      for (int d = 0; d < kStepDepth2 - 1; d++)
        if (j + d < n) step(d, j + d);
      __syncthreads();
    } else {
      const _Float16* hp = ch.hi + (size_t)prow * I + (size_t)kb0 * kBlock + kg * 32;
      const _Float16* lp = ch.lo + (size_t)prow * I + (size_t)kb0 * kBlock + kg * 32;
      const float* sp[4];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int dr = 4 * kg + r;
        sp[r] = ch.scale + (size_t)(row0 + (dr < M ? dr : 0)) * KB + kb0;
      }
      for (int j = 0; j < n; j++) {
        const v8i b = load_v8i(bp + (size_t)j * kBlock);
        v8h ah[4], al[4];
        load_v8h4(hp + (size_t)j * kBlock, ah);
        load_v8h4(lp + (size_t)j * kBlock, al);
        float sa[4];
#pragma unroll
        for (int r = 0; r < 4; r++) sa[r] = sp[r][j];
        const float sw = swp[j];
        v8h b16[4];
        widen_fp8_operand(b, b16);
        v4f p = mfma_f16_block(ah, b16, v4f{0.f, 0.f, 0.f, 0.f});
        p = mfma_f16_block(al, b16, p);
#pragma unroll
        for (int r = 0; r < 4; r++) acc[r] += p[r] * (sa[r] * sw);
      }
    }
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int row = 4 * kg + r;
      if (row < M) {
        const int p = row0 + row;
        store_shared_f32(obuf + ((size_t)p * S + du.s) * H + cg * 16 + lr, acc[r] * pl.perm_w[p]);
      }
    }
    // output columns [64 cb, 64 cb + 64) are complete once all n_mt * S units of the column
    // block stored their rows.  (Every unit loading its first combine pass's token slots before
    // the arrival, so the last one skips that round trip: +0.3 us at T = 16, +1.4 at 64, measured;
    // all units of the launch then read the same few lines.)
    if (arrive_last(pl.counters2 + du.cb * kCounterStride, n_mt * S, &last_s))
      combine_columns(slot_s, obuf, out, T, H, S, du.cb * 16 * kDecBlockWaves, pl.shared, pl.shared_dt,
                      pl.out_f32, pl.info[0]);
  }
}

// Resident capacity of the 4-wave decode GEMMs, in workgroups, and the number of
// 16-column groups one workgroup unit covers.
int decode_grid1() { return num_compute_units() * kDec1BlocksPerCU; }
int decode_grid2() { return num_compute_units() * kDec2BlocksPerCU; }
int decode_unit_groups() { return kDecBlockWaves; }

void launch_gemm1_decode(const Problem& pb, const Plan& pl, const DecodePlanArgs& da, float* gbuf, const CHalf& ch,
                         hipStream_t stream) {
  hipLaunchKernelGGL(gemm1_decode_kernel, dim3(decode_grid1()), dim3(64 * kDecBlockWaves), 0, stream, pb, pl, da,
                     gbuf, ch);
}

void launch_gemm2_decode(const Problem& pb, const Plan& pl, const CHalf& ch, float* obuf, void* out,
                        hipStream_t stream) {
  if (pb.T <= 0) return;
  hipLaunchKernelGGL(gemm2_decode_kernel, dim3(decode_grid2()), dim3(64 * kDecBlockWaves), 0, stream, pb, pl, ch,
                     obuf, out);
}

}  // namespace moefp8
