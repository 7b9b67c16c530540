// Grouped expert GEMMs for T > 64 (prefill): LDS-staged activations, per-wavefront
// weight streams.
//
// A workgroup of 4 wavefronts owns one unit = (m-block of BM = 16*MT rows of one expert,
// block of 128 output columns).  Each wavefront streams its own 32 or 64 weight rows
// straight from HBM into a 2-deep register ring (no sharing needed: no other wavefront
// of the workgroup uses them) and keeps MT x NT 16x16 accumulators.  The BM activation
// rows, shared by all 4 wavefronts, are copied HBM/L2 -> LDS by DMA (global_load_lds,
// no registers) into a 3-stage ring one K-block per stage, together with their per-row
// scales.  LDS operand reads are issued as inline ds_read_b128 together with their
// lgkmcnt wait: the compiler cannot prove that an LDS read does not alias a DMA in
// flight to another stage and would otherwise drain every outstanding load before it.
// Every wavefront issues the same number of memory operations per K-block, so one
// vmcnt wait (explicit count) plus s_barrier per K-block publishes the stage.
//
// Block scales are applied per 128-K block in fp32: acc += MFMA(A_kb, B_kb) * sa[row] * sw.
//
// GEMM1  G1 = A_e W13_e^T on the e4m3 MFMA (m-blocks holding a pair predicted to need exact
//        products: f16 MFMA on widened operands), SwiGLU in the epilogue (main.py:229-233),
//        and C written as hi = f16(C/s), s = max|C row block| / 448 per 128 cols, and
//        lo = f16(C/s - hi) (22 significant bits together).
// flags  per m-block, whether GEMM2 needs both terms of C (needs_two_terms on each row's max |C|
//        per 128 columns, from the scales GEMM1 wrote).
// GEMM2  O = C W2_e^T (main.py:234-238): C's hi term on the f16 MFMA against W2 widened
//        to f16 (exact products, 2^-11 relative input error); m-blocks flagged by GEMM1 add
//        the lo term on the f16 MFMA.  Rows are scaled by the routing weight (main.py:240)
//        and summed per token by the combine kernel.
#include <type_traits>

#include "moefp8_device.h"
#include "moefp8_launch.h"

namespace moefp8 {

constexpr int kLgWaves = 4;
constexpr int kLgThreads = 64 * kLgWaves;
constexpr int kLgDepth = 2;                  // weight K-blocks in flight per wavefront
constexpr int kLgStages = kLgDepth + 1;      // activation stages in LDS

template <int kCount>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(kCount >= 0 && kCount < 64, "vmcnt range");
  // gfx9 s_waitcnt encoding: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14
  __builtin_amdgcn_s_waitcnt((kCount & 15) | (7 << 4) | (15 << 8) | ((kCount >> 4) << 14));
}

// LDS operand reads and their completion wait in one asm statement: the results are defined
// only after the wait, so the compiler can place nothing (e.g. a register copy) that reads
// a destination register while its LDS read is still in flight.
__device__ __forceinline__ void lds_read3(uint32_t a0, uint32_t a1, uint32_t a2, v4i& r0, v4i& r1, v4i& r2) {
  asm volatile(
      "ds_read_b128 %0, %3\n\t"
      "ds_read_b128 %1, %4\n\t"
      "ds_read_b128 %2, %5\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2)
      : "v"(a0), "v"(a1), "v"(a2)
      : "memory");
}
__device__ __forceinline__ void lds_read2(uint32_t a0, uint32_t a1, v4i& r0, v4i& r1) {
  asm volatile(
      "ds_read_b128 %0, %2\n\t"
      "ds_read_b128 %1, %3\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1)
      : "v"(a0), "v"(a1)
      : "memory");
}
__device__ __forceinline__ void lds_read4(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, v4i& r0, v4i& r1,
                                          v4i& r2, v4i& r3) {
  asm volatile(
      "ds_read_b128 %0, %4\n\t"
      "ds_read_b128 %1, %5\n\t"
      "ds_read_b128 %2, %6\n\t"
      "ds_read_b128 %3, %7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
      : "v"(a0), "v"(a1), "v"(a2), "v"(a3)
      : "memory");
}
__device__ __forceinline__ void lds_read5(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3, uint32_t a4, v4i& r0,
                                          v4i& r1, v4i& r2, v4i& r3, v4i& r4) {
  asm volatile(
      "ds_read_b128 %0, %5\n\t"
      "ds_read_b128 %1, %6\n\t"
      "ds_read_b128 %2, %7\n\t"
      "ds_read_b128 %3, %8\n\t"
      "ds_read_b128 %4, %9\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3), "=&v"(r4)
      : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "v"(a4)
      : "memory");
}

// s_barrier, then no memory access may move above it
__device__ __forceinline__ void barrier_lds() {
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
#define MOEFP8_WAIT_VMCNT(n) asm volatile("s_waitcnt vmcnt(" #n ")" ::: "memory")
// The same for a wave-uniform count n in [2, 7] (the count is an immediate of the instruction).
__device__ __forceinline__ void wait_vmcnt_2to7(int n) {
  if (n <= 2) MOEFP8_WAIT_VMCNT(2);
  else if (n == 3) MOEFP8_WAIT_VMCNT(3);
  else if (n == 4) MOEFP8_WAIT_VMCNT(4);
  else if (n == 5) MOEFP8_WAIT_VMCNT(5);
  else if (n == 6) MOEFP8_WAIT_VMCNT(6);
  else MOEFP8_WAIT_VMCNT(7);
}

// Wave-uniform read of kernel-constant data through the constant address space, so the
// compiler can use a scalar load (counted by lgkmcnt, not by the vmcnt pipeline above).
__device__ __forceinline__ float load_uniform(const float* p) {
  return *(const __attribute__((address_space(4))) float*)p;
}

__device__ __forceinline__ v8i load_w(const uint8_t* p) {
  const v4i* q = reinterpret_cast<const v4i*>(p);
  const v4i x = q[0], y = q[1];
  return __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ v8i cat(v4i x, v4i y) { return __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7); }

__device__ __forceinline__ v8h as_v8h(v4i x) { return __builtin_bit_cast(v8h, x); }

// Writes C's two f16 terms of one element at p * I + col.
__device__ __forceinline__ void store_c(const CHalf8& ch, size_t p, int I, int col, float c, float inv) {
  const float v = fminf(fmaxf(c * inv, -448.0f), 448.0f);
  const _Float16 hi = (_Float16)v;
  ch.hi[p * I + col] = hi;
  ch.lo16[p * I + col] = (_Float16)(v - (float)hi);
}

// ------------------------------------------------------------------------------------------ units
// Units (m-block, column block) are ordered expert by expert, then column block by column block,
// the expert's m-blocks innermost, and the order is cut into eighths.  Workgroup b of a grid that
// is a multiple of 8 runs on XCD b % 8 (workgroups are dispatched to the XCDs round robin) and works
// through eighth b % 8 with the other workgroups of its XCD, in order: the units that run at the
// same time on one XCD share their expert's weight column blocks and activation blocks through that
// XCD's L2 instead of each XCD fetching them from HBM.  Its first unit is eighth[b / 8]; later ones
// come from a per-XCD queue (queue x counts the units of eighth x handed out past the first
// round), claimed when the workgroup is free, and a workgroup whose eighth is used up takes units
// from the other eighths: unit costs differ (block heights, precision modes), and a static split
// would leave XCDs idle at the end.  The counters sit on separate 256-byte lines.  The smaller-T
// kernels (about one unit per workgroup) keep the static split: workgroup b takes units
// eighth[b / 8], eighth[b / 8 + grid / 8], ... (measured faster there than claiming).
struct UnitEighths {
  int nx, x, per;
  __device__ __forceinline__ UnitEighths() {
    nx = gridDim.x % 8 == 0 ? 8 : 1;
    x = blockIdx.x % nx;
    per = gridDim.x / nx;
  }
  __device__ __forceinline__ int lo(int n_units, int y) const { return (int)((int64_t)n_units * y / nx); }
};
// Thread 0 claims; -1 when every eighth is used up.
__device__ __forceinline__ int grab_unit(int* queues, int n_units) {
  const UnitEighths u;
  for (int d = 0; d < u.nx; d++) {
    const int y = (u.x + d) % u.nx;
    const int lo = u.lo(n_units, y), n = u.lo(n_units, y + 1) - lo;
    int* q = queues + y * kQueueStride;
    // a relaxed load first, so that a used-up eighth costs no atomic
    if (u.per + __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= n) continue;
    const int k = u.per + __hip_atomic_fetch_add(q, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (k < n) return lo + k;
  }
  return -1;
}

__device__ __forceinline__ int first_unit(int* queues, int n_units) {
  const UnitEighths u;
  const int v = u.lo(n_units, u.x) + (int)blockIdx.x / u.nx;
  return v < u.lo(n_units, u.x + 1) ? v : grab_unit(queues, n_units);
}

// Unit v of that order as {m-block, column block}; mbgroup[g] = {first m-block of g's expert,
// the expert's m-blocks}, so the units of an expert are [first * NC, (first + count) * NC).
__device__ __forceinline__ int2 unit_at(const int2* mbgroup, int v, int NC) {
  const int2 g = mbgroup[v / NC];
  const int local = v - g.x * NC;
  return int2{g.x + local % g.y, local / g.y};
}

// ------------------------------------------------------------------------------------------ GEMM1
// LDS stage: MT m-tiles x [8 chunks of 16 B][16 rows][16 B] of e4m3 activations, then 4 x 64
// row scales (one slot per wavefront; rows >= BM are padding).
template <int MT>
struct G1L {
  static constexpr int kA = MT * 2048;
  static constexpr int kStage = kA + kLgWaves * 64 * 4;
  static constexpr int kDmaA = MT / 2;                 // 1 KB activation DMAs per wave per K-block
  static constexpr int kOps = kDmaA + 1 + 8;           // + row-scale DMA + 4 weight tiles x 2 loads
};

// One pass over K for m-tiles [i0, i0 + NA) of the unit's m-block (the DMA always stages all
// MT m-tiles, so every pass issues the same operations).  kExact: the pass runs on the f16
// MFMA with widened operands (exact products).
//
// Every m-tile of the pass is computed, also past the block's last row (those rows hold
// clamped copies and are never stored): a K step is straight-line code with no branch between
// an MFMA and the VALU instructions that read its result.  The compiler's hazard check does
// not count the wait states of an MFMA in a conditional block correctly for a reader in a
// later block (a scaled 16x16x128 MFMA needs 12, it inserted 8), and the reader then sees
// the register's previous contents.
template <int MT, int NA, bool kExact>
__device__ __forceinline__ void gemm1_large_pass(const Problem& pb, const Plan& pl, uint8_t* ring, int e, int row0,
                                                 int rows, int cb, int i0, v4f (&acc)[NA][4]) {
  using L = G1L<MT>;
  const int H = pb.H, I = pb.I, T = pb.T, KB = H / kBlock, NCB = I / kBlock;
  const int wave = wave_index(), lane = lane_id(), lr = lane & 15, kg = lane >> 4;
  const int col0 = cb * kBlock + 32 * wave;
  const uint8_t* bp = pb.w13 + ((size_t)e * 2 * I + col0 + lr) * H + kg * 32;
  const size_t gate_off = (size_t)I * H;
  const float* swu = pb.s13 + ((size_t)e * (2 * I / kBlock) + cb) * KB;
  const float* swg = swu + (size_t)NCB * KB;
  // activation DMA sources: wave w carries m-tiles (w/2) + 2r, chunk half w%2
  const uint8_t* asrc[L::kDmaA];
#pragma unroll
  for (int r = 0; r < L::kDmaA; r++) {
    const int row = 16 * ((wave >> 1) + 2 * r) + lr;
    const int tok = clamp_index(pl.perm_token[row0 + min(row, rows - 1)], T);
    asrc[r] = pb.hidden + (size_t)tok * H + (4 * (wave & 1) + kg) * 16;
  }
  const int srow = min(64 * wave + lane, rows - 1);
  const float* ssrc = pb.hscale + clamp_index(pl.perm_token[row0 + srow], T);
#pragma unroll
  for (int i = 0; i < NA; i++)
#pragma unroll
    for (int n = 0; n < 4; n++) acc[i][n] = v4f{0.f, 0.f, 0.f, 0.f};
  v8i B[kLgDepth][4];
  float SU[kLgDepth], SG[kLgDepth];

  auto issue = [&](int d, int j) {
    const int k = min(j, KB - 1);
    uint8_t* st = ring + (j % kLgStages) * L::kStage;
#pragma unroll
    for (int r = 0; r < L::kDmaA; r++)
      __builtin_amdgcn_global_load_lds(asrc[r] + (size_t)k * kBlock,
                                       st + (((wave >> 1) + 2 * r) * 2048 + (wave & 1) * 1024), 16, 0, 0);
    __builtin_amdgcn_global_load_lds(ssrc + (size_t)k * T, st + L::kA + wave * 256, 4, 0, 0);
    const uint8_t* b = bp + (size_t)k * kBlock;
    B[d][0] = load_w(b);
    B[d][1] = load_w(b + (size_t)16 * H);
    B[d][2] = load_w(b + gate_off);
    B[d][3] = load_w(b + gate_off + (size_t)16 * H);
    SU[d] = load_uniform(swu + k);
    SG[d] = load_uniform(swg + k);
  };
  auto step = [&](int d, int j) {
    // at most the operations of the following kLgDepth - 1 steps may still be in flight
    // (every wavefront issues at least L::kOps vector-memory operations per step)
    wait_vmcnt<(kLgDepth - 1) * L::kOps>();
    __builtin_amdgcn_s_barrier();
    const uint8_t* st = ring + (j % kLgStages) * L::kStage;
#pragma unroll
    for (int ia = 0; ia < NA; ia++) {
      const int i = i0 + ia;
      v4i x, y, s4;
      lds_read3(lds_addr(st + i * 2048 + ((2 * kg) * 16 + lr) * 16),
                lds_addr(st + i * 2048 + ((2 * kg + 1) * 16 + lr) * 16), lds_addr(st + L::kA + (16 * i + 4 * kg) * 4),
                x, y, s4);
      const v8i a = cat(x, y);
      const float4 sa = __builtin_bit_cast(float4, s4);
      if constexpr (!kExact) {
#pragma unroll
        for (int n = 0; n < 4; n++) {
          const float sw = n < 2 ? SU[d] : SG[d];
          const v4f p = mfma16x16x128(a, B[d][n], v4f{0.f, 0.f, 0.f, 0.f});
          acc[ia][n][0] += p[0] * (sa.x * sw);
          acc[ia][n][1] += p[1] * (sa.y * sw);
          acc[ia][n][2] += p[2] * (sa.z * sw);
          acc[ia][n][3] += p[3] * (sa.w * sw);
        }
      } else {
        v8h a16[4];
        widen_fp8_operand(a, a16);
#pragma unroll
        for (int n = 0; n < 4; n++) {
          const float sw = n < 2 ? SU[d] : SG[d];
          v8h b16[4];
          widen_fp8_operand(B[d][n], b16);
          const v4f p = mfma_f16_block(a16, b16, v4f{0.f, 0.f, 0.f, 0.f});
          acc[ia][n][0] += p[0] * (sa.x * sw);
          acc[ia][n][1] += p[1] * (sa.y * sw);
          acc[ia][n][2] += p[2] * (sa.z * sw);
          acc[ia][n][3] += p[3] * (sa.w * sw);
        }
      }
    }
    // stage (j + kLgDepth) % kLgStages was last read at step j - 1, before this barrier
    issue(d, j + kLgDepth);
    __builtin_amdgcn_sched_barrier(0);
  };

  // the previous pass's LDS reads are complete before its stages are refilled
  __syncthreads();
  // stage d's operations must all be issued before stage d + 1's: the per-step vmcnt wait
  // counts operations in issue order
#pragma unroll
  for (int d = 0; d < kLgDepth; d++) {
    issue(d, d);
    __builtin_amdgcn_sched_barrier(0);
  }
  int j = 0;
  for (; j + 2 * kLgDepth <= KB; j += 2 * kLgDepth) {
#pragma unroll
    for (int d = 0; d < 2 * kLgDepth; d++) step(d % kLgDepth, j + d);
  }
  for (; j < KB; j += kLgDepth) {
#pragma unroll
    for (int d = 0; d < kLgDepth; d++)
      if (j + d < KB) step(d, j + d);
  }
  // no DMA may still target the ring when the next pass refills it or the workgroup ends
  wait_vmcnt<0>();
}

// Epilogue of m-tiles [i0, i0 + NA): C = silu(gate) * up and its split into two f16 terms.
// amax_s holds, per wavefront and row, the largest |C| of the wavefront's 32 columns.
template <int MT, int NA>
__device__ __forceinline__ void gemm1_large_store(const CHalf8& ch, float (*amax_s)[16 * MT], int I, int row0,
                                                  int rows, int cb, int i0, const v4f (&acc)[NA][4]) {
  const int NCB = I / kBlock;
  const int wave = wave_index(), lane = lane_id(), lr = lane & 15, kg = lane >> 4;
  const int col0 = cb * kBlock + 32 * wave;
  float c[NA][2][4];
#pragma unroll
  for (int ia = 0; ia < NA; ia++)
#pragma unroll
    for (int jn = 0; jn < 2; jn++)
#pragma unroll
      for (int r = 0; r < 4; r++) c[ia][jn][r] = silu_f32(acc[ia][jn + 2][r]) * acc[ia][jn][r];
#pragma unroll
  for (int ia = 0; ia < NA; ia++) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      float m = fmaxf(fabsf(c[ia][0][r]), fabsf(c[ia][1][r]));
      m = fmaxf(m, dpp_f32<kDppXor1>(m));
      m = fmaxf(m, dpp_f32<kDppXor2>(m));
      m = fmaxf(m, dpp_f32<kDppHalfMirror>(m));
      m = fmaxf(m, dpp_f32<kDppRowMirror>(m));
      if (lr == 0) amax_s[wave][16 * (i0 + ia) + 4 * kg + r] = m;
    }
  }
  __syncthreads();
#pragma unroll
  for (int ia = 0; ia < NA; ia++) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int row = 16 * (i0 + ia) + 4 * kg + r;
      if (row >= rows) continue;
      const float amax = fmaxf(fmaxf(amax_s[0][row], amax_s[1][row]), fmaxf(amax_s[2][row], amax_s[3][row]));
      float inv, scale;
      split_scale(amax, inv, scale);
      const size_t p = (size_t)(row0 + row);
#pragma unroll
      for (int jn = 0; jn < 2; jn++) store_c(ch, p, I, col0 + 16 * jn + lr, c[ia][jn][r], inv);
      if (wave == 0 && lr == 0) ch.scale[p * NCB + cb] = scale;
    }
  }
  // amax_s is rewritten by the next store
  __syncthreads();
}

// Units (m-block, 128 output columns) over GEMM1's blocks.
template <int MT>
__global__ __launch_bounds__(kLgThreads, 2) void gemm1_large_kernel(Problem pb, Plan pl, CHalf8 ch) {
  using L = G1L<MT>;
  static_assert(MT % 2 == 0, "two activation DMAs per m-tile");
  __shared__ __attribute__((aligned(16))) uint8_t ring[kLgStages * L::kStage];
  __shared__ float amax_s[kLgWaves][16 * MT];
  const int I = pb.I, NCB = I / kBlock;
  const UnitEighths u;
  const int n_units = pl.info[2] * NCB, end = u.lo(n_units, u.x + 1);
  for (int v = u.lo(n_units, u.x) + (int)blockIdx.x / u.nx; v < end; v += u.per) {
    const int2 uc = unit_at(pl.mbgroup, v, NCB);
    const int mb = uniform(uc.x), cb = uniform(uc.y);
    const int4 blk = pl.mblocks[mb];
    const int e = uniform(blk.x), row0 = uniform(blk.y), rows = uniform(blk.z), flags = uniform(blk.w);
    const int mvalid = (rows + 15) / 16;
    if (!(flags & kFlagExactProducts)) {
      v4f acc[MT][4];
      gemm1_large_pass<MT, MT, false>(pb, pl, ring, e, row0, rows, cb, 0, acc);
      gemm1_large_store<MT, MT>(ch, amax_s, I, row0, rows, cb, 0, acc);
    } else {
      // two m-tiles per pass over K, with exact products (the f16 MFMA on widened operands
      // needs the registers of the fp8 path twice over)
      for (int i0 = 0; i0 < mvalid; i0 += 2) {
        v4f acc[2][4];
        gemm1_large_pass<MT, 2, true>(pb, pl, ring, e, row0, rows, cb, i0, acc);
        gemm1_large_store<MT, 2>(ch, amax_s, I, row0, rows, cb, i0, acc);
      }
    }
  }
}

// ------------------------------------------------------------------------------ GEMM1, 128-row m-blocks
// For the 128-row blocks over an expert's class 0 and 1 rows.  A workgroup of 8 wavefronts (one
// per CU, two per SIMD, 148 KB of LDS) owns one unit = (m-block, 128 C columns = 256 weight rows,
// 128 up and 128 gate) and stages BOTH operands of each K-block through a 3-stage LDS ring by
// DMA: the weight rows are read once per unit and shared by the block's 128 rows (the
// per-wavefront weight streams above re-read them per 64 rows through the vector-memory path).
// Wavefront w = (wm, wn) = (w % 2, w / 2) computes rows 64 wm .. 64 wm + 63 x its 64 weight rows
// (C columns 32 wn .. 32 wn + 31, up and gate): 4 x 4 MFMA 16x16x128 tiles per K-block, 64
// accumulator registers, so that the two wavefronts of a SIMD hide each other's MFMA and LDS
// latencies.
//
// The DMAs and their wait are inline asm and the LDS operand reads ordinary loads: the compiler
// schedules the reads with exact lgkmcnt waits and never drains the DMAs before them.
//
// LDS stage: A [128 rows][128 B], B [256 rows][128 B], 128 row scales.  A row's 16-byte chunk c
// sits in slot c ^ slot_key8(row): a DMA instruction writes 8
// rows x 8 slots in lane order (each lane fetching the chunk that belongs in its slot, 8 lanes
// per 128-byte row segment), and an MFMA operand read (16 rows, two chunks per lane) puts any 16
// consecutive lanes on distinct 16-byte bank groups of a 256-byte bank row (and any 8 on distinct
// ones of a 128-byte row).
constexpr int kBgWaves = 8;
constexpr int kBgThreads = 64 * kBgWaves;
constexpr int kBgRows = 128;
constexpr int kBgWRows = 256;
constexpr int kBgStages = 3;
constexpr int kBgA = kBgRows * 128;
constexpr int kBgB = kBgWRows * 128;
constexpr int kBgStage = kBgA + kBgB + kBgRows * 4;
constexpr int kBgOps = 2 + 4 + 1;            // per wavefront and K-block: A, B and row-scale DMAs

// LDS row R of a 128-row unit -> row of the permuted pairs.  Regular blocks: R < rows.  A mixed
// block (an expert's last regular block with its <= 32 exact-product rows folded in) puts its
// regular rows at LDS rows [0, cap) and its exact rows at [cap, 128), cap = 128 - 16 ceil(x / 16);
// the exact rows follow the regular ones in the permuted order.  Rows from xfrom on (0 for an
// exact-product block, cap for a mixed one, 128 otherwise) get exact products and an f16 lo term.
struct RowMap {
  int row0, rows, cap, xrows, xfrom;
  __device__ __forceinline__ int src(int R) const {
    return R < cap ? row0 + min(R, rows - 1) : row0 + rows + min(R - cap, xrows - 1);
  }
  __device__ __forceinline__ bool valid(int R) const { return R < cap ? R < rows : R - cap < xrows; }
};
__device__ __forceinline__ RowMap row_map(int row0, int rows, int flags) {
  if (flags & kFlagMixed) {
    const int x = flags >> kMixedShift, cap = kBgRows - 16 * ((x + 15) / 16);
    return RowMap{row0, rows, cap, x, cap};
  }
  return RowMap{row0, rows, kBgRows, 0, (flags & kFlagExactProducts) ? 0 : kBgRows};
}

// A mixed block's m-tiles for wavefront half wm: nf regular tiles from tf0 and nx exact tiles from
// tx0.  An exact tile costs about three regular ones, so with two exact tiles each half takes one
// of them and half of the regular tiles, and with one the other half takes more regular tiles.
struct TileSplit {
  int nf, nx, tf0, tx0;
};
__device__ __forceinline__ TileSplit mixed_split(const RowMap& rm, int wm) {
  const int nr = (rm.rows + 15) / 16;
  if (rm.cap == kBgRows - 32) {
    const int a = (nr + 1) / 2;
    return wm == 0 ? TileSplit{a, 1, 0, 6} : TileSplit{nr - a, 1, a, 7};
  }
  const int a = min(min(nr, 4), (nr + 4) / 2);
  return wm == 0 ? TileSplit{a, 0, 0, 0} : TileSplit{nr - a, 1, a, 7};
}

// One unit.  Wavefront (wm, wn) computes m-tiles NT wm .. NT wm + NT - 1: NT = 4 for blocks of more
// than 64 rows, 2 for 33..64 rows and 1 for at most 32 (the short last blocks of an expert's
// classes cost a quarter of the MFMA and VALU work of a full one).  kExact (blocks of at most 32
// exact-product rows, NT = 1): the f16 MFMA on operands widened exactly, and C's lo term in f16.
// kOnce: the block is its expert's only one, so each weight line is read once per call, by one
// DMA instruction (8 lanes x 16 B), and its DMAs carry the non-temporal hint: 5% less GEMM1
// time at 1024 tokens (about one block per expert), measured.  Experts with several blocks keep
// ordinary DMAs, which let the blocks share the weights through L2 (the hint on every block cost
// 20% at 8192 tokens, measured).  A template parameter, not a branch: the branch in the K loop
// cost up to 4% on the other blocks, measured.
template <int NT, bool kExact, bool kOnce>
__device__ __forceinline__ void gemm1_big_unit(const Problem& pb, const Plan& pl, const CHalf8& ch, uint8_t* ring,
                                               uint32_t ring_lds, uint32_t sink_lds, const float2* sw_s,
                                               float (*amax_s)[kBgRows],
                                               int e, int row0, int rows, int cb, int* next_s, int n_units) {
  static_assert(NT == 1 || NT == 2 || NT == 4, "m-tiles per wavefront");
  static_assert(!kExact || NT == 1, "exact-product blocks hold at most 32 rows");
  const int H = pb.H, I = pb.I, T = pb.T, KB = H / kBlock, NCB = I / kBlock;
  const int wave = wave_index(), lane = lane_id(), lr = lane & 15, kg = lane >> 4;
  const int wm = wave & 1, wn = wave >> 1;
  // DMA lane roles: row (lane / 8) of an 8-row group, slot lane % 8
  const int drow = lane >> 3, dslot = lane & 7;
  // operand read offsets inside a 16-row tile (swizzled chunks 2kg and 2kg + 1 of row lr)
  const int rd0 = lr * 128 + (((2 * kg) ^ slot_key8(lr)) * 16);
  const int rd1 = lr * 128 + (((2 * kg + 1) ^ slot_key8(lr)) * 16);
  // DMA sources as per-lane byte offsets from wave-uniform bases: A rows 16w + 8q + drow (the
  // tokens' hidden rows, clamped to the block), B LDS rows 32w + 8q + drow (LDS row R holds n-tile
  // (R % 64) / 16 of weight-row group R / 64: 0, 1 up, 2, 3 gate), row scales of rows 64 (w % 2) + lane
  uint32_t aoff[2], boff[4];
#pragma unroll
  for (int q = 0; q < 2; q++) {
    const int r = 16 * wave + 8 * q + drow;
    const int tok = clamp_index(pl.perm_token[row0 + min(r, rows - 1)], T);
    aoff[q] = (uint32_t)tok * (uint32_t)H + (uint32_t)((dslot ^ slot_key8(r)) * 16);
  }
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int R = 32 * wave + 8 * q + drow;
    const int g = R >> 6, n = (R >> 4) & 3, rr = R & 15;
    const int wrow = (n < 2 ? 0 : I) + cb * kBlock + 32 * g + 16 * (n & 1) + rr;
    boff[q] = (uint32_t)wrow * (uint32_t)H + (uint32_t)((dslot ^ slot_key8(R)) * 16);
  }
  const uint32_t soff =
      wave < 2 ? 4u * (uint32_t)clamp_index(pl.perm_token[row0 + min(64 * (wave & 1) + lane, rows - 1)], T) : 0u;
  const uint8_t* wbase = pb.w13 + (size_t)e * 2 * I * H;
  auto issue = [&](int j) {
    const int k = min(j, KB - 1);
    const uint32_t st = ring_lds + (uint32_t)((j % kBgStages) * kBgStage);
    const uint8_t* abase = pb.hidden + (size_t)k * kBlock;
    const uint8_t* bbase = wbase + (size_t)k * kBlock;
    const float* sbase = pb.hscale + (size_t)k * T;
#pragma unroll
    for (int q = 0; q < 2; q++) dma_lds16_s(aoff[q], abase, st + (16 * wave + 8 * q) * 128);
    if (kOnce) {
#pragma unroll
      for (int q = 0; q < 4; q++) dma_lds16_s_nt(boff[q], bbase, st + kBgA + (32 * wave + 8 * q) * 128);
    } else {
#pragma unroll
      for (int q = 0; q < 4; q++) dma_lds16_s(boff[q], bbase, st + kBgA + (32 * wave + 8 * q) * 128);
    }
    // every wavefront issues the same operations: wavefronts 0 and 1 DMA the row scales of rows
    // 64 w + lane, 2..7 one 4-byte word (one line, all lanes) into a sink: GEMM1 -3 / -4 to -8 µs
    // at T = 1024 / 8192 against all eight DMAing the 64 scattered scales of 0 and 1 (measured)
    dma_lds4_s(soff, sbase, wave < 2 ? st + kBgA + kBgB + (wave & 1) * 256 : sink_lds);
  };

  // the table and scale loads of the unit are complete: only DMAs count from here
  MOEFP8_WAIT_VMCNT(0);
  for (int d = 0; d < kBgStages - 1; d++) issue(d);
  v4f acc[NT][4];
#pragma unroll
  for (int i = 0; i < NT; i++)
#pragma unroll
    for (int n = 0; n < 4; n++) acc[i][n] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int j = 0; j < KB; j++) {
    // stage j's DMAs are done once only the following stage's (7 per wavefront) may be in flight
    static_assert((kBgStages - 2) * kBgOps == 7, "wait count");
    MOEFP8_WAIT_VMCNT(7);
    barrier_lds();
    const uint8_t* st = ring + (j % kBgStages) * kBgStage;
    v8i B[4];
#pragma unroll
    for (int n = 0; n < 4; n++) {
      const uint8_t* bt = st + kBgA + (64 * wn + 16 * n) * 128;
      B[n] = cat(*reinterpret_cast<const v4i*>(bt + rd0), *reinterpret_cast<const v4i*>(bt + rd1));
    }
    const float2 sw = sw_s[j];
#pragma unroll
    for (int i = 0; i < NT; i++) {
      const int t = NT * wm + i;
      const uint8_t* at = st + t * 16 * 128;
      const v8i a = cat(*reinterpret_cast<const v4i*>(at + rd0), *reinterpret_cast<const v4i*>(at + rd1));
      const float4 sa = *reinterpret_cast<const float4*>(st + kBgA + kBgB + (16 * t + 4 * kg) * 4);
      const float4 su = {sa.x * sw.x, sa.y * sw.x, sa.z * sw.x, sa.w * sw.x};
      const float4 sg = {sa.x * sw.y, sa.y * sw.y, sa.z * sw.y, sa.w * sw.y};
      v8h a16[4];
      if constexpr (kExact) widen_fp8_operand(a, a16);
#pragma unroll
      for (int n = 0; n < 4; n++) {
        const float4 sc = n < 2 ? su : sg;
        v4f p;
        if constexpr (kExact) {
          v8h b16[4];
          widen_fp8_operand(B[n], b16);
          p = mfma_f16_block(a16, b16, v4f{0.f, 0.f, 0.f, 0.f});
        } else {
          p = mfma16x16x128(a, B[n], v4f{0.f, 0.f, 0.f, 0.f});
        }
        acc[i][n][0] += p[0] * sc.x;
        acc[i][n][1] += p[1] * sc.y;
        acc[i][n][2] += p[2] * sc.z;
        acc[i][n][3] += p[3] * sc.w;
      }
    }
    // stage (j + 2) % 3 was last read at step j - 1, before this step's barrier
    issue(j + kBgStages - 1);
  }
  MOEFP8_WAIT_VMCNT(0);
  // the workgroup's next unit, claimed now so that the atomic overlaps the epilogue
  if (threadIdx.x == 0) *next_s = grab_unit(pl.queues, n_units);

  // epilogue: C = silu(gate) * up, per-row max over the unit's 128 columns, hi/lo split
  const int col0 = cb * kBlock + 32 * wn;
  float c[NT][2][4];
#pragma unroll
  for (int i = 0; i < NT; i++)
#pragma unroll
    for (int jn = 0; jn < 2; jn++)
#pragma unroll
      for (int r = 0; r < 4; r++) c[i][jn][r] = silu_f32(acc[i][jn + 2][r]) * acc[i][jn][r];
#pragma unroll
  for (int i = 0; i < NT; i++) {
    const int t = NT * wm + i;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      float m = fmaxf(fabsf(c[i][0][r]), fabsf(c[i][1][r]));
      m = fmaxf(m, dpp_f32<kDppXor1>(m));
      m = fmaxf(m, dpp_f32<kDppXor2>(m));
      m = fmaxf(m, dpp_f32<kDppHalfMirror>(m));
      m = fmaxf(m, dpp_f32<kDppRowMirror>(m));
      if (lr == 0) amax_s[wn][16 * t + 4 * kg + r] = m;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NT; i++) {
    const int t = NT * wm + i;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int row = 16 * t + 4 * kg + r;
      if (row >= rows) continue;
      const float amax = fmaxf(fmaxf(amax_s[0][row], amax_s[1][row]), fmaxf(amax_s[2][row], amax_s[3][row]));
      float inv, scale;
      split_scale(amax, inv, scale);
      const size_t p = (size_t)(row0 + row);
#pragma unroll
      for (int jn = 0; jn < 2; jn++) store_c(ch, p, I, col0 + 16 * jn + lr, c[i][jn][r], inv);
      if (wn == 0 && lr == 0) ch.scale[p * NCB + cb] = scale;
    }
  }
}

// One unit of a mixed block.  This wavefront computes NF m-tiles tf0 .. tf0 + NF - 1 on the e4m3
// MFMA and NX m-tiles tx0 .. tx0 + NX - 1 with exact products (the f16 MFMA on operands widened
// exactly), its half of the block's tiles (mixed_split); every wavefront issues the same DMAs and
// barriers.  (Kept apart from gemm1_big_unit: the compiler schedules the regular blocks' K loop
// worse in this general form, LDS reads no longer hoisted ahead of the MFMAs, ~10% slower.)
template <int NF, int NX>
__device__ __forceinline__ void gemm1_big_mixed_unit(const Problem& pb, const Plan& pl, const CHalf8& ch, uint8_t* ring,
                                               uint32_t ring_lds, uint32_t sink_lds, const float2* sw_s,
                                               float (*amax_s)[kBgRows],
                                               int e, const RowMap& rm, int cb, int tf0, int tx0, int* next_s,
                                               int n_units) {
  constexpr int NT = NF + NX;
  static_assert(NT >= 1 && NT <= 4, "m-tiles per wavefront");
  const int H = pb.H, I = pb.I, T = pb.T, KB = H / kBlock, NCB = I / kBlock;
  const int wave = wave_index(), lane = lane_id(), lr = lane & 15, kg = lane >> 4;
  const int wn = wave >> 1;
  auto tile = [&](int i) { return i < NF ? tf0 + i : tx0 + (i - NF); };
  // DMA lane roles: row (lane / 8) of an 8-row group, slot lane % 8
  const int drow = lane >> 3, dslot = lane & 7;
  // operand read offsets inside a 16-row tile (swizzled chunks 2kg and 2kg + 1 of row lr)
  const int rd0 = lr * 128 + (((2 * kg) ^ slot_key8(lr)) * 16);
  const int rd1 = lr * 128 + (((2 * kg + 1) ^ slot_key8(lr)) * 16);
  // DMA sources as per-lane byte offsets from wave-uniform bases: A rows 16w + 8q + drow (the
  // tokens' hidden rows), B LDS rows 32w + 8q + drow (LDS row R holds n-tile (R % 64) / 16 of
  // weight-row group R / 64: 0, 1 up, 2, 3 gate), row scales of rows 64 (w % 2) + lane
  uint32_t aoff[2], boff[4];
#pragma unroll
  for (int q = 0; q < 2; q++) {
    const int r = 16 * wave + 8 * q + drow;
    const int tok = clamp_index(pl.perm_token[rm.src(r)], T);
    aoff[q] = (uint32_t)tok * (uint32_t)H + (uint32_t)((dslot ^ slot_key8(r)) * 16);
  }
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int R = 32 * wave + 8 * q + drow;
    const int g = R >> 6, n = (R >> 4) & 3, rr = R & 15;
    const int wrow = (n < 2 ? 0 : I) + cb * kBlock + 32 * g + 16 * (n & 1) + rr;
    boff[q] = (uint32_t)wrow * (uint32_t)H + (uint32_t)((dslot ^ slot_key8(R)) * 16);
  }
  const uint32_t soff = wave < 2 ? 4u * (uint32_t)clamp_index(pl.perm_token[rm.src(64 * (wave & 1) + lane)], T) : 0u;
  const uint8_t* wbase = pb.w13 + (size_t)e * 2 * I * H;
  auto issue = [&](int j) {
    const int k = min(j, KB - 1);
    const uint32_t st = ring_lds + (uint32_t)((j % kBgStages) * kBgStage);
    const uint8_t* abase = pb.hidden + (size_t)k * kBlock;
    const uint8_t* bbase = wbase + (size_t)k * kBlock;
    const float* sbase = pb.hscale + (size_t)k * T;
#pragma unroll
    for (int q = 0; q < 2; q++) dma_lds16_s(aoff[q], abase, st + (16 * wave + 8 * q) * 128);
#pragma unroll
    for (int q = 0; q < 4; q++) dma_lds16_s(boff[q], bbase, st + kBgA + (32 * wave + 8 * q) * 128);
    // every wavefront issues the same operations: wavefronts 0 and 1 DMA the row scales of rows
    // 64 w + lane, 2..7 one 4-byte word (one line, all lanes) into a sink: GEMM1 -3 / -4 to -8 µs
    // at T = 1024 / 8192 against all eight DMAing the 64 scattered scales of 0 and 1 (measured)
    dma_lds4_s(soff, sbase, wave < 2 ? st + kBgA + kBgB + (wave & 1) * 256 : sink_lds);
  };

  // the table and scale loads of the unit are complete: only DMAs count from here
  MOEFP8_WAIT_VMCNT(0);
  for (int d = 0; d < kBgStages - 1; d++) issue(d);
  v4f acc[NT][4];
#pragma unroll
  for (int i = 0; i < NT; i++)
#pragma unroll
    for (int n = 0; n < 4; n++) acc[i][n] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int j = 0; j < KB; j++) {
    // stage j's DMAs are done once only the following stage's (7 per wavefront) may be in flight
    static_assert((kBgStages - 2) * kBgOps == 7, "wait count");
    MOEFP8_WAIT_VMCNT(7);
    barrier_lds();
    const uint8_t* st = ring + (j % kBgStages) * kBgStage;
    v8i B[4];
#pragma unroll
    for (int n = 0; n < 4; n++) {
      const uint8_t* bt = st + kBgA + (64 * wn + 16 * n) * 128;
      B[n] = cat(*reinterpret_cast<const v4i*>(bt + rd0), *reinterpret_cast<const v4i*>(bt + rd1));
    }
    const float2 sw = sw_s[j];
#pragma unroll
    for (int i = 0; i < NT; i++) {
      const int t = tile(i);
      const uint8_t* at = st + t * 16 * 128;
      const v8i a = cat(*reinterpret_cast<const v4i*>(at + rd0), *reinterpret_cast<const v4i*>(at + rd1));
      const float4 sa = *reinterpret_cast<const float4*>(st + kBgA + kBgB + (16 * t + 4 * kg) * 4);
      const float4 su = {sa.x * sw.x, sa.y * sw.x, sa.z * sw.x, sa.w * sw.x};
      const float4 sg = {sa.x * sw.y, sa.y * sw.y, sa.z * sw.y, sa.w * sw.y};
      v8h a16[4];
      if (i >= NF) widen_fp8_operand(a, a16);
#pragma unroll
      for (int n = 0; n < 4; n++) {
        const float4 sc = n < 2 ? su : sg;
        v4f p;
        if (i >= NF) {
          v8h b16[4];
          widen_fp8_operand(B[n], b16);
          p = mfma_f16_block(a16, b16, v4f{0.f, 0.f, 0.f, 0.f});
        } else {
          p = mfma16x16x128(a, B[n], v4f{0.f, 0.f, 0.f, 0.f});
        }
        acc[i][n][0] += p[0] * sc.x;
        acc[i][n][1] += p[1] * sc.y;
        acc[i][n][2] += p[2] * sc.z;
        acc[i][n][3] += p[3] * sc.w;
      }
    }
    // stage (j + 2) % 3 was last read at step j - 1, before this step's barrier
    issue(j + kBgStages - 1);
  }
  MOEFP8_WAIT_VMCNT(0);
  // the workgroup's next unit, claimed now so that the atomic overlaps the epilogue
  if (threadIdx.x == 0) *next_s = grab_unit(pl.queues, n_units);

  // epilogue: C = silu(gate) * up, per-row max over the unit's 128 columns, hi/lo split
  const int col0 = cb * kBlock + 32 * wn;
  float c[NT][2][4];
#pragma unroll
  for (int i = 0; i < NT; i++)
#pragma unroll
    for (int jn = 0; jn < 2; jn++)
#pragma unroll
      for (int r = 0; r < 4; r++) c[i][jn][r] = silu_f32(acc[i][jn + 2][r]) * acc[i][jn][r];
#pragma unroll
  for (int i = 0; i < NT; i++) {
    const int t = tile(i);
#pragma unroll
    for (int r = 0; r < 4; r++) {
      float m = fmaxf(fabsf(c[i][0][r]), fabsf(c[i][1][r]));
      m = fmaxf(m, dpp_f32<kDppXor1>(m));
      m = fmaxf(m, dpp_f32<kDppXor2>(m));
      m = fmaxf(m, dpp_f32<kDppHalfMirror>(m));
      m = fmaxf(m, dpp_f32<kDppRowMirror>(m));
      if (lr == 0) amax_s[wn][16 * t + 4 * kg + r] = m;
    }
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < NT; i++) {
    const int t = tile(i);
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int R = 16 * t + 4 * kg + r;
      if (!rm.valid(R)) continue;
      const float amax = fmaxf(fmaxf(amax_s[0][R], amax_s[1][R]), fmaxf(amax_s[2][R], amax_s[3][R]));
      float inv, scale;
      split_scale(amax, inv, scale);
      const size_t p = (size_t)rm.src(R);
#pragma unroll
      for (int jn = 0; jn < 2; jn++) store_c(ch, p, I, col0 + 16 * jn + lr, c[i][jn][r], inv);
      if (wn == 0 && lr == 0) ch.scale[p * NCB + cb] = scale;
    }
  }
}

// Units (m-block, 128 C columns) over the blocks (128-row class 0/1 blocks, mixed blocks and
// 32-row exact-product blocks).
// One workgroup per CU (its LDS ring), i.e. two wavefronts per SIMD: stated, so that the compiler
// schedules the K loop for that occupancy instead of squeezing registers for three.
__global__ __launch_bounds__(kBgThreads, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm1_big_kernel(
    Problem pb, Plan pl, CHalf8 ch) {
  __shared__ __attribute__((aligned(16))) uint8_t ring[kBgStages * kBgStage];
  __shared__ __attribute__((aligned(16))) float2 sw_s[kBigMaxKB];
  __shared__ float amax_s[4][kBgRows];
  const int H = pb.H, I = pb.I, KB = H / kBlock, NCB = I / kBlock;
  // where wavefronts 2..7 put their row-scale DMA (never read)
  __shared__ __attribute__((aligned(16))) uint32_t dma_sink[64];
  const uint32_t sink_lds = uniform((int)lds_addr(dma_sink));
  __shared__ int next_s;
  const uint32_t ring_lds = uniform((int)lds_addr(ring));
  const int n_units = pl.info[2] * NCB;
  if (threadIdx.x == 0) next_s = first_unit(pl.queues, n_units);
  __syncthreads();
  for (int v = uniform(next_s); v >= 0; v = uniform(next_s)) {
    const int2 uc = unit_at(pl.mbgroup, v, NCB);
    const int mb = uniform(uc.x), cb = uniform(uc.y);
    const int4 blk = pl.mblocks[mb];
    const int e = uniform(blk.x), row0 = uniform(blk.y), rows = uniform(blk.z), flags = uniform(blk.w);
    const bool once = uniform(pl.mbgroup[mb].y) == 1;   // the expert's only m-block
    // the previous unit's readers are done with the ring, amax_s and sw_s, and every thread has
    // read next_s
    __syncthreads();
    // weight scales of the unit: {up, gate} per K-block
    {
      const float* su = pb.s13 + ((size_t)e * (2 * I / kBlock) + cb) * KB;
      const float* sg = su + (size_t)NCB * KB;
      const int t = threadIdx.x;
      if (t < KB) sw_s[t] = float2{su[t], sg[t]};
    }
    __syncthreads();
    const RowMap rm = row_map(row0, rows, flags);
    const int wm = wave_index() & 1;
#define MOEFP8_G1_UNIT(NF, NX, TF0, TX0) \
  gemm1_big_mixed_unit<NF, NX>(pb, pl, ch, ring, ring_lds, sink_lds, sw_s, amax_s, e, rm, cb, TF0, TX0, &next_s, \
                               n_units)
    if (flags & kFlagMixed) {
      const TileSplit ts = mixed_split(rm, wm);
      const int nf = uniform(ts.nf), tf0 = uniform(ts.tf0), tx0 = uniform(ts.tx0);
      if (ts.nx == 0) {
        if (nf == 1) MOEFP8_G1_UNIT(1, 0, tf0, 0);
        else if (nf == 2) MOEFP8_G1_UNIT(2, 0, tf0, 0);
        else if (nf == 3) MOEFP8_G1_UNIT(3, 0, tf0, 0);
        else MOEFP8_G1_UNIT(4, 0, tf0, 0);
      } else {
        if (nf == 0) MOEFP8_G1_UNIT(0, 1, 0, tx0);
        else if (nf == 1) MOEFP8_G1_UNIT(1, 1, tf0, tx0);
        else if (nf == 2) MOEFP8_G1_UNIT(2, 1, tf0, tx0);
        else MOEFP8_G1_UNIT(3, 1, tf0, tx0);
      }
    } else {
#define MOEFP8_G1_REG(NT, EXACT) \
  if (once) gemm1_big_unit<NT, EXACT, true>(pb, pl, ch, ring, ring_lds, sink_lds, sw_s, amax_s, e, row0, rows, cb, \
                                            &next_s, n_units); \
  else gemm1_big_unit<NT, EXACT, false>(pb, pl, ch, ring, ring_lds, sink_lds, sw_s, amax_s, e, row0, rows, cb, \
                                        &next_s, n_units)
      if (flags & kFlagExactProducts) {
        MOEFP8_G1_REG(1, true);
      } else if (rows <= 32) {
        MOEFP8_G1_REG(1, false);
      } else if (rows <= 64) {
        MOEFP8_G1_REG(2, false);
      } else {
        MOEFP8_G1_REG(4, false);
      }
#undef MOEFP8_G1_REG
    }
#undef MOEFP8_G1_UNIT
    // next_s is written
    __syncthreads();
  }
}

// ------------------------------------------------------------------------------------------ GEMM2
// Modes of an m-block: one term (C's hi only, MT m-tiles per pass), or two terms (hi and the f16
// lo term, for blocks GEMM1 flagged; MT/2 m-tiles per pass so that both planes fit the stage).
constexpr int kOneTerm = 0, kTwoTerms = 1;

// LDS stage: [hi: MT x 4096 B][4 x 64 row scales].  An m-tile's hi (and lo) term is [16 chunks of
// 16 B][16 rows][16 B].  The two-term mode puts its NP = MT/2 m-tiles of hi at 0 and of lo at
// NP x 4096.
template <int MT>
struct G2L {
  static constexpr int kHi = MT * 4096;
  static constexpr int kScales = kHi;
  static constexpr int kStage = kScales + kLgWaves * 64 * 4;
};

// Vector-memory operations per wavefront and K step: hi DMAs (one 1 KB quarter of each m-tile),
// lo DMAs, the row-scale DMA and 2 weight tiles x 2 loads.
template <int NP, int kMode>
constexpr int g2_ops() {
  return NP + (kMode == kTwoTerms ? NP : 0) + 1 + 4;
}

// One pass over K for m-tiles [i0, i0 + NP) of the unit's m-block.  As in GEMM1, every m-tile
// of the pass is computed and a K step has no branch between an MFMA and the instructions that
// read its result.
template <int MT, int NP, int kMode>
__device__ __forceinline__ void gemm2_large_pass(const Problem& pb, const CHalf8& ch, uint8_t* ring, int e, int row0,
                                                 int rows, int hb, int i0, v4f (&acc)[NP][2]) {
  using L = G2L<MT>;
  constexpr int kLoDma = kMode == kTwoTerms ? NP : 0;
  const int H = pb.H, I = pb.I, KB = I / kBlock, HB = H / kBlock;
  const int wave = wave_index(), lane = lane_id(), lr = lane & 15, kg = lane >> 4;
  const uint8_t* bp = pb.w2 + ((size_t)e * H + hb * kBlock + 32 * wave + lr) * I + kg * 32;
  const float* swp = pb.s2 + ((size_t)e * HB + hb) * KB;
  // hi and lo DMAs: wave w carries quarter w of every m-tile
  const _Float16* hsrc[NP];
#pragma unroll
  for (int i = 0; i < NP; i++) {
    const int p = row0 + min(16 * (i0 + i) + lr, rows - 1);
    hsrc[i] = ch.hi + (size_t)p * I + (4 * wave + kg) * 8;
  }
  const uint8_t* lsrc[kLoDma > 0 ? kLoDma : 1];
#pragma unroll
  for (int r = 0; r < kLoDma; r++) {
    const int p = row0 + min(16 * (i0 + r) + lr, rows - 1);
    lsrc[r] = reinterpret_cast<const uint8_t*>(ch.lo16 + (size_t)p * I + (4 * wave + kg) * 8);
  }
  const float* ssrc = ch.scale + (size_t)(row0 + min(16 * i0 + 64 * wave + lane, rows - 1)) * KB;

  v8i B[kLgDepth][2];
  float SW[kLgDepth];
  auto issue = [&](int d, int j) {
    const int k = min(j, KB - 1);
    uint8_t* st = ring + (j % kLgStages) * L::kStage;
#pragma unroll
    for (int i = 0; i < NP; i++)
      __builtin_amdgcn_global_load_lds(hsrc[i] + (size_t)k * kBlock, st + i * 4096 + wave * 1024, 16, 0, 0);
#pragma unroll
    for (int r = 0; r < kLoDma; r++)
      __builtin_amdgcn_global_load_lds(lsrc[r] + (size_t)k * kBlock * 2, st + (NP + r) * 4096 + wave * 1024, 16, 0,
                                       0);
    __builtin_amdgcn_global_load_lds(ssrc + k, st + L::kScales + wave * 256, 4, 0, 0);
    const uint8_t* b = bp + (size_t)k * kBlock;
    B[d][0] = load_w(b);
    B[d][1] = load_w(b + (size_t)16 * I);
    SW[d] = load_uniform(swp + k);
  };
  auto step = [&](int d, int j) {
    // at most the operations of the following kLgDepth - 1 steps may still be in flight
    wait_vmcnt<(kLgDepth - 1) * g2_ops<NP, kMode>()>();
    __builtin_amdgcn_s_barrier();
    const uint8_t* st = ring + (j % kLgStages) * L::kStage;
    v8h b16[2][4];
    widen_fp8_operand(B[d][0], b16[0]);
    widen_fp8_operand(B[d][1], b16[1]);
#pragma unroll
    for (int i = 0; i < NP; i++) {
      const uint8_t* ti = st + i * 4096;
      v4i h0, h1, h2, h3, s4;
      lds_read5(lds_addr(ti + ((4 * kg + 0) * 16 + lr) * 16), lds_addr(ti + ((4 * kg + 1) * 16 + lr) * 16),
                lds_addr(ti + ((4 * kg + 2) * 16 + lr) * 16), lds_addr(ti + ((4 * kg + 3) * 16 + lr) * 16),
                lds_addr(st + L::kScales + (16 * i + 4 * kg) * 4), h0, h1, h2, h3, s4);
      const v8h ah[4] = {as_v8h(h0), as_v8h(h1), as_v8h(h2), as_v8h(h3)};
      const float4 sa = __builtin_bit_cast(float4, s4);
      v8h al16[4] = {};
      if constexpr (kMode == kTwoTerms) {
        const uint8_t* tl = st + (NP + i) * 4096;
        v4i l0, l1, l2, l3;
        lds_read4(lds_addr(tl + ((4 * kg + 0) * 16 + lr) * 16), lds_addr(tl + ((4 * kg + 1) * 16 + lr) * 16),
                  lds_addr(tl + ((4 * kg + 2) * 16 + lr) * 16), lds_addr(tl + ((4 * kg + 3) * 16 + lr) * 16), l0, l1,
                  l2, l3);
        al16[0] = as_v8h(l0);
        al16[1] = as_v8h(l1);
        al16[2] = as_v8h(l2);
        al16[3] = as_v8h(l3);
      }
#pragma unroll
      for (int n = 0; n < 2; n++) {
        v4f p = mfma_f16_block(ah, b16[n], v4f{0.f, 0.f, 0.f, 0.f});
        if constexpr (kMode == kTwoTerms) p = mfma_f16_block(al16, b16[n], p);
        acc[i][n][0] += p[0] * (sa.x * SW[d]);
        acc[i][n][1] += p[1] * (sa.y * SW[d]);
        acc[i][n][2] += p[2] * (sa.z * SW[d]);
        acc[i][n][3] += p[3] * (sa.w * SW[d]);
      }
    }
    issue(d, j + kLgDepth);
    __builtin_amdgcn_sched_barrier(0);
  };

  __syncthreads();
  // stage d's operations must all be issued before stage d + 1's: the per-step vmcnt wait
  // counts operations in issue order
#pragma unroll
  for (int d = 0; d < kLgDepth; d++) {
    issue(d, d);
    __builtin_amdgcn_sched_barrier(0);
  }
  int j = 0;
  for (; j + 2 * kLgDepth <= KB; j += 2 * kLgDepth) {
#pragma unroll
    for (int d = 0; d < 2 * kLgDepth; d++) step(d % kLgDepth, j + d);
  }
  for (; j < KB; j += kLgDepth) {
#pragma unroll
    for (int d = 0; d < kLgDepth; d++)
      if (j + d < KB) step(d, j + d);
  }
  // no DMA may still target the ring when the next pass refills it or the workgroup ends
  wait_vmcnt<0>();
}

// O rows of m-tiles [i0, i0 + NP), scaled by the routing weight.
template <int NP>
__device__ __forceinline__ void gemm2_large_store(const Plan& pl, float* __restrict__ obuf, int H, int row0, int rows,
                                                  int hb, int i0, const v4f (&acc)[NP][2]) {
  const int wave = wave_index(), lane = lane_id(), lr = lane & 15, kg = lane >> 4;
#pragma unroll
  for (int i = 0; i < NP; i++) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int row = 16 * (i0 + i) + 4 * kg + r;
      if (row < rows) {
        const int p = row0 + row;
        const float w = pl.perm_w[p];
#pragma unroll
        for (int n = 0; n < 2; n++) obuf[(size_t)p * H + hb * kBlock + 32 * wave + 16 * n + lr] = acc[i][n][r] * w;
      }
    }
  }
}

// Units (m-block, 128 output columns) over GEMM2's blocks; a block taller than 16 MT rows is taken
// 16 MT rows at a time.
template <int MT>
__global__ __launch_bounds__(kLgThreads, 2) void gemm2_large_kernel(Problem pb, Plan pl, CHalf8 ch,
                                                                     float* __restrict__ obuf) {
  using L = G2L<MT>;
  constexpr int NP = MT / 2;
  __shared__ __attribute__((aligned(16))) uint8_t ring[kLgStages * L::kStage];
  const int H = pb.H, HB = H / kBlock;
  const UnitEighths u;
  const int n_units = pl.info[2] * HB, end = u.lo(n_units, u.x + 1);
  for (int v = u.lo(n_units, u.x) + (int)blockIdx.x / u.nx; v < end; v += u.per) {
    const int2 uc = unit_at(pl.mbgroup, v, HB);
    const int mb = uniform(uc.x), hb = uniform(uc.y);
    const int4 blk = pl.mblocks[mb];
    const int e = uniform(blk.x);
    const bool two = uniform(pl.two_term[mb]) != 0;
    for (int s0 = 0; s0 < blk.z; s0 += 16 * MT) {
      const int row0 = uniform(blk.y + s0), rows = uniform(min(16 * MT, blk.z - s0));
      const int mvalid = (rows + 15) / 16;
      if (two) {
        for (int i0 = 0; i0 < mvalid; i0 += NP) {
          v4f acc[NP][2];
#pragma unroll
          for (int i = 0; i < NP; i++) acc[i][0] = acc[i][1] = v4f{0.f, 0.f, 0.f, 0.f};
          gemm2_large_pass<MT, NP, kTwoTerms>(pb, ch, ring, e, row0, rows, hb, i0, acc);
          gemm2_large_store<NP>(pl, obuf, H, row0, rows, hb, i0, acc);
        }
      } else {
        v4f acc[MT][2];
#pragma unroll
        for (int i = 0; i < MT; i++) acc[i][0] = acc[i][1] = v4f{0.f, 0.f, 0.f, 0.f};
        gemm2_large_pass<MT, MT, kOneTerm>(pb, ch, ring, e, row0, rows, hb, 0, acc);
        gemm2_large_store<MT>(pl, obuf, H, row0, rows, hb, 0, acc);
      }
    }
  }
}

// ------------------------------------------------------------------------------ GEMM2, 128-row m-blocks
// For the 128-row blocks.  A workgroup of 8 wavefronts (one per CU, two per SIMD) owns one unit =
// (m-block, 256 output columns) and stages C's hi term (f16), in blocks GEMM1 flagged also its lo
// term (f16), and the W2 rows by DMA through a 3-stage LDS ring, 64 K per stage.  Wavefront
// (wm, wn) = (w % 2, w / 2) computes rows 64 wm .. +63 x output columns 64 wn .. +63 on the f16
// MFMA 16x16x32 (W2 widened to f16 exactly; the lo term's products chained onto the hi ones).
// The block's rows come through its row map (a mixed block keeps its exact-product rows in its
// last m-tiles; GEMM2 treats them like the others).
//
// Within a 64-K stage, lane group kg of an MFMA operand holds k = 16 kg + 8 t + (0..7) for the
// two 32-K MFMAs t = 0, 1 (the same order for both operands): its W2 bytes are one 16-byte
// chunk, its hi (and lo) values two.
//
// LDS stage: hi [128 rows][128 B] and lo [128 rows][128 B] (chunks swizzled by slot_key8), W2
// [256 rows][64 B] (chunk c of row r in slot c ^ bg_key4(r)), 128 row scales of C.
constexpr int kB2Cols = 256;
constexpr int kB2Hi = kBgRows * 128;
constexpr int kB2Lo = kBgRows * 128;
constexpr int kB2W = kB2Cols * 64;
constexpr int kB2Stage = kB2Hi + kB2Lo + kB2W + kBgRows * 4;
constexpr int kB2Stages = 3;

// 4-slot swizzle of 64-byte rows: chunk c of row r sits in slot c ^ key(r), key linear in the row
// bits 1, 2, 3 (weights 1, 2, 3).  An MFMA operand read has lanes (row r = 0..15, chunk kg), and the
// slots are conflict-free whether the LDS serves a 16-byte read 8, 16 or 32 lanes at a time (over
// 128, 256 or 512 bytes of banks): 8 rows of one parity, 16 consecutive rows and rows r, r + 8 with
// kg, kg ^ 1 all land on distinct 16-byte bank groups.
__device__ __forceinline__ int bg_key4(int row) { return ((row >> 1) & 3) ^ (((row >> 3) & 1) * 3); }

// e4m3 x 16 -> two f16 x 8 (MFMA operand order k = 8t + 0..7), exactly
__device__ __forceinline__ void widen16(const v4i& x, v8h& t0, v8h& t1) {
#pragma unroll
  for (int w = 0; w < 4; w++) {
    const uint32_t word = (uint32_t)x[w];
    const v2h lo = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(word, 1.0f, false);
    const v2h hi = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(word, 1.0f, true);
    v8h& t = w < 2 ? t0 : t1;
    const int o = 4 * (w & 1);
    t[o + 0] = lo[0];
    t[o + 1] = lo[1];
    t[o + 2] = hi[0];
    t[o + 3] = hi[1];
  }
}

// GEMM2's rows of a unit: LDS row R holds pair rowp[R] (staged in LDS from the row table, rows
// past the block's last repeating it: computed, never stored).
struct G2Rows {
  const int* rowp;
  int rows;
  __device__ __forceinline__ int src(int R) const { return rowp[R]; }
  __device__ __forceinline__ bool valid(int R) const { return R < rows; }
};

// One unit.  Wavefront (wm, wn) computes m-tiles NT wm .. NT wm + NT - 1 (NT = 4, 2 or 1 for
// blocks whose rows reach past LDS row 64, 32, or not).  kTwo: C's lo term too.
template <bool kTwo, int NT>
__device__ __forceinline__ void gemm2_big_unit(const Problem& pb, const Plan& pl, const CHalf8& ch, uint8_t* ring,
                                               uint32_t ring_lds, const float* sw2_s, const float* pw_s, int e,
                                               const G2Rows& rm, int hc, float* __restrict__ obuf, int ocol0,
                                               int ocols, int orows, int* queues, int* next_s, int n_units) {
  static_assert(NT == 1 || NT == 2 || NT == 4, "m-tiles per wavefront");
  const int H = pb.H, I = pb.I, KB = I / kBlock, KS = I / 64;
  // lane-dependent addresses are formed per unit (hoisted out of the unit loop, some of them spill)
  int lane = lane_id();
  asm volatile("" : "+v"(lane));
  const int wave = wave_index(), lr = lane & 15, kg = lane >> 4;
  const int wm = wave & 1, wn = wave >> 1;
  // DMA roles.  A stage waits for its slowest wavefront, and every DMA instruction costs the
  // wavefront that issues it, so each wavefront issues only DMAs of rows the block computes, and
  // the row scales go with the odd 64-K stage of a 128-K block only (the stage that applies them):
  // GEMM2 114 -> 112, 229 -> 217 and 410 -> 389 µs at T = 1024 / 5000 / 8192 against every
  // wavefront DMAing 16 rows of hi (and lo) and the scales each stage (measured).
  //   hi / lo rows, in groups of 8 (one DMA each): NT = 4, groups 2w and 2w + 1; NT = 2 (rows <=
  //   64), group w; NT = 1 (rows <= 32), groups 0..3 by waves 2..5.
  //   W2 rows 32w + 16q + (lane / 4), 4 slots per row, 2 DMAs per wavefront.
  //   row scales: NT = 4, rows 64 (w % 2) + lane by waves 0 and 1; NT = 2 / 1, rows 0..63 by
  //   wave 0 / 6.
  constexpr int kHiPer = NT == 4 ? 2 : 1;
  const int hi0 = NT == 4 ? 2 * wave : NT == 2 ? wave : max(wave - 2, 0);   // first group carried
  const bool hcar = NT != 1 || (wave >= 2 && wave < 6);
  const bool scar = NT == 4 ? wave < 2 : NT == 2 ? wave == 0 : wave == 6;
  const int sslot = NT == 4 ? (wave & 1) : 0;
  const int n_even = 2 + (hcar ? kHiPer * (kTwo ? 2 : 1) : 0);   // DMAs of an even stage
  const int n_odd = n_even + (scar ? 1 : 0);                      // of an odd one
  uint32_t hoff[kHiPer], woff[2];
#pragma unroll
  for (int q = 0; q < kHiPer; q++) {
    const int r = 8 * (hi0 + q) + (lane >> 3);
    hoff[q] = (uint32_t)clamp_index(rm.src(r), pl.pair_rows) * (uint32_t)(2 * I) +
              (uint32_t)((((lane & 7) ^ slot_key8(r))) * 16);
  }
#pragma unroll
  for (int q = 0; q < 2; q++) {
    const int R = 32 * wave + 16 * q + (lane >> 2);
    woff[q] = (uint32_t)(hc * kB2Cols + R) * (uint32_t)I + (uint32_t)((((lane & 3) ^ bg_key4(R))) * 16);
  }
  const uint32_t soff = 4u * (uint32_t)(clamp_index(rm.src(64 * sslot + lane), pl.pair_rows) * KB);
  const uint8_t* wbase = pb.w2 + (size_t)e * H * I;
  auto issue = [&](int j) {
    const int k = min(j, KS - 1);
    const uint32_t st = ring_lds + (uint32_t)((j % kB2Stages) * kB2Stage);
    const uint8_t* hbase = reinterpret_cast<const uint8_t*>(ch.hi) + (size_t)k * 128;
    if (hcar) {
#pragma unroll
      for (int q = 0; q < kHiPer; q++) dma_lds16_s(hoff[q], hbase, st + 8 * (hi0 + q) * 128);
      if (kTwo) {
        const uint8_t* lbase = reinterpret_cast<const uint8_t*>(ch.lo16) + (size_t)k * 128;
#pragma unroll
        for (int q = 0; q < kHiPer; q++) dma_lds16_s(hoff[q], lbase, st + kB2Hi + 8 * (hi0 + q) * 128);
      }
    }
#pragma unroll
    for (int q = 0; q < 2; q++)
      dma_lds16_s(woff[q], wbase + (size_t)k * 64, st + kB2Hi + kB2Lo + (32 * wave + 16 * q) * 64);
    if (scar && (j & 1)) dma_lds4_s(soff, ch.scale + k / 2, st + kB2Hi + kB2Lo + kB2W + sslot * 256);
  };
  // operand read offsets: hi / lo chunks 2kg + t of row lr (slot_key8), W2 chunk kg of row lr (bg_key4)
  const int rh0 = lr * 128 + (((2 * kg) ^ slot_key8(lr)) * 16);
  const int rh1 = lr * 128 + (((2 * kg + 1) ^ slot_key8(lr)) * 16);
  const int rq = lr * 64 + ((kg ^ bg_key4(lr)) * 16);

  MOEFP8_WAIT_VMCNT(0);
  for (int d = 0; d < kB2Stages - 1; d++) issue(d);
  v4f acc[NT][4];
#pragma unroll
  for (int i = 0; i < NT; i++)
#pragma unroll
    for (int n = 0; n < 4; n++) acc[i][n] = v4f{0.f, 0.f, 0.f, 0.f};
  // The two 64-K stages of a 128-K scale block chain their MFMAs into one product per tile
  // (pp), scaled into acc once per block: half the scale FMAs and products of a stage each.
  v4f pp[NT][4];
  auto stage = [&](int j, auto first_c) {
    constexpr bool kFirst = decltype(first_c)::value;
    // one stage in flight past the current one: stage j + 1's DMAs (an odd stage's when j is even)
    static_assert(kB2Stages == 3, "wait count");
    wait_vmcnt_2to7(kFirst ? n_odd : n_even);
    barrier_lds();
    const uint8_t* st = ring + (j % kB2Stages) * kB2Stage;
    v8h b16[4][2];
#pragma unroll
    for (int n = 0; n < 4; n++)
      widen16(*reinterpret_cast<const v4i*>(st + kB2Hi + kB2Lo + (64 * wn + 16 * n) * 64 + rq), b16[n][0], b16[n][1]);
    const float sw = sw2_s[(j / 2) * 2 + (wn >> 1)];
#pragma unroll
    for (int i = 0; i < NT; i++) {
      const int t = NT * wm + i;
      const uint8_t* ht = st + t * 16 * 128;
      const v8h a0 = as_v8h(*reinterpret_cast<const v4i*>(ht + rh0));
      const v8h a1 = as_v8h(*reinterpret_cast<const v4i*>(ht + rh1));
      v8h l0 = {}, l1 = {};
      if constexpr (kTwo) {
        l0 = as_v8h(*reinterpret_cast<const v4i*>(ht + kB2Hi + rh0));
        l1 = as_v8h(*reinterpret_cast<const v4i*>(ht + kB2Hi + rh1));
      }
#pragma unroll
      for (int n = 0; n < 4; n++) {
        v4f p = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b16[n][0], kFirst ? v4f{0.f, 0.f, 0.f, 0.f} : pp[i][n],
                                                       0, 0, 0);
        p = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b16[n][1], p, 0, 0, 0);
        if constexpr (kTwo) {
          p = __builtin_amdgcn_mfma_f32_16x16x32_f16(l0, b16[n][0], p, 0, 0, 0);
          p = __builtin_amdgcn_mfma_f32_16x16x32_f16(l1, b16[n][1], p, 0, 0, 0);
        }
        pp[i][n] = p;
      }
      if constexpr (!kFirst) {
        const float4 sa = *reinterpret_cast<const float4*>(st + kB2Hi + kB2Lo + kB2W + (16 * t + 4 * kg) * 4);
        const float4 sc = {sa.x * sw, sa.y * sw, sa.z * sw, sa.w * sw};
#pragma unroll
        for (int n = 0; n < 4; n++) {
          acc[i][n][0] += pp[i][n][0] * sc.x;
          acc[i][n][1] += pp[i][n][1] * sc.y;
          acc[i][n][2] += pp[i][n][2] * sc.z;
          acc[i][n][3] += pp[i][n][3] * sc.w;
        }
      }
    }
    issue(j + kB2Stages - 1);
  };
  // KS = I / 64 is even (I is a multiple of 128)
  for (int j = 0; j < KS; j += 2) {
    stage(j, std::true_type{});
    stage(j + 1, std::false_type{});
  }
  MOEFP8_WAIT_VMCNT(0);
  // the workgroup's next unit, claimed now so that the atomic overlaps the epilogue
  if (threadIdx.x == 0) *next_s = grab_unit(queues, n_units);
#pragma unroll
  for (int i = 0; i < NT; i++) {
    const int t = NT * wm + i;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int R = 16 * t + 4 * kg + r;
      if (rm.valid(R)) {
        const int p = clamp_index(rm.src(R), orows);
        const float w = pw_s[R];
#pragma unroll
        for (int n = 0; n < 4; n++) obuf[(size_t)p * ocols + ocol0 + 64 * wn + 16 * n + lr] = acc[i][n][r] * w;
      }
    }
  }
}

// Units (m-block, 256 output columns) over GEMM2's own row table (Plan::g2_*): an expert's
// one-term blocks, then its two-term blocks; the column blocks of output pass `pass` (out_pass),
// written to O rows of the pass's length from column 0; `pass` also picks the pass's unit queues.
__global__ __launch_bounds__(kBgThreads, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm2_big_kernel(
    Problem pb, Plan pl, CHalf8 ch, float* __restrict__ obuf, int o_rows, int pass) {
  __shared__ __attribute__((aligned(16))) uint8_t ring[kB2Stages * kB2Stage];
  __shared__ float sw2_s[2 * kBigMaxKB];
  __shared__ float pw_s[kBgRows];
  __shared__ int rowp_s[kBgRows];
  // the row table's groups: per expert its first GEMM2 row, one- and two-term row counts, first block
  __shared__ int g_off[kEGlobal + 1], g_c1[kEGlobal], g_c2[kEGlobal], g_first[kEGlobal + 1];
  const int H = pb.H, I = pb.I, KB = I / kBlock, HB = H / kBlock, E = pb.E_local;
  __shared__ int next_s;
  const uint32_t ring_lds = uniform((int)lds_addr(ring));
  const OutPass op = out_pass(pl.info[0], H, o_rows, pass, pl.pair_rows);
  const int hc0 = op.c0 / kB2Cols, hcn = (op.c1 - op.c0) / kB2Cols, ocols = op.ocols;
  // a pass without columns (the second, for a call whose pairs fit O's rows) ends here, before
  // any queue is touched
  if (hcn == 0) return;
  for (int i = threadIdx.x; i <= E; i += blockDim.x) {
    g_off[i] = pl.expert_offsets[i];
    if (i < E) {
      g_c1[i] = pl.g2_ctl[2 * i];
      g_c2[i] = pl.g2_ctl[2 * i + 1];
    }
  }
  __syncthreads();
  // blocks of up to 128 rows per group, numbered expert by expert
  if (threadIdx.x < kWave) {
    int carry = 0;
    for (int e0 = 0; e0 < E; e0 += kWave) {
      const int ee = e0 + (int)threadIdx.x;
      const int nb = ee < E ? (g_c1[ee] + kBgRows - 1) / kBgRows + (g_c2[ee] + kBgRows - 1) / kBgRows : 0;
      const int first = carry + wave_exclusive_sum(nb);
      if (ee < E) g_first[ee] = first;
      carry = __builtin_amdgcn_readlane(first + nb, kWave - 1);
    }
    if (threadIdx.x == 0) g_first[E] = carry;
  }
  __syncthreads();
  const int n_units = g_first[E] * hcn;
  int* queues = pl.queues + (8 + 8 * pass) * kQueueStride;
  if (threadIdx.x == 0) next_s = first_unit(queues, n_units);
  __syncthreads();
  for (int v = uniform(next_s); v >= 0; v = uniform(next_s)) {
    // unit v -> expert (the last whose first unit is <= v; empty experts share their successor's),
    // then column block and block, the expert's blocks innermost; the block's group and rows
    int lo = 0, hi = E;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (g_first[mid] * hcn <= v) lo = mid;
      else hi = mid;
    }
    const int e = uniform(lo), nb = g_first[e + 1] - g_first[e], local = v - g_first[e] * hcn;
    const int hcl = uniform(local / nb), hc = hc0 + hcl, b = local % nb;
    const int c1 = g_c1[e], b1 = (c1 + kBgRows - 1) / kBgRows;
    const bool two = uniform(b >= b1 ? 1 : 0) != 0;
    const int j = two ? b - b1 : b;
    const int row0 = uniform(g_off[e] + (two ? c1 : 0) + kBgRows * j);
    const int rows = uniform(min(kBgRows, (two ? g_c2[e] : c1) - kBgRows * j));
    // the previous unit's readers are done with the ring, sw2_s, pw_s and rowp_s, and every thread
    // has read next_s
    __syncthreads();
    // W2 block scales of the unit's two 128-column blocks, per 128-K block, and each LDS row's pair
    // and routing weight (for the DMA sources and the epilogue)
    {
      const int t = threadIdx.x;
      if (t < 2 * KB) sw2_s[t] = pb.s2[((size_t)e * HB + 2 * hc + (t & 1)) * KB + (t >> 1)];
      if (t < kBgRows) {
        const int p = clamp_index(pl.g2_pair[row0 + min(t, rows - 1)], pl.pair_rows);
        rowp_s[t] = p;
        pw_s[t] = pl.perm_w[p];
      }
    }
    __syncthreads();
    const G2Rows rm{rowp_s, rows};
#define MOEFP8_G2_UNIT(TWO, NT)                                                                               \
  gemm2_big_unit<TWO, NT>(pb, pl, ch, ring, ring_lds, sw2_s, pw_s, e, rm, hc, obuf, hcl * kB2Cols, ocols,          \
                          op.rows_cap, queues, &next_s, n_units)
    if (two) {
      if (rows <= 32) MOEFP8_G2_UNIT(true, 1);
      else if (rows <= 64) MOEFP8_G2_UNIT(true, 2);
      else MOEFP8_G2_UNIT(true, 4);
    } else {
      if (rows <= 32) MOEFP8_G2_UNIT(false, 1);
      else if (rows <= 64) MOEFP8_G2_UNIT(false, 2);
      else MOEFP8_G2_UNIT(false, 4);
    }
#undef MOEFP8_G2_UNIT
    // next_s is written
    __syncthreads();
  }
}

// ------------------------------------------------------------------------------------------ flags
// GEMM2's precision flag of m-block g: two terms of C where the permutation's estimate put class 1
// rows (kFlagTwoTermC), or where one of the block's rows needs them by its measured C
// (needs_two_terms on the row's max |C| per 128 columns, 448 x the scales GEMM1 wrote).  A launch
// of its own between the GEMMs: the same test inside GEMM1's epilogue made the compiler schedule
// GEMM1's K loop worse.
__global__ __launch_bounds__(256) void c_flags_kernel(Plan pl, CHalf8 ch, int I) {
  constexpr int kBatch = 8;   // scales per thread loaded together (a 128-row block at I = 2048: all)
  const int g = blockIdx.x;
  // the block count and the block (the table holds the launch's grid of entries) in one round of
  // loads, then the block's scales, routing weights and W2 estimate in another
  const int n_blocks = pl.info[2];
  const int4 blk = pl.mblocks[g];
  if (g >= n_blocks) return;
  // a mixed block's exact rows follow its regular rows
  const int n = blk.z + ((blk.w & kFlagMixed) ? (blk.w >> kMixedShift) : 0);
  const int NCB = I / kBlock, total = n * NCB;
  const float sqrt_i = sqrtf((float)I);
  bool need = (blk.w & kFlagTwoTermC) != 0;
  for (int i0 = 0; i0 < total; i0 += kBatch * (int)blockDim.x) {
    float sc[kBatch], w[kBatch];
#pragma unroll
    for (int q = 0; q < kBatch; q++) {
      const int i = min(i0 + q * (int)blockDim.x + (int)threadIdx.x, total - 1);
      const int p = blk.y + i / NCB;
      sc[q] = ch.scale[(size_t)p * NCB + i % NCB];
      w[q] = pl.perm_w[p];
    }
    const float sigma2 = pl.esig[2 * blk.x + 1];
#pragma unroll
    for (int q = 0; q < kBatch; q++)
      need |= i0 + q * (int)blockDim.x + (int)threadIdx.x < total && needs_two_terms(w[q], sigma2, 448.0f * sc[q], sqrt_i);
  }
  need = __syncthreads_or(need);
  if (threadIdx.x == 0) pl.two_term[g] = need ? 1 : 0;
}

void launch_c_flags(const Plan& pl, const CHalf8& ch, int I, int max_blocks, hipStream_t stream) {
  if (max_blocks <= 0) return;
  hipLaunchKernelGGL(c_flags_kernel, dim3(max_blocks), dim3(256), 0, stream, pl, ch, I);
}

// GEMM2's row table for the 128-row path.  Thread = pair row p (GEMM1's row order): both f16
// terms of C where needs_two_terms holds on the largest of its C scales (the measured bound q: a row
// at or below kOneTermQ keeps its one-term error within the bound whatever its class), or where the
// row took GEMM1's exact products (magnitude class 2: the expert's rows from xrow[e] on; such rows
// are large enough for either rounding to matter, and stay on 22 bits); its GEMM2 row is claimed
// from the front (one term) or the back (two terms) of its expert's rows, through per-expert
// counters, so that each expert's rows split into a one-term and a two-term group (GEMM2 cuts the
// groups into blocks of up to 128 rows from the counts).  The order inside a group depends on the
// claims, the results do not: every row is computed on its own.
constexpr int kG2PlanThreads = 256;
__global__ __launch_bounds__(kG2PlanThreads) void g2_plan_kernel(Plan pl, CHalf8 ch, int* __restrict__ g2_pair, int E,
                                                                 int I) {
  __shared__ int cnt[2 * kEGlobal], base[2 * kEGlobal];
  __shared__ int eoff[kEGlobal + 1], xs[kEGlobal];
  __shared__ float sig2[kEGlobal];
  const int tid = threadIdx.x, NCB = I / kBlock;
  const int p = blockIdx.x * kG2PlanThreads + tid, pc = min(p, pl.pair_rows - 1);
  // every input in one round of loads: the pair count, the pair's weight and C scales (rows past the
  // call's pairs read in range and are ignored), the experts' offsets, first exact rows and W2 scales
  const int P = pl.info[0];
  const float w = pl.perm_w[pc];
  float smax = 0.f;
  if (NCB % 4 == 0) {
    for (int cb = 0; cb < NCB; cb += 4) {
      const float4 s = *reinterpret_cast<const float4*>(ch.scale + (size_t)pc * NCB + cb);
      smax = fmaxf(fmaxf(smax, fmaxf(s.x, s.y)), fmaxf(s.z, s.w));
    }
  } else {
    for (int cb = 0; cb < NCB; cb++) smax = fmaxf(smax, ch.scale[(size_t)pc * NCB + cb]);
  }
  for (int i = tid; i <= E; i += kG2PlanThreads) {
    eoff[i] = pl.expert_offsets[i];
    if (i < E) {
      xs[i] = pl.xrow[i];
      sig2[i] = pl.esig[2 * i + 1];
    }
  }
  for (int i = tid; i < 2 * E; i += kG2PlanThreads) cnt[i] = 0;
  // workgroups past the last pair have nothing to place
  if ((int)blockIdx.x * kG2PlanThreads >= P) return;
  __syncthreads();
  // the pair's expert: the last e with eoff[e] <= p (empty experts share their successor's offset)
  const int pp = min(p, P - 1);
  int lo = 0, hi = E;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (eoff[mid] <= pp) lo = mid;
    else hi = mid;
  }
  const int e = lo;
  const bool two = pp >= xs[e] || needs_two_terms(w, sig2[e], 448.0f * smax, sqrtf((float)I));
  const int key = 2 * e + (two ? 1 : 0);
  int r = 0;
  if (p < P) r = atomicAdd(&cnt[key], 1);
  __syncthreads();
  for (int i = tid; i < 2 * E; i += kG2PlanThreads)
    if (cnt[i] > 0) base[i] = atomicAdd(&pl.g2_ctl[i], cnt[i]);
  __syncthreads();
  if (p < P) {
    const int pos = two ? eoff[e + 1] - 1 - (base[key] + r) : eoff[e] + base[key] + r;
    g2_pair[pos] = p;
  }
}

void launch_g2_plan(const Problem& pb, const Plan& pl, const CHalf8& ch, int pmax, hipStream_t stream) {
  if (pmax <= 0) return;
  const int grid = (pmax + kG2PlanThreads - 1) / kG2PlanThreads;
  hipLaunchKernelGGL(g2_plan_kernel, dim3(grid), dim3(kG2PlanThreads), 0, stream, pl, ch,
                     const_cast<int*>(pl.g2_pair), pb.E_local, pb.I);
}

// ------------------------------------------------------------------------------------------ launch
int large_grid() { return num_compute_units() * 2; }

void launch_gemm1_large(const Problem& pb, const Plan& pl, const CHalf8& ch, int mt, int max_units,
                        hipStream_t stream) {
  const int grid = max_units < large_grid() ? max_units : large_grid();
  if (grid <= 0) return;
  switch (mt) {
    case 2:
      hipLaunchKernelGGL(gemm1_large_kernel<2>, dim3(grid), dim3(kLgThreads), 0, stream, pb, pl, ch);
      break;
    default:
      hipLaunchKernelGGL(gemm1_large_kernel<4>, dim3(grid), dim3(kLgThreads), 0, stream, pb, pl, ch);
      break;
  }
}

void launch_gemm1_big(const Problem& pb, const Plan& pl, const CHalf8& ch, int max_units, hipStream_t stream) {
  static_assert(kBigRows == kBgRows, "block height");
  const int cus = num_compute_units();
  const int grid = max_units < cus ? max_units : cus;
  if (grid <= 0) return;
  hipLaunchKernelGGL(gemm1_big_kernel, dim3(grid), dim3(kBgThreads), 0, stream, pb, pl, ch);
}

void launch_gemm2_large(const Problem& pb, const Plan& pl, const CHalf8& ch, float* obuf, int mt, int max_units,
                        hipStream_t stream) {
  const int grid = max_units < large_grid() ? max_units : large_grid();
  if (grid <= 0) return;
  switch (mt) {
    case 2:
      hipLaunchKernelGGL(gemm2_large_kernel<2>, dim3(grid), dim3(kLgThreads), 0, stream, pb, pl, ch, obuf);
      break;
    default:
      hipLaunchKernelGGL(gemm2_large_kernel<4>, dim3(grid), dim3(kLgThreads), 0, stream, pb, pl, ch, obuf);
      break;
  }
}

void launch_gemm2_big(const Problem& pb, const Plan& pl, const CHalf8& ch, float* obuf, int max_units, int o_rows,
                      int pass, hipStream_t stream) {
  const int cus = num_compute_units();
  const int grid = max_units < cus ? max_units : cus;
  if (grid <= 0) return;
  hipLaunchKernelGGL(gemm2_big_kernel, dim3(grid), dim3(kBgThreads), 0, stream, pb, pl, ch, obuf, o_rows, pass);
}

}  // namespace moefp8
