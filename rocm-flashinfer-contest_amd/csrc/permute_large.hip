// Permutation of the (token, local expert) pairs for T > 64, in two launches over blocks of
// 256 tokens (one token per thread):
//
//   count  per block, the number of pairs in each bucket (local expert, magnitude class)
//   place  per block, from all blocks' counts (staged in LDS): every bucket's total and this
//          block's prefix of it, hence the bucket and expert offsets; each pair's rank inside its
//          bucket in token order then gives its row, the rank inside its expert alone its
//          canonical row.  Block 0 also writes the offsets and the m-block table of the grouped
//          GEMMs.  (A one-workgroup scan launch between the two took 5-7 us plus a launch
//          boundary at T = 1024-8192; every block redoing the sums it needs costs it one round of
//          loads.)
//
// Rows of an expert are grouped by magnitude class (class 0 first), each group in token
// order, so pairs that need the exact-product or two-term paths share m-tiles instead of
// spreading over all of them.  The canonical order -- for each local expert in
// ascending order, its tokens ascending, as torch.nonzero yields them in
// solutions/moe_fp8/main.py:216-226 -- is written separately (canon_token) for callers
// that ask for the permutation.  Everything is a deterministic function of the routing.
#include "moefp8_device.h"
#include "moefp8_launch.h"

namespace moefp8 {

constexpr int kBlkTokens = 256;
constexpr int kBlkWaves = kBlkTokens / kWave;
constexpr int kClasses = 3;

// 0: one f16 term of C is enough; 1: two terms; 2: two terms and exact GEMM1 products (GEMM2
// may still take two terms for a class 0 block, from the C that GEMM1 writes).
__device__ __forceinline__ int magnitude_class(float pred) {
  return pred > kPreciseRms ? 2 : (pred > kOneTermRms ? 1 : 0);
}

__device__ __forceinline__ int class_flags(int c) {
  return c == 0 ? 0 : (c == 1 ? kFlagTwoTermC : kFlagTwoTermC | kFlagExactProducts);
}

// Does an expert with n01 class 0/1 rows and n2 exact-product rows fold the latter into its last
// class 0/1 block (a mixed block: the exact rows take the block's last ceil(n2 / 16) m-tiles)?
// Only with 128-row blocks, at most 32 exact rows and room for them.
__device__ __forceinline__ bool folds_exact(const LargePermArgs& a, int n01, int n2) {
  if (!a.mixed || n2 < 1 || n2 > 32 || n01 < 1) return false;
  const int last = n01 - (n01 - 1) / a.rows_a * a.rows_a;
  return last <= a.rows_a - 16 * ((n2 + 15) / 16);
}

// A token's 8 slots (local expert or -1, routing weight) and squared norm, and one thread's share
// of the experts' estimates for the workgroup's LDS copy: every global input of the permutation's
// per-token kernels in one round of loads (16-byte loads, clamped indices, no branch between them;
// loads under a per-slot branch were each waited for before the next).
struct TokenSlots {
  int le[kTopK];
  float w[kTopK];
  float a2;
  float es[2];   // esig[tid], esig[tid + kBlkTokens] (clamped)
};
__device__ __forceinline__ void load_token_slots(const LargePermArgs& a, int t, TokenSlots& ts) {
  static_assert(2 * kBlkTokens >= 2 * kEGlobal, "two estimates per thread cover every expert");
  const int tc = min(t, a.T - 1), tid = threadIdx.x, ne = 2 * a.E_local;
  const int4* ip = reinterpret_cast<const int4*>(a.topk_ids + (size_t)tc * kTopK);
  const float4* wp = reinterpret_cast<const float4*>(a.topk_w + (size_t)tc * kTopK);
  const int4 i0 = ip[0], i1 = ip[1];
  const float4 w0 = wp[0], w1 = wp[1];
  ts.a2 = a.tok_a2[tc];
  ts.es[0] = a.esig[min(tid, ne - 1)];
  ts.es[1] = a.esig[min(tid + kBlkTokens, ne - 1)];
  const int id[kTopK] = {i0.x, i0.y, i0.z, i0.w, i1.x, i1.y, i1.z, i1.w};
  const float wv[kTopK] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
  for (int k = 0; k < kTopK; k++) {
    const int le = id[k] - a.offset;
    ts.le[k] = le >= 0 && le < a.E_local ? le : -1;
    ts.w[k] = wv[k];
  }
}
// The workgroup's LDS copy of the expert estimates (the caller's barrier publishes it).
__device__ __forceinline__ void stage_esig(const LargePermArgs& a, const TokenSlots& ts, float* es) {
  const int tid = threadIdx.x, ne = 2 * a.E_local;
  if (tid < ne) es[tid] = ts.es[0];
  if (tid + kBlkTokens < ne) es[tid + kBlkTokens] = ts.es[1];
}
// Bucket (local expert x magnitude class) of slot k, or -1 if the expert is not local.
__device__ __forceinline__ int slot_bucket(const LargePermArgs& a, const TokenSlots& ts, int k, const float* es) {
  const int le = ts.le[k];
  if (le < 0) return -1;
  const float pred = predicted_output_rms(ts.a2, ts.w[k], es[2 * le], es[2 * le + 1], a.sqrt_i);
  return le * kClasses + magnitude_class(pred);
}

__global__ __launch_bounds__(kBlkTokens) void perm_count_kernel(LargePermArgs a) {
  __shared__ int cnt[kEGlobal * kClasses];
  __shared__ float es[2 * kEGlobal];
  const int E3 = a.E_local * kClasses, tid = threadIdx.x;
  const int t = blockIdx.x * kBlkTokens + tid;
  TokenSlots ts;
  load_token_slots(a, t, ts);
  for (int i = tid; i < E3; i += kBlkTokens) cnt[i] = 0;
  stage_esig(a, ts, es);
  __syncthreads();
  if (t < a.T) {
#pragma unroll
    for (int k = 0; k < kTopK; k++) {
      const int b = slot_bucket(a, ts, k, es);
      if (b >= 0) atomicAdd(&cnt[b], 1);
    }
  }
  __syncthreads();
  for (int i = tid; i < E3; i += kBlkTokens) a.bcnt[(size_t)blockIdx.x * E3 + i] = cnt[i];
}

constexpr int kPlaceLdsInts = 6144;   // 24 KB of staged counts per round

// tot[i] = bucket i's pairs over all blocks, pre[i] = over the blocks before `me` (E3 buckets),
// from the per-block counts staged through LDS a chunk of blocks at a time (all of a chunk's
// counts in one round of loads).  All threads of the block; ends with a barrier.
__device__ void bucket_sums(const LargePermArgs& a, int me, int* tot, int* pre, int* stage) {
  const int E3 = a.E_local * kClasses, nb = a.nblk, tid = threadIdx.x;
  constexpr int kPer = kPlaceLdsInts / kBlkTokens;
  static_assert(kPlaceLdsInts >= kEGlobal * kClasses, "a chunk holds at least one block");
  const int chunk = min(nb, kPlaceLdsInts / E3);
  for (int i = tid; i < E3; i += kBlkTokens) {
    tot[i] = 0;
    pre[i] = 0;
  }
  for (int b0 = 0; b0 < nb; b0 += chunk) {
    const int n = min(chunk, nb - b0) * E3;
    int v[kPer];
#pragma unroll
    for (int q = 0; q < kPer; q++) v[q] = a.bcnt[(size_t)b0 * E3 + min(tid + q * kBlkTokens, n - 1)];
    // the previous chunk's readers are done
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kPer; q++)
      if (tid + q * kBlkTokens < n) stage[tid + q * kBlkTokens] = v[q];
    __syncthreads();
    for (int i = tid; i < E3; i += kBlkTokens) {
      int t = tot[i], pb = pre[i];
      for (int b = 0; b * E3 < n; b++) {
        const int c = stage[b * E3 + i];
        t += c;
        pb += b0 + b < me ? c : 0;
      }
      tot[i] = t;
      pre[i] = pb;
    }
  }
  __syncthreads();
}

// First index i in [0, n) with v[i] > x (v ascending).
__device__ __forceinline__ int upper_bound(const int* v, int n, int x) {
  int lo = 0, hi = n;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (v[mid] <= x) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

// Expert offsets, 16-row m-tile offsets and m-block offsets, expert by expert, from the bucket
// totals (one wavefront): blocks of rows_a rows over an expert's class 0 and 1 rows (two-term C in
// the blocks that hold class 1 rows), then blocks of rows_b rows over its class 2 rows, or those
// folded into its last class 0/1 block (folds_exact: 27 of 107 blocks at T = 8192 held <= 32 exact
// rows each, a quarter of the GEMMs' weight streams for 5% of the rows).  The grouped GEMMs run
// this one table (GEMM2 on separate class 0 and class 1 blocks had 11% more blocks, hence more
// weight streams, and was 4% slower at T = 8192; the 128-row GEMM2 builds its own from measured C).
// An expert's blocks are consecutive, so the units that stream its weights run close together in
// time and share them through L2.  With `write`, also the path's global tables.
__device__ void expert_offsets(const LargePermArgs& a, const int* tot, int* eoff, int* emt, int* eb1, bool write) {
  const int E = a.E_local, lane = lane_id();
  int carry = 0, carry_mt = 0, carry_1 = 0, carry_act = 0;
  for (int e0 = 0; e0 < E; e0 += kWave) {
    const int e = e0 + lane;
    const int n0 = e < E ? tot[kClasses * e] : 0, n1 = e < E ? tot[kClasses * e + 1] : 0;
    const int n2 = e < E ? tot[kClasses * e + 2] : 0, n = n0 + n1 + n2;
    const int mt = (n + 15) / 16;
    const int ba = (n0 + n1 + a.rows_a - 1) / a.rows_a;
    const int bx = folds_exact(a, n0 + n1, n2) ? 0 : (n2 + a.rows_b - 1) / a.rows_b;
    const int b1 = ba + bx;
    const int pn = wave_exclusive_sum(n), pmt = wave_exclusive_sum(mt);
    const int p1 = wave_exclusive_sum(b1);
    const uint64_t act = __ballot(n > 0);
    if (e < E) {
      eoff[e] = carry + pn;
      emt[e] = carry_mt + pmt;
      eb1[e] = carry_1 + p1;
      if (write) {
        a.expert_offsets[e] = carry + pn;
        a.mtile_offsets[e] = carry_mt + pmt;
        a.xrow[e] = carry + pn + n0 + n1;
        if (n > 0) a.active[carry_act + lanes_below(act)] = e;
      }
    }
    carry += __builtin_amdgcn_readlane(pn + n, kWave - 1);
    carry_mt += __builtin_amdgcn_readlane(pmt + mt, kWave - 1);
    carry_1 += __builtin_amdgcn_readlane(p1 + b1, kWave - 1);
    carry_act += (int)__popcll(act);
  }
  if (lane == 0) {
    eoff[E] = carry;
    emt[E] = carry_mt;
    eb1[E] = carry_1;
    if (write) {
      a.expert_offsets[E] = carry;
      a.mtile_offsets[E] = carry_mt;
      a.info[0] = carry;                // P
      a.info[1] = carry_act;            // active experts
      a.info[2] = carry_1;              // GEMM1 m-blocks
      a.info[3] = 1;                    // K-splits (small-T GEMMs only)
      a.info[4] = 1;
      a.info[5] = carry_1;              // GEMM2 m-blocks of the grouped path: the same table
      a.info[6] = carry_mt;             // 16-row m-tiles
    }
  }
}

// The m-block table {expert, first row, rows, flags} and each block's expert group (all threads).
__device__ void write_mblocks(const LargePermArgs& a, const int* tot, const int* eoff, const int* eb1) {
  const int E = a.E_local;
  for (int g = threadIdx.x; g < eb1[E]; g += blockDim.x) {
    const int e = upper_bound(eb1, E + 1, g) - 1, j = g - eb1[e];
    const int c0 = tot[kClasses * e], c01 = c0 + tot[kClasses * e + 1], n = eoff[e + 1] - eoff[e];
    const int ba = (c01 + a.rows_a - 1) / a.rows_a;
    if (j < ba) {
      const int r0 = j * a.rows_a, rows = min(a.rows_a, c01 - r0);
      int flags = r0 + rows > c0 ? class_flags(1) : 0;
      if (j == ba - 1 && folds_exact(a, c01, n - c01)) flags |= kFlagMixed | ((n - c01) << kMixedShift);
      a.mblocks[g] = int4{e, eoff[e] + r0, rows, flags};
    } else {
      const int r0 = c01 + (j - ba) * a.rows_b;
      a.mblocks[g] = int4{e, eoff[e] + r0, min(a.rows_b, n - r0), class_flags(2)};
    }
    a.mbgroup[g] = int2{eb1[e], eb1[e + 1] - eb1[e]};
  }
}

// Rank of each slot's key among the lower lanes of the wavefront holding the same key (keys of
// one lane are distinct or -1).  Every lane ORs its bit into the LDS lane masks of its keys (the
// wavefront's own masks; OR is order-free, so the result is deterministic), and a rank is the
// count of lower lanes in its key's mask.  A wavefront's LDS operations complete in issue order,
// so its reads see all of its ORs.
__device__ __forceinline__ void wave_key_ranks(const int (&key)[kTopK], int (&rank)[kTopK],
                                               unsigned long long* masks) {
  const unsigned long long me = 1ull << lane_id();
#pragma unroll
  for (int k = 0; k < kTopK; k++)
    if (key[k] >= 0) atomicOr(&masks[key[k]], me);
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int k = 0; k < kTopK; k++) rank[k] = key[k] >= 0 ? (int)__popcll(masks[key[k]] & (me - 1)) : 0;
}

__global__ __launch_bounds__(kBlkTokens) void perm_place_kernel(LargePermArgs a) {
  // per wavefront and key, the lanes holding it: buckets (expert x class) and experts
  __shared__ unsigned long long bmask[kBlkWaves][kEGlobal * kClasses];
  __shared__ unsigned long long emask[kBlkWaves][kEGlobal];
  __shared__ float es[2 * kEGlobal];
  // bucket totals and this block's prefix of them; expert, m-tile and m-block offsets
  __shared__ int tot[kEGlobal * kClasses], pre[kEGlobal * kClasses];
  __shared__ int eoff[kEGlobal + 1], emt[kEGlobal + 1], eb1[kEGlobal + 1];
  __shared__ int stage[kPlaceLdsInts];
  const int E = a.E_local, E3 = E * kClasses, tid = threadIdx.x, wave = tid >> 6;
  const int t = blockIdx.x * kBlkTokens + tid;
  const bool in = t < a.T;
  TokenSlots ts;
  load_token_slots(a, t, ts);
  for (int i = tid; i < kBlkWaves * E3; i += kBlkTokens) bmask[i / E3][i % E3] = 0ull;
  for (int i = tid; i < kBlkWaves * E; i += kBlkTokens) emask[i / E][i % E] = 0ull;
  stage_esig(a, ts, es);
  bucket_sums(a, blockIdx.x, tot, pre, stage);
  const bool first = blockIdx.x == 0;
  if (wave == 0) expert_offsets(a, tot, eoff, emt, eb1, first);
  if (first) {
    // the grouped GEMMs' unit queues and the 128-row GEMM2's row-table counters start at zero
    if (tid < kUnitQueues) a.queues[tid * kQueueStride] = 0;
    for (int i = tid; a.g2_ctl && i < 2 * E; i += kBlkTokens) a.g2_ctl[i] = 0;
  }
  __syncthreads();
  if (first) write_mblocks(a, tot, eoff, eb1);
  int bk[kTopK], ek[kTopK], rb[kTopK], re[kTopK];
#pragma unroll
  for (int k = 0; k < kTopK; k++) {
    bk[k] = in ? slot_bucket(a, ts, k, es) : -1;
    ek[k] = bk[k] >= 0 ? ts.le[k] : -1;
    rb[k] = 0;
    re[k] = 0;
  }
  // the block's bases: bucket (e, c) starts after the expert's lower classes and this block's
  // prefix of its own count; the expert's canonical rows after this block's prefix of its three
  // buckets (slot 0's key where a slot is not local: in range, unused)
  int bb[kTopK], cb[kTopK];
#pragma unroll
  for (int k = 0; k < kTopK; k++) {
    const int b3 = max(bk[k], 0), e = b3 / kClasses, c = b3 - e * kClasses;
    bb[k] = eoff[e] + (c > 0 ? tot[kClasses * e] : 0) + (c > 1 ? tot[kClasses * e + 1] : 0) + pre[b3];
    cb[k] = eoff[e] + pre[kClasses * e] + pre[kClasses * e + 1] + pre[kClasses * e + 2];
  }
  wave_key_ranks(bk, rb, bmask[wave]);
  wave_key_ranks(ek, re, emask[wave]);
  __syncthreads();
  if (!in) return;
  int n_local = 0;
#pragma unroll
  for (int k = 0; k < kTopK; k++) {
    if (bk[k] < 0) continue;
    n_local++;
    int pos = bb[k] + rb[k];
    int cpos = cb[k] + re[k];
    for (int w = 0; w < wave; w++) {
      pos += (int)__popcll(bmask[w][bk[k]]);
      cpos += (int)__popcll(emask[w][ek[k]]);
    }
    a.perm_token[pos] = t;
    a.perm_w[pos] = ts.w[k];
    a.canon_token[cpos] = t;
    // slot = rank of the local expert among the token's local experts: the combine adds a
    // token's rows in ascending expert order
    int slot = 0;
#pragma unroll
    for (int q = 0; q < kTopK; q++) slot += (ek[q] >= 0 && ek[q] < ek[k]) ? 1 : 0;
    a.tok_slot[(size_t)t * kTopK + slot] = pos;
  }
  for (int kk = n_local; kk < kTopK; kk++) a.tok_slot[(size_t)t * kTopK + kk] = -1;
}

void launch_permute_large(const LargePermArgs& args, hipStream_t stream) {
  if (args.nblk <= 0) return;
  hipLaunchKernelGGL(perm_count_kernel, dim3(args.nblk), dim3(kBlkTokens), 0, stream, args);
  hipLaunchKernelGGL(perm_place_kernel, dim3(args.nblk), dim3(kBlkTokens), 0, stream, args);
}

int permute_large_blocks(int64_t T) { return (int)((T + kBlkTokens - 1) / kBlkTokens); }

}  // namespace moefp8
