// extern "C" boundary of the gfx950 MoE operator (declared in include/moefp8.h).
//
// moefp8_run replaces the Python entry point solutions/moe_fp8/main.py:173-243.
// It checks every argument on the host, carves the caller's workspace, and
// enqueues on the caller's stream:
//   route -> permute -> GEMM1(+SwiGLU) -> GEMM2 -> combine
// with no host synchronisation and no allocation.  The small-T variant streams
// weights; the large-T variant stages activations through LDS.  Both are
// chosen by T alone, so the launch sequence is fixed for given sizes.
#include <atomic>
#include <cstring>

#include "moefp8.h"
#include "moefp8_device.h"
#include "moefp8_launch.h"

namespace moefp8 {

// Largest T served by the weight-streaming kernels.
constexpr int64_t kDecodeMaxT = 64;

// Large-T m-blocks.  From T = 128 the class 0/1 rows of an expert go in 128-row blocks for the
// LDS-staged 128-row GEMMs and its exact-product rows in 32-row blocks (or folded into the last
// class 0/1 block): even with a few rows per expert these stream each weight slice once per
// block and took 253 / 249 / 277 / 311 µs at T = 128 / 256 / 512 / 1024 against 262 / 252 / 288
// / 389 µs for the 4-wave kernels below.  Those (blocks of 16 * large_mt(T) rows) remain for
// 64 < T < 128 and for shapes the 128-row kernels do not take.
constexpr int64_t kBigT = 128;
constexpr int kExactRows = 32;
// The 128-row kernels address their DMA sources with 32-bit per-lane byte offsets from a
// wave-uniform base: hidden rows (token x H, GEMM1) and C rows (pair x 2I, GEMM2).  Shapes whose
// offsets could pass 2^31 (T x H) or 2^32 (Pmax x 2I, Pmax = T x min(8, E_local)) take the 4-wave
// kernels, which form 64-bit addresses.
bool large_big(int64_t T, int E_local, int H, int I) {
  const int64_t pmax = T * (E_local < kTopK ? E_local : kTopK);
  return T >= kBigT && H / kBlock <= kBigMaxKB && I / kBlock <= kBigMaxKB && H % 256 == 0 &&
         T * H < ((int64_t)1 << 31) && pmax * 2 * I < ((int64_t)1 << 32);
}
int large_mt(int64_t T) { return T / 32 >= 48 ? 4 : 2; }

// The 128-row path's fp32 per-pair output rows O: above this many bytes for Pmax rows (T > 4681 at
// H = 7168 with E_local >= 8) the workspace holds ceil(Pmax / 2) rows of all H columns.  A call with
// at most that many local pairs (every routing that averages up to 4 local experts per token; the
// T = 8192 benchmark has 8,587 of 65,536) runs GEMM2 and the combine once over all columns; a call
// with more runs them once per half of the columns (blocks of 256), each pass's rows then being
// half as long.  W2 rows are output columns, so no weight is read twice.  The kernels take the
// decision from the pair count on the device; the host launches both passes.
constexpr size_t kOutRowsBudget = (size_t)1 << 30;
int64_t output_rows(int64_t T, int E_local, int H, int I) {
  const int64_t pmax = T * (E_local < kTopK ? E_local : kTopK);
  if (T <= kDecodeMaxT || !large_big(T, E_local, H, I) || (size_t)pmax * H * 4 <= kOutRowsBudget) return pmax;
  // rows of the first (larger) half of the columns for every pair: ceil(pmax * half / H) full rows
  const int64_t half = (H / 256 + 1) / 2 * 256;
  return (pmax * half + H - 1) / H;
}
int large_rows_a(int64_t T, int E, int H, int I) { return large_big(T, E, H, I) ? kBigRows : 16 * large_mt(T); }
int large_rows_b(int64_t T, int E, int H, int I) { return large_big(T, E, H, I) ? kExactRows : 16 * large_mt(T); }

struct Layout {
  size_t topk_ids, topk_w, expert_offsets, active, mtile_offsets, info, perm_token, perm_w, tok_slot;
  size_t tok_a2, esig, mtiles, counters, c16, c16_scale, gbuf, obuf;
  size_t canon_token, bcnt, mblocks, mbgroup, two_term, queues, c_hi, c_lo16, c_scale;
  size_t g2_pair, g2_ctl, xrow;
  size_t total;
  int64_t pmax, max_mtiles, rows_cap, c_plane, max_blocks, max_blocks2, n_counters1, n_counters;
  int64_t o_rows;
  int nblk;
};

static size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

static Layout make_layout(int64_t T, int E_local, int H, int I) {
  Layout L = {};
  const int64_t pmax = T * (E_local < kTopK ? E_local : kTopK);
  L.pmax = pmax;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o = align_up(o + bytes);
    return at;
  };
  L.topk_ids = take((size_t)T * kTopK * 4);
  L.topk_w = take((size_t)T * kTopK * 4);
  L.expert_offsets = take((size_t)(E_local + 1) * 4);
  L.active = take((size_t)E_local * 4);
  L.mtile_offsets = take((size_t)(E_local + 1) * 4);
  L.info = take(64);
  L.perm_token = take((size_t)pmax * 4);
  L.perm_w = take((size_t)pmax * 4);
  L.tok_slot = take((size_t)T * kTopK * 4);
  L.tok_a2 = take((size_t)T * 4);
  L.esig = take((size_t)E_local * 2 * 4);
  L.max_mtiles = (pmax + 15) / 16 + E_local;
  L.c_plane = (int64_t)align_up((size_t)pmax * I);
  if (T <= kDecodeMaxT) {
    // small T: m-tile table, GEMM1 partials [rows][2I] fp32, C as f16 hi/lo planes + scales,
    // GEMM2 partials [rows][H] fp32; rows = pairs x K-split <= rows_cap
    // (every split count the K-split policy can pick: up to 8 while 8 * pairs <= 1024, and
    // at least ceil(K-blocks / 64) of either GEMM)
    const int64_t r8 = 8 * pmax < 1024 ? 8 * pmax : 1024;
    const int64_t kbmax = (H > I ? H : I) / kBlock, smin = (kbmax + 63) / 64;
    L.rows_cap = pmax * smin > r8 ? pmax * smin : r8;
    L.mtiles = take((size_t)L.max_mtiles * 16);
    // arrival counters: per (m-tile, 128 C columns) for GEMM1, then per output column block,
    // then GEMM2's precision flag per m-tile (all zeroed by the routing kernel), one 128-byte
    // line each
    L.n_counters1 = L.max_mtiles * (I / kBlock);
    L.n_counters = L.n_counters1 + H / (16 * decode_unit_groups());
    L.counters = take((size_t)(L.n_counters + L.max_mtiles) * 4 * kCounterStride);
    L.gbuf = take((size_t)L.rows_cap * 2 * I * 4);
    L.c16 = take((size_t)L.c_plane * 2 * 2);
    L.c16_scale = take((size_t)pmax * (I / kBlock) * 4);
    L.obuf = take((size_t)L.rows_cap * H * 4);
    L.total = o;
    return L;
  }
  // large T: permutation scratch and tables, C (f16 hi and lo, fp32 scales), O [pmax][H] fp32
  L.rows_cap = pmax;
  L.nblk = permute_large_blocks(T);
  const int ra = large_rows_a(T, E_local, H, I), rb = large_rows_b(T, E_local, H, I);
  // blocks per expert (both GEMMs): ceil(class 0+1 rows / ra) + ceil(class 2 rows / rb)
  const int64_t exact_blocks = (pmax + rb - 1) / rb + E_local;
  L.max_blocks = (pmax + ra - 1) / ra + E_local + exact_blocks;
  L.canon_token = take((size_t)pmax * 4);
  L.bcnt = take((size_t)L.nblk * E_local * 3 * 4);
  L.mblocks = take((size_t)L.max_blocks * 16);
  L.mbgroup = take((size_t)L.max_blocks * 8);
  L.two_term = take((size_t)L.max_blocks * 4);
  L.queues = take((size_t)kUnitQueues * kQueueStride * 4);
  // GEMM2's row table (128-row path): its blocks split each expert's rows in two groups
  L.max_blocks2 = (pmax + kBigRows - 1) / kBigRows + 2 * (int64_t)E_local;
  L.g2_pair = take((size_t)pmax * 4);
  L.g2_ctl = take((size_t)(2 * E_local) * 4);
  L.xrow = take((size_t)E_local * 4);
  L.c_hi = take((size_t)pmax * I * 2);
  L.c_lo16 = take((size_t)pmax * I * 2);
  L.c_scale = take((size_t)pmax * (I / kBlock) * 4);
  L.o_rows = output_rows(T, E_local, H, I);
  L.obuf = take((size_t)L.o_rows * H * 4);
  L.total = o;
  return L;
}

// Device memory of the no-allocation entry point: one static array per device that loads the
// library, held until the process ends.  Host code never uses the name `scratch` as an address
// (on the host it is a stand-in, not device memory): the device address comes from
// hipGetSymbolAddress, once per device, and is kept in g_scratch_ptr.
constexpr size_t kScratchBytes = MOEFP8_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
static std::atomic<void*> g_scratch_ptr[64];

// This device's address of `scratch` (the device must be current); NULL if the runtime cannot
// give it.
static void* scratch_address(int dev) {
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p) return p;
  if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
  g_scratch_ptr[dev].store(p, std::memory_order_release);   // same value if two threads race here
  return p;
}

static std::atomic<int> g_cu_count[64];
static std::atomic<int> g_arch_ok[64];  // 0 unknown, 1 gfx950, -1 other

static int query_device(int* dev_out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return MOEFP8_ERR_DEVICE;
  *dev_out = dev;
  if (dev < 0 || dev >= 64) return MOEFP8_ERR_DEVICE;
  if (g_arch_ok[dev].load(std::memory_order_acquire) == 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return MOEFP8_ERR_DEVICE;
    g_cu_count[dev].store(prop.multiProcessorCount, std::memory_order_relaxed);
    const bool ok = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    g_arch_ok[dev].store(ok ? 1 : -1, std::memory_order_release);
  }
  return g_arch_ok[dev].load(std::memory_order_acquire) == 1 ? MOEFP8_OK : MOEFP8_ERR_DEVICE;
}

int num_compute_units() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  const int n = g_cu_count[dev].load(std::memory_order_relaxed);
  return n > 0 ? n : 256;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// The routing kernel reads logits and bias 4 elements at a time with 8-byte loads (load4_as_f32):
// fp32 tensors must be 16-byte aligned, 16-bit ones 8-byte aligned.
static bool aligned_for_dtype(const void* p, int dt) {
  return ((uintptr_t)p & (dt == 0 ? 15u : 7u)) == 0;
}

static int check_sizes(int64_t T, int E_local, int H, int I) {
  if (T < 0 || T > (int64_t)1 << 24) return MOEFP8_ERR_SHAPE;
  if (E_local < 1 || E_local > kEGlobal) return MOEFP8_ERR_SHAPE;
  if (H <= 0 || I <= 0 || H % kBlock != 0 || I % kBlock != 0) return MOEFP8_ERR_SHAPE;
  return MOEFP8_OK;
}

static int check_dtype(int dt) { return (dt >= 0 && dt <= 2) ? MOEFP8_OK : MOEFP8_ERR_DTYPE; }

}  // namespace moefp8

using namespace moefp8;

// Launch-error check and the optional debug copies that end every moefp8_run.
static int finish(const moefp8_args* a, const Layout& L, const int* topk_ids, const float* topk_w, const Plan& pl,
                  hipStream_t s) {
  if (hipGetLastError() != hipSuccess) return MOEFP8_ERR_LAUNCH;
  const int64_t T = a->num_tokens;
  struct Copy {
    void* dst;
    const void* src;
    size_t bytes;
  } copies[] = {{a->topk_ids, topk_ids, (size_t)T * kTopK * 4},
                {a->topk_weights, topk_w, (size_t)T * kTopK * 4},
                {a->expert_offsets, pl.expert_offsets, (size_t)(a->num_local_experts + 1) * 4},
                {a->permuted_tokens, pl.canon_token, (size_t)L.pmax * 4}};
  for (const Copy& c : copies)
    if (c.dst && hipMemcpyAsync(c.dst, c.src, c.bytes, hipMemcpyDeviceToDevice, s) != hipSuccess)
      return MOEFP8_ERR_LAUNCH;
  return MOEFP8_OK;
}

extern "C" {

int moefp8_abi_version(void) { return MOEFP8_ABI_VERSION; }

const char* moefp8_strerror(int status) {
  switch (status) {
    case MOEFP8_OK: return "ok";
    case MOEFP8_ERR_NULL_POINTER: return "a required pointer is NULL";
    case MOEFP8_ERR_SHAPE: return "bad shape: need T >= 0, 1 <= E_local <= 256, H and I positive multiples of 128";
    case MOEFP8_ERR_DTYPE: return "unsupported dtype code for routing logits or bias";
    case MOEFP8_ERR_ALIGNMENT: return "a tensor pointer is not 16-byte aligned";
    case MOEFP8_ERR_WORKSPACE: return "workspace is NULL or smaller than moefp8_workspace_size()";
    case MOEFP8_ERR_LAUNCH: return "kernel launch failed";
    case MOEFP8_ERR_DEVICE: return "current HIP device is not gfx950 or the HIP runtime failed";
    case MOEFP8_ERR_SCRATCH_LIMIT:
      return "sizes need more workspace than moefp8_run_noalloc's static scratch (MOEFP8_NOALLOC_SCRATCH_BYTES, "
             "64 MiB)";
    default: return "unknown status";
  }
}

int moefp8_workspace_size(int64_t num_tokens, int32_t num_local_experts, int32_t hidden_size,
                          int32_t intermediate_size, size_t* bytes) {
  if (!bytes) return MOEFP8_ERR_NULL_POINTER;
  const int rc = check_sizes(num_tokens, num_local_experts, hidden_size, intermediate_size);
  if (rc) return rc;
  *bytes = make_layout(num_tokens, num_local_experts, hidden_size, intermediate_size).total;
  return MOEFP8_OK;
}

int moefp8_path(int64_t num_tokens, int32_t num_local_experts, int32_t hidden_size, int32_t intermediate_size) {
  const int rc = check_sizes(num_tokens, num_local_experts, hidden_size, intermediate_size);
  if (rc) return rc;
  if (num_tokens <= kDecodeMaxT) return MOEFP8_PATH_SMALL_T;
  return large_big(num_tokens, num_local_experts, hidden_size, intermediate_size) ? MOEFP8_PATH_ROWS128
                                                                                    : MOEFP8_PATH_GROUPED;
}

int moefp8_output_passes(int64_t num_tokens, int32_t num_local_experts, int32_t hidden_size,
                         int32_t intermediate_size, int64_t num_pairs) {
  const int rc = check_sizes(num_tokens, num_local_experts, hidden_size, intermediate_size);
  if (rc) return rc;
  if (num_pairs < 0) return MOEFP8_ERR_SHAPE;
  return num_pairs > output_rows(num_tokens, num_local_experts, hidden_size, intermediate_size) ? 2 : 1;
}

int moefp8_route(const void* routing_logits, int32_t logits_dtype, const void* routing_bias, int32_t bias_dtype,
                 int64_t num_tokens, float routed_scaling_factor, int32_t* topk_ids, float* topk_weights,
                 void* stream) {
  if (num_tokens < 0 || num_tokens > (int64_t)1 << 24) return MOEFP8_ERR_SHAPE;
  if (check_dtype(logits_dtype) || check_dtype(bias_dtype)) return MOEFP8_ERR_DTYPE;
  if (num_tokens == 0) return MOEFP8_OK;
  if (!routing_logits || !routing_bias || !topk_ids || !topk_weights) return MOEFP8_ERR_NULL_POINTER;
  if (!aligned_for_dtype(routing_logits, logits_dtype) || !aligned_for_dtype(routing_bias, bias_dtype) ||
      ((uintptr_t)topk_ids & 3u) || ((uintptr_t)topk_weights & 3u))
    return MOEFP8_ERR_ALIGNMENT;
  int dev;
  if (query_device(&dev)) return MOEFP8_ERR_DEVICE;
  hipStream_t s = (hipStream_t)stream;
  launch_route(routing_logits, logits_dtype, routing_bias, bias_dtype, num_tokens, routed_scaling_factor, topk_ids,
               topk_weights, nullptr, nullptr, 0, s);
  return hipGetLastError() == hipSuccess ? MOEFP8_OK : MOEFP8_ERR_LAUNCH;
}

int moefp8_quantize_hidden(const void* x, int32_t x_dtype, int64_t num_tokens, int32_t hidden_size,
                           void* hidden_out, float* scale_out, void* stream) {
  if (num_tokens < 0 || num_tokens > (int64_t)1 << 24) return MOEFP8_ERR_SHAPE;
  if (hidden_size <= 0 || hidden_size % kBlock != 0) return MOEFP8_ERR_SHAPE;
  if (x_dtype != 0 && x_dtype != 1) return MOEFP8_ERR_DTYPE;
  if (num_tokens == 0) return MOEFP8_OK;
  if (!x || !hidden_out || !scale_out) return MOEFP8_ERR_NULL_POINTER;
  if (!aligned16(x) || ((uintptr_t)hidden_out & 7u) || ((uintptr_t)scale_out & 3u)) return MOEFP8_ERR_ALIGNMENT;
  int dev;
  if (query_device(&dev)) return MOEFP8_ERR_DEVICE;
  launch_quantize_hidden(x, x_dtype, num_tokens, hidden_size, reinterpret_cast<uint8_t*>(hidden_out), scale_out,
                         (hipStream_t)stream);
  return hipGetLastError() == hipSuccess ? MOEFP8_OK : MOEFP8_ERR_LAUNCH;
}

// The operator on the caller's workspace, or with `noalloc` on this device's static scratch, for
// sizes whose workspace fits it (moefp8_run_noalloc).
static int run_impl(const moefp8_args* a, void* workspace, size_t workspace_bytes, void* stream, bool noalloc) {
  if (!a) return MOEFP8_ERR_NULL_POINTER;
  const int64_t T = a->num_tokens;
  const int E_local = a->num_local_experts, H = a->hidden_size, I = a->intermediate_size;
  int rc = check_sizes(T, E_local, H, I);
  if (rc) return rc;
  if (check_dtype(a->logits_dtype) || check_dtype(a->bias_dtype)) return MOEFP8_ERR_DTYPE;
  if (T == 0) return MOEFP8_OK;
  if (!a->routing_logits || !a->routing_bias || !a->hidden_states || !a->hidden_states_scale ||
      !a->gemm1_weights || !a->gemm1_weights_scale || !a->gemm2_weights || !a->gemm2_weights_scale || !a->output)
    return MOEFP8_ERR_NULL_POINTER;
  const void* ptrs16[] = {a->hidden_states, a->gemm1_weights, a->gemm2_weights, a->output};
  for (const void* p : ptrs16)
    if (!aligned16(p)) return MOEFP8_ERR_ALIGNMENT;
  const void* ptrs4[] = {a->hidden_states_scale, a->gemm1_weights_scale, a->gemm2_weights_scale};
  for (const void* p : ptrs4)
    if (((uintptr_t)p & 3u) != 0) return MOEFP8_ERR_ALIGNMENT;
  if (!aligned_for_dtype(a->routing_logits, a->logits_dtype) || !aligned_for_dtype(a->routing_bias, a->bias_dtype))
    return MOEFP8_ERR_ALIGNMENT;
  if (a->output_f32 != 0 && a->output_f32 != 1) return MOEFP8_ERR_DTYPE;
  if (a->shared_output) {
    if (a->shared_dtype != MOEFP8_DTYPE_F32 && a->shared_dtype != MOEFP8_DTYPE_BF16) return MOEFP8_ERR_DTYPE;
    if (!aligned16(a->shared_output)) return MOEFP8_ERR_ALIGNMENT;
  }
  const Layout L = make_layout(T, E_local, H, I);
  if (noalloc) {
    if (L.total > kScratchBytes) return MOEFP8_ERR_SCRATCH_LIMIT;
  } else if (!workspace || workspace_bytes < L.total || !aligned16(workspace)) {
    return MOEFP8_ERR_WORKSPACE;
  }
  int dev;
  if (query_device(&dev)) return MOEFP8_ERR_DEVICE;
  if (noalloc && !(workspace = scratch_address(dev))) return MOEFP8_ERR_DEVICE;

  hipStream_t s = (hipStream_t)stream;
  uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
  int* topk_ids = reinterpret_cast<int*>(ws + L.topk_ids);
  float* topk_w = reinterpret_cast<float*>(ws + L.topk_w);
  Plan pl;
  pl.expert_offsets = reinterpret_cast<int*>(ws + L.expert_offsets);
  pl.perm_token = reinterpret_cast<int*>(ws + L.perm_token);
  pl.perm_w = reinterpret_cast<float*>(ws + L.perm_w);
  pl.tok_slot = reinterpret_cast<int*>(ws + L.tok_slot);
  pl.active = reinterpret_cast<int*>(ws + L.active);
  pl.mtile_offsets = reinterpret_cast<int*>(ws + L.mtile_offsets);
  pl.info = reinterpret_cast<int*>(ws + L.info);
  pl.mtiles = nullptr;
  pl.mblocks = nullptr;
  pl.mbgroup = nullptr;
  pl.queues = nullptr;
  pl.canon_token = pl.perm_token;
  pl.counters = nullptr;
  pl.counters2 = nullptr;
  pl.esig = reinterpret_cast<const float*>(ws + L.esig);
  pl.two_term = nullptr;
  pl.g2_pair = nullptr;
  pl.g2_ctl = nullptr;
  pl.xrow = nullptr;
  pl.shared = a->shared_output;
  pl.shared_dt = a->shared_dtype;
  pl.out_f32 = a->output_f32;
  pl.pair_rows = (int)L.pmax;
  float* tok_a2 = reinterpret_cast<float*>(ws + L.tok_a2);
  float* esig = reinterpret_cast<float*>(ws + L.esig);

  Problem pb;
  pb.hidden = a->hidden_states;
  pb.hscale = a->hidden_states_scale;
  pb.w13 = a->gemm1_weights;
  pb.s13 = a->gemm1_weights_scale;
  pb.w2 = a->gemm2_weights;
  pb.s2 = a->gemm2_weights_scale;
  pb.T = (int)T;
  pb.E_local = E_local;
  pb.H = H;
  pb.I = I;

  hipEvent_t* ev = reinterpret_cast<hipEvent_t*>(a->stage_events);
  auto mark = [&](int i) {
    if (ev) (void)hipEventRecord(ev[i], s);
  };
  MagInputs mag = {a->hidden_states, a->hidden_states_scale, a->gemm1_weights_scale, a->gemm2_weights_scale,
                   H, I, E_local, tok_a2, esig};
  if (T <= kDecodeMaxT) {
    // small T: routing (+ scale estimates), GEMM1 (+ permutation plan, SwiGLU), GEMM2 (+ combine)
    const int groups = decode_unit_groups();
    const SplitPolicy sp = {decode_grid1(), 2 * I / (16 * groups), H / kBlock, (int)L.rows_cap,
                            decode_grid2(), H / (16 * groups),     I / kBlock, (int)L.rows_cap,
                            2 * num_compute_units()};
    pl.mtiles = reinterpret_cast<const int4*>(ws + L.mtiles);
    pl.counters = reinterpret_cast<int*>(ws + L.counters);
    pl.counters2 = pl.counters + L.n_counters1 * kCounterStride;
    pl.two_term = pl.counters + L.n_counters * kCounterStride;
    DecodePlanArgs da;
    da.topk_ids = topk_ids;
    da.topk_w = topk_w;
    da.tok_a2 = tok_a2;
    da.esig = esig;
    da.T = (int)T;
    da.E_local = E_local;
    da.offset = a->local_expert_offset;
    da.sqrt_i = sqrtf((float)I);
    da.sp = sp;
    da.expert_offsets = const_cast<int*>(pl.expert_offsets);
    da.mtile_offsets = const_cast<int*>(pl.mtile_offsets);
    da.active = const_cast<int*>(pl.active);
    da.info = const_cast<int*>(pl.info);
    da.perm_token = const_cast<int*>(pl.perm_token);
    da.perm_w = const_cast<float*>(pl.perm_w);
    da.tok_slot = const_cast<int*>(pl.tok_slot);
    da.mtiles = const_cast<int4*>(pl.mtiles);
    mark(0);
    launch_route(a->routing_logits, a->logits_dtype, a->routing_bias, a->bias_dtype, T, a->routed_scaling_factor,
                 topk_ids, topk_w, &mag, pl.counters, (int)(L.n_counters + L.max_mtiles), s);
    mark(1);
    mark(2);   // the permutation is rebuilt by every GEMM1 workgroup: empty permute stage
    float* gbuf = reinterpret_cast<float*>(ws + L.gbuf);
    float* obuf = reinterpret_cast<float*>(ws + L.obuf);
    CHalf ch;
    ch.hi = reinterpret_cast<_Float16*>(ws + L.c16);
    ch.lo = ch.hi + L.c_plane;
    ch.scale = reinterpret_cast<float*>(ws + L.c16_scale);
    launch_gemm1_decode(pb, pl, da, gbuf, ch, s);
    mark(3);
    mark(4);   // SwiGLU is GEMM1's epilogue: empty activation stage
    launch_gemm2_decode(pb, pl, ch, obuf, a->output, s);
    mark(5);
    mark(6);   // the combine is GEMM2's epilogue: empty combine stage
    mark(7);   // one pass over the output columns: empty second-pass stages
    mark(8);
    return finish(a, L, topk_ids, topk_w, pl, s);
  }
  // large T: routing, permutation (3 launches), GEMM1 (+SwiGLU, C split), GEMM2, combine
  LargePermArgs pa = {};
  pa.topk_ids = topk_ids;
  pa.topk_w = topk_w;
  pa.tok_a2 = tok_a2;
  pa.esig = esig;
  pa.T = (int)T;
  pa.E_local = E_local;
  pa.offset = a->local_expert_offset;
  pa.sqrt_i = sqrtf((float)I);
  pa.nblk = L.nblk;
  pa.bcnt = reinterpret_cast<int*>(ws + L.bcnt);
  pa.expert_offsets = const_cast<int*>(pl.expert_offsets);
  pa.mtile_offsets = const_cast<int*>(pl.mtile_offsets);
  pa.active = const_cast<int*>(pl.active);
  pa.info = const_cast<int*>(pl.info);
  pa.perm_token = const_cast<int*>(pl.perm_token);
  pa.perm_w = const_cast<float*>(pl.perm_w);
  pa.canon_token = reinterpret_cast<int*>(ws + L.canon_token);
  pa.tok_slot = const_cast<int*>(pl.tok_slot);
  pa.mblocks = reinterpret_cast<int4*>(ws + L.mblocks);
  pa.mbgroup = reinterpret_cast<int2*>(ws + L.mbgroup);
  pa.queues = reinterpret_cast<int*>(ws + L.queues);
  const bool big = large_big(T, E_local, H, I);
  pa.mixed = big ? 1 : 0;   // the 128-row GEMMs run mixed blocks
  pa.rows_a = large_rows_a(T, E_local, H, I);
  pa.rows_b = large_rows_b(T, E_local, H, I);
  pl.canon_token = pa.canon_token;
  pl.mblocks = pa.mblocks;
  pl.mbgroup = pa.mbgroup;
  pl.queues = pa.queues;
  pl.two_term = reinterpret_cast<int*>(ws + L.two_term);
  pl.g2_pair = reinterpret_cast<const int*>(ws + L.g2_pair);
  pl.g2_ctl = reinterpret_cast<int*>(ws + L.g2_ctl);
  pa.g2_ctl = big ? pl.g2_ctl : nullptr;
  pa.xrow = reinterpret_cast<int*>(ws + L.xrow);
  pl.xrow = pa.xrow;
  CHalf8 ch;
  ch.hi = reinterpret_cast<_Float16*>(ws + L.c_hi);
  ch.lo16 = reinterpret_cast<_Float16*>(ws + L.c_lo16);
  ch.scale = reinterpret_cast<float*>(ws + L.c_scale);
  float* obuf = reinterpret_cast<float*>(ws + L.obuf);
  mark(0);
  launch_route(a->routing_logits, a->logits_dtype, a->routing_bias, a->bias_dtype, T, a->routed_scaling_factor,
               topk_ids, topk_w, &mag, nullptr, 0, s);
  mark(1);
  launch_permute_large(pa, s);
  mark(2);
  if (big) {
    launch_gemm1_big(pb, pl, ch, (int)(L.max_blocks * (I / kBlock)), s);
  } else {
    launch_gemm1_large(pb, pl, ch, large_mt(T), (int)(L.max_blocks * (I / kBlock)), s);
  }
  mark(3);
  // GEMM2's precision from the C that GEMM1 wrote (the activation stage): per pair, with GEMM2's
  // own row table, on the 128-row path; per m-block otherwise
  if (big) {
    launch_g2_plan(pb, pl, ch, (int)L.pmax, s);
  } else {
    launch_c_flags(pl, ch, I, (int)L.max_blocks, s);
  }
  mark(4);
  if (big) {
    // GEMM2 and the combine over the output columns: one pass, or two when the call's pairs
    // outnumber O's rows (the kernels decide from the pair count; a pass with nothing to do exits).
    // O holds every pair a call can have whenever it has Pmax rows: no second pass is launched then
    // (its two empty launches cost ~7 us per call, measured)
    const int passes = L.o_rows >= L.pmax ? 1 : 2;
    for (int pass = 0; pass < 2; pass++) {
      if (pass < passes) launch_gemm2_big(pb, pl, ch, obuf, (int)(L.max_blocks2 * (H / 256)), (int)L.o_rows, pass, s);
      mark(5 + 2 * pass);
      if (pass < passes) launch_combine_pass(pl, obuf, a->output, (int)T, H, (int)L.o_rows, pass, s);
      mark(6 + 2 * pass);
    }
  } else {
    launch_gemm2_large(pb, pl, ch, obuf, large_mt(T), (int)(L.max_blocks * (H / kBlock)), s);
    mark(5);
    launch_combine(pl, obuf, a->output, (int)T, H, s);
    mark(6);
    mark(7);
    mark(8);
  }
  return finish(a, L, topk_ids, topk_w, pl, s);
}

int moefp8_run(const moefp8_args* a, void* workspace, size_t workspace_bytes, void* stream) {
  return run_impl(a, workspace, workspace_bytes, stream, false);
}

int moefp8_run_noalloc(const moefp8_args* a, void* stream) { return run_impl(a, nullptr, 0, stream, true); }

}  // extern "C"
