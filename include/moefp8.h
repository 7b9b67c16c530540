/*
 * moefp8.h -- C ABI of the MI355X (gfx950) fp8 block-scale MoE operator
 * "moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048".
 *
 * The reference operator is the Python entry point
 *   solutions/moe_fp8/main.py:173-243   run(routing_logits, routing_bias,
 *       hidden_states, hidden_states_scale, gemm1_weights, gemm1_weights_scale,
 *       gemm2_weights, gemm2_weights_scale, local_expert_offset,
 *       routed_scaling_factor) -> bf16 [T, H]
 * packed as solutions/moe_fp8/solution.json:5-15 (entry_point main.py::run,
 * destination_passing_style=false).  That reference exposes no C ABI; the
 * functions below are what its Python binding (a ctypes stub, see the
 * integration notes shipped with this library) calls.
 *
 * Conventions
 *   - Every pointer in moefp8_args is a device pointer on the current HIP device.
 *   - Tensors are dense row-major with the shapes given below.
 *   - The caller owns all memory: output and workspace are passed in; the
 *     library allocates nothing and never synchronises the host.
 *   - All work is enqueued on `stream`, in order.  Calls on one stream are
 *     serialised by the stream; the library keeps no mutable global state.
 *   - Every function returns MOEFP8_OK (0) or a negative moefp8_status.
 *     Argument errors are detected on the host before any launch.
 */
#ifndef MOEFP8_H_
#define MOEFP8_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MOEFP8_ABI_VERSION 7

/* Operator constants (solutions/moe_fp8/main.py:22-29). */
#define MOEFP8_E_GLOBAL 256
#define MOEFP8_TOP_K 8
#define MOEFP8_N_GROUP 8
#define MOEFP8_TOPK_GROUP 4
#define MOEFP8_BLOCK 128

typedef enum moefp8_status {
  MOEFP8_OK = 0,
  MOEFP8_ERR_NULL_POINTER = -1,   /* a required pointer is NULL */
  MOEFP8_ERR_SHAPE = -2,          /* T < 0, E_local out of [1,256], H or I not a positive multiple of 128 */
  MOEFP8_ERR_DTYPE = -3,          /* unsupported logits / bias dtype code */
  MOEFP8_ERR_ALIGNMENT = -4,      /* a pointer is not 16-byte aligned */
  MOEFP8_ERR_WORKSPACE = -5,      /* workspace NULL or smaller than moefp8_workspace_size() */
  MOEFP8_ERR_LAUNCH = -6,         /* a kernel launch failed (hipGetLastError) */
  MOEFP8_ERR_DEVICE = -7,         /* current device is not gfx950 / HIP runtime error */
  MOEFP8_ERR_SCRATCH_LIMIT = -8   /* moefp8_run_noalloc: the sizes need more than its static scratch */
} moefp8_status;

/* dtype codes for routing_logits / routing_bias (main.py:145-146 upcast both to fp32). */
typedef enum moefp8_dtype {
  MOEFP8_DTYPE_F32 = 0,
  MOEFP8_DTYPE_BF16 = 1,
  MOEFP8_DTYPE_F16 = 2
} moefp8_dtype;

typedef struct moefp8_args {
  /* inputs (main.py:173-184) */
  const void* routing_logits;        /* [T, 256], logits_dtype                      */
  const void* routing_bias;          /* [256], bias_dtype                           */
  const uint8_t* hidden_states;      /* [T, H] float8_e4m3fn (OCP)                  */
  const float* hidden_states_scale;  /* [H/128, T] fp32, scale[kb, t] (transposed)  */
  const uint8_t* gemm1_weights;      /* [E_local, 2I, H] e4m3fn; rows [0,I) up, [I,2I) gate */
  const float* gemm1_weights_scale;  /* [E_local, 2I/128, H/128] fp32               */
  const uint8_t* gemm2_weights;      /* [E_local, H, I] e4m3fn                      */
  const float* gemm2_weights_scale;  /* [E_local, H/128, I/128] fp32                */
  int64_t num_tokens;                /* T >= 0                                      */
  int32_t num_local_experts;         /* E_local = gemm1_weights.shape[0], 1..256    */
  int32_t hidden_size;               /* H, multiple of 128 (7168 for the operator)  */
  int32_t intermediate_size;         /* I, multiple of 128 (2048 for the operator)  */
  int32_t local_expert_offset;       /* global id of local expert 0 (main.py:188-191, 219-221) */
  float routed_scaling_factor;       /* main.py:164, 192-193                        */
  int32_t logits_dtype;              /* moefp8_dtype                                */
  int32_t bias_dtype;                /* moefp8_dtype                                */
  /* output (main.py:243): bf16 [T, H] (fp32 with output_f32); rows of tokens with no local
   * expert are 0 */
  void* output;
  /* optional outputs, may be NULL (used by parity tests):
   *   topk_ids        [T, 8] int32, the routed global expert ids, ascending
   *   topk_weights    [T, 8] fp32, weights[t, topk_ids[t, j]] of main.py:164
   *   expert_offsets  [E_local + 1] int32, exclusive prefix of per-expert token counts
   *   permuted_tokens [T * min(8, E_local)] int32; entries [offsets[e], offsets[e+1])
   *                   are the tokens routed to local expert e in ascending order
   *                   (main.py:222-225); the tail past offsets[E_local] is unspecified */
  int32_t* topk_ids;
  float* topk_weights;
  int32_t* expert_offsets;
  int32_t* permuted_tokens;
  /* optional, may be NULL: array of MOEFP8_NUM_STAGE_EVENTS hipEvent_t created by the
   * caller.  Event i is recorded on `stream` before stage i (route, permute, GEMM1,
   * activation, GEMM2, combine, then GEMM2 and combine of the second half of the output
   * columns; GEMM1 applies SwiGLU itself, so the activation stage is empty, for T <= 64 GEMM2
   * also does the combine, leaving that stage empty too, and calls whose per-pair output rows
   * fit the workspace in one pass leave the last two stages empty) and the last one after the
   * last combine, so stage i's device time is hipEventElapsedTime(ev[i], ev[i+1]).  Used for
   * live per-kernel timing. */
  void* stage_events;
  /* optional, may be NULL: [T, H] dense rows in shared_dtype (MOEFP8_DTYPE_F32 or
   * MOEFP8_DTYPE_BF16, 16-byte aligned) added to each token's routed sum in fp32 before its
   * single bf16 rounding: output[t] = bf16(sum_e w_e O_e[t] + shared_output[t]).  This is
   * DeepSeek-V3's shared-expert add fused into the combine (no counterpart in the reference
   * operator, whose callers add the shared expert's output afterwards).  Tokens with no local
   * expert get bf16(shared_output[t]). */
  const void* shared_output;
  int32_t shared_dtype;
  /* 0: bf16 output, as the reference's run.  1: fp32 output, the same per-token sum before
   * its bf16 rounding (bf16(fp32 output) equals the bf16 output bit for bit), for callers that
   * add further partial sums and round once, such as expert-parallel ranks reducing their
   * outputs (no counterpart in the reference, whose ranks each return bf16). */
  int32_t output_f32;
} moefp8_args;

#define MOEFP8_NUM_STAGE_EVENTS 9

/* ABI version of the loaded library (MOEFP8_ABI_VERSION of its build). */
int moefp8_abi_version(void);

/* Human-readable text of a status code (static storage). */
const char* moefp8_strerror(int status);

/* Bytes of device workspace that moefp8_run needs for these sizes
 * (no counterpart in the reference: main.py:202 allocates its scratch through
 * the torch allocator inside run()). */
int moefp8_workspace_size(int64_t num_tokens, int32_t num_local_experts, int32_t hidden_size,
                          int32_t intermediate_size, size_t* bytes);

/* Kernel family moefp8_run uses for these sizes (host only, no device needed; no counterpart in
 * the reference, whose run() always loops over experts in Python, main.py:218-241):
 * MOEFP8_PATH_SMALL_T (T <= 64: weight-streaming GEMMs), MOEFP8_PATH_GROUPED (4-wave grouped
 * GEMMs) or MOEFP8_PATH_ROWS128 (128-row LDS-staged grouped GEMMs), or a negative status. */
#define MOEFP8_PATH_SMALL_T 0
#define MOEFP8_PATH_GROUPED 1
#define MOEFP8_PATH_ROWS128 2
int moefp8_path(int64_t num_tokens, int32_t num_local_experts, int32_t hidden_size, int32_t intermediate_size);

/* Passes moefp8_run makes over the output columns for these sizes when the routing yields
 * num_pairs local (token, expert) pairs (host only; no counterpart in the reference): 1, or 2 on
 * the MOEFP8_PATH_ROWS128 path when the workspace's fp32 per-pair output rows cannot hold all
 * columns of every pair.  Above 1 GiB for T x min(8, E_local) rows, the workspace holds rows for
 * half that many pairs (T > 4681 at H = 7168, E_local >= 8); a call with more pairs runs GEMM2 and
 * the combine once per half of the output columns.  A negative status for bad sizes. */
int moefp8_output_passes(int64_t num_tokens, int32_t num_local_experts, int32_t hidden_size,
                         int32_t intermediate_size, int64_t num_pairs);

/* The operator: replaces solutions/moe_fp8/main.py:173-243 (run).
 * routing (main.py:139-165) -> token permutation (main.py:216-226) ->
 * GEMM1 + SwiGLU (main.py:229-233) -> GEMM2 (main.py:234-238) ->
 * weighted combine + bf16 round (main.py:240-243), all enqueued on `stream`
 * (a hipStream_t; NULL = legacy default stream). */
int moefp8_run(const moefp8_args* args, void* workspace, size_t workspace_bytes, void* stream);

/* The operator without allocation.  No counterpart in the reference: for callers that cannot
 * allocate device memory, such as code under HIP graph capture, tight serving loops and harnesses
 * that forbid hipMalloc.  Same arguments, work and results as moefp8_run, but the workspace is a
 * static device array of MOEFP8_NOALLOC_SCRATCH_BYTES (64 MiB) per device that loads the library,
 * held until the process ends; sizes whose moefp8_workspace_size() exceeds it return
 * MOEFP8_ERR_SCRATCH_LIMIT before any launch (at H = 7168, I = 2048 it covers every T <= 226 for
 * E_local 8, 32 or 256: the small-T and grouped paths and the 128-row path up to T = 226).  The
 * call itself allocates nothing.  Every call on a device shares that device's array: calls that overlap on
 * one device (different streams, or other host threads) race and must be serialised by the
 * caller; calls on one stream are ordered by it.  Each call initialises what it reads. */
#define MOEFP8_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int moefp8_run_noalloc(const moefp8_args* args, void* stream);

/* Routing alone: replaces solutions/moe_fp8/main.py:139-165 (_route).
 * Writes topk_ids [T, 8] int32 (ascending ids) and topk_weights [T, 8] fp32. */
int moefp8_route(const void* routing_logits, int32_t logits_dtype, const void* routing_bias,
                 int32_t bias_dtype, int64_t num_tokens, float routed_scaling_factor,
                 int32_t* topk_ids, float* topk_weights, void* stream);

/* Per-token 1x128 quantization of the hidden states, the step before the operator: produces
 * the hidden_states / hidden_states_scale pair that moefp8_run reads (and that
 * solutions/moe_fp8/main.py:129-136 dequantizes).  x [T, H] bf16 (x_dtype 1) or fp32 (0),
 * row-major, 16-byte aligned; per token and 128 columns scale = amax / 448 (1 for an all-zero
 * block), q = e4m3fn(x / scale) rounded to nearest even.  Writes hidden_out e4m3fn [T, H]
 * (8-byte aligned) and scale_out fp32 [H/128, T].  Inputs must be finite. */
int moefp8_quantize_hidden(const void* x, int32_t x_dtype, int64_t num_tokens, int32_t hidden_size,
                           void* hidden_out, float* scale_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOEFP8_H_ */
