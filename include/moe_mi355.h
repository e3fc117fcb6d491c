/*
 * moe_mi355.h -- C ABI of the MI355X (gfx950) fused-MoE operator
 *   moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048
 *
 * Plain pointers and sizes only: every tensor argument is a device pointer the
 * caller owns, laid out exactly like the reference's torch tensors (row-major,
 * contiguous).  All work is enqueued on `stream` (a hipStream_t, 0 = null stream);
 * nothing synchronises the host.  Functions return MOE_OK (0) or a negative
 * moe_mi355_status; moe_mi355_strerror() names it.
 *
 * Reference interfaces replaced (paths under the reference repository):
 *   moe_mi355_forward   <- solution/python/main.cpp:66-266  run(...) (pybind `run`,
 *                          main.cpp:268-270) behind kernel.py:95-120 kernel(...)
 *   moe_mi355_route     <- solution/python/kernel.h:39-48 launch_noaux_routing_topk8
 *                          (kernel.cu:56-200)
 *   moe_mi355_dispatch  <- solution/python/kernel.h launch_compute_offsets +
 *                          launch_fill_local_assignments_with_inverse +
 *                          launch_build_padded_arrays (kernel.cu:503-547, 321-351,
 *                          676-757), main.cpp:98-161
 *   moe_mi355_workspace_bytes <- the ~20 per-call torch temporaries of
 *                          main.cpp:87-231, replaced by one caller-provided buffer
 */
#ifndef MOE_MI355_H_
#define MOE_MI355_H_

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__)
#define MOE_MI355_API __attribute__((visibility("default")))
#else
#define MOE_MI355_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Fixed geometry (reference solution/python/kernel.h:9-25). */
#define MOE_MI355_HIDDEN 7168
#define MOE_MI355_INTERMEDIATE 2048
#define MOE_MI355_EXPERTS_GLOBAL 256
#define MOE_MI355_EXPERTS_LOCAL 32
#define MOE_MI355_TOP_K 8
#define MOE_MI355_N_GROUP 8
#define MOE_MI355_TOPK_GROUP 4
#define MOE_MI355_BLOCK 128

/* Largest token count of one call (8T rows stay inside int32 and T * 7168 below 2^32). */
#define MOE_MI355_MAX_TOKENS 524288

typedef enum moe_mi355_status {
    MOE_OK = 0,
    MOE_ERR_NULL_POINTER = -1,     /* a required pointer is NULL */
    MOE_ERR_BAD_SIZE = -2,         /* T < 0 or T > MOE_MI355_MAX_TOKENS */
    MOE_ERR_WORKSPACE = -3,        /* workspace NULL, misaligned or too small */
    MOE_ERR_MISALIGNED = -4,       /* a tensor pointer is not 16-byte aligned */
    MOE_ERR_HIP = -5,              /* a HIP launch failed (see moe_mi355_last_hip_error) */
    MOE_ERR_BAD_TILE = -6,         /* tile_m not supported */
    MOE_ERR_BAD_FLAGS = -7,        /* unknown flag bits, or a forced kernel plan that
                                      cannot run (MOE_MI355_FLAG_FORCE_PLAN) */
    MOE_ERR_BAD_PLAN = -8,         /* internal: a kernel plan names a variant that its
                                      launcher does not have (earlier launches of the
                                      call may have run; the output is not valid) */
    MOE_ERR_NOALLOC_SIZE = -9,     /* moe_mi355_forward_noalloc: T above
                                      MOE_MI355_NOALLOC_MAX_TOKENS */
    MOE_ERR_DEVICE = -10           /* the stream is not on the current device, or the
                                      library's scratch has no address there */
} moe_mi355_status;

/* Arguments of one forward call.  Mirrors kernel.py:95-107 / main.cpp:66-77:
 *   routing_logits       fp32   [T, 256]
 *   routing_bias         bf16   [256]                (raw bf16 bits)
 *   hidden_states        e4m3fn [T, 7168]            (raw bytes)
 *   hidden_states_scale  fp32   [56, T]              (note: block-major)
 *   gemm1_weights        e4m3fn [32, 4096, 7168]
 *   gemm1_weights_scale  fp32   [32, 32, 56]
 *   gemm2_weights        e4m3fn [32, 7168, 2048]
 *   gemm2_weights_scale  fp32   [32, 56, 16]
 *   local_expert_offset  global id of local expert 0 (experts outside [0,256) are
 *                        never selected, as in moe.cu:213-214)
 *   routed_scaling_factor  multiplies the normalised weights (cast to fp32)
 *   output               bf16   [T, 7168]            fully overwritten (DPS)
 *   workspace            device buffer of >= moe_mi355_workspace_bytes(T) bytes,
 *                        256-byte aligned; contents need no initialisation */
typedef struct moe_mi355_args {
    const float* routing_logits;
    const uint16_t* routing_bias;
    const uint8_t* hidden_states;
    const float* hidden_states_scale;
    const uint8_t* gemm1_weights;
    const float* gemm1_weights_scale;
    const uint8_t* gemm2_weights;
    const float* gemm2_weights_scale;
    int64_t local_expert_offset;
    double routed_scaling_factor;
    uint16_t* output;
    int32_t T;
    int32_t flags;      /* MOE_MI355_FLAG_* */
    void* workspace;
    size_t workspace_bytes;
} moe_mi355_args;

/* Call flags (moe_mi355_args.flags).  Without any, the library picks its kernel plan
 * from T alone; nothing else (no environment variable) changes it.
 *   MOE_MI355_FLAG_PROFILE         time each kernel with HIP events (moe_mi355_profile_*)
 *   MOE_MI355_FLAG_FORCE_PLAN      run the GEMM1 / GEMM2 variant pair in bits 8-11 /
 *                                  12-15 (MOE_MI355_FLAGS_PLAN(g1, g2)); for tuning
 *                                  sweeps and tests.  GEMM1: 1 streaming 16-row tiles,
 *                                  2 streaming 32-row tiles, 4 prefill 256-row tiles,
 *                                  7 streaming with shared token rows, 64-row tiles
 *                                  (pairs with GEMM2 5 and 7 only), two workgroups per
 *                                  CU, 8 the same held to three per CU, of which it runs
 *                                  three or two by the call's tile count (the default
 *                                  for 200 <= T <= 1344);
 *                                  GEMM2: 1 streaming 16-row, 3 streaming 32-row,
 *                                  5 prefill on a second list of 128-row tiles (the
 *                                  default for 560 <= T), 7 streaming with shared C
 *                                  rows on the 64-row tiles of GEMM1 7 or 8 (the default
 *                                  for 200 <= T <= 559).  A pair that cannot run
 *                                  together, or an unknown variant, gives
 *                                  MOE_ERR_BAD_FLAGS.
 *                                  GEMM1 variant 5 is variant 1 with the dispatch
 *                                  computed inside it (T <= 64, the default there; pairs
 *                                  with GEMM2 variants 1 and 6): bit-identical output,
 *                                  one launch fewer.  GEMM2 variant 6 is variant 1 with
 *                                  the combine computed inside it (T <= 32, the default
 *                                  up to T = 22, after GEMM1 variant 5, 1 or 9): bit-identical
 *                                  output, one launch fewer.  GEMM1 variant 9 is variant 5
 *                                  with the routing computed inside it too (T <= 8, the
 *                                  default there; pairs with GEMM2 variant 6 only):
 *                                  bit-identical output and workspace routing, one launch
 *                                  fewer.  No kernel clears the C-range flag word (meta[35])
 *                                  before it, so GEMM2 variant 6 checks a set word against
 *                                  C's group exponents (and clears a stale one).
 *   MOE_MI355_FLAG_ROW_SCALES_ON / _OFF  GEMM1 reads the token scales gathered into row
 *                                  order / straight by token (default: gathered from
 *                                  T = 512, except under GEMM1 variants 7 and 8, which gather
 *                                  them itself).  Bit-identical results either way.  GEMM1
 *                                  variants 5 and 9 read them by token: _ON selects the
 *                                  separate dispatch at T <= 64 (and is an error with
 *                                  variant 5 or 9 forced).
 *   MOE_MI355_FLAG_LIST_ORDER      the prefill GEMM1 (variant 4) takes its work items in
 *                                  tile-list order also at T <= 3500 (by default it
 *                                  ranks them by expert rows there, which balances the
 *                                  workgroups' loads); which workgroup computes an item
 *                                  is all that changes, so the output is bit-identical
 *                                  either way.
 * Every variant meets the same tolerance; the flags change speed only. */
#define MOE_MI355_FLAG_PROFILE 1
#define MOE_MI355_FLAG_FORCE_PLAN 2
#define MOE_MI355_FLAG_ROW_SCALES_ON 4
#define MOE_MI355_FLAG_ROW_SCALES_OFF 8
#define MOE_MI355_FLAG_LIST_ORDER 16
#define MOE_MI355_FLAGS_PLAN(g1, g2) \
    (MOE_MI355_FLAG_FORCE_PLAN | (((g1) & 15) << 8) | (((g2) & 15) << 12))
#define MOE_MI355_FLAGS_G1(flags) (((flags) >> 8) & 15)
#define MOE_MI355_FLAGS_G2(flags) (((flags) >> 12) & 15)

/* Bytes of workspace a forward call over T tokens needs. */
MOE_MI355_API size_t moe_mi355_workspace_bytes(int32_t T);

/* The whole operator: routing -> dispatch -> GEMM1+SwiGLU -> GEMM2 -> combine.
 * Replaces main.cpp:66-266 run(). */
MOE_MI355_API int moe_mi355_forward(const moe_mi355_args* args, void* stream);

/* The forward without a workspace argument and without any allocation: no reference
 * counterpart.  It is for callers that cannot allocate device memory -- code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc.  The
 * workspace is the library's own file-scope device array (about 46 MB,
 * moe_mi355_noalloc_scratch_bytes()), one copy on each GPU the library runs on,
 * held until the process ends; its address on a GPU is looked up on the first call
 * there.  args->workspace and args->workspace_bytes are ignored.
 *   - T must be at most MOE_MI355_NOALLOC_MAX_TOKENS (MOE_ERR_NOALLOC_SIZE beyond).
 *   - `stream` must belong to the current device (MOE_ERR_DEVICE otherwise).
 *   - Calls on one GPU share the array: calls that overlap in time on one GPU (on
 *     different streams) race and must not be issued; calls on one stream are
 *     ordered and safe.  Nothing in the array needs clearing between calls.
 *   - Under HIP graph capture: make one eager call on that device first.  The first
 *     call on a device looks up the array's address (hipGetSymbolAddress) and, for
 *     T <= 64, the launch grid (an occupancy query); after it, calls only enqueue
 *     kernels and can be captured (tested for T = 8 and 256). 
 * Results are bit-identical to moe_mi355_forward's. */
#define MOE_MI355_NOALLOC_MAX_TOKENS 256
MOE_MI355_API int moe_mi355_forward_noalloc(const moe_mi355_args* args, void* stream);
/* Size in bytes of that per-GPU array. */
MOE_MI355_API size_t moe_mi355_noalloc_scratch_bytes(void);

/* Routing only (kernel.cu:56-200): topk_ids int32 [T,8], topk_weights fp32 [T,8],
 * ids in selection order (score desc, index asc).  routing_bias is bf16 bits. */
MOE_MI355_API int moe_mi355_route(const float* routing_logits, const uint16_t* routing_bias, int32_t T,
                    double routed_scaling_factor, int32_t* topk_ids, float* topk_weights,
                    void* stream);

/* Dispatch only (kernel.cu:503-547, 321-351): from topk ids/weights build the
 * canonical (local expert asc, token asc) permutation.
 *   expert_offsets int32 [33]   exclusive scan of per-expert counts ([32] = N_a)
 *   sorted_tokens  int32 [8T]   token of row r (rows >= N_a untouched)
 *   sorted_weights fp32  [8T]   routing weight of row r
 *   inverse_rows   int32 [T,8]  row of assignment (t,k) or -1 if not local
 *   tiles          int32 [moe_mi355_max_tiles(T,tile_m), 4]  (expert, first row,
 *                               rows, 0) per tile of <= tile_m rows
 *   num_tiles      int32 [1]
 *   chunk_counts   int32 [ceil(T/256) * 32] scratch (may be NULL when T <= 1024)
 * tile_m must be 16, 32, 64, 128 or 256. */
MOE_MI355_API int moe_mi355_dispatch(const int32_t* topk_ids, const float* topk_weights, int32_t T,
                       int64_t local_expert_offset, int32_t tile_m,
                       int32_t* expert_offsets, int32_t* sorted_tokens,
                       float* sorted_weights, int32_t* inverse_rows, int32_t* tiles,
                       int32_t* num_tiles, int32_t* chunk_counts, void* stream);

/* Blockwise FP8 quantizer of activations, the step before the operator (replaces the
 * reference's quantize_fp8_blockwise_kernel, solution/python/kernel.cu:998-1062, which
 * takes fp32 input and is not launched by the reference operator).  x [rows, cols] is
 * fp32 (x_dtype = MOE_MI355_DTYPE_F32) or bf16 bits (MOE_MI355_DTYPE_BF16).  Per row and
 * 128-column block: scale = absmax / 448 (1 for an all-zero block; NaN is ignored by
 * the absmax), q = e4m3(clamp(x * (1 / scale), -448, 448)) rounded to nearest even
 * (a NaN input gives -448, as the reference's fmaxf/fminf clamp does).
 *   q      e4m3 [rows, cols]
 *   scales fp32 [cols / 128, rows]  (the layout of hidden_states_scale)
 * cols must be a positive multiple of 128, at most MOE_MI355_QUANT_MAX_COLS; x 16-byte,
 * q 8-byte, scales 4-byte aligned. */
#define MOE_MI355_DTYPE_F32 0
#define MOE_MI355_DTYPE_BF16 1
#define MOE_MI355_QUANT_MAX_COLS 32768
MOE_MI355_API int moe_mi355_quantize_fp8_blockwise(const void* x, int32_t x_dtype, int32_t rows,
                                                   int32_t cols, uint8_t* q, float* scales,
                                                   void* stream);

/* Upper bound on the number of row tiles for T tokens and tile height tile_m. */
MOE_MI355_API int32_t moe_mi355_max_tiles(int32_t T, int32_t tile_m);

/* Where a forward call keeps its intermediate arrays inside the workspace (byte
 * offsets), so a caller can inspect routing and dispatch results after the call. */
typedef struct moe_mi355_workspace_layout {
    size_t topk_ids;        /* int32 [T,8] */
    size_t topk_weights;    /* fp32  [T,8] */
    size_t inverse_rows;    /* int32 [T,8] */
    size_t meta;            /* int32 [64]: [0..32] expert offsets, [33] num tiles,
                               [34] tiles of the second list (plans whose GEMM2 runs
                               on 128-row tiles under a GEMM1 on other tiles),
                               [35] nonzero when C went beyond the fp16 range (formats
                               0 and 2), [36] nonzero when an expert row did */
    size_t tiles;           /* int32 [2*max_tiles,4]: the tile list of GEMM1 (tile_m
                               rows), then, for those plans, a second list of 128-row
                               tiles for GEMM2 right after the first list's
                               moe_mi355_max_tiles(T, tile_m) entries */
    size_t sorted_tokens;   /* int32 [8T] */
    size_t sorted_weights;  /* fp32  [8T] */
    size_t chunk_counts;    /* int32 [ceil(T/256), 32] dispatch scratch */
    size_t token_masks;     /* uint32 [T]: each token's local experts (bit e: local expert
                               e), written by the route kernel where the dispatch counts
                               from them (400 <= T <= 16384) */
    size_t row_scales;      /* fp32  [56, 8T]: hidden_states_scale gathered into row order,
                               [kb][row] = scale[kb][sorted_tokens[row]] (the rows
                               in use, for the token counts where GEMM1 reads them) */
    size_t intermediate;    /* SwiGLU output rows C, 8T x (2048 x 4 + 128) bytes:
                               e4m3 hi [8T, 2048], e4m3 lo [8T, 2048]  (hi/lo form:
                                  C = s * (hi + lo / 16), s from intermediate_scales),
                               fp16 [8T, 2048]                          (fp16 form),
                               uint8 [8T, 128] the fp16 form's exponents: per row and
                                  16-column group e >= 0, the values held as
                                  fp16(C 2^-e); e = 0 unless the group holds a value
                                  beyond the fp16 range (meta[35] set).
                               intermediate_format: 0 fp16 form, 1 hi/lo form, 2 fp16
                               form converted to the hi/lo form before GEMM2 */
    size_t intermediate_scales; /* fp32 [16, 8T]: s of row r, 128-column block b at [b][r] */
    size_t expert_out;      /* fp16  [8T, 7168]  GEMM2 output rows */
    size_t expert_out_exp;  /* uint8 [8T, 448]   their 16-column group exponents, as for
                               the fp16 form of C (meta[36] set when one is nonzero) */
    size_t total;
    int32_t tile_m;
    int32_t max_tiles;
    int32_t intermediate_format;
    int32_t dispatch_in_gemm1;  /* 1: GEMM1 computes the dispatch (no dispatch launch) */
    int32_t combine_in_gemm2;   /* 1: GEMM2 writes the output itself (no combine launch;
                                   the expert_out rows are not written) */
} moe_mi355_workspace_layout;

/* The layout of a call over T tokens with the given call flags: the regions do not
 * depend on the flags; tile_m and intermediate_format report the kernel plan that a
 * forward call with the same T and flags runs. */
MOE_MI355_API int moe_mi355_get_workspace_layout(int32_t T, int32_t flags,
                                                 moe_mi355_workspace_layout* out);

/* Stage profiler: with MOE_MI355_FLAG_PROFILE set, each forward call (up to
 * `max_calls` of them) times each of its kernels with a pair of HIP events that the
 * runtime stamps at the kernel's own start and end (hipExtLaunchKernelGGL), so the
 * gaps between kernels are not counted.  moe_mi355_profile_read synchronises those
 * events and writes, for each stage, the sum of its kernels' durations in
 * milliseconds averaged over the recorded calls into stage_ms[0..n) (stage order:
 * route, dispatch (with the token-scale gather), gemm1, gemm2 (with the conversion of
 * C, and the combine when GEMM2 computes it), combine) and returns the number of
 * calls averaged.  A stage without a kernel in the call's plan reads 0. */
MOE_MI355_API int moe_mi355_profile_begin(int32_t max_calls);
MOE_MI355_API int moe_mi355_profile_read(float* stage_ms, int32_t n);
MOE_MI355_API int moe_mi355_profile_end(void);
#define MOE_MI355_NUM_STAGES 5

/* Debug: widen n e4m3 bytes (n % 4 == 0) to bf16 bits with the conversion the GEMM2
 * kernel uses on its bf16 form of C.  No reference counterpart (the reference never
 * widens e4m3); it lets a test pin that conversion against the OCP e4m3 table. */
MOE_MI355_API int moe_mi355_debug_e4m3_to_bf16(const uint8_t* in, uint16_t* out, int32_t n, void* stream);

/* Debug: the same for fp16 bits, the conversion of GEMM2's (default) fp16 form of C.
 * No reference counterpart; a test pins it against the OCP e4m3 table. */
MOE_MI355_API int moe_mi355_debug_e4m3_to_f16(const uint8_t* in, uint16_t* out, int32_t n, void* stream);

MOE_MI355_API const char* moe_mi355_strerror(int status);
/* Text of the last HIP error seen by this library in the calling thread. */
MOE_MI355_API const char* moe_mi355_last_hip_error(void);
/* Library version string. */
MOE_MI355_API const char* moe_mi355_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MOE_MI355_H_ */
