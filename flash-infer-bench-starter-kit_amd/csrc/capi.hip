// capi.hip -- C ABI of the fused-MoE operator: argument checks, workspace layout,
// the launch sequence and a small stage profiler.
//
// Replaces the host orchestration of the reference (solution/python/main.cpp:66-266):
// there ~16 launches and ~20 torch allocations per call; here two to eight launches on
// the caller's stream over one caller-provided workspace, no host synchronisation and no
// allocation:
//   route    (T/4 workgroups; inside GEMM1 for T <= 8) -> topk ids / weights
//   dispatch (1 workgroup, or count + place kernels; inside GEMM1 for T <= 64)
//                                  -> expert offsets, row tiles, permutation, inverse map
//   (gather  -> token scales in row order, for the plans that read them so)
//   gemm1    (persistent)          -> SwiGLU rows C      [N_a, 2048] (fp16 or fp8 hi/lo)
//   (cform   (persistent)          -> fp16 C as hi/lo, for the plans that need it)
//   gemm2    (persistent)          -> fp16 expert rows   [N_a, 7168]
//   combine  (7 T workgroups; inside GEMM2 for T <= 32) -> bf16 output [T, 7168]
// The GEMM grids are sized from the host-known bound on the tile count; each
// workgroup reads the real count written by dispatch and exits when it runs out.  The
// plan, the workspace layout and the argument checks are host_plan.h's.

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "host_plan.h"
#include "moe_device.h"
#include "moe_mi355.h"

namespace moe {
void launch_route(const float*, const uint16_t*, int, float, int*, float*, int*, uint32_t*, int,
                  hipStream_t);
bool launch_dispatch(const int*, const float*, int, int, int, int, int*, int*, int4*, int*, float*,
                     int*, int*, hipStream_t, int*, int4*);
bool launch_dispatch_masks(const int*, const float*, const uint32_t*, int, int, int, int, int*, int*,
                           int4*, int*, int4*, int*, float*, int*, const float*, float*, int,
                           hipStream_t);
bool launch_gemm1(int, const uint8_t*, const TokenScales&, int, const uint8_t*, const float*,
                  const int4*, const int*, const int*, int, const int*, const Intermediate&,
                  bool, hipStream_t);
bool launch_gemm1_dispatch(const RouteIn&, int*, float*, int, int, const uint8_t*, const float*,
                           const uint8_t*, const float*, int*, int4*, int*, float*, int*,
                           const Intermediate&, hipStream_t);
bool launch_gemm2(int, const Intermediate&, const uint8_t*, const float*, const int4*, const int*,
                  const int*, int, const ExpertRows&, hipStream_t);
bool launch_gemm2_combine(const Intermediate&, const uint8_t*, const float*, const int4*, const int*,
                          int*, const int*, const float*, int, uint16_t*, hipStream_t);
void launch_combine(const ExpertRows&, const int*, const float*, const int*, int, uint16_t*, hipStream_t);
void launch_e4m3_to_bf16(const uint8_t*, uint16_t*, int, hipStream_t);
void launch_c_f16_to_hilo(const Intermediate&, const int*, hipStream_t);
void launch_gather_row_scales(const float*, int, const int*, const int*, float*, int, hipStream_t);
void launch_e4m3_to_f16(const uint8_t*, uint16_t*, int, hipStream_t);
void launch_quantize_fp8_blockwise(const void*, int, int, int, uint8_t*, float*, hipStream_t);
}  // namespace moe

namespace moe {
thread_local KernelTimer* g_kernel_timer = nullptr;
}  // namespace moe

namespace {

using moe::host::aligned16;
using moe::host::check_forward_args;
using moe::host::clamp_offset;
using moe::host::fill_layout;
using moe::host::kMaxT;
using moe::host::kRankedMaxT;
using moe::host::Plan;
using moe::host::workspace_regions;

thread_local char g_hip_error[256] = "";

int hip_status(hipError_t e) {
    if (e == hipSuccess) return MOE_OK;
    snprintf(g_hip_error, sizeof g_hip_error, "%s (%d)", hipGetErrorString(e), (int)e);
    return MOE_ERR_HIP;
}

// ---- stage profiler ------------------------------------------------------------
// One record per profiled call: a start and a stop event for each of its kernels
// (launch_kernel fills them) and the stage of each kernel.
constexpr int kMaxTimedLaunches = 8;   // kernels of one forward call
struct Profiler {
    hipEvent_t* ev = nullptr;          // [slots][2 kMaxTimedLaunches]
    int* stage = nullptr;              // [slots][kMaxTimedLaunches]
    moe::KernelTimer* rec = nullptr;   // [slots]
    int slots = 0;
    int used = 0;
};
Profiler g_prof;

// ---- the library's own workspace (moe_mi355_forward_noalloc) ---------------------
// A workspace for calls of up to MOE_MI355_NOALLOC_MAX_TOKENS tokens in a file-scope
// device array: the code object's loader places one copy on every GPU the library
// runs on, held until the process ends, so a call needs no allocation.  In host code
// `scratch` names a host-side stand-in, never the device memory: its device address
// on the current GPU comes from hipGetSymbolAddress, once per device (kept in
// g_scratch_dev), and only that address reaches the kernels.  Every call on one GPU
// shares the array: nothing in it needs to start at zero (the route kernel clears the
// flag words, or GEMM1 variant 9 marks them with the call's own tag; dispatch writes
// every offset, count and row the later kernels read),
// and calls that overlap on one GPU (two streams) race on it.
constexpr size_t kScratchBytes = workspace_regions(MOE_MI355_NOALLOC_MAX_TOKENS).total;
static_assert(kScratchBytes <= (size_t)64 << 20, "keep the per-GPU scratch array modest");
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices] = {};

}  // namespace

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

// Device address of `scratch` on the current GPU, looked up on the first call there.
int scratch_on_current_device(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_status(e);
    if (dev < 0 || dev >= kMaxDevices) return MOE_ERR_DEVICE;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_dev[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_status(e);
        if (p == nullptr || ((uintptr_t)p & 255u)) return MOE_ERR_DEVICE;
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return MOE_OK;
}

// The forward's launch sequence over a workspace of ws_bytes at ws (the caller's, or
// for moe_mi355_forward_noalloc the library's own).  Returns MOE_OK or a status; a
// status from a failed launch means the earlier launches of the call may have run.
int forward_impl(const moe_mi355_args& a, void* workspace, size_t ws_bytes, hipStream_t s) {
    const int32_t T = a.T;
    moe_mi355_workspace_layout L;
    Plan plan;
    const int cst = check_forward_args(a, workspace, ws_bytes, &L, &plan);
    if (cst != MOE_OK || T == 0) return cst;

    uint8_t* ws = static_cast<uint8_t*>(workspace);
    int* ids = reinterpret_cast<int*>(ws + L.topk_ids);
    float* wts = reinterpret_cast<float*>(ws + L.topk_weights);
    int* inv = reinterpret_cast<int*>(ws + L.inverse_rows);
    int* meta = reinterpret_cast<int*>(ws + L.meta);
    int4* tiles = reinterpret_cast<int4*>(ws + L.tiles);
    int* stok = reinterpret_cast<int*>(ws + L.sorted_tokens);
    float* sw = reinterpret_cast<float*>(ws + L.sorted_weights);
    const moe::Intermediate inter{ws + L.intermediate, reinterpret_cast<float*>(ws + L.intermediate_scales),
                                  T * moe::kTopK};
    const moe::ExpertRows rows{reinterpret_cast<uint16_t*>(ws + L.expert_out),
                               ws + L.expert_out_exp};
    int* chunk_cnt = reinterpret_cast<int*>(ws + L.chunk_counts);
    float* row_scales = reinterpret_cast<float*>(ws + L.row_scales);
    int* num_tiles = meta + moe::kEL + 1;

    // The status reports this call's launches only: an error some earlier, unrelated
    // HIP call left in this thread's last-error slot is cleared first.
    (void)hipGetLastError();
    const bool prof = (a.flags & MOE_MI355_FLAG_PROFILE) && g_prof.rec && g_prof.used < g_prof.slots;
    const bool ranked = !(a.flags & MOE_MI355_FLAG_LIST_ORDER) && T <= kRankedMaxT;
    moe::KernelTimer* timer = prof ? &g_prof.rec[g_prof.used++] : nullptr;
    if (timer) timer->n = 0;
    auto stage = [timer](int st) {
        if (timer) timer->cur_stage = st;
    };
    moe::g_kernel_timer = timer;   // the launches below time themselves (cleared before return)

    // GEMM1 variant 9 routes the tokens itself (timed as the GEMM1 stage)
    const int offset = clamp_offset(a.local_expert_offset);
    // the dispatch in one launch from the route kernel's local-expert masks (with the
    // token-scale gather when GEMM1 reads the scales in row order)
    const bool by_masks =
        !plan.dispatch_in_gemm1 && T >= moe::kMaskDispatchMinT && T <= moe::kMaskDispatchMaxT;
    uint32_t* masks = by_masks ? reinterpret_cast<uint32_t*>(ws + L.token_masks) : nullptr;
    stage(0);
    if (!plan.route_in_gemm1)
        moe::launch_route(a.routing_logits, a.routing_bias, T, (float)a.routed_scaling_factor, ids,
                          wts, meta + moe::kCWideFlag, masks, offset, s);
    stage(1);
    const int max_tiles = moe::dispatch_max_tiles(T, plan.tm);
    const bool half = plan.tm2 > 0;   // GEMM2 walks the second (128-row) tile list
    int4* tiles2 = tiles + max_tiles;
    int* num_tiles2 = meta + moe::kEL + 2;
    // GEMM1 variant 5 computes the dispatch itself (timed as the GEMM1 stage)
    bool ok = true;
    if (by_masks)
        ok = moe::launch_dispatch_masks(ids, wts, masks, T, offset, plan.tm, plan.tm2, meta, num_tiles,
                                        tiles, half ? num_tiles2 : nullptr, half ? tiles2 : nullptr,
                                        stok, sw, inv, plan.by_row ? a.hidden_states_scale : nullptr,
                                        plan.by_row ? row_scales : nullptr, T * moe::kTopK, s);
    else if (!plan.dispatch_in_gemm1)
        ok = moe::launch_dispatch(ids, wts, T, offset, plan.tm, plan.tm2, meta, num_tiles, tiles, stok,
                                  sw, inv, chunk_cnt, s, half ? num_tiles2 : nullptr,
                                  half ? tiles2 : nullptr);
    // GEMM1 reads the token scales gathered into row order (counted in the dispatch stage)
    // or, where the gather would cost more than it saves, straight by token
    if (ok && plan.by_row && !by_masks)
        moe::launch_gather_row_scales(a.hidden_states_scale, T, stok, meta, row_scales,
                                      T * moe::kTopK, s);
    const moe::TokenScales sa = plan.by_row ? moe::TokenScales{row_scales, T * moe::kTopK, 1}
                                            : moe::TokenScales{a.hidden_states_scale, T, 0};
    stage(2);
    if (plan.dispatch_in_gemm1) {
        const moe::RouteIn rin{plan.route_in_gemm1 ? a.routing_logits : nullptr, a.routing_bias,
                               (float)a.routed_scaling_factor};
        ok = ok && moe::launch_gemm1_dispatch(rin, ids, wts, T, offset,
                                              a.hidden_states, a.hidden_states_scale,
                                              a.gemm1_weights, a.gemm1_weights_scale, meta, tiles,
                                              stok, sw, inv, inter, s);
    }
    else
        ok = ok && moe::launch_gemm1(plan.g1, a.hidden_states, sa, T, a.gemm1_weights,
                                     a.gemm1_weights_scale, tiles, num_tiles, meta, max_tiles,
                                     stok, inter, ranked, s);
    stage(3);
    if (ok && plan.convert) moe::launch_c_f16_to_hilo(inter, meta, s);   // in the GEMM2 stage
    if (ok && plan.combine_in_gemm2)      // GEMM2 writes the output (timed as the GEMM2 stage)
        ok = moe::launch_gemm2_combine(inter, a.gemm2_weights, a.gemm2_weights_scale, tiles,
                                       num_tiles, meta, inv, sw, T, a.output, s);
    else if (ok && half)
        ok = moe::launch_gemm2(plan.g2, inter, a.gemm2_weights, a.gemm2_weights_scale, tiles2,
                               num_tiles2, meta, moe::dispatch_max_tiles(T, plan.tm2), rows, s);
    else if (ok)
        ok = moe::launch_gemm2(plan.g2, inter, a.gemm2_weights, a.gemm2_weights_scale, tiles,
                               num_tiles, meta, max_tiles, rows, s);
    stage(4);
    if (ok && !plan.combine_in_gemm2)
        moe::launch_combine(rows, meta + moe::kRowsWideFlag, sw, inv, T, a.output, s);
    moe::g_kernel_timer = nullptr;
    const int hst = hip_status(hipGetLastError());
    if (hst != MOE_OK) return hst;
    return ok ? MOE_OK : MOE_ERR_BAD_PLAN;
}

}  // namespace

extern "C" {

// The build passes a hash of the sources (build.py, source_hash) that the loader
// compares with the sources next to the library before it loads it.
#ifndef MOE_MI355_SRC_HASH
#define MOE_MI355_SRC_HASH "0000000000000000"
#endif
const char* moe_mi355_version(void) { return "moe_mi355 0.1 gfx950; moe_mi355 src " MOE_MI355_SRC_HASH; }

const char* moe_mi355_last_hip_error(void) { return g_hip_error; }

const char* moe_mi355_strerror(int status) {
    switch (status) {
        case MOE_OK: return "ok";
        case MOE_ERR_NULL_POINTER: return "a required pointer is NULL";
        case MOE_ERR_BAD_SIZE: return "token count out of range";
        case MOE_ERR_WORKSPACE: return "workspace NULL, not 256-byte aligned, or too small";
        case MOE_ERR_MISALIGNED: return "a tensor pointer is not 16-byte aligned";
        case MOE_ERR_HIP: return "HIP launch failed";
        case MOE_ERR_BAD_TILE: return "unsupported tile height";
        case MOE_ERR_BAD_FLAGS: return "unknown flag bits, or a forced kernel plan that cannot run";
        case MOE_ERR_BAD_PLAN: return "a kernel plan names a variant its launcher does not have";
        case MOE_ERR_NOALLOC_SIZE:
            return "moe_mi355_forward_noalloc: T beyond MOE_MI355_NOALLOC_MAX_TOKENS (use moe_mi355_forward with a workspace)";
        case MOE_ERR_DEVICE: return "the stream is not on the current device, or no device scratch there";
        default: return "unknown status";
    }
}

int32_t moe_mi355_max_tiles(int32_t T, int32_t tile_m) {
    if (T < 0 || tile_m <= 0) return 0;
    return moe::dispatch_max_tiles(T, tile_m);
}

size_t moe_mi355_workspace_bytes(int32_t T) {
    moe_mi355_workspace_layout L;
    if (fill_layout(T, 0, &L) != MOE_OK) return 0;
    return L.total;
}

int moe_mi355_get_workspace_layout(int32_t T, int32_t flags, moe_mi355_workspace_layout* out) {
    if (!out) return MOE_ERR_NULL_POINTER;
    return fill_layout(T, flags, out);
}

int moe_mi355_route(const float* routing_logits, const uint16_t* routing_bias, int32_t T,
                    double routed_scaling_factor, int32_t* topk_ids, float* topk_weights,
                    void* stream) {
    if (T < 0 || T > kMaxT) return MOE_ERR_BAD_SIZE;
    if (T == 0) return MOE_OK;
    if (!routing_logits || !routing_bias || !topk_ids || !topk_weights) return MOE_ERR_NULL_POINTER;
    if (!aligned16(routing_logits) || ((uintptr_t)routing_bias & 7u)) return MOE_ERR_MISALIGNED;
    hipStream_t s = (hipStream_t)stream;
    moe::launch_route(routing_logits, routing_bias, T, (float)routed_scaling_factor, topk_ids,
                      topk_weights, nullptr, nullptr, 0, s);
    return hip_status(hipGetLastError());
}

int moe_mi355_quantize_fp8_blockwise(const void* x, int32_t x_dtype, int32_t rows, int32_t cols,
                                     uint8_t* q, float* scales, void* stream) {
    if (x_dtype != MOE_MI355_DTYPE_F32 && x_dtype != MOE_MI355_DTYPE_BF16) return MOE_ERR_BAD_SIZE;
    if (rows < 0 || cols <= 0 || cols % MOE_MI355_BLOCK != 0 || cols > MOE_MI355_QUANT_MAX_COLS)
        return MOE_ERR_BAD_SIZE;
    if (rows == 0) return MOE_OK;
    if (!x || !q || !scales) return MOE_ERR_NULL_POINTER;
    if (!aligned16(x) || ((uintptr_t)q & 7u) || ((uintptr_t)scales & 3u)) return MOE_ERR_MISALIGNED;
    moe::launch_quantize_fp8_blockwise(x, x_dtype, rows, cols, q, scales, (hipStream_t)stream);
    return hip_status(hipGetLastError());
}

int moe_mi355_dispatch(const int32_t* topk_ids, const float* topk_weights, int32_t T,
                       int64_t local_expert_offset, int32_t tile_m, int32_t* expert_offsets,
                       int32_t* sorted_tokens, float* sorted_weights, int32_t* inverse_rows,
                       int32_t* tiles, int32_t* num_tiles, int32_t* chunk_counts, void* stream) {
    if (T < 0 || T > kMaxT) return MOE_ERR_BAD_SIZE;
    if (tile_m != 16 && tile_m != 32 && tile_m != 64 && tile_m != 128 && tile_m != 256)
        return MOE_ERR_BAD_TILE;
    if (!topk_ids || !topk_weights || !expert_offsets || !sorted_tokens || !sorted_weights ||
        !inverse_rows || !tiles || !num_tiles || (T > 1024 && !chunk_counts))
        return MOE_ERR_NULL_POINTER;
    if (!aligned16(tiles) || !aligned16(topk_ids) || !aligned16(topk_weights))
        return MOE_ERR_MISALIGNED;
    hipStream_t s = (hipStream_t)stream;
    moe::launch_dispatch(topk_ids, topk_weights, T, clamp_offset(local_expert_offset), tile_m, 0,
                         expert_offsets, num_tiles, reinterpret_cast<int4*>(tiles), sorted_tokens,
                         sorted_weights, inverse_rows, chunk_counts, s, nullptr, nullptr);
    return hip_status(hipGetLastError());
}

int moe_mi355_forward(const moe_mi355_args* a, void* stream) {
    if (!a) return MOE_ERR_NULL_POINTER;
    return forward_impl(*a, a->workspace, a->workspace_bytes, (hipStream_t)stream);
}

int moe_mi355_forward_noalloc(const moe_mi355_args* a, void* stream) {
    if (!a) return MOE_ERR_NULL_POINTER;
    if (a->T < 0) return MOE_ERR_BAD_SIZE;
    if (a->T > MOE_MI355_NOALLOC_MAX_TOKENS) return MOE_ERR_NOALLOC_SIZE;
    if (a->T == 0) return MOE_OK;
    hipStream_t s = (hipStream_t)stream;
    int cur = -1, sdev = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return hip_status(e);
    e = hipStreamGetDevice(s, &sdev);
    if (e != hipSuccess) return hip_status(e);
    if (sdev != cur) return MOE_ERR_DEVICE;
    void* ws = nullptr;
    const int st = scratch_on_current_device(&ws);
    if (st != MOE_OK) return st;
    return forward_impl(*a, ws, kScratchBytes, s);
}

size_t moe_mi355_noalloc_scratch_bytes(void) { return kScratchBytes; }

int moe_mi355_profile_begin(int32_t max_calls) {
    moe_mi355_profile_end();
    if (max_calls <= 0) return MOE_ERR_BAD_SIZE;
    const int n = max_calls * 2 * kMaxTimedLaunches;
    g_prof.ev = new hipEvent_t[n];
    for (int i = 0; i < n; ++i) {
        const hipError_t e = hipEventCreate(&g_prof.ev[i]);
        if (e != hipSuccess) {
            for (int j = 0; j < i; ++j) (void)hipEventDestroy(g_prof.ev[j]);
            delete[] g_prof.ev;
            g_prof.ev = nullptr;
            return hip_status(e);
        }
    }
    g_prof.stage = new int[max_calls * kMaxTimedLaunches];
    g_prof.rec = new moe::KernelTimer[max_calls];
    for (int c = 0; c < max_calls; ++c)
        g_prof.rec[c] = {g_prof.ev + c * 2 * kMaxTimedLaunches, g_prof.stage + c * kMaxTimedLaunches,
                         kMaxTimedLaunches, 0, 0};
    g_prof.slots = max_calls;
    g_prof.used = 0;
    return MOE_OK;
}

// Average over the recorded calls of each stage's time: the sum of its kernels' times,
// each from the HIP events stamped at that kernel's start and end.
int moe_mi355_profile_read(float* stage_ms, int32_t n) {
    if (!stage_ms) return MOE_ERR_NULL_POINTER;
    if (!g_prof.rec || g_prof.used == 0) return 0;
    const int ns = MOE_MI355_NUM_STAGES;
    double sum[MOE_MI355_NUM_STAGES] = {0};
    for (int c = 0; c < g_prof.used; ++c) {
        const moe::KernelTimer& r = g_prof.rec[c];
        for (int i = 0; i < r.n; ++i) {
            const hipError_t e = hipEventSynchronize(r.ev[2 * i + 1]);
            if (e != hipSuccess) return hip_status(e);
            float ms = 0.f;
            const hipError_t e2 = hipEventElapsedTime(&ms, r.ev[2 * i], r.ev[2 * i + 1]);
            if (e2 != hipSuccess) return hip_status(e2);
            if (r.stage[i] >= 0 && r.stage[i] < ns) sum[r.stage[i]] += ms;
        }
    }
    for (int st = 0; st < ns && st < n; ++st) stage_ms[st] = (float)(sum[st] / g_prof.used);
    return g_prof.used;
}

int moe_mi355_profile_end(void) {
    if (g_prof.ev) {
        for (int i = 0; i < g_prof.slots * 2 * kMaxTimedLaunches; ++i) (void)hipEventDestroy(g_prof.ev[i]);
        delete[] g_prof.ev;
    }
    delete[] g_prof.stage;
    delete[] g_prof.rec;
    g_prof = Profiler{};
    return MOE_OK;
}

int moe_mi355_debug_e4m3_to_bf16(const uint8_t* in, uint16_t* out, int32_t n, void* stream) {
    if (!in || !out) return MOE_ERR_NULL_POINTER;
    if (n < 0 || (n & 3)) return MOE_ERR_BAD_SIZE;
    moe::launch_e4m3_to_bf16(in, out, n, (hipStream_t)stream);
    return hip_status(hipGetLastError());
}

int moe_mi355_debug_e4m3_to_f16(const uint8_t* in, uint16_t* out, int32_t n, void* stream) {
    if (!in || !out) return MOE_ERR_NULL_POINTER;
    if (n < 0 || (n & 3)) return MOE_ERR_BAD_SIZE;
    moe::launch_e4m3_to_f16(in, out, n, (hipStream_t)stream);
    return hip_status(hipGetLastError());
}

}  // extern "C"
