// capi.hip -- C ABI of the fused-MoE operator: argument checks, workspace layout,
// the launch sequence and a small stage profiler.
//
// Replaces the host orchestration of the reference (solution/python/main.cpp:66-266):
// there ~16 launches and ~20 torch allocations per call; here five launches on the
// caller's stream over one caller-provided workspace, no host synchronisation and no
// allocation:
//   route    (T/4 workgroups)      -> topk ids / weights
//   dispatch (1 workgroup)         -> expert offsets, row tiles, permutation, inverse map
//   gemm1    (persistent)          -> SwiGLU rows C      [N_a, 2048] (fp16 or fp8 hi/lo)
//   (cform   (persistent)          -> fp16 C as hi/lo, for the plans that need it)
//   gemm2    (persistent)          -> fp16 expert rows   [N_a, 7168]
//   combine  (7 T workgroups)      -> bf16 output        [T, 7168]
// The GEMM grids are sized from the host-known bound on the tile count; each
// workgroup reads the real count written by dispatch and exits when it runs out.

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "moe_device.h"
#include "moe_mi355.h"

namespace moe {
void launch_route(const float*, const uint16_t*, int, float, int*, float*, int*, hipStream_t);
bool launch_dispatch(const int*, const float*, int, int, int, int, int*, int*, int4*, int*, float*,
                     int*, int*, hipStream_t, int*, int4*);
int dispatch_max_tiles(int T, int tm);
bool launch_gemm1(int, const uint8_t*, const TokenScales&, int, const uint8_t*, const float*,
                  const int4*, const int*, const int*, int, const int*, const Intermediate&,
                  bool, hipStream_t);
bool launch_gemm1_dispatch(const int*, const float*, int, int, const uint8_t*, const float*,
                           const uint8_t*, const float*, int*, int4*, int*, float*, int*,
                           const Intermediate&, hipStream_t);
constexpr int kDispatchInGemm1MaxT = 64;
bool launch_gemm2(int, const Intermediate&, const uint8_t*, const float*, const int4*, const int*,
                  const int*, int, const ExpertRows&, hipStream_t);
void launch_combine(const ExpertRows&, const int*, const float*, const int*, int, uint16_t*, hipStream_t);
void launch_e4m3_to_bf16(const uint8_t*, uint16_t*, int, hipStream_t);
void launch_c_f16_to_hilo(const Intermediate&, const int*, hipStream_t);
void launch_gather_row_scales(const float*, int, const int*, const int*, float*, int, hipStream_t);
void launch_e4m3_to_f16(const uint8_t*, uint16_t*, int, hipStream_t);
void launch_quantize_fp8_blockwise(const void*, int, int, int, uint8_t*, float*, hipStream_t);
}  // namespace moe

namespace {

// Largest T: 8T rows stay inside int32 and T * 7168 (the byte offset of the last
// token row, used as a 32-bit buffer offset by the prefill kernels) below 2^32.
constexpr int32_t kMaxT = 1 << 19;
constexpr int kMinTileM = 16;           // smallest row tile; sizes the tile list

// Kernel plan per token count: the GEMM1 / GEMM2 variants (ids of launch_gemm1 /
// launch_gemm2) and what they imply: the tile height of the dispatch's first list (the
// GEMM1's), an optional second list of 128-row tiles (GEMM2 variant 5), and whether the
// fp16 C of a streaming GEMM1 is converted to the hi/lo form for a prefill GEMM2.
// Small T streams weights with the register-staged kernels, C in fp16: 16-row tiles up
// to T = 88, 32-row tiles (GEMM1 with two column groups per wave, GEMM2 with two row
// blocks per wave) beyond.  From T = 300 GEMM1 is the token-sharing kernel on 64-row
// tiles (fewer requests per output once an expert has dozens of rows), feeding the
// prefill GEMM2 (128-row tiles, FP8 MFMA on the hi/lo form): up to T = 960 with three
// workgroups per CU (variant 8), then with two (variant 7), whose fewer resident
// workgroups split the items of the larger tile lists into better-filled rounds; from
// T = 1345 both GEMMs are the MFMA-bound prefill kernels on 256-row tiles (GEMM2 on the
// 128-row second list).  The boundaries come from wall-clock sweeps of the pairs at
// T = 72 .. 2560 on MI355X over five routing seeds (light to heavy routing to the local
// experts): between T = 960 and 1344 the best pair depends on the routing (heavy routing
// prefers the prefill pair, light routing the token-sharing one).
struct Plan {
    int tm;        // tile height of the first list
    int tm2;       // tile height of the second list (0: none)
    int g1, g2;
    bool convert;  // fp16 C converted to the hi/lo form between the GEMMs
    bool by_row;   // GEMM1 reads the token scales gathered into row order
    bool dispatch_in_gemm1;   // GEMM1 variant 5 computes the dispatch itself (no launch)
};

int g1_tile_m(int v) { return v == 1 || v == 5 ? 16 : v == 2 ? 32 : v == 7 || v == 8 ? 64 : 256; }
bool g1_hilo(int v) { return v == 4; }        // GEMM1 writes the hi/lo form
bool g2_hilo(int v) { return v == 5; }        // GEMM2 reads the hi/lo form

// The plan of a GEMM1 / GEMM2 pair, false when they cannot run together.  GEMM1
// variant 5 is variant 1 with the dispatch folded in (T <= 64): every workgroup of a
// persistent grid computes the call's dispatch from the routing ids, and the separate
// dispatch launch goes away.
bool make_plan(int g1, int g2, int32_t T, Plan* p) {
    if (g1 == 5) {
        if (g2 != 1 || T > moe::kDispatchInGemm1MaxT) return false;
        *p = {16, 0, 5, g2, false, false, true};
        return true;
    }
    if ((g1 != 1 && g1 != 2 && g1 != 4 && g1 != 7 && g1 != 8) || (g2 != 1 && g2 != 3 && g2 != 5)) return false;
    const int tm = g1_tile_m(g1);
    if (g1_hilo(g1) && !g2_hilo(g2)) return false;      // the fp16 GEMM2s need fp16 C
    if (g2 == 5) {                                       // the second list, 128-row tiles
        *p = {tm, 128, g1, g2, !g1_hilo(g1), false, false};
        return true;
    }
    const int tm_g2 = g2 == 1 ? 16 : 32;
    if (tm_g2 != tm) return false;
    *p = {tm, 0, g1, g2, g1_hilo(g1) != g2_hilo(g2), false, false};
    return true;
}

// GEMM1 reads the token scales gathered into row order (see gather_row_scales_kernel)
// from T = kRowScalesMinT on; below, the gather costs more than it saves.  The
// token-sharing GEMM1 (variant 7) moves a tile's 64 scales per K block with one gathering
// DMA instruction either way, so it reads them by token and the gather launch goes away
// (-1 us at T = 600 .. 1280).
constexpr int32_t kRowScalesMinT = 512;

// The prefill GEMM1 takes its items ranked by expert rows (prefill_items_ranked) up to
// T = kRankedMaxT and in tile-list order beyond.  Measured on three routings each at
// T = 1400 .. 3500 the ranked order was 4-24 us faster on 17 of 21 (GEMM1 ~180-270 us)
// and at most 6 us slower; at T = 4096 (skewed), 5000 and 8192 it was 4-19 us slower.
constexpr int32_t kRankedMaxT = 3500;
constexpr int32_t kKnownFlags = MOE_MI355_FLAG_PROFILE | MOE_MI355_FLAG_FORCE_PLAN |
                                MOE_MI355_FLAG_ROW_SCALES_ON | MOE_MI355_FLAG_ROW_SCALES_OFF |
                                MOE_MI355_FLAG_LIST_ORDER | (0xff << 8);

// The plan of a call over T tokens: chosen from T alone, unless the caller's flags force
// a GEMM pair or the token-scale form (tuning sweeps and the tests of every variant).
// Nothing outside the call's arguments (no environment) changes it.
int plan_for(int32_t T, int32_t flags, Plan* p) {
    if (flags & ~kKnownFlags) return MOE_ERR_BAD_FLAGS;
    const bool on = flags & MOE_MI355_FLAG_ROW_SCALES_ON, off = flags & MOE_MI355_FLAG_ROW_SCALES_OFF;
    int g1, g2;
    // GEMM1 with the dispatch folded in reads the token scales by token: asking for the
    // gathered ones selects the separate dispatch there
    if (T <= moe::kDispatchInGemm1MaxT && !on) g1 = 5, g2 = 1;
    else if (T <= 88) g1 = 1, g2 = 1;
    else if (T <= 299) g1 = 2, g2 = 3;
    else if (T <= 960) g1 = 8, g2 = 5;
    else if (T <= 1344) g1 = 7, g2 = 5;
    else g1 = 4, g2 = 5;
    if (flags & MOE_MI355_FLAG_FORCE_PLAN) {
        g1 = MOE_MI355_FLAGS_G1(flags);
        g2 = MOE_MI355_FLAGS_G2(flags);
    } else if (flags & (0xff << 8)) {
        return MOE_ERR_BAD_FLAGS;            // variant bits without the force bit
    }
    if (!make_plan(g1, g2, T, p)) return MOE_ERR_BAD_FLAGS;
    if (on && (off || p->dispatch_in_gemm1)) return MOE_ERR_BAD_FLAGS;
    p->by_row = on ? true : off ? false : (T >= kRowScalesMinT && p->g1 != 7 && p->g1 != 8);
    return MOE_OK;
}

thread_local char g_hip_error[256] = "";

constexpr size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

// Byte offsets of the workspace regions of a call over T tokens (all 256-aligned).
// constexpr, so that the library's own scratch array (moe_mi355_forward_noalloc) is
// sized by the same arithmetic as a caller's workspace.
constexpr moe_mi355_workspace_layout workspace_regions(int32_t T) {
    moe_mi355_workspace_layout L{};
    const size_t R = (size_t)T * moe::kTopK;
    const int mt = (int)((R + kMinTileM - 1) / kMinTileM) + moe::kEL;   // dispatch_max_tiles
    size_t off = 0;
    auto take = [&off](size_t bytes) {
        const size_t o = off;
        off = align_up(off + bytes);
        return o;
    };
    L.topk_ids = take(R * 4);
    L.topk_weights = take(R * 4);
    L.inverse_rows = take(R * 4);
    L.meta = take(64 * 4);
    L.tiles = take((size_t)mt * 2 * 16);   // room for a second, half-height tile list
    L.sorted_tokens = take(R * 4);
    L.sorted_weights = take(R * 4);
    L.chunk_counts = take((size_t)((T + 255) / 256) * moe::kEL * 4);
    L.row_scales = take(R * moe::kHB * 4);        // token scales in row order, [56, 8T]
    // hi/lo, fp16 and the fp16 form's group exponents
    L.intermediate = take(R * (moe::kI * 4 + moe::kI / moe::kGroup16));
    L.intermediate_scales = take(R * moe::kIB * 4);
    L.expert_out = take(R * moe::kH * 2);
    L.expert_out_exp = take(R * (moe::kH / moe::kGroup16));
    L.total = off;
    L.max_tiles = mt;
    return L;
}

// Workspace layout of a call over T tokens with the given flags (the regions do not
// depend on the flags; tile_m and intermediate_format report the plan they choose).
int fill_layout(int32_t T, int32_t flags, moe_mi355_workspace_layout* L) {
    if (T < 0 || T > kMaxT) return MOE_ERR_BAD_SIZE;
    Plan plan;
    const int st = plan_for(T, flags, &plan);
    if (st != MOE_OK) return st;
    *L = workspace_regions(T);
    L->tile_m = plan.tm;
    L->intermediate_format = g1_hilo(plan.g1) ? 1 : plan.convert ? 2 : 0;
    L->dispatch_in_gemm1 = plan.dispatch_in_gemm1 ? 1 : 0;
    return MOE_OK;
}

int hip_status(hipError_t e) {
    if (e == hipSuccess) return MOE_OK;
    snprintf(g_hip_error, sizeof g_hip_error, "%s (%d)", hipGetErrorString(e), (int)e);
    return MOE_ERR_HIP;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int clamp_offset(int64_t off) {
    if (off > (int64_t)(1 << 30)) return 1 << 30;
    if (off < -(int64_t)(1 << 30)) return -(1 << 30);
    return (int)off;
}

// ---- stage profiler ------------------------------------------------------------
struct Profiler {
    hipEvent_t* ev = nullptr;   // [slots][kNumStages + 1]
    int slots = 0;
    int used = 0;
};
Profiler g_prof;

void prof_record(int slot, int stage, hipStream_t s) {
    (void)hipEventRecord(g_prof.ev[slot * (MOE_MI355_NUM_STAGES + 1) + stage], s);
}

// ---- the library's own workspace (moe_mi355_forward_noalloc) ---------------------
// A workspace for calls of up to MOE_MI355_NOALLOC_MAX_TOKENS tokens in a file-scope
// device array: the code object's loader places one copy on every GPU the library
// runs on, held until the process ends, so a call needs no allocation.  In host code
// `scratch` names a host-side stand-in, never the device memory: its device address
// on the current GPU comes from hipGetSymbolAddress, once per device (kept in
// g_scratch_dev), and only that address reaches the kernels.  Every call on one GPU
// shares the array: nothing in it needs to start at zero (the route kernel clears the
// flag words, dispatch writes every offset, count and row the later kernels read),
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
    const int lst = fill_layout(T, a.flags, &L);
    if (lst != MOE_OK) return lst;
    if (T == 0) return MOE_OK;
    if (!a.routing_logits || !a.routing_bias || !a.hidden_states || !a.hidden_states_scale ||
        !a.gemm1_weights || !a.gemm1_weights_scale || !a.gemm2_weights ||
        !a.gemm2_weights_scale || !a.output)
        return MOE_ERR_NULL_POINTER;
    if (!aligned16(a.routing_logits) || ((uintptr_t)a.routing_bias & 7u) ||
        !aligned16(a.hidden_states) || ((uintptr_t)a.hidden_states_scale & 3u) ||
        !aligned16(a.gemm1_weights) || ((uintptr_t)a.gemm1_weights_scale & 3u) ||
        !aligned16(a.gemm2_weights) || ((uintptr_t)a.gemm2_weights_scale & 3u) ||
        !aligned16(a.output))
        return MOE_ERR_MISALIGNED;
    if (!workspace || ((uintptr_t)workspace & 255u) || ws_bytes < L.total)
        return MOE_ERR_WORKSPACE;
    Plan plan;
    if (plan_for(T, a.flags, &plan) != MOE_OK) return MOE_ERR_BAD_FLAGS;

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
    const bool prof = (a.flags & MOE_MI355_FLAG_PROFILE) && g_prof.ev && g_prof.used < g_prof.slots;
    const bool ranked = !(a.flags & MOE_MI355_FLAG_LIST_ORDER) && T <= kRankedMaxT;
    const int slot = prof ? g_prof.used++ : 0;

    if (prof) prof_record(slot, 0, s);
    moe::launch_route(a.routing_logits, a.routing_bias, T, (float)a.routed_scaling_factor, ids,
                      wts, meta + moe::kCWideFlag, s);
    if (prof) prof_record(slot, 1, s);
    const int max_tiles = moe::dispatch_max_tiles(T, plan.tm);
    const bool half = plan.tm2 > 0;   // GEMM2 walks the second (128-row) tile list
    int4* tiles2 = tiles + max_tiles;
    int* num_tiles2 = meta + moe::kEL + 2;
    // GEMM1 variant 5 computes the dispatch itself (timed as the GEMM1 stage)
    bool ok = plan.dispatch_in_gemm1 ||
              moe::launch_dispatch(ids, wts, T, clamp_offset(a.local_expert_offset), plan.tm,
                                   plan.tm2, meta, num_tiles, tiles, stok, sw, inv, chunk_cnt, s,
                                   half ? num_tiles2 : nullptr, half ? tiles2 : nullptr);
    // GEMM1 reads the token scales gathered into row order (counted in the dispatch stage)
    // or, where the gather would cost more than it saves, straight by token
    if (ok && plan.by_row)
        moe::launch_gather_row_scales(a.hidden_states_scale, T, stok, meta, row_scales,
                                      T * moe::kTopK, s);
    const moe::TokenScales sa = plan.by_row ? moe::TokenScales{row_scales, T * moe::kTopK, 1}
                                            : moe::TokenScales{a.hidden_states_scale, T, 0};
    if (prof) prof_record(slot, 2, s);
    if (plan.dispatch_in_gemm1)
        ok = ok && moe::launch_gemm1_dispatch(ids, wts, T, clamp_offset(a.local_expert_offset),
                                              a.hidden_states, a.hidden_states_scale,
                                              a.gemm1_weights, a.gemm1_weights_scale, meta, tiles,
                                              stok, sw, inv, inter, s);
    else
        ok = ok && moe::launch_gemm1(plan.g1, a.hidden_states, sa, T, a.gemm1_weights,
                                     a.gemm1_weights_scale, tiles, num_tiles, meta, max_tiles,
                                     stok, inter, ranked, s);
    if (prof) prof_record(slot, 3, s);
    if (ok && plan.convert) moe::launch_c_f16_to_hilo(inter, meta, s);   // in the GEMM2 stage
    if (ok && half)
        ok = moe::launch_gemm2(plan.g2, inter, a.gemm2_weights, a.gemm2_weights_scale, tiles2,
                               num_tiles2, meta, moe::dispatch_max_tiles(T, plan.tm2), rows, s);
    else if (ok)
        ok = moe::launch_gemm2(plan.g2, inter, a.gemm2_weights, a.gemm2_weights_scale, tiles,
                               num_tiles, meta, max_tiles, rows, s);
    if (prof) prof_record(slot, 4, s);
    if (ok) moe::launch_combine(rows, meta + moe::kRowsWideFlag, sw, inv, T, a.output, s);
    if (prof) prof_record(slot, 5, s);
    const int hst = hip_status(hipGetLastError());
    if (hst != MOE_OK) return hst;
    return ok ? MOE_OK : MOE_ERR_BAD_PLAN;
}

}  // namespace

extern "C" {

const char* moe_mi355_version(void) { return "moe_mi355 0.1 gfx950"; }

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
                      topk_weights, nullptr, s);
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
    const int n = max_calls * (MOE_MI355_NUM_STAGES + 1);
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
    g_prof.slots = max_calls;
    g_prof.used = 0;
    return MOE_OK;
}

int moe_mi355_profile_read(float* stage_ms, int32_t n) {
    if (!stage_ms) return MOE_ERR_NULL_POINTER;
    if (!g_prof.ev || g_prof.used == 0) return 0;
    const int ns = MOE_MI355_NUM_STAGES;
    double sum[MOE_MI355_NUM_STAGES] = {0};
    for (int c = 0; c < g_prof.used; ++c) {
        hipEvent_t* ev = g_prof.ev + c * (ns + 1);
        const hipError_t e = hipEventSynchronize(ev[ns]);
        if (e != hipSuccess) return hip_status(e);
        for (int st = 0; st < ns; ++st) {
            float ms = 0.f;
            const hipError_t e2 = hipEventElapsedTime(&ms, ev[st], ev[st + 1]);
            if (e2 != hipSuccess) return hip_status(e2);
            sum[st] += ms;
        }
    }
    for (int st = 0; st < ns && st < n; ++st) stage_ms[st] = (float)(sum[st] / g_prof.used);
    return g_prof.used;
}

int moe_mi355_profile_end(void) {
    if (g_prof.ev) {
        for (int i = 0; i < g_prof.slots * (MOE_MI355_NUM_STAGES + 1); ++i)
            (void)hipEventDestroy(g_prof.ev[i]);
        delete[] g_prof.ev;
    }
    g_prof.ev = nullptr;
    g_prof.slots = 0;
    g_prof.used = 0;
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
