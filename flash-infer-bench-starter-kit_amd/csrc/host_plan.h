// host_plan.h -- the host-side logic of the C ABI that needs no GPU: the kernel plan of a
// call, the workspace layout, and the argument checks of moe_mi355_forward.  Plain C++
// (no HIP types), so that tests can build it with g++ under AddressSanitizer and
// UndefinedBehaviorSanitizer; capi.hip uses exactly these functions.
//
// Replaces the host-side decisions of the reference's run() (solution/python/main.cpp:
// 79-109: TORCH_CHECKs, the small/large path switch at LARGE_SEQ_THRESHOLD) and its
// per-call torch temporaries (main.cpp:87-231), which here are regions of one
// caller-provided workspace.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "moe_mi355.h"
#include "moe_shape.h"

namespace moe {
namespace host {

// Largest T: 8T rows stay inside int32 and T * 7168 (the byte offset of the last token
// row, used as a 32-bit buffer offset by the prefill kernels) below 2^32.
constexpr int32_t kMaxT = 1 << 19;
static_assert(kMaxT == MOE_MI355_MAX_TOKENS, "the header's limit");
constexpr int kMinTileM = 16;           // smallest row tile; sizes the tile list

// Kernel plan per token count: the GEMM1 / GEMM2 variants (ids of launch_gemm1 /
// launch_gemm2) and what they imply: the tile height of the dispatch's first list (the
// GEMM1's), an optional second list of 128-row tiles (GEMM2 variant 5), and whether the
// fp16 C of a streaming GEMM1 is converted to the hi/lo form for a prefill GEMM2.
// Small T streams weights with the register-staged kernels, C in fp16: 16-row tiles up
// to T = 88, 32-row tiles (GEMM1 with two column groups per wave, GEMM2 with two row
// blocks per wave) beyond.  From T = 200 GEMM1 is the token-sharing kernel on 64-row
// tiles (fewer requests per output once an expert has dozens of rows; variant 8, which
// runs three or two workgroups per CU as the call's tile count makes best), feeding up to
// T = 559 the token-sharing GEMM2 on the same tiles (variant 7: fp16 C, no conversion;
// 1-13 us faster than the neighbouring pairs at T = 200 .. 560 over three routings) and
// beyond the prefill GEMM2 (128-row tiles, FP8 MFMA on the hi/lo form); from T = 1345 both
// GEMMs are the MFMA-bound prefill kernels on 256-row tiles (GEMM2 on the 128-row second
// list).  The boundaries come from wall-clock sweeps of the pairs at T = 72 .. 2560 on
// MI355X over routing seeds from light to heavy routing to the local experts.  Between T = 961 and
// 1344 variant 8 was 6-25 us faster than variant 7 (always two per CU) on three routings
// and 4-10 us slower on three; heavier routing there can prefer the prefill pair.
struct Plan {
    int tm;        // tile height of the first list
    int tm2;       // tile height of the second list (0: none)
    int g1, g2;
    bool convert;  // fp16 C converted to the hi/lo form between the GEMMs
    bool by_row;   // GEMM1 reads the token scales gathered into row order
    bool dispatch_in_gemm1;   // GEMM1 variant 5 computes the dispatch itself (no launch)
    bool combine_in_gemm2;    // GEMM2 variant 6 writes the output itself (no combine launch)
    bool route_in_gemm1;      // GEMM1 variant 9 routes the tokens itself (no route launch)
};

inline int g1_tile_m(int v) { return v == 1 || v == 5 || v == 9 ? 16 : v == 2 ? 32 : v == 7 || v == 8 ? 64 : 256; }
inline bool g1_hilo(int v) { return v == 4; }        // GEMM1 writes the hi/lo form
inline bool g2_hilo(int v) { return v == 5; }        // GEMM2 reads the hi/lo form (7: fp16)

// The plan of a GEMM1 / GEMM2 pair, false when they cannot run together.  GEMM1
// variant 5 is variant 1 with the dispatch folded in (T <= 64): every workgroup of a
// persistent grid computes the call's dispatch from the routing ids, and the separate
// dispatch launch goes away.  GEMM1 variant 9 is variant 5 with the routing folded in too
// (T <= kRouteInGemm1MaxT, GEMM2 variant 6 only): every workgroup routes the call's
// tokens from the logits, and the route launch goes away.
inline bool make_plan(int g1, int g2, int32_t T, Plan* p) {
    // GEMM2 variant 6 is variant 1 (16-row tiles, fp16 C) with the combine folded in,
    // for T <= kFusedCombineMaxT
    if (g2 == 6 && (T > kFusedCombineMaxT || (g1 != 1 && g1 != 5 && g1 != 9))) return false;
    if (g1 == 9) {
        if (g2 != 6 || T > kRouteInGemm1MaxT) return false;
        *p = {16, 0, 9, 6, false, false, true, true, true};
        return true;
    }
    if (g1 == 5) {
        if ((g2 != 1 && g2 != 6) || T > kDispatchInGemm1MaxT) return false;
        *p = {16, 0, 5, g2, false, false, true, g2 == 6};
        return true;
    }
    if (g1 == 1 && g2 == 6) {
        *p = {16, 0, 1, 6, false, false, false, true};
        return true;
    }
    if (g2 == 7) {   // the token-sharing GEMM2 over the token-sharing GEMM1's 64-row tiles
        if (g1 != 7 && g1 != 8) return false;
        *p = {64, 0, g1, 7, false, false, false, false};
        return true;
    }
    if ((g1 != 1 && g1 != 2 && g1 != 4 && g1 != 7 && g1 != 8) || (g2 != 1 && g2 != 3 && g2 != 5)) return false;
    const int tm = g1_tile_m(g1);
    if (g1_hilo(g1) && !g2_hilo(g2)) return false;      // the fp16 GEMM2s need fp16 C
    if (g2 == 5) {                                       // the second list, 128-row tiles
        *p = {tm, 128, g1, g2, !g1_hilo(g1), false, false, false};
        return true;
    }
    const int tm_g2 = g2 == 1 ? 16 : 32;
    if (tm_g2 != tm) return false;
    *p = {tm, 0, g1, g2, g1_hilo(g1) != g2_hilo(g2), false, false, false};
    return true;
}

// GEMM1 reads the token scales gathered into row order (see gather_row_scales_kernel)
// from T = kRowScalesMinT on; below, the gather costs more than it saves.  The
// token-sharing GEMM1 (variants 7, 8) moves a tile's 64 scales per K block with one
// gathering DMA instruction either way, so it reads them by token and the gather launch
// goes away (-1 us at T = 600 .. 1280).
constexpr int32_t kRowScalesMinT = 512;

// The prefill GEMM1 takes its items ranked by expert rows (prefill_items_ranked) up to
// T = kRankedMaxT and in tile-list order beyond.  Measured on three routings each at
// T = 1400 .. 3500 the ranked order was 4-24 us faster on 17 of 21 (GEMM1 ~180-270 us)
// and at most 6 us slower; at T = 4096 (skewed), 5000 and 8192 it was 4-19 us slower.
constexpr int32_t kRankedMaxT = 3500;

// GEMM2 computes the combine itself (variant 6, after GEMM1 variant 5) up to T =
// kFusedCombinePlanMaxT, though it can up to kFusedCombineMaxT: measured against GEMM2
// variant 1 and the combine launch (wall time per call, three runs each), it is 0.6-3.2 us
// faster at T = 12 .. 20 and 0.3-0.9 us slower at T = 24 .. 32, where each of its 224
// workgroups walks the more tiles of the call that variant 1 spreads over all CUs.
constexpr int32_t kFusedCombinePlanMaxT = 22;
constexpr int32_t kKnownFlags = MOE_MI355_FLAG_PROFILE | MOE_MI355_FLAG_FORCE_PLAN |
                                MOE_MI355_FLAG_ROW_SCALES_ON | MOE_MI355_FLAG_ROW_SCALES_OFF |
                                MOE_MI355_FLAG_LIST_ORDER | (0xff << 8);

// The plan of a call over T tokens: chosen from T alone, unless the caller's flags force
// a GEMM pair or the token-scale form (tuning sweeps and the tests of every variant).
// Nothing outside the call's arguments (no environment) changes it.
inline int plan_for(int32_t T, int32_t flags, Plan* p) {
    if (flags & ~kKnownFlags) return MOE_ERR_BAD_FLAGS;
    const bool on = flags & MOE_MI355_FLAG_ROW_SCALES_ON, off = flags & MOE_MI355_FLAG_ROW_SCALES_OFF;
    int g1, g2;
    // GEMM1 with the dispatch folded in reads the token scales by token: asking for the
    // gathered ones selects the separate dispatch there
    if (T <= kRouteInGemm1MaxT && !on) g1 = 9, g2 = 6;   // T <= 8
    else if (T <= kFusedCombinePlanMaxT && !on) g1 = 5, g2 = 6;
    else if (T <= kDispatchInGemm1MaxT && !on) g1 = 5, g2 = 1;
    else if (T <= 88) g1 = 1, g2 = 1;
    else if (T <= 199) g1 = 2, g2 = 3;
    else if (T <= 559) g1 = 8, g2 = 7;
    else if (T <= 1344) g1 = 8, g2 = 5;
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

constexpr size_t align_up(size_t x) { return (x + 255) & ~(size_t)255; }

// Byte offsets of the workspace regions of a call over T tokens (all 256-aligned).
// constexpr, so that the library's own scratch array (moe_mi355_forward_noalloc) is
// sized by the same arithmetic as a caller's workspace.
constexpr moe_mi355_workspace_layout workspace_regions(int32_t T) {
    moe_mi355_workspace_layout L{};
    const size_t R = (size_t)T * kTopK;
    const int mt = dispatch_max_tiles(T, kMinTileM);
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
    L.chunk_counts = take((size_t)((T + 255) / 256) * kEL * 4);
    L.token_masks = take((size_t)T * 4);
    L.row_scales = take(R * kHB * 4);        // token scales in row order, [56, 8T]
    // hi/lo, fp16 and the fp16 form's group exponents
    L.intermediate = take(R * (kI * 4 + kI / kGroup16));
    L.intermediate_scales = take(R * kIB * 4);
    L.expert_out = take(R * kH * 2);
    L.expert_out_exp = take(R * (kH / kGroup16));
    L.total = off;
    L.max_tiles = mt;
    return L;
}

// Workspace layout of a call over T tokens with the given flags (the regions do not
// depend on the flags; tile_m and intermediate_format report the plan they choose).
inline int fill_layout(int32_t T, int32_t flags, moe_mi355_workspace_layout* L) {
    if (T < 0 || T > kMaxT) return MOE_ERR_BAD_SIZE;
    Plan plan;
    const int st = plan_for(T, flags, &plan);
    if (st != MOE_OK) return st;
    *L = workspace_regions(T);
    L->tile_m = plan.tm;
    L->intermediate_format = g1_hilo(plan.g1) ? 1 : plan.convert ? 2 : 0;
    L->dispatch_in_gemm1 = plan.dispatch_in_gemm1 ? 1 : 0;
    L->combine_in_gemm2 = plan.combine_in_gemm2 ? 1 : 0;
    return MOE_OK;
}

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// local_expert_offset as the kernels take it: any int64 maps into +-2^30, which keeps
// id - offset from overflowing int32 and selects no local expert when the offset lies
// outside [-256, 256] (global ids are 0 .. 255).
inline int clamp_offset(int64_t off) {
    if (off > (int64_t)(1 << 30)) return 1 << 30;
    if (off < -(int64_t)(1 << 30)) return -(1 << 30);
    return (int)off;
}

// The checks of moe_mi355_forward before anything is launched, in the order the status
// reports them: T and flags (fill_layout), then (T > 0) NULL tensor pointers, their
// alignment, and the workspace.  On MOE_OK, *L holds the call's layout and *plan its plan.
inline int check_forward_args(const moe_mi355_args& a, const void* workspace, size_t ws_bytes,
                              moe_mi355_workspace_layout* L, Plan* plan) {
    const int lst = fill_layout(a.T, a.flags, L);
    if (lst != MOE_OK) return lst;
    if (plan_for(a.T, a.flags, plan) != MOE_OK) return MOE_ERR_BAD_FLAGS;
    if (a.T == 0) return MOE_OK;
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
    if (!workspace || ((uintptr_t)workspace & 255u) || ws_bytes < L->total)
        return MOE_ERR_WORKSPACE;
    return MOE_OK;
}

}  // namespace host
}  // namespace moe
