// moe_shape.h -- geometry and workspace-word constants shared by host and device code
// (plain C++, no HIP types, so the host logic can also be built with g++ alone).
#pragma once

namespace moe {

// Geometry (reference solution/python/kernel.h:9-25).
constexpr int kH = 7168;           // hidden
constexpr int kI = 2048;           // intermediate
constexpr int kN1 = 2 * kI;        // GEMM1 output width (gate rows | up rows)
constexpr int kEG = 256;           // global experts
constexpr int kEL = 32;            // local experts
constexpr int kTopK = 8;
constexpr int kNGroup = 8;
constexpr int kGroupSize = 32;
constexpr int kTopKGroup = 4;
constexpr int kBlk = 128;          // quantisation block edge
constexpr int kHB = kH / kBlk;     // 56 hidden blocks
constexpr int kIB = kI / kBlk;     // 16 intermediate blocks
constexpr int kN1B = kN1 / kBlk;   // 32 GEMM1 output blocks

// Words of the workspace's meta region after the 33 expert offsets [0 .. kEL]: the tile
// count of the first list, of the second list, then two per-call flag words (cleared by
// the route kernel): C of GEMM1 exceeds the fp16 range, an expert row of GEMM2 does.
// Where no route kernel runs (GEMM1 variant 9 routes its tokens itself), nothing clears
// the first word: that GEMM1 sets it as the others do, and its GEMM2 (variant 6) takes
// a zero word as C within the fp16 range and checks a nonzero one against C's group
// exponents, which GEMM1 writes for every row on every call (a stale word only costs
// the check; the GEMM2 clears a word the check finds stale).
constexpr int kCWideFlag = kEL + 3;
constexpr int kRowsWideFlag = kEL + 4;
constexpr int kGroup16 = 16;       // columns per fp16-form exponent byte

// Largest T whose dispatch runs inside the GEMM1 launch (GEMM1 variant 5): the kernel
// keeps that call's permutation and tile list in LDS, sized by this bound.
constexpr int kDispatchInGemm1MaxT = 64;

// Largest T whose routing also runs inside the GEMM1 launch (GEMM1 variant 9): every
// workgroup routes the call's tokens, one per wave, before its items (T <= 4: the 4 waves
// of the usual workgroup; 5 <= T <= 8: workgroups of 8 waves, one per CU, working as two
// groups of four after routing).  A wave's routing is a dependent chain of ~600
// instructions; two tokens on one wave delayed the first weight load by more than the
// route launch costs, and so did six routing waves on one SIMD.
constexpr int kRouteInGemm1MaxT = 8;

// Token counts whose forward dispatch is one launch over the local-expert masks the route
// kernel writes (dispatch_masks_kernel): every workgroup counts the experts of all T tokens
// from the masks, which replaces the count launch (and, where GEMM1 reads the token scales
// in row order, the gather launch).  Up to kMaskDispatchMaxT a workgroup's count reads at
// most 64 masks per thread; beyond, the count and place launches run.  Below
// kMaskDispatchMinT the one-workgroup dispatch is as fast or faster (measured: T = 300
// +0.4 us, 350 even, 400 -0.5, 600 -1.3 us for the masks).
constexpr int kMaskDispatchMinT = 400;
constexpr int kMaskDispatchMaxT = 16384;

// Largest T whose GEMM2 runs with the combine folded in (GEMM2 variant 6): the kernel
// keeps every expert row of the call (8 T rows) for its 32 output columns in LDS.
constexpr int kFusedCombineMaxT = 32;

// Upper bound on the row tiles of tm rows a call over T tokens can have: every local
// expert's last tile may be partial.
constexpr int dispatch_max_tiles(int T, int tm) {
    return (int)(((long long)T * kTopK + tm - 1) / tm) + kEL;
}

}  // namespace moe
