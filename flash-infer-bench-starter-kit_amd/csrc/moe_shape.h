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
constexpr int kCWideFlag = kEL + 3;
constexpr int kRowsWideFlag = kEL + 4;
constexpr int kGroup16 = 16;       // columns per fp16-form exponent byte

// Largest T whose dispatch runs inside the GEMM1 launch (GEMM1 variant 5): the kernel
// keeps that call's permutation and tile list in LDS, sized by this bound.
constexpr int kDispatchInGemm1MaxT = 64;

// Largest T whose GEMM2 runs with the combine folded in (GEMM2 variant 6): the kernel
// keeps every expert row of the call (8 T rows) for its 32 output columns in LDS.
constexpr int kFusedCombineMaxT = 32;

// Upper bound on the row tiles of tm rows a call over T tokens can have: every local
// expert's last tile may be partial.
constexpr int dispatch_max_tiles(int T, int tm) {
    return (int)(((long long)T * kTopK + tm - 1) / tm) + kEL;
}

}  // namespace moe
