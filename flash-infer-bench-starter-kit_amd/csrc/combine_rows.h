// combine_rows.h -- the weighted sum of one token's expert rows into 8 bf16 outputs
// (the body of the combine kernel, combine.hip).
#pragma once

#include "moe_device.h"

namespace moe {


__device__ __forceinline__ void cswap(int& a, int& b) {
    const int x = min(a, b), y = max(a, b);
    a = x;
    b = y;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Output columns h0 .. h0 + 7 of one token: inv_t[0..8) are the token's 8 assignment
// rows (negative: not local), sorted_w the routing weight of each row; the rows are
// added in ascending order (ascending local expert) in fp32 and rounded once to bf16
// into dst[0..8).  `wide` (uniform): GEMM2 flagged a value beyond the fp16 range, so
// the rows' group exponents apply (moe_device.h).
__device__ __forceinline__ void combine_token8(const ExpertRows& rows, bool wide, const int* inv_t,
                                               const float* sorted_w, int h0, uint16_t* dst) {
    // o * w, then + in ascending row order, never an fma: the fp32 accumulation of
    // moe.cu:233-239, bit for bit, wherever this is inlined
#pragma clang fp contract(off)
    int r[kTopK];
#pragma unroll
    for (int k = 0; k < kTopK; ++k) {
        const int v = inv_t[k];
        r[k] = v < 0 ? 0x7fffffff : v;
    }
    // 8-input sorting network (19 compare-exchanges)
    cswap(r[0], r[1]); cswap(r[2], r[3]); cswap(r[4], r[5]); cswap(r[6], r[7]);
    cswap(r[0], r[2]); cswap(r[1], r[3]); cswap(r[4], r[6]); cswap(r[5], r[7]);
    cswap(r[1], r[2]); cswap(r[5], r[6]); cswap(r[0], r[4]); cswap(r[3], r[7]);
    cswap(r[1], r[5]); cswap(r[2], r[6]);
    cswap(r[1], r[4]); cswap(r[3], r[6]);
    cswap(r[2], r[4]); cswap(r[3], r[5]);
    cswap(r[3], r[4]);

    // the valid rows are a prefix r[0 .. nr); a kernel body per row count issues every
    // row load of the token before the first add, then adds in ascending row order
    int nr = 0;
#pragma unroll
    for (int k = 0; k < kTopK; ++k) nr += (r[k] != 0x7fffffff) ? 1 : 0;
    auto body = [&](auto nrows_c, auto wide_c) {
        constexpr int N = decltype(nrows_c)::value;
        constexpr bool kWide = decltype(wide_c)::value != 0;
        float acc[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
        uint4 a[N > 0 ? N : 1];
        float w[N > 0 ? N : 1];
#pragma unroll
        for (int k = 0; k < N; ++k) {
            a[k] = *reinterpret_cast<const uint4*>(rows.f16 + (size_t)r[k] * kH + h0);
            w[k] = sorted_w[r[k]];
        }
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const uint32_t hw[4] = {a[k].x, a[k].y, a[k].z, a[k].w};
            float o[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = f16_bits_to_f32((hw[j >> 1] >> (16 * (j & 1))) & 0xffffu);
            if constexpr (kWide) {
                const int e = rows.exp[(size_t)r[k] * (kH / kGroup16) + h0 / kGroup16];
#pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = e ? ldexpf(o[j], e) : o[j];
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float prod = o[j] * w[k];
                acc[j] = acc[j] + prod;
            }
        }
        uint4 pk;
        pk.x = f32_to_bf16_bits(acc[0]) | (f32_to_bf16_bits(acc[1]) << 16);
        pk.y = f32_to_bf16_bits(acc[2]) | (f32_to_bf16_bits(acc[3]) << 16);
        pk.z = f32_to_bf16_bits(acc[4]) | (f32_to_bf16_bits(acc[5]) << 16);
        pk.w = f32_to_bf16_bits(acc[6]) | (f32_to_bf16_bits(acc[7]) << 16);
        *reinterpret_cast<uint4*>(dst) = pk;
    };
    auto rows_of = [&](auto wide_c) {
        switch (nr) {    // uniform per workgroup (one token)
            case 0: body(IntC<0>{}, wide_c); break;
            case 1: body(IntC<1>{}, wide_c); break;
            case 2: body(IntC<2>{}, wide_c); break;
            case 3: body(IntC<3>{}, wide_c); break;
            case 4: body(IntC<4>{}, wide_c); break;
            case 5: body(IntC<5>{}, wide_c); break;
            case 6: body(IntC<6>{}, wide_c); break;
            case 7: body(IntC<7>{}, wide_c); break;
            default: body(IntC<8>{}, wide_c); break;
        }
    };
    if (!wide) rows_of(IntC<0>{});
    else rows_of(IntC<1>{});
}

}  // namespace moe
