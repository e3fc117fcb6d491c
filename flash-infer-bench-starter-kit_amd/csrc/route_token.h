// route_token.h -- DeepSeek-V3 no-aux routing of one token on one wave64, shared by the
// route kernel (route.hip) and the decode GEMM1 that routes its few tokens itself
// (gemm1.hip).
//
// Semantics: reference solution/cuda/moe.cu:178-206 (sigmoid, +bias, group top-2
// sums, top-4 groups, top-8 experts, renormalised unbiased weights * factor) with
// the tie rule of solution/python/kernel.cu:84-178 (ties go to the lower index) and
// the selection-order weight sum of kernel.cu:181-185.
//
// Layout on the wave: lane l owns experts 4l..4l+3, so group g = l/8 lives on
// lanes 8g..8g+7.  Scores travel as order-preserving 32-bit images of fp32;
// reductions and exchanges use DPP (quad permutes, row rotations) and the lane-swap
// instructions v_permlane16_swap / v_permlane32_swap, so every lane holds their results,
// and ties between equal scores are broken toward the lower expert with a ballot.
//
// The sigmoid is evaluated in binary64 with an exp built from IEEE operations only
// (Cody-Waite reduction, degree-13 Taylor polynomial, explicit fma) and rounded
// once to fp32, which makes every score reproducible bit for bit on any IEEE host.
// The floating-point functions switch contraction off in their bodies: every product
// and sum rounds on its own, as the reference's host restatement does.
#pragma once

#include "moe_device.h"

namespace moe {

__device__ __forceinline__ double canon_exp64(double t) {
#pragma clang fp contract(off)
    const double inv_ln2 = 0x1.71547652b82fep+0;
    const double ln2_hi = 0x1.62e42fefa39efp-1;
    const double ln2_lo = 0x1.abc9e3b39803fp-56;
    const double k = rint(t * inv_ln2);
    double r = __builtin_fma(-k, ln2_hi, t);
    r = __builtin_fma(-k, ln2_lo, r);
    double p = 0x1.6124613a86d09p-33;             // 1/13!
    p = __builtin_fma(p, r, 0x1.1eed8eff8d898p-29);  // 1/12!
    p = __builtin_fma(p, r, 0x1.ae64567f544e4p-26);  // 1/11!
    p = __builtin_fma(p, r, 0x1.27e4fb7789f5cp-22);  // 1/10!
    p = __builtin_fma(p, r, 0x1.71de3a556c734p-19);  // 1/9!
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-16);  // 1/8!
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-13);  // 1/7!
    p = __builtin_fma(p, r, 0x1.6c16c16c16c17p-10);  // 1/6!
    p = __builtin_fma(p, r, 0x1.1111111111111p-7);   // 1/5!
    p = __builtin_fma(p, r, 0x1.5555555555555p-5);   // 1/4!
    p = __builtin_fma(p, r, 0x1.5555555555555p-3);   // 1/3!
    p = __builtin_fma(p, r, 0x1.0p-1);               // 1/2!
    p = __builtin_fma(p, r, 0x1.0p+0);               // 1/1!
    p = __builtin_fma(p, r, 0x1.0p+0);               // 1/0!
    return ldexp(p, (int)k);
}

// sigmoid(x) = 1 / (1 + exp(-x)) in binary64, rounded once to fp32; 0 for -x > 700, 1 for
// -x < -700, x for a NaN.  The exp runs on -x clamped to [-700, 700], which gives those
// two results by itself (1 / (1 + exp(700)) ~ 1e-304 rounds to fp32 0, and 1 + exp(-700)
// rounds to 1 in binary64), so only the NaN needs a select: the code has no branches, and
// a lane's four sigmoids interleave instead of running one dependency chain after another
// (-0.4 to -0.7 us per call at T <= 64).
__device__ __forceinline__ float canon_sigmoid(float x) {
#pragma clang fp contract(off)
    const double t = __builtin_fmin(__builtin_fmax(-(double)x, -700.0), 700.0);
    const float r = (float)(1.0 / (1.0 + canon_exp64(t)));
    return (x != x) ? x : r;
}

// max over the whole wave, held in every lane: quad exchanges, rotations by 4 and 8
// inside each row, then the row and half swaps (each lane meets every other lane's
// value; no lane reads past its row)
__device__ __forceinline__ uint32_t wave_max_all(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xb1, 0xf, 0xf, true));   // quad_perm [1,0,3,2]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4e, 0xf, 0xf, true));   // quad_perm [2,3,0,1]
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xf, 0xf, true));  // row_ror:4
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, true));  // row_ror:8
    auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max((uint32_t)p[0], (uint32_t)p[1]);
    p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return max((uint32_t)p[0], (uint32_t)p[1]);
}

// merge (a1 >= a2) with the pair of another lane: the two largest of the four
__device__ __forceinline__ void top2_merge(uint32_t& a1, uint32_t& a2, uint32_t b1, uint32_t b2) {
    const uint32_t hi = max(a1, b1), lo = min(a1, b1);
    a2 = max(lo, max(a2, b2));
    a1 = hi;
}


// Routes one token on the whole wave: lg holds this lane's four logits (experts
// 4 lane .. 4 lane + 3), bb their four bf16 biases.  Lane j < 8 receives the token's
// j-th pick in selection order: expert id and weight s / (sum of the 8 s + 1e-20) *
// factor, the sum taken in selection order.  sel_s / sel_id are 8 LDS slots each,
// written and read by this wave only.
__device__ __forceinline__ void route_token(const float4 lg, const uint2 bb, int lane, float factor,
                                            float* sel_s, int* sel_id, int& my_id, float& my_w) {
#pragma clang fp contract(off)
    const float lgv[4] = {lg.x, lg.y, lg.z, lg.w};
    const float bv[4] = {bf16_bits_to_f32(bb.x & 0xffffu), bf16_bits_to_f32(bb.x >> 16),
                         bf16_bits_to_f32(bb.y & 0xffffu), bf16_bits_to_f32(bb.y >> 16)};
    float s[4];
    uint32_t key[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        s[j] = canon_sigmoid(lgv[j]);
        key[j] = order_bits(s[j] + bv[j]);
    }

    // group score = best + second best s+bias of the group (moe.cu:186-188), on the
    // octet of lanes holding the group; a duplicated maximum counts twice
    uint32_t a1 = max(key[0], key[1]), a2 = min(key[0], key[1]);
    top2_merge(a1, a2, max(key[2], key[3]), min(key[2], key[3]));
    top2_merge(a1, a2, xor1(a1), xor1(a2));
    top2_merge(a1, a2, xor2(a1), xor2(a2));
    top2_merge(a1, a2, xor4(a1), xor4(a2));
    const float gscore = order_bits_inv(a1) + order_bits_inv(a2);

    // keep the 4 best groups, ties to the lower group (kernel.cu:96-115): every lane of
    // the octet of group g holds its score; an xor butterfly over the octets gives each
    // lane all eight (gk[j]: group g ^ j), and the lane ranks its own group against them
    // (a group beats it with a larger score, or an equal one at a lower index).  The kept
    // groups are those ranked 0..3, the set that four picks of the best remaining group,
    // ties to the lower, select.
    const int g = lane >> 3;
    uint32_t gk[kNGroup];
    gk[0] = order_bits(gscore);
    gk[1] = xor8(gk[0]);
    gk[2] = xor16(gk[0], lane);
    gk[3] = xor16(gk[1], lane);
#pragma unroll
    for (int j = 0; j < 4; ++j) gk[4 + j] = xor32(gk[j], lane);
    int rank = 0;
#pragma unroll
    for (int j = 1; j < kNGroup; ++j)
        rank += (gk[j] > gk[0] || (gk[j] == gk[0] && (g ^ j) < g)) ? 1 : 0;
    const bool kept = rank < kTopKGroup;

    // top-8 (moe.cu:198-200): candidate key = orderable score + 1 for kept experts,
    // 1 for pruned ones, 0 once taken.  Per round the wave maximum is found with DPP and
    // lane swaps (held in every lane), the lowest lane holding it with a ballot, and that
    // lane's lowest slot with it; lane l holds experts 4l..4l+3, so this is the lowest
    // expert index.  The owner notes the round in the slot; the picks are gathered in
    // round order through LDS afterwards.
    uint32_t ck[4];
    int round_of[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        ck[j] = kept ? key[j] + 1u : 1u;
        round_of[j] = -1;
    }
#pragma unroll
    for (int j = 0; j < kTopK; ++j) {
        const uint32_t lm = max(max(ck[0], ck[1]), max(ck[2], ck[3]));
        const uint32_t m = wave_max_all(lm);
        const int owner = (int)__builtin_ctzll(__ballot(lm == m));
        int sub = 3;
#pragma unroll
        for (int q = 2; q >= 0; --q) sub = (ck[q] == m) ? q : sub;
        const bool own = lane == owner;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const bool take = own && q == sub;
            ck[q] = take ? 0u : ck[q];
            round_of[q] = take ? j : round_of[q];
        }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        if (round_of[q] >= 0) {
            sel_s[round_of[q]] = s[q];
            sel_id[round_of[q]] = 4 * lane + q;
        }
    }
    __builtin_amdgcn_wave_barrier();   // the wave's LDS writes before its reads (in order)
    float ssel[kTopK];
#pragma unroll
    for (int j = 0; j < kTopK; ++j) ssel[j] = sel_s[j];
    my_id = lane < kTopK ? sel_id[lane] : 0;
    const float my_s = lane < kTopK ? sel_s[lane] : 0.0f;

    // w = s / (sum + 1e-20) * factor, summed in selection order
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < kTopK; ++j) sum = sum + ssel[j];
    const float denom = sum + 1e-20f;
    const float q = my_s / denom;
    my_w = q * factor;
}

}  // namespace moe
