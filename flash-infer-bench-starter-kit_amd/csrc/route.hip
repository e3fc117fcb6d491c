// route.hip -- DeepSeek-V3 no-aux routing, one wave64 per token.
//
// Semantics: reference solution/cuda/moe.cu:178-206 (sigmoid, +bias, group top-2
// sums, top-4 groups, top-8 experts, renormalised unbiased weights * factor) with
// the tie rule of solution/python/kernel.cu:84-178 (ties go to the lower index) and
// the selection-order weight sum of kernel.cu:181-185.
//
// Layout on the wave: lane l owns experts 4l..4l+3, so group g = l/8 lives on
// lanes 8g..8g+7.  Scores travel as 64-bit keys (orderable fp32 bits << 32 |
// 256 - expert) so one max-reduction picks the highest score and, among equal
// scores, the lowest expert.
//
// The sigmoid is evaluated in binary64 with an exp built from IEEE operations only
// (Cody-Waite reduction, degree-13 Taylor polynomial, explicit fma) and rounded
// once to fp32, which makes every score reproducible bit for bit on any IEEE host.

#include "moe_device.h"

namespace moe {

#pragma clang fp contract(off)

__device__ __forceinline__ double canon_exp64(double t) {
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

__device__ __forceinline__ float canon_sigmoid(float x) {
    const double t = -(double)x;
    if (t != t) return x;
    if (t > 700.0) return 0.0f;
    if (t < -700.0) return 1.0f;
    const double e = canon_exp64(t);
    return (float)(1.0 / (1.0 + e));
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    const int lo = __shfl_xor((int)(uint32_t)v, m);
    const int hi = __shfl_xor((int)(uint32_t)(v >> 32), m);
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

// max over the 8 lanes of an aligned lane octet (one expert group)
__device__ __forceinline__ uint64_t octet_max(uint64_t v) {
    v = max_u64(v, shfl_xor_u64(v, 1));
    v = max_u64(v, shfl_xor_u64(v, 2));
    v = max_u64(v, shfl_xor_u64(v, 4));
    return v;
}

__device__ __forceinline__ uint64_t wave_max(uint64_t v) {
    v = octet_max(v);
    v = max_u64(v, shfl_xor_u64(v, 8));
    v = max_u64(v, shfl_xor_u64(v, 16));
    v = max_u64(v, shfl_xor_u64(v, 32));
    return v;
}

__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits,
                                                    const uint16_t* __restrict__ bias,
                                                    int T, float factor,
                                                    int* __restrict__ topk_ids,
                                                    float* __restrict__ topk_w) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T) return;  // uniform per wave

    const float4 lg = reinterpret_cast<const float4*>(logits + (size_t)t * kEG)[lane];
    const uint2 bb = reinterpret_cast<const uint2*>(bias)[lane];
    const float lgv[4] = {lg.x, lg.y, lg.z, lg.w};
    const float bv[4] = {bf16_bits_to_f32(bb.x & 0xffffu), bf16_bits_to_f32(bb.x >> 16),
                         bf16_bits_to_f32(bb.y & 0xffffu), bf16_bits_to_f32(bb.y >> 16)};
    float s[4];
    uint64_t key[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        s[j] = canon_sigmoid(lgv[j]);
        const float sb = s[j] + bv[j];
        key[j] = ((uint64_t)order_bits(sb) << 32) | (uint32_t)(256 - (4 * lane + j));
    }

    // group score: best + second best of the group (moe.cu:186-188)
    uint64_t m = max_u64(max_u64(key[0], key[1]), max_u64(key[2], key[3]));
    const uint64_t m1 = octet_max(m);
    uint64_t m2l = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (key[j] != m1) m2l = max_u64(m2l, key[j]);
    const uint64_t m2 = octet_max(m2l);
    const float gscore = order_bits_inv((uint32_t)(m1 >> 32)) + order_bits_inv((uint32_t)(m2 >> 32));

    // keep the 4 best groups, ties to the lower group (kernel.cu:96-115)
    uint32_t gk[kNGroup];
#pragma unroll
    for (int g = 0; g < kNGroup; ++g) gk[g] = order_bits(__shfl(gscore, 8 * g));
    uint32_t keep = 0;
#pragma unroll
    for (int j = 0; j < kTopKGroup; ++j) {
        int best = -1;
        uint32_t bk = 0;
#pragma unroll
        for (int g = 0; g < kNGroup; ++g) {
            const bool free_g = ((keep >> g) & 1u) == 0u;
            if (free_g && (best < 0 || gk[g] > bk)) { best = g; bk = gk[g]; }
        }
        keep |= 1u << best;
    }

    // top-8 over kept groups (moe.cu:198-200); pruned experts keep only the index
    // part so they rank below every kept expert; 0 marks a taken expert.
    const bool kept = ((keep >> (lane >> 3)) & 1u) != 0u;
    uint64_t ck[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) ck[j] = kept ? key[j] : (uint64_t)(uint32_t)(256 - (4 * lane + j));

    int my_id = 0;
    float my_s = 0.0f;
    float ssel[kTopK];
#pragma unroll
    for (int j = 0; j < kTopK; ++j) {
        const uint64_t lm = max_u64(max_u64(ck[0], ck[1]), max_u64(ck[2], ck[3]));
        const uint64_t wm = wave_max(lm);
        const int e = 256 - (int)(uint32_t)(wm & 0x1ffu);
        const int owner = e >> 2, sub = e & 3;
        float spick = s[0];
#pragma unroll
        for (int q = 1; q < 4; ++q) spick = (sub == q) ? s[q] : spick;
        const float se = __shfl(spick, owner);
        if (lane == owner) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (q == sub) ck[q] = 0;
        }
        ssel[j] = se;
        if (lane == j) { my_id = e; my_s = se; }
    }

    // w = s / (sum + 1e-20) * factor, summed in selection order
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < kTopK; ++j) sum = sum + ssel[j];
    const float denom = sum + 1e-20f;
    if (lane < kTopK) {
        const float q = my_s / denom;
        topk_ids[(size_t)t * kTopK + lane] = my_id;
        topk_w[(size_t)t * kTopK + lane] = q * factor;
    }
}

void launch_route(const float* logits, const uint16_t* bias, int T, float factor,
                  int* topk_ids, float* topk_w, hipStream_t stream) {
    if (T <= 0) return;
    hipLaunchKernelGGL(route_kernel, dim3((T + 3) / 4), dim3(256), 0, stream, logits, bias,
                       T, factor, topk_ids, topk_w);
}

}  // namespace moe
