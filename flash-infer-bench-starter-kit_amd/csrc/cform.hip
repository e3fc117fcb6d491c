// cform.hip -- the fp16 SwiGLU rows of the streaming GEMM1 kernels converted to the
// fp8 hi/lo form of the prefill GEMM2 kernel, for the plans that pair the two (the
// streaming GEMM1 is the faster GEMM1 up to T ~ 1300, the prefill GEMM2 the faster
// GEMM2 from T ~ 800; moe_device.h, Intermediate, has both forms).
//
// Per row and 128-column block, the arithmetic of the prefill GEMM1 epilogue
// (gemm1.hip, store_c_hilo): s = amax/448 (1 for an all-zero block),
// hi = e4m3(clamp(c * 448/amax)), lo = e4m3(clamp((c - hi*s) * 16*448/amax)) with
// c - hi*s one fma.  On a call where GEMM1 flagged a value beyond the fp16 range, c is
// the fp16 value times its group exponent (moe_device.h).

#include "moe_device.h"

namespace moe {

// One row per workgroup pass; wave w converts columns 512 w .. 512 w + 511, lane l eight
// of them, and the 16 lanes of each 128-column block share its absmax by xor shuffles.
__global__ __launch_bounds__(256) void c_f16_to_hilo_kernel(Intermediate C, const int* __restrict__ meta) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int col = wave * 512 + lane * 8;
    const int block = col >> 7;
    // the first row's values are read before the row count, so that the two loads are in
    // flight together (blockIdx.x < the grid <= the row capacity of C; a workgroup past
    // the count does not use them); each later row's values are read ahead of the
    // conversion of the row before
    uint4 hv = *reinterpret_cast<const uint4*>(C.f16() + (size_t)blockIdx.x * kI + col);
    const int na = meta[kEL];                 // rows of this call
    const bool wide = meta[kCWideFlag] != 0;
    for (int row = blockIdx.x; row < na; row += gridDim.x) {
        const size_t off = (size_t)row * kI + col;
        const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
        if (row + (int)gridDim.x < na)
            hv = *reinterpret_cast<const uint4*>(C.f16() + off + (size_t)gridDim.x * kI);
        // the group exponent applies only on a call whose flag is raised
        const int e = wide ? C.f16_exp()[(size_t)row * (kI / kGroup16) + col / kGroup16] : 0;
        float x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = f16_scaled_to_f32((hw[j >> 1] >> (16 * (j & 1))) & 0xffffu, e);
        float m = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) m = fmaxf(m, fabsf(x[j]));
#pragma unroll
        for (int sh = 1; sh < 16; sh <<= 1) m = fmaxf(m, __shfl_xor(m, sh));
        const float sc = m > 0.f ? m / 448.f : 1.f;
        const float inv = m > 0.f ? 448.f / m : 1.f;
        const float inv16 = inv * 16.f;
        uint32_t hq[2], lq[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const float* v = x + 4 * q;
            const uint32_t h = e4m3x4_from_f32(clamp448(v[0] * inv), clamp448(v[1] * inv),
                                               clamp448(v[2] * inv), clamp448(v[3] * inv));
            const auto h01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h, false);
            const auto h23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h, true);
            const float hd[4] = {h01[0], h01[1], h23[0], h23[1]};
            float l[4];
#pragma unroll
            for (int v4 = 0; v4 < 4; ++v4) l[v4] = clamp448(__builtin_fmaf(-hd[v4], sc, v[v4]) * inv16);
            hq[q] = h;
            lq[q] = e4m3x4_from_f32(l[0], l[1], l[2], l[3]);
        }
        *reinterpret_cast<uint2*>(C.hi() + off) = make_uint2(hq[0], hq[1]);
        *reinterpret_cast<uint2*>(C.lo() + off) = make_uint2(lq[0], lq[1]);
        if ((lane & 15) == 0) C.scales[(size_t)block * C.rows_cap + row] = sc;
    }
}

// meta: the forward's meta words (row count at [32], the fp16-range flag).
void launch_c_f16_to_hilo(const Intermediate& C, const int* meta, hipStream_t stream) {
    const int grid = C.rows_cap < 2048 ? C.rows_cap : 2048;
    if (grid <= 0) return;
    launch_kernel(c_f16_to_hilo_kernel, dim3(grid), dim3(256), 0, stream, C, meta);
}

}  // namespace moe
