// gemm2.hip -- grouped GEMM2 (2048 -> 7168) on bf16 MFMA.
//
// Semantics: reference solution/cuda/moe.cu:231 (O = C @ W2[e]^T) with the 128x128
// block scales of gemm2_weights_scale applied per K block in the fp32 accumulator
// (the reference's CUTLASS path applies them in its mainloop,
// moe_grouped_gemm_fp8.cu:274-322):
//   O[r, h] = sum_kb sb2[e, h/128, kb] * sum_{i in kb} C[r, i] * W2[e, h, i]
// C is the bf16 SwiGLU output of GEMM1; W2 e4m3 bytes are widened to bf16 in
// registers (exact: every e4m3 value is a bf16 value).  The reference re-quantises
// C to fp8 per (row, 128) (kernel.cu:1086-1145); keeping C in bf16 keeps GEMM2 within
// atol = rtol = 1e-2 of the fp32 restatement.
//
// Work item = (row tile of <= 16*MAXCB rows of one expert, 16 output columns h).
// The 4 waves split the 16 K blocks and reduce through LDS in a fixed order.
// MFMA v_mfma_f32_16x16x32_bf16: operand A = 16 W2 rows, operand B = 16 C rows;
// lane l supplies row l%16 and K elements 32*(l/16) + 8j..8j+7 of the block for MFMA
// j = 0..3 on both operands, and receives D[h = 4*(l/16)+v][row = l%16].

#include "moe_device.h"

namespace moe {

__device__ __forceinline__ uint32_t pack_bf16_pair_from_f32(float lo, float hi) {
    // exact: the inputs are widened e4m3 values, whose low 16 fp32 bits are zero
    return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
}

// 4 e4m3 bytes -> 4 bf16 (2 dwords)
__device__ __forceinline__ void e4m3x4_to_bf16x4(uint32_t w, uint32_t& d0, uint32_t& d1) {
    const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
    const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
    d0 = pack_bf16_pair_from_f32(lo[0], lo[1]);
    d1 = pack_bf16_pair_from_f32(hi[0], hi[1]);
}

__device__ __forceinline__ v8bf as_v8bf(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    v4u t = {a, b, c, d};
    return __builtin_bit_cast(v8bf, t);
}

template <int MAXCB>
__global__ __launch_bounds__(256) void gemm2_kernel(
    const uint16_t* __restrict__ inter, const uint8_t* __restrict__ w2,
    const float* __restrict__ s2, const int4* __restrict__ tiles,
    const int* __restrict__ num_tiles, float* __restrict__ out_rows) {
    constexpr int kGroups = kH / 16;      // 448
    constexpr int kKbPerWave = kIB / 4;   // 4
    __shared__ v4f red[4][MAXCB][64];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    const int nwork = (*num_tiles) * kGroups;

    for (int work = blockIdx.x; work < nwork; work += gridDim.x) {
        const int4 tile = tiles[work / kGroups];
        const int hg = work % kGroups;
        const int le = tile.x, row0 = tile.y, nrows = tile.z;
        const int ncb = (nrows + 15) >> 4;

        int crow[MAXCB];
#pragma unroll
        for (int cb = 0; cb < MAXCB; ++cb) crow[cb] = row0 + min(cb * 16 + r16, nrows - 1);

        const uint8_t* wp = w2 + (size_t)(le * kH + hg * 16 + r16) * kI + kq * 32;
        const float* sp = s2 + (size_t)(le * kHB + (hg >> 3)) * kIB;

        v4f acc[MAXCB];
#pragma unroll
        for (int cb = 0; cb < MAXCB; ++cb) acc[cb] = v4f{0.f, 0.f, 0.f, 0.f};
        const v4f zero = {0.f, 0.f, 0.f, 0.f};

#pragma unroll
        for (int kk = 0; kk < kKbPerWave; ++kk) {
            const int kb = wave * kKbPerWave + kk;
            const v4u* wq = reinterpret_cast<const v4u*>(wp + kb * kBlk);
            const v4u wa = __builtin_nontemporal_load(wq);
            const v4u wb = __builtin_nontemporal_load(wq + 1);
            const uint32_t ww[8] = {wa[0], wa[1], wa[2], wa[3], wb[0], wb[1], wb[2], wb[3]};
            v8bf bw[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                uint32_t d0, d1, d2, d3;
                e4m3x4_to_bf16x4(ww[2 * j], d0, d1);
                e4m3x4_to_bf16x4(ww[2 * j + 1], d2, d3);
                bw[j] = as_v8bf(d0, d1, d2, d3);
            }
            const float sb = sp[kb];
#pragma unroll
            for (int cb = 0; cb < MAXCB; ++cb) {
                if (cb < ncb) {
                    const uint4* cp = reinterpret_cast<const uint4*>(
                        inter + (size_t)crow[cb] * kI + kb * kBlk + kq * 32);
                    v4f t = zero;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint4 c4 = cp[j];
                        t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bw[j], as_v8bf(c4.x, c4.y, c4.z, c4.w), t, 0, 0, 0);
                    }
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[cb][v] = __builtin_fmaf(t[v], sb, acc[cb][v]);
                }
            }
        }

#pragma unroll
        for (int cb = 0; cb < MAXCB; ++cb)
            if (cb < ncb) red[wave][cb][lane] = acc[cb];
        __syncthreads();
        for (int cb = wave; cb < ncb; cb += 4) {
            v4f o = red[0][cb][lane];
#pragma unroll
            for (int w = 1; w < 4; ++w) o += red[w][cb][lane];
            const int r = cb * 16 + r16;
            if (r < nrows)
                *reinterpret_cast<v4f*>(out_rows + (size_t)(row0 + r) * kH + hg * 16 + kq * 4) = o;
        }
        __syncthreads();
    }
}

// Debug: widen e4m3 bytes to bf16 with the same conversion GEMM2 uses (n % 4 == 0).
__global__ void e4m3_to_bf16_kernel(const uint32_t* __restrict__ in, uint2* __restrict__ out, int nwords) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nwords) return;
    uint32_t d0, d1;
    e4m3x4_to_bf16x4(in[i], d0, d1);
    out[i] = make_uint2(d0, d1);
}

void launch_gemm2(const uint16_t* inter, const uint8_t* w2, const float* s2, const int4* tiles,
                  const int* num_tiles, int max_tiles, float* out_rows, hipStream_t stream) {
    constexpr int kGroups = kH / 16;
    long long work = (long long)max_tiles * kGroups;
    const int grid = (int)(work < 4096 ? work : 4096);
    hipLaunchKernelGGL(gemm2_kernel<4>, dim3(grid), dim3(256), 0, stream, inter, w2, s2, tiles,
                       num_tiles, out_rows);
}

void launch_e4m3_to_bf16(const uint8_t* in, uint16_t* out, int n, hipStream_t stream) {
    const int nwords = n / 4;
    if (nwords <= 0) return;
    hipLaunchKernelGGL(e4m3_to_bf16_kernel, dim3((nwords + 255) / 256), dim3(256), 0, stream,
                       reinterpret_cast<const uint32_t*>(in), reinterpret_cast<uint2*>(out), nwords);
}

}  // namespace moe
