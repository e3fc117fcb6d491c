// gemm1.hip -- grouped FP8 GEMM1 (7168 -> 2 x 2048) with the SwiGLU epilogue fused.
//
// Semantics: reference solution/cuda/moe.cu:222-229 on block-scaled inputs
// (moe_grouped_gemm_fp8.cu:194-264 applies the same scales inside the CUTLASS
// mainloop):
//   G1[r, n] = sum_kb sa[kb, tok(r)] * sb[e, n/128, kb] * sum_{k in kb} A[tok(r), k] W1[e, n, k]
//   C[r, i]  = silu(G1[r, 2048 + i]) * G1[r, i]        (kernel.cu:1104-1108 convention)
// C is written as bf16 rows (one per routed assignment) for GEMM2.
//
// Work item = (row tile of <= 16*MAXCB rows of one expert, group of 16 gate rows
// n..n+15 paired with the 16 up rows 2048+n..).  The 4 waves of a workgroup split
// the 56 K blocks (14 each) and reduce through LDS in a fixed order, so results do
// not depend on scheduling.
//
// MFMA: v_mfma_f32_16x16x128_f8f6f4 (e4m3 x e4m3), one instruction per 128-wide K
// block, so the per-block scales multiply a fresh fp32 partial before it joins the
// accumulator.  Weight rows feed operand A (16 n rows), gathered token rows feed
// operand B (16 tokens); lane l holds row/token l%16 and K bytes 32*(l/16)..+31 of
// the block for both operands, and receives D[n = 4*(l/16)+v][token = l%16].
// Weight bytes stream from HBM straight into registers (each byte is used by exactly
// one wave); the small token rows are re-read through L1/L2.

#include "moe_device.h"

namespace moe {

__device__ __forceinline__ v8i load_v8i(const uint8_t* p) {
    const uint4* q = reinterpret_cast<const uint4*>(p);
    const uint4 a = q[0];
    const uint4 b = q[1];
    v8i r;
    r[0] = (int)a.x; r[1] = (int)a.y; r[2] = (int)a.z; r[3] = (int)a.w;
    r[4] = (int)b.x; r[5] = (int)b.y; r[6] = (int)b.z; r[7] = (int)b.w;
    return r;
}

__device__ __forceinline__ v8i load_v8i_stream(const uint8_t* p) {
    const v4f* q = reinterpret_cast<const v4f*>(p);
    const v4f a = __builtin_nontemporal_load(q);
    const v4f b = __builtin_nontemporal_load(q + 1);
    v8i r;
    r[0] = __float_as_int(a[0]); r[1] = __float_as_int(a[1]);
    r[2] = __float_as_int(a[2]); r[3] = __float_as_int(a[3]);
    r[4] = __float_as_int(b[0]); r[5] = __float_as_int(b[1]);
    r[6] = __float_as_int(b[2]); r[7] = __float_as_int(b[3]);
    return r;
}

__device__ __forceinline__ v4f mfma_fp8(const v8i& a, const v8i& b, const v4f& c) {
    // scale operands 0 -> plain (unscaled) e4m3 x e4m3 MFMA
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }

template <int MAXCB>
__global__ __launch_bounds__(256) void gemm1_swiglu_kernel(
    const uint8_t* __restrict__ hidden, const float* __restrict__ hs_scale, int T,
    const uint8_t* __restrict__ w1, const float* __restrict__ s1,
    const int4* __restrict__ tiles, const int* __restrict__ num_tiles,
    const int* __restrict__ sorted_tok, uint16_t* __restrict__ inter) {
    constexpr int kGroups = kI / 16;         // 128 gate/up row-group pairs
    constexpr int kKbPerWave = kHB / 4;      // 14
    __shared__ v4f red[4][2][MAXCB][64];

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    const int nwork = (*num_tiles) * kGroups;

    for (int work = blockIdx.x; work < nwork; work += gridDim.x) {
        const int4 tile = tiles[work / kGroups];
        const int ng = work % kGroups;
        const int le = tile.x, row0 = tile.y, nrows = tile.z;
        const int ncb = (nrows + 15) >> 4;

        int tok[MAXCB];
#pragma unroll
        for (int cb = 0; cb < MAXCB; ++cb) tok[cb] = sorted_tok[row0 + min(cb * 16 + r16, nrows - 1)];

        const uint8_t* wg = w1 + (size_t)(le * kN1 + ng * 16 + r16) * kH + kq * 32;
        const uint8_t* wu = wg + (size_t)kI * kH;
        const float* sg = s1 + (size_t)(le * kN1B + (ng >> 3)) * kHB;
        const float* su = sg + (size_t)kIB * kHB;

        v4f ag[MAXCB], au[MAXCB];
#pragma unroll
        for (int cb = 0; cb < MAXCB; ++cb) {
            ag[cb] = v4f{0.f, 0.f, 0.f, 0.f};
            au[cb] = v4f{0.f, 0.f, 0.f, 0.f};
        }
        const v4f zero = {0.f, 0.f, 0.f, 0.f};
        const int kb0 = wave * kKbPerWave;
#pragma unroll 2
        for (int kk = 0; kk < kKbPerWave; ++kk) {
            const int kb = kb0 + kk;
            const v8i bwg = load_v8i_stream(wg + kb * kBlk);
            const v8i bwu = load_v8i_stream(wu + kb * kBlk);
            const float sbg = sg[kb];
            const float sbu = su[kb];
#pragma unroll
            for (int cb = 0; cb < MAXCB; ++cb) {
                if (cb < ncb) {
                    const v8i a = load_v8i(hidden + (size_t)tok[cb] * kH + kb * kBlk + kq * 32);
                    const float sa = hs_scale[(size_t)kb * T + tok[cb]];
                    const v4f tg = mfma_fp8(bwg, a, zero);
                    const v4f tu = mfma_fp8(bwu, a, zero);
                    const float fg = sa * sbg, fu = sa * sbu;
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        ag[cb][v] = __builtin_fmaf(tg[v], fg, ag[cb][v]);
                        au[cb][v] = __builtin_fmaf(tu[v], fu, au[cb][v]);
                    }
                }
            }
        }

#pragma unroll
        for (int cb = 0; cb < MAXCB; ++cb) {
            if (cb < ncb) {
                red[wave][0][cb][lane] = ag[cb];
                red[wave][1][cb][lane] = au[cb];
            }
        }
        __syncthreads();
        for (int cb = wave; cb < ncb; cb += 4) {
            v4f g = red[0][0][cb][lane];
            v4f u = red[0][1][cb][lane];
#pragma unroll
            for (int w = 1; w < 4; ++w) {
                g += red[w][0][cb][lane];
                u += red[w][1][cb][lane];
            }
            const int r = cb * 16 + r16;
            if (r < nrows) {
                uint32_t h[4];
#pragma unroll
                for (int v = 0; v < 4; ++v) h[v] = f32_to_bf16_bits(silu_f32(u[v]) * g[v]);
                uint2 pk;
                pk.x = h[0] | (h[1] << 16);
                pk.y = h[2] | (h[3] << 16);
                *reinterpret_cast<uint2*>(inter + (size_t)(row0 + r) * kI + ng * 16 + kq * 4) = pk;
            }
        }
        __syncthreads();
    }
}

void launch_gemm1(const uint8_t* hidden, const float* hs_scale, int T, const uint8_t* w1,
                  const float* s1, const int4* tiles, const int* num_tiles, int max_tiles,
                  const int* sorted_tok, uint16_t* inter, hipStream_t stream) {
    constexpr int kGroups = kI / 16;
    long long work = (long long)max_tiles * kGroups;
    const int grid = (int)(work < 4096 ? work : 4096);
    hipLaunchKernelGGL(gemm1_swiglu_kernel<4>, dim3(grid), dim3(256), 0, stream, hidden,
                       hs_scale, T, w1, s1, tiles, num_tiles, sorted_tok, inter);
}

}  // namespace moe
