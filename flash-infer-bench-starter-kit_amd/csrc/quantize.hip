// quantize.hip -- blockwise FP8 quantizer of activations, the step before the MoE
// operator: per row and 128-column block
//   scale = absmax / 448            (1 for an all-zero block)
//   q     = e4m3(clamp(x * (1 / scale), -448, 448)), round to nearest even
// q e4m3 [rows, cols]; scales fp32 [cols / 128, rows] (column-major, the layout of
// hidden_states_scale).  The arithmetic follows the reference's
// quantize_fp8_blockwise_kernel (solution/python/kernel.cu:998-1062, fp32 input there,
// defined but not launched by the operator): absmax ignores NaN (fmaxf), the
// reciprocal is taken once per block and multiplied in, and the clamp runs fmaxf then
// fminf, so a NaN input becomes -448.

#include "moe_device.h"

namespace moe {

constexpr int kQuantMaxCols = 32768;
constexpr int kQuantRows = 8;      // rows (waves) per workgroup

__device__ __forceinline__ void load8(const uint16_t* __restrict__ p, float (&v)[8]) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = bf16_bits_to_f32(w[i] & 0xffffu);
        v[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
    }
}

__device__ __forceinline__ void load8(const float* __restrict__ p, float (&v)[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// One wave per row.  A 128-column block is 16 lanes x 8 elements (one 16-byte bf16
// load or two 16-byte fp32 loads per lane), so a wave covers 4 blocks per pass and
// takes the block absmax with a 4-step xor shuffle inside its 16 lanes.  The 8 waves
// of a workgroup hold 8 consecutive rows; their scales go through LDS so each block's
// 8 scales leave as one contiguous 32-byte run of the column-major scale array.
template <typename In, int NP>
__global__ __launch_bounds__(64 * kQuantRows) void quantize_fp8_blockwise_kernel(
    const In* __restrict__ x, int rows, int cols, uint8_t* __restrict__ q,
    float* __restrict__ scales) {
    __shared__ float sc[kQuantMaxCols / 128][kQuantRows];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    // workgroup b takes row group (b % 8) G/8 + b/8 (when 8 divides the grid): workgroup b
    // runs on XCD b mod 8, so the four row groups whose scales share a 128-byte line of
    // the column-major scale array run on one XCD, whose L2 assembles the whole line
    // (-2% at 8192 rows, -4% at 32768)
    const int G = gridDim.x;
    const int gb = (G % 8 == 0) ? (blockIdx.x % 8) * (G / 8) + blockIdx.x / 8 : blockIdx.x;
    const int row0 = gb * kQuantRows;
    const int row = row0 + wave;
    const int nb = cols >> 7;
    const int g = lane >> 4;
    const int e0 = (lane & 15) * 8;
    // one 128-column block of 16 lanes: absmax, scale, 8 codes, scale to LDS
    auto block = [&](int b, const float (&v)[8], uint8_t* qr) {
        float m = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
        m = fmaxf(m, __shfl_xor(m, 1, 16));
        m = fmaxf(m, __shfl_xor(m, 2, 16));
        m = fmaxf(m, __shfl_xor(m, 4, 16));
        m = fmaxf(m, __shfl_xor(m, 8, 16));
        const float scale = (m > 0.0f) ? (m / 448.0f) : 1.0f;
        const float inv = 1.0f / scale;
        uint2 pk;
        pk.x = e4m3x4_from_f32(clamp448(v[0] * inv), clamp448(v[1] * inv),
                               clamp448(v[2] * inv), clamp448(v[3] * inv));
        pk.y = e4m3x4_from_f32(clamp448(v[4] * inv), clamp448(v[5] * inv),
                               clamp448(v[6] * inv), clamp448(v[7] * inv));
        *reinterpret_cast<uint2*>(qr + b * 128 + e0) = pk;
        if ((lane & 15) == 0) sc[b][wave] = scale;
    };
    if (row < rows) {
        const In* xr = x + (size_t)row * cols;
        uint8_t* qr = q + (size_t)row * cols;
        if constexpr (NP > 0) {
            // width known at compile time (NP passes of 4 blocks): every load of the
            // row is issued before the first conversion
            float v[NP][8];
#pragma unroll
            for (int p = 0; p < NP; ++p) load8(xr + (4 * p + g) * 128 + e0, v[p]);
#pragma unroll
            for (int p = 0; p < NP; ++p) block(4 * p + g, v[p], qr);
        } else {
            // the next pass's load is issued before this pass's conversion, so each
            // wave keeps two 16-byte loads in flight
            float v[8], vn[8];
            if (g < nb) load8(xr + g * 128 + e0, v);
            for (int b0 = 0; b0 < nb; b0 += 4) {
                const int b = b0 + g;
                if (b + 4 < nb) load8(xr + (b + 4) * 128 + e0, vn);
                if (b < nb) block(b, v, qr);        // uniform inside each 16-lane group
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = vn[i];
            }
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < nb * kQuantRows; i += blockDim.x) {
        const int b = i / kQuantRows, r = i % kQuantRows;
        if (row0 + r < rows) scales[(size_t)b * rows + row0 + r] = sc[b][r];
    }
}

// x_dtype: 0 = fp32, 1 = bf16 bits.  The caller has checked 0 < cols <= kQuantMaxCols,
// cols % 128 == 0, rows >= 0 and the alignments.
void launch_quantize_fp8_blockwise(const void* x, int x_dtype, int rows, int cols, uint8_t* q,
                                   float* scales, hipStream_t stream) {
    if (rows <= 0) return;
    const dim3 grid((unsigned)((rows + kQuantRows - 1) / kQuantRows)), block(64 * kQuantRows);
    const bool hidden = cols == kH;       // the operator's width: 14 passes of 512 columns
    if (x_dtype == 1) {
        const uint16_t* xb = static_cast<const uint16_t*>(x);
        if (hidden) hipLaunchKernelGGL((quantize_fp8_blockwise_kernel<uint16_t, kH / 512>), grid, block, 0, stream, xb, rows, cols, q, scales);
        else hipLaunchKernelGGL((quantize_fp8_blockwise_kernel<uint16_t, 0>), grid, block, 0, stream, xb, rows, cols, q, scales);
    } else {
        const float* xf = static_cast<const float*>(x);
        if (hidden) hipLaunchKernelGGL((quantize_fp8_blockwise_kernel<float, kH / 512>), grid, block, 0, stream, xf, rows, cols, q, scales);
        else hipLaunchKernelGGL((quantize_fp8_blockwise_kernel<float, 0>), grid, block, 0, stream, xf, rows, cols, q, scales);
    }
}

}  // namespace moe
