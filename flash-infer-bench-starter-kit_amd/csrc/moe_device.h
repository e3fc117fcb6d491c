// moe_device.h -- shared constants and device helpers of the gfx950 fused-MoE kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

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

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// Round-to-nearest-even fp32 -> bf16 bits (NaN -> quiet NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u | ((u >> 16) & 0x8000u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
    return __uint_as_float(h << 16);
}

// Order-preserving 32-bit image of an fp32 score; NaN maps to 0 (never preferred).
__device__ __forceinline__ uint32_t order_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if (f != f) return 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float order_bits_inv(uint32_t k) {
    uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(u);
}

// One global_load_lds_dwordx4: lane L copies the 16 bytes at its own address g to
// LDS l + 16 L (l must be wave-uniform).
__device__ __forceinline__ void dma16(const uint8_t* g, uint8_t* l) {
    __builtin_amdgcn_global_load_lds(g, l, 16, 0, 0);
}

// s_waitcnt immediate that waits until at most v vector-memory operations are
// outstanding (gfx9 layout: vmcnt[3:0] bits 3:0, vmcnt[5:4] bits 15:14; expcnt and
// lgkmcnt left at their maxima).
__device__ __forceinline__ constexpr int vmcnt_imm(int v) {
    return (v & 15) | ((v >> 4) << 14) | (7 << 4) | (15 << 8);
}

}  // namespace moe
