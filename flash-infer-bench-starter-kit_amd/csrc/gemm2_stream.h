// gemm2_stream.h -- the register-staged weight-streaming GEMM2 work items (fp16 MFMA
// on the fp16 form of C, or bf16 on the rare calls where C went beyond the fp16
// range), used by gemm2_rstream_kernel (gemm2.hip).
#pragma once

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

// 4 e4m3 bytes -> 4 fp16 (2 dwords); v_cvt_scalef32_pk_f16_fp8 with scale 1 is exact
__device__ __forceinline__ void e4m3x4_to_f16x4(uint32_t w, uint32_t& d0, uint32_t& d1) {
    d0 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w, 1.0f, false));
    d1 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8((int)w, 1.0f, true));
}

// 8 fp16 C values of one 16-column group (exponent e) as bf16 (round to nearest even).
__device__ __forceinline__ v4u c_f16_scaled_to_bf16(const v4u& h, int e) {
    v4u r;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        r[i] = f32_to_bf16_bits(f16_scaled_to_f32(h[i] & 0xffffu, e)) |
               (f32_to_bf16_bits(f16_scaled_to_f32(h[i] >> 16, e)) << 16);
    return r;
}

// One 16x16x32 MFMA of 8 widened W2 values per lane (e4m3 words w0, w1) against 8 C
// values (bf16 or fp16 bits, as the kernel's C form)
template <bool F16>
__device__ __forceinline__ v4f mfma_w2_c(uint32_t w0, uint32_t w1, const v4u& c, const v4f& acc) {
    uint32_t d0, d1, d2, d3;
    if constexpr (F16) {
        e4m3x4_to_f16x4(w0, d0, d1);
        e4m3x4_to_f16x4(w1, d2, d3);
        const v4u t = {d0, d1, d2, d3};
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, t), __builtin_bit_cast(v8h, c), acc, 0, 0, 0);
    } else {
        e4m3x4_to_bf16x4(w0, d0, d1);
        e4m3x4_to_bf16x4(w1, d2, d3);
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_v8bf(d0, d1, d2, d3), __builtin_bit_cast(v8bf, c), acc, 0, 0, 0);
    }
}

// End of a streaming work item: the KSPLIT waves of each column group add their K
// partials through LDS in a fixed order (so results do not depend on scheduling), and the
// first of them writes the expert rows that exist (fp16, see ExpertRows).
template <int KSPLIT, int HF, int CB>
__device__ __forceinline__ void reduce_store(const v4f (&acc)[HF][CB], v4f (*red)[HF][CB][64], int wave,
                                             int lane, int ks, int row0, int nrows, int hg,
                                             const ExpertRows& rows, int* __restrict__ rows_wide) {
    const int r16 = lane & 15, kq = lane >> 4;
#pragma unroll
    for (int hf = 0; hf < HF; ++hf)
#pragma unroll
        for (int c = 0; c < CB; ++c) red[wave][hf][c][lane] = acc[hf][c];
    __syncthreads();
    if (ks == 0) {
#pragma unroll
        for (int c = 0; c < CB; ++c) {
#pragma unroll
            for (int hf = 0; hf < HF; ++hf) {
                v4f o = red[wave][hf][c][lane];
#pragma unroll
                for (int q = 1; q < KSPLIT; ++q) o += red[wave + q][hf][c][lane];
                store_rows4(rows, rows_wide, row0 + 16 * c + r16, (hg + hf) * 16 + kq * 4, o,
                            16 * c + r16 < nrows);
            }
        }
    }
    __syncthreads();
}

// Register-staged W2 streaming (decode and small prefill).  One work item: a wave owns HF
// groups of 16 output columns (W2 rows, from hg0 + HF (wave / KSPLIT)) of local expert
// le for the row tile of 16 CB rows from row0 (nrows of them), over
// 16 / KSPLIT consecutive K blocks (partials of the KSPLIT waves of an item reduced
// through LDS in a fixed order).  The W2 bytes of a K block (16 HF rows x 128 B,
// full-line loads) and the fp16 C fragments are held in a ring of D K blocks in
// VGPRs, and each W2 block is moved to the MFMA layout through a per-wave LDS slot.
// Without an LDS ring more waves fit per CU, so more bytes are in flight; HF > 1
// shares each C fragment load among HF groups of 16 output columns, and CB > 1
// feeds each widened W2 fragment to CB blocks of 16 C rows.
// The kernel reads GEMM1's fp16-range flag once: fp16 C (the normal case) runs here.
template <int D, int KSPLIT, int HF, int CB>
__device__ __forceinline__ void gemm2_rstream_item(
    const uint16_t* __restrict__ inter, const uint8_t* __restrict__ w2,
    const float* __restrict__ s2, int le, int row0, int nrows, int hg0, const ExpertRows& rows,
    int* __restrict__ rows_wide, uint8_t (*slot_lds)[16 * HF * kBlk], v4f (*red)[HF][CB][64],
    int wave) {
    constexpr int KB = kIB / KSPLIT;
    constexpr int kVmPerKb = 2 * HF + 4 * CB;         // W2 loads, 4 C loads per row block
    static_assert(D >= 2 && (D - 1) * kVmPerKb < 64, "ring depth");
    static_assert(KSPLIT > 1, "the partials are reduced through LDS");

    const int lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    const int ngl = wave / KSPLIT, ks = wave % KSPLIT;
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
    uint8_t* slot = &slot_lds[wave][0];
    const int drow = lane >> 3, dchunk = lane & 7;
    const int swz = swz128(r16);
    const int rd0 = r16 * kBlk + (((2 * kq) ^ swz) << 4);
    const int rd1 = r16 * kBlk + (((2 * kq + 1) ^ swz) << 4);
    int wr[2 * HF];
#pragma unroll
    for (int i = 0; i < 2 * HF; ++i) {
        const int r = 8 * i + drow;
        wr[i] = r * kBlk + ((dchunk ^ swz128(r)) << 4);
    }
    const int kb0 = ks * KB;

    const int hg = hg0 + ngl * HF;                        // first of HF column groups
    // C row 16 c + r16: bf16 elements 32 kq + 8 j .. of each K block feed MFMA j
    const uint8_t* cp[CB];
#pragma unroll
    for (int c = 0; c < CB; ++c)
        cp[c] = reinterpret_cast<const uint8_t*>(inter + (size_t)(row0 + min(16 * c + r16, nrows - 1)) * kI) + kq * 64;
    const uint8_t* wsrc[2 * HF];
#pragma unroll
    for (int i = 0; i < 2 * HF; ++i)
        wsrc[i] = w2 + (size_t)(le * kH + hg * 16 + 8 * i + drow) * kI + dchunk * 16;
    // the wave's block scales, loaded ahead of its first W2 loads (in the K loop the first
    // would come due at the first K block's LDS accesses, which wait for every scalar
    // load in flight)
    float sbv[HF][KB];
#pragma unroll
    for (int hf = 0; hf < HF; ++hf) {
        const float* sp = s2 + (size_t)(le * kHB + ((hg + hf) >> 3)) * kIB;
#pragma unroll
        for (int k = 0; k < KB; ++k) sbv[hf][k] = sp[kb0 + k];
    }
    __builtin_amdgcn_sched_barrier(0);

    v4u bw[D][2 * HF];
    v4u bc[D][CB][4];
    auto issue = [&](int k) {
        const int kb = kb0 + k;
#pragma unroll
        for (int i = 0; i < 2 * HF; ++i) bw[k % D][i] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(wsrc[i] + kb * kBlk));
#pragma unroll
        for (int c = 0; c < CB; ++c)
#pragma unroll
            for (int j = 0; j < 4; ++j) bc[k % D][c][j] = *reinterpret_cast<const v4u*>(cp[c] + kb * 2 * kBlk + 16 * j);
    };
#pragma unroll
    for (int k = 0; k < D - 1 && k < KB; ++k) {
        issue(k);
        __builtin_amdgcn_sched_barrier(0);
    }
    v4f acc[HF][CB];
#pragma unroll
    for (int hf = 0; hf < HF; ++hf)
#pragma unroll
        for (int c = 0; c < CB; ++c) acc[hf][c] = zero;
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        if (k + D - 1 < KB) issue(k + D - 1);
        __builtin_amdgcn_sched_barrier(0);
        const int younger = (KB - 1 - k) < (D - 1) ? (KB - 1 - k) : (D - 1);
        switch (younger) {   // resolved at compile time after unrolling
            case 0: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
            case 1: __builtin_amdgcn_s_waitcnt(vmcnt_imm(1 * kVmPerKb)); break;
            case 2: __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * kVmPerKb)); break;
            case 3: __builtin_amdgcn_s_waitcnt(vmcnt_imm(3 * kVmPerKb)); break;
            case 4: __builtin_amdgcn_s_waitcnt(vmcnt_imm(4 * kVmPerKb)); break;
            case 5: __builtin_amdgcn_s_waitcnt(vmcnt_imm(5 * kVmPerKb)); break;
            case 6: __builtin_amdgcn_s_waitcnt(vmcnt_imm(6 * kVmPerKb)); break;
            default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(7 * kVmPerKb)); break;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < 2 * HF; ++i) *reinterpret_cast<v4u*>(slot + wr[i]) = bw[k % D][i];
#pragma unroll
        for (int hf = 0; hf < HF; ++hf) {
            const v4u x0 = *reinterpret_cast<const v4u*>(slot + hf * 16 * kBlk + rd0);
            const v4u x1 = *reinterpret_cast<const v4u*>(slot + hf * 16 * kBlk + rd1);
            const uint32_t ww[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
            v4f t[CB];
#pragma unroll
            for (int c = 0; c < CB; ++c) t[c] = zero;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int c = 0; c < CB; ++c) t[c] = mfma_w2_c<true>(ww[2 * j], ww[2 * j + 1], bc[k % D][c][j], t[c]);
            const float sb = sbv[hf][k];
#pragma unroll
            for (int c = 0; c < CB; ++c)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[hf][c][v] = __builtin_fmaf(t[c][v], sb, acc[hf][c][v]);
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    reduce_store<KSPLIT, HF, CB>(acc, red, wave, lane, ks, row0, nrows, hg, rows, rows_wide);
}

// The K partial of one wave of a work item when C went beyond the fp16 range somewhere
// (rare): bf16 MFMAs on C rebuilt from its fp16 form and group exponents, over K blocks
// ks KB .. ks KB + KB - 1 of the HF groups of 16 output columns from hg, for the CB
// 16-row blocks of the tile from row0.  Plain loads in the MFMA layout, one K block at a
// time: slow, but light on registers, so the normal path keeps its occupancy.
template <int KSPLIT, int HF, int CB>
__device__ __forceinline__ void gemm2_rare_partial(
    const uint16_t* __restrict__ inter, const uint8_t* __restrict__ inter_exp,
    const uint8_t* __restrict__ w2, const float* __restrict__ s2, int le, int row0, int nrows,
    int hg, int ks, v4f (&acc)[HF][CB]) {
    constexpr int KB = kIB / KSPLIT;
    const int lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int hf = 0; hf < HF; ++hf)
#pragma unroll
        for (int c = 0; c < CB; ++c) acc[hf][c] = zero;
#pragma unroll 1
    for (int kb = ks * KB; kb < (ks + 1) * KB; ++kb) {
        v4u cf[CB][4];
#pragma unroll
        for (int c = 0; c < CB; ++c) {
            const int row = row0 + min(16 * c + r16, nrows - 1);
            const size_t off = (size_t)row * kI + kb * kBlk + kq * 32;
            const uint8_t* ep = inter_exp + (size_t)row * (kI / kGroup16) + (kb * kBlk + kq * 32) / kGroup16;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                cf[c][j] = c_f16_scaled_to_bf16(*reinterpret_cast<const v4u*>(inter + off + 8 * j), ep[j >> 1]);
        }
#pragma unroll
        for (int hf = 0; hf < HF; ++hf) {
            const uint8_t* wp = w2 + (size_t)(le * kH + (hg + hf) * 16 + r16) * kI + kb * kBlk + kq * 32;
            const v4u x0 = *reinterpret_cast<const v4u*>(wp);
            const v4u x1 = *reinterpret_cast<const v4u*>(wp + 16);
            const uint32_t ww[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
            v4f t[CB];
#pragma unroll
            for (int c = 0; c < CB; ++c) t[c] = zero;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int c = 0; c < CB; ++c) t[c] = mfma_w2_c<false>(ww[2 * j], ww[2 * j + 1], cf[c][j], t[c]);
            const float sb = s2[(size_t)(le * kHB + ((hg + hf) >> 3)) * kIB + kb];
#pragma unroll
            for (int c = 0; c < CB; ++c)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[hf][c][v] = __builtin_fmaf(t[c][v], sb, acc[hf][c][v]);
        }
    }
}

// The work items of gemm2_rstream_item when C went beyond the fp16 range: each wave's K
// partial on the rare path, reduced and stored as the normal path does.
template <int KSPLIT, int HF, int CB>
__device__ __forceinline__ void gemm2_rstream_rare_item(
    const uint16_t* __restrict__ inter, const uint8_t* __restrict__ inter_exp,
    const uint8_t* __restrict__ w2, const float* __restrict__ s2, int le, int row0, int nrows,
    int hg0, const ExpertRows& rows, int* __restrict__ rows_wide, v4f (*red)[HF][CB][64], int wave) {
    const int lane = threadIdx.x & 63;
    const int ngl = wave / KSPLIT, ks = wave % KSPLIT;
    const int hg = hg0 + ngl * HF;
    v4f acc[HF][CB];
    gemm2_rare_partial<KSPLIT, HF, CB>(inter, inter_exp, w2, s2, le, row0, nrows, hg, ks, acc);
    reduce_store<KSPLIT, HF, CB>(acc, red, wave, lane, ks, row0, nrows, hg, rows, rows_wide);
}

}  // namespace moe
