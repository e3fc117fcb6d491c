// gemm1_stream.h -- SwiGLU helpers of the GEMM1 kernels and the work item of the
// register-staged weight-streaming GEMM1, shared by the streaming GEMM1 kernels of
// gemm1.hip.
#pragma once

#include "moe_device.h"

namespace moe {

__device__ __forceinline__ v4f mfma_fp8(const v8i& a, const v8i& b, const v4f& c) {
    // scale operands 0 -> plain (unscaled) e4m3 x e4m3 MFMA
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// SiLU x / (1 + e^-x) = x * rcp(1 + 2^(-x log2 e)) on the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32, about 1 ulp each): five instructions instead of a libm expf and
// an IEEE division, which made the GEMM1 epilogues VALU-bound.  Large |x| behave as the
// exact form: 2^+big -> inf -> rcp 0 -> -0 for x << 0, 2^-big -> 0 -> x for x >> 0.
__device__ __forceinline__ float silu_f32(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

// Four SwiGLU values of row `row`, columns n0..n0+3, in the fp16 form of C with its
// 16-column group exponent (moe_device.h): the plain fp16 rounding unless the group
// holds a value beyond the fp16 range, which sets the flag word *c_wide to 1 (a word in
// global memory or in LDS).  Every lane of the wave calls it; lanes with `valid` false
// (rows past the tile) store nothing.
__device__ __forceinline__ void store_swiglu4(const Intermediate& C, int* __restrict__ c_wide, int row,
                                              int n0, const v4f& g, const v4f& u, bool valid) {
    float c[4];
    float m = 0.f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
        c[v] = silu_f32(u[v]) * g[v];
        m = fmaxf(m, fabsf(c[v]));
    }
    if (!beyond_f16_in_wave(m)) {     // the usual case: every exponent of the call is 0
        if (!valid) return;
        store_f16x4_scaled(C.f16() + (size_t)row * kI + n0, c, 0);
        if ((n0 & (kGroup16 - 1)) == 0) C.f16_exp()[(size_t)row * (kI / kGroup16) + n0 / kGroup16] = 0;
        return;
    }
    const int e = group_exponent(m);
    if (!valid) return;
    store_f16x4_scaled(C.f16() + (size_t)row * kI + n0, c, e);
    if ((n0 & (kGroup16 - 1)) == 0) C.f16_exp()[(size_t)row * (kI / kGroup16) + n0 / kGroup16] = (uint8_t)e;
    if (e) *c_wide = 1;
}

// ---------------------------------------------------------------------------
// Register-staged weight streaming (decode and small prefill).  A work item is one row
// tile x one group of 16 SwiGLU columns (16 gate + 16 up weight rows); the 4 waves of
// a workgroup take 14 of its 56 K blocks each and reduce through LDS in a fixed order.
// Weight bytes come into registers with full-line loads (global_load_dwordx4, lane l
// reads row 8i + l/8, 16-byte chunk l%8 of the K block: 8 rows x 128 B per
// instruction) through a ring of D K blocks held in VGPRs, and each K block is turned
// into the MFMA layout through a 4 KB per-wave LDS slot (ds_write_b128 at the
// swizzled position, then ds_read_b128 by the MFMA lanes).  Keeping the in-flight
// bytes in VGPRs instead of an LDS ring lets more waves run per CU, so more bytes are
// in flight per CU (a streaming probe of this access pattern: 7.1 TB/s against
// 6.3 TB/s for LDS-landed DMA).
// A tile holds CB blocks of 16 token rows: every weight fragment feeds 2 CB MFMAs, so
// an expert with up to 16 CB routed rows streams its weights once.  An item covers
// NGRP groups of 16 SwiGLU columns, so each token fragment a wave loads feeds NGRP
// weight groups: token re-reads, which hit L2 but still take the CU's outstanding
// request slots, fall from half of the requests (NGRP = 1, CB = 2) to a third.
// TL: token rows take the weights' path too (full-line loads into the ring, then the
// LDS slot), instead of each lane loading its 32 MFMA-layout bytes, which covers half
// of 16 lines per instruction.  That pays on 32-row tiles (T = 193 .. 1536), where the
// kernel is bound by the CU's requests, and not on 16-row tiles.
// ---------------------------------------------------------------------------
// Streaming GEMM1 geometry: work items per row tile (one per NGRP groups of 16 SwiGLU
// columns) and the LDS each wave uses (its transpose slot: 32 NGRP weight rows, then,
// with TL, 16 CB token rows, 128 bytes each).
template <int CB, int NGRP, bool TL>
struct Gemm1Stream {
    static constexpr int kItems = kI / (16 * NGRP);
    static constexpr int kTok = 32 * NGRP * kBlk;
    static constexpr int kSlot = kTok + (TL ? 16 * CB * kBlk : 0);
};

// One work item of the streaming GEMM1: row tile (local expert le, rows row0 ..
// row0 + nrows - 1, whose tokens tok_of(row) gives) x the NGRP groups of 16 SwiGLU
// columns from ng on.  The 4 waves of the workgroup take 14 K blocks each and reduce
// through red[] in a fixed order; wave 0 writes the rows of C.
template <int D, int CB, int NGRP, bool TL, class TokOf>
__device__ __forceinline__ void gemm1_rstream_item(
    const uint8_t* __restrict__ hidden, const TokenScales& sa, const uint8_t* __restrict__ w1,
    const float* __restrict__ s1, int le, int row0, int nrows, int ng,
    const TokOf& tok_of, const Intermediate& C, int* __restrict__ c_wide,
    uint8_t (*slot_lds)[Gemm1Stream<CB, NGRP, TL>::kSlot], v4f (*red)[2][NGRP * CB][64], int wave) {
    constexpr int KSPLIT = 4;
    constexpr int KB = kHB / KSPLIT;                  // 14 K blocks per wave
    constexpr int NW = 4 * NGRP;                      // weight loads per K block (8 rows each)
    constexpr int kVmPerKb = NW + 3 * CB;             // per row block 2 token loads + 1 scale
    static_assert(D >= 2 && D <= 8 && (D - 1) * kVmPerKb < 64, "ring depth");
    static_assert(NGRP == 1 || NGRP == 2, "column groups per item");
    constexpr int kTok = 32 * NGRP * kBlk;           // token rows after the weight rows

    const int lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    const int ks = wave;
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
    uint8_t* slot = &slot_lds[wave][0];
    const int drow = lane >> 3, dchunk = lane & 7;
    const int swz = swz128(r16);
    const int rd_g0 = r16 * kBlk + (((2 * kq) ^ swz) << 4);
    const int rd_g1 = r16 * kBlk + (((2 * kq + 1) ^ swz) << 4);
    int wr[NW];                                        // LDS position of this lane's chunk
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const int r = 8 * i + drow;
        wr[i] = r * kBlk + ((dchunk ^ swz128(r)) << 4);
    }
    int twr[2 * CB];                                   // the same for the token rows
#pragma unroll
    for (int i = 0; i < 2 * CB; ++i) {
        const int r = 8 * i + drow;
        twr[i] = kTok + r * kBlk + ((dchunk ^ swz128(r)) << 4);
    }
    const int kb0 = ks * KB;

    // TL: token rows also come as full 128-byte lines (lane l: row 8 i + l / 8, chunk
    // l % 8; offsets fit 32 bits, T * 7168 < 2^32) and reach the MFMA layout through
    // the slot.  Otherwise each lane loads its 32 MFMA-layout bytes of row r16.
    uint32_t toff[2 * CB];
#pragma unroll
    for (int i = 0; i < 2 * CB; ++i) {
        if (TL) toff[i] = (uint32_t)tok_of(row0 + min(8 * i + drow, nrows - 1)) * kH + dchunk * 16;
        else if (i < CB) toff[i] = (uint32_t)tok_of(row0 + min(16 * i + r16, nrows - 1)) * kH + kq * 32;
    }
    const float* sp[CB];
#pragma unroll
    for (int c = 0; c < CB; ++c) {
        const int row = row0 + min(16 * c + r16, nrows - 1);
        sp[c] = sa.p + (sa.by_row ? row : tok_of(row));
    }
    // slot rows 32 gi + 0..15: gate rows of group ng + gi, 32 gi + 16..31: its up rows
    const uint8_t* wsrc[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) {
        const int r = 8 * i + drow;
        const int gi = r >> 5, rr = r & 31;
        const int n = (rr < 16) ? (ng + gi) * 16 + rr : kI + (ng + gi) * 16 + (rr - 16);
        wsrc[i] = w1 + (size_t)(le * kN1 + n) * kH + dchunk * 16;
    }
    // the NGRP groups lie in one 128-column scale block (16 NGRP divides 128).  The
    // wave's KB gate and up scales are loaded here, ahead of its first weight loads:
    // loaded in the K loop, the first of them would come due at the first K block's LDS
    // accesses, which wait for every scalar load in flight.
    const float* sg = s1 + (size_t)(le * kN1B + (ng >> 3)) * kHB;
    const float* su = sg + (size_t)kIB * kHB;
    float wgv[KB], wuv[KB];
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        wgv[k] = sg[kb0 + k];
        wuv[k] = su[kb0 + k];
    }
    __builtin_amdgcn_sched_barrier(0);

    v4u bw[D][NW];
    v4u bt[D][2 * CB];
    float bs[D][CB];
    auto issue = [&](int k) {
        const int kb = kb0 + k;
#pragma unroll
        for (int i = 0; i < NW; ++i) bw[k % D][i] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(wsrc[i] + kb * kBlk));
#pragma unroll
        for (int i = 0; i < 2 * CB; ++i) {
            const uint32_t o = TL ? toff[i] : toff[i >> 1] + 16 * (i & 1);
            bt[k % D][i] = *reinterpret_cast<const v4u*>(hidden + o + kb * kBlk);
        }
#pragma unroll
        for (int c = 0; c < CB; ++c) bs[k % D][c] = sp[c][(size_t)kb * sa.stride];
    };
#pragma unroll
    for (int k = 0; k < D - 1; ++k) {
        issue(k);
        __builtin_amdgcn_sched_barrier(0);
    }
    v4f ag[NGRP][CB], au[NGRP][CB];
#pragma unroll
    for (int gi = 0; gi < NGRP; ++gi)
#pragma unroll
        for (int c = 0; c < CB; ++c) ag[gi][c] = au[gi][c] = zero;
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
        for (int i = 0; i < NW; ++i) *reinterpret_cast<v4u*>(slot + wr[i]) = bw[k % D][i];
        v8i ba[CB];
        if constexpr (TL) {
#pragma unroll
            for (int i = 0; i < 2 * CB; ++i) *reinterpret_cast<v4u*>(slot + twr[i]) = bt[k % D][i];
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                const uint8_t* ts = slot + kTok + 16 * c * kBlk;
                const v4u a0 = *reinterpret_cast<const v4u*>(ts + rd_g0);
                const v4u a1 = *reinterpret_cast<const v4u*>(ts + rd_g1);
                ba[c] = v8i{(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
            }
        } else {
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                const v4u a0 = bt[k % D][2 * c], a1 = bt[k % D][2 * c + 1];
                ba[c] = v8i{(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
            }
        }
        const float wg = wgv[k], wu = wuv[k];
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi) {
            const uint8_t* gs = slot + gi * 32 * kBlk;
            const v4u g0 = *reinterpret_cast<const v4u*>(gs + rd_g0);
            const v4u g1 = *reinterpret_cast<const v4u*>(gs + rd_g1);
            const v4u u0 = *reinterpret_cast<const v4u*>(gs + 16 * kBlk + rd_g0);
            const v4u u1 = *reinterpret_cast<const v4u*>(gs + 16 * kBlk + rd_g1);
            const v8i bg = {(int)g0[0], (int)g0[1], (int)g0[2], (int)g0[3], (int)g1[0], (int)g1[1], (int)g1[2], (int)g1[3]};
            const v8i bu = {(int)u0[0], (int)u0[1], (int)u0[2], (int)u0[3], (int)u1[0], (int)u1[1], (int)u1[2], (int)u1[3]};
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                const float fg = bs[k % D][c] * wg, fu = bs[k % D][c] * wu;
                const v4f tg = mfma_fp8(bg, ba[c], zero);
                const v4f tu = mfma_fp8(bu, ba[c], zero);
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    ag[gi][c][v] = __builtin_fmaf(tg[v], fg, ag[gi][c][v]);
                    au[gi][c][v] = __builtin_fmaf(tu[v], fu, au[gi][c][v]);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }

#pragma unroll
    for (int gi = 0; gi < NGRP; ++gi)
#pragma unroll
        for (int c = 0; c < CB; ++c) {
            red[wave][0][gi * CB + c][lane] = ag[gi][c];
            red[wave][1][gi * CB + c][lane] = au[gi][c];
        }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int gi = 0; gi < NGRP; ++gi)
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                v4f g = red[0][0][gi * CB + c][lane], u = red[0][1][gi * CB + c][lane];
#pragma unroll
                for (int q = 1; q < KSPLIT; ++q) {
                    g += red[q][0][gi * CB + c][lane];
                    u += red[q][1][gi * CB + c][lane];
                }
                store_swiglu4(C, c_wide, row0 + 16 * c + r16, (ng + gi) * 16 + kq * 4, g, u,
                              16 * c + r16 < nrows);
            }
    }
    __syncthreads();
}

}  // namespace moe
