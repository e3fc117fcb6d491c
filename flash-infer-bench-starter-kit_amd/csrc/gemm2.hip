// gemm2.hip -- grouped GEMM2 (2048 -> 7168): fp16 MFMA for the streaming kernels, FP8
// MFMA on the hi/lo form of C for the prefill kernel.
//
// Semantics: reference solution/cuda/moe.cu:231 (O = C @ W2[e]^T) with the 128x128
// block scales of gemm2_weights_scale applied per K block in the fp32 accumulator
// (the reference's CUTLASS path applies them in its mainloop,
// moe_grouped_gemm_fp8.cu:274-322):
//   O[r, h] = sum_kb sb2[e, h/128, kb] * sum_{i in kb} C[r, i] * W2[e, h, i]
// Streaming kernels: C is the fp16 SwiGLU output of GEMM1; when GEMM1 flagged a value
// beyond the fp16 range, C runs through bf16 instead, rebuilt from the fp16 values and
// their 16-column group exponents.  W2 e4m3 bytes are widened in registers to the same type
// (exact: every e4m3 value is an fp16 and a bf16 value) for
// v_mfma_f32_16x16x32_{f16,bf16}, operand A = 16 W2 rows, operand B = 16 C rows; lane l
// supplies row l%16 and K elements 32*(l/16) + 8j..8j+7 of the block for MFMA j = 0..3
// on both operands, and receives D[h = 4*(l/16)+v][row = l%16].  A work item's K blocks
// are split over waves and reduced through LDS in a fixed order.
// Prefill kernel: FP8 MFMA on the hi/lo form of C (see gemm2_prefill8_kernel).
// Expert rows O go to the combine in fp16 (ExpertRows: bf16 rows break the 1e-2
// tolerance where two large expert rows cancel, fp16 rows do not).  The reference re-quantises C to
// one e4m3 per element (kernel.cu:1086-1145), which does not meet atol = rtol = 1e-2
// against the fp32 restatement; both forms used here do.

#include "gemm2_stream.h"

MOE_STAMP_TABLE(gemm2)

namespace moe {

template <int D, int KSPLIT, int HF, int CB>
__global__ __launch_bounds__(256) void gemm2_rstream_kernel(
    Intermediate C, int* __restrict__ flags, const uint8_t* __restrict__ w2,
    const float* __restrict__ s2, const int4* __restrict__ tiles,
    const int* __restrict__ num_tiles, ExpertRows rows) {
    // flags[0]: C beyond the fp16 range (set by GEMM1); flags[1]: an expert row beyond it
    constexpr int NGW = 4 / KSPLIT;
    constexpr int kItems = (kH / 16) / (NGW * HF);
    __shared__ __attribute__((aligned(1024))) uint8_t slot_lds[4][16 * HF * kBlk];
    __shared__ v4f red[4][HF][CB][64];
    MOE_STAMP(2 * (int)blockIdx.x);
    // The first item's tile is read before the tile count, so that the two loads are in
    // flight together instead of one after the other: blockIdx.x / kItems is inside the
    // list's capacity (the grid has at most capacity x kItems workgroups), and a workgroup
    // past the count does not use what it read.  Each later tile is read after the item
    // before it.
    const int4 tl0 = tiles[blockIdx.x / kItems];
    int te = __builtin_amdgcn_readfirstlane(tl0.x), tr = __builtin_amdgcn_readfirstlane(tl0.y),
        tn = __builtin_amdgcn_readfirstlane(tl0.z);
    const int nwork = (*num_tiles) * kItems;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // the two paths keep separate loops, so each is register-allocated on its own
    if (__builtin_amdgcn_readfirstlane(flags[0]) == 0) {
        for (int work = blockIdx.x; work < nwork; work += gridDim.x) {
            gemm2_rstream_item<D, KSPLIT, HF, CB>(C.f16(), w2, s2, te, tr, tn,
                                                  (work % kItems) * NGW * HF, rows, flags + 1,
                                                  slot_lds, red, wave);
            if (work + (int)gridDim.x < nwork) {
                const int4 t = tiles[(work + gridDim.x) / kItems];
                te = t.x;
                tr = t.y;
                tn = t.z;
            }
        }
    } else {
        for (int work = blockIdx.x; work < nwork; work += gridDim.x) {
            const int4 tile = tiles[work / kItems];
            gemm2_rstream_rare_item<KSPLIT, HF, CB>(C.f16(), C.f16_exp(), w2, s2, tile.x, tile.y,
                                                    tile.z, (work % kItems) * NGW * HF, rows,
                                                    flags + 1, red, wave);
        }
    }
    MOE_STAMP(2 * (int)blockIdx.x + 1);
}

// Prefill GEMM2 (many tokens per expert): MFMA-bound tiling on FP8 MFMA with C in
// the fp8 hi/lo form written by the prefill GEMM1 kernels (C ~ sC * (hi + lo/16)).
// Per K block and 16 x 16 output block:
//   t   = mfma(W2, C_hi)                          v_mfma_f32_16x16x128_f8f6f4
//   t   = mfma_scaled(W2, C_lo, t, B scale 2^-4)  v_mfma_scale_..., E8M0 scale 123:
//                                                  exact, the products are fp8 x fp8
//   acc = fma(t, sC[row, kb] * sW2[h/128, kb], acc)
// so GEMM2 runs at the FP8 rate with no operand widening, and C keeps about 8
// significant bits (the fp32 SwiGLU value to within 2^-8 of its block maximum).
// Workgroup tile: 128 C rows x 256 output columns; waves 2 (rows) x 4 (columns),
// each 64 rows x 64 columns, inside one W2 row block (one W2 scale per K block).
// Stage (two, 64.5 KB each): C hi rows 16 KB | C lo rows 16 KB | W2 rows 32 KB |
// C row scales 512 B, all by buffer_load ... lds in two bursts per K block (C right
// after the barrier, W2 once this K block's operand reads are under way, ahead of its
// first MFMAs; issuing W2 after the second column block's MFMAs was 4% slower at
// T = 8192); rows keep 16-byte chunk c
// at c ^ swz128(r).  Items (128-row piece, 256-column group) are grouped up to 4
// pieces of one expert x all column groups with an XCD-contiguous mapping, as in
// the prefill GEMM1 (list order: the ranked order of the prefill GEMM1 was not faster
// here, 83-90 us either way at T = 1024 .. 2600).  A workgroup resolves the metadata of all its items at kernel
// start (prefill_items) and issues the first stage of its next item at the top of
// the current item's last K block, so the next item's data arrives while the last
// block computes and the epilogue stores.  In a K block, each 16 x 16 block's hi
// and lo MFMAs are separated by the other row blocks' MFMAs, and the fresh partials
// of one column block are scaled into the accumulators while the next column
// block's MFMAs run (fixed order), so no instruction waits on the MFMA before it.
// Tiles hold at most 128 rows.
struct Gemm2Item {
    __amdgpu_buffer_rsrc_t hi, lo, cs, w;
    uint32_t coff[2], csoff;
    int le, row0, nrows, hg;
    bool c_live;
};

__global__ __launch_bounds__(512, 1) void gemm2_prefill8_kernel(
    Intermediate C, const uint8_t* __restrict__ w2, const float* __restrict__ s2,
    const int4* __restrict__ tiles, const int* __restrict__ num_tiles,
    const int* __restrict__ exp_off, ExpertRows rows, int* __restrict__ rows_wide) {
    constexpr int NS = 2;
    constexpr int BM = 128;
    constexpr int NG = kH / 256;                // 28 column groups
    constexpr int kC = BM * kBlk;               // 16 KB per C half
    constexpr int kW = 256 * kBlk;              // 32 KB of W2 rows
    constexpr int kStage = 2 * kC + kW + BM * 4;
    constexpr int kWeightBurstAfter = 0;       // W2 burst in the first column block, before its MFMAs
    constexpr int kItemCap = 1024;              // per-workgroup item table (16 KB of LDS)
    static_assert(kIB % 2 == 0, "the next item's first stage must be stage 0");
    // one LDS object: the stages, then the item table
    __shared__ __attribute__((aligned(1024))) uint8_t lds[NS * kStage + kItemCap * sizeof(int4)];
    int4* const s_items = reinterpret_cast<int4*>(lds + NS * kStage);

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    const int wm = wave >> 2, wn = wave & 3;
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
    const int nitems = *num_tiles * NG;
    const int G = gridDim.x;
    const int base = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);   // XCD-contiguous slot
    const int drow = lane >> 3, dchunk = lane & 7;
    const int swz = swz128(r16);
    const int c0 = ((2 * kq) ^ swz) << 4, c1 = ((2 * kq + 1) ^ swz) << 4;
    // W2 rows of a wave's DMA do not depend on the item
    uint32_t woff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 32 * wave + 8 * i + drow;
        woff[i] = (uint32_t)r * kI + ((dchunk ^ swz128(r)) << 4);
    }

    const int nr = prefill_items<BM>(s_items, kItemCap, nitems, NG, base, G, tiles, exp_off);
    if (nr == 0) return;   // uniform: the whole workgroup has no item
    __syncthreads();

    auto make_item = [&](int r) {
        const int4 m = prefill_item<BM>(s_items, kItemCap, r, NG, base, G, tiles, exp_off);
        Gemm2Item it;
        const int le = m.x;
        it.le = le;
        it.row0 = m.y;
        it.nrows = m.z;
        it.hg = m.w;
        it.hi = buffer_rsrc(C.hi() + (size_t)it.row0 * kI, BM * kI);
        it.lo = buffer_rsrc(C.lo() + (size_t)it.row0 * kI, BM * kI);
        it.cs = buffer_rsrc(C.scales + it.row0, (uint32_t)(kIB * C.rows_cap - it.row0) * 4);
        it.w = buffer_rsrc(w2 + ((size_t)le * kH + it.hg * 256) * kI, 256 * kI);
        // wave w moves C rows 16w..16w+15 (hi and lo) and W2 rows 32w..32w+31; waves 0
        // and 1 move the row scales of rows 64w..64w+63
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int r = 16 * wave + 8 * i + drow;
            it.coff[i] = (uint32_t)min(r, it.nrows - 1) * kI + ((dchunk ^ swz128(r)) << 4);
        }
        it.csoff = (uint32_t)min(64 * wave + lane, it.nrows - 1) * 4;
        // a wave whose 16 C rows all lie past the tile moves nothing: they would only
        // repeat the last row, and the MFMAs of their 16-row block are skipped
        it.c_live = 16 * wave < it.nrows;
        return it;
    };
    auto issue_c = [&](const Gemm2Item& it, int kb) {
        uint8_t* st = lds + (kb & 1) * kStage;
        if (it.c_live) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                bdma16(it.hi, it.coff[i], (uint32_t)kb * kBlk, st + (16 * wave + 8 * i) * kBlk);
                bdma16(it.lo, it.coff[i], (uint32_t)kb * kBlk, st + kC + (16 * wave + 8 * i) * kBlk);
            }
        }
        if (wave < 2 && 64 * wave < it.nrows)
            bdma4(it.cs, it.csoff, (uint32_t)kb * C.rows_cap * 4, st + 2 * kC + kW + wave * 256);
    };
    auto issue_w = [&](const Gemm2Item& it, int kb) {
        uint8_t* st = lds + (kb & 1) * kStage;
#pragma unroll
        for (int i = 0; i < 4; ++i) bdma16(it.w, woff[i], (uint32_t)kb * kBlk, st + 2 * kC + (32 * wave + 8 * i) * kBlk);
    };

    Gemm2Item cur = make_item(0), nxt = cur;
    issue_c(cur, 0);
    issue_w(cur, 0);
    for (int r = 0; r < nr; ++r) {
        const bool more = r + 1 < nr;
        // W2 block scales of this wave's columns (scalar loads from the kernel argument)
        const float* sbp = s2 + (size_t)(cur.le * kHB + 2 * cur.hg + (wn >> 1)) * kIB;
        v4f acc[4][4];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int n = 0; n < 4; ++n) acc[s][n] = zero;

        // 16-row blocks of this wave that exist: padding blocks skip their MFMAs
        auto kloop = [&](auto live) {
        constexpr int NLIVE = decltype(live)::value;
        constexpr int NT = NLIVE > 0 ? NLIVE : 1;
#pragma unroll 1
        for (int kb = 0; kb < kIB; ++kb) {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            __syncthreads();
            if (kb + 1 < kIB) {
                issue_c(cur, kb + 1);
                if (kWeightBurstAfter < 0 || NLIVE == 0) issue_w(cur, kb + 1);
            } else if (more) {
                // stage 0 is free (every wave is past K block kIB - 2): the next item's first stage
                nxt = make_item(r + 1);
                issue_c(nxt, 0);
                issue_w(nxt, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (NLIVE == 0) continue;

            const uint8_t* st = lds + (kb & 1) * kStage;
            const float sw = sbp[kb];
            const float* csr = reinterpret_cast<const float*>(st + 2 * kC + kW);
            v8i ch[4], cl[4];
            float f[4];
#pragma unroll
            for (int s = 0; s < NLIVE; ++s) {
                const int rr = 64 * wm + 16 * s + r16;
                const uint8_t* ph = st + rr * kBlk;
                const uint8_t* pl = st + kC + rr * kBlk;
                const v4u h0 = *reinterpret_cast<const v4u*>(ph + c0);
                const v4u h1 = *reinterpret_cast<const v4u*>(ph + c1);
                const v4u l0 = *reinterpret_cast<const v4u*>(pl + c0);
                const v4u l1 = *reinterpret_cast<const v4u*>(pl + c1);
                ch[s] = v8i{(int)h0[0], (int)h0[1], (int)h0[2], (int)h0[3], (int)h1[0], (int)h1[1], (int)h1[2], (int)h1[3]};
                cl[s] = v8i{(int)l0[0], (int)l0[1], (int)l0[2], (int)l0[3], (int)l1[0], (int)l1[1], (int)l1[2], (int)l1[3]};
                f[s] = csr[rr] * sw;
            }
            auto read_w = [&](int n) {
                const uint8_t* rp = st + 2 * kC + (64 * wn + 16 * n + r16) * kBlk;
                const v4u x0 = *reinterpret_cast<const v4u*>(rp + c0);
                const v4u x1 = *reinterpret_cast<const v4u*>(rp + c1);
                return v8i{(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3], (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
            };
            v8i w = read_w(0);
            v4f tp[NT];
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                v8i wnx = w;
                if (n < 3) wnx = read_w(n + 1);
                if (n == kWeightBurstAfter && kb + 1 < kIB) {
                    __builtin_amdgcn_sched_barrier(0);
                    issue_w(cur, kb + 1);
                }
                v4f tc[NT];
#pragma unroll
                for (int s = 0; s < NLIVE; ++s) {
                    __builtin_amdgcn_sched_barrier(0);
                    tc[s] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w, ch[s], zero, 0, 0, 0, 0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                    if (n > 0) {
#pragma unroll
                        for (int v = 0; v < 4; ++v) acc[s][n - 1][v] = __builtin_fmaf(tp[s][v], f[s], acc[s][n - 1][v]);
                    }
                }
#pragma unroll
                for (int s = 0; s < NLIVE; ++s) {
                    __builtin_amdgcn_sched_barrier(0);
                    tc[s] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w, cl[s], tc[s], 0, 0, 0, 127, 0, 123);
                }
#pragma unroll
                for (int s = 0; s < NLIVE; ++s) tp[s] = tc[s];
                w = wnx;
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < NLIVE; ++s)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[s][3][v] = __builtin_fmaf(tp[s][v], f[s], acc[s][3][v]);
        }
        };
        with_live_blocks(live_blocks(64 * wm, cur.nrows), kloop);

        // lane holds D[h = 64 wn + 16 n + 4 kq + v][row = 64 wm + 16 s + r16]
        float mx = 0.f;
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int n = 0; n < 4; ++n)
#pragma unroll
                for (int v = 0; v < 4; ++v) mx = fmaxf(mx, fabsf(acc[s][n][v]));
        if (!beyond_f16_in_wave(mx)) {
            // the usual case: plain fp16, and the 4 zero exponents of a row's 64 columns
            // as one 4-byte store (lane kq = 0 of the row).  The fp16 pairs of column
            // blocks (0, 1) and (2, 3) are exchanged across the row's 4 lanes (lanes l,
            // l+16, l+32, l+48: a 32-lane then a 16-lane swap) so that lane kq holds
            // columns 8 kq .. 8 kq + 7 of the pair: one 16-byte store writes 64
            // consecutive bytes of the row.
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int rr = 64 * wm + 16 * s + r16;
                uint32_t w[4][2];
#pragma unroll
                for (int n = 0; n < 4; ++n)
#pragma unroll
                    for (int q = 0; q < 2; ++q)
                        w[n][q] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)acc[s][n][2 * q]) |
                                  ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)acc[s][n][2 * q + 1]) << 16);
#pragma unroll
                for (int pr = 0; pr < 2; ++pr) {
                    const int a = 2 * pr, b = 2 * pr + 1;
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        const auto p = __builtin_amdgcn_permlane32_swap(w[a][q], w[b][q], false, false);
                        w[a][q] = p[0];
                        w[b][q] = p[1];
                    }
#pragma unroll
                    for (int q = 0; q < 2; ++q) {
                        const auto p = __builtin_amdgcn_permlane16_swap(w[a][q], w[b][q], false, false);
                        w[a][q] = p[0];
                        w[b][q] = p[1];
                    }
                }
                if (rr >= cur.nrows) continue;   // after the swaps: every lane takes part
                const size_t row = (size_t)(cur.row0 + rr);
                const int c0 = cur.hg * 256 + 64 * wn;
#pragma unroll
                for (int pr = 0; pr < 2; ++pr)
                    *reinterpret_cast<v4u*>(rows.f16 + row * kH + c0 + 32 * pr + 8 * kq) =
                        v4u{w[2 * pr][0], w[2 * pr][1], w[2 * pr + 1][0], w[2 * pr + 1][1]};
                if (kq == 0) *reinterpret_cast<uint32_t*>(rows.exp + row * (kH / kGroup16) + c0 / kGroup16) = 0u;
            }
        } else {
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int rr = 64 * wm + 16 * s + r16;
#pragma unroll
                for (int n = 0; n < 4; ++n)
                    store_rows4(rows, rows_wide, cur.row0 + rr, cur.hg * 256 + 64 * wn + 16 * n + 4 * kq,
                                acc[s][n], rr < cur.nrows);
            }
        }
        cur = nxt;
    }
}

__global__ void e4m3_to_bf16_kernel(const uint32_t* __restrict__ in, uint2* __restrict__ out, int nwords) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nwords) return;
    uint32_t d0, d1;
    e4m3x4_to_bf16x4(in[i], d0, d1);
    out[i] = make_uint2(d0, d1);
}

// Debug: widen e4m3 bytes to fp16 with the conversion of GEMM2's fp16 form.
__global__ void e4m3_to_f16_kernel(const uint32_t* __restrict__ in, uint2* __restrict__ out, int nwords) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nwords) return;
    uint32_t d0, d1;
    e4m3x4_to_f16x4(in[i], d0, d1);
    out[i] = make_uint2(d0, d1);
}

static int grid_for2(long long work) { return (int)(work < 4096 ? work : 4096); }

bool launch_gemm2_shared(const Intermediate&, int*, const uint8_t*, const float*, const int4*, const int*,
                         int, const ExpertRows&, hipStream_t);

// Variants (the tile height of the dispatch they expect, and the form of C they read):
//   1  register-staged streaming, 32 columns x 1 row block per wave      16-row   fp16
//   3  register-staged streaming, 64 columns x 2 row blocks per wave     32-row   fp16
//   5  prefill, 8 waves, 128 x 256 workgroup tile, over the 128-row second tile list
//      of the dispatch (whatever the first list's height)                         hi/lo
//   7  token-sharing: 64-row tile x 128 columns, C rows shared in LDS (gemm2_shared.hip)
//                                                                      64-row   fp16
bool launch_gemm2(int variant, const Intermediate& C, const uint8_t* w2, const float* s2,
                  const int4* tiles, const int* num_tiles, const int* exp_off, int max_tiles,
                  const ExpertRows& rows, hipStream_t stream) {
    int* flags = const_cast<int*>(exp_off) + kCWideFlag;   // [C beyond fp16, rows beyond fp16]
    const long long mt = max_tiles;
    constexpr int G = kH / 16;      // 16-column groups
    switch (variant) {
        case 1:
            launch_kernel((gemm2_rstream_kernel<4, 4, 2, 1>), dim3(grid_for2(mt * G / 2)), dim3(256), 0,
                               stream, C, flags, w2, s2, tiles, num_tiles, rows);
            return true;
        case 3:
            launch_kernel((gemm2_rstream_kernel<3, 4, 4, 2>), dim3(grid_for2(mt * G / 4)), dim3(256), 0,
                               stream, C, flags, w2, s2, tiles, num_tiles, rows);
            return true;
        case 5:
            launch_kernel(gemm2_prefill8_kernel, dim3(256), dim3(512), 0, stream, C, w2, s2, tiles,
                               num_tiles, exp_off, rows, flags + 1);
            return true;
        case 7:
            return launch_gemm2_shared(C, flags, w2, s2, tiles, num_tiles, max_tiles, rows, stream);
        default: return false;
    }
}

void launch_e4m3_to_f16(const uint8_t* in, uint16_t* out, int n, hipStream_t stream) {
    const int nwords = n / 4;
    if (nwords <= 0) return;
    hipLaunchKernelGGL(e4m3_to_f16_kernel, dim3((nwords + 255) / 256), dim3(256), 0, stream,
                       reinterpret_cast<const uint32_t*>(in), reinterpret_cast<uint2*>(out), nwords);
}

void launch_e4m3_to_bf16(const uint8_t* in, uint16_t* out, int n, hipStream_t stream) {
    const int nwords = n / 4;
    if (nwords <= 0) return;
    hipLaunchKernelGGL(e4m3_to_bf16_kernel, dim3((nwords + 255) / 256), dim3(256), 0, stream,
                       reinterpret_cast<const uint32_t*>(in), reinterpret_cast<uint2*>(out), nwords);
}

}  // namespace moe
