// gemm1.hip -- grouped FP8 GEMM1 (7168 -> 2 x 2048) with the SwiGLU epilogue fused.
//
// Semantics: reference solution/cuda/moe.cu:222-229 on block-scaled inputs
// (moe_grouped_gemm_fp8.cu:194-264 applies the same scales inside the CUTLASS
// mainloop):
//   G1[r, n] = sum_kb sa[kb, tok(r)] * sb[e, n/128, kb] * sum_{k in kb} A[tok(r), k] W1[e, n, k]
//   C[r, i]  = silu(G1[r, 2048 + i]) * G1[r, i]        (kernel.cu:1104-1108 convention)
// C is written as one row per routed assignment for GEMM2: the fp16 form (fp16 values
// with a power-of-two exponent byte per 16-column group, nonzero only where a group
// holds a value beyond the fp16 range) by the streaming kernels, the fp8 hi/lo form by
// the prefill kernels (moe_device.h, Intermediate).
//
// Kernels: register-staged weight streaming for small T (a work item is one row tile
// of 16 or 32 rows x 16 gate + 16 up rows, its 56 K blocks split over the 4 waves of
// a workgroup and reduced through LDS in a fixed order, so results do not depend on
// scheduling), the same streaming with a 64-row tile's token rows shared by the
// workgroup for mid-size T, and MFMA-bound prefill kernels for large T (256-row tiles).
//
// MFMA: v_mfma_f32_16x16x128_f8f6f4 (e4m3 x e4m3), one instruction per 128-wide K
// block, so the per-block scales multiply a fresh fp32 partial before it joins the
// accumulator.  Weight rows feed operand A (16 n rows), gathered token rows feed
// operand B (16 tokens); lane l holds row/token l%16 and K bytes 32*(l/16)..+31 of
// the block for both operands, and receives D[n = 4*(l/16)+v][token = l%16].

#include "dispatch_rows.h"
#include "gemm1_stream.h"
#include "route_token.h"

#include <mutex>

MOE_STAMP_TABLE(gemm1)

namespace moe {

// The streaming GEMM1 over the row tiles of a dispatch (see gemm1_rstream_item).
template <int D, int CB, int NGRP, bool TL>
__global__ __launch_bounds__(256) void gemm1_rstream_kernel(
    const uint8_t* __restrict__ hidden, TokenScales sa, int T,
    const uint8_t* __restrict__ w1, const float* __restrict__ s1,
    const int4* __restrict__ tiles, const int* __restrict__ num_tiles,
    const int* __restrict__ sorted_tok, Intermediate C, int* __restrict__ c_wide) {
    using S = Gemm1Stream<CB, NGRP, TL>;
    __shared__ __attribute__((aligned(1024))) uint8_t slot_lds[4][S::kSlot];
    __shared__ v4f red[4][2][NGRP * CB][64];
    // the first item's tile read before the tile count, both loads in flight together
    // (blockIdx.x / kItems is inside the list's capacity: the grid has at most capacity x
    // kItems workgroups; a workgroup past the count does not use what it read); each later
    // tile is read after the item before it
    const int4 tl0 = tiles[blockIdx.x / S::kItems];
    int te = __builtin_amdgcn_readfirstlane(tl0.x), tr = __builtin_amdgcn_readfirstlane(tl0.y),
        tn = __builtin_amdgcn_readfirstlane(tl0.z);
    const int nwork = (*num_tiles) * S::kItems;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    for (int work = blockIdx.x; work < nwork; work += gridDim.x) {
        gemm1_rstream_item<D, CB, NGRP, TL>(hidden, sa, w1, s1, te, tr, tn,
                                            (work % S::kItems) * NGRP,
                                            [&](int row) { return sorted_tok[row]; }, C, c_wide,
                                            slot_lds, red, wave);
        if (work + (int)gridDim.x < nwork) {
            const int4 t = tiles[(work + gridDim.x) / S::kItems];
            te = t.x;
            tr = t.y;
            tn = t.z;
        }
    }
}

// Streaming GEMM1 with the tile's token rows shared by the workgroup.  A work item is one
// row tile of up to 64 rows x 16 NWV SwiGLU columns; each of the NWV waves streams its
// own 16 gate + 16 up weight rows over all 56 K blocks through a register ring, as the
// other streaming kernels do, while the token rows of a K block come once for the whole
// workgroup by buffer_load ... lds into a ring of LDS stages (wave w moves rows
// 64/NWV w .. 64/NWV (w + 1) - 1, wave 0 the 64 token scales).  With 8 waves the
// workgroup requests 32 KB of weights and at most 8 KB of token rows per K block for
// 64 x 128 outputs, where the 32-row kernel, whose waves split K and each load the
// tile's rows, requests 12 KB for 32 x 32; and an expert of up to 64 rows streams its
// weights once.  Each wave owns its columns over the whole K, so there is no cross-wave
// reduction; one barrier per K block hands the token stage over.
// D: register ring depth (K blocks of weights per wave); the token stages are one more,
// so that the loads of block kb + D - 1 can go out before the barrier of block kb.
template <int D, int NWV>
struct Gemm1Shared {
    static_assert(NWV == 4 || NWV == 8, "waves per workgroup");
    static constexpr int kSlot = 32 * kBlk;                 // a wave's weight transpose slot
    static constexpr int kTokStage = 64 * kBlk + 64 * 4;    // 64 token rows + their scales
    static constexpr int kStages = D + 1;
    static constexpr int kLds = NWV * kSlot + kStages * kTokStage;
    static constexpr int kItems = kI / (16 * NWV);          // work items per tile
    static constexpr int kRowsPerWave = 64 / NWV;           // token rows each wave moves
};

// One item of gemm1_shared_kernel with CB live 16-row blocks (the tile has 16 CB - 15 ..
// 16 CB rows): wave `wave` computes SwiGLU columns 16 ng .. 16 ng + 15 of rows row0 ..
// row0 + nrows - 1.
template <int D, int NWV, int CB>
__device__ __forceinline__ void gemm1_shared_item(
    const uint8_t* __restrict__ hidden, const TokenScales& sa, __amdgpu_buffer_rsrc_t rs_h,
    __amdgpu_buffer_rsrc_t rs_s, const uint8_t* __restrict__ w1, const float* __restrict__ s1,
    int le, int row0, int nrows, int ng, const int* __restrict__ sorted_tok, const Intermediate& C,
    int* __restrict__ c_wide, uint8_t* lds, int wave) {
    using S = Gemm1Shared<D, NWV>;
    static_assert(kHB % D == 0, "the K loop runs in steps of the ring depth");
    const int lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    const int drow = lane >> 3, dchunk = lane & 7;
    const int swz = swz128(r16);
    const int rd_g0 = r16 * kBlk + (((2 * kq) ^ swz) << 4);
    const int rd_g1 = r16 * kBlk + (((2 * kq + 1) ^ swz) << 4);
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
    uint8_t* const slot = lds + wave * S::kSlot;
    uint8_t* const tok0 = lds + NWV * S::kSlot;

    // weight rows of this wave: slot rows 0..15 gate rows of group ng, 16..31 its up rows,
    // by buffer loads over the expert's W1 (32-bit offsets: one VGPR per load, the K block
    // in the scalar offset)
    const __amdgpu_buffer_rsrc_t rs_w = buffer_rsrc(w1 + (size_t)le * kN1 * kH, (uint32_t)kN1 * kH);
    uint32_t woff[4];
    int wr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 8 * i + drow;
        const int n = (r < 16) ? ng * 16 + r : kI + ng * 16 + (r - 16);
        woff[i] = (uint32_t)n * kH + dchunk * 16;
        wr[i] = r * kBlk + ((dchunk ^ swz128(r)) << 4);
    }
    // the NWV groups of a workgroup lie in one 128-column scale block
    const float* sg = s1 + (size_t)(le * kN1B + (ng >> 3)) * kHB;
    const float* su = sg + (size_t)kIB * kHB;
    // token rows of this wave, 8 per instruction (clamped into the tile), for the live
    // blocks: the stage rows of a live block are always written, so no stale row
    // reaches an MFMA
    constexpr int NT = S::kRowsPerWave / 8;
    bool tlive[NT];
    uint32_t toff[NT];
    int ntok = 0;
#pragma unroll
    for (int i = 0; i < NT; ++i) {
        const int tr = S::kRowsPerWave * wave + 8 * i + drow;
        tlive[i] = S::kRowsPerWave * wave + 8 * i < 16 * CB;
        toff[i] = (uint32_t)sorted_tok[row0 + min(tr, nrows - 1)] * kH + ((dchunk ^ swz128(tr)) << 4);
        ntok += tlive[i] ? 1 : 0;
    }
    const int sr = min(lane, nrows - 1);
    const uint32_t soff = (uint32_t)(sa.by_row ? row0 + sr : sorted_tok[row0 + sr]) * 4;
    const int nvm = 4 + ntok + (wave == 0 ? 1 : 0);   // loads per K block

    // K block kb: weights in ring slot kb % D, token rows in stage kb % (D + 1)
    v4u bw[D][4];
    auto issue = [&](int kb, int ring) {
#pragma unroll
        for (int i = 0; i < 4; ++i)   // aux 2: nt, the weights are read once
            bw[ring][i] = __builtin_amdgcn_raw_buffer_load_b128(rs_w, woff[i], (uint32_t)kb * kBlk, 2);
        uint8_t* st = tok0 + (kb % S::kStages) * S::kTokStage;
#pragma unroll
        for (int i = 0; i < NT; ++i)
            if (tlive[i]) bdma16(rs_h, toff[i], (uint32_t)kb * kBlk, st + (S::kRowsPerWave * wave + 8 * i) * kBlk);
        if (wave == 0) bdma4(rs_s, soff, (uint32_t)kb * sa.stride * 4, st + 64 * kBlk);
    };
#pragma unroll
    for (int k = 0; k < D - 1; ++k) issue(k, k);

    v4f ag[CB], au[CB];
#pragma unroll
    for (int c = 0; c < CB; ++c) ag[c] = au[c] = zero;
#pragma unroll 1
    for (int kb0 = 0; kb0 < kHB; kb0 += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            const int kb = kb0 + j;
            // block kb + D - 1 goes to the ring slot block kb - 1 used (written to the LDS
            // slot before) and to the stage of block kb - 2, which every wave finished
            // reading before the barrier of block kb - 1
            if (kb + D - 1 < kHB) issue(kb + D - 1, (j + D - 1) % D);
            __builtin_amdgcn_sched_barrier(0);
            // this wave's loads of block kb are in (those of the D - 1 blocks after it
            // may stay in flight); after the barrier, every wave's (the token stage)
            wait_vm_upto24(min(kHB - 1 - kb, D - 1) * nvm);
            lds_barrier();
#pragma unroll
            for (int i = 0; i < 4; ++i) *reinterpret_cast<v4u*>(slot + wr[i]) = bw[j][i];
            const uint8_t* st = tok0 + (kb % S::kStages) * S::kTokStage;
            const float* ssc = reinterpret_cast<const float*>(st + 64 * kBlk);
            const float wg = sg[kb], wu = su[kb];
            const v4u g0 = *reinterpret_cast<const v4u*>(slot + rd_g0);
            const v4u g1 = *reinterpret_cast<const v4u*>(slot + rd_g1);
            const v4u u0 = *reinterpret_cast<const v4u*>(slot + 16 * kBlk + rd_g0);
            const v4u u1 = *reinterpret_cast<const v4u*>(slot + 16 * kBlk + rd_g1);
            const v8i bg = {(int)g0[0], (int)g0[1], (int)g0[2], (int)g0[3], (int)g1[0], (int)g1[1], (int)g1[2], (int)g1[3]};
            const v8i bu = {(int)u0[0], (int)u0[1], (int)u0[2], (int)u0[3], (int)u1[0], (int)u1[1], (int)u1[2], (int)u1[3]};
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                __builtin_amdgcn_sched_barrier(0);   // one row block at a time: short live ranges
                const uint8_t* ts = st + 16 * c * kBlk;
                const v4u a0 = *reinterpret_cast<const v4u*>(ts + rd_g0);
                const v4u a1 = *reinterpret_cast<const v4u*>(ts + rd_g1);
                const v8i ba = {(int)a0[0], (int)a0[1], (int)a0[2], (int)a0[3], (int)a1[0], (int)a1[1], (int)a1[2], (int)a1[3]};
                const float sc = ssc[16 * c + r16];
                const float fg = sc * wg, fu = sc * wu;
                const v4f tg = mfma_fp8(bg, ba, zero);
                const v4f tu = mfma_fp8(bu, ba, zero);
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    ag[c][v] = __builtin_fmaf(tg[v], fg, ag[c][v]);
                    au[c][v] = __builtin_fmaf(tu[v], fu, au[c][v]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int c = 0; c < CB; ++c)
        store_swiglu4(C, c_wide, row0 + 16 * c + r16, ng * 16 + kq * 4, ag[c], au[c], 16 * c + r16 < nrows);
}

// WPE: the waves per SIMD the register allocation is held to (1: the compiler's choice,
// 172 registers, two workgroups per CU; 3: 153 registers, three).
// With three per CU the kernel chooses, from the call's tile count, how many of its 768
// workgroups work: items are equal (an item streams 128 weight rows over all of K), so the
// rounds decide the time, and 768 < items <= 1024 takes two rounds either way, where two
// workgroups per CU run each item faster; then workgroups 512 .. 767 exit at once and the
// other 512 (two per CU, the workgroups being spread over the CUs in launch order) take
// the items.  Otherwise all 768 work (fewer rounds).  Which workgroup computes an item
// changes nothing in the result.
template <int D, int NWV, int WPE>
__global__ __launch_bounds__(64 * NWV) __attribute__((amdgpu_waves_per_eu(WPE))) void gemm1_shared_kernel(
    const uint8_t* __restrict__ hidden, TokenScales sa, int T,
    const uint8_t* __restrict__ w1, const float* __restrict__ s1,
    const int4* __restrict__ tiles, const int* __restrict__ num_tiles,
    const int* __restrict__ sorted_tok, Intermediate C, int* __restrict__ c_wide) {
    using S = Gemm1Shared<D, NWV>;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[S::kLds];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // token rows: T * 7168 < 2^32 (kMaxT); token scales: 56 x stride floats
    const __amdgpu_buffer_rsrc_t rs_h = buffer_rsrc(hidden, (uint32_t)T * kH);
    const __amdgpu_buffer_rsrc_t rs_s = buffer_rsrc(sa.p, (uint32_t)kHB * (uint32_t)sa.stride * 4);
    // the first item's tile read before the tile count, both loads in flight together
    // (blockIdx.x / kItems is inside the list's capacity: the grid has at most capacity x
    // kItems workgroups; a workgroup past the count does not use what it read); each later
    // tile is read after the item before it
    const int4 tl0 = tiles[blockIdx.x / S::kItems];
    int te = __builtin_amdgcn_readfirstlane(tl0.x), tr = __builtin_amdgcn_readfirstlane(tl0.y),
        tn = __builtin_amdgcn_readfirstlane(tl0.z);
    const int nwork = (*num_tiles) * S::kItems;
    int G = gridDim.x;
    if (WPE == 3 && G == 768 && nwork > 768 && nwork <= 1024) G = 512;
    if ((int)blockIdx.x >= G) return;   // uniform: the whole workgroup
    for (int work = blockIdx.x; work < nwork; work += G) {
        const int ng = (work % S::kItems) * NWV + wave;
        with_live_blocks(live_blocks(0, tn), [&](auto live) {
            constexpr int CB = decltype(live)::value;
            if constexpr (CB > 0)
                gemm1_shared_item<D, NWV, CB>(hidden, sa, rs_h, rs_s, w1, s1, te, tr, tn, ng,
                                         sorted_tok, C, c_wide, lds, wave);
        });
        if (work + G < nwork) {
            const int4 t = tiles[(work + G) / S::kItems];
            te = t.x;
            tr = t.y;
            tn = t.z;
        }
        __syncthreads();   // the next item's first loads reuse the token stages
    }
}

// The streaming GEMM1 of variant 1 with the dispatch folded in, for T <= 64: every
// workgroup of a persistent grid computes the part of the call's dispatch its items need,
// into LDS.  Wave 0 takes one ballot per local expert over the tokens (lane = token),
// which gives each expert's row count, the tile list, and each row's rank among the
// expert's rows (rows follow token order); then all four waves place the tokens of the
// rows, two of each token's eight routes per wave.  The last workgroup, which has the
// fewest items (none up to T = 32), also writes the whole dispatch to the workspace
// (expert offsets, tile count and list, permutation, row weights, inverse map), where
// the GEMM2 and combine kernels after this one read it.  Workgroup b takes items b,
// b + G, ..., so the items of an expert's consecutive tiles that read the same weight
// rows (128 items apart) run on one XCD.  The dispatch launch goes away; the part of the
// dispatch before the first weight load costs a workgroup about what the separate
// kernel's two dependent loads (tile list, then permutation) cost.
//
// NRW > 0 (T <= NRW): the routing too.  Every workgroup routes the call's tokens itself
// from the logits (route_token, the route kernel's computation: wave w takes token w) into
// LDS, where the dispatch reads them; the last workgroup also writes them to the
// workspace.  NRW = 8 (5 <= T <= 8) runs workgroups of 8 waves, one per CU, so that a SIMD
// routes two tokens, not six; its waves then work as two groups of four, each taking every
// other of the workgroup's items, in step (a group without an item passes the item's two
// barriers), so a CU still streams two items at a time.  The route launch, its kernel boundary
// and the dispatch's dependent load of the routing ids go away.  Nothing clears the
// C-range flag word before this kernel: it sets the word when C goes beyond the fp16
// range, and the GEMM2 after it (variant 6) checks a nonzero word against C's group
// exponents (a stale nonzero word left by earlier calls or other data only costs that check,
// and the GEMM2 clears it).
constexpr int kDG1MaxTiles = dispatch_max_tiles(kDispatchInGemm1MaxT, 16);   // 64

template <int NRW>
__global__ __launch_bounds__(NRW == 8 ? 512 : 256) void gemm1_rstream_dispatch_kernel(
    RouteIn rin, int* __restrict__ topk_ids, float* __restrict__ topk_w, int T, int offset,
    const uint8_t* __restrict__ hidden, const float* __restrict__ hs_scale,
    const uint8_t* __restrict__ w1, const float* __restrict__ s1, int* __restrict__ meta,
    int4* __restrict__ tiles, int* __restrict__ sorted_tok, float* __restrict__ sorted_w,
    int* __restrict__ inv, Intermediate C) {
    using S = Gemm1Stream<1, 1, false>;
    constexpr int R = kDispatchInGemm1MaxT * kTopK;
    constexpr int NG = NRW == 8 ? 2 : 1;   // groups of 4 waves taking items
    __shared__ __attribute__((aligned(1024))) uint8_t slot_lds[4 * NG][S::kSlot];
    __shared__ v4f red[4 * NG][2][1][64];
    __shared__ int s_exp_off[kEL + 1];
    __shared__ int s_num_tiles;
    __shared__ int4 s_tiles[kDG1MaxTiles];
    __shared__ int s_stok[R];
    __shared__ int8_t s_lek[kDispatchInGemm1MaxT][kTopK];
    __shared__ float s_wk[kDispatchInGemm1MaxT][kTopK];
    __shared__ DispatchWaveLds s_dw;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const bool writer = blockIdx.x == gridDim.x - 1;
    MOE_STAMP(3 * (int)blockIdx.x);
    const int* ids_src = topk_ids;
    const float* w_src = topk_w;
    if constexpr (NRW > 0) {
        static_assert(NRW == 4 || NRW == 8, "one token per wave");
        static_assert(kRouteInGemm1MaxT <= 8, "at most 8 waves route");
        __shared__ __attribute__((aligned(16))) int s_rid[NRW][kTopK];
        __shared__ __attribute__((aligned(16))) float s_rw[NRW][kTopK];
        __shared__ float s_sel[NRW][kTopK];
        __shared__ int s_sel_id[NRW][kTopK];
        const int t = wave;
        if (t < T) {   // uniform per wave
            const float4 lg = reinterpret_cast<const float4*>(rin.logits + (size_t)t * kEG)[lane];
            const uint2 bb = reinterpret_cast<const uint2*>(rin.bias)[lane];
            int id;
            float w;
            route_token(lg, bb, lane, rin.factor, s_sel[wave], s_sel_id[wave], id, w);
            if (lane < kTopK) {
                s_rid[t][lane] = id;
                s_rw[t][lane] = w;
                if (writer) {
                    topk_ids[t * kTopK + lane] = id;
                    topk_w[t * kTopK + lane] = w;
                }
            }
        }
        __syncthreads();
        ids_src = &s_rid[0][0];
        w_src = &s_rw[0][0];
    }
    if (wave == 0) {
        const TokenRoutes r = load_routes(ids_src, w_src, lane, T, offset);
        wave_ballots(r, 0, lane, s_dw.wcnt, s_dw.bal);
#pragma unroll
        for (int k = 0; k < kTopK; ++k) {
            s_lek[lane][k] = (int8_t)r.lek[k];
            s_wk[lane][k] = r.wk[k];
        }
        __builtin_amdgcn_wave_barrier();
        write_offsets_and_tiles<16, 0>(lane < kEL ? s_dw.wcnt[0][lane] : 0, lane, s_dw.off,
                                       s_exp_off, &s_num_tiles, s_tiles, nullptr, nullptr);
    }
    __syncthreads();
    const int ntiles = s_num_tiles;
    if (wave < 4 && lane < T) {   // token lane: its routes 2 wave and 2 wave + 1
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int k = 2 * wave + kk;
            const int le = s_lek[lane][k];
            int row = -1;
            if (le >= 0) {
                const uint64_t b = s_dw.bal[le];
                row = s_exp_off[le] + (int)__builtin_amdgcn_mbcnt_hi(
                                          (uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
                s_stok[row] = lane;
                if (writer) {
                    sorted_tok[row] = lane;
                    sorted_w[row] = s_wk[lane][k];
                }
            }
            if (writer) inv[lane * kTopK + k] = row;
        }
    }
    if (writer) {
        for (int i = tid; i <= kEL; i += 256) meta[i] = s_exp_off[i];
        if (tid == 0) meta[kEL + 1] = ntiles;
        for (int i = tid; i < ntiles; i += 256) tiles[i] = s_tiles[i];
    }
    __syncthreads();
    MOE_STAMP(3 * (int)blockIdx.x + 1);
    const TokenScales sa{hs_scale, T, 0};
    const int nwork = ntiles * S::kItems;
    int* const c_wide = meta + kCWideFlag;
    if constexpr (NG == 2) {
        // group g takes the workgroup's items 2 i + g (items b, b + G, b + 2 G, ...)
        const int grp = wave >> 2, w4 = wave & 3;
        const int G = gridDim.x, b = blockIdx.x;
        const int mine = b < nwork ? (nwork - b + G - 1) / G : 0;
        for (int i = 0; i < (mine + 1) / 2; ++i) {
            const int k = 2 * i + grp;
            if (k < mine) {   // uniform per wave
                const int work = b + k * G;
                const int4 tile = s_tiles[work / S::kItems];
                gemm1_rstream_item<4, 1, 1, false>(hidden, sa, w1, s1, tile.x, tile.y, tile.z,
                                                   work % S::kItems, [&](int row) { return s_stok[row]; },
                                                   C, c_wide, &slot_lds[4 * grp], &red[4 * grp], w4);
            } else {
                __syncthreads();   // the two barriers of the item the other group runs
                __syncthreads();
            }
        }
    } else {
        for (int work = blockIdx.x; work < nwork; work += gridDim.x) {
            const int4 tile = s_tiles[work / S::kItems];
            gemm1_rstream_item<4, 1, 1, false>(hidden, sa, w1, s1, tile.x, tile.y, tile.z,
                                               work % S::kItems, [&](int row) { return s_stok[row]; },
                                               C, c_wide, slot_lds, red, wave);
        }
    }
    MOE_STAMP(3 * (int)blockIdx.x + 2);
}

// Epilogue of the prefill GEMM1 kernels: SwiGLU, then the fp8 hi/lo form of C.
// The wave holds 64 rows x 64 SwiGLU columns (acc[s][j]: j < 4 gate, j >= 4 up; lane
// holds D[col 16j + 4kq + v][row 16s + r16]); its partner wave (wn ^ 1) holds the other
// 64 columns of the 128-column block ng, so the row amax is combined across the two
// through LDS (xch, 2 KB, reusing the operand ring: every wave must have left the
// K loop, hence the first barrier).  Per row: s = amax/448 (1 for an all-zero row),
// hi = e4m3(c * 448/amax), lo = e4m3((c - hi*s) * 16*448/amax).
// A lane's 4 bytes of a row in each of the 4 column blocks are transposed across the
// row's 4 lanes (lanes l, l+16, l+32, l+48) with v_permlane32_swap / v_permlane16_swap,
// after which lane kq holds 16 consecutive bytes: one 16-byte store per form and row
// block instead of four 4-byte ones, each row's 64 bytes written by one instruction.
__device__ __forceinline__ void store_c_hilo(const v4f (&acc)[4][8], float* xch, int wm, int wn,
                                             int kq, int r16, int row0, int nrows, int ng,
                                             const Intermediate& C) {
    float c[4][4][4];
    float m[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        m[s] = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                c[s][j][v] = silu_f32(acc[s][j + 4][v]) * acc[s][j][v];
                m[s] = fmaxf(m[s], fabsf(c[s][j][v]));
            }
        m[s] = fmaxf(m[s], __shfl_xor(m[s], 16));
        m[s] = fmaxf(m[s], __shfl_xor(m[s], 32));
    }
    __syncthreads();
    if (kq == 0) {
#pragma unroll
        for (int s = 0; s < 4; ++s) xch[(wm * 2 + wn) * 64 + 16 * s + r16] = m[s];
    }
    __syncthreads();
    // 4 x 4 transpose of 32-bit words over the 16-lane rows of the wave (word j of row kq
    // -> word kq of row j): 32-lane then 16-lane swaps
    auto transpose4 = [](uint32_t (&w)[4]) {
        auto p = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
        w[0] = p[0]; w[2] = p[1];
        p = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
        w[1] = p[0]; w[3] = p[1];
        p = __builtin_amdgcn_permlane16_swap(w[0], w[1], false, false);
        w[0] = p[0]; w[1] = p[1];
        p = __builtin_amdgcn_permlane16_swap(w[2], w[3], false, false);
        w[2] = p[0]; w[3] = p[1];
    };
#pragma unroll
    for (int s = 0; s < 4; ++s) {
        const float amax = fmaxf(m[s], xch[(wm * 2 + (wn ^ 1)) * 64 + 16 * s + r16]);
        const int r = 64 * wm + 16 * s + r16;
        const float sc = amax > 0.f ? amax / 448.f : 1.f;
        const float inv = amax > 0.f ? 448.f / amax : 1.f;
        const float inv16 = inv * 16.f;
        uint32_t h[4], l[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float* x = c[s][j];
            h[j] = e4m3x4_from_f32(clamp448(x[0] * inv), clamp448(x[1] * inv),
                                   clamp448(x[2] * inv), clamp448(x[3] * inv));
            const auto h01 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h[j], false);
            const auto h23 = __builtin_amdgcn_cvt_pk_f32_fp8((int)h[j], true);
            const float hv[4] = {h01[0], h01[1], h23[0], h23[1]};
            float lq[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) lq[v] = clamp448(__builtin_fmaf(-hv[v], sc, x[v]) * inv16);
            l[j] = e4m3x4_from_f32(lq[0], lq[1], lq[2], lq[3]);
        }
        // every lane of the wave takes part in the swaps (the 4 lanes of a row share its
        // validity); lane kq then holds bytes 16 kq .. 16 kq + 15 of the wave's 64
        transpose4(h);
        transpose4(l);
        if (r >= nrows) continue;
        const size_t off = (size_t)(row0 + r) * kI + ng * 128 + 64 * wn + 16 * kq;
        *reinterpret_cast<v4u*>(C.hi() + off) = v4u{h[0], h[1], h[2], h[3]};
        *reinterpret_cast<v4u*>(C.lo() + off) = v4u{l[0], l[1], l[2], l[3]};
        if (wn == 0 && kq == 0) C.scales[(size_t)ng * C.rows_cap + row0 + r] = sc;
    }
}

// ---------------------------------------------------------------------------
// Prefill GEMM1 (many tokens per expert), MFMA-bound tiling: workgroup tile 256
// gathered token rows x 256 weight rows (128 gate rows n0..n0+127 and the matching
// 128 up rows 2048+n0.., i.e. 256 x 128 SwiGLU outputs), waves 4 (tokens) x 2
// (weights), each 64 tokens x (64 gate + 64 up) rows: per K block 32 MFMA 16x16x128
// (4 token blocks x 8 weight blocks) whose fresh partials are scaled by
// sa[token] * sb[block] into fp32 accumulators.  Two waves per SIMD let one wave's
// scale FMAs and LDS reads run under the other's MFMAs; registers stay <= 256 per
// lane for that.  Two 66 KB stages; rows keep 16-byte chunk c at c ^ swz128(r), so
// ds_read_b128 in the MFMA layout is conflict-free.  Padding row blocks skip their
// MFMAs.  Items (row tile, 128-column group) follow prefill_items_ranked when `ranked`
// is set, else grouped_item, with an XCD-contiguous mapping of each round.
//
// Operand DMA is buffer_load ... lds (addresses in SGPR resources, 32-bit lane
// offsets, the K step in the scalar offset), issued in two bursts per K block:
// the token rows right after the barrier, the weight rows and token scales after
// the third weight block's MFMAs, so the texture path is not flooded at once.
// Each weight operand is read from LDS one block ahead of its MFMAs, and each fresh
// partial is scaled into its accumulator only after the next weight block's MFMA of
// the same token block has issued (fixed order), so no FMA waits on its MFMA.
// A workgroup resolves the metadata of all its items at kernel start
// (prefill_items) and issues the first stage of its next item at the top of the
// current item's last K block; the epilogue's row-maximum exchange therefore uses
// stage 1, which the last K block reads.
// Token offsets are 32-bit: T * 7168 < 2^32 (T <= 2^19, checked by the host).
// ---------------------------------------------------------------------------
struct Gemm1Item {   // uniform part of an item; the per-lane DMA offsets live apart
    __amdgpu_buffer_rsrc_t w;
    int le, row0, nrows, ng;
    bool tok_live, sca_live;
};

__global__ __launch_bounds__(512, 1) void gemm1_prefill8_kernel(
    const uint8_t* __restrict__ hidden, TokenScales sa, int T,
    const uint8_t* __restrict__ w1, const float* __restrict__ s1,
    const int4* __restrict__ tiles, const int* __restrict__ num_tiles,
    const int* __restrict__ exp_off, const int* __restrict__ sorted_tok, Intermediate C, int ranked) {
    constexpr int NS = 2;
    constexpr int BM = 256;
    constexpr int NG = kI / 128;
    constexpr int kA = BM * kBlk;               // 32 KB token rows
    constexpr int kW = 256 * kBlk;              // 32 KB weight rows
    constexpr int kStage = kA + kW + 8 * 256;   // + per-wave token-scale rows
    constexpr int kWeightBurstAfter = 2;        // weight block after which burst 2 goes
    constexpr int kItemCap = 1024;              // per-workgroup item table (16 KB of LDS)
    static_assert(kHB % 2 == 0, "the next item's first stage must be stage 0");
    // one LDS object: the stages, then the item table
    __shared__ __attribute__((aligned(1024))) uint8_t lds[NS * kStage + kItemCap * sizeof(int4)];
    int4* const s_items = reinterpret_cast<int4*>(lds + NS * kStage);

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    const int wm = wave >> 1, wn = wave & 1;
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
    const int nitems = *num_tiles * NG;
    const int G = gridDim.x;
    const int base = (blockIdx.x & 7) * (G >> 3) + (blockIdx.x >> 3);   // XCD-contiguous slot
    const int drow = lane >> 3, dchunk = lane & 7;
    const int swz = swz128(r16);
    const int c0 = ((2 * kq) ^ swz) << 4, c1 = ((2 * kq + 1) ^ swz) << 4;
    const __amdgpu_buffer_rsrc_t rs_tok = buffer_rsrc(hidden, (uint32_t)T * kH);
    const __amdgpu_buffer_rsrc_t rs_sca = buffer_rsrc(sa.p, (uint32_t)sa.stride * kHB * 4);
    // wave w moves token rows 32w..32w+31 and weight rows 32w..32w+31 of the stage; the
    // weight rows' lane offsets are relative to the item's first gate row (the resource
    // base), so they do not depend on the item
    uint32_t woff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 32 * wave + 8 * i + drow;
        const int n = (r < 128) ? r : kI + (r - 128);
        woff[i] = (uint32_t)n * kH + ((dchunk ^ swz128(r)) << 4);
    }

    static_assert(kRankThreads == 512 && kRankScratch <= NS * kStage, "ranked order: threads, scratch");
    int nr = ranked ? prefill_items_ranked<BM>(s_items, kItemCap, NG, base, G, exp_off, lds) : -1;
    if (nr < 0) nr = prefill_items<BM>(s_items, kItemCap, nitems, NG, base, G, tiles, exp_off);
    if (nr == 0) return;   // uniform: the whole workgroup has no item
    __syncthreads();

    // token-row and token-scale offsets of the item whose stages are being fetched
    uint32_t aoff[4], soff;
    auto make_item = [&](int r) {
        const int4 m = prefill_item<BM>(s_items, kItemCap, r, NG, base, G, tiles, exp_off);
        Gemm1Item it;
        it.le = m.x;
        it.row0 = m.y;
        it.nrows = m.z;
        it.ng = m.w;
        const size_t first = (size_t)it.le * kN1 + (size_t)it.ng * 128;
        it.w = buffer_rsrc(w1 + first * kH, (uint32_t)(((size_t)(it.le + 1) * kN1 - first) * kH));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = 32 * wave + 8 * i + drow;
            const int tok = sorted_tok[it.row0 + min(r, it.nrows - 1)];
            aoff[i] = (uint32_t)tok * kH + ((dchunk ^ swz128(r)) << 4);
        }
        const int srow = it.row0 + min(64 * wm + lane, it.nrows - 1);
        soff = (uint32_t)(sa.by_row ? srow : sorted_tok[srow]) * 4;
        // a wave whose 32 token rows all lie past the tile moves nothing: they would only
        // repeat the last row, and the MFMAs of their 16-row blocks are skipped
        it.tok_live = 32 * wave < it.nrows;
        it.sca_live = 64 * wm < it.nrows;
        return it;
    };
    auto issue_tokens = [&](const Gemm1Item& it, int kb) {
        uint8_t* st = lds + (kb & 1) * kStage;
        if (it.tok_live) {
#pragma unroll
            for (int i = 0; i < 4; ++i) bdma16(rs_tok, aoff[i], (uint32_t)kb * kBlk, st + (32 * wave + 8 * i) * kBlk);
        }
    };
    auto issue_weights = [&](const Gemm1Item& it, int kb) {
        uint8_t* st = lds + (kb & 1) * kStage;
#pragma unroll
        for (int i = 0; i < 4; ++i) bdma16(it.w, woff[i], (uint32_t)kb * kBlk, st + kA + (32 * wave + 8 * i) * kBlk);
        if (it.sca_live) bdma4(rs_sca, soff, (uint32_t)kb * sa.stride * 4, st + kA + kW + wave * 256);
    };

    Gemm1Item cur = make_item(0), nxt = cur;
    issue_tokens(cur, 0);
    issue_weights(cur, 0);
    for (int r = 0; r < nr; ++r) {
        const bool more = r + 1 < nr;
        // weight block scales of the gate and up rows (scalar loads from the kernel argument)
        const float* sgp = s1 + (size_t)(cur.le * kN1B + cur.ng) * kHB;
        const float* sup = sgp + (size_t)kIB * kHB;
        v4f acc[4][8];
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[s][j] = zero;

        // token rows 64 wm + 16 s .. of this wave that exist: the MFMAs of padding
        // blocks are skipped (the DMA and barriers stay the same for every wave)
        auto kloop = [&](auto live) {
        constexpr int NLIVE = decltype(live)::value;
        constexpr int NT = NLIVE > 0 ? NLIVE : 1;
#pragma unroll 1
        for (int kb = 0; kb < kHB; ++kb) {
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            __syncthreads();
            if (kb + 1 < kHB) {
                issue_tokens(cur, kb + 1);
                if (kWeightBurstAfter < 0 || NLIVE == 0) issue_weights(cur, kb + 1);
            } else if (more) {
                // stage 0 is free (every wave is past K block kHB - 2): the next item's first stage
                nxt = make_item(r + 1);
                issue_tokens(nxt, 0);
                issue_weights(nxt, 0);
            }
            __builtin_amdgcn_sched_barrier(0);
            if (NLIVE == 0) continue;

            const uint8_t* st = lds + (kb & 1) * kStage;
            const float fsg = sgp[kb], fsu = sup[kb];
            const float* sar = reinterpret_cast<const float*>(st + kA + kW + wave * 256);
            v8i bt[4];
            float fg[4], fu[4];
#pragma unroll
            for (int s = 0; s < NLIVE; ++s) {
                const uint8_t* rp = st + (64 * wm + 16 * s + r16) * kBlk;
                const v4u x0 = *reinterpret_cast<const v4u*>(rp + c0);
                const v4u x1 = *reinterpret_cast<const v4u*>(rp + c1);
                bt[s] = v8i{(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3], (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
                const float sa = sar[16 * s + r16];
                fg[s] = sa * fsg;
                fu[s] = sa * fsu;
            }
            auto read_w = [&](int j) {
                const int r = (j < 4) ? (64 * wn + 16 * j) : (128 + 64 * wn + 16 * (j - 4));
                const uint8_t* rp = st + kA + (r + r16) * kBlk;
                const v4u x0 = *reinterpret_cast<const v4u*>(rp + c0);
                const v4u x1 = *reinterpret_cast<const v4u*>(rp + c1);
                return v8i{(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3], (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
            };
            v8i bw = read_w(0);
            v4f tp[NT];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                v8i bwn = bw;
                if (j < 7) bwn = read_w(j + 1);
                if (j == kWeightBurstAfter && kb + 1 < kHB) {
                    __builtin_amdgcn_sched_barrier(0);
                    issue_weights(cur, kb + 1);
                }
#pragma unroll
                for (int s = 0; s < NLIVE; ++s) {
                    __builtin_amdgcn_sched_barrier(0);
                    const v4f tc = mfma_fp8(bw, bt[s], zero);
                    __builtin_amdgcn_sched_barrier(0);
                    if (j > 0) {
                        const float f = (j - 1 < 4) ? fg[s] : fu[s];
#pragma unroll
                        for (int v = 0; v < 4; ++v) acc[s][j - 1][v] = __builtin_fmaf(tp[s][v], f, acc[s][j - 1][v]);
                    }
                    tp[s] = tc;
                }
                bw = bwn;
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int s = 0; s < NLIVE; ++s)
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[s][7][v] = __builtin_fmaf(tp[s][v], fu[s], acc[s][7][v]);
        }
        };
        with_live_blocks(live_blocks(64 * wm, cur.nrows), kloop);

        // the next item's first stage is landing in stage 0: the exchange uses stage 1
        store_c_hilo(acc, reinterpret_cast<float*>(lds + kStage), wm, wn, kq, r16, cur.row0, cur.nrows,
                     cur.ng, C);
        cur = nxt;
    }
}

static int grid_for(long long work) { return (int)(work < 4096 ? work : 4096); }

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_dg1_mu;
int g_dg1_grid[3][kMaxDevices] = {};
}  // namespace

// GEMM1 with the dispatch folded in (and with rin.logits set, T <= kRouteInGemm1MaxT, the
// routing too): a persistent grid of as many workgroups as the device holds at once
// (occupancy x CUs, looked up once per device and kernel; with the 8-wave routing of
// 5 <= T <= 8, one per CU, so that a SIMD routes two tokens, not six), capped by the most
// work items T tokens can have.  Without the routing, topk_ids / topk_w hold the routing;
// with it, the kernel writes them.  It sets the C-range flag word when C goes beyond the
// fp16 range (cleared by the route kernel, or with the routing not cleared at all).
bool launch_gemm1_dispatch(const RouteIn& rin, int* topk_ids, float* topk_w, int T, int offset,
                           const uint8_t* hidden, const float* hs_scale, const uint8_t* w1,
                           const float* s1, int* meta, int4* tiles, int* sorted_tok,
                           float* sorted_w, int* inv, const Intermediate& C,
                           hipStream_t stream) {
    const bool route = rin.logits != nullptr;
    if (T <= 0 || T > (route ? kRouteInGemm1MaxT : kDispatchInGemm1MaxT)) return false;
    if (route && rin.bias == nullptr) return false;
    const int nrw = route ? (T <= 4 ? 4 : 8) : 0;   // routing waves
    const int kind = nrw / 4;                        // 0, 1, 2
    const void* fn = nrw == 8 ? reinterpret_cast<const void*>(gemm1_rstream_dispatch_kernel<8>)
                   : nrw == 4 ? reinterpret_cast<const void*>(gemm1_rstream_dispatch_kernel<4>)
                              : reinterpret_cast<const void*>(gemm1_rstream_dispatch_kernel<0>);
    const int threads = nrw == 8 ? 512 : 256;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
    int resident = 0;
    {
        std::lock_guard<std::mutex> lock(g_dg1_mu);
        int& g = g_dg1_grid[kind][dev];
        if (g == 0) {
            int per_cu = 0, cus = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, threads, 0) != hipSuccess ||
                hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
                per_cu * cus <= 0)
                return false;
            g = nrw == 8 ? cus : per_cu * cus;
        }
        resident = g;
    }
    const long long items = (long long)(((long long)T * kTopK + 15) / 16 + kEL) * Gemm1Stream<1, 1, false>::kItems;
    const int grid = (int)(items < resident ? items : resident);
    if (nrw == 8)
        launch_kernel(gemm1_rstream_dispatch_kernel<8>, dim3(grid), dim3(512), 0, stream, rin,
                      topk_ids, topk_w, T, offset, hidden, hs_scale, w1, s1, meta, tiles,
                      sorted_tok, sorted_w, inv, C);
    else if (nrw == 4)
        launch_kernel(gemm1_rstream_dispatch_kernel<4>, dim3(grid), dim3(256), 0, stream, rin,
                      topk_ids, topk_w, T, offset, hidden, hs_scale, w1, s1, meta, tiles,
                      sorted_tok, sorted_w, inv, C);
    else
        launch_kernel(gemm1_rstream_dispatch_kernel<0>, dim3(grid), dim3(256), 0, stream, rin,
                      topk_ids, topk_w, T, offset, hidden, hs_scale, w1, s1, meta, tiles,
                      sorted_tok, sorted_w, inv, C);
    return true;
}

// Variants (the tile height of the dispatch they expect, and the form of C they write):
//   1  register-staged streaming, 1 row block per item    16-row tiles   fp16 (+ exponents)
//   2  register-staged, 2 row blocks x 2 column groups   32-row tiles   fp16 (+ exponents)
//   4  prefill, 8 waves, 256 x 256 workgroup tile        256-row tiles  fp8 hi/lo
//   7  register-staged weights, token rows shared in LDS  64-row tiles   fp16 (+ exponents)
//   8  variant 7 with three workgroups per CU (more loads in flight, more L2 pressure)
// (variant 5, the dispatch folded into variant 1, has its own launcher)
bool launch_gemm1(int variant, const uint8_t* hidden, const TokenScales& sa, int T,
                  const uint8_t* w1, const float* s1, const int4* tiles, const int* num_tiles,
                  const int* exp_off, int max_tiles, const int* sorted_tok, const Intermediate& C,
                  bool ranked, hipStream_t stream) {
    int* c_wide = const_cast<int*>(exp_off) + kCWideFlag;   // meta word, cleared by the route kernel
    const int prefill_grid = 256;   // one resident workgroup per CU (LDS-bound)
    constexpr int G = kI / 16;      // 16-column groups
    const long long mt = max_tiles;
    switch (variant) {
        case 1:
            launch_kernel((gemm1_rstream_kernel<4, 1, 1, false>), dim3(grid_for(mt * G)), dim3(256), 0, stream,
                               hidden, sa, T, w1, s1, tiles, num_tiles, sorted_tok, C, c_wide);
            return true;
        case 2:
            launch_kernel((gemm1_rstream_kernel<2, 2, 2, true>), dim3(grid_for(mt * G / 2)), dim3(256), 0, stream,
                               hidden, sa, T, w1, s1, tiles, num_tiles, sorted_tok, C, c_wide);
            return true;
        case 7: {   // 4-wave workgroups, two resident per CU (registers)
            const long long items = mt * Gemm1Shared<2, 4>::kItems;
            launch_kernel((gemm1_shared_kernel<2, 4, 1>), dim3((int)(items < 768 ? items : 768)), dim3(256), 0,
                               stream, hidden, sa, T, w1, s1, tiles, num_tiles, sorted_tok, C, c_wide);
            return true;
        }
        case 8: {   // the same held to three resident per CU
            const long long items = mt * Gemm1Shared<2, 4>::kItems;
            launch_kernel((gemm1_shared_kernel<2, 4, 3>), dim3((int)(items < 768 ? items : 768)), dim3(256), 0,
                               stream, hidden, sa, T, w1, s1, tiles, num_tiles, sorted_tok, C, c_wide);
            return true;
        }
        case 4:
            launch_kernel(gemm1_prefill8_kernel, dim3(prefill_grid), dim3(512), 0, stream,
                               hidden, sa, T, w1, s1, tiles, num_tiles, exp_off, sorted_tok, C,
                               ranked ? 1 : 0);
            return true;
        default: return false;
    }
}

}  // namespace moe
