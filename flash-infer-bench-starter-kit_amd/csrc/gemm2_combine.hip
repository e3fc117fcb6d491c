// gemm2_combine.hip -- GEMM2 with the combine folded in, for a few tokens (decode).
//
// Semantics: reference solution/cuda/moe.cu:231-239 (O = C @ W2[e]^T per expert, then
// output[t] = sum over the token's local experts, ascending, of O * w in fp32 and one
// bf16 rounding), which the separate kernels compute as gemm2_rstream_kernel<4, 4, 2, 1>
// (gemm2.hip) followed by combine_kernel (combine.hip).  This kernel gives the same
// output bit for bit: the same K split, partial sums added in the same order, each
// expert row rounded to the same fp16 form (group exponents included), and the same
// ordered fp32 combine; only the expert rows stay in LDS instead of HBM.
//
// Work split: a workgroup owns 32 output columns (two groups of 16) of every row tile of
// the call, so it holds every expert row of the call for those columns and can combine
// them itself; the combine launch and its dependent loads of the rows go away.  Each of
// the 4 waves takes 4 of the 16 K blocks of every tile, one continuous stream of
// (tile, K block) steps through a register ring of 4 steps (W2 bytes as full-line loads,
// moved to the MFMA layout through the wave's LDS slot, and fp16 C fragments), so the
// loads of the next tile are in flight while this one computes.  After every 4 tiles the
// waves add the 4 K partials of a tile each (waves 0, 1, 2, 3 in that order) and keep
// the rows in LDS.  The token's routing weights, the inverse row map and the tile list
// come in by LDS DMA at kernel start, and each step's W2 block scale with the step's
// loads, so the loop issues no scalar load (an LDS access waits for every scalar load
// in flight, as both count on one counter).  224 workgroups stream the same bytes per CU as the separate GEMM2
// (448 items of 32 columns over 256 CUs); the LDS holds the rows of up to
// kFusedCombineMaxT tokens.  Two groups of 4 waves take alternate tiles, so the
// workgroup has as many waves in flight as two of the separate GEMM2's.

#include "combine_rows.h"
#include "gemm2_stream.h"

MOE_STAMP_TABLE(gemm2_combine)

namespace moe {

constexpr int kFusedRows = kFusedCombineMaxT * kTopK;        // expert rows in LDS
constexpr int kFusedCols = 32;                                // output columns per workgroup

// NG groups of 4 waves (64 NG threads x 4): group g takes tiles g, g + NG, g + 2 NG, ...,
// wave ks of a group K blocks 4 ks .. 4 ks + 3 of each, so every wave's partial of a
// tile is the one the separate GEMM2's wave ks computes.
template <int NG>
__global__ __launch_bounds__(256 * NG, 1) void gemm2_combine_kernel(
    Intermediate C, int* __restrict__ flags, const uint8_t* __restrict__ w2,
    const float* __restrict__ s2, const int4* __restrict__ tiles,
    const int* __restrict__ num_tiles, const int* __restrict__ inv,
    const float* __restrict__ sorted_w, int T, uint16_t* __restrict__ out) {
    constexpr int HF = 2, KSPLIT = 4, KB = kIB / KSPLIT, D = KB;
    constexpr int NW = KSPLIT * NG;           // waves
    constexpr int CH = 4 * NG;                // tiles per reduction round (4 per group)
    constexpr int kVmPerStep = 2 * HF + 5;    // W2 loads, C loads, block scale of one (tile, K block)
    static_assert(HF == 2, "the HF column groups of a workgroup share one W2 scale block");
    // flags[0]: C went beyond the fp16 range, when zero certainly not (GEMM1 sets it, and
    // with a route kernel before it, that kernel clears it; without one a nonzero word may
    // be stale and is checked against C's group exponents); flags[1]: an expert row went
    // beyond the range (set here; nothing after this kernel reads it).
    __shared__ __attribute__((aligned(1024))) uint8_t slot_lds[NW][16 * HF * kBlk];
    __shared__ v4f red[KSPLIT][CH][HF][64];          // K partials of one round of tiles
    __shared__ float o_lds[kFusedRows][kFusedCols];  // expert rows (as the combine reads them)
    __shared__ int s_inv[kFusedRows];
    __shared__ float s_w[kFusedRows];
    __shared__ int4 s_tiles[64];
    __shared__ int s_beyond[NW];                     // a wave read a nonzero group exponent
    __shared__ int s_flag;                           // flags[0] as this workgroup read it

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int ks = wave % KSPLIT, grp = wave / KSPLIT;
    const int r16 = lane & 15, kq = lane >> 4;
    const int drow = lane >> 3, dchunk = lane & 7;
    const int hg = blockIdx.x * HF;                  // first 16-column group
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
    const int R = T * kTopK;
    MOE_STAMP(2 * (int)blockIdx.x);

    // Straight into LDS: the routing weights of the rows and the inverse map (read by
    // the combine at the end; the waits of the K loop or the barrier before the combine
    // cover them), and the whole tile list as far as the workspace holds it (the last
    // wave; waited for below).  A tile read from LDS keeps the K loop free of scalar
    // loads, whose completion every LDS access after them would wait for.
    {
        const __amdgpu_buffer_rsrc_t rs_inv = buffer_rsrc(inv, (uint32_t)R * 4);
        const __amdgpu_buffer_rsrc_t rs_w = buffer_rsrc(sorted_w, (uint32_t)R * 4);
        for (int b = 64 * wave; b < kFusedRows; b += 64 * NW) {   // uniform per wave
            bdma4(rs_inv, (uint32_t)(b + lane) * 4, 0, s_inv + b);
            bdma4(rs_w, (uint32_t)(b + lane) * 4, 0, s_w + b);
        }
        if (wave == NW - 1) {
            const __amdgpu_buffer_rsrc_t rs_t = buffer_rsrc(tiles, (uint32_t)dispatch_max_tiles(T, 16) * 16);
            bdma16(rs_t, (uint32_t)lane * 16, 0, s_tiles);
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
        }
    }
    const int nt = __builtin_amdgcn_readfirstlane(*num_tiles);
    // flags[0] is read once for the workgroup: another workgroup may clear it (below)
    // between two waves' reads, and the waves must all take the same branch (barriers)
    if (wave == 0) {
        const int f = __builtin_amdgcn_readfirstlane(flags[0]);
        if (lane == 0) s_flag = f;
    }
    __syncthreads();   // the tile list and the flag word are in LDS
    const int c_flag = __builtin_amdgcn_readfirstlane(s_flag);

    // A nonzero flag word is checked against C's group exponents of every row in the
    // tiles (GEMM1 writes each one on every call): wave (grp, ks) reads bytes 32 ks ..
    // 32 ks + 31 of rows 64 i + 32 grp + lane / 2, in 16-byte halves, so the 8 waves cover
    // every exponent; rows past the last tile read 0.  A word the check finds stale is
    // cleared (a workgroup that reads it cleared takes the usual path, as the check would
    // have sent it there).
    bool beyond = false;
    if (c_flag != 0) {
        static_assert(NG == 2 && kFusedRows % 64 == 0, "exponent rows: 32 per wave and load");
        const int4 last = nt > 0 ? s_tiles[nt - 1] : int4{0, 0, 0, 0};
        const uint32_t rows = (uint32_t)__builtin_amdgcn_readfirstlane(last.y + last.z);
        const __amdgpu_buffer_rsrc_t rs_ex = buffer_rsrc(C.f16_exp(), rows * (kI / kGroup16));
        uint32_t ex = 0;
#pragma unroll
        for (int i = 0; i < kFusedRows / 64; ++i) {
            const uint32_t row = 64 * i + 32 * grp + (lane >> 1);
            const v4u e = __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(
                rs_ex, row * (kI / kGroup16) + 32 * ks + 16 * (lane & 1), 0, 0));
            ex |= e[0] | e[1] | e[2] | e[3];
        }
        const bool mine = __ballot(ex != 0) != 0;
        if (lane == 0) s_beyond[wave] = mine;
        __syncthreads();
#pragma unroll
        for (int w = 0; w < NW; ++w) beyond = beyond || s_beyond[w] != 0;
        if (!beyond && tid == 0) flags[0] = 0;
    }

    // tile t: local expert, first row, rows
    auto tile_of = [&](int t) {
        const int4 tl = s_tiles[t];
        return int4{__builtin_amdgcn_readfirstlane(tl.x), __builtin_amdgcn_readfirstlane(tl.y),
                    __builtin_amdgcn_readfirstlane(tl.z), 0};
    };

    // After the K partials of tiles c0 .. c0 + CH - 1 (those below nt) are in red: wave w
    // adds the 4 partials of tile c0 + w in wave order (ks = 0, 1, 2, 3) and keeps the
    // row values in o_lds in the fp16 form of store_rows4, read back as combine_token8
    // reads it.
    bool any_e = false;
    auto reduce_round = [&](int c0) {
        lds_barrier();
        const int t = c0 + wave;
        if (t < nt) {   // uniform per wave
            const int4 tl = tile_of(t);
            const bool valid = r16 < tl.z;
#pragma unroll
            for (int hf = 0; hf < HF; ++hf) {
                v4f o = red[0][wave][hf][lane];
#pragma unroll
                for (int q = 1; q < KSPLIT; ++q) o += red[q][wave][hf][lane];
                const float x[4] = {o[0], o[1], o[2], o[3]};
                const float m = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
                int e = 0;
                if (beyond_f16_in_wave(m)) e = group_exponent(m);
                if (valid) {
                    float* dst = &o_lds[tl.y + r16][hf * 16 + kq * 4];
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)(e ? ldexpf(x[v], -e) : x[v]));
                        dst[v] = f16_scaled_to_f32(h, e);
                    }
                    any_e = any_e || e != 0;
                }
            }
        }
        lds_barrier();
    };

    // this group's tiles: grp + NG i for i < nt_g; every wave runs imax rounds of i (the
    // reduction barriers), a group without a tile at some i only waits there
    const int imax = (nt + NG - 1) / NG;
    const int nt_g = (nt - grp + NG - 1) / NG;
    if (!beyond) {   // the usual path: C within the fp16 range (every group exponent 0)
        // ---- the stream of (tile, K block) steps of this wave: step 4 i + j is tile
        // grp + NG i, K block 4 ks + j, held in ring slot j
        uint8_t* slot = &slot_lds[wave][0];
        const int swz = swz128(r16);
        const int rd0 = r16 * kBlk + (((2 * kq) ^ swz) << 4);
        const int rd1 = r16 * kBlk + (((2 * kq + 1) ^ swz) << 4);
        int wr[2 * HF];
#pragma unroll
        for (int i = 0; i < 2 * HF; ++i) {
            const int r = 8 * i + drow;
            wr[i] = r * kBlk + ((dchunk ^ swz128(r)) << 4);
        }
        v4u bw[D][2 * HF];
        v4u bc[D][4];
        float bsc[D];
        // the W2 block scale of a step comes with its loads (a vector load: it is waited
        // for with them), so the loop reads no scale through the scalar cache
        const __amdgpu_buffer_rsrc_t rs_s2 = buffer_rsrc(s2, (uint32_t)(kEL * kHB * kIB * 4));
        auto issue = [&](const int4& tl, int j) {   // tile tl, K block 4 ks + j -> slot j
            const int kb = ks * KB + j;
#pragma unroll
            for (int i = 0; i < 2 * HF; ++i) {
                const uint8_t* src = w2 + (size_t)(tl.x * kH + hg * 16 + 8 * i + drow) * kI + dchunk * 16;
                bw[j][i] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(src + kb * kBlk));
            }
            const uint8_t* cp = reinterpret_cast<const uint8_t*>(C.f16() + (size_t)(tl.y + min(r16, tl.z - 1)) * kI) + kq * 64;
#pragma unroll
            for (int q = 0; q < 4; ++q) bc[j][q] = *reinterpret_cast<const v4u*>(cp + kb * 2 * kBlk + 16 * q);
            bsc[j] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                rs_s2, (uint32_t)(((tl.x * kHB + (hg >> 3)) * kIB + kb) * 4), 0, 0));
        };
        const int nsteps = nt_g * D;
        int4 cur = nt_g > 0 ? tile_of(grp) : int4{0, 0, 1, 0};
        if (nt_g > 0) {
#pragma unroll
            for (int j = 0; j < D - 1; ++j) {
                issue(cur, j);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
#pragma unroll 1
        for (int i = 0; i < imax; ++i) {
            if (i < nt_g) {   // uniform per wave
                const int4 nxt = i + 1 < nt_g ? tile_of(grp + NG * (i + 1)) : cur;
                v4f acc[HF] = {zero, zero};
#pragma unroll
                for (int j = 0; j < D; ++j) {
                    const int s = D * i + j;
                    // step s + D - 1 into the slot step s - 1 used
                    if (s + D - 1 < nsteps) issue(j == 0 ? cur : nxt, (j + D - 1) % D);
                    __builtin_amdgcn_sched_barrier(0);
                    switch (min(nsteps - 1 - s, D - 1)) {   // steps younger than s still in flight
                        case 0: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
                        case 1: __builtin_amdgcn_s_waitcnt(vmcnt_imm(1 * kVmPerStep)); break;
                        case 2: __builtin_amdgcn_s_waitcnt(vmcnt_imm(2 * kVmPerStep)); break;
                        default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(3 * kVmPerStep)); break;
                    }
                    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                    for (int q = 0; q < 2 * HF; ++q) *reinterpret_cast<v4u*>(slot + wr[q]) = bw[j][q];
#pragma unroll
                    for (int hf = 0; hf < HF; ++hf) {
                        const v4u x0 = *reinterpret_cast<const v4u*>(slot + hf * 16 * kBlk + rd0);
                        const v4u x1 = *reinterpret_cast<const v4u*>(slot + hf * 16 * kBlk + rd1);
                        const uint32_t ww[8] = {x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
                        v4f tp = zero;
#pragma unroll
                        for (int q = 0; q < 4; ++q) tp = mfma_w2_c<true>(ww[2 * q], ww[2 * q + 1], bc[j][q], tp);
#pragma unroll
                        for (int v = 0; v < 4; ++v) acc[hf][v] = __builtin_fmaf(tp[v], bsc[j], acc[hf][v]);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                const int slot_t = grp + NG * (i & 3);          // tile index inside the round
#pragma unroll
                for (int hf = 0; hf < HF; ++hf) red[ks][slot_t][hf][lane] = acc[hf];
                cur = nxt;
            }
            if ((i & 3) == 3 || i == imax - 1) reduce_round(CH * (i >> 2));
        }
    } else {
        // ---- C went beyond the fp16 range: the rare path, one tile at a time per group
#pragma unroll 1
        for (int i = 0; i < imax; ++i) {
            if (i < nt_g) {
                const int4 tl = tile_of(grp + NG * i);
                v4f acc[HF][1];
                gemm2_rare_partial<KSPLIT, HF, 1>(C.f16(), C.f16_exp(), w2, s2, tl.x, tl.y, tl.z, hg, ks, acc);
#pragma unroll
                for (int hf = 0; hf < HF; ++hf) red[ks][grp + NG * (i & 3)][hf][lane] = acc[hf][0];
            }
            if ((i & 3) == 3 || i == imax - 1) reduce_round(CH * (i >> 2));
        }
    }
    if (any_e) flags[1] = 1;   // an expert row went beyond the fp16 range
    __syncthreads();             // every row in o_lds, the routing tables landed

    // ---- the combine of the workgroup's 32 columns: thread (token t, column pair p),
    // the token's rows in ascending order, o * w added in fp32, one bf16 rounding
    // (combine_token8's arithmetic, bit for bit)
    for (int i = tid; i < T * (kFusedCols / 2); i += 256 * NG) {
#pragma clang fp contract(off)
        const int t = i / (kFusedCols / 2), p = i % (kFusedCols / 2);
        int r[kTopK];
#pragma unroll
        for (int k = 0; k < kTopK; ++k) {
            const int v = s_inv[t * kTopK + k];
            r[k] = v < 0 ? 0x7fffffff : v;
        }
        cswap(r[0], r[1]); cswap(r[2], r[3]); cswap(r[4], r[5]); cswap(r[6], r[7]);
        cswap(r[0], r[2]); cswap(r[1], r[3]); cswap(r[4], r[6]); cswap(r[5], r[7]);
        cswap(r[1], r[2]); cswap(r[5], r[6]); cswap(r[0], r[4]); cswap(r[3], r[7]);
        cswap(r[1], r[5]); cswap(r[2], r[6]);
        cswap(r[1], r[4]); cswap(r[3], r[6]);
        cswap(r[2], r[4]); cswap(r[3], r[5]);
        cswap(r[3], r[4]);
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int k = 0; k < kTopK; ++k) {
            if (r[k] == 0x7fffffff) break;
            const float w = s_w[r[k]];
            const float p0 = o_lds[r[k]][2 * p] * w, p1 = o_lds[r[k]][2 * p + 1] * w;
            a0 = a0 + p0;
            a1 = a1 + p1;
        }
        *reinterpret_cast<uint32_t*>(out + (size_t)t * kH + blockIdx.x * kFusedCols + 2 * p) =
            f32_to_bf16_bits(a0) | (f32_to_bf16_bits(a1) << 16);
    }
    MOE_STAMP(2 * (int)blockIdx.x + 1);
}

// GEMM2 variant 6: the streaming GEMM2 of variant 1 (16-row tiles, fp16 C) with the
// combine folded in, for T <= kFusedCombineMaxT; writes the bf16 output itself.  C went
// beyond the fp16 range when the C-range flag word is set and C's group exponents confirm
// it (GEMM1 variant 9 sets the word, but no route kernel clears it before).
bool launch_gemm2_combine(const Intermediate& C, const uint8_t* w2, const float* s2,
                          const int4* tiles, const int* num_tiles, int* meta, const int* inv,
                          const float* sorted_w, int T, uint16_t* out, hipStream_t stream) {
    if (T <= 0 || T > kFusedCombineMaxT) return false;
    launch_kernel((gemm2_combine_kernel<2>), dim3(kH / kFusedCols), dim3(512), 0, stream, C,
                  meta + kCWideFlag, w2, s2, tiles, num_tiles, inv, sorted_w, T, out);
    return true;
}

}  // namespace moe
