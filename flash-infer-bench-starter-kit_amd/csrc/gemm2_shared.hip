// gemm2_shared.hip -- GEMM2 for mid-size T with the row tile's C rows shared by the
// workgroup: the counterpart of the token-sharing GEMM1 (gemm1_shared_kernel, gemm1.hip),
// which writes the fp16 C rows this kernel reads, over the same 64-row tile list.
//
// Semantics: reference solution/cuda/moe.cu:231 (O = C @ W2[e]^T) with the 128x128 block
// scales of gemm2_weights_scale applied per K block in the fp32 accumulator, as the
// streaming GEMM2 (gemm2.hip) computes it: W2 e4m3 bytes widened exactly to fp16,
// v_mfma_f32_16x16x32_f16 against the fp16 C rows, each K block's fresh partial scaled into
// the accumulator in K order; expert rows to the combine in the fp16 row form.
//
// Work item: one row tile of up to 64 rows x 128 output columns (one W2 scale block).  Each
// of the 4 waves owns 32 of the columns (two groups of 16 W2 rows) over all 16 K blocks,
// so there is no cross-wave reduction.  The W2 bytes stream HBM -> VGPR through a ring of
// D K blocks (full-line loads, moved to the MFMA layout through the wave's LDS slot, as
// in the streaming kernels), together with the K block's W2 scale (a vector load, so the
// K loop issues no scalar load that an LDS access would wait for).  The tile's C rows of
// a K block (64 rows x 256 bytes of fp16) come once for the whole workgroup by
// buffer_load ... lds into a ring of D + 1 stages (wave w moves rows 16 w .. 16 w + 15;
// a 16-row block past the tile moves nothing and its MFMAs are skipped); one barrier per
// K block hands a stage over.  In a stage, row r keeps its 16-byte chunk c at position
// c ^ (r mod 16), so the 16 rows an MFMA operand read touches land on 16 different bank
// groups.  It reads C in the fp16 form the token-sharing GEMM1 writes, so the fp16 ->
// hi/lo conversion launch of the prefill GEMM2 goes away, and it has two workgroups per CU
// (212 registers, 64 KB of LDS) where the prefill GEMM2 has one.  Measured against that
// pair it is faster while the tiles hold few rows (T = 200 .. 559, the plan there) and
// slower beyond, where it moves about as much C per item as W2 at a similar per-CU rate.
// When GEMM1 flagged C beyond the fp16 range, each wave computes its columns on the rare
// path of the streaming GEMM2 (bf16 MFMAs on C rebuilt from its group exponents), one
// 16-row block at a time.

#include "gemm2_stream.h"

#include <mutex>

namespace moe {

template <int D, int HF>
struct Gemm2Shared {
    static constexpr int NWV = 4;                          // waves per workgroup
    static constexpr int kSlot = 16 * HF * kBlk;           // a wave's W2 transpose slot
    static constexpr int kRow = 2 * kBlk;                  // bytes of a C row per K block
    static constexpr int kCStage = 64 * kRow;              // 64 C rows
    static constexpr int kStages = D + 1;
    static constexpr int kLds = NWV * kSlot + kStages * kCStage;
    static constexpr int kCols = 16 * HF * NWV;            // output columns per item
    static constexpr int kItems = kH / kCols;              // work items per tile
    static_assert(kCols == kBlk, "an item's columns form one W2 scale block");
};

// One item with CB live 16-row blocks (the tile has 16 CB - 15 .. 16 CB rows): wave `wave`
// computes output columns 16 (hg0 + HF wave) .. + 16 HF - 1 of rows row0 .. row0 + nrows - 1.
template <int D, int HF, int CB>
__device__ __forceinline__ void gemm2_shared_item(
    const Intermediate& C, const uint8_t* __restrict__ w2, const float* __restrict__ s2, int le,
    int row0, int nrows, int hg0, const ExpertRows& rows, int* __restrict__ rows_wide, uint8_t* lds,
    int wave) {
    using S = Gemm2Shared<D, HF>;
    static_assert(kIB % D == 0, "the K loop runs in steps of the ring depth");
    const int lane = threadIdx.x & 63;
    const int r16 = lane & 15, kq = lane >> 4;
    const int drow = lane >> 3, dchunk = lane & 7;
    const int swz = swz128(r16);
    const int rd0 = r16 * kBlk + (((2 * kq) ^ swz) << 4);
    const int rd1 = r16 * kBlk + (((2 * kq + 1) ^ swz) << 4);
    const v4f zero = {0.f, 0.f, 0.f, 0.f};
    uint8_t* const slot = lds + wave * S::kSlot;
    uint8_t* const cst0 = lds + S::NWV * S::kSlot;
    const int hg = hg0 + HF * wave;                         // this wave's first column group

    // W2 rows of this wave (slot row r: W2 row 16 hg + r), by buffer loads over its 16 HF
    // rows (32-bit offsets, the K block in the scalar offset)
    const __amdgpu_buffer_rsrc_t rs_w = buffer_rsrc(w2 + ((size_t)le * kH + hg * 16) * kI, 16 * HF * kI);
    uint32_t woff[2 * HF];
    int wr[2 * HF];
#pragma unroll
    for (int i = 0; i < 2 * HF; ++i) {
        const int r = 8 * i + drow;
        woff[i] = (uint32_t)r * kI + dchunk * 16;
        wr[i] = r * kBlk + ((dchunk ^ swz128(r)) << 4);
    }
    // the item's W2 scale block: one scale per K block for every wave
    const __amdgpu_buffer_rsrc_t rs_s = buffer_rsrc(s2 + (size_t)(le * kHB + (hg0 >> 3)) * kIB, kIB * 4);
    // C rows 16 wave .. 16 wave + 15 of the tile (clamped into it), 4 rows per instruction:
    // lane L moves row 4 i + L / 16 of them into stage chunk L % 16, which holds the row's
    // chunk (L % 16) ^ (row % 16)
    const __amdgpu_buffer_rsrc_t rs_c = buffer_rsrc(C.f16() + (size_t)row0 * kI, 64u * kI * 2);
    const bool clive = 16 * wave < nrows;
    uint32_t coff[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int r = 16 * wave + 4 * i + (lane >> 4);
        coff[i] = (uint32_t)min(r, nrows - 1) * (kI * 2) + (uint32_t)(((lane & 15) ^ (r & 15)) << 4);
    }
    const int nvm = 2 * HF + 1 + (clive ? 4 : 0);   // loads per K block

    // K block kb: W2 rows and scale in ring slot kb % D, C rows in stage kb % (D + 1)
    v4u bw[D][2 * HF];
    float bsc[D];
    auto issue = [&](int kb, int ring) {
#pragma unroll
        for (int i = 0; i < 2 * HF; ++i)   // aux 2: nt, W2 is read once
            bw[ring][i] = __builtin_amdgcn_raw_buffer_load_b128(rs_w, woff[i], (uint32_t)kb * kBlk, 2);
        bsc[ring] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs_s, 0u, (uint32_t)kb * 4, 0));
        uint8_t* st = cst0 + (kb % S::kStages) * S::kCStage;
        if (clive) {
#pragma unroll
            for (int i = 0; i < 4; ++i) bdma16(rs_c, coff[i], (uint32_t)kb * S::kRow, st + (16 * wave + 4 * i) * S::kRow);
        }
    };
#pragma unroll
    for (int k = 0; k < D - 1; ++k) issue(k, k);

    v4f acc[HF][CB];
#pragma unroll
    for (int hf = 0; hf < HF; ++hf)
#pragma unroll
        for (int c = 0; c < CB; ++c) acc[hf][c] = zero;
#pragma unroll 1
    for (int kb0 = 0; kb0 < kIB; kb0 += D) {
#pragma unroll
        for (int j = 0; j < D; ++j) {
            const int kb = kb0 + j;
            // block kb + D - 1 goes to the ring slot block kb - 1 used (written to the LDS
            // slot before) and to the stage of block kb - 2, which every wave finished
            // reading before the barrier of block kb - 1
            if (kb + D - 1 < kIB) issue(kb + D - 1, (j + D - 1) % D);
            __builtin_amdgcn_sched_barrier(0);
            // this wave's loads of block kb are in (those of the D - 1 blocks after it may
            // stay in flight); after the barrier, every wave's (the C stage)
            wait_vm_upto24(min(kIB - 1 - kb, D - 1) * nvm);
            lds_barrier();
#pragma unroll
            for (int i = 0; i < 2 * HF; ++i) *reinterpret_cast<v4u*>(slot + wr[i]) = bw[j][i];
            uint32_t ww[HF][8];
#pragma unroll
            for (int hf = 0; hf < HF; ++hf) {
                const v4u x0 = *reinterpret_cast<const v4u*>(slot + hf * 16 * kBlk + rd0);
                const v4u x1 = *reinterpret_cast<const v4u*>(slot + hf * 16 * kBlk + rd1);
                ww[hf][0] = x0[0]; ww[hf][1] = x0[1]; ww[hf][2] = x0[2]; ww[hf][3] = x0[3];
                ww[hf][4] = x1[0]; ww[hf][5] = x1[1]; ww[hf][6] = x1[2]; ww[hf][7] = x1[3];
            }
            const uint8_t* st = cst0 + (kb % S::kStages) * S::kCStage;
            const float sb = bsc[j];
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                __builtin_amdgcn_sched_barrier(0);   // one row block at a time: short live ranges
                // C row 16 c + r16, elements 32 kq + 8 q .. + 7 of the K block for MFMA q
                const uint8_t* crow = st + (16 * c + r16) * S::kRow;
                v4u cf[4];
#pragma unroll
                for (int q = 0; q < 4; ++q) cf[q] = *reinterpret_cast<const v4u*>(crow + (((4 * kq + q) ^ r16) << 4));
#pragma unroll
                for (int hf = 0; hf < HF; ++hf) {
                    v4f t = zero;
#pragma unroll
                    for (int q = 0; q < 4; ++q) t = mfma_w2_c<true>(ww[hf][2 * q], ww[hf][2 * q + 1], cf[q], t);
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[hf][c][v] = __builtin_fmaf(t[v], sb, acc[hf][c][v]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int c = 0; c < CB; ++c)
#pragma unroll
        for (int hf = 0; hf < HF; ++hf)
            store_rows4(rows, rows_wide, row0 + 16 * c + r16, (hg + hf) * 16 + kq * 4, acc[hf][c],
                        16 * c + r16 < nrows);
}

// Items w = tile * kItems + column block; workgroup b takes b, b + G, ...  flags[0]: C
// beyond the fp16 range (set by GEMM1); flags[1]: an expert row beyond it (set here).
template <int D, int HF>
__global__ __launch_bounds__(256) void gemm2_shared_kernel(
    Intermediate C, int* __restrict__ flags, const uint8_t* __restrict__ w2,
    const float* __restrict__ s2, const int4* __restrict__ tiles,
    const int* __restrict__ num_tiles, ExpertRows rows) {
    using S = Gemm2Shared<D, HF>;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[S::kLds];
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // the first item's tile read before the tile count, both loads in flight together
    // (blockIdx.x / kItems is inside the list's capacity: the grid has at most capacity x
    // kItems workgroups; a workgroup past the count does not use what it read); each later
    // tile is read after the item before it
    const int4 tl0 = tiles[blockIdx.x / S::kItems];
    int te = __builtin_amdgcn_readfirstlane(tl0.x), tr = __builtin_amdgcn_readfirstlane(tl0.y),
        tn = __builtin_amdgcn_readfirstlane(tl0.z);
    const int nwork = (*num_tiles) * S::kItems;
    const bool normal = __builtin_amdgcn_readfirstlane(flags[0]) == 0;
    for (int work = blockIdx.x; work < nwork; work += gridDim.x) {
        const int hg0 = (work % S::kItems) * (S::kCols / 16);
        with_live_blocks(live_blocks(0, tn), [&](auto live) {
            constexpr int CB = decltype(live)::value;
            if constexpr (CB > 0) {
                if (normal) {
                    gemm2_shared_item<D, HF, CB>(C, w2, s2, te, tr, tn, hg0, rows, flags + 1, lds, wave);
                } else {
                    // the rare path one 16-row block at a time, so that its registers stay
                    // below the normal path's
                    const int hg = hg0 + HF * wave;
                    const int lane = threadIdx.x & 63;
#pragma unroll 1
                    for (int c = 0; c < CB; ++c) {
                        v4f acc[HF][1];
                        gemm2_rare_partial<1, HF, 1>(C.f16(), C.f16_exp(), w2, s2, te, tr + 16 * c, tn - 16 * c,
                                                     hg, 0, acc);
#pragma unroll
                        for (int hf = 0; hf < HF; ++hf)
                            store_rows4(rows, flags + 1, tr + 16 * c + (lane & 15), (hg + hf) * 16 + (lane >> 4) * 4,
                                        acc[hf][0], 16 * c + (lane & 15) < tn);
                    }
                }
            }
        });
        if (work + (int)gridDim.x < nwork) {
            const int4 t = tiles[(work + gridDim.x) / S::kItems];
            te = t.x;
            tr = t.y;
            tn = t.z;
        }
        __syncthreads();   // the next item's first DMA reuses the C stages
    }
}

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_g2s_mu;
int g_g2s_grid[kMaxDevices] = {};
}  // namespace

// GEMM2 variant 7: over the first tile list (64-row tiles of the token-sharing GEMM1,
// fp16 C), a persistent grid of as many workgroups as the device holds at once.
bool launch_gemm2_shared(const Intermediate& C, int* flags, const uint8_t* w2, const float* s2,
                         const int4* tiles, const int* num_tiles, int max_tiles, const ExpertRows& rows,
                         hipStream_t stream) {
    using S = Gemm2Shared<2, 2>;
    if (max_tiles <= 0) return false;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
    int resident = 0;
    {
        std::lock_guard<std::mutex> lock(g_g2s_mu);
        if (g_g2s_grid[dev] == 0) {
            int per_cu = 0, cus = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemm2_shared_kernel<2, 2>, 256, 0) != hipSuccess ||
                hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
                per_cu * cus <= 0)
                return false;
            g_g2s_grid[dev] = per_cu * cus;
        }
        resident = g_g2s_grid[dev];
    }
    const long long items = (long long)max_tiles * S::kItems;
    const int grid = (int)(items < resident ? items : resident);
    launch_kernel((gemm2_shared_kernel<2, 2>), dim3(grid), dim3(256), 0, stream, C, flags, w2, s2,
                  tiles, num_tiles, rows);
    return true;
}

}  // namespace moe
