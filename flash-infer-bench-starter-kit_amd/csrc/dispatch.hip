// dispatch.hip -- local-expert histogram, exclusive scan and the deterministic
// (local expert asc, token asc) permutation.
//
// Reference: solution/python/kernel.cu:503-547 (exclusive scan of the counts),
// kernel.cu:321-351 (fill + inverse slot map; there the slot inside an expert comes
// from an atomicAdd and is run-to-run nondeterministic), kernel.cu:676-757 (padded
// arrays).  The order produced here is the canonical one of
// solution/triton/kernel.py:294-344 (stable sort by expert) and of the expert loop in
// solution/cuda/moe.cu:212-220 (tokens ascending per expert).
//
// Instead of padding rows in memory, rows stay compact (row = position in the
// permutation) and the GEMMs walk a list of row tiles of <= TM rows, each inside one
// expert: tiles[i] = (expert, first row, rows, 0).
//
// Placement is atomic-free: one token per thread; for each expert a wave ballot gives
// every lane its rank inside the wave and the wave's count.  Up to kDispatchSmallMaxT
// tokens one workgroup (sized to T) does everything in one pass; beyond that a count kernel
// writes per-chunk (256 tokens) expert counts and a place kernel (one workgroup per
// chunk) turns them into each chunk's base and writes the permutation.

#include "dispatch_rows.h"

namespace moe {

constexpr int kDispatchSmallMaxT = 640;

// T <= kDispatchSmallMaxT: one workgroup of NW waves (64 NW >= T), one token per thread, one
// pass over the routes.  Beyond 640 tokens the two-kernel pass over 256-token chunks is
// faster (-1.6 us at T = 1024, -0.8 us at 800; +0.4 us at 600): one workgroup's ballots and
// scans serialise over T / 64 waves.
template <int TM, int TM2, int NW>
__global__ __launch_bounds__(64 * NW) void dispatch_small_kernel(
    const int* __restrict__ topk_ids, const float* __restrict__ topk_w, int T, int offset,
    int* __restrict__ exp_off, int* __restrict__ num_tiles, int4* __restrict__ tiles,
    int* __restrict__ num_tiles2, int4* __restrict__ tiles2,
    int* __restrict__ sorted_tok, float* __restrict__ sorted_w, int* __restrict__ inv) {
    __shared__ int wcnt[NW][kEL];
    __shared__ int wbase[NW][kEL];
    __shared__ int off[kEL];
    __shared__ uint64_t bal[NW][kEL];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

    const TokenRoutes r = load_routes(topk_ids, topk_w, tid, T, offset);
    int rank[kTopK];
    wave_ranks(r, wave, lane, wcnt, bal[wave], rank);
    __syncthreads();
    if (wave == 0) {
        int c = 0;
        if (lane < kEL)
            for (int w = 0; w < NW; ++w) c += wcnt[w][lane];
        write_offsets_and_tiles<TM, TM2>(lane < kEL ? c : 0, lane, off, exp_off, num_tiles, tiles,
                                         num_tiles2, tiles2);
    }
    __syncthreads();
    if (tid < kEL) {
        int run = off[tid];
        for (int w = 0; w < NW; ++w) {
            wbase[w][tid] = run;
            run += wcnt[w][tid];
        }
    }
    __syncthreads();
    place(r, rank, tid, T, wbase[wave], sorted_tok, sorted_w, inv);
}

// T > kDispatchSmallMaxT, pass 1: chunk c (kChunk tokens) writes its per-expert counts.
constexpr int kChunk = 256;
constexpr int kChunkWaves = kChunk / 64;

__global__ __launch_bounds__(kChunk) void dispatch_count_kernel(
    const int* __restrict__ topk_ids, const float* __restrict__ topk_w, int T, int offset,
    int* __restrict__ chunk_cnt) {
    __shared__ int wcnt[kChunkWaves][kEL];
    __shared__ uint64_t bal[kChunkWaves][kEL];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const TokenRoutes r = load_routes(topk_ids, topk_w, blockIdx.x * kChunk + tid, T, offset);
    int rank[kTopK];
    wave_ranks(r, wave, lane, wcnt, bal[wave], rank);
    __syncthreads();
    if (tid < kEL) {
        int c = 0;
        for (int w = 0; w < kChunkWaves; ++w) c += wcnt[w][tid];
        chunk_cnt[blockIdx.x * kEL + tid] = c;
    }
}

// T > kDispatchSmallMaxT, pass 2: every chunk derives the expert offsets and its own base from the
// chunk count table (thread t sums expert t % 32 over chunks = t / 32 mod 8, then the
// eight partial sums are added in a fixed order), places its tokens; chunk 0 also
// writes offsets and tiles.
template <int TM, int TM2>
__global__ __launch_bounds__(kChunk) void dispatch_place_kernel(
    const int* __restrict__ topk_ids, const float* __restrict__ topk_w, int T, int offset,
    const int* __restrict__ chunk_cnt, int nchunks, int* __restrict__ exp_off,
    int* __restrict__ num_tiles, int4* __restrict__ tiles, int* __restrict__ num_tiles2,
    int4* __restrict__ tiles2, int* __restrict__ sorted_tok, float* __restrict__ sorted_w,
    int* __restrict__ inv) {
    constexpr int kGroups = kChunk / kEL;       // 8 chunk strides
    __shared__ int wcnt[kChunkWaves][kEL];
    __shared__ int wbase[kChunkWaves][kEL];
    __shared__ int off[kEL];
    __shared__ int cbase[kEL];
    __shared__ int part[2][kGroups][kEL];
    __shared__ uint64_t bal[kChunkWaves][kEL];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int chunk = blockIdx.x;

    const TokenRoutes r = load_routes(topk_ids, topk_w, chunk * kChunk + tid, T, offset);
    // thread (g, e) sums expert e's counts over chunks g, g + kGroups, ...: the first kPre of
    // them are read here, together with the routes, and summed after the ranks (up to
    // T = kChunk * kGroups * kPre every count; beyond, the rest one stride at a time)
    constexpr int kPre = 8;
    const int e = tid % kEL, g = tid / kEL;
    int pre[kPre];
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
        const int c = g + i * kGroups;
        pre[i] = c < nchunks ? chunk_cnt[c * kEL + e] : 0;
    }
    int rank[kTopK];
    wave_ranks(r, wave, lane, wcnt, bal[wave], rank);
    {
        int total = 0, before = 0;
#pragma unroll
        for (int i = 0; i < kPre; ++i) {
            const int c = g + i * kGroups;
            before += (c < chunk) ? pre[i] : 0;
            total += pre[i];
        }
        for (int c = g + kPre * kGroups; c < nchunks; c += kGroups) {
            const int v = chunk_cnt[c * kEL + e];
            before += (c < chunk) ? v : 0;
            total += v;
        }
        part[0][g][e] = total;
        part[1][g][e] = before;
    }
    __syncthreads();
    if (wave == 0) {
        int total = 0, before = 0;
        if (lane < kEL) {
            for (int g = 0; g < kGroups; ++g) {
                total += part[0][g][lane];
                before += part[1][g][lane];
            }
        }
        if (chunk == 0) {
            write_offsets_and_tiles<TM, TM2>(lane < kEL ? total : 0, lane, off, exp_off, num_tiles, tiles,
                                             num_tiles2, tiles2);
        } else {
            const int ci = scan32(lane < kEL ? total : 0, lane);
            if (lane < kEL) off[lane] = ci - total;
        }
        if (lane < kEL) cbase[lane] = before;
    }
    __syncthreads();
    if (tid < kEL) {
        int run = off[tid] + cbase[tid];
        for (int w = 0; w < kChunkWaves; ++w) {
            wbase[w][tid] = run;
            run += wcnt[w][tid];
        }
    }
    __syncthreads();
    place(r, rank, chunk * kChunk + tid, T, wbase[wave], sorted_tok, sorted_w, inv);
}

// ---------------------------------------------------------------------------
// The forward's dispatch in one launch (kMaskDispatchMinT <= T <= kMaskDispatchMaxT),
// from the route kernel's per-token local-expert masks (bit e: local expert e).  One
// workgroup per 256-token chunk, as in the place kernel, but each workgroup counts every
// expert over all T tokens itself, so no count launch runs before it: in each row of 16
// lanes, 16 masks are transposed as two 16 x 16 bit matrices (lane i of the row then
// holds bit i and bit 16 + i of the row's 16 masks), and two popcounts give the counts
// of experts i and 16 + i over them.  The totals give the expert offsets (and, in the extra
// workgroup below, the tile lists), the counts of the chunks before this one its base in
// each expert;
// the ranks inside the chunk and the placement are the place kernel's.  With row_scales
// set, the workgroups also write the token scales of the rows in row order (the gather
// launch's work), spread over gridDim.y workgroups per chunk: each computes the chunk's
// dispatch (only the first, y = 0, stores it) and writes the scales of its share of the
// 56 K blocks; its chunk's token scales of those K blocks come into LDS by DMA at kernel
// start, and its rows are written one contiguous run per expert.  One more workgroup
// (x = the chunk count, y = 0) counts the totals as the others do and writes only the
// expert offsets and the tile lists: written by a chunk's workgroup, they delayed its end,
// and with it the kernel's, by ~2 us at T = 8192.

// Stage s of the transpose (s = 1, 2, 4, 8): lanes l and l ^ s swap the off-diagonal
// s x s blocks of their 2s x 2s block.  The lower lane keeps its bits at positions with
// bit s clear (keep = M_s) and takes the partner's there, moved up by s (rot = 32 - s, a
// rotation right); the upper lane keeps the positions with bit s set (keep = ~M_s) and
// takes the partner's moved down by s (rot = s).  The bits a rotation wraps around land
// where keep selects the lane's own bits, and no bit crosses between the two 16-bit halves.
__device__ __forceinline__ uint32_t transpose_stage(uint32_t x, uint32_t partner, uint32_t rot,
                                                    uint32_t keep) {
    const uint32_t q = __builtin_amdgcn_alignbit(partner, partner, rot);
    return (x & keep) | (q & ~keep);
}

static_assert(kMaskDispatchMaxT <= 64 * kChunk, "the count reads at most 64 chunks");

// Token-scale K blocks per gathering workgroup: 8 workgroups per chunk up to 32 chunks,
// 4 beyond (about 256 workgroups in all).
template <int NB>
constexpr int kMasksKbPerSlice = NB <= 32 ? kHB / 8 : kHB / 4;
static_assert(kHB % 8 == 0, "the K blocks split evenly over 8 or 4 workgroups");
static_assert(kChunk <= 256, "a token's index in its chunk is kept in one byte");

// NB: chunks the count reads (a power of two >= ceil(T / 256)); masks past T read 0.
// GATHER: row_scales is written (a template parameter, so that the wait for the first
// mask counts the token-scale DMA issued after it exactly and does not wait for it).
template <int NB, bool GATHER>
__global__ __launch_bounds__(kChunk) void dispatch_masks_kernel(
    const int* __restrict__ topk_ids, const float* __restrict__ topk_w,
    const uint32_t* __restrict__ masks, int T, int offset, int tm, int tm2,
    int* __restrict__ exp_off, int* __restrict__ num_tiles, int4* __restrict__ tiles,
    int* __restrict__ num_tiles2, int4* __restrict__ tiles2, int* __restrict__ sorted_tok,
    float* __restrict__ sorted_w, int* __restrict__ inv, const float* __restrict__ hs_scale,
    float* __restrict__ row_scales, int rows_cap) {
    __shared__ int wcnt[kChunkWaves][kEL];
    __shared__ int wbase[kChunkWaves][kEL];
    __shared__ int off[kEL];
    __shared__ int cbase[kEL];
    __shared__ int cpre[kEL + 1];                  // the chunk's rows before expert e
    __shared__ int part[2][kChunkWaves][kEL];
    __shared__ uint64_t bal[kChunkWaves][kEL];
    __shared__ float s_hs[kHB][kChunk];            // the chunk's token scales [kb][token]
    __shared__ int s_row[kChunk * kTopK];          // the chunk's rows, expert-major
    __shared__ uint8_t s_tok[kChunk * kTopK];      // their tokens (index in the chunk)
    load_args_into_sgprs(topk_ids, topk_w, masks, T, offset, tm, tm2, exp_off, num_tiles, tiles,
                         num_tiles2, tiles2, sorted_tok, sorted_w, inv, hs_scale, row_scales, rows_cap);
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int chunk = blockIdx.x;
    const int t = chunk * kChunk + tid;
    const bool tiler = chunk == (int)gridDim.x - 1;          // writes the offsets and tile lists
    if (tiler && blockIdx.y != 0) return;                     // uniform: one tiler
    const bool lead = blockIdx.y == 0;                       // stores the dispatch
    // its token-scale K blocks: KPB of them from kb0 (gridDim.y = kHB / KPB workgroups per
    // chunk); a compile-time count, so that the waits for the loads issued before the DMA
    // count it exactly
    constexpr int KPB = kMasksKbPerSlice<NB>;
    const int kb0 = (int)blockIdx.y * KPB;

    // every load first, in the order they are needed: this chunk's routes, the masks of
    // every chunk, then the chunk's token scales straight into LDS (reads past T return 0
    // and are not used)
    v4u rid[2], rw[2];
    {
        const __amdgpu_buffer_rsrc_t rs_i = buffer_rsrc(topk_ids, (uint32_t)T * kTopK * 4);
        const __amdgpu_buffer_rsrc_t rs_w = buffer_rsrc(topk_w, (uint32_t)T * kTopK * 4);
        const uint32_t o = (uint32_t)t * kTopK * 4;
        rid[0] = __builtin_amdgcn_raw_buffer_load_b128(rs_i, o, 0, 0);
        rid[1] = __builtin_amdgcn_raw_buffer_load_b128(rs_i, o + 16, 0, 0);
        rw[0] = __builtin_amdgcn_raw_buffer_load_b128(rs_w, o, 0, 0);
        rw[1] = __builtin_amdgcn_raw_buffer_load_b128(rs_w, o + 16, 0, 0);
    }
    // wave w counts chunks w, w + 4, ...: one 16-byte load gives each lane 4 consecutive
    // tokens' masks of a chunk, 4 blocks of 64 tokens per load (the route kernel writes 0
    // for the tokens from T up to 4 ceil(T / 4); loads past them read 0)
    constexpr int NL = NB / kChunkWaves;
    v4u mk[NL];
    {
        const __amdgpu_buffer_rsrc_t rs_m = buffer_rsrc(masks, (uint32_t)((T + 3) & ~3) * 4);
#pragma unroll
        for (int i = 0; i < NL; ++i)
            mk[i] = __builtin_amdgcn_raw_buffer_load_b128(
                rs_m, (uint32_t)((kChunkWaves * i + wave) * kChunk + 4 * lane) * 4, 0, 0);
    }
    if constexpr (GATHER) {   // (the tiler's DMA is not used; skipping it under a branch
                              // made the waits below count it conservatively)
        const __amdgpu_buffer_rsrc_t rs_s = buffer_rsrc(hs_scale, (uint32_t)T * kHB * 4);
#pragma unroll
        for (int k = 0; k < KPB; ++k)
            bdma4(rs_s, (uint32_t)t * 4, (uint32_t)(kb0 + k) * T * 4, &s_hs[kb0 + k][64 * wave]);
    }
    TokenRoutes r;
    {
        const int ids[kTopK] = {(int)rid[0][0], (int)rid[0][1], (int)rid[0][2], (int)rid[0][3],
                                (int)rid[1][0], (int)rid[1][1], (int)rid[1][2], (int)rid[1][3]};
        // each element into a scalar first: hipcc's __builtin_bit_cast of a vector element
        // taken with a subscript read element 0 whatever the index
        float ws[kTopK];
#pragma unroll
        for (int k = 0; k < kTopK; ++k) {
            const uint32_t u = rw[k >> 2][k & 3];
            ws[k] = __builtin_bit_cast(float, u);
        }
        r = decode_routes(ids, ws, t, T, offset);
    }

    // expert counts over this wave's chunks (tot) and over those of them before this
    // workgroup's chunk (bef): lane l holds experts l % 16 (lo) and 16 + l % 16 (hi) over
    // the tokens of its row of 16 lanes; the rows, then the four waves, are added after
    uint32_t rot[4], keep[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        constexpr uint32_t kM[4] = {0x55555555u, 0x33333333u, 0x0f0f0f0fu, 0x00ff00ffu};
        const uint32_t sft = 1u << i;
        const bool lower = (lane & sft) == 0;
        rot[i] = lower ? 32u - sft : sft;
        keep[i] = lower ? kM[i] : ~kM[i];
    }
    uint32_t tot_lo = 0, tot_hi = 0, bef_lo = 0, bef_hi = 0;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
        // the load's 4 blocks stage by stage, so that their chains interleave
        uint32_t x[4] = {mk[i][0], mk[i][1], mk[i][2], mk[i][3]};
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = transpose_stage(x[j], xor1(x[j]), rot[0], keep[0]);
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = transpose_stage(x[j], xor2(x[j]), rot[1], keep[1]);
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = transpose_stage(x[j], xor4(x[j]), rot[2], keep[2]);
#pragma unroll
        for (int j = 0; j < 4; ++j) x[j] = transpose_stage(x[j], xor8(x[j]), rot[3], keep[3]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // opaque to the optimiser: it would otherwise push the half-word masks below
            // back through every stage, computing each stage's select three times over
            __asm__("" : "+v"(x[j]));
            tot_lo += (uint32_t)__builtin_popcount(x[j] & 0xffffu);
            tot_hi += (uint32_t)__builtin_popcount(x[j] >> 16);
        }
        if (kChunkWaves * i + wave < chunk) {   // uniform: this load's chunk is before ours
            bef_lo = tot_lo;
            bef_hi = tot_hi;
        }
    }
    // add the four rows (lanes l, l ^ 16, l ^ 32, l ^ 48): lane i < 16 then holds experts
    // i and 16 + i over all of the wave's tokens
    tot_lo += xor16(tot_lo, lane);
    tot_hi += xor16(tot_hi, lane);
    bef_lo += xor16(bef_lo, lane);
    bef_hi += xor16(bef_hi, lane);
    tot_lo += xor32(tot_lo, lane);
    tot_hi += xor32(tot_hi, lane);
    bef_lo += xor32(bef_lo, lane);
    bef_hi += xor32(bef_hi, lane);
    if (lane < 16) {
        part[0][wave][lane] = (int)tot_lo;
        part[0][wave][16 + lane] = (int)tot_hi;
        part[1][wave][lane] = (int)bef_lo;
        part[1][wave][16 + lane] = (int)bef_hi;
    }

    // LDS-only barriers below: __syncthreads would also wait for the token-scale DMA
    // and for the place stores
    int rank[kTopK];
    wave_ranks(r, wave, lane, wcnt, bal[wave], rank);
    lds_barrier();
    // this wave's token-scale DMA (issued before the count, landed by now): waited for
    // here, before any store, so that the wait covers nothing else
    if constexpr (GATHER) __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    if (wave == 0) {
        int total = 0, before = 0, cc = 0;
        if (lane < kEL) {
            for (int w = 0; w < kChunkWaves; ++w) {
                total += part[0][w][lane];
                before += part[1][w][lane];
                cc += wcnt[w][lane];
            }
        }
        if (tiler) {
            write_offsets_and_tiles_rt(lane < kEL ? total : 0, lane, off, exp_off, num_tiles, tiles, tm,
                                       num_tiles2, tiles2, tm2);
        } else {
            const int ci = scan32(lane < kEL ? total : 0, lane);
            if (lane < kEL) off[lane] = ci - total;
        }
        const int cp = scan32(lane < kEL ? cc : 0, lane);
        if (lane < kEL) {
            cbase[lane] = before;
            cpre[lane] = cp - cc;
        }
        if (lane == kEL - 1) cpre[kEL] = cp;
    }
    if (tiler) return;   // uniform
    lds_barrier();
    if (tid < kEL) {
        int run = off[tid] + cbase[tid];
        for (int w = 0; w < kChunkWaves; ++w) {
            wbase[w][tid] = run;
            run += wcnt[w][tid];
        }
    }
    lds_barrier();
    if (lead) place(r, rank, t, T, wbase[wave], sorted_tok, sorted_w, inv);
    if constexpr (!GATHER) return;

    // the chunk's rows of expert e are wbase[0][e] .. + count - 1, entries cpre[e] .. of
    // the expert-major list; then every row's scale of each K block
    if (t < T) {
#pragma unroll
        for (int k = 0; k < kTopK; ++k) {
            const int e = r.lek[k];
            if (e >= 0) {
                const int row = wbase[wave][e] + rank[k];
                const int q = cpre[e] + (row - wbase[0][e]);
                s_row[q] = row;
                s_tok[q] = (uint8_t)tid;
            }
        }
    }
    lds_barrier();   // s_row / s_tok, and every wave's token scales (waited for above)
    const int nq = cpre[kEL];
    for (int q = tid; q < nq; q += kChunk) {
        const int row = s_row[q], tk = s_tok[q];
#pragma unroll 8
        for (int k = 0; k < KPB; ++k) row_scales[(size_t)(kb0 + k) * rows_cap + row] = s_hs[kb0 + k][tk];
    }
}

// The forward's dispatch from the token masks; hs_scale / row_scales (both or neither)
// add the gather of the token scales into row order (rows_cap: row_scales' row stride).
bool launch_dispatch_masks(const int* topk_ids, const float* topk_w, const uint32_t* masks, int T,
                           int offset, int tm, int tm2, int* exp_off, int* num_tiles, int4* tiles,
                           int* num_tiles2, int4* tiles2, int* sorted_tok, float* sorted_w,
                           int* inv, const float* hs_scale, float* row_scales, int rows_cap,
                           hipStream_t stream) {
    if (T < 1 || T > kMaskDispatchMaxT || masks == nullptr) return false;
    if (tm != 16 && tm != 32 && tm != 64 && tm != 128 && tm != 256) return false;
    if (tm2 != 0 && (tm2 != 128 || !tiles2 || !num_tiles2)) return false;
    if ((hs_scale == nullptr) != (row_scales == nullptr)) return false;
    const int nchunks = (T + kChunk - 1) / kChunk;
    // with the gather, about 256 workgroups: 8 or 4 per chunk, each writing the token
    // scales of 7 or 14 of the 56 K blocks (the stores are what takes the time there)
    auto run = [&](auto nb, auto gather) {
        constexpr int NBv = decltype(nb)::value;
        const int slices = decltype(gather)::value ? kHB / kMasksKbPerSlice<NBv> : 1;
        launch_kernel((dispatch_masks_kernel<NBv, decltype(gather)::value>),
                      dim3(nchunks + 1, slices), dim3(kChunk), 0, stream, topk_ids, topk_w, masks, T, offset, tm,
                      tm2, exp_off, num_tiles, tiles, num_tiles2, tiles2, sorted_tok, sorted_w, inv,
                      hs_scale, row_scales, rows_cap);
    };
    auto by_nb = [&](auto gather) {
        if (nchunks <= 8) run(IntC<8>{}, gather);
        else if (nchunks <= 16) run(IntC<16>{}, gather);
        else if (nchunks <= 32) run(IntC<32>{}, gather);
        else run(IntC<64>{}, gather);
    };
    if (row_scales) by_nb(BoolC<true>{});
    else by_nb(BoolC<false>{});
    return true;
}

// Token scales in row order for GEMM1 (reference kernel.cu:204-230, prepare_sfa_kernel,
// builds the same table over its padded rows): row_scales[kb][row] =
// hs_scale[kb][sorted_tok[row]] for the exp_off[32] rows of the permutation.  A GEMM1
// tile then reads its rows' scales of a K block as one contiguous run.  Grid: y = K
// block, x strides over rows (one pass up to 16384 rows); rows_cap is the row stride.
__global__ __launch_bounds__(256) void gather_row_scales_kernel(
    const float* __restrict__ hs_scale, int T, const int* __restrict__ sorted_tok,
    const int* __restrict__ exp_off, float* __restrict__ row_scales, int rows_cap) {
    // the first row's token is read before the row count, so that the two loads are in
    // flight together (its index clamped to the permutation's capacity; a thread past the
    // count does not use it, and no scale is read before the count says the token is real)
    const int row0 = blockIdx.x * 256 + threadIdx.x;
    int tok = sorted_tok[min(row0, rows_cap - 1)];
    const int na = exp_off[kEL];
    const int kb = blockIdx.y;
    for (int row = row0; row < na; row += gridDim.x * 256) {
        if (row != row0) tok = sorted_tok[row];
        row_scales[(size_t)kb * rows_cap + row] = hs_scale[(size_t)kb * T + tok];
    }
}

void launch_gather_row_scales(const float* hs_scale, int T, const int* sorted_tok,
                              const int* exp_off, float* row_scales, int rows_cap,
                              hipStream_t stream) {
    if (rows_cap <= 0) return;
    const int gx = min((rows_cap + 255) / 256, 64);
    launch_kernel(gather_row_scales_kernel, dim3(gx, kHB), dim3(256), 0, stream, hs_scale, T,
                       sorted_tok, exp_off, row_scales, rows_cap);
}

template <int TM, int TM2>
static void launch_dispatch_tm(const int* topk_ids, const float* topk_w, int T, int offset,
                               int* exp_off, int* num_tiles, int4* tiles, int* num_tiles2,
                               int4* tiles2, int* sorted_tok, float* sorted_w, int* inv,
                               int* chunk_cnt, hipStream_t stream) {
    // without chunk_cnt (allowed up to T = 1024 by the C ABI) the one-workgroup pass runs
    if (T <= kDispatchSmallMaxT || (chunk_cnt == nullptr && T <= 1024)) {
#define DISPATCH_SMALL(NW)                                                                        \
    launch_kernel((dispatch_small_kernel<TM, TM2, NW>), dim3(1), dim3(64 * NW), 0, stream,   \
                       topk_ids, topk_w, T, offset, exp_off, num_tiles, tiles, num_tiles2, tiles2, \
                       sorted_tok, sorted_w, inv)
        if (T <= 64) DISPATCH_SMALL(1);
        else if (T <= 256) DISPATCH_SMALL(4);
        else DISPATCH_SMALL(16);
#undef DISPATCH_SMALL
        return;
    }
    const int nchunks = (T + kChunk - 1) / kChunk;
    launch_kernel(dispatch_count_kernel, dim3(nchunks), dim3(kChunk), 0, stream, topk_ids, topk_w,
                       T, offset, chunk_cnt);
    launch_kernel((dispatch_place_kernel<TM, TM2>), dim3(nchunks), dim3(kChunk), 0, stream, topk_ids,
                       topk_w, T, offset, chunk_cnt, nchunks, exp_off, num_tiles, tiles,
                       num_tiles2, tiles2, sorted_tok, sorted_w, inv);
}

// chunk_cnt: int32 [ceil(T/256) * 32] scratch, needed when T > kDispatchSmallMaxT.  tm2 > 0 (with
// tiles2 / num_tiles2): a second tile list of tm2 rows over the same rows.  Tile
// heights: tm in {16, 32, 64, 128, 256} alone, or the pairs (256, 128), (64, 128),
// (32, 128) and (16, 128) the kernel plans use.
bool launch_dispatch(const int* topk_ids, const float* topk_w, int T, int offset, int tm, int tm2,
                     int* exp_off, int* num_tiles, int4* tiles, int* sorted_tok,
                     float* sorted_w, int* inv, int* chunk_cnt, hipStream_t stream,
                     int* num_tiles2, int4* tiles2) {
    auto run = [&](auto tm_c, auto tm2_c) {
        launch_dispatch_tm<decltype(tm_c)::value, decltype(tm2_c)::value>(
            topk_ids, topk_w, T, offset, exp_off, num_tiles, tiles, num_tiles2, tiles2, sorted_tok,
            sorted_w, inv, chunk_cnt, stream);
        return true;
    };
    if (tm2 == 0) {
        switch (tm) {
            case 16: return run(IntC<16>{}, IntC<0>{});
            case 32: return run(IntC<32>{}, IntC<0>{});
            case 64: return run(IntC<64>{}, IntC<0>{});
            case 128: return run(IntC<128>{}, IntC<0>{});
            case 256: return run(IntC<256>{}, IntC<0>{});
            default: return false;
        }
    }
    if (!tiles2 || !num_tiles2 || tm2 != 128) return false;
    switch (tm) {
        case 16: return run(IntC<16>{}, IntC<128>{});
        case 32: return run(IntC<32>{}, IntC<128>{});
        case 64: return run(IntC<64>{}, IntC<128>{});
        case 256: return run(IntC<256>{}, IntC<128>{});
        default: return false;
    }
}

}  // namespace moe
