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
