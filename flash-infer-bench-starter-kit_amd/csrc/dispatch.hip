// dispatch.hip -- local-expert histogram, exclusive scan and the deterministic
// (local expert asc, token asc) permutation, in one 1024-thread workgroup.
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
// Placement is atomic-free: tokens are taken in chunks of 1024 (one per thread); for
// each expert a wave ballot gives every lane its rank inside the wave, a per-wave
// count table gives the wave's base, and a running cursor per expert carries the
// position across chunks.

#include "moe_device.h"

namespace moe {

// inclusive prefix sum over lanes 0..31 of a wave (lanes >= 32 unused)
__device__ __forceinline__ int scan32(int v, int lane) {
#pragma unroll
    for (int off = 1; off < 32; off <<= 1) {
        const int o = __shfl_up(v, off, 64);
        if (lane >= off) v += o;
    }
    return v;
}

template <int TM>
__global__ __launch_bounds__(1024) void dispatch_kernel(
    const int* __restrict__ topk_ids, const float* __restrict__ topk_w, int T, int offset,
    int* __restrict__ exp_off, int* __restrict__ num_tiles, int4* __restrict__ tiles,
    int* __restrict__ sorted_tok, float* __restrict__ sorted_w, int* __restrict__ inv) {
    __shared__ int cnt[kEL];
    __shared__ int off[kEL + 1];
    __shared__ int cursor[kEL];
    __shared__ int wcnt[16][kEL];
    __shared__ int wbase[16][kEL];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;

    if (tid < kEL) cnt[tid] = 0;
    __syncthreads();

    // pass 1: per-expert counts (LDS atomics; the totals do not depend on order)
    const long long nassign = (long long)T * kTopK;
    for (long long i = tid; i < nassign; i += 1024) {
        const int le = topk_ids[i] - offset;
        if ((unsigned)le < (unsigned)kEL) atomicAdd(&cnt[le], 1);
    }
    __syncthreads();

    // exclusive scans of the counts and of the tile counts (wave 0, lane = expert)
    if (wave == 0) {
        const int c = lane < kEL ? cnt[lane] : 0;
        const int nt = (c + TM - 1) / TM;
        const int ci = scan32(c, lane);
        const int ti = scan32(nt, lane);
        if (lane < kEL) {
            const int o = ci - c, to = ti - nt;
            off[lane] = o;
            cursor[lane] = o;
            exp_off[lane] = o;
            for (int j = 0; j < nt; ++j)
                tiles[to + j] = make_int4(lane, o + j * TM, min(TM, c - j * TM), 0);
        }
        if (lane == kEL - 1) {
            off[kEL] = ci;
            exp_off[kEL] = ci;
            *num_tiles = ti;
        }
    }
    __syncthreads();

    // pass 2: placement, 1024 tokens per chunk, one per thread
    for (int base = 0; base < T; base += 1024) {
        const int t = base + tid;
        int lek[kTopK];
        float wk[kTopK];
        uint32_t mask = 0;
        if (t < T) {
            const int4* ip = reinterpret_cast<const int4*>(topk_ids + (size_t)t * kTopK);
            const float4* wp = reinterpret_cast<const float4*>(topk_w + (size_t)t * kTopK);
            const int4 i0 = ip[0], i1 = ip[1];
            const float4 w0 = wp[0], w1 = wp[1];
            const int ids[kTopK] = {i0.x, i0.y, i0.z, i0.w, i1.x, i1.y, i1.z, i1.w};
            const float ws[kTopK] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int k = 0; k < kTopK; ++k) {
                const int le = ids[k] - offset;
                const bool loc = (unsigned)le < (unsigned)kEL;
                lek[k] = loc ? le : -1;
                wk[k] = ws[k];
                if (loc) mask |= 1u << le;
            }
        } else {
#pragma unroll
            for (int k = 0; k < kTopK; ++k) { lek[k] = -1; wk[k] = 0.f; }
        }
        // rank of this token among the chunk's tokens of each of its experts
        int rank[kTopK];
#pragma unroll
        for (int k = 0; k < kTopK; ++k) rank[k] = 0;
        for (int e = 0; e < kEL; ++e) {
            const uint64_t b = __ballot((mask >> e) & 1u);
            if (lane == 0) wcnt[wave][e] = __popcll(b);
            const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32),
                                                        __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
#pragma unroll
            for (int k = 0; k < kTopK; ++k) rank[k] = (lek[k] == e) ? below : rank[k];
        }
        __syncthreads();
        if (tid < kEL) {
            int run = cursor[tid];
#pragma unroll
            for (int w = 0; w < 16; ++w) {
                wbase[w][tid] = run;
                run += wcnt[w][tid];
            }
            cursor[tid] = run;
        }
        __syncthreads();
        if (t < T) {
#pragma unroll
            for (int k = 0; k < kTopK; ++k) {
                int r = -1;
                if (lek[k] >= 0) {
                    r = wbase[wave][lek[k]] + rank[k];
                    sorted_tok[r] = t;
                    sorted_w[r] = wk[k];
                }
                inv[(size_t)t * kTopK + k] = r;
            }
        }
        __syncthreads();
    }
}

int dispatch_max_tiles(int T, int tm) {
    const long long rows = (long long)T * kTopK;
    return (int)((rows + tm - 1) / tm) + kEL;
}

bool launch_dispatch(const int* topk_ids, const float* topk_w, int T, int offset, int tm,
                     int* exp_off, int* num_tiles, int4* tiles, int* sorted_tok,
                     float* sorted_w, int* inv, hipStream_t stream) {
    switch (tm) {
        case 16:
            hipLaunchKernelGGL(dispatch_kernel<16>, dim3(1), dim3(1024), 0, stream, topk_ids,
                               topk_w, T, offset, exp_off, num_tiles, tiles, sorted_tok,
                               sorted_w, inv);
            return true;
        case 32:
            hipLaunchKernelGGL(dispatch_kernel<32>, dim3(1), dim3(1024), 0, stream, topk_ids,
                               topk_w, T, offset, exp_off, num_tiles, tiles, sorted_tok,
                               sorted_w, inv);
            return true;
        case 64:
            hipLaunchKernelGGL(dispatch_kernel<64>, dim3(1), dim3(1024), 0, stream, topk_ids,
                               topk_w, T, offset, exp_off, num_tiles, tiles, sorted_tok,
                               sorted_w, inv);
            return true;
        default:
            return false;
    }
}

}  // namespace moe
