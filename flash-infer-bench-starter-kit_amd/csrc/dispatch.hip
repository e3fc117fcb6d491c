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

template <int TM>
__global__ __launch_bounds__(1024) void dispatch_kernel(
    const int* __restrict__ topk_ids, const float* __restrict__ topk_w, int T, int offset,
    int* __restrict__ exp_off, int* __restrict__ num_tiles, int4* __restrict__ tiles,
    int* __restrict__ sorted_tok, float* __restrict__ sorted_w, int* __restrict__ inv) {
    __shared__ int cnt[kEL];
    __shared__ int off[kEL + 1];
    __shared__ int toff[kEL + 1];
    __shared__ int cursor[kEL];
    __shared__ int wcnt[16][kEL];
    __shared__ int wbase[16][kEL];

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;

    if (tid < kEL) cnt[tid] = 0;
    __syncthreads();

    const long long nassign = (long long)T * kTopK;
    for (long long i = tid; i < nassign; i += 1024) {
        const int le = topk_ids[i] - offset;
        if ((unsigned)le < (unsigned)kEL) atomicAdd(&cnt[le], 1);
    }
    __syncthreads();

    if (tid == 0) {
        int a = 0, b = 0;
        for (int e = 0; e < kEL; ++e) {
            off[e] = a;
            toff[e] = b;
            a += cnt[e];
            b += (cnt[e] + TM - 1) / TM;
        }
        off[kEL] = a;
        toff[kEL] = b;
    }
    __syncthreads();

    if (tid <= kEL) exp_off[tid] = off[tid];
    if (tid == 0) *num_tiles = toff[kEL];
    for (int e = 0; e < kEL; ++e) {
        const int nt = toff[e + 1] - toff[e];
        for (int j = tid; j < nt; j += 1024) {
            const int rows = min(TM, cnt[e] - j * TM);
            tiles[toff[e] + j] = make_int4(e, off[e] + j * TM, rows, 0);
        }
    }
    if (tid < kEL) cursor[tid] = off[tid];
    __syncthreads();

    for (int base = 0; base < T; base += 1024) {
        const int t = base + tid;
        int lek[kTopK];
        uint32_t mask = 0;
#pragma unroll
        for (int k = 0; k < kTopK; ++k) {
            lek[k] = -1;
            if (t < T) {
                const int le = topk_ids[(size_t)t * kTopK + k] - offset;
                if ((unsigned)le < (unsigned)kEL) {
                    lek[k] = le;
                    mask |= 1u << le;
                }
            }
        }
        for (int e = 0; e < kEL; ++e) {
            const uint64_t b = __ballot((mask >> e) & 1u);
            if (lane == 0) wcnt[wave][e] = __popcll(b);
        }
        __syncthreads();
        if (tid < kEL) {
            int run = cursor[tid];
            for (int w = 0; w < 16; ++w) {
                wbase[w][tid] = run;
                run += wcnt[w][tid];
            }
            cursor[tid] = run;
        }
        __syncthreads();
        for (int e = 0; e < kEL; ++e) {
            const uint64_t b = __ballot((mask >> e) & 1u);
            if ((mask >> e) & 1u) {
                const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32),
                                                            __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
                const int r = wbase[wave][e] + below;
#pragma unroll
                for (int k = 0; k < kTopK; ++k) {
                    if (lek[k] == e) {
                        sorted_tok[r] = t;
                        sorted_w[r] = topk_w[(size_t)t * kTopK + k];
                        inv[(size_t)t * kTopK + k] = r;
                    }
                }
            }
        }
        if (t < T) {
#pragma unroll
            for (int k = 0; k < kTopK; ++k)
                if (lek[k] < 0) inv[(size_t)t * kTopK + k] = -1;
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
