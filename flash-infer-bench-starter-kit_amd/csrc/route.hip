// route.hip -- DeepSeek-V3 no-aux routing, one wave64 per token (route_token.h holds
// the routing of a token and its semantics: reference solution/cuda/moe.cu:178-206,
// ties per solution/python/kernel.cu:84-178, the weight sum per kernel.cu:181-185).

#include "route_token.h"

MOE_STAMP_TABLE(route)

namespace moe {

__global__ __launch_bounds__(256) void route_kernel(const float* __restrict__ logits,
                                                    const uint16_t* __restrict__ bias,
                                                    int T, float factor,
                                                    int* __restrict__ topk_ids,
                                                    float* __restrict__ topk_w,
                                                    int* __restrict__ clear_word,
                                                    uint32_t* __restrict__ masks, int offset) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    // the forward's two per-call flag words (C and expert rows beyond the fp16 range, set
    // by GEMM1 and GEMM2, read by GEMM2 and the combine) start at 0
    MOE_STAMP(2 * (int)blockIdx.x);
    if (clear_word != nullptr && blockIdx.x == 0 && threadIdx.x < 2) clear_word[threadIdx.x] = 0;
    if (t >= T) {   // uniform per wave
        // the masks of the grid's last tokens up to 4 ceil(T / 4) are 0: the dispatch
        // reads them four at a time
        if (masks != nullptr && lane == 0) masks[t] = 0u;
        return;
    }

    const float4 lg = reinterpret_cast<const float4*>(logits + (size_t)t * kEG)[lane];
    const uint2 bb = reinterpret_cast<const uint2*>(bias)[lane];
    __shared__ float s_sel[4][kTopK];
    __shared__ int s_sel_id[4][kTopK];
    const int wv = threadIdx.x >> 6;
    int my_id;
    float my_w;
    route_token(lg, bb, lane, factor, s_sel[wv], s_sel_id[wv], my_id, my_w);
    if (lane < kTopK) {
        topk_ids[(size_t)t * kTopK + lane] = my_id;
        topk_w[(size_t)t * kTopK + lane] = my_w;
    }
    // the token's local experts as one word (bit e: local expert e), for the dispatch that
    // counts every token's experts in each workgroup: an OR over the 8 pick lanes
    if (masks != nullptr) {   // uniform
        const int le = my_id - offset;
        uint32_t bit = (lane < kTopK && (unsigned)le < (unsigned)kEL) ? 1u << le : 0u;
        bit |= xor1(bit);
        bit |= xor2(bit);
        bit |= xor4(bit);
        if (lane == 0) masks[t] = bit;
    }
    MOE_STAMP(2 * (int)blockIdx.x + 1);
}

// clear_word (may be null): two ints the kernel sets to 0 for the kernels after it.
// masks (may be null): uint32 [4 ceil(T / 4)], each token's local experts (ids offset ..
// offset + 31), 0 past T.
void launch_route(const float* logits, const uint16_t* bias, int T, float factor,
                  int* topk_ids, float* topk_w, int* clear_word, uint32_t* masks, int offset,
                  hipStream_t stream) {
    if (T <= 0) return;
    launch_kernel(route_kernel, dim3((T + 3) / 4), dim3(256), 0, stream, logits, bias,
                       T, factor, topk_ids, topk_w, clear_word, masks, offset);
}

}  // namespace moe
