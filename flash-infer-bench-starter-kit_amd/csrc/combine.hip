// combine.hip -- routing-weighted combine of the expert rows into the bf16 output.
//
// Semantics: reference solution/cuda/moe.cu:210, 233-239: acc starts at 0, each local
// expert in ascending order adds round(O * w) into the fp32 accumulator, then one
// bf16 round-to-nearest-even.  The reference's live kernels do this with a gather
// over the inverse slot map (finalize_weighted_bf16_kernel, kernel.cu:809-839) or
// with bf16 atomics (kernel.cu:431-455); here it is a gather with a fixed order and
// no atomics, so the output is identical run to run.
//
// Rows of one token are visited in ascending row index, which is ascending local
// expert because the permutation is expert-major.  Tokens with no local expert get
// +0.0.  One thread produces 8 consecutive outputs (one 16-byte store), with the loads
// of all the token's rows in flight together.  The expert rows arrive in fp16
// (ExpertRows); on a call where GEMM2 flagged a value beyond the fp16 range, the
// rows' group exponents scale them back.

#include "combine_rows.h"

MOE_STAMP_TABLE(combine)

namespace moe {

__global__ __launch_bounds__(128) void combine_kernel(ExpertRows rows, const int* __restrict__ rows_wide,
                                                      const float* __restrict__ sorted_w,
                                                      const int* __restrict__ inv, int T,
                                                      uint16_t* __restrict__ out) {
    constexpr int kParts = kH / (128 * 8);  // 7 blocks of 128 threads per token
    const int t = blockIdx.x / kParts;
    const int h0 = ((blockIdx.x % kParts) * 128 + threadIdx.x) * 8;
    MOE_STAMP(2 * (int)blockIdx.x);
    if (t >= T) return;
    combine_token8(rows, __builtin_amdgcn_readfirstlane(*rows_wide) != 0, inv + (size_t)t * kTopK,
                   sorted_w, h0, out + (size_t)t * kH + h0);
    MOE_STAMP(2 * (int)blockIdx.x + 1);
}

void launch_combine(const ExpertRows& rows, const int* rows_wide, const float* sorted_w, const int* inv,
                    int T, uint16_t* out, hipStream_t stream) {
    if (T <= 0) return;
    constexpr int kParts = kH / (128 * 8);
    launch_kernel(combine_kernel, dim3((unsigned)T * kParts), dim3(128), 0, stream, rows,
                       rows_wide, sorted_w, inv, T, out);
}

}  // namespace moe
