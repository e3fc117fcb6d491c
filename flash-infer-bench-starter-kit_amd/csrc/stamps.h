// stamps.h -- in-kernel timeline stamps of the decode chain, compiled in only when the
// library is built with -DMOE_MI355_STAMPS (build.py --stamps; stamp_timeline.py reads
// them).  The default build defines both macros as nothing.
//
// Each source file that stamps holds its own device table of kStampSlots 64-bit entries
// (MOE_STAMP_TABLE(name) at namespace scope) and exports
//   int moe_mi355_stamps_<name>(void* host_dst, int reset)
// which copies the table to host_dst (kStampSlots * 8 bytes) or, with reset != 0, zeroes
// it.  MOE_STAMP(slot) writes the constant-rate clock (s_memrealtime, 100 MHz, one clock
// for the whole device) from thread 0 of the workgroup; slots outside the table are
// dropped.  A stamp is a vector store of a scalar read of the clock: no scalar-cache
// write is involved.
#pragma once

#include <hip/hip_runtime.h>

namespace moe {
constexpr int kStampSlots = 8192;
}

#ifdef MOE_MI355_STAMPS

namespace moe {
__device__ __forceinline__ void stamp_write(unsigned long long* table, int slot) {
    const unsigned long long t = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0 && slot >= 0 && slot < kStampSlots) table[slot] = t;
}
}  // namespace moe

#define MOE_STAMP_TABLE(NAME)                                                                     \
    static __device__ unsigned long long g_stamps[::moe::kStampSlots];                            \
    extern "C" __attribute__((visibility("default"))) int moe_mi355_stamps_##NAME(void* dst,      \
                                                                                   int reset) {   \
        static unsigned long long zero[::moe::kStampSlots];                                       \
        if (reset)                                                                                \
            return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_stamps), zero, sizeof(zero), 0,            \
                                          hipMemcpyHostToDevice);                                 \
        if (dst == nullptr) return (int)hipErrorInvalidValue;                                     \
        return (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_stamps), sizeof(g_stamps), 0,           \
                                        hipMemcpyDeviceToHost);                                   \
    }
#define MOE_STAMP(slot) ::moe::stamp_write(g_stamps, (slot))

#else

#define MOE_STAMP_TABLE(NAME)
#define MOE_STAMP(slot) ((void)0)

#endif
