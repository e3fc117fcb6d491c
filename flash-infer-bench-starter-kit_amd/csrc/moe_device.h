// moe_device.h -- shared constants and device helpers of the gfx950 fused-MoE kernels.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

#include "moe_shape.h"
#include "stamps.h"

namespace moe {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef short v8s __attribute__((ext_vector_type(8)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// Kernel timing of the stage profiler (MOE_MI355_FLAG_PROFILE).  While a profiled
// forward call enqueues its kernels, g_kernel_timer points at that call's record: every
// launch made through launch_kernel takes the next pair of HIP events, which the runtime
// stamps when the kernel itself starts and ends (hipExtLaunchKernelGGL), so a kernel's
// time excludes the launch gap before it; the record keeps the stage of each launch.
// Outside profiled calls the pointer is null and launch_kernel is a plain launch.
struct KernelTimer {
    hipEvent_t* ev;   // [2 cap]: start, stop of launch i at 2 i, 2 i + 1
    int* stage;       // [cap]
    int cap, n, cur_stage;
};
extern thread_local KernelTimer* g_kernel_timer;

template <typename K, typename... Args>
inline void launch_kernel(K kernel, dim3 grid, dim3 block, uint32_t shmem, hipStream_t s, Args... args) {
    KernelTimer* t = g_kernel_timer;
    if (t != nullptr && t->n < t->cap) {
        const int i = t->n++;
        t->stage[i] = t->cur_stage;
        hipExtLaunchKernelGGL(kernel, grid, block, shmem, s, t->ev[2 * i], t->ev[2 * i + 1], 0, args...);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, shmem, s, args...);
    }
}

// Round-to-nearest-even fp32 -> bf16 bits (NaN -> quiet NaN).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u | ((u >> 16) & 0x8000u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
    return __uint_as_float(h << 16);
}

// Four floats -> four e4m3 bytes (v_cvt_pk_fp8_f32: round to nearest even, OCP e4m3fn,
// the same rounding as torch's float8_e4m3fn cast; inputs are clamped to +-448
// beforehand so nothing overflows to NaN).
__device__ __forceinline__ uint32_t e4m3x4_from_f32(float a, float b, float c, float d) {
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, w, true);
    return (uint32_t)w;
}

__device__ __forceinline__ float clamp448(float x) { return fminf(fmaxf(x, -448.f), 448.f); }

// Order-preserving 32-bit image of an fp32 score; NaN maps to 0 (never preferred).
__device__ __forceinline__ uint32_t order_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if (f != f) return 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ float order_bits_inv(uint32_t k) {
    uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(u);
}

// Chunk swizzle for LDS rows of 128 bytes (8 chunks of 16 B): row r keeps chunk c at
// position c ^ swz128(r).
//
// gfx950 LDS, as measured with SQ_LDS_BANK_CONFLICT on two-lane probes: 64 banks of
// 4 bytes (a 256-byte period), and a ds_read_b128 runs in 4 cycles of 16 lanes.  In
// each half wave, lane quads q = (lane >> 2) & 7 of even bit parity (0, 3, 5, 6) share
// a cycle and those of odd parity (1, 2, 4, 7) share the other.  An MFMA operand read
// has lane (r, kq) (r = lane & 15, kq = lane >> 4) read chunk 2 kq + h of row r.  A
// cycle then holds rows {0-3, 12-15} at one chunk and rows {4-11} at the chunk two
// further on.  With positions c ^ ((r >> 1) & 5), the rows of each parity take the 4
// values {0, 1, 4, 5} on either side; XOR with 2 keeps the sides apart, so every
// cycle hits 16 different 16-byte bank groups (4 cycles per read, none lost).  A row
// stays one contiguous 128-byte line, so the DMA still moves whole lines.
__device__ __forceinline__ constexpr int swz128(int r) { return (r >> 1) & 5; }

// Work-item order of the prefill GEMMs (item = (row tile, column group)).  The row
// tiles of each expert (consecutive in the list, TM rows each but the last) form
// groups of up to 4; the items of a group are numbered column group major, row tile
// fastest, so the items that read the same weight columns of one expert are
// adjacent and run on one XCD in the same round (the weight block is fetched from
// HBM once for all of them).  The group of tiles [f, f + gm) owns items
// [f * ncol, (f + gm) * ncol), so the tile at item / ncol names the group.
template <int TM>
__device__ __forceinline__ void grouped_item(int item, int ncol, const int4* __restrict__ tiles,
                                             const int* __restrict__ exp_off, int& tile, int& col) {
    constexpr int GM = 4;
    const int nominal = item / ncol;
    const int4 t = tiles[nominal];
    const int base = exp_off[t.x];
    const int nt = (exp_off[t.x + 1] - base + TM - 1) / TM;   // tiles of this expert
    const int j = (t.y - base) / TM;                          // index among them
    const int k = j - j % GM;
    const int first = nominal - (j - k);
    const int gm = min(GM, nt - k);
    const int in = item - first * ncol;
    tile = first + in % gm;
    col = in / gm;
}

// Work list of one workgroup of a prefill GEMM: round r handles item r * G + base
// (base = XCD-aware slot of the workgroup, G = grid size), and {expert, first row,
// rows, column group} of that item is one grouped_item chain of three dependent loads.
// prefill_items resolves the chains of all rounds at once, one lane per round, into
// `tab` (LDS, `cap` entries), so that a workgroup waits for one chain at kernel start
// instead of one per item; rounds past `cap` are resolved when they come
// (prefill_item).  Returns the number of rounds that have an item.
template <int TM>
__device__ __forceinline__ int prefill_items(int4* tab, int cap, int nitems, int ncol, int base,
                                             int G, const int4* __restrict__ tiles,
                                             const int* __restrict__ exp_off) {
    const int nr = nitems > base ? (nitems - base + G - 1) / G : 0;
    for (int r = threadIdx.x; r < min(nr, cap); r += blockDim.x) {
        int tix, col;
        grouped_item<TM>(r * G + base, ncol, tiles, exp_off, tix, col);
        const int4 t = tiles[tix];
        tab[r] = int4{t.x, t.y, t.z, col};
    }
    return nr;
}

template <int TM>
__device__ __forceinline__ int4 prefill_item(const int4* tab, int cap, int r, int ncol, int base,
                                             int G, const int4* __restrict__ tiles,
                                             const int* __restrict__ exp_off) {
    int4 m;
    if (r < cap) {
        m = tab[r];
    } else {
        int tix, col;
        grouped_item<TM>(r * G + base, ncol, tiles, exp_off, tix, col);
        const int4 t = tiles[tix];
        m = int4{t.x, t.y, t.z, col};
    }
    // the same for every lane: keep it in scalar registers (buffer resources, loop bounds)
    return int4{__builtin_amdgcn_readfirstlane(m.x), __builtin_amdgcn_readfirstlane(m.y),
                __builtin_amdgcn_readfirstlane(m.z), __builtin_amdgcn_readfirstlane(m.w)};
}

// Ranked order of the same groups, the prefill GEMM1's default up to a few thousand
// tokens.  The experts are ranked by rows (descending, ties by index), each expert's
// groups staying together in list order, and round r gives slot p = base on even and
// G - 1 - base on odd rounds the item r * G + p of that order: the first rounds take
// the experts with the most rows (full tiles), the lighter ones fill the last rounds,
// and those rounds alternate their direction over the slots, so a slot that took one of
// the heaviest items in one round takes one of the lightest in the next instead of two
// heavy ones.  An expert's items stay adjacent, so the items that read the same weight
// columns still run together.  The whole workgroup (kRankThreads threads) computes it
// from the expert offsets alone (tile j of expert e holds rows exp_off[e] + j TM .., as
// the dispatch lists them) in `scr`, kRankScratch bytes of LDS (16-byte aligned) that
// are free until the caller's next barrier.  Returns -1 when there are more than
// kRankMaxGroups groups or `cap` rounds (the caller then uses list order), else the
// number of rounds that have an item for this slot, their items in tab[0 ..).
constexpr int kRankThreads = 512;
constexpr int kRankMaxGroups = kRankThreads;
constexpr int kRankScratch = kRankMaxGroups * 16 + 4 * (2 * 33 + 2 * kRankMaxGroups + 1 + kRankThreads / 64);

template <int TM>
__device__ int prefill_items_ranked(int4* tab, int cap, int ncol, int base, int G,
                                    const int* __restrict__ exp_off, uint8_t* scr) {
    int4* s_g = reinterpret_cast<int4*>(scr);        // [group] {expert, first tile, tiles, expert rows}
    int* s_off = reinterpret_cast<int*>(s_g + kRankMaxGroups);   // [33] expert offsets
    int* s_gs = s_off + 33;                           // [33] first group of each expert, total
    int* s_pos = s_gs + 33;                           // [rank] group
    int* s_start = s_pos + kRankMaxGroups;            // [rank + 1] first item of each rank
    int* s_wsum = s_start + kRankMaxGroups + 1;       // [wave] scan totals
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    if (tid <= kEL) s_off[tid] = exp_off[tid];
    __syncthreads();
    if (wave == 0) {   // groups per expert, exclusive scan over the experts
        int v = 0;
        if (lane < kEL) v = ((s_off[lane + 1] - s_off[lane] + TM - 1) / TM + 3) / 4;
        int incl = v;
#pragma unroll
        for (int d = 1; d < kEL; d <<= 1) {
            const int u = __shfl_up(incl, d);
            if (lane >= d) incl += u;
        }
        if (lane < kEL) s_gs[lane] = incl - v;
        if (lane == kEL - 1) s_gs[kEL] = incl;
    }
    __syncthreads();
    const int ngr = s_gs[kEL];
    if (ngr > kRankMaxGroups) return -1;   // the same in every workgroup (expert offsets only)
    if (ngr == 0) return 0;
    for (int j = tid; j < ngr; j += kRankThreads) {
        int lo = 0, hi = kEL;   // s_gs[lo] <= j < s_gs[hi]: the expert owning group j
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (s_gs[mid] <= j) lo = mid;
            else hi = mid;
        }
        const int rows = s_off[lo + 1] - s_off[lo];
        const int t0 = 4 * (j - s_gs[lo]);
        const int gm = min(4, (rows + TM - 1) / TM - t0);
        s_g[j] = int4{lo, t0, gm, rows};
    }
    __syncthreads();
    // rank of group j: the groups of experts with more rows, and those of equal rows
    // before it in the list (the earlier experts', and the expert's own earlier groups)
    for (int j = tid; j < ngr; j += kRankThreads) {
        const int4 gj = s_g[j];
        int rank = 0;
        for (int i = 0; i < ngr; ++i) {
            const int4 gi = s_g[i];
            rank += (gi.w > gj.w || (gi.w == gj.w && i < j)) ? 1 : 0;
        }
        s_pos[rank] = j;
    }
    __syncthreads();
    {   // first item of each rank: exclusive scan of tiles x ncol over the ranks
        const int v = tid < ngr ? s_g[s_pos[tid]].z * ncol : 0;
        int incl = v;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int u = __shfl_up(incl, d);
            if (lane >= d) incl += u;
        }
        if (lane == 63) s_wsum[wave] = incl;
        __syncthreads();
        for (int w = 0; w < wave; ++w) incl += s_wsum[w];
        if (tid < ngr) s_start[tid] = incl - v;
        if (tid == ngr - 1) s_start[ngr] = incl;
    }
    __syncthreads();
    const int nitems = s_start[ngr];
    // the same decision in every workgroup of the grid (it depends on nitems and G
    // only): no slot gets more than ceil(nitems / G) rounds, so none overflows tab[cap]
    // and either all workgroups take the ranked order or all take list order
    if ((nitems + G - 1) / G > cap) return -1;
    const int R = nitems / G, rem = nitems - R * G;
    const int nr = R + ((((R & 1) ? G - 1 - base : base) < rem) ? 1 : 0);
    for (int r = tid; r < nr; r += kRankThreads) {
        const int i = r * G + ((r & 1) ? G - 1 - base : base);
        int lo = 0, hi = ngr;   // s_start[lo] <= i < s_start[hi]
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (s_start[mid] <= i) lo = mid;
            else hi = mid;
        }
        const int4 g = s_g[s_pos[lo]];
        const int in = i - s_start[lo];
        const int tix = g.y + in % g.z;
        const int rows = s_off[g.x + 1] - s_off[g.x];
        tab[r] = int4{g.x, s_off[g.x] + tix * TM, min(TM, rows - tix * TM), in / g.z};
    }
    return nr;
}

// Token scales as GEMM1 reads them: p[kb * stride + i], where i is the token (by_row 0:
// the caller's hidden_states_scale [56, T], stride T) or the row of the permutation
// (by_row 1: the gathered row scales [56, rows_cap], stride rows_cap, in which the rows
// of a tile are contiguous, so a tile's scales of one K block are one or a few lines
// instead of one 4-byte load per token).
struct TokenScales {
    const float* p;
    int stride;
    int by_row;
};

// The routing inputs of a GEMM1 that routes its tokens itself (logits null: it does not).
struct RouteIn {
    const float* logits;      // [T, 256] fp32
    const uint16_t* bias;     // [256] bf16
    float factor;             // routed scaling factor
};

// One global_load_lds_dwordx4: lane L copies the 16 bytes at its own address g to
// LDS l + 16 L (l must be wave-uniform).
__device__ __forceinline__ void dma16(const uint8_t* g, uint8_t* l) {
    __builtin_amdgcn_global_load_lds(g, l, 16, 0, 0);
}

// One global_load_lds_dword: lane L copies the 4 bytes at g to LDS l + 4 L.
__device__ __forceinline__ void dma4(const void* g, void* l) {
    __builtin_amdgcn_global_load_lds(g, l, 4, 0, 0);
}

// s_waitcnt immediate that waits until at most v vector-memory operations are
// outstanding (gfx9 layout: vmcnt[3:0] bits 3:0, vmcnt[5:4] bits 15:14; expcnt and
// lgkmcnt left at their maxima).
__device__ __forceinline__ constexpr int vmcnt_imm(int v) {
    return (v & 15) | ((v >> 4) << 14) | (7 << 4) | (15 << 8);
}

// vmcnt immediate for v = 0 .. 24 (uniform v; the switch keeps every wait an immediate)
__device__ __forceinline__ void wait_vm_upto24(int v) {
    switch (v) {
#define MOE_WAIT_CASE(n) case n: __builtin_amdgcn_s_waitcnt(vmcnt_imm(n)); break;
        MOE_WAIT_CASE(1) MOE_WAIT_CASE(2) MOE_WAIT_CASE(3) MOE_WAIT_CASE(4) MOE_WAIT_CASE(5)
        MOE_WAIT_CASE(6) MOE_WAIT_CASE(7) MOE_WAIT_CASE(8) MOE_WAIT_CASE(9) MOE_WAIT_CASE(10)
        MOE_WAIT_CASE(11) MOE_WAIT_CASE(12) MOE_WAIT_CASE(13) MOE_WAIT_CASE(14) MOE_WAIT_CASE(15)
        MOE_WAIT_CASE(16) MOE_WAIT_CASE(17) MOE_WAIT_CASE(18) MOE_WAIT_CASE(19) MOE_WAIT_CASE(20)
        MOE_WAIT_CASE(21) MOE_WAIT_CASE(22) MOE_WAIT_CASE(23) MOE_WAIT_CASE(24)
#undef MOE_WAIT_CASE
        default: __builtin_amdgcn_s_waitcnt(vmcnt_imm(0)); break;
    }
}

// Workgroup barrier that orders LDS only.  __syncthreads() is a release/acquire of all
// memory at workgroup scope, which waits for every outstanding vector-memory load
// (vmcnt(0)) and would drain the weight ring at every K block; here the caller has
// already waited for whatever global loads the barrier hands over (its own LDS-DMA
// loads of a K block), and register-staged loads stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
    __asm__ volatile("" ::: "memory");   // no memory access moves across (compiler level)
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's LDS reads and writes are done
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    __asm__ volatile("" ::: "memory");
}

// Loads kernel arguments into SGPRs at the point of the call: an empty asm statement that
// takes each one as an SGPR operand, so the compiler loads them from the kernel-argument
// segment there instead of deferring each load to its first use, where a wave would wait
// a memory round trip for it mid-kernel.  The values are not modified, so a pointer keeps
// its inferred address space (global stores, not flat ones).
template <class A>
__device__ __forceinline__ void load_arg_into_sgprs(const A& a) {
    __asm__ volatile("" ::"s"(a));
}
template <class... A>
__device__ __forceinline__ void load_args_into_sgprs(const A&... a) {
    (load_arg_into_sgprs(a), ...);
}

// Compile-time int for generic lambdas (kernels specialise their K loop on the number
// of 16-row blocks of a tile a wave actually has to compute).
template <int N>
struct IntC {
    static constexpr int value = N;
};
template <bool B>
struct BoolC {
    static constexpr bool value = B;
};

// Calls f(IntC<n>{}) for n in 0..4.
template <typename F>
__device__ __forceinline__ void with_live_blocks(int n, F&& f) {
    switch (n) {
        case 4: f(IntC<4>{}); break;
        case 3: f(IntC<3>{}); break;
        case 2: f(IntC<2>{}); break;
        case 1: f(IntC<1>{}); break;
        default: f(IntC<0>{}); break;
    }
}

// 16-row blocks of a wave's 64 rows starting at row `first` that hold rows < nrows.
__device__ __forceinline__ int live_blocks(int first, int nrows) {
    return min(4, max(0, (nrows - first + 15) >> 4));
}

// Raw buffer resource over [base, base + bytes): 32-bit offsets, the address kept in
// SGPRs (saves the per-lane 64-bit pointers of global_load_lds), out-of-range reads
// return zero.  Word 3 = 0x00020000: raw (unformatted) 32-bit data, stride 0.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}

typedef __attribute__((address_space(3))) void lds_void_t;

// buffer_load_dwordx4 ... lds: lane L copies 16 bytes from voff + soff to LDS l + 16 L.
__device__ __forceinline__ void bdma16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                       void* l) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)l, 16, voff, soff, 0, 0);
}

// buffer_load_dword ... lds: lane L copies 4 bytes from voff + soff to LDS l + 4 L.
__device__ __forceinline__ void bdma4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff,
                                      void* l) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)l, 4, voff, soff, 0, 0);
}

// Values beyond the fp16 range.  The fp16 forms below (C of the streaming GEMM1, the
// expert rows of GEMM2) keep 11 significant bits, but overflow past 65504.  Each
// (row, 16-column group) therefore carries a power-of-two exponent e >= 0 in one byte
// and holds fp16(x * 2^-e): e = 0, the plain fp16 rounding, unless the group holds a
// value beyond the fp16 range (then |x| 2^-e < 2^15 for every value of the group).
// Readers that find the call's flag word raised apply the exponents; otherwise they
// read the fp16 values as they are.
// The flag words are kCWideFlag / kRowsWideFlag of the meta region, the exponent
// groups kGroup16 columns wide (moe_shape.h).
constexpr float kF16Max = 65504.f;

// Exponent of a 16-column group of which this lane holds 4 values (the other 12 are in
// lanes l ^ 16, l ^ 32, l ^ 48: the same row, the other column quads of an MFMA 16x16
// output block), from m = the largest |x| of the lane's 4.  Every lane of the wave must
// call it (it exchanges across lanes).
__device__ __forceinline__ int group_exponent(float m) {
    m = fmaxf(m, __shfl_xor(m, 16));
    m = fmaxf(m, __shfl_xor(m, 32));
    if (!(m > kF16Max) || !(m < __builtin_inff())) return 0;
    int k;
    (void)frexpf(m, &k);        // m in [2^(k-1), 2^k)
    return k - 15;              // m 2^-e in [2^14, 2^15)
}

// Whether some lane's largest |x| (m) is a finite value beyond the fp16 range: the
// only case in which a group exponent can differ from 0.  Uniform across the wave, so
// the callers take group_exponent's lane exchanges only then.
__device__ __forceinline__ bool beyond_f16_in_wave(float m) {
    return __any(m > kF16Max && m < __builtin_inff());
}

// Four fp16 values of a group with exponent e (element offset `off` of a row-major
// [rows, width] array of fp16 bits), written as one 8-byte store.
__device__ __forceinline__ void store_f16x4_scaled(uint16_t* __restrict__ dst, const float (&x)[4], int e) {
    uint32_t h[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) h[v] = __builtin_bit_cast(uint16_t, (_Float16)(e ? ldexpf(x[v], -e) : x[v]));
    *reinterpret_cast<uint2*>(dst) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
}

// The SwiGLU rows C [rows, 2048] between GEMM1 and GEMM2 live in one workspace region
// of rows_cap x (2048 x 4 + 128) bytes, in up to two forms chosen by the kernel plan:
//   fp8 hi/lo (bytes [0, 4 rows_cap) x 512; written by the prefill GEMM1 kernels, or
//     converted from the fp16 form, and read by the prefill GEMM2 kernel): per row and
//     128-column block b a scale s = amax/448 and two e4m3 rows hi = e4m3(C/s),
//     lo = e4m3((C - hi*s) * 16/s), so C ~ s*(hi + lo/16) (GEMM2 then runs two FP8
//     MFMAs per block, the second with an exact 2^-4 operand scale).  hi occupies the
//     first rows_cap*2048 bytes, lo the next; the scales are fp32 [16, rows_cap]
//     (block-major, so a tile's rows are contiguous).
//   fp16 (written by the streaming GEMM1 kernels): C rounded to fp16 in the next
//     rows_cap*2048 halves, then the group exponents, uint8 [rows_cap, 128].  fp16 keeps
//     11 significant bits, and so GEMM2 adds no error that matters next to the bf16
//     output rounding (bf16 C, 8 bits, reaches the 1e-2 tolerance on tokens whose 8
//     experts are all local).  A group beyond the fp16 range raises meta[kCWideFlag].
// GEMM2's output, one row of 7168 per routed assignment, read by the combine: fp16
// rows (11 significant bits keep the combine's result as close to the fp32 sums as
// fp32 rows do, at half the bytes; bf16 rows were tried and break the 1e-2 tolerance
// where large rows cancel), and their group exponents, uint8 [rows, 448]; a group
// beyond the fp16 range raises meta[kRowsWideFlag].
struct ExpertRows {
    uint16_t* f16;
    uint8_t* exp;
};

// Four consecutive values of an expert row (element offset `off`; row `row`, columns
// col .. col + 3): fp16 with the group exponent, and the exponent byte from the lane of
// the group's first column quad.  Every lane of the wave must call it; lanes with
// `valid` false (rows past a tile) store nothing.
__device__ __forceinline__ void store_rows4(const ExpertRows& rows, int* __restrict__ wide_flag,
                                            int row, int col, const v4f& o, bool valid) {
    const float x[4] = {o[0], o[1], o[2], o[3]};
    const float m = fmaxf(fmaxf(fabsf(x[0]), fabsf(x[1])), fmaxf(fabsf(x[2]), fabsf(x[3])));
    if (!beyond_f16_in_wave(m)) {     // the usual case: every exponent of the call is 0
        if (!valid) return;
        store_f16x4_scaled(rows.f16 + (size_t)row * kH + col, x, 0);
        if ((col & (kGroup16 - 1)) == 0) rows.exp[(size_t)row * (kH / kGroup16) + col / kGroup16] = 0;
        return;
    }
    const int e = group_exponent(m);
    if (!valid) return;
    store_f16x4_scaled(rows.f16 + (size_t)row * kH + col, x, e);
    if ((col & (kGroup16 - 1)) == 0) rows.exp[(size_t)row * (kH / kGroup16) + col / kGroup16] = (uint8_t)e;
    if (e) *wide_flag = 1;
}

struct Intermediate {
    void* base;
    float* scales;
    int rows_cap;
    __host__ __device__ uint16_t* f16() const {
        return static_cast<uint16_t*>(base) + (size_t)rows_cap * kI;
    }
    __host__ __device__ uint8_t* f16_exp() const {
        return static_cast<uint8_t*>(base) + 4 * (size_t)rows_cap * kI;
    }
    __host__ __device__ uint8_t* hi() const { return static_cast<uint8_t*>(base); }
    __host__ __device__ uint8_t* lo() const {
        return static_cast<uint8_t*>(base) + (size_t)rows_cap * kI;
    }
};

// fp16 bits and group exponent -> fp32 (exact: the fp16 value times 2^e).
__device__ __forceinline__ float f16_scaled_to_f32(uint32_t h, int e) {
    const float v = (float)__builtin_bit_cast(_Float16, (uint16_t)h);
    return e ? ldexpf(v, e) : v;
}

// ---- lane exchanges (DPP and the lane-swap instructions) ----------------------

// value of lane i^1, i^2 (quad permutes) and i^4 (swap of the two quads of an octet).
// Where every lane has a source lane (quad permutes, row rotations) the DPP moves are
// written with old = 0 and bound_ctrl set, which lets the compiler fold each into the
// max or min that consumes it (v_max_u32_dpp): the same values, one instruction fewer.
__device__ __forceinline__ uint32_t xor1(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xb1, 0xf, 0xf, true);  // quad_perm [1,0,3,2]
}
__device__ __forceinline__ uint32_t xor2(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4e, 0xf, 0xf, true);  // quad_perm [2,3,0,1]
}
__device__ __forceinline__ uint32_t xor4(uint32_t v) {
    // banks 0,2 (lanes 0-3, 8-11 of a row) read lane+4; banks 1,3 read lane-4
    const int a = __builtin_amdgcn_update_dpp((int)v, (int)v, 0x104, 0xf, 0x5, false);  // row_shl:4
    return (uint32_t)__builtin_amdgcn_update_dpp(a, (int)v, 0x114, 0xf, 0xa, false);     // row_shr:4
}

// value of lane i^8 (rotation by 8 inside each row of 16 lanes)
__device__ __forceinline__ uint32_t xor8(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, true);  // row_ror:8
}
// value of lane i^16 and i^32: v_permlane16_swap / v_permlane32_swap of v with itself
// leave the value of the partner row (half) in the second result for even rows (the
// lower half) and in the first for odd rows (the upper half)
__device__ __forceinline__ uint32_t xor16(uint32_t v, int lane) {
    const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return ((lane >> 4) & 1) ? p[0] : p[1];
}
__device__ __forceinline__ uint32_t xor32(uint32_t v, int lane) {
    const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return (lane >> 5) ? p[0] : p[1];
}

}  // namespace moe
