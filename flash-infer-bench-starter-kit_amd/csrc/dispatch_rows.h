// dispatch_rows.h -- building blocks of the dispatch (per-expert ranks from wave
// ballots, the scan of the counts, the tile list and the placement of rows), shared by
// the dispatch kernels (dispatch.hip) and the GEMM1 that computes the dispatch of its
// few tokens in every workgroup (gemm1_rstream_dispatch_kernel, gemm1.hip, T <= 64).
#pragma once

#include "moe_device.h"

namespace moe {

// inclusive prefix sum over lanes 0..31 of a wave (lanes >= 32 unused; every lane of
// the wave must be active).  DPP: shifts by 1, 2, 4, 8 inside each row of 16 lanes (a
// source outside the row reads 0), then lane 15's row total is added to lanes 16..31.
__device__ __forceinline__ int scan32(int v, int lane) {
    (void)lane;
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);   // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);   // row_bcast:15
    return v;
}

// Per-thread view of one token's 8 assignments: local expert (or -1), weight, and a
// 32-bit mask of its local experts.
struct TokenRoutes {
    int lek[kTopK];
    float wk[kTopK];
    uint32_t mask;
};

// A token's routes from its 8 ids and weights (t >= T: no route).
__device__ __forceinline__ TokenRoutes decode_routes(const int* ids, const float* ws, int t, int T,
                                                     int offset) {
    TokenRoutes r;
    r.mask = 0;
#pragma unroll
    for (int k = 0; k < kTopK; ++k) {
        const int le = ids[k] - offset;
        const bool loc = t < T && (unsigned)le < (unsigned)kEL;
        r.lek[k] = loc ? le : -1;
        r.wk[k] = t < T ? ws[k] : 0.f;
        if (loc) r.mask |= 1u << le;
    }
    return r;
}

__device__ __forceinline__ TokenRoutes load_routes(const int* __restrict__ topk_ids,
                                                   const float* __restrict__ topk_w, int t, int T,
                                                   int offset) {
    TokenRoutes r;
    r.mask = 0;
    if (t < T) {
        const int4* ip = reinterpret_cast<const int4*>(topk_ids + (size_t)t * kTopK);
        const float4* wp = reinterpret_cast<const float4*>(topk_w + (size_t)t * kTopK);
        const int4 i0 = ip[0], i1 = ip[1];
        const float4 w0 = wp[0], w1 = wp[1];
        const int ids[kTopK] = {i0.x, i0.y, i0.z, i0.w, i1.x, i1.y, i1.z, i1.w};
        const float ws[kTopK] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        r = decode_routes(ids, ws, t, T, offset);
    } else {
#pragma unroll
        for (int k = 0; k < kTopK; ++k) { r.lek[k] = -1; r.wk[k] = 0.f; }
    }
    return r;
}

// The ballot of expert BASE + (lane & (2^(BIT+1) - 1)) for this lane: a selection tree
// over the bits of the lane index, whose leaves are the ballots of experts BASE ..
// BASE + 2^(BIT+1) - 1.
template <int BIT, int BASE>
__device__ __forceinline__ uint64_t ballot_for_lane(uint32_t mask, int lane) {
    if constexpr (BIT < 0) {
        return __ballot((mask >> BASE) & 1u);
    } else {
        const uint64_t lo = ballot_for_lane<BIT - 1, BASE>(mask, lane);
        const uint64_t hi = ballot_for_lane<BIT - 1, BASE + (1 << BIT)>(mask, lane);
        return ((lane >> BIT) & 1) ? hi : lo;
    }
}

// For each expert e: the wave's ballot of the lanes routed to it into bal[e] and their
// count into wcnt[wave][e] (LDS).  One ballot per expert; lane e keeps expert e's
// ballot, picked by a selection tree over the bits of the lane index (five levels of
// independent selects; a select per expert in turn made a 32-step dependent chain).
__device__ __forceinline__ void wave_ballots(const TokenRoutes& r, int wave, int lane,
                                             int (*wcnt)[kEL], uint64_t* bal) {
    static_assert(kEL == 32, "the selection tree covers 32 experts");
    const uint64_t mine = ballot_for_lane<4, 0>(r.mask, lane);
    if (lane < kEL) {
        bal[lane] = mine;
        wcnt[wave][lane] = __popcll(mine);
    }
}

// For each expert e: the wave's count into wcnt[wave][e]; returns in rank[k] this
// lane's rank among the wave's lanes holding expert lek[k].  The wave's ballot table
// bal[kEL] (wave_ballots, LDS) is written and read by the same wave only (LDS
// operations of a wave complete in order): every lane reads the ballots of its own
// experts.
__device__ __forceinline__ void wave_ranks(const TokenRoutes& r, int wave, int lane,
                                           int (*wcnt)[kEL], uint64_t* bal, int* rank) {
    wave_ballots(r, wave, lane, wcnt, bal);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int k = 0; k < kTopK; ++k) {
        rank[k] = 0;
        if (r.lek[k] >= 0) {
            const uint64_t b = bal[r.lek[k]];
            rank[k] = __builtin_amdgcn_mbcnt_hi((uint32_t)(b >> 32),
                                                __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
        }
    }
}

__device__ __forceinline__ void place(const TokenRoutes& r, const int* rank, int t, int T,
                                      const int* base, int* __restrict__ sorted_tok,
                                      float* __restrict__ sorted_w, int* __restrict__ inv) {
    if (t >= T) return;
#pragma unroll
    for (int k = 0; k < kTopK; ++k) {
        int row = -1;
        if (r.lek[k] >= 0) {
            row = base[r.lek[k]] + rank[k];
            sorted_tok[row] = t;
            sorted_w[row] = r.wk[k];
        }
        inv[(size_t)t * kTopK + k] = row;
    }
}

// expert offsets, tile list and tile count from the per-expert totals (wave 0).
// With tm2 > 0 (and tiles2 set), also a second list of tiles of tm2 rows over the same
// rows (num_tiles2 = its count), for a GEMM2 that walks other tiles than the GEMM1.
__device__ __forceinline__ void write_offsets_and_tiles_rt(int c, int lane, int* off_lds,
                                                           int* __restrict__ exp_off,
                                                           int* __restrict__ num_tiles,
                                                           int4* __restrict__ tiles, int tm,
                                                           int* __restrict__ num_tiles2,
                                                           int4* __restrict__ tiles2, int tm2) {
    const int tm2r = tm2 > 0 ? tm2 : tm;
    const int nt = (c + tm - 1) / tm;
    const int nt2 = (c + tm2r - 1) / tm2r;
    const int ci = scan32(c, lane);
    const int ti = scan32(nt, lane);
    const int ti2 = scan32(nt2, lane);
    if (lane < kEL) {
        const int o = ci - c, to = ti - nt;
        off_lds[lane] = o;
        exp_off[lane] = o;
        for (int j = 0; j < nt; ++j) tiles[to + j] = make_int4(lane, o + j * tm, min(tm, c - j * tm), 0);
        if (tm2 > 0 && tiles2) {
            const int to2 = ti2 - nt2;
            for (int j = 0; j < nt2; ++j)
                tiles2[to2 + j] = make_int4(lane, o + j * tm2r, min(tm2r, c - j * tm2r), 0);
        }
    }
    if (lane == kEL - 1) {
        exp_off[kEL] = ci;
        *num_tiles = ti;
        if (tm2 > 0 && tiles2) *num_tiles2 = ti2;
    }
}

// The same with the tile heights known at compile time.
template <int TM, int TM2>
__device__ __forceinline__ void write_offsets_and_tiles(int c, int lane, int* off_lds,
                                                        int* __restrict__ exp_off,
                                                        int* __restrict__ num_tiles,
                                                        int4* __restrict__ tiles,
                                                        int* __restrict__ num_tiles2,
                                                        int4* __restrict__ tiles2) {
    write_offsets_and_tiles_rt(c, lane, off_lds, exp_off, num_tiles, tiles, TM, num_tiles2, tiles2,
                               TM2);
}

// Per-wave LDS of dispatch_wave.
struct DispatchWaveLds {
    int wcnt[1][kEL];
    int off[kEL];
    uint64_t bal[kEL];
};

// The dispatch of up to 64 tokens by one wave (lane = token): the computation of
// dispatch_small_kernel<TM, 0, 1> -- expert offsets, the tile list of TM-row tiles, the
// permutation with each row's routing weight, and the inverse map -- written through
// generic pointers, so the results may land in LDS or in global memory.  The whole wave
// must execute it; its LDS tables are written and read by this wave only.
template <int TM>
__device__ __forceinline__ void dispatch_wave(const int* __restrict__ topk_ids,
                                              const float* __restrict__ topk_w, int T, int offset,
                                              int lane, DispatchWaveLds& s, int* exp_off,
                                              int* num_tiles, int4* tiles, int* sorted_tok,
                                              float* sorted_w, int* inv) {
    const TokenRoutes r = load_routes(topk_ids, topk_w, lane, T, offset);
    int rank[kTopK];
    wave_ranks(r, 0, lane, s.wcnt, s.bal, rank);
    __builtin_amdgcn_wave_barrier();
    write_offsets_and_tiles<TM, 0>(lane < kEL ? s.wcnt[0][lane] : 0, lane, s.off, exp_off,
                                   num_tiles, tiles, nullptr, nullptr);
    __builtin_amdgcn_wave_barrier();
    place(r, rank, lane, T, s.off, sorted_tok, sorted_w, inv);
}

}  // namespace moe
