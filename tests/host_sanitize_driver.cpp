// Drives the C ABI's host logic (csrc/host_plan.h: plan choice, workspace layout,
// argument checks, offset clamping) over edge-case token counts, every flag
// combination and NULL / misaligned pointers, checking its invariants.  Built with g++
// twice by tests/test_host_sanitize.py, plainly and under -fsanitize=address,undefined;
// both builds must print the same lines and exit 0.
#include <limits.h>
#include <initializer_list>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

#include "host_plan.h"

using namespace moe::host;

static int g_fail = 0;
#define CHECK(c)                                                               \
    do {                                                                       \
        if (!(c)) {                                                            \
            printf("FAIL %s:%d %s\n", __FILE__, __LINE__, #c);                 \
            ++g_fail;                                                          \
        }                                                                      \
    } while (0)

static const int32_t kTs[] = {INT32_MIN, -1, 0, 1, 2, 4, 5, 8, 9, 16, 22, 23, 32, 33, 63, 64, 65, 88, 89, 199, 200,
                              299, 300, 511, 559, 560,
                              512, 960, 961, 1024, 1344, 1345, 3500, 3501, 8192,
                              (1 << 19) - 1, 1 << 19, (1 << 19) + 1, INT32_MAX};

// Invariants of a layout: regions in order, 256-aligned, each large enough for T.
static void check_layout(int32_t T, const moe_mi355_workspace_layout& L) {
    const size_t R = (size_t)T * 8;
    const size_t off[] = {L.topk_ids, L.topk_weights, L.inverse_rows, L.meta, L.tiles,
                          L.sorted_tokens, L.sorted_weights, L.chunk_counts, L.token_masks,
                          L.row_scales, L.intermediate, L.intermediate_scales, L.expert_out,
                          L.expert_out_exp, L.total};
    const size_t need[] = {R * 4, R * 4, R * 4, 256, (size_t)L.max_tiles * 32, R * 4, R * 4,
                           (size_t)((T + 255) / 256) * 128, (size_t)T * 4, R * 56 * 4,
                           R * (2048 * 4 + 128),
                           R * 16 * 4, R * 7168 * 2, R * 448};
    for (size_t i = 0; i + 1 < sizeof off / sizeof off[0]; ++i) {
        CHECK(off[i] % 256 == 0);
        CHECK(off[i + 1] >= off[i] + need[i]);
    }
    CHECK(L.total % 256 == 0);
    CHECK(L.max_tiles == moe::dispatch_max_tiles(T, 16));
    CHECK(L.tile_m == 16 || L.tile_m == 32 || L.tile_m == 64 || L.tile_m == 256);
    CHECK(L.intermediate_format >= 0 && L.intermediate_format <= 2);
}

// Every T x flag combination: the status is one the header names, and on MOE_OK the
// plan and layout agree with each other.  Returns a checksum of the outcomes.
static unsigned long long sweep_plans() {
    unsigned long long sum = 0;
    int ok = 0, bad = 0;
    const int32_t base_bits[] = {0, MOE_MI355_FLAG_PROFILE, MOE_MI355_FLAG_ROW_SCALES_ON,
                                 MOE_MI355_FLAG_ROW_SCALES_OFF,
                                 MOE_MI355_FLAG_ROW_SCALES_ON | MOE_MI355_FLAG_ROW_SCALES_OFF,
                                 MOE_MI355_FLAG_LIST_ORDER, 1 << 20, 1 << 30, INT32_MIN, -1};
    for (int32_t T : kTs) {
        for (int32_t bb : base_bits) {
            for (int g = -1; g < 256; ++g) {   // -1: no forced plan; else g1 = g & 15, g2 = g >> 4
                const int32_t flags = g < 0 ? bb : (bb | MOE_MI355_FLAG_FORCE_PLAN |
                                                    MOE_MI355_FLAGS_PLAN(g & 15, g >> 4));
                moe_mi355_workspace_layout L;
                memset(&L, 0xab, sizeof L);
                const int st = fill_layout(T, flags, &L);
                CHECK(st == MOE_OK || st == MOE_ERR_BAD_SIZE || st == MOE_ERR_BAD_FLAGS);
                if (T < 0 || T > kMaxT) CHECK(st == MOE_ERR_BAD_SIZE);
                if (bb & ~kKnownFlags) CHECK(st != MOE_OK);
                sum = sum * 1000003ull + (unsigned)(st + 100);
                if (st != MOE_OK) {
                    ++bad;
                    continue;
                }
                ++ok;
                Plan p;
                CHECK(plan_for(T, flags, &p) == MOE_OK);
                CHECK(p.tm == L.tile_m);
                CHECK(p.tm2 == 0 || p.tm2 == 128);
                CHECK(!p.dispatch_in_gemm1 || T <= moe::kDispatchInGemm1MaxT);
                CHECK(!p.route_in_gemm1 || (T <= moe::kRouteInGemm1MaxT && p.dispatch_in_gemm1 &&
                                             p.combine_in_gemm2 && p.g1 == 9));
                CHECK(!p.combine_in_gemm2 || (T <= moe::kFusedCombineMaxT && p.tm == 16));
                CHECK(L.combine_in_gemm2 == (p.combine_in_gemm2 ? 1 : 0));
                check_layout(T, L);
                sum = sum * 1000003ull + (unsigned)(p.g1 * 16 + p.g2) + (p.by_row ? 1000 : 0) +
                      (p.convert ? 2000 : 0) + (unsigned long long)L.total;
            }
        }
    }
    printf("plans ok %d rejected %d checksum %llu\n", ok, bad, sum);
    return sum;
}

// The default plan of each T (no flags) and its boundaries.
static void default_plans() {
    for (int32_t T : kTs) {
        Plan p;
        const int st = (T < 0 || T > kMaxT) ? MOE_ERR_BAD_SIZE : plan_for(T, 0, &p);
        if (st != MOE_OK) {
            printf("T %d status %d\n", T, st);
            continue;
        }
        printf("T %d plan g1 %d g2 %d tm %d tm2 %d convert %d by_row %d dispatch_in_gemm1 %d combine_in_gemm2 %d\n",
               T, p.g1, p.g2, p.tm, p.tm2, (int)p.convert, (int)p.by_row, (int)p.dispatch_in_gemm1,
               (int)p.combine_in_gemm2);
    }
}

static void check_args() {
    alignas(256) static unsigned char buf[4096];
    const int32_t T = 8;
    moe_mi355_workspace_layout L0;
    CHECK(fill_layout(T, 0, &L0) == MOE_OK);
    moe_mi355_args a;
    memset(&a, 0, sizeof a);
    a.routing_logits = (const float*)buf;
    a.routing_bias = (const uint16_t*)buf;
    a.hidden_states = buf;
    a.hidden_states_scale = (const float*)buf;
    a.gemm1_weights = buf;
    a.gemm1_weights_scale = (const float*)buf;
    a.gemm2_weights = buf;
    a.gemm2_weights_scale = (const float*)buf;
    a.output = (uint16_t*)buf;
    a.T = T;
    moe_mi355_workspace_layout L;
    Plan p;
    // pointers are never dereferenced: a fake 256-aligned workspace address suffices
    void* ws = (void*)(uintptr_t)0x100000;
    CHECK(check_forward_args(a, ws, L0.total, &L, &p) == MOE_OK);
    CHECK(check_forward_args(a, ws, L0.total - 1, &L, &p) == MOE_ERR_WORKSPACE);
    CHECK(check_forward_args(a, nullptr, L0.total, &L, &p) == MOE_ERR_WORKSPACE);
    CHECK(check_forward_args(a, (void*)(uintptr_t)0x100080, L0.total, &L, &p) == MOE_ERR_WORKSPACE);
    // each tensor pointer NULL in turn, then misaligned by every offset below its need
    const void** ptrs[] = {(const void**)&a.routing_logits, (const void**)&a.routing_bias,
                           (const void**)&a.hidden_states, (const void**)&a.hidden_states_scale,
                           (const void**)&a.gemm1_weights, (const void**)&a.gemm1_weights_scale,
                           (const void**)&a.gemm2_weights, (const void**)&a.gemm2_weights_scale,
                           (const void**)&a.output};
    const int align[] = {16, 8, 16, 4, 16, 4, 16, 4, 16};
    int nulls = 0, misal = 0;
    for (int i = 0; i < 9; ++i) {
        const void* keep = *ptrs[i];
        *ptrs[i] = nullptr;
        nulls += check_forward_args(a, ws, L0.total, &L, &p) == MOE_ERR_NULL_POINTER;
        for (int o = 1; o < 16; ++o) {
            *ptrs[i] = buf + o;
            const int st = check_forward_args(a, ws, L0.total, &L, &p);
            if (o % align[i]) misal += st == MOE_ERR_MISALIGNED;
            else CHECK(st == MOE_OK);
        }
        *ptrs[i] = keep;
    }
    CHECK(nulls == 9);
    CHECK(misal == 15 * 5 + 14 + 3 * 12);
    // T = 0 needs no pointers; bad T or flags are reported before the pointers
    moe_mi355_args z;
    memset(&z, 0, sizeof z);
    CHECK(check_forward_args(z, nullptr, 0, &L, &p) == MOE_OK);
    z.T = -1;
    CHECK(check_forward_args(z, nullptr, 0, &L, &p) == MOE_ERR_BAD_SIZE);
    z.T = kMaxT + 1;
    CHECK(check_forward_args(z, nullptr, 0, &L, &p) == MOE_ERR_BAD_SIZE);
    z.T = 1;
    z.flags = 1 << 30;
    CHECK(check_forward_args(z, nullptr, 0, &L, &p) == MOE_ERR_BAD_FLAGS);
    printf("args nulls %d misaligned %d\n", nulls, misal);
}

static void check_offsets() {
    const int64_t offs[] = {INT64_MIN, -(int64_t)1 << 40, -(1 << 30) - 1, -(1 << 30), -257, -1, 0, 64,
                            224, 256, (1 << 30), (int64_t)(1 << 30) + 1, (int64_t)1 << 40, INT64_MAX};
    for (int64_t o : offs) {
        const int c = clamp_offset(o);
        CHECK(c >= -(1 << 30) && c <= (1 << 30));
        if (o >= -(1 << 30) && o <= (1 << 30)) CHECK(c == (int)o);
        // id - offset stays inside int32 for every global id 0..255
        for (int id : {0, 255}) {
            const long long d = (long long)id - c;
            CHECK(d > INT32_MIN && d < INT32_MAX);
        }
        printf("offset %lld -> %d\n", (long long)o, c);
    }
}

int main() {
    sweep_plans();
    default_plans();
    check_args();
    check_offsets();
    const moe_mi355_workspace_layout big = workspace_regions(kMaxT);
    printf("workspace at T = %d: %zu bytes, %d tiles\n", kMaxT, big.total, big.max_tiles);
    printf("%s (%d failures)\n", g_fail ? "FAILED" : "OK", g_fail);
    return g_fail ? 1 : 0;
}
