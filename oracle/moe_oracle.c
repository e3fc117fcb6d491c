/*
 * moe_oracle.c -- CPU restatement of the fused-MoE routing and token dispatch.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker for the HIP library, never
 * part of it: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * load it.  The product path (flash-infer-bench-starter-kit_amd/) never links it.
 *
 * What it restates (reference = /root/reference, the fused_moe starter kit):
 *   - sigmoid / score / group selection / top-8 / weight normalisation of the
 *     DeepSeek-V3 no-aux router: solution/cuda/moe.cu:178-206 (ATen spec) with the
 *     tie rule of solution/python/kernel.cu:84-178 (ties -> lower index) and the
 *     sequential selection-order weight sum of kernel.cu:181-185.
 *   - local-expert counting, exclusive scan and the canonical (expert asc, token asc)
 *     permutation: solution/python/kernel.cu:503-547 (scan), kernel.cu:321-351 (fill +
 *     inverse slot) with the order of solution/triton/kernel.py:294-344 (stable sort)
 *     and solution/cuda/moe.cu:212-220 (expert-ascending loop, nonzero() tokens).
 *   - OCP e4m3fn decode: solution/cuda/moe.cu:24-42.
 *
 * Canonical sigmoid: s = fp32( 1 / (1 + exp(-x)) ) evaluated in IEEE binary64 with a
 * self-contained exp (Cody-Waite reduction + degree-13 Taylor polynomial, explicit
 * fma), so the HIP kernel, which restates the same arithmetic, is bit-identical.
 * It is pinned against torch's float64 sigmoid rounded to fp32 in the tests.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off; no fast-math).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define H_SIZE 7168
#define I_SIZE 2048
#define E_GLOBAL 256
#define E_LOCAL 32
#define TOP_K 8
#define N_GROUP 8
#define GROUP_SIZE 32
#define TOPK_GROUP 4

/* Planted-mistake switch for the tests that show the pinning checks catch errors
 * (0 = the restatement as written).  1: group score = top-1 only; 2: group ties
 * go to the higher group; 3: weights normalised with s+bias instead of s;
 * 4: expert ties go to the higher index; 5: permutation ties (same expert) by
 * token descending; 6: the last row tile of an expert claims a full tile. */
static int g_mutation = 0;
void moe_oracle_set_mutation(int m) { g_mutation = m; }

/* ------------------------------------------------------------------------- */
/* canonical exp / sigmoid                                                    */
/* ------------------------------------------------------------------------- */

/* exp(t) for |t| <= 700: t = k*ln2 + r, |r| <= ln2/2, e^r by Taylor to r^13. */
double moe_oracle_exp64(double t) {
    const double inv_ln2 = 0x1.71547652b82fep+0;
    const double ln2_hi = 0x1.62e42fefa39efp-1;
    const double ln2_lo = 0x1.abc9e3b39803fp-56;
    double k = rint(t * inv_ln2);
    double r = fma(-k, ln2_hi, t);
    r = fma(-k, ln2_lo, r);
    /* 1/n! for n = 13 .. 0 */
    static const double c[14] = {
        0x1.6124613a86d09p-33, /* 1/13! */
        0x1.1eed8eff8d898p-29, /* 1/12! */
        0x1.ae64567f544e4p-26, /* 1/11! */
        0x1.27e4fb7789f5cp-22, /* 1/10! */
        0x1.71de3a556c734p-19, /* 1/9! */
        0x1.a01a01a01a01ap-16, /* 1/8! */
        0x1.a01a01a01a01ap-13, /* 1/7! */
        0x1.6c16c16c16c17p-10, /* 1/6! */
        0x1.1111111111111p-7,  /* 1/5! */
        0x1.5555555555555p-5,  /* 1/4! */
        0x1.5555555555555p-3,  /* 1/3! */
        0x1.0000000000000p-1,  /* 1/2! */
        0x1.0000000000000p+0,  /* 1/1! */
        0x1.0000000000000p+0,  /* 1/0! */
    };
    double p = c[0];
    for (int i = 1; i < 14; ++i) p = fma(p, r, c[i]);
    return ldexp(p, (int)k);
}

float moe_oracle_sigmoid(float x) {
    double t = -(double)x;
    if (t != t) return x;            /* NaN passes through */
    if (t > 700.0) return 0.0f;      /* 1/(1+e^700) rounds to +0 in fp32 */
    if (t < -700.0) return 1.0f;     /* 1 + e^-700 == 1 in binary64 */
    double e = moe_oracle_exp64(t);
    return (float)(1.0 / (1.0 + e));
}

/* ------------------------------------------------------------------------- */
/* e4m3fn / bf16 helpers                                                      */
/* ------------------------------------------------------------------------- */

/* OCP e4m3fn: bias 7, subnormal m*2^-9, 0x7F/0xFF NaN, no inf (moe.cu:24-42). */
float moe_oracle_e4m3_decode(uint8_t b) {
    uint32_t s = b >> 7, e = (b >> 3) & 15u, m = b & 7u;
    float v;
    if (e == 15u && m == 7u) return NAN;
    if (e == 0u) v = ldexpf((float)m, -9);
    else v = ldexpf((float)(m | 8u), (int)e - 10);
    return s ? -v : v;
}

void moe_oracle_e4m3_table(float* out256) {
    for (int i = 0; i < 256; ++i) out256[i] = moe_oracle_e4m3_decode((uint8_t)i);
}

static float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Orderable key: larger fp32 -> larger key; NaN and pruned entries get key 0. */
static uint32_t order_bits(float f) {
    uint32_t u;
    if (f != f) return 0u;
    memcpy(&u, &f, 4);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* ------------------------------------------------------------------------- */
/* routing (moe.cu:178-206; kernel.cu:56-200 tie rule)                        */
/* ------------------------------------------------------------------------- */

/* Per-token routing.  Optional debug outputs (may be NULL):
 *   s_out[256], sb_out[256], gscore_out[8], keep_out (bitmask of kept groups). */
void moe_oracle_route_token(const float* logit_row, const uint16_t* bias, double factor,
                            int32_t* ids, float* w, float* s_out, float* sb_out,
                            float* gscore_out, int32_t* keep_out) {
    float s[E_GLOBAL], sb[E_GLOBAL];
    for (int e = 0; e < E_GLOBAL; ++e) {
        s[e] = moe_oracle_sigmoid(logit_row[e]);
        sb[e] = s[e] + bf16_to_f32(bias[e]);
    }
    /* group score = top1 + top2 of sb within the group (moe.cu:186-188).  With a
     * duplicated maximum both copies are taken, like topk(2). */
    float gscore[N_GROUP];
    for (int g = 0; g < N_GROUP; ++g) {
        int b1 = -1;
        for (int j = 0; j < GROUP_SIZE; ++j) {
            int e = g * GROUP_SIZE + j;
            if (b1 < 0 || order_bits(sb[e]) > order_bits(sb[b1])) b1 = e;
        }
        int b2 = -1;
        for (int j = 0; j < GROUP_SIZE; ++j) {
            int e = g * GROUP_SIZE + j;
            if (e == b1) continue;
            if (b2 < 0 || order_bits(sb[e]) > order_bits(sb[b2])) b2 = e;
        }
        gscore[g] = g_mutation == 1 ? sb[b1] : sb[b1] + sb[b2];
    }
    /* keep 4 groups, strict '>' scan -> ties to the lower group (kernel.cu:96-115) */
    uint32_t keep = 0;
    for (int j = 0; j < TOPK_GROUP; ++j) {
        int best = -1;
        for (int g = 0; g < N_GROUP; ++g) {
            if (keep & (1u << g)) continue;
            if (best < 0 || order_bits(gscore[g]) > order_bits(gscore[best]) ||
                (g_mutation == 2 && order_bits(gscore[g]) == order_bits(gscore[best])))
                best = g;
        }
        keep |= 1u << best;
    }
    /* top-8 of the kept experts by (sb desc, index asc) (moe.cu:198-200) */
    uint8_t taken[E_GLOBAL];
    memset(taken, 0, sizeof taken);
    float ssel[TOP_K];
    for (int j = 0; j < TOP_K; ++j) {
        int best = -1;
        uint64_t bestk = 0;
        for (int e = 0; e < E_GLOBAL; ++e) {
            if (taken[e]) continue;
            uint32_t ob = (keep >> (e / GROUP_SIZE)) & 1u ? order_bits(sb[e]) : 0u;
            uint64_t k = ((uint64_t)ob << 32) | (uint64_t)(g_mutation == 4 ? e : 255 - e);
            if (best < 0 || k > bestk) { best = e; bestk = k; }
        }
        taken[best] = 1;
        ids[j] = best;
        ssel[j] = g_mutation == 3 ? sb[best] : s[best];
    }
    /* w = s / (sum + 1e-20) * factor, sum in selection order (moe.cu:202-206,
     * kernel.cu:181-190) */
    float sum = 0.0f;
    for (int j = 0; j < TOP_K; ++j) sum = sum + ssel[j];
    float denom = sum + 1e-20f;
    float f = (float)factor;
    for (int j = 0; j < TOP_K; ++j) {
        float q = ssel[j] / denom;
        w[j] = q * f;
    }
    if (s_out) memcpy(s_out, s, sizeof s);
    if (sb_out) memcpy(sb_out, sb, sizeof sb);
    if (gscore_out) memcpy(gscore_out, gscore, sizeof gscore);
    if (keep_out) *keep_out = (int32_t)keep;
}

void moe_oracle_route(const float* logits, const uint16_t* bias, int32_t T, double factor,
                      int32_t* ids, float* w) {
    for (int32_t t = 0; t < T; ++t)
        moe_oracle_route_token(logits + (size_t)t * E_GLOBAL, bias, factor,
                               ids + (size_t)t * TOP_K, w + (size_t)t * TOP_K,
                               NULL, NULL, NULL, NULL);
}

/* ------------------------------------------------------------------------- */
/* dispatch (kernel.cu:503-547, 321-351, 676-757; triton/kernel.py:294-344)   */
/* ------------------------------------------------------------------------- */

/* Canonical permutation: rows sorted by (local expert asc, token asc).
 * Outputs:
 *   exp_off[33]      exclusive scan of per-expert counts (exp_off[32] = N_a)
 *   sorted_tok[N_a]  token of each row;  sorted_w[N_a] its routing weight
 *   inv[T*8]         row of assignment (t,k), -1 when ids[t,k] is not local
 *   tiles[4*MT]      (expert, first row, row count, 0) per row tile of <= TM rows,
 *                    experts ascending, tiles of one expert consecutive
 * Returns the tile count. */
int32_t moe_oracle_dispatch(const int32_t* ids, const float* w, int32_t T,
                            int64_t offset, int32_t TM, int32_t* exp_off,
                            int32_t* sorted_tok, float* sorted_w, int32_t* inv,
                            int32_t* tiles) {
    int32_t cnt[E_LOCAL];
    memset(cnt, 0, sizeof cnt);
    for (int64_t i = 0; i < (int64_t)T * TOP_K; ++i) {
        int64_t le = (int64_t)ids[i] - offset;
        if (le >= 0 && le < E_LOCAL) cnt[le]++;
    }
    exp_off[0] = 0;
    for (int e = 0; e < E_LOCAL; ++e) exp_off[e + 1] = exp_off[e] + cnt[e];
    int32_t cursor[E_LOCAL];
    for (int e = 0; e < E_LOCAL; ++e) cursor[e] = exp_off[e];
    for (int32_t tt = 0; tt < T; ++tt) {
        int32_t t = g_mutation == 5 ? T - 1 - tt : tt;
        for (int k = 0; k < TOP_K; ++k) {
            size_t i = (size_t)t * TOP_K + k;
            int64_t le = (int64_t)ids[i] - offset;
            if (le >= 0 && le < E_LOCAL) {
                int32_t r = cursor[le]++;
                sorted_tok[r] = t;
                sorted_w[r] = w[i];
                inv[i] = r;
            } else {
                inv[i] = -1;
            }
        }
    }
    int32_t nt = 0;
    for (int e = 0; e < E_LOCAL; ++e) {
        for (int32_t r0 = 0; r0 < cnt[e]; r0 += TM) {
            int32_t n = (cnt[e] - r0 < TM && g_mutation != 6) ? cnt[e] - r0 : TM;
            tiles[4 * nt + 0] = e;
            tiles[4 * nt + 1] = exp_off[e] + r0;
            tiles[4 * nt + 2] = n;
            tiles[4 * nt + 3] = 0;
            ++nt;
        }
    }
    return nt;
}
