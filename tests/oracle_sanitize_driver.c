/* Test driver (CPU only): runs the C oracle's routing and dispatch on inputs read from
 * a file and writes their outputs, so tests/test_oracle_sanitize.py can run the oracle
 * built with AddressSanitizer and UndefinedBehaviorSanitizer and compare its results
 * with the normal build's.
 * Input:  int32 T, int64 offset, int32 tile_m, double factor, fp32 logits [T,256],
 *         uint16 bias [256].
 * Output: int32 ids [T,8], fp32 w [T,8], int32 exp_off [33], int32 n_tiles,
 *         int32 sorted_tok [N_a], fp32 sorted_w [N_a], int32 inv [T,8], int32 tiles [n_tiles,4]. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

void moe_oracle_route(const float* logits, const uint16_t* bias, int32_t T, double factor,
                      int32_t* ids, float* w);
int32_t moe_oracle_dispatch(const int32_t* ids, const float* w, int32_t T, int64_t offset,
                            int32_t TM, int32_t* exp_off, int32_t* sorted_tok, float* sorted_w,
                            int32_t* inv, int32_t* tiles);

static void must_read(void* p, size_t sz, size_t n, FILE* f) {
    if (n && fread(p, sz, n, f) != n) { fprintf(stderr, "short input\n"); exit(2); }
}

int main(int argc, char** argv) {
    if (argc != 3) { fprintf(stderr, "usage: %s in out\n", argv[0]); return 2; }
    FILE* in = fopen(argv[1], "rb");
    if (!in) return 2;
    int32_t T, tm;
    int64_t offset;
    double factor;
    must_read(&T, 4, 1, in);
    must_read(&offset, 8, 1, in);
    must_read(&tm, 4, 1, in);
    must_read(&factor, 8, 1, in);
    /* exact-size allocations, so the sanitizer sees any access past the arrays */
    float* logits = malloc((size_t)T * 256 * 4 + 1);
    uint16_t* bias = malloc(256 * 2);
    must_read(logits, 4, (size_t)T * 256, in);
    must_read(bias, 2, 256, in);
    fclose(in);
    const size_t R = (size_t)T * 8;
    const int32_t mt = (int32_t)((R + tm - 1) / tm) + 32;
    int32_t* ids = malloc(R * 4 + 1);
    float* w = malloc(R * 4 + 1);
    int32_t* exp_off = malloc(33 * 4);
    int32_t* stok = malloc(R * 4 + 1);
    float* sw = malloc(R * 4 + 1);
    int32_t* inv = malloc(R * 4 + 1);
    int32_t* tiles = malloc((size_t)mt * 16);
    moe_oracle_route(logits, bias, T, factor, ids, w);
    const int32_t nt = moe_oracle_dispatch(ids, w, T, offset, tm, exp_off, stok, sw, inv, tiles);
    FILE* out = fopen(argv[2], "wb");
    if (!out) return 2;
    fwrite(ids, 4, R, out);
    fwrite(w, 4, R, out);
    fwrite(exp_off, 4, 33, out);
    fwrite(&nt, 4, 1, out);
    fwrite(stok, 4, (size_t)exp_off[32], out);
    fwrite(sw, 4, (size_t)exp_off[32], out);
    fwrite(inv, 4, R, out);
    fwrite(tiles, 4, (size_t)nt * 4, out);
    fclose(out);
    free(logits); free(bias); free(ids); free(w); free(exp_off); free(stok); free(sw); free(inv);
    free(tiles);
    return 0;
}
