/* Host sanitizer driver for the oracle (test infrastructure): quantize, accessors, the
 * threaded products and the decoder pieces on small random shapes, under
 * AddressSanitizer + UndefinedBehaviorSanitizer or ThreadSanitizer (see run.sh).
 * Exits non-zero on a status or consistency failure; the sanitizers abort on their own
 * findings. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../oracle/kt_oracle.h"

static uint64_t state = 0x9E3779B97F4A7C15ull;
static float uniform(void) {
    state ^= state << 13;
    state ^= state >> 7;
    state ^= state << 17;
    return (float)((state >> 40) * (1.0 / 16777216.0)) * 2.0f - 1.0f;
}

static int check_shape(int rows, int cols, int bits, int g, int m, int threads) {
    const int groups = ko_groups(rows, g), bpr = ko_bytes_per_row(cols, bits);
    float* w = malloc(sizeof(float) * rows * cols);
    float* a = malloc(sizeof(float) * m * rows);
    float* c1 = calloc((size_t)m * cols, sizeof(float));
    float* c2 = calloc((size_t)m * cols, sizeof(float));
    float* dx = calloc((size_t)m * rows, sizeof(float));
    float* row = malloc(sizeof(float) * cols);
    float* col = malloc(sizeof(float) * rows);
    uint8_t* q = malloc((size_t)rows * bpr);
    float* s = malloc(sizeof(float) * groups * cols);
    int8_t* z = bits == 4 ? malloc((size_t)groups * cols) : NULL;
    for (int i = 0; i < rows * cols; ++i) w[i] = 0.02f * uniform();
    for (int i = 0; i < m * rows; ++i) a[i] = uniform();
    int bad = ko_quantize(w, rows, cols, bits, g, q, s, z) != KO_OK;
    ko_qweight qw = {q, s, z, rows, cols, bits, g};
    bad |= ko_multiply_quantized(a, &qw, c1, m, 0, 1.0f, 1) != KO_OK;
    bad |= ko_multiply_quantized(a, &qw, c2, m, 0, 1.0f, threads) != KO_OK;
    bad |= memcmp(c1, c2, sizeof(float) * m * cols) != 0; /* thread count never changes bits */
    bad |= ko_multiply_by_quantized_transposed(c1, &qw, dx, m, 0, threads) != KO_OK;
    ko_dequantize_row(&qw, rows - 1, row);
    ko_dequantize_column(&qw, cols - 1, col);
    bad |= ko_value(&qw, rows - 1, cols - 1) != row[cols - 1];
    int32_t units[6];
    ko_row_units(&qw, units);
    free(w); free(a); free(c1); free(c2); free(dx); free(row); free(col); free(q); free(s); free(z);
    return bad;
}

static int check_decoder(void) {
    enum { T = 3, HEADS = 4, KV = 2, HD = 16, SEQ = 8, DIM = HEADS * HD };
    float x[T * DIM], wt[DIM], out[T * DIM], inv[HD / 2];
    float keys[SEQ * KV * HD], values[SEQ * KV * HD], ctx[T * DIM], scores[SEQ];
    for (int i = 0; i < T * DIM; ++i) x[i] = uniform();
    for (int i = 0; i < DIM; ++i) wt[i] = 1.0f + 0.1f * uniform();
    for (int i = 0; i < SEQ * KV * HD; ++i) { keys[i] = uniform(); values[i] = uniform(); }
    ko_rmsnorm(x, T, DIM, wt, 1e-5f, out);
    ko_rope_inv_freq(HD, 500000.0f, 8.0f, 1.0f, 4.0f, 8192, inv);
    ko_rope_rows(out, T, DIM, HD, inv, 2);
    ko_attend(out, T, 2, keys, values, 0, HEADS, KV, HD, SEQ, ctx, scores);
    ko_silu_mul(out, x, T * DIM);
    return ko_argmax(ctx, T * DIM) < 0;
}

int main(void) {
    int bad = 0;
    const int shapes[][5] = {{64, 48, 4, 32, 1}, {70, 9, 4, 64, 3}, {300, 2100, 4, 64, 1}, {96, 33, 8, 32, 5},
                             {128, 256, 8, 128, 17}, {33, 7, 4, 16, 2}};
    for (size_t i = 0; i < sizeof(shapes) / sizeof(shapes[0]); ++i)
        bad |= check_shape(shapes[i][0], shapes[i][1], shapes[i][2], shapes[i][3], shapes[i][4], 4);
    bad |= check_decoder();
    int nan_seen = 0;
    bad |= ko_java_round(NAN, &nan_seen) != 0 || !nan_seen;
    printf("oracle driver: %s\n", bad ? "FAILED" : "ok");
    return bad;
}
