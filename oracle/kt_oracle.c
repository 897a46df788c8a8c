/*
 * kt_oracle.c -- CPU restatement of Kotensor's group-wise INT8/INT4 weight-only
 * quantization path. TEST INFRASTRUCTURE ONLY: the checker for the HIP path and
 * the CPU baseline of the benchmark; never linked by the product library.
 *
 * Built with -ffp-contract=off so every float product and sum is rounded on its
 * own, as JVM float arithmetic is in the scalar reference kernels. Pinning
 * status of each function is listed in kt_oracle.h.
 */
#include "kt_oracle.h"

#include <float.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>

/* MatMul constants, K/MatMul.kt:16-28. */
#define TILE_M 32
#define TILE_N 256
#define MAX_ROW_UNITS 32
#define TARGET_UNITS 48
#define UNIT_WORK 65536LL
#define COLUMN_SPLIT_COLUMNS 8192
#define MIN_BLOCK_BYTES 128
#define BLOCK_ALIGN 64

int32_t ko_groups(int32_t rows, int32_t group_size) {
    return (rows + group_size - 1) / group_size; /* K/QuantizedTensor.kt:47 */
}

int32_t ko_bytes_per_row(int32_t columns, int32_t bits) {
    /* storedColumns = N + N % 2 for 4-bit, bytesPerRow = storedColumns / 2,
     * K/QuantizedTensor.kt:48-49 */
    return bits == 4 ? (columns + columns % 2) / 2 : columns;
}

/* Nearest integer with ties toward +inf, saturating; the contract of Math.round
 * (float) that Float.roundToInt() delegates to after rejecting NaN. Written from
 * that contract: for |x| < 2^31 the fractional part x - floor(x) is compared
 * with one half (the subtraction is exact whenever the result can be near 1/2). */
int32_t ko_java_round(float x, int32_t* nan_seen) {
    if (x != x) {
        *nan_seen = 1;
        return 0;
    }
    if (x >= 2147483648.0f) return INT32_MAX;
    if (x <= -2147483648.0f) return INT32_MIN;
    float f = floorf(x);
    float frac = x - f;
    int32_t r = (int32_t)f;
    if (frac >= 0.5f) r += 1;
    return r;
}

static int32_t clampi(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

/* quantizeSymmetric, K/QuantizedTensor.kt:280-294. */
static void quantize_symmetric(const float* data, int32_t columns, int32_t row_start,
                               int32_t row_end, int32_t column, int32_t bytes_per_row,
                               uint8_t* qdata, float* scales, int32_t scale_index,
                               int32_t* nan_seen) {
    float max_abs = 0.0f;
    for (int32_t r = row_start; r < row_end; ++r) {
        float v = fabsf(data[(size_t)r * columns + column]);
        if (v > max_abs) max_abs = v;
    }
    float scale = max_abs > 0.0f ? max_abs / 127.0f : 1.0f;
    scales[scale_index] = scale;
    float inverse = 1.0f / scale;
    for (int32_t r = row_start; r < row_end; ++r) {
        int32_t q = clampi(ko_java_round(data[(size_t)r * columns + column] * inverse, nan_seen), -127, 127);
        qdata[(size_t)r * bytes_per_row + column] = (uint8_t)(int8_t)q;
    }
}

/* quantizeAsymmetric with split-half packing, K/QuantizedTensor.kt:296-324. */
static void quantize_asymmetric(const float* data, int32_t columns, int32_t row_start,
                                int32_t row_end, int32_t column, int32_t half,
                                uint8_t* qdata, float* scales, int8_t* zeros,
                                int32_t scale_index, int32_t* nan_seen) {
    float mn = FLT_MAX;
    float mx = -FLT_MAX;
    for (int32_t r = row_start; r < row_end; ++r) {
        float v = data[(size_t)r * columns + column];
        if (v < mn) mn = v;
        if (v > mx) mx = v;
    }
    if (mn > 0.0f) mn = 0.0f;
    if (mx < 0.0f) mx = 0.0f;
    float range = mx - mn;
    float scale = range > 0.0f ? range / 15.0f : 1.0f;
    int32_t zero = clampi(ko_java_round(-mn / scale, nan_seen), 0, 15);
    scales[scale_index] = scale;
    zeros[scale_index] = (int8_t)zero;
    float inverse = 1.0f / scale;
    for (int32_t r = row_start; r < row_end; ++r) {
        int32_t rounded = ko_java_round(data[(size_t)r * columns + column] * inverse, nan_seen);
        /* Kotlin Int addition wraps on overflow. */
        int32_t q = clampi((int32_t)((uint32_t)rounded + (uint32_t)zero), 0, 15);
        size_t index = (size_t)r * half + column % half;
        uint8_t existing = qdata[index];
        qdata[index] = column < half ? (uint8_t)((existing & 0xF0) | q)
                                     : (uint8_t)((existing & 0x0F) | (q << 4));
    }
}

int32_t ko_quantize(const float* data, int32_t rows, int32_t columns, int32_t bits,
                    int32_t group_size, uint8_t* qdata, float* scales, int8_t* zeros) {
    if ((bits != 4 && bits != 8) || group_size <= 0 || rows <= 0 || columns <= 0) return KO_ERR_ARG;
    if (bits == 4 && zeros == NULL) return KO_ERR_ARG;
    int32_t groups = ko_groups(rows, group_size);
    int32_t bpr = ko_bytes_per_row(columns, bits);
    /* QuantizedTensor.empty(): every byte starts at 0 (K/QuantizedTensor.kt:252-254). */
    memset(qdata, 0, (size_t)rows * bpr);
    int32_t nan_seen = 0;
    for (int32_t group = 0; group < groups; ++group) {
        int32_t row_start = group * group_size;
        int32_t row_end = row_start + group_size < rows ? row_start + group_size : rows;
        int32_t group_offset = group * columns;
        for (int32_t c = 0; c < columns; ++c) {
            if (bits == 8) {
                quantize_symmetric(data, columns, row_start, row_end, c, bpr, qdata, scales,
                                   group_offset + c, &nan_seen);
            } else {
                quantize_asymmetric(data, columns, row_start, row_end, c, bpr, qdata, scales, zeros,
                                    group_offset + c, &nan_seen);
            }
        }
    }
    return nan_seen ? KO_ERR_NAN : KO_OK;
}

/* rawValue, K/QuantizedTensor.kt:172-180: signed byte for 8-bit, nibble for 4-bit. */
int32_t ko_raw_value(const ko_qweight* w, int32_t row, int32_t column) {
    int32_t bpr = ko_bytes_per_row(w->columns, w->bits);
    if (w->bits == 8) return (int32_t)(int8_t)w->qdata[(size_t)row * bpr + column];
    int32_t half = bpr;
    int32_t byte = (int32_t)(int8_t)w->qdata[(size_t)row * bpr + column % half];
    return column < half ? (byte & 0xF) : ((byte >> 4) & 0xF);
}

/* value, K/QuantizedTensor.kt:182-186: scale * (raw - zero), integer difference first. */
float ko_value(const ko_qweight* w, int32_t row, int32_t column) {
    size_t index = (size_t)(row / w->group_size) * w->columns + column;
    int32_t zero = w->zeros ? (int32_t)w->zeros[index] : 0;
    return w->scales[index] * (float)(ko_raw_value(w, row, column) - zero);
}

/* dequantizeRow, K/QuantizedTensor.kt:188-213 (8-bit rows ignore zero points there). */
void ko_dequantize_row(const ko_qweight* w, int32_t row, float* dest) {
    int32_t n = w->columns;
    int32_t bpr = ko_bytes_per_row(n, w->bits);
    size_t group_offset = (size_t)(row / w->group_size) * n;
    const uint8_t* q = w->qdata + (size_t)row * bpr;
    if (w->bits == 8) {
        for (int32_t c = 0; c < n; ++c) dest[c] = w->scales[group_offset + c] * (float)(int8_t)q[c];
    } else {
        int32_t half = bpr;
        for (int32_t c = 0; c < n; ++c) {
            int32_t byte = q[c % half];
            int32_t raw = c < half ? (byte & 0xF) : ((byte >> 4) & 0xF);
            dest[c] = w->scales[group_offset + c] * (float)(raw - (int32_t)w->zeros[group_offset + c]);
        }
    }
}

/* dequantizeColumn, K/QuantizedTensor.kt:235-241. */
void ko_dequantize_column(const ko_qweight* w, int32_t column, float* dest) {
    for (int32_t r = 0; r < w->rows; ++r) dest[r] = ko_value(w, r, column);
}

/* ---------------------------------------------------------------------------
 * Work-stealing unit runner: the shape of MatMul.runUnits/UnitWorker
 * (K/MatMul.kt:573-597). Results never depend on which thread runs a unit.
 * ------------------------------------------------------------------------- */
typedef void (*unit_fn)(void* ctx, int32_t unit);

typedef struct {
    unit_fn fn;
    void* ctx;
    int32_t units;
    atomic_int next;
} unit_pool;

static void* unit_worker(void* arg) {
    unit_pool* p = (unit_pool*)arg;
    for (;;) {
        int32_t unit = atomic_fetch_add(&p->next, 1);
        if (unit >= p->units) return NULL;
        p->fn(p->ctx, unit);
    }
}

static void run_units(int32_t units, int32_t threads, unit_fn fn, void* ctx) {
    if (threads <= 1 || units <= 1) {
        for (int32_t u = 0; u < units; ++u) fn(ctx, u);
        return;
    }
    unit_pool pool;
    pool.fn = fn;
    pool.ctx = ctx;
    pool.units = units;
    atomic_init(&pool.next, 0);
    int32_t workers = threads < units ? threads : units;
    pthread_t* ids = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)workers);
    int32_t started = 0;
    for (int32_t t = 1; t < workers; ++t) {
        if (pthread_create(&ids[t], NULL, unit_worker, &pool) == 0) started = t;
        else break;
    }
    unit_worker(&pool);
    for (int32_t t = 1; t <= started; ++t) pthread_join(ids[t], NULL);
    free(ids);
}

/* ---------------------------------------------------------------------------
 * M == 1 row kernel, K/MatMul.kt:494-536 and rowUnitInto :599-682.
 * ------------------------------------------------------------------------- */
void ko_row_units(const ko_qweight* w, int32_t* out6) {
    int32_t k = w->rows, n = w->columns;
    int32_t row_bytes = ko_bytes_per_row(n, w->bits);
    int32_t groups = ko_groups(k, w->group_size);
    long long t = (long long)k * n / UNIT_WORK;
    int32_t target_units = (int32_t)(t < 1 ? 1 : (t > TARGET_UNITS ? TARGET_UNITS : t));
    int32_t rows_per_unit, wanted_column_units;
    if (n >= COLUMN_SPLIT_COLUMNS) {
        rows_per_unit = k;
        wanted_column_units = target_units;
    } else {
        int32_t groups_per_unit = (groups + MAX_ROW_UNITS - 1) / MAX_ROW_UNITS;
        long long rpu = (long long)groups_per_unit * w->group_size;
        rows_per_unit = rpu < k ? (int32_t)rpu : k;
        wanted_column_units = (target_units * rows_per_unit + k - 1) / k;
    }
    int32_t row_units = (k + rows_per_unit - 1) / rows_per_unit;
    int32_t max_cols = row_bytes / MIN_BLOCK_BYTES > 1 ? row_bytes / MIN_BLOCK_BYTES : 1;
    int32_t column_units = clampi(wanted_column_units, 1, max_cols);
    int32_t per = (row_bytes + column_units - 1) / column_units;
    int32_t aligned = (per + BLOCK_ALIGN - 1) / BLOCK_ALIGN * BLOCK_ALIGN;
    int32_t block_bytes = row_bytes < aligned ? row_bytes : aligned;
    int32_t blocks = (row_bytes + block_bytes - 1) / block_bytes;
    out6[0] = target_units;
    out6[1] = rows_per_unit;
    out6[2] = row_units;
    out6[3] = column_units;
    out6[4] = block_bytes;
    out6[5] = blocks;
}

typedef struct {
    const float* a;
    const ko_qweight* w;
    float* c;
    float* partials;
    float alpha;
    int32_t rows_per_unit, blocks, block_bytes, row_bytes;
} row_ctx;

/* One unit: rows [r0, r1) x byte block [b0, b1). Per group, each column's
 * accumulator and the row sum are built in row order (the 4-row and 8-row
 * batching of rowUnitInto/unpack4/lookup4 keeps that order), then combined as
 * out += alpha * scale * (acc - zero * rowSum)  (combineGroup :804-828). */
static void row_unit(void* vctx, int32_t unit) {
    row_ctx* x = (row_ctx*)vctx;
    const ko_qweight* w = x->w;
    int32_t k = w->rows, n = w->columns, g = w->group_size;
    int32_t row_unit_index = unit / x->blocks;
    int32_t r0 = row_unit_index * x->rows_per_unit;
    int32_t r1 = r0 + x->rows_per_unit < k ? r0 + x->rows_per_unit : k;
    int32_t b0 = (unit % x->blocks) * x->block_bytes;
    int32_t b1 = b0 + x->block_bytes < x->row_bytes ? b0 + x->block_bytes : x->row_bytes;
    float* out = x->partials ? x->partials + (size_t)row_unit_index * n : x->c;
    int32_t width = b1 - b0;
    int32_t packed = w->bits == 4;
    int32_t rb = x->row_bytes;
    int32_t high_columns = packed ? ((rb + b1 < n ? rb + b1 : n) - (rb + b0)) : 0;
    float* low = (float*)malloc(sizeof(float) * (size_t)width * 2);
    float* high = low + width;
    int32_t row = r0;
    while (row < r1) {
        int32_t group = row / g;
        int32_t group_end = (group + 1) * g < r1 ? (group + 1) * g : r1;
        memset(low, 0, sizeof(float) * (size_t)width * 2);
        float row_sum = 0.0f;
        for (int32_t l = row; l < group_end; ++l) {
            float al = x->a[l];
            row_sum += al;
            const uint8_t* q = w->qdata + (size_t)l * rb + b0;
            if (packed) {
                for (int32_t c = 0; c < width; ++c) {
                    low[c] += al * (float)(q[c] & 15);
                    high[c] += al * (float)((q[c] >> 4) & 15);
                }
            } else {
                for (int32_t c = 0; c < width; ++c) low[c] += al * (float)(int8_t)q[c];
            }
        }
        const float* s = w->scales + (size_t)group * n;
        const int8_t* z = w->zeros ? w->zeros + (size_t)group * n : NULL;
        float alpha = x->alpha;
        for (int32_t c = 0; c < width; ++c) {
            int32_t col = b0 + c;
            if (z) out[col] += alpha * s[col] * (low[c] - (float)z[col] * row_sum);
            else out[col] += alpha * s[col] * low[c];
        }
        for (int32_t c = 0; c < high_columns; ++c) {
            int32_t col = rb + b0 + c;
            if (z) out[col] += alpha * s[col] * (high[c] - (float)z[col] * row_sum);
            else out[col] += alpha * s[col] * high[c];
        }
        row = group_end;
    }
    free(low);
}

static void multiply_quantized_row(const float* a, const ko_qweight* w, float* c,
                                   int32_t accumulate, float alpha, int32_t threads) {
    int32_t u[6];
    ko_row_units(w, u);
    int32_t n = w->columns;
    row_ctx x;
    x.a = a;
    x.w = w;
    x.c = c;
    x.alpha = alpha;
    x.rows_per_unit = u[1];
    x.block_bytes = u[4];
    x.blocks = u[5];
    x.row_bytes = ko_bytes_per_row(n, w->bits);
    int32_t row_units = u[2];
    x.partials = row_units > 1 ? (float*)calloc((size_t)row_units * n, sizeof(float)) : NULL;
    if (!accumulate) memset(c, 0, sizeof(float) * (size_t)n);
    run_units(row_units * u[5], threads, row_unit, &x);
    if (x.partials) {
        for (int32_t r = 0; r < row_units; ++r) {
            const float* p = x.partials + (size_t)r * n;
            for (int32_t j = 0; j < n; ++j) c[j] += p[j];
        }
        free(x.partials);
    }
}

/* ---------------------------------------------------------------------------
 * M > 1 tile kernel, computeQuantizedTile K/MatMul.kt:830-881 with the scalar
 * axpy4/axpy of :355-380. Every output element is independent of the tile
 * shape: ct = (accumulate ? c : 0); per group, acc and rowSum in row order,
 * then ct += alpha * scale * (acc - zero * rowSum) (combine[WithZeroPoint] :942-952).
 * ------------------------------------------------------------------------- */
static float weight_as_float(const ko_qweight* w, int32_t row_bytes, int32_t l, int32_t j) {
    if (w->bits == 8) return (float)(int8_t)w->qdata[(size_t)l * row_bytes + j];
    int32_t half = row_bytes;
    uint8_t byte = w->qdata[(size_t)l * row_bytes + j % half];
    return (float)(j < half ? (byte & 15) : ((byte >> 4) & 15));
}

typedef struct {
    const float* a;
    const ko_qweight* w;
    float* c;
    int32_t m, accumulate, tiles_n, width;
    float alpha;
} tile_ctx;

static void tile_unit(void* vctx, int32_t tile) {
    tile_ctx* x = (tile_ctx*)vctx;
    const ko_qweight* w = x->w;
    int32_t k = w->rows, n = w->columns, g = w->group_size;
    int32_t groups = ko_groups(k, g);
    int32_t rb = ko_bytes_per_row(n, w->bits);
    int32_t i0 = (tile / x->tiles_n) * TILE_M;
    int32_t j0 = (tile % x->tiles_n) * x->width;
    int32_t rows = x->m - i0 < TILE_M ? x->m - i0 : TILE_M;
    int32_t len = n - j0 < x->width ? n - j0 : x->width;
    float* ct = (float*)malloc(sizeof(float) * (size_t)TILE_M * len * 2 + sizeof(float) * (size_t)len);
    float* acc = ct + (size_t)TILE_M * len;
    float* brow = acc + (size_t)TILE_M * len;
    float row_sums[TILE_M];
    for (int32_t r = 0; r < rows; ++r)
        for (int32_t j = 0; j < len; ++j)
            ct[(size_t)r * len + j] = x->accumulate ? x->c[(size_t)(i0 + r) * n + j0 + j] : 0.0f;
    for (int32_t group = 0; group < groups; ++group) {
        int32_t k0 = group * g;
        int32_t k1 = k0 + g < k ? k0 + g : k;
        memset(acc, 0, sizeof(float) * (size_t)rows * len);
        for (int32_t r = 0; r < rows; ++r) row_sums[r] = 0.0f;
        for (int32_t l = k0; l < k1; ++l) {
            for (int32_t j = 0; j < len; ++j) brow[j] = weight_as_float(w, rb, l, j0 + j);
            for (int32_t r = 0; r < rows; ++r) {
                float ar = x->a[(size_t)(i0 + r) * k + l];
                float* y = acc + (size_t)r * len;
                for (int32_t j = 0; j < len; ++j) y[j] += ar * brow[j];
                row_sums[r] += ar;
            }
        }
        const float* s = w->scales + (size_t)group * n + j0;
        const int8_t* z = w->zeros ? w->zeros + (size_t)group * n + j0 : NULL;
        for (int32_t r = 0; r < rows; ++r) {
            float* y = ct + (size_t)r * len;
            const float* av = acc + (size_t)r * len;
            if (z) {
                for (int32_t j = 0; j < len; ++j) y[j] += x->alpha * s[j] * (av[j] - (float)z[j] * row_sums[r]);
            } else {
                for (int32_t j = 0; j < len; ++j) y[j] += x->alpha * s[j] * av[j];
            }
        }
    }
    for (int32_t r = 0; r < rows; ++r)
        memcpy(x->c + (size_t)(i0 + r) * n + j0, ct + (size_t)r * len, sizeof(float) * (size_t)len);
    free(ct);
}

/* quantizedTileWidth, K/MatMul.kt:488-492. */
static int32_t quantized_tile_width(int32_t n) {
    if (n >= TARGET_UNITS * TILE_N) return TILE_N;
    int32_t wanted = (n + TARGET_UNITS - 1) / TARGET_UNITS;
    return clampi((wanted + BLOCK_ALIGN - 1) / BLOCK_ALIGN * BLOCK_ALIGN, BLOCK_ALIGN, TILE_N);
}

static int32_t check_weight(const ko_qweight* w) {
    if (!w || !w->qdata || !w->scales) return KO_ERR_ARG;
    if ((w->bits != 4 && w->bits != 8) || w->group_size <= 0 || w->rows <= 0 || w->columns <= 0) return KO_ERR_ARG;
    if (w->bits == 4 && !w->zeros) return KO_ERR_ARG; /* K/QuantizedTensor.kt:69 */
    return KO_OK;
}

int32_t ko_multiply_quantized(const float* a, const ko_qweight* w, float* c, int32_t m,
                              int32_t accumulate, float alpha, int32_t threads) {
    if (m < 0) return KO_ERR_ARG;
    int32_t st = check_weight(w);
    if (st) return st;
    if (m == 0) return KO_OK;
    if (m == 1) {
        multiply_quantized_row(a, w, c, accumulate, alpha, threads);
        return KO_OK;
    }
    tile_ctx x;
    x.a = a;
    x.w = w;
    x.c = c;
    x.m = m;
    x.accumulate = accumulate;
    x.alpha = alpha;
    x.width = quantized_tile_width(w->columns);
    x.tiles_n = (w->columns + x.width - 1) / x.width;
    int32_t tiles = ((m + TILE_M - 1) / TILE_M) * x.tiles_n;
    run_units(tiles, threads, tile_unit, &x);
    return KO_OK;
}

/* ---------------------------------------------------------------------------
 * dX = dY . deq(W)^T, K/MatMul.kt:954-981 with the scalar dot of :983-1003.
 * ------------------------------------------------------------------------- */
typedef struct {
    const float* dy;
    const ko_qweight* w;
    float* dx;
    int32_t m;
} tr_ctx;

static float dot4(const float* a, const float* b, int32_t len) {
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    int32_t j = 0;
    for (; j + 4 <= len; j += 4) {
        s0 += a[j] * b[j];
        s1 += a[j + 1] * b[j + 1];
        s2 += a[j + 2] * b[j + 2];
        s3 += a[j + 3] * b[j + 3];
    }
    float sum = (s0 + s1) + (s2 + s3);
    for (; j < len; ++j) sum += a[j] * b[j];
    return sum;
}

static void tr_unit(void* vctx, int32_t tile) {
    tr_ctx* x = (tr_ctx*)vctx;
    int32_t k = x->w->rows, n = x->w->columns;
    float* wrow = (float*)malloc(sizeof(float) * (size_t)n);
    int32_t k0 = tile * TILE_M;
    int32_t k1 = k0 + TILE_M < k ? k0 + TILE_M : k;
    for (int32_t l = k0; l < k1; ++l) {
        ko_dequantize_row(x->w, l, wrow);
        for (int32_t i = 0; i < x->m; ++i) x->dx[(size_t)i * k + l] += dot4(x->dy + (size_t)i * n, wrow, n);
    }
    free(wrow);
}

int32_t ko_multiply_by_quantized_transposed(const float* dy, const ko_qweight* w, float* dx,
                                            int32_t m, int32_t accumulate, int32_t threads) {
    if (m < 0) return KO_ERR_ARG;
    int32_t st = check_weight(w);
    if (st) return st;
    if (m == 0) return KO_OK;
    if (!accumulate) memset(dx, 0, sizeof(float) * (size_t)m * w->rows);
    tr_ctx x;
    x.dy = dy;
    x.w = w;
    x.dx = dx;
    x.m = m;
    run_units((w->rows + TILE_M - 1) / TILE_M, threads, tr_unit, &x);
    return KO_OK;
}
