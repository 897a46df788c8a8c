// kt_misc.hip -- the kernels that complete the API around the fast paths:
//   * generic_matmul: any shape and alignment (odd widths, group sizes that are
//     not a multiple of 4, misaligned pointers), one thread per output element,
//     group by group with the reference's combine
//     out += scale * (sum_k a*q - zero * sum_k a)  (MatMul.kt:804-828,942-952);
//   * transposed: dx = dy . deq(W)^T (MatMul.kt:954-981), 8-bit rows dequantized
//     without zero points as QuantizedTensor.dequantizeRow does (QuantizedTensor.kt:198-202);
//   * dequantize_rows / dequantize_columns: the embedding gathers
//     (QuantizedTensor.kt:188-241, Embedding.kt:73-136).
// File paths are relative to Engine/kotensor/src/main/kotlin/.
#include "kt_common.h"

namespace kt {
namespace {

__device__ __forceinline__ int32_t raw_value(const uint8_t* q, int32_t bits, int32_t bpr, int32_t k, int32_t n) {
    if (bits == 8) return static_cast<int8_t>(q[static_cast<size_t>(k) * bpr + n]);
    const int32_t half = bpr;
    const uint8_t byte = q[static_cast<size_t>(k) * bpr + (n < half ? n : n - half)];
    return n < half ? (byte & 0xF) : ((byte >> 4) & 0xF);
}

__global__ void __launch_bounds__(256)
    generic_matmul(const float* __restrict__ a, int32_t M, const uint8_t* __restrict__ q, const float* __restrict__ s,
                   const int8_t* __restrict__ z, int32_t K, int32_t N, int32_t bits, int32_t bpr, int32_t g,
                   float* __restrict__ c, const float* __restrict__ bias, float alpha, int32_t accumulate) {
    const int32_t col_blocks = ceil_div(N, 256);
    const int32_t m = blockIdx.x / col_blocks;
    const int32_t n = (blockIdx.x % col_blocks) * 256 + threadIdx.x;
    if (m >= M || n >= N) return;
    const float* arow = a + static_cast<size_t>(m) * K;
    float out = 0.0f;
    for (int32_t k0 = 0, gi = 0; k0 < K; k0 += g, ++gi) {
        const int32_t k1 = min(k0 + g, K);
        float acc = 0.0f, rsum = 0.0f;
        for (int32_t k = k0; k < k1; ++k) {
            const float ak = arow[k];
            acc = fmaf(ak, static_cast<float>(raw_value(q, bits, bpr, k, n)), acc);
            rsum += ak;
        }
        const size_t idx = static_cast<size_t>(gi) * N + n;
        const float zero = z ? static_cast<float>(z[idx]) : 0.0f;
        out = fmaf(s[idx], fmaf(-zero, rsum, acc), out);
    }
    float* dst = c + static_cast<size_t>(m) * N + n;
    float o = accumulate ? *dst : 0.0f;
    o = fmaf(alpha, out, o);
    if (bias) o += bias[n];
    *dst = o;
}

// dequantizeRow value of element (k, n): 8-bit ignores zero points there.
__device__ __forceinline__ float row_value(const uint8_t* q, const float* s, const int8_t* z, int32_t bits, int32_t bpr,
                                           int32_t N, int32_t g, int32_t k, int32_t n) {
    const size_t idx = static_cast<size_t>(k / g) * N + n;
    const int32_t raw = raw_value(q, bits, bpr, k, n);
    if (bits == 8) return s[idx] * static_cast<float>(raw);
    return s[idx] * static_cast<float>(raw - static_cast<int32_t>(z[idx]));
}

// One workgroup per (weight row l, chunk of 8 dy rows): partial dots over n, then
// a fixed-order tree in LDS.
constexpr int TR_ROWS = 8;
__global__ void __launch_bounds__(256)
    transposed_kernel(const float* __restrict__ dy, int32_t M, const uint8_t* __restrict__ q, const float* __restrict__ s,
                      const int8_t* __restrict__ z, int32_t K, int32_t N, int32_t bits, int32_t bpr, int32_t g,
                      float* __restrict__ dx, int32_t accumulate) {
    __shared__ float red[TR_ROWS][256];
    const int32_t chunks = ceil_div(M, TR_ROWS);
    const int32_t l = blockIdx.x / chunks;
    const int32_t i0 = (blockIdx.x % chunks) * TR_ROWS;
    const int32_t t = threadIdx.x;
    float part[TR_ROWS];
#pragma unroll
    for (int r = 0; r < TR_ROWS; ++r) part[r] = 0.0f;
    for (int32_t n = t; n < N; n += 256) {
        const float wv = row_value(q, s, z, bits, bpr, N, g, l, n);
#pragma unroll
        for (int r = 0; r < TR_ROWS; ++r)
            if (i0 + r < M) part[r] = fmaf(dy[static_cast<size_t>(i0 + r) * N + n], wv, part[r]);
    }
#pragma unroll
    for (int r = 0; r < TR_ROWS; ++r) red[r][t] = part[r];
    __syncthreads();
    for (int32_t w = 128; w > 0; w >>= 1) {
        if (t < w) {
#pragma unroll
            for (int r = 0; r < TR_ROWS; ++r) red[r][t] += red[r][t + w];
        }
        __syncthreads();
    }
    if (t < TR_ROWS && i0 + t < M) {
        float* dst = dx + static_cast<size_t>(i0 + t) * K + l;
        *dst = (accumulate ? *dst : 0.0f) + red[t][0];
    }
}

__global__ void __launch_bounds__(256)
    dequant_rows_kernel(const uint8_t* __restrict__ q, const float* __restrict__ s, const int8_t* __restrict__ z,
                        int32_t bits, int32_t bpr, int32_t K, int32_t N, int32_t g, const int32_t* __restrict__ rows,
                        int32_t count, float* __restrict__ out) {
    const int32_t col_blocks = ceil_div(N, 256);
    const int32_t i = blockIdx.x / col_blocks;
    const int32_t n = (blockIdx.x % col_blocks) * 256 + threadIdx.x;
    if (i >= count || n >= N) return;
    const int32_t k = rows[i];
    // An index outside the table yields a NaN row instead of an out-of-bounds read.
    out[static_cast<size_t>(i) * N + n] = (k >= 0 && k < K) ? row_value(q, s, z, bits, bpr, N, g, k, n) : __builtin_nanf("");
}

__global__ void __launch_bounds__(256)
    dequant_columns_kernel(const uint8_t* __restrict__ q, const float* __restrict__ s, const int8_t* __restrict__ z,
                           int32_t bits, int32_t bpr, int32_t K, int32_t N, int32_t g, const int32_t* __restrict__ cols,
                           int32_t count, float* __restrict__ out) {
    const int32_t row_blocks = ceil_div(K, 256);
    const int32_t i = blockIdx.x / row_blocks;
    const int32_t k = (blockIdx.x % row_blocks) * 256 + threadIdx.x;
    if (i >= count || k >= K) return;
    const int32_t n = cols[i];
    float* dst = out + static_cast<size_t>(i) * K + k;
    if (n < 0 || n >= N) {  // NaN instead of an out-of-bounds read
        *dst = __builtin_nanf("");
        return;
    }
    // value(): scale * (raw - zero), zero = 0 without zero points (QuantizedTensor.kt:182-186).
    const size_t idx = static_cast<size_t>(k / g) * N + n;
    const int32_t zero = z ? static_cast<int32_t>(z[idx]) : 0;
    *dst = s[idx] * static_cast<float>(raw_value(q, bits, bpr, k, n) - zero);
}

int32_t grid_1d(int64_t blocks, dim3* grid) {
    if (blocks <= 0 || blocks > INT32_MAX) return fail(KT_ERR_SHAPE, "grid of %lld blocks is out of range", static_cast<long long>(blocks));
    *grid = dim3(static_cast<uint32_t>(blocks));
    return KT_OK;
}

}  // namespace

int32_t launch_generic(const float* a, int32_t m, const WeightView& w, float* c, int32_t accumulate, float alpha,
                       const float* bias, hipStream_t st) {
    dim3 grid;
    int32_t status = grid_1d(static_cast<int64_t>(m) * ceil_div(w.N, 256), &grid);
    if (status) return status;
    generic_matmul<<<grid, 256, 0, st>>>(a, m, w.q, w.s, w.z, w.K, w.N, w.bits, w.bpr, w.g, c, bias, alpha, accumulate);
    KT_LAUNCHED("qmatmul: generic kernel");
    return KT_OK;
}

int32_t launch_transposed(const float* dy, int32_t m, const WeightView& w, float* dx, int32_t accumulate,
                          hipStream_t st) {
    dim3 grid;
    int32_t status = grid_1d(static_cast<int64_t>(w.K) * ceil_div(m, TR_ROWS), &grid);
    if (status) return status;
    transposed_kernel<<<grid, 256, 0, st>>>(dy, m, w.q, w.s, w.z, w.K, w.N, w.bits, w.bpr, w.g, dx, accumulate);
    KT_LAUNCHED("qmatmul_transposed: kernel");
    return KT_OK;
}

int32_t launch_dequantize_rows(const WeightView& w, const int32_t* rows, int32_t count, float* out, hipStream_t st) {
    dim3 grid;
    int32_t status = grid_1d(static_cast<int64_t>(count) * ceil_div(w.N, 256), &grid);
    if (status) return status;
    dequant_rows_kernel<<<grid, 256, 0, st>>>(w.q, w.s, w.z, w.bits, w.bpr, w.K, w.N, w.g, rows, count, out);
    KT_LAUNCHED("dequantize_rows: kernel");
    return KT_OK;
}

int32_t launch_dequantize_columns(const WeightView& w, const int32_t* cols, int32_t count, float* out,
                                  hipStream_t st) {
    dim3 grid;
    int32_t status = grid_1d(static_cast<int64_t>(count) * ceil_div(w.K, 256), &grid);
    if (status) return status;
    dequant_columns_kernel<<<grid, 256, 0, st>>>(w.q, w.s, w.z, w.bits, w.bpr, w.K, w.N, w.g, cols, count, out);
    KT_LAUNCHED("dequantize_columns: kernel");
    return KT_OK;
}

}  // namespace kt
