// kt_loss.hip -- the fused projection + cross-entropy with a quantized head:
// fusedCrossEntropyLoss(hidden, QuantizedLinear head, targets, ignoreIndex)
// (Engine/kotensor/src/main/kotlin/Loss.kt:114-219), forward loss and the gradients its
// backward closure adds for an upstream gradient of 1.
//
// Like the reference, the active rows (those whose target is not ignore_index) are
// gathered in order and go through in chunks of 2^22 / N of them (activeRows,
// projectRows, Loss.kt:129-133, :236-260), so the logits never exist for all rows at
// once, and a chunk's rows, and with them the kernel that makes its logits, do not depend
// on how many ignored rows lie between them. Per chunk: the logits by kt_qmatmul
// (the prefill GEMM or the small-M kernels, with the bias), one workgroup per row for the
// row's max, sum of exponentials, loss and (in place) its logit gradients
// scale * (softmax - onehot) (logitGradients, Loss.kt:275-291), then the bias gradient as
// column sums in row order and the hidden gradient by the transposed product
// (MatMul.multiplyByQuantizedTransposed, K/MatMul.kt:954-981). exp and ln are Kotlin's
// Float forms: the double function rounded to float. The hidden gradient of a chunk goes
// back to its rows' places; ignored rows get zero (or keep theirs, accumulating). The
// per-row losses are added in a fixed order at the end, so the result does not depend
// on timing.
#include "kt_common.h"

#include <vector>

namespace kt {
namespace {

constexpr int CE_THREADS = 256;
constexpr int32_t FUSED_CHUNK_ELEMENTS = 1 << 22;  // Loss.kt:8

__device__ __forceinline__ float kexp(float x) { return static_cast<float>(exp(static_cast<double>(x))); }
__device__ __forceinline__ float kln(float x) { return static_cast<float>(log(static_cast<double>(x))); }

// Block reductions in a fixed order: lanes by xor butterfly, then the four waves in order.
__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int w = 1; w < CE_THREADS / 64; ++w) m = fmaxf(m, red[w]);
    return m;
}
__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const int wave = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[wave] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int w = 1; w < CE_THREADS / 64; ++w) s += red[w];
    return s;
}

// One workgroup per row of the chunk: the loss term max + ln(sum) - l[target]
// (Loss.kt:146-164, the max starting at -1e9 as there) and, with grads, the logit
// gradients in place.
__global__ void __launch_bounds__(CE_THREADS)
    ce_rows_kernel(float* __restrict__ logits, int32_t V, const int32_t* __restrict__ targets, int32_t ignore,
                   float scale, float* __restrict__ row_loss, int32_t grads) {
    __shared__ float red[CE_THREADS / 64];
    const int32_t r = blockIdx.x;
    float* l = logits + static_cast<int64_t>(r) * V;
    const int32_t t = targets[r];
    if (t == ignore) {
        if (threadIdx.x == 0) row_loss[r] = 0.0f;
        if (grads)
            for (int32_t v = threadIdx.x; v < V; v += CE_THREADS) l[v] = 0.0f;
        return;
    }
    float m = -1e9f;
    for (int32_t v = threadIdx.x; v < V; v += CE_THREADS) m = fmaxf(m, l[v]);
    m = block_max(m, red);
    float s = 0.0f;
    for (int32_t v = threadIdx.x; v < V; v += CE_THREADS) s += kexp(l[v] - m);
    s = block_sum(s, red);
    if (threadIdx.x == 0) row_loss[r] = m + kln(s) - l[t];
    if (!grads) return;
    __syncthreads();  // l[t] is read above before any thread overwrites it
    const float inv = 1.0f / s;
    for (int32_t v = threadIdx.x; v < V; v += CE_THREADS) {
        const float prob = kexp(l[v] - m) * inv;
        l[v] = scale * (prob - (v == t ? 1.0f : 0.0f));
    }
}

// bias_grad[v] = (accumulate ? bias_grad[v] : 0) + the chunk's column sum, rows in order.
__global__ void __launch_bounds__(256)
    ce_bias_grad_kernel(const float* __restrict__ g, int32_t count, int32_t V, float* __restrict__ bias_grad,
                        int32_t accumulate) {
    const int32_t v = blockIdx.x * 256 + threadIdx.x;
    if (v >= V) return;
    float s = 0.0f;
    for (int32_t r = 0; r < count; ++r) s += g[static_cast<int64_t>(r) * V + v];
    bias_grad[v] = accumulate ? bias_grad[v] + s : s;
}

// The mean over the active rows of the per-row losses, added in a fixed order.
__global__ void __launch_bounds__(CE_THREADS)
    ce_loss_kernel(const float* __restrict__ row_loss, int32_t rows, int32_t active, float* __restrict__ loss) {
    __shared__ float red[CE_THREADS / 64];
    float s = 0.0f;
    for (int32_t r = threadIdx.x; r < rows; r += CE_THREADS) s += row_loss[r];
    s = block_sum(s, red);
    if (threadIdx.x == 0) *loss = active > 0 ? s / static_cast<float>(active) : 0.0f;
}

// dst[r] = src[rows[r]] for the chunk's rows (K floats each): the gathered input.
__global__ void __launch_bounds__(256)
    gather_rows_kernel(const float* __restrict__ src, int32_t K, const int32_t* __restrict__ rows,
                       float* __restrict__ dst) {
    const float* s = src + static_cast<int64_t>(rows[blockIdx.x]) * K;
    float* d = dst + static_cast<int64_t>(blockIdx.x) * K;
    for (int32_t k = threadIdx.x; k < K; k += 256) d[k] = s[k];
}

// dst[rows[r]] (+)= src[r]: the chunk's hidden gradient back to its rows' places.
__global__ void __launch_bounds__(256)
    scatter_rows_kernel(const float* __restrict__ src, int32_t K, const int32_t* __restrict__ rows,
                        float* __restrict__ dst, int32_t accumulate) {
    const float* s = src + static_cast<int64_t>(blockIdx.x) * K;
    float* d = dst + static_cast<int64_t>(rows[blockIdx.x]) * K;
    for (int32_t k = threadIdx.x; k < K; k += 256) d[k] = accumulate ? d[k] + s[k] : s[k];
}

__global__ void fill_kernel(float* __restrict__ p, int64_t n, float value) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
        p[i] = value;
}

int32_t fill(float* p, int64_t n, float value, hipStream_t st) {
    if (n <= 0) return KT_OK;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
    fill_kernel<<<static_cast<uint32_t>(blocks), 256, 0, st>>>(p, n, value);
    KT_LAUNCHED("fused cross-entropy: fill");
    return KT_OK;
}

}  // namespace
}  // namespace kt

using namespace kt;

extern "C" int32_t kt_fused_cross_entropy(const float* hidden, int32_t rows, const kt_qweight* head, const float* bias,
                                          const int32_t* targets, int32_t ignore_index, float* loss,
                                          float* hidden_grad, float* bias_grad, int32_t accumulate, void* stream) {
    WeightView w;
    int32_t status = view_weight(head, &w);
    if (status) return status;
    if (rows <= 0 || !targets) return fail(KT_ERR_ARGUMENT, "targets cannot be empty");
    if (!hidden || !loss) return fail(KT_ERR_ARGUMENT, "fused cross-entropy with a NULL hidden or loss");
    const int32_t V = w.N, K = w.K;
    // activeRows (Loss.kt:236-249): every target is ignore_index or in [0, V); the active
    // rows' indices, then their targets, in row order
    std::vector<int32_t> act;
    for (int32_t i = 0; i < rows; ++i) {
        if (targets[i] == ignore_index) continue;
        if (targets[i] < 0 || targets[i] >= V) return fail(KT_ERR_ARGUMENT, "target %d out of bounds %d", targets[i], V);
        act.push_back(i);
    }
    const int32_t active = static_cast<int32_t>(act.size());
    for (int32_t i = 0; i < active; ++i) act.push_back(targets[act[i]]);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const bool grads = hidden_grad || bias_grad;
    if (active == 0) {  // emptyLoss(): no gradient flows
        if ((status = fill(loss, 1, 0.0f, st))) return status;
        if (!accumulate && hidden_grad && (status = fill(hidden_grad, static_cast<int64_t>(rows) * K, 0.0f, st)))
            return status;
        if (!accumulate && bias_grad && (status = fill(bias_grad, V, 0.0f, st))) return status;
        return KT_OK;
    }
    const int32_t chunk = std::max(1, std::min(FUSED_CHUNK_ELEMENTS / V, active));  // chunkRows
    // device scratch for this call: the chunk's logits, its gathered rows and their hidden
    // gradient, the per-row losses, the active rows' indices and targets
    const size_t logit_bytes = static_cast<size_t>(chunk) * V * sizeof(float);
    const size_t row_bytes = static_cast<size_t>(chunk) * K * sizeof(float);
    const size_t bytes = logit_bytes + 2 * row_bytes + static_cast<size_t>(active) * (sizeof(float) + 2 * sizeof(int32_t));
    void* scratch = nullptr;
    KT_HIP(hipMallocAsync(&scratch, bytes, st));
    float* logits = static_cast<float*>(scratch);
    float* inputs = reinterpret_cast<float*>(static_cast<char*>(scratch) + logit_bytes);
    float* chunk_grad = reinterpret_cast<float*>(static_cast<char*>(scratch) + logit_bytes + row_bytes);
    float* row_loss = reinterpret_cast<float*>(static_cast<char*>(scratch) + logit_bytes + 2 * row_bytes);
    int32_t* drows = reinterpret_cast<int32_t*>(row_loss + active);
    int32_t* dtargets = drows + active;
    status = [&]() -> int32_t {
        // pageable source: the copy has read it when the call returns
        KT_HIP(hipMemcpyAsync(drows, act.data(), act.size() * sizeof(int32_t), hipMemcpyHostToDevice, st));
        if (hidden_grad && !accumulate) {  // ignored rows' gradient is zero
            const int32_t f = fill(hidden_grad, static_cast<int64_t>(rows) * K, 0.0f, st);
            if (f) return f;
        }
        const float scale = 1.0f / static_cast<float>(active);
        for (int32_t start = 0; start < active; start += chunk) {
            const int32_t count = std::min(chunk, active - start);
            gather_rows_kernel<<<count, 256, 0, st>>>(hidden, K, drows + start, inputs);
            KT_LAUNCHED("fused cross-entropy: gather rows");
            int32_t s = qmatmul(inputs, count, head, logits, 0, 1.0f, bias, st);
            if (s) return s;
            ce_rows_kernel<<<count, CE_THREADS, 0, st>>>(logits, V, dtargets + start, ignore_index, scale,
                                                         row_loss + start, grads ? 1 : 0);
            KT_LAUNCHED("fused cross-entropy: rows");
            if (bias_grad) {
                ce_bias_grad_kernel<<<ceil_div(V, 256), 256, 0, st>>>(logits, count, V, bias_grad,
                                                                       (accumulate || start > 0) ? 1 : 0);
                KT_LAUNCHED("fused cross-entropy: bias gradient");
            }
            if (hidden_grad) {
                s = launch_transposed(logits, count, w, chunk_grad, 0, st);
                if (s) return s;
                scatter_rows_kernel<<<count, 256, 0, st>>>(chunk_grad, K, drows + start, hidden_grad, accumulate);
                KT_LAUNCHED("fused cross-entropy: scatter rows");
            }
        }
        ce_loss_kernel<<<1, CE_THREADS, 0, st>>>(row_loss, active, active, loss);
        KT_LAUNCHED("fused cross-entropy: loss");
        return KT_OK;
    }();
    const hipError_t freed = hipFreeAsync(scratch, st);
    if (status) return status;
    if (freed != hipSuccess) return hip_fail(freed, "hipFreeAsync");
    return KT_OK;
}
