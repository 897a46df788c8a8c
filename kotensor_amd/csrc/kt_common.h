// kt_common.h -- internals shared by the translation units of libkotensor_hip.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kotensor_hip.h"

namespace kt {

// Records a message for kt_last_error() on the calling thread and returns status.
int32_t fail(int32_t status, const char* fmt, ...);
// Maps a HIP error to a positive status (and records its message).
int32_t hip_fail(hipError_t err, const char* what);

#define KT_HIP(call)                                             \
    do {                                                         \
        hipError_t kt_err_ = (call);                             \
        if (kt_err_ != hipSuccess) return ::kt::hip_fail(kt_err_, #call); \
    } while (0)

// Checks the launch that was just enqueued.
#define KT_LAUNCHED(name)                                        \
    do {                                                         \
        hipError_t kt_err_ = hipGetLastError();                  \
        if (kt_err_ != hipSuccess) return ::kt::hip_fail(kt_err_, name); \
    } while (0)

// Device workspace owned by the library, one per (device, stream). Calls on one
// stream are ordered by that stream, so they may reuse the same bytes. Growing it
// waits for the stream before the old allocation is released.
int32_t workspace(hipStream_t stream, size_t bytes, void** out);
// The same workspace plus `count` uint32 counters that are zero on entry; a kernel
// that takes them must leave every one at zero when it completes.
int32_t workspace_counters(hipStream_t stream, size_t bytes, size_t count, void** general, uint32_t** counters);
// The counter region holds 16384 words; the last 512 are the decode attention's RoPE
// cache (ROPE_CACHE_WORD), which keeps its contents between calls.
constexpr size_t MAX_COUNTERS = (64 << 10) / sizeof(uint32_t) - 512;
constexpr size_t ROPE_CACHE_WORD = MAX_COUNTERS;
// The counters plus `doubles` fp64 accumulators that are zero on entry; a kernel that
// uses them leaves them at zero.
int32_t workspace_accumulators(hipStream_t stream, size_t count, size_t doubles, uint32_t** counters, double** accs);
// The counters, `doubles` zeroed fp64 words (left at zero by the kernel, as above) and
// `bytes` of general area, all of one stream's workspace.
int32_t workspace_regions(hipStream_t stream, size_t doubles, size_t bytes, uint32_t** counters, double** accs,
                          void** general);

// Give-up reports of bounded waits. A kernel whose wait runs out of polls stores a
// nonzero code into its stream's fault word (pinned host memory mapped into the device;
// nullptr for calls on a caller's fixed workspace, which run no waiting kernel), goes on,
// and the stream's next kt_stream_sync / kt_memcpy_d2h returns KT_ERR_STATE after
// re-zeroing the stream's counters (a late producer may have left words behind).
constexpr int32_t FAULT_CHAIN_WAIT = 1;  // a chained stage's wait for the previous stage's flags
constexpr int32_t FAULT_MERGE_WAIT = 2;  // the decode attention's wait for other splits' sums
int32_t stream_fault_word(hipStream_t stream, int32_t** dev_word);
// The poll budget of the waits (0 = each kernel's own default) and whether producers
// withhold their signals, both set by kt_debug_wait_limits for tests of the give-up path.
struct WaitLimits {
    uint32_t spin_limit;
    int32_t withhold;
};
WaitLimits wait_limits();

// Validated view of a kt_qweight, with the derived layout numbers.
struct WeightView {
    const uint8_t* q;
    const float* s;
    const int8_t* z;  // nullptr when the weight has no zero points
    const uint8_t* p;  // the column-run copy (kt_qweight_pack), or nullptr
    int32_t K, N, bits, g, G, bpr;
};
int32_t view_weight(const kt_qweight* w, WeightView* v);

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }
__host__ __device__ inline int32_t ceil_div(int32_t a, int32_t b) { return (a + b - 1) / b; }

// RMSNorm's reduction (K/RMSNorm.kt), shared by rmsnorm_kernel and the GEMV that takes
// RMSNorm's input row, so both get the same scale r = 1 / sqrt(mean(x^2) + eps): thread
// t < NORM_THREADS sums squares over the float4s t, t + 256, ... (zero past the row) in
// this fmaf order, each 64-lane wave adds its lanes by xor butterfly, and the four wave
// sums are added in wave order.
constexpr int NORM_THREADS = 256;
constexpr int NORM_F4 = 8;  // float4 per thread: rows of up to 8192 floats
typedef float norm_v4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float norm_wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
__device__ __forceinline__ float norm_partial(const norm_v4 (&v)[NORM_F4], int32_t tid, int32_t n4) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NORM_F4; ++i) {
        const norm_v4 u = tid + i * NORM_THREADS < n4 ? v[i] : norm_v4{0.0f, 0.0f, 0.0f, 0.0f};
        s = fmaf(u[0], u[0], fmaf(u[1], u[1], fmaf(u[2], u[2], fmaf(u[3], u[3], s))));
    }
    return s;
}
__device__ __forceinline__ float norm_scale(const float (&wave_sums)[NORM_THREADS / 64], int32_t dim, float eps) {
    float total = 0.0f;
#pragma unroll
    for (int i = 0; i < NORM_THREADS / 64; ++i) total += wave_sums[i];
    return 1.0f / sqrtf(total / static_cast<float>(dim) + eps);
}

// Number of compute units of the current device (cached per device).
int32_t cu_count();

// Launch entry points implemented by the kernel translation units. All take
// validated arguments. bias may be nullptr; partial results never leave the stream.
// A NaN input stores epoch into *nan_slot (device address of pinned host memory).
int32_t launch_quantize(const float* data, int32_t K, int32_t N, int32_t bits, int32_t g,
                        uint8_t* q, float* s, int8_t* z, int32_t* nan_slot, int32_t epoch, hipStream_t st);
int32_t launch_gemv(const float* a, const WeightView& w, float* c, int32_t accumulate, float alpha,
                    const float* bias, hipStream_t st);
// One launch for up to four weights that share the input row (same K, bits, group size).
int32_t launch_gemv_group(const float* a, const WeightView* ws, float* const* cs, const float* const* biases,
                          int32_t count, int32_t accumulate, float alpha, hipStream_t st);
int32_t launch_gemm(const float* a, int32_t m, const WeightView& w, float* c, int32_t accumulate,
                    float alpha, const float* bias, hipStream_t st);
// Weights sharing a (K, bits, group size, zero points): one x preparation and one GEMM launch.
int32_t launch_gemm_group(const float* a, int32_t m, const WeightView* ws, float* const* cs, const float* const* biases,
                          int32_t count, int32_t accumulate, float alpha, hipStream_t st);
int32_t launch_generic(const float* a, int32_t m, const WeightView& w, float* c, int32_t accumulate,
                       float alpha, const float* bias, hipStream_t st);
int32_t launch_transposed(const float* dy, int32_t m, const WeightView& w, float* dx,
                          int32_t accumulate, hipStream_t st);
int32_t launch_dequantize_rows(const WeightView& w, const int32_t* rows, int32_t count, float* out,
                               hipStream_t st);
int32_t launch_dequantize_columns(const WeightView& w, const int32_t* cols, int32_t count, float* out,
                                  hipStream_t st);

// Forces the lane vector width, split count and waves per workgroup of the M == 1
// kernel (0 = automatic).
void set_gemv_config(int32_t vec, int32_t splits, int32_t waves);
// How split sums are combined: 0 automatic, 1 reduction kernel, 2 inside the kernel.
void set_gemv_reduce_mode(int32_t mode);

// The MFMA GEMV for 1..16 rows: support check, launch (up to four weights sharing the
// input) and its knobs (0 = automatic; disable routes M == 1 to the VALU GEMV).
bool gemv_mfma_supported(const float* a, int32_t m, const WeightView& w, const float* c);
int32_t launch_gemv_mfma(const float* a, int32_t M, const WeightView* ws, float* const* cs, const float* const* biases,
                         int32_t count, int32_t accumulate, float alpha, hipStream_t st);
void set_gemv_mfma_config(int32_t slices, int32_t waves, int32_t reduce, int32_t disable);
// The M == 1 MFMA kernel on 512-byte row strips (kt_gemv_wide.hip).
bool gemv_wide_supported(const float* a, int32_t m, const WeightView& w, const float* c);
int32_t launch_gemv_wide(const float* a, const WeightView* ws, float* const* cs, const float* const* biases, int32_t count,
                         int32_t accumulate, float alpha, hipStream_t st, const float* up = nullptr,
                         const float* norm_weight = nullptr, float eps = 0.0f);
void set_gemv_wide_config(int32_t slices, int32_t waves);
// The kernel choice of kt_set_kernel_config (0 automatic).
int32_t gemv_kind();
// kt_qmatmul with a bias (kt_qlinear_forward with accumulate and alpha).
int32_t qmatmul(const float* a, int32_t m, const kt_qweight* w, float* c, int32_t accumulate, float alpha,
                const float* bias, void* stream);
// Whether the automatic choice takes the wide-strip kernel for these weights.
bool gemv_wide_preferred(const WeightView* ws, int32_t count);
// The M == 1 latency kernel on 16-byte column strips over all of K (kt_gemv_strip.hip).
bool gemv_strip_supported(const float* a, int32_t m, const WeightView& w, const float* c);
int32_t launch_gemv_strip(const float* a, const WeightView* ws, float* const* cs, const float* const* biases,
                          int32_t count, int32_t accumulate, float alpha, hipStream_t st);
// Whether the automatic choice takes the column-strip kernel for these weights.
bool gemv_strip_preferred(const WeightView* ws, int32_t count);

// The one-row GEMV on the column-run copy (kt_gemv_packed.hip): bytes of the copy, the
// kernel that writes it, support check, launch (up to four weights sharing the input;
// up = SwiGLU's up row, norm_weight = RMSNorm's weight, as in launch_gemv_wide) and its
// knobs (K-parts per column set, waves per workgroup, ring depth 4 or 8 = 8 or 16 KB per
// wave; 0 = automatic).
int64_t packed_bytes(int32_t rows, int32_t columns, int32_t bits, int32_t group_size);
int64_t packed_weight_bytes(int32_t rows, int32_t columns, int32_t bits);  // the weight blocks alone
// The copy ends in a 16-byte trailer: the largest |scale| of the weight (fp32), then zeros.
constexpr int64_t PACKED_TRAILER_BYTES = 16;
const float* packed_scale_max(const WeightView& w);  // the trailer's maximum (device address)
int32_t launch_pack(const WeightView& w, void* packed, hipStream_t st);
bool gemv_packed_supported(const float* a, int32_t m, const WeightView& w, const float* c);
// glu: ws[0], ws[1] are SwiGLU's gate and up weights; cs[0] receives silu(gate) * up and
// cs[1] up (no accumulate); needs gemv_packed_pair_supported.
int32_t launch_gemv_packed(const float* a, const WeightView* ws, float* const* cs, const float* const* biases,
                           int32_t count, int32_t accumulate, float alpha, hipStream_t st, const float* up = nullptr,
                           const float* norm_weight = nullptr, float eps = 0.0f, bool glu = false);
bool gemv_packed_pair_supported(const float* a, const WeightView* ws, float* const* cs);
// Dependent column-run GEMVs as one launch (each step's input may be an earlier step's
// output): the arguments of one launch_gemv_packed call per step.
struct ChainStep {
    const float* a;
    const WeightView* ws;
    float* const* cs;
    const float* const* biases;
    int32_t count, accumulate;
    float alpha;
    const float* up;
    const float* norm_weight;
    float eps;
    bool glu;
};
int32_t gemv_chain_max_steps();
int32_t gemv_chain_max_k();  // the longest input row a chained step takes
int32_t launch_gemv_chain(const ChainStep* steps, int32_t n, hipStream_t st);
void set_gemv_packed_config(int32_t ks, int32_t waves, int32_t ring);
void set_gemv_rows_packed_reduce(int32_t mode);  // 0 automatic, 1 K-parts meet in the workgroup, 2 across
int32_t packed_forced_ks();  // the K-parts set by set_gemv_packed_config (0: automatic)
// 2..16 rows of small weights as one-row products in one launch (each row's bits are its
// one-row result): the automatic choice's rule, and the launches (one weight; up to four
// sharing x).
bool gemv_packed_rows_rep_preferred(int32_t m, const WeightView* ws, int32_t count);
int32_t launch_gemv_packed_rows_rep(const float* a, int32_t m, const WeightView& w, float* c, const float* bias,
                                    int32_t accumulate, float alpha, hipStream_t st);
int32_t launch_gemv_packed_group_rep(const float* a, int32_t m, const WeightView* ws, float* const* cs,
                                     const float* const* biases, int32_t count, int32_t accumulate, float alpha,
                                     hipStream_t st);

// 2 to 16 rows on the column-run copy (kt_gemv_rows_packed.hip): support check and launch
// (up to four weights sharing the input: one preparation of x, one launch per weight).
bool gemv_rows_packed_supported(const float* a, int32_t m, const WeightView& w, const float* c);
bool gemv_rows_packed_preferred(const WeightView& w);  // the automatic choice takes it
int32_t launch_gemv_rows_packed(const float* a, int32_t m, const WeightView* ws, float* const* cs,
                                const float* const* biases, int32_t count, int32_t accumulate, float alpha,
                                hipStream_t st);

// Whether the fast GEMV / GEMM kernels accept this weight (layout and alignment);
// otherwise the generic kernel runs.
bool gemv_supported(const float* a, const WeightView& w, const float* c);
bool gemm_supported(const float* a, int32_t m, const WeightView& w, const float* c);

}  // namespace kt
