// kt_gemv_strip.hip -- the M == 1 dequant-GEMV for small and medium weights, built for
// latency: c[1 x N] = (accumulate ? c : 0) + alpha * x[1 x K] . deq(W) (+ bias),
// MatMul.multiplyQuantizedRow (Engine/kotensor/src/main/kotlin/MatMul.kt:494-536).
//
// A decode step is a chain of small products (0.1-16 MB each): their time is the launch
// plus the longest dependent chain of memory round trips inside the kernel, not the
// bytes. Measured on MI355X in graph replay: an empty kernel costs 1.7 us, one that
// also reads 1 MB cold 1.8 us, and one more device-scope atomic round trip (the counter
// of a last-arriver reduction) 4.5 us. So this kernel has no reduction across
// workgroups at all:
//
//   * a workgroup owns a 16-byte column strip of the packed rows over all of K
//     (32 columns for INT4: low nibbles b0..b0+15 and high nibbles H+b0.., H = bytes
//     per row; 16 columns for INT8) and writes its outputs itself;
//   * thread t takes the contiguous rows [t*RB, t*RB + RB) (RB a multiple of 8 chosen so
//     that 256 threads cover K), in chunks of 8 rows whose weights and x are in flight
//     while the previous chunk computes; a chunk never straddles a group, and a group's
//     scales are loaded with its first chunk;
//   * the time to the first weight load is one batch of argument loads: the job of a
//     grouped launch is blockIdx.y, and no branch precedes the loads;
//   * per group, sum(x * q) per column and sum(x) in fp32, then
//     out += scale * (sum(x*q) - zero * sum(x)) -- the reference's combineGroup form
//     (MatMul.kt:804-828); the threads' partial outputs meet in LDS;
//   * XCD-aware strip order: workgroup i runs on XCD i % 8, and the eight strips that
//     share a 128-byte line of a row go to eight workgroups of the same XCD dispatched
//     together, so that XCD's L2 fetches each line from HBM once.
#include "kt_common.h"

#include <algorithm>

namespace kt {
namespace {

constexpr int THREADS = 256;
constexpr int MAX_JOBS = 4;
constexpr int CH = 8;  // rows per chunk
// The automatic choice takes this kernel for K <= 2048 (one chunk of 8 rows per thread)
// up to these packed weight bytes per launch; past them the wide MFMA kernel, which
// spreads a product over all CUs, is faster (MI355X, graph replay: Qwen2-0.5B q/k/v
// 6.9 us against 8.8, 2048x2048 INT4 7.7 against 8.0, INT8 5.8 against 6.4; a
// 2048 -> 3072 INT4 group 8.8 against 8.0).
constexpr int32_t STRIP_MAX_K = 2048;
constexpr int64_t STRIP_MAX_BYTES_INT4 = int64_t(5) << 19;  // 2.5 MiB
constexpr int64_t STRIP_MAX_BYTES_INT8 = int64_t(9) << 19;  // 4.5 MiB

struct StripJob {
    const uint8_t* q;
    const float* s;
    const int8_t* z;
    float* out;
    const float* bias;
    int32_t N, bpr, strips;  // strips = bpr / 16
};

struct StripJobs {
    StripJob job[MAX_JOBS];  // job j runs on the workgroups with blockIdx.y == j
};

// Byte j of w as a float (one v_cvt_f32_ubyte{j}).
__device__ __forceinline__ float byte_u(uint32_t w, int j) { return static_cast<float>((w >> (8 * j)) & 0xFFu); }
__device__ __forceinline__ float byte_s(uint32_t w, int j) {
    return static_cast<float>(static_cast<int32_t>(w << (24 - 8 * j)) >> 24);
}

template <int BITS, bool ZP>
__global__ void __launch_bounds__(THREADS) gemv_strip_kernel(StripJobs jobs, const float* __restrict__ x, int32_t K,
                                                             int32_t g, int32_t rb, int32_t accumulate,
                                                             float alpha) {
    constexpr int NC = BITS == 4 ? 32 : 16;  // columns per strip
    __shared__ float red[THREADS][NC + 1];

    // The job is blockIdx.y, known when the wave starts, so its fields need no other
    // loaded value. The empty asm reads every argument at once: the compiler then
    // issues all the argument loads as one batch with one wait, instead of sinking
    // each next to its first use (three dependent scalar round trips, about 0.5 us
    // each, before the first weight load).
    const StripJob jb = jobs.job[blockIdx.y];
    asm volatile("" ::"s"(x), "s"(K), "s"(g), "s"(rb), "s"(accumulate), "s"(alpha), "s"(jb.q), "s"(jb.s), "s"(jb.z),
                 "s"(jb.out), "s"(jb.bias), "s"(jb.N), "s"(jb.bpr), "s"(jb.strips));
    // XCD-aware strip order: workgroup i runs on XCD i % 8, so each whole block of 64
    // workgroups hands strips 8j..8j+7 (one 128-byte line of a row) to eight workgroups
    // of XCD j % 8; the last partial block keeps the plain order. A workgroup past its
    // job's strips (a grouped launch whose jobs differ in width) reads strip 0 and
    // writes nothing: no early exit, whose branch would hold back the argument loads.
    const int32_t i = blockIdx.x, full = jb.strips & ~63;
    int32_t f = i;
    if (i < full) {
        const int32_t xcd = i & 7, k = (i >> 3) & 7;
        f = (i & ~63) + 8 * xcd + k;
    }
    const bool live = f < jb.strips;
    if (!live) f = 0;
    const int32_t b0 = f * 16;  // first byte of the strip in a row
    const int32_t N = jb.N, H = jb.bpr;

    const int32_t t = threadIdx.x;
    const int32_t r0 = t * rb;
    const int32_t r1 = min(K, r0 + rb);

    // threads 0..NC-1 write column b0 + t % 16 (INT4: of the high half for t >= 16);
    // what the epilogue adds to their sums (the old output, the bias) is loaded now
    const int32_t ebyte = b0 + (t & 15);
    const int32_t ecol = (BITS == 4 && t >= 16) ? H + ebyte : ebyte;
    const bool writer = live && t < NC && ecol < N;
    // (unconditional loads from valid addresses, then selects: a branch here would
    // also hold back the argument loads the main loop needs)
    const int32_t lcol = writer ? ecol : 0;
    const float old_out = jb.out[lcol];
    const float bias_in = (jb.bias ? jb.bias : jb.out)[lcol];
    const float prior = accumulate ? old_out : 0.0f;
    const float badd = jb.bias ? bias_in : 0.0f;

    float out[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) out[c] = 0.0f;

    // Every thread runs rb / 8 chunks (a uniform loop, no branch that would wait on
    // loads in flight); rows at or past r1 load row r1 - 1 (K - 1 for a thread past K)
    // and take x = 0, adding exact zeros.
    const int32_t last = r1 > r0 ? r1 - 1 : K - 1;
    const int32_t nch = rb / CH;
    float acc[NC];
    float sx = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) acc[c] = 0.0f;
    // chunk loads: 8 rows of 16 bytes and their 8 x values
    auto load_w = [&](uint4 (&w)[CH], int32_t c0) {
#pragma unroll
        for (int r = 0; r < CH; ++r) {
            const int32_t row = min(c0 + r, last);
            w[r] = *reinterpret_cast<const uint4*>(jb.q + static_cast<size_t>(row) * H + b0);
        }
    };
    auto load_x = [&](float (&xv)[CH], int32_t c0) {
#pragma unroll
        for (int r = 0; r < CH; ++r) xv[r] = x[min(c0 + r, last)];
    };
    // a group's scales (and zero points): the first group's are loaded with the first
    // chunk, a later group's when the one before it closes
    float4 sc4[NC / 4];
    uint32_t zw[NC / 4];
    auto load_scales = [&](int32_t gi) {
        const float* sp = jb.s + static_cast<size_t>(gi) * N;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            sc4[q4] = *reinterpret_cast<const float4*>(sp + b0 + 4 * q4);
            if constexpr (BITS == 4) sc4[4 + q4] = *reinterpret_cast<const float4*>(sp + H + b0 + 4 * q4);
        }
        if constexpr (ZP) {
            const int8_t* zp = jb.z + static_cast<size_t>(gi) * N;
            const uint4 za = *reinterpret_cast<const uint4*>(zp + b0);
            zw[0] = za.x; zw[1] = za.y; zw[2] = za.z; zw[3] = za.w;
            if constexpr (BITS == 4) {
                const uint2 zb0 = *reinterpret_cast<const uint2*>(zp + H + b0);
                const uint2 zb1 = *reinterpret_cast<const uint2*>(zp + H + b0 + 8);
                zw[4] = zb0.x; zw[5] = zb0.y; zw[6] = zb1.x; zw[7] = zb1.y;
            }
        }
    };
    auto flush = [&]() {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            const float4 a = sc4[c >> 2];
            const float scv = (c & 3) == 0 ? a.x : (c & 3) == 1 ? a.y : (c & 3) == 2 ? a.z : a.w;
            const float d = ZP ? fmaf(-byte_s(zw[c >> 2], c & 3), sx, acc[c]) : acc[c];
            out[c] = fmaf(scv, d, out[c]);
            acc[c] = 0.0f;
        }
        sx = 0.0f;
    };

    uint4 w[CH], wn[CH];
    float xv[CH], xn[CH];
    int32_t gi = min(r0, K - 1) / g;
    load_w(w, r0);
    load_x(xv, r0);
    load_scales(gi);
    __builtin_amdgcn_sched_barrier(0);  // the first loads all issue before any wait
    for (int32_t ch = 0, c0 = r0; ch < nch; ++ch, c0 += CH) {
        const bool more = ch + 1 < nch;  // uniform
        if (more) {
            load_w(wn, c0 + CH);
            load_x(xn, c0 + CH);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int r = 0; r < CH; ++r) {
            const float xr = c0 + r < r1 ? xv[r] : 0.0f;
            sx += xr;
            const uint32_t wd[4] = {w[r].x, w[r].y, w[r].z, w[r].w};
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                if constexpr (BITS == 4) {
                    const uint32_t lo = wd[d] & 0x0F0F0F0Fu, hi = (wd[d] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) {
                        acc[4 * d + jj] = fmaf(xr, byte_u(lo, jj), acc[4 * d + jj]);
                        acc[16 + 4 * d + jj] = fmaf(xr, byte_u(hi, jj), acc[16 + 4 * d + jj]);
                    }
                } else {
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) acc[4 * d + jj] = fmaf(xr, byte_s(wd[d], jj), acc[4 * d + jj]);
                }
            }
        }
        const int32_t next = c0 + CH;
        if (next >= r1 || next / g != gi) {  // the group ends with this chunk
            flush();
            if (next < r1) {
                gi = next / g;
                load_scales(gi);
            }
        }
        if (more) {
#pragma unroll
            for (int r = 0; r < CH; ++r) {
                w[r] = wn[r];
                xv[r] = xn[r];
            }
        }
    }

    // the threads' partial outputs meet in LDS: thread t sums column t % NC over a
    // slice of the threads, then one pass adds the slices
#pragma unroll
    for (int c = 0; c < NC; ++c) red[t][c] = out[c];
    __syncthreads();
    constexpr int SLICES = THREADS / NC;  // 8 (INT4) or 16 (INT8)
    const int32_t col = t % NC, sl = t / NC;
    float v = 0.0f;
    for (int32_t tt = sl; tt < THREADS; tt += SLICES) v += red[tt][col];
    __syncthreads();
    red[sl][col] = v;
    __syncthreads();
    if (writer) {
        float s = 0.0f;
#pragma unroll
        for (int p = 0; p < SLICES; ++p) s += red[p][t];
        float o = fmaf(alpha, s, prior);
        if (jb.bias) o += badd;
        jb.out[ecol] = o;
    }
}

}  // namespace

bool gemv_strip_preferred(const WeightView* ws, int32_t count) {
    int64_t bytes = 0;
    for (int32_t i = 0; i < count; ++i) bytes += static_cast<int64_t>(ws[i].K) * ws[i].bpr;
    if (ws[0].K > STRIP_MAX_K) return false;
    return bytes <= (ws[0].bits == 4 ? STRIP_MAX_BYTES_INT4 : STRIP_MAX_BYTES_INT8);
}

bool gemv_strip_supported(const float* a, int32_t m, const WeightView& w, const float* c) {
    (void)a;
    (void)c;
    if (m != 1) return false;
    if (w.bpr % 16 != 0 || !aligned(w.q, 16)) return false;     // 16-byte lane strips
    if (w.g % CH != 0) return false;                            // chunks inside one group
    if (!aligned(w.s, 16) || (w.z && !aligned(w.z, 16))) return false;
    if (w.bits == 4 && w.N % 16 != 0) return false;             // high-half scales 16-byte aligned
    if (w.bits == 8 && w.N % 4 != 0) return false;
    if (w.z && w.N % 16 != 0) return false;                     // zero-point rows 16-byte aligned
    return true;
}

int32_t launch_gemv_strip(const float* a, const WeightView* ws, float* const* cs, const float* const* biases,
                          int32_t count, int32_t accumulate, float alpha, hipStream_t st) {
    const WeightView& w0 = ws[0];
    bool zp = false;
    for (int32_t i = 0; i < count; ++i) zp = zp || ws[i].z != nullptr;
    if (zp)
        for (int32_t i = 0; i < count; ++i)
            if (!ws[i].z) return fail(KT_ERR_ARGUMENT, "grouped weights must all have zero points or none");
    if (count > MAX_JOBS) return fail(KT_ERR_ARGUMENT, "at most %d grouped weights", MAX_JOBS);
    StripJobs jobs{};
    int32_t most = 0;
    for (int32_t i = 0; i < count; ++i) {
        StripJob& jb = jobs.job[i];
        jb.q = ws[i].q;
        jb.s = ws[i].s;
        jb.z = ws[i].z;
        jb.out = cs[i];
        jb.bias = biases ? biases[i] : nullptr;
        jb.N = ws[i].N;
        jb.bpr = ws[i].bpr;
        jb.strips = ws[i].bpr / 16;
        most = std::max(most, jb.strips);
    }
    // rows per thread: a multiple of 8 that covers K with 256 threads
    int32_t rb = ceil_div(ceil_div(w0.K, THREADS), CH) * CH;
    if (rb < CH) rb = CH;
    const dim3 grid(static_cast<uint32_t>(most), static_cast<uint32_t>(count));
    if (w0.bits == 4)
        gemv_strip_kernel<4, true><<<grid, THREADS, 0, st>>>(jobs, a, w0.K, w0.g, rb, accumulate, alpha);
    else if (zp)
        gemv_strip_kernel<8, true><<<grid, THREADS, 0, st>>>(jobs, a, w0.K, w0.g, rb, accumulate, alpha);
    else
        gemv_strip_kernel<8, false><<<grid, THREADS, 0, st>>>(jobs, a, w0.K, w0.g, rb, accumulate, alpha);
    KT_LAUNCHED("qmatmul: strip gemv kernel");
    return KT_OK;
}

}  // namespace kt
