// kt_gemv.hip -- decode dequant-GEMV (M == 1) for gfx950:
//   c[N] = (accumulate ? c : 0) + alpha * x[K] . deq(W) (+ bias),
// the M == 1 branch of MatMul.multiplyQuantized (Engine/kotensor/src/main/kotlin/
// MatMul.kt:475-477 -> multiplyQuantizedRow :494-536 / rowUnitInto :599-682).
//
// HBM-bound: every packed weight byte, scale and zero is read exactly once.
// Work layout (reference layout, no repack):
//   * a lane owns VEC contiguous bytes of every row (VEC = 16, 8 or 4; 16 is one
//     128-bit load), so a wave reads 64*VEC contiguous bytes of a row per load;
//     for INT4 those bytes hold VEC low-nibble columns b.. and VEC high-nibble
//     columns half+b.. (split-half packing), for INT8 VEC columns;
//   * a workgroup is WAVES waves over the same column tile; wave w of split s
//     takes groups s*gps + w, s*gps + w + WAVES, ... so a wave always works on
//     whole groups and applies each group's scale and zero once;
//   * x[k] is uniform across the wave and lives in scalar registers, so the inner
//     loop is one v_cvt_f32_ubyte + one v_fma per weight; the signed INT8 byte is
//     biased by 128 (xor 0x80) and the bias folded into the zero-point term, the
//     INT4 high nibble is used in place (value 16*n) and rescaled by 1/16 exactly;
//   * per group: res += scale * (acc - zero * rowSum), acc = sum x[k]*q[k] and
//     rowSum = sum x[k] over the group's rows (the reference's combineGroup form);
//   * waves are combined through LDS in a fixed order; with more than one split,
//     partial sums go to a workspace and a second kernel adds them in split order,
//     so the result is bit-reproducible run to run.
#include "kt_common.h"

namespace kt {
namespace {

constexpr int WAVES = 4;
constexpr int UNROLL = 8;

template <int VEC>
struct Chunk;
template <>
struct Chunk<16> {
    using T = uint4;
    __device__ static uint32_t word(const T& v, int i) { return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w)); }
};
template <>
struct Chunk<8> {
    using T = uint2;
    __device__ static uint32_t word(const T& v, int i) { return i == 0 ? v.x : v.y; }
};
template <>
struct Chunk<4> {
    using T = uint32_t;
    __device__ static uint32_t word(const T& v, int) { return v; }
};

// Keeps the compiler from folding a byte mask into per-element bit-field extracts:
// after the mask, each byte converts with one v_cvt_f32_ubyte{0,1,2,3}.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

template <int BITS, int VEC>
__device__ __forceinline__ void accumulate_row(const typename Chunk<VEC>::T& v, float xk, float* acc) {
#pragma unroll
    for (int i = 0; i < VEC / 4; ++i) {
        const uint32_t w = Chunk<VEC>::word(v, i);
        if (BITS == 8) {
            const uint32_t u = opaque(w ^ 0x80808080u);  // q + 128 in every byte
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[4 * i + j] = fmaf(xk, static_cast<float>((u >> (8 * j)) & 0xFFu), acc[4 * i + j]);
        } else {
            const uint32_t lo = opaque(w & 0x0F0F0F0Fu);
            const uint32_t hi = opaque(w & 0xF0F0F0F0u);  // 16 * high nibble
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[4 * i + j] = fmaf(xk, static_cast<float>((lo >> (8 * j)) & 0xFFu), acc[4 * i + j]);
                acc[VEC + 4 * i + j] = fmaf(xk, static_cast<float>((hi >> (8 * j)) & 0xFFu), acc[VEC + 4 * i + j]);
            }
        }
    }
}

template <int BITS, int VEC>
__global__ void __launch_bounds__(64 * WAVES)
    gemv_kernel(const float* __restrict__ x, const uint8_t* __restrict__ q, const float* __restrict__ s,
                const int8_t* __restrict__ z, float* __restrict__ out, float* __restrict__ partials,
                const float* __restrict__ bias, int32_t K, int32_t N, int32_t bpr, int32_t g, int32_t G,
                int32_t tiles, int32_t gps, float alpha, int32_t accumulate) {
    using CT = typename Chunk<VEC>::T;
    constexpr int NC = BITS == 4 ? 2 * VEC : VEC;  // columns per lane
    __shared__ float red[WAVES][NC][64];

    const int32_t ln = threadIdx.x & 63;
    // Wave-uniform values in scalar registers: row offsets and x[k] then come from
    // SGPRs (x through the scalar cache) and each row load is base(SGPR) + lane offset.
    const int32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int32_t tile = blockIdx.x % tiles;
    const int32_t split = blockIdx.x / tiles;
    const int32_t boff = tile * 64 * VEC + ln * VEC;
    const bool active = boff < bpr;
    const int32_t half = bpr;
    const int32_t g_begin = split * gps;
    const int32_t g_end = min(g_begin + gps, G);

    float res[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) res[c] = 0.0f;

    if (active) {
        for (int32_t gi = g_begin + wave; gi < g_end; gi += WAVES) {
            const int32_t r0 = gi * g;
            const int32_t r1 = min(r0 + g, K);
            float acc[NC];
#pragma unroll
            for (int c = 0; c < NC; ++c) acc[c] = 0.0f;
            float rsum = 0.0f;
            int32_t l = r0;
            for (; l + UNROLL <= r1; l += UNROLL) {
                CT v[UNROLL];
#pragma unroll
                for (int u = 0; u < UNROLL; ++u)
                    v[u] = *reinterpret_cast<const CT*>(q + static_cast<size_t>(l + u) * bpr + boff);
                float xs[UNROLL];
#pragma unroll
                for (int u = 0; u < UNROLL; ++u) xs[u] = x[l + u];
#pragma unroll
                for (int u = 0; u < UNROLL; ++u) {
                    rsum += xs[u];
                    accumulate_row<BITS, VEC>(v[u], xs[u], acc);
                }
            }
            for (; l < r1; ++l) {
                const CT v = *reinterpret_cast<const CT*>(q + static_cast<size_t>(l) * bpr + boff);
                const float xk = x[l];
                rsum += xk;
                accumulate_row<BITS, VEC>(v, xk, acc);
            }
            // res += scale * (acc - zero * rowSum), per column.
            const float* srow = s + static_cast<size_t>(gi) * N;
            const int8_t* zrow = z ? z + static_cast<size_t>(gi) * N : nullptr;
#pragma unroll
            for (int side = 0; side < (BITS == 4 ? 2 : 1); ++side) {
                const int32_t col0 = side ? half + boff : boff;
                const float unit = side ? 0.0625f : 1.0f;
#pragma unroll
                for (int i = 0; i < VEC / 4; ++i) {
                    const float4 sc = *reinterpret_cast<const float4*>(srow + col0 + 4 * i);
                    uint32_t zw = 0;
                    if (zrow) zw = *reinterpret_cast<const uint32_t*>(zrow + col0 + 4 * i);
                    const float scv[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        float zero = static_cast<float>(static_cast<int8_t>((zw >> (8 * j)) & 0xFFu));
                        if (BITS == 8) zero += 128.0f;
                        const int c = side * VEC + 4 * i + j;
                        res[c] = fmaf(scv[j], fmaf(-zero, rsum, acc[c] * unit), res[c]);
                    }
                }
            }
        }
    }

#pragma unroll
    for (int c = 0; c < NC; ++c) red[wave][c][ln] = res[c];
    __syncthreads();
    if (wave != 0 || !active) return;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        float t = red[0][c][ln];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) t += red[w][c][ln];
        res[c] = t;
    }
#pragma unroll
    for (int side = 0; side < (BITS == 4 ? 2 : 1); ++side) {
        const int32_t col0 = side ? half + boff : boff;
#pragma unroll
        for (int i = 0; i < VEC / 4; ++i) {
            const int32_t col = col0 + 4 * i;
            const int c = side * VEC + 4 * i;
            float4 r = make_float4(res[c], res[c + 1], res[c + 2], res[c + 3]);
            if (partials) {
                *reinterpret_cast<float4*>(partials + static_cast<size_t>(split) * N + col) = r;
            } else {
                float4 o = accumulate ? *reinterpret_cast<const float4*>(out + col) : make_float4(0.f, 0.f, 0.f, 0.f);
                o.x = fmaf(alpha, r.x, o.x);
                o.y = fmaf(alpha, r.y, o.y);
                o.z = fmaf(alpha, r.z, o.z);
                o.w = fmaf(alpha, r.w, o.w);
                if (bias) {
                    const float4 b = *reinterpret_cast<const float4*>(bias + col);
                    o.x += b.x;
                    o.y += b.y;
                    o.z += b.z;
                    o.w += b.w;
                }
                *reinterpret_cast<float4*>(out + col) = o;
            }
        }
    }
}

// Adds the split partials in split order: out = (accumulate ? out : 0) + alpha * sum (+ bias).
__global__ void __launch_bounds__(256)
    gemv_reduce(const float* __restrict__ partials, int32_t splits, int32_t N, float* __restrict__ out,
                const float* __restrict__ bias, float alpha, int32_t accumulate) {
    const int32_t col = blockIdx.x * 256 + threadIdx.x;
    if (col >= N) return;
    float t = partials[col];
    for (int32_t sp = 1; sp < splits; ++sp) t += partials[static_cast<size_t>(sp) * N + col];
    float o = accumulate ? out[col] : 0.0f;
    o = fmaf(alpha, t, o);
    if (bias) o += bias[col];
    out[col] = o;
}

struct Config {
    int vec = 0;
    int splits = 0;
};
Config g_forced;

template <int BITS>
int32_t launch_bits(const float* a, const WeightView& w, float* c, int32_t accumulate, float alpha,
                    const float* bias, hipStream_t st) {
    // Widest lane vector the row pitch and base alignment allow.
    int vec = 4;
    if (w.bpr % 16 == 0 && aligned(w.q, 16)) vec = 16;
    else if (w.bpr % 8 == 0 && aligned(w.q, 8)) vec = 8;
    // Enough waves to keep every CU's memory pipe busy: narrow the lane vector
    // first (more column tiles), then split the groups over workgroups.
    const int32_t target = cu_count() * 8;
    const int32_t max_splits = w.G / WAVES > 1 ? w.G / WAVES : 1;
    auto waves_for = [&](int v, int32_t sp) { return static_cast<int64_t>(ceil_div(w.bpr, 64 * v)) * sp * WAVES; };
    while (vec > 4 && waves_for(vec, max_splits) < target) vec /= 2;
    if (g_forced.vec && w.bpr % g_forced.vec == 0 && aligned(w.q, g_forced.vec)) vec = g_forced.vec;
    const int32_t tiles = ceil_div(w.bpr, 64 * vec);
    int32_t splits = ceil_div(target, tiles * WAVES);
    if (splits > max_splits) splits = max_splits;
    if (splits < 1) splits = 1;
    if (g_forced.splits) splits = g_forced.splits < w.G ? g_forced.splits : w.G;
    const int32_t gps = ceil_div(w.G, splits);
    splits = ceil_div(w.G, gps);

    float* partials = nullptr;
    if (splits > 1) {
        void* ws = nullptr;
        int32_t status = workspace(st, static_cast<size_t>(splits) * w.N * sizeof(float), &ws);
        if (status) return status;
        partials = static_cast<float*>(ws);
    }
    const dim3 grid(static_cast<uint32_t>(tiles * splits));
    const dim3 block(64 * WAVES);
#define KT_GEMV_CASE(V)                                                                                       \
    case V:                                                                                                   \
        gemv_kernel<BITS, V><<<grid, block, 0, st>>>(a, w.q, w.s, w.z, c, partials, bias, w.K, w.N, w.bpr, w.g, \
                                                     w.G, tiles, gps, alpha, accumulate);                    \
        break;
    switch (vec) {
        KT_GEMV_CASE(16)
        KT_GEMV_CASE(8)
        KT_GEMV_CASE(4)
    }
#undef KT_GEMV_CASE
    KT_LAUNCHED("qmatmul: gemv kernel");
    if (splits > 1) {
        gemv_reduce<<<ceil_div(w.N, 256), 256, 0, st>>>(partials, splits, w.N, c, bias, alpha, accumulate);
        KT_LAUNCHED("qmatmul: gemv reduce");
    }
    return KT_OK;
}

}  // namespace

bool gemv_supported(const float* a, const WeightView& w, const float* c) {
    // Lanes need 4-column scale/zero vectors and 16-byte-aligned output quads.
    if (w.N % (w.bits == 4 ? 8 : 4) != 0) return false;
    if (!aligned(w.q, 4) || !aligned(w.s, 16) || (w.z && !aligned(w.z, 4)) || !aligned(c, 16)) return false;
    return aligned(a, 4);
}

int32_t launch_gemv(const float* a, const WeightView& w, float* c, int32_t accumulate, float alpha,
                    const float* bias, hipStream_t st) {
    if (bias && !aligned(bias, 16)) return launch_generic(a, 1, w, c, accumulate, alpha, bias, st);
    return w.bits == 4 ? launch_bits<4>(a, w, c, accumulate, alpha, bias, st)
                       : launch_bits<8>(a, w, c, accumulate, alpha, bias, st);
}

void set_gemv_config(int32_t vec, int32_t splits) {
    g_forced.vec = (vec == 4 || vec == 8 || vec == 16) ? vec : 0;
    g_forced.splits = splits > 0 ? splits : 0;
}

}  // namespace kt
