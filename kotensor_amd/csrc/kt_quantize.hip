// kt_quantize.hip -- fp32 [K x N] -> group-wise INT8 (symmetric) or INT4 (asymmetric,
// split-half packed) on gfx950, bit-exact with QuantizedTensor.quantize
// (Engine/kotensor/src/main/kotlin/QuantizedTensor.kt:256-324).
//
// HBM-bound: reads 4 B per weight once, writes 1 B (INT8) or 0.5 B (INT4) plus
// the per-(group, column) scale and zero. Layout of the work:
//   * a workgroup owns one group and 64 column units (a 1-D grid, group-major);
//     a column unit is 4 adjacent columns (INT8) or 4 adjacent bytes (INT4: the
//     low-nibble columns b..b+3 and the high-nibble columns half+b..half+b+3);
//   * the group's rows are split over the workgroup's waves, RPW rows each, and
//     stay in registers between the min/max pass and the rounding pass, so every
//     input float is read from HBM exactly once (each wave row is 1 KB contiguous);
//   * per-column min/max partials are combined across waves through LDS.
// Shapes the vector kernels cannot take (odd widths, misaligned pointers, group
// sizes beyond 16 waves' rows) use a one-thread-per-column kernel that scans twice.
//
// Arithmetic follows the reference operation by operation, in IEEE fp32 without
// contraction (this file is compiled with -ffp-contract=off), with the
// correctly-rounded '/' HIP uses by default: scale = maxAbs / 127, inverse = 1 / scale,
// q = round(x * inverse) with Math.round's ties-toward-+inf, saturating conversion
// and Kotlin's wrapping Int addition of the zero point.
#include <float.h>

#include "kt_common.h"

namespace kt {
namespace {

// Math.round(float) contract: nearest integer, ties toward +inf, saturating at the
// int range. NaN is what Float.roundToInt() rejects; it raises the error flag.
__device__ __forceinline__ int32_t java_round(float x, bool& nan_seen) {
    if (x != x) {
        nan_seen = true;
        return 0;
    }
    if (x >= 2147483648.0f) return INT32_MAX;
    if (x <= -2147483648.0f) return INT32_MIN;
    float f = floorf(x);
    float frac = x - f;  // exact whenever it can be close to one half
    int32_t r = static_cast<int32_t>(f);
    return frac >= 0.5f ? r + 1 : r;
}

__device__ __forceinline__ int32_t clampi(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}

__device__ __forceinline__ int32_t wrap_add(int32_t a, int32_t b) {
    return static_cast<int32_t>(static_cast<uint32_t>(a) + static_cast<uint32_t>(b));
}

__device__ __forceinline__ float lane(const float4& v, int j) {
    return j == 0 ? v.x : (j == 1 ? v.y : (j == 2 ? v.z : v.w));
}

__global__ void clear_flag(int32_t* flag) { *flag = 0; }

// INT8, 4 columns per lane, RPW rows per wave, ceil(g / RPW) waves per workgroup.
template <int RPW>
__global__ void __launch_bounds__(1024) quant8_vec(const float* __restrict__ data, int32_t K, int32_t N,
                                                   int32_t g, uint8_t* __restrict__ q, float* __restrict__ s,
                                                   int32_t* __restrict__ nan_flag) {
    extern __shared__ float red[];  // [waves][64][4]
    const int32_t ln = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const int32_t col_blocks = ceil_div(N >> 2, 64);
    const int32_t group = blockIdx.x / col_blocks;
    const int32_t unit = (blockIdx.x % col_blocks) * 64 + ln;
    const bool active = unit < (N >> 2);
    const int32_t r0 = group * g;
    const int32_t r1 = min(r0 + g, K);
    const int32_t wr0 = r0 + wave * RPW;
    const int32_t c0 = unit * 4;
    float4 v[RPW];
    float mx[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int32_t r = wr0 + i;
        if (active && r < r1) {
            v[i] = *reinterpret_cast<const float4*>(data + static_cast<size_t>(r) * N + c0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float a = fabsf(lane(v[i], j));
                if (a > mx[j]) mx[j] = a;
            }
        }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) red[(wave * 64 + ln) * 4 + j] = mx[j];
    __syncthreads();
    float scale[4], inverse[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float m = 0.0f;
        for (int w = 0; w < waves; ++w) {
            float a = red[(w * 64 + ln) * 4 + j];
            if (a > m) m = a;
        }
        scale[j] = m > 0.0f ? m / 127.0f : 1.0f;
        inverse[j] = 1.0f / scale[j];
    }
    if (!active) return;
    if (wave == 0)
        *reinterpret_cast<float4*>(s + static_cast<size_t>(group) * N + c0) =
            make_float4(scale[0], scale[1], scale[2], scale[3]);
    bool nan_seen = false;
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int32_t r = wr0 + i;
        if (r < r1) {
            uint32_t packed = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                int32_t qv = clampi(java_round(lane(v[i], j) * inverse[j], nan_seen), -127, 127);
                packed |= (static_cast<uint32_t>(qv) & 0xFFu) << (8 * j);
            }
            *reinterpret_cast<uint32_t*>(q + static_cast<size_t>(r) * N + c0) = packed;
        }
    }
    if (nan_seen) *nan_flag = 1;
}

// INT4, 4 bytes (8 columns) per lane, RPW rows per wave.
template <int RPW>
__global__ void __launch_bounds__(1024) quant4_vec(const float* __restrict__ data, int32_t K, int32_t N,
                                                   int32_t g, uint8_t* __restrict__ q, float* __restrict__ s,
                                                   int8_t* __restrict__ z, int32_t* __restrict__ nan_flag) {
    extern __shared__ float red[];  // [waves][64][16]: min lo, max lo, min hi, max hi (4 each)
    const int32_t half = N >> 1;    // N % 8 == 0 here, so half == bytes per row
    const int32_t ln = threadIdx.x & 63, wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
    const int32_t col_blocks = ceil_div(half >> 2, 64);
    const int32_t group = blockIdx.x / col_blocks;
    const int32_t unit = (blockIdx.x % col_blocks) * 64 + ln;
    const bool active = unit < (half >> 2);
    const int32_t r0 = group * g;
    const int32_t r1 = min(r0 + g, K);
    const int32_t wr0 = r0 + wave * RPW;
    const int32_t b0 = unit * 4;
    float4 lo[RPW], hi[RPW];
    float mnl[4], mxl[4], mnh[4], mxh[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        mnl[j] = FLT_MAX;
        mxl[j] = -FLT_MAX;
        mnh[j] = FLT_MAX;
        mxh[j] = -FLT_MAX;
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int32_t r = wr0 + i;
        if (active && r < r1) {
            const float* row = data + static_cast<size_t>(r) * N;
            lo[i] = *reinterpret_cast<const float4*>(row + b0);
            hi[i] = *reinterpret_cast<const float4*>(row + half + b0);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float a = lane(lo[i], j), b = lane(hi[i], j);
                if (a < mnl[j]) mnl[j] = a;
                if (a > mxl[j]) mxl[j] = a;
                if (b < mnh[j]) mnh[j] = b;
                if (b > mxh[j]) mxh[j] = b;
            }
        }
    }
    float* mine = red + (wave * 64 + ln) * 16;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        mine[j] = mnl[j];
        mine[4 + j] = mxl[j];
        mine[8 + j] = mnh[j];
        mine[12 + j] = mxh[j];
    }
    __syncthreads();
    // Min and max are exact and order-free up to the sign of a zero, which no
    // output depends on.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        for (int w = 0; w < waves; ++w) {
            const float* other = red + (w * 64 + ln) * 16;
            if (other[j] < mnl[j]) mnl[j] = other[j];
            if (other[4 + j] > mxl[j]) mxl[j] = other[4 + j];
            if (other[8 + j] < mnh[j]) mnh[j] = other[8 + j];
            if (other[12 + j] > mxh[j]) mxh[j] = other[12 + j];
        }
    }
    if (!active) return;
    bool nan_seen = false;
    float sl[4], sh[4], il[4], ih[4];
    int32_t zl[4], zh[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float mn = mnl[j] > 0.0f ? 0.0f : mnl[j];
        float mx = mxl[j] < 0.0f ? 0.0f : mxl[j];
        float range = mx - mn;
        sl[j] = range > 0.0f ? range / 15.0f : 1.0f;
        zl[j] = clampi(java_round(-mn / sl[j], nan_seen), 0, 15);
        il[j] = 1.0f / sl[j];
        mn = mnh[j] > 0.0f ? 0.0f : mnh[j];
        mx = mxh[j] < 0.0f ? 0.0f : mxh[j];
        range = mx - mn;
        sh[j] = range > 0.0f ? range / 15.0f : 1.0f;
        zh[j] = clampi(java_round(-mn / sh[j], nan_seen), 0, 15);
        ih[j] = 1.0f / sh[j];
    }
    if (wave == 0) {
        float* srow = s + static_cast<size_t>(group) * N;
        *reinterpret_cast<float4*>(srow + b0) = make_float4(sl[0], sl[1], sl[2], sl[3]);
        *reinterpret_cast<float4*>(srow + half + b0) = make_float4(sh[0], sh[1], sh[2], sh[3]);
        int8_t* zrow = z + static_cast<size_t>(group) * N;
        uint32_t zlp = 0, zhp = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            zlp |= static_cast<uint32_t>(zl[j]) << (8 * j);
            zhp |= static_cast<uint32_t>(zh[j]) << (8 * j);
        }
        *reinterpret_cast<uint32_t*>(zrow + b0) = zlp;
        *reinterpret_cast<uint32_t*>(zrow + half + b0) = zhp;
    }
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
        const int32_t r = wr0 + i;
        if (r < r1) {
            uint32_t packed = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                int32_t ql = clampi(wrap_add(java_round(lane(lo[i], j) * il[j], nan_seen), zl[j]), 0, 15);
                int32_t qh = clampi(wrap_add(java_round(lane(hi[i], j) * ih[j], nan_seen), zh[j]), 0, 15);
                packed |= static_cast<uint32_t>(ql | (qh << 4)) << (8 * j);
            }
            *reinterpret_cast<uint32_t*>(q + static_cast<size_t>(r) * half + b0) = packed;
        }
    }
    if (nan_seen) *nan_flag = 1;
}

// Any shape: one thread per (group, column) for INT8 or per (group, byte) for INT4,
// scanning the group twice (the second scan is served mostly by L2).
__global__ void __launch_bounds__(256) quant_generic(const float* __restrict__ data, int32_t K, int32_t N,
                                                    int32_t bits, int32_t g, int32_t bpr,
                                                    uint8_t* __restrict__ q, float* __restrict__ s,
                                                    int8_t* __restrict__ z, int32_t* __restrict__ nan_flag) {
    const int32_t units = bits == 8 ? N : bpr;
    const int32_t col_blocks = ceil_div(units, static_cast<int32_t>(blockDim.x));
    const int32_t group = blockIdx.x / col_blocks;
    const int32_t unit = (blockIdx.x % col_blocks) * blockDim.x + threadIdx.x;
    const int32_t r0 = group * g;
    const int32_t r1 = min(r0 + g, K);
    bool nan_seen = false;
    if (bits == 8) {
        if (unit >= N) return;
        const int32_t c = unit;
        float m = 0.0f;
        for (int32_t r = r0; r < r1; ++r) {
            float a = fabsf(data[static_cast<size_t>(r) * N + c]);
            if (a > m) m = a;
        }
        float scale = m > 0.0f ? m / 127.0f : 1.0f;
        s[static_cast<size_t>(group) * N + c] = scale;
        float inverse = 1.0f / scale;
        for (int32_t r = r0; r < r1; ++r) {
            int32_t qv = clampi(java_round(data[static_cast<size_t>(r) * N + c] * inverse, nan_seen), -127, 127);
            q[static_cast<size_t>(r) * N + c] = static_cast<uint8_t>(qv & 0xFF);
        }
    } else {
        if (unit >= bpr) return;
        const int32_t half = bpr;
        const int32_t cl = unit, ch = half + unit;
        const bool has_high = ch < N;
        float scale[2] = {1.0f, 1.0f}, inverse[2] = {1.0f, 1.0f};
        int32_t zero[2] = {0, 0};
        for (int side = 0; side < (has_high ? 2 : 1); ++side) {
            const int32_t c = side ? ch : cl;
            float mn = FLT_MAX, mx = -FLT_MAX;
            for (int32_t r = r0; r < r1; ++r) {
                float v = data[static_cast<size_t>(r) * N + c];
                if (v < mn) mn = v;
                if (v > mx) mx = v;
            }
            if (mn > 0.0f) mn = 0.0f;
            if (mx < 0.0f) mx = 0.0f;
            float range = mx - mn;
            scale[side] = range > 0.0f ? range / 15.0f : 1.0f;
            zero[side] = clampi(java_round(-mn / scale[side], nan_seen), 0, 15);
            inverse[side] = 1.0f / scale[side];
            s[static_cast<size_t>(group) * N + c] = scale[side];
            z[static_cast<size_t>(group) * N + c] = static_cast<int8_t>(zero[side]);
        }
        for (int32_t r = r0; r < r1; ++r) {
            const float* row = data + static_cast<size_t>(r) * N;
            int32_t ql = clampi(wrap_add(java_round(row[cl] * inverse[0], nan_seen), zero[0]), 0, 15);
            int32_t qh = 0;
            if (has_high) qh = clampi(wrap_add(java_round(row[ch] * inverse[1], nan_seen), zero[1]), 0, 15);
            q[static_cast<size_t>(r) * half + unit] = static_cast<uint8_t>(ql | (qh << 4));
        }
    }
    if (nan_seen) *nan_flag = 1;
}

}  // namespace

int32_t launch_quantize(const float* data, int32_t K, int32_t N, int32_t bits, int32_t g, uint8_t* q, float* s,
                        int8_t* z, int32_t* nan_flag, hipStream_t st) {
    clear_flag<<<1, 1, 0, st>>>(nan_flag);
    KT_LAUNCHED("quantize: clear flag");
    const int32_t G = ceil_div(K, g);
    const int32_t bpr = bits == 4 ? (N + N % 2) / 2 : N;
    const bool ptrs = aligned(data, 16) && aligned(q, 4) && aligned(s, 16) && (!z || aligned(z, 4));
    if (bits == 8 && ptrs && N % 4 == 0 && g <= 16 * 16) {
        constexpr int RPW = 16;
        const int32_t waves = ceil_div(g, RPW);
        const int64_t blocks = static_cast<int64_t>(ceil_div(N / 4, 64)) * G;
        if (blocks > INT32_MAX) return fail(KT_ERR_SHAPE, "quantize: grid too large");
        const dim3 grid(static_cast<uint32_t>(blocks));
        quant8_vec<RPW><<<grid, 64 * waves, waves * 64 * 4 * sizeof(float), st>>>(data, K, N, g, q, s, nan_flag);
        KT_LAUNCHED("quantize: int8 kernel");
        return KT_OK;
    }
    if (bits == 4 && ptrs && N % 8 == 0 && g <= 16 * 8) {
        constexpr int RPW = 8;
        const int32_t waves = ceil_div(g, RPW);
        const int64_t blocks = static_cast<int64_t>(ceil_div(N / 8, 64)) * G;
        if (blocks > INT32_MAX) return fail(KT_ERR_SHAPE, "quantize: grid too large");
        const dim3 grid(static_cast<uint32_t>(blocks));
        quant4_vec<RPW><<<grid, 64 * waves, waves * 64 * 16 * sizeof(float), st>>>(data, K, N, g, q, s, z, nan_flag);
        KT_LAUNCHED("quantize: int4 kernel");
        return KT_OK;
    }
    // quant_generic writes every byte, the pad nibble of an odd width as 0.
    const int32_t units = bits == 8 ? N : bpr;
    const int64_t blocks = static_cast<int64_t>(ceil_div(units, 256)) * G;
    if (blocks > INT32_MAX) return fail(KT_ERR_SHAPE, "quantize: grid too large");
    const dim3 grid(static_cast<uint32_t>(blocks));
    quant_generic<<<grid, 256, 0, st>>>(data, K, N, bits, g, bpr, q, s, z, nan_flag);
    KT_LAUNCHED("quantize: generic kernel");
    return KT_OK;
}

}  // namespace kt
