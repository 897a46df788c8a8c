// kt_quantize.hip -- fp32 [K x N] -> group-wise INT8 (symmetric) or INT4 (asymmetric,
// split-half packed) on gfx950, bit-exact with QuantizedTensor.quantize
// (Engine/kotensor/src/main/kotlin/QuantizedTensor.kt:256-324).
//
// HBM-bound: reads 4 B per weight once, writes 1 B (INT8) or 0.5 B (INT4) plus
// the per-(group, column) scale and zero. Layout of the work:
//   * an item is one group and 64 column units (group-major); a column unit is 4
//     adjacent columns (INT8) or 4 adjacent bytes (INT4: the low-nibble columns
//     b..b+3 and the high-nibble columns half+b..half+b+3); the workgroups are one
//     resident round and take the items in turn, the next item's loads in flight
//     while the current one is reduced;
//   * an item's rows are split over the workgroup's waves, RPW rows each, and
//     stay in registers between the min/max pass and the rounding pass, so every
//     input float is read from HBM exactly once (each wave row is 1 KB contiguous);
//   * per-column min/max partials are combined across waves through LDS, and each
//     column's scale, zero and inverse are computed once per workgroup.
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
// Branch-free: v_cvt_i32_f32 saturates out-of-range values (infinities included) to
// INT32_MIN / INT32_MAX and turns NaN into 0, which is the contract for every input
// whose floor is out of range; the +1 of a fraction >= 1/2 only occurs below 2^23.
__device__ __forceinline__ int32_t cvt_sat(float f) {
    int32_t r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(f));
    return r;
}
__device__ __forceinline__ int32_t java_round(float x, bool& nan_seen) {
    nan_seen |= x != x;
    const float f = floorf(x);
    const float frac = x - f;  // exact whenever it can be close to one half; NaN for +-inf
    const int32_t r = cvt_sat(f);
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

// A NaN input marks the call: the kernel stores the call's epoch into its slot of a
// pinned host array (system scope, so the host reads it after the stream syncs). Slots
// are never cleared; an older call's mark holds another epoch.
struct NanFlag {
    int32_t* slot;
    int32_t epoch;
};
__device__ __forceinline__ void mark_nan(const NanFlag& f) {
    __hip_atomic_store(f.slot, f.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The vector kernels: an item is one group and 64 column units, its rows split over the
// workgroup's waves (RPW each) and kept in registers. A workgroup takes items blockIdx.x,
// blockIdx.x + gridDim.x, ... (one round of workgroups for the whole call) and issues the
// next item's loads before it reduces the current one, so the stream of reads does not
// stop while a workgroup turns its extrema into scales. Every row load is issued (rows past
// the group's end read its last row again, which changes no extremum, and are not stored),
// so the loads in flight are the same count every time. Per-lane partial extrema go to LDS
// as [wave][component][lane] (lanes contiguous: no bank conflicts); then every thread takes
// whole columns of the item (consecutive threads, consecutive columns: coalesced scale and
// zero stores), reduces the waves' partials, computes the scale, zero and inverse once (the
// three correctly rounded divisions per column are not repeated in every wave) and
// publishes inverse and zero as [component][lane] for the rounding pass. Min and max are
// exact and order-free up to the sign of a zero, which no output depends on; a NaN input
// makes the call fail whatever they hold. The input is read once: non-temporal loads.

typedef float nt4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 load_nt(const float* p) {
    const nt4 v = __builtin_nontemporal_load(reinterpret_cast<const nt4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

// INT8, 4 columns per lane (256 columns per item), RPW rows per wave.
template <int RPW>
__global__ void __launch_bounds__(1024) quant8_vec(const float* __restrict__ data, int32_t K, int32_t N,
                                                   int32_t g, uint8_t* __restrict__ q, float* __restrict__ s,
                                                   NanFlag nan_flag) {
    extern __shared__ float red[];  // [waves][4][64] max |x|, then [4][64] inverses
    const int32_t t = threadIdx.x, ln = t & 63, wave = t >> 6, waves = blockDim.x >> 6;
    const int32_t units = N >> 2;
    const int32_t col_blocks = ceil_div(units, 64);
    const int32_t items = ceil_div(K, g) * col_blocks;
    float* inv = red + waves * 4 * 64;  // [4][64]
    bool nan_seen = false;
    auto load = [&](int32_t item, float4 (&v)[RPW]) {
        const int32_t group = item / col_blocks, unit = (item % col_blocks) * 64 + ln;
        const int32_t r1 = min(group * g + g, K);
        const int32_t c0 = (unit < units ? unit : 0) * 4;
#pragma unroll
        for (int i = 0; i < RPW; ++i)
            v[i] = load_nt(data + static_cast<size_t>(min(group * g + wave * RPW + i, r1 - 1)) * N + c0);
    };
    auto process = [&](int32_t item, const float4 (&v)[RPW]) {
        const int32_t group = item / col_blocks, cb = item % col_blocks;
        const int32_t unit = cb * 64 + ln;
        const int32_t r1 = min(group * g + g, K);
        const int32_t wr0 = group * g + wave * RPW;
        const int32_t c0 = (unit < units ? unit : 0) * 4;
        float mx[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int i = 0; i < RPW; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) mx[j] = fmaxf(mx[j], fabsf(lane(v[i], j)));
#pragma unroll
        for (int j = 0; j < 4; ++j) red[(wave * 4 + j) * 64 + ln] = mx[j];
        __syncthreads();  // every wave is also done with the previous item's inverses
        for (int32_t c = t; c < 256; c += blockDim.x) {  // item column c = 4 * lane + j
            const int32_t cl = c >> 2, j = c & 3;
            float m = 0.0f;
            for (int w = 0; w < waves; ++w) m = fmaxf(m, red[(w * 4 + j) * 64 + cl]);
            const float scale = m > 0.0f ? m / 127.0f : 1.0f;
            inv[j * 64 + cl] = 1.0f / scale;
            if (cb * 64 + cl < units) s[static_cast<size_t>(group) * N + cb * 256 + c] = scale;
        }
        __syncthreads();
        float inverse[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) inverse[j] = inv[j * 64 + ln];
        if (unit < units) {
#pragma unroll
            for (int i = 0; i < RPW; ++i) {
                const int32_t r = wr0 + i;
                if (r < r1) {
                    uint32_t packed = 0;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int32_t qv = clampi(java_round(lane(v[i], j) * inverse[j], nan_seen), -127, 127);
                        packed |= (static_cast<uint32_t>(qv) & 0xFFu) << (8 * j);
                    }
                    *reinterpret_cast<uint32_t*>(q + static_cast<size_t>(r) * N + c0) = packed;
                }
            }
        }
    };
    float4 va[RPW];
    if constexpr (RPW <= 8) {
        // two register sets, alternating (indices fixed at compile time)
        float4 vb[RPW];
        int32_t item = blockIdx.x;
        load(item, va);
        while (true) {
            if (item + static_cast<int32_t>(gridDim.x) < items) load(item + gridDim.x, vb);
            process(item, va);
            item += gridDim.x;
            if (item >= items) break;
            if (item + static_cast<int32_t>(gridDim.x) < items) load(item + gridDim.x, va);
            process(item, vb);
            item += gridDim.x;
            if (item >= items) break;
        }
    } else {
        // sixteen rows a wave: one set (two would not fit the registers of 16 waves)
        for (int32_t item = blockIdx.x; item < items; item += gridDim.x) {
            load(item, va);
            process(item, va);
        }
    }
    if (nan_seen) mark_nan(nan_flag);
}

// INT4, 4 bytes (8 columns: 4 low-nibble, 4 high-nibble) per lane, 512 columns per item,
// RPW rows per wave.
template <int RPW>
__global__ void __launch_bounds__(1024) quant4_vec(const float* __restrict__ data, int32_t K, int32_t N,
                                                   int32_t g, uint8_t* __restrict__ q, float* __restrict__ s,
                                                   int8_t* __restrict__ z, NanFlag nan_flag) {
    // [waves][16][64] partials (min lo, max lo, min hi, max hi, 4 each), then
    // [8][64] inverses and [8][64] zeros (component side * 4 + j)
    extern __shared__ float red[];
    const int32_t half = N >> 1;  // N % 8 == 0 here, so half == bytes per row
    const int32_t t = threadIdx.x, ln = t & 63, wave = t >> 6, waves = blockDim.x >> 6;
    const int32_t units = half >> 2;
    const int32_t col_blocks = ceil_div(units, 64);
    const int32_t items = ceil_div(K, g) * col_blocks;
    float* inv = red + waves * 16 * 64;                        // [8][64]
    int32_t* zer = reinterpret_cast<int32_t*>(inv + 8 * 64);  // [8][64]
    bool nan_seen = false;
    auto load = [&](int32_t item, float4 (&lo)[RPW], float4 (&hi)[RPW]) {
        const int32_t group = item / col_blocks, unit = (item % col_blocks) * 64 + ln;
        const int32_t r1 = min(group * g + g, K);
        const int32_t b0 = (unit < units ? unit : 0) * 4;
#pragma unroll
        for (int i = 0; i < RPW; ++i) {
            const float* row = data + static_cast<size_t>(min(group * g + wave * RPW + i, r1 - 1)) * N;
            lo[i] = load_nt(row + b0);
            hi[i] = load_nt(row + half + b0);
        }
    };
    auto process = [&](int32_t item, const float4 (&lo)[RPW], const float4 (&hi)[RPW]) {
        const int32_t group = item / col_blocks, cb = item % col_blocks;
        const int32_t unit = cb * 64 + ln;
        const int32_t r1 = min(group * g + g, K);
        const int32_t wr0 = group * g + wave * RPW;
        const int32_t b0 = (unit < units ? unit : 0) * 4;
        float mnl[4], mxl[4], mnh[4], mxh[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            mnl[j] = FLT_MAX;
            mxl[j] = -FLT_MAX;
            mnh[j] = FLT_MAX;
            mxh[j] = -FLT_MAX;
        }
#pragma unroll
        for (int i = 0; i < RPW; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                mnl[j] = fminf(mnl[j], lane(lo[i], j));
                mxl[j] = fmaxf(mxl[j], lane(lo[i], j));
                mnh[j] = fminf(mnh[j], lane(hi[i], j));
                mxh[j] = fmaxf(mxh[j], lane(hi[i], j));
            }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            red[(wave * 16 + j) * 64 + ln] = mnl[j];
            red[(wave * 16 + 4 + j) * 64 + ln] = mxl[j];
            red[(wave * 16 + 8 + j) * 64 + ln] = mnh[j];
            red[(wave * 16 + 12 + j) * 64 + ln] = mxh[j];
        }
        __syncthreads();  // every wave is also done with the previous item's inverses and zeros
        for (int32_t c = t; c < 512; c += blockDim.x) {  // side c / 256, byte 4 * lane + j
            const int32_t side = c >> 8, cl = (c & 255) >> 2, j = c & 3;
            float mn = FLT_MAX, mx = -FLT_MAX;
            for (int w = 0; w < waves; ++w) {
                mn = fminf(mn, red[(w * 16 + side * 8 + j) * 64 + cl]);
                mx = fmaxf(mx, red[(w * 16 + side * 8 + 4 + j) * 64 + cl]);
            }
            mn = mn > 0.0f ? 0.0f : mn;
            mx = mx < 0.0f ? 0.0f : mx;
            const float range = mx - mn;
            const float scale = range > 0.0f ? range / 15.0f : 1.0f;
            const int32_t zero = clampi(java_round(-mn / scale, nan_seen), 0, 15);
            inv[(side * 4 + j) * 64 + cl] = 1.0f / scale;
            zer[(side * 4 + j) * 64 + cl] = zero;
            if (cb * 64 + cl < units) {
                const size_t col = static_cast<size_t>(group) * N + (side ? half : 0) + cb * 256 + (c & 255);
                s[col] = scale;
                z[col] = static_cast<int8_t>(zero);
            }
        }
        __syncthreads();
        float il[4], ih[4];
        int32_t zl[4], zh[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            il[j] = inv[j * 64 + ln];
            ih[j] = inv[(4 + j) * 64 + ln];
            zl[j] = zer[j * 64 + ln];
            zh[j] = zer[(4 + j) * 64 + ln];
        }
        if (unit < units) {
#pragma unroll
            for (int i = 0; i < RPW; ++i) {
                const int32_t r = wr0 + i;
                if (r < r1) {
                    uint32_t packed = 0;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int32_t ql = clampi(wrap_add(java_round(lane(lo[i], j) * il[j], nan_seen), zl[j]), 0, 15);
                        const int32_t qh = clampi(wrap_add(java_round(lane(hi[i], j) * ih[j], nan_seen), zh[j]), 0, 15);
                        packed |= static_cast<uint32_t>(ql | (qh << 4)) << (8 * j);
                    }
                    *reinterpret_cast<uint32_t*>(q + static_cast<size_t>(r) * half + b0) = packed;
                }
            }
        }
    };
    float4 loa[RPW], hia[RPW];
    if constexpr (RPW <= 4) {
        // two register sets, alternating (indices fixed at compile time)
        float4 lob[RPW], hib[RPW];
        int32_t item = blockIdx.x;
        load(item, loa, hia);
        while (true) {
            if (item + static_cast<int32_t>(gridDim.x) < items) load(item + gridDim.x, lob, hib);
            process(item, loa, hia);
            item += gridDim.x;
            if (item >= items) break;
            if (item + static_cast<int32_t>(gridDim.x) < items) load(item + gridDim.x, loa, hia);
            process(item, lob, hib);
            item += gridDim.x;
            if (item >= items) break;
        }
    } else {
        // eight rows a wave: one set (two would not fit the registers of 16 waves)
        for (int32_t item = blockIdx.x; item < items; item += gridDim.x) {
            load(item, loa, hia);
            process(item, loa, hia);
        }
    }
    if (nan_seen) mark_nan(nan_flag);
}

// Any shape: one thread per (group, column) for INT8 or per (group, byte) for INT4,
// scanning the group twice (the second scan is served mostly by L2).
__global__ void __launch_bounds__(256) quant_generic(const float* __restrict__ data, int32_t K, int32_t N,
                                                    int32_t bits, int32_t g, int32_t bpr,
                                                    uint8_t* __restrict__ q, float* __restrict__ s,
                                                    int8_t* __restrict__ z, NanFlag nan_flag) {
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
    if (nan_seen) mark_nan(nan_flag);
}

}  // namespace

// One round of workgroups for the vector kernels: as many as fit on every CU at once,
// never more than the items. LDS beyond the 64 KB default (up to 68 KB at sixteen INT4
// waves) raises the kernel's attribute first (gfx950 gives a workgroup up to 160 KB).
template <typename Kern>
static int32_t resident_grid(Kern kern, int32_t threads, size_t lds, int64_t items, uint32_t* grid) {
    if (lds > (64u << 10))
        KT_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                                   160 << 10));
    int per_cu = 0;
    KT_HIP(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, threads, lds));
    const int64_t resident = static_cast<int64_t>(per_cu > 0 ? per_cu : 1) * cu_count();
    *grid = static_cast<uint32_t>(items < resident ? items : resident);
    return KT_OK;
}

int32_t launch_quantize(const float* data, int32_t K, int32_t N, int32_t bits, int32_t g, uint8_t* q, float* s,
                        int8_t* z, int32_t* nan_slot, int32_t epoch, hipStream_t st) {
    const NanFlag nan_flag{nan_slot, epoch};
    const int32_t G = ceil_div(K, g);
    const int32_t bpr = bits == 4 ? (N + N % 2) / 2 : N;
    const bool ptrs = aligned(data, 16) && aligned(q, 4) && aligned(s, 16) && (!z || aligned(z, 4));
    if (bits == 8 && ptrs && N % 4 == 0 && g <= 16 * 16) {
        const int64_t items = static_cast<int64_t>(ceil_div(N / 4, 64)) * G;
        if (items > INT32_MAX) return fail(KT_ERR_SHAPE, "quantize: grid too large");
        uint32_t grid = 0;
        // eight rows per wave up to g = 128 (more waves in flight per CU), sixteen beyond
        if (g <= 16 * 8) {
            const int32_t waves = ceil_div(g, 8);
            const size_t lds = (waves + 1) * 4 * 64 * sizeof(float);
            if (const int32_t st2 = resident_grid(quant8_vec<8>, 64 * waves, lds, items, &grid)) return st2;
            quant8_vec<8><<<grid, 64 * waves, lds, st>>>(data, K, N, g, q, s, nan_flag);
        } else {
            const int32_t waves = ceil_div(g, 16);
            const size_t lds = (waves + 1) * 4 * 64 * sizeof(float);
            if (const int32_t st2 = resident_grid(quant8_vec<16>, 64 * waves, lds, items, &grid)) return st2;
            quant8_vec<16><<<grid, 64 * waves, lds, st>>>(data, K, N, g, q, s, nan_flag);
        }
        KT_LAUNCHED("quantize: int8 kernel");
        return KT_OK;
    }
    if (bits == 4 && ptrs && N % 8 == 0 && g <= 16 * 8) {
        const int64_t items = static_cast<int64_t>(ceil_div(N / 8, 64)) * G;
        if (items > INT32_MAX) return fail(KT_ERR_SHAPE, "quantize: grid too large");
        uint32_t grid = 0;
        // four rows per wave up to g = 64 (more waves in flight per CU), eight beyond
        if (g <= 16 * 4) {
            const int32_t waves = ceil_div(g, 4);
            const size_t lds = (waves * 16 + 16) * 64 * sizeof(float);  // 68 KB at 16 waves
            if (const int32_t st2 = resident_grid(quant4_vec<4>, 64 * waves, lds, items, &grid)) return st2;
            quant4_vec<4><<<grid, 64 * waves, lds, st>>>(data, K, N, g, q, s, z, nan_flag);
        } else {
            const int32_t waves = ceil_div(g, 8);
            const size_t lds = (waves * 16 + 16) * 64 * sizeof(float);
            if (const int32_t st2 = resident_grid(quant4_vec<8>, 64 * waves, lds, items, &grid)) return st2;
            quant4_vec<8><<<grid, 64 * waves, lds, st>>>(data, K, N, g, q, s, z, nan_flag);
        }
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
