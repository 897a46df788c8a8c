// kt_gemv_mfma.hip -- decode dequant-GEMV for M = 1..16 rows on gfx950 MFMA:
//   c[M x N] = (accumulate ? c : 0) + alpha * x[M x K] . deq(W) (+ bias),
// the small-M case of MatMul.multiplyQuantized (Engine/kotensor/src/main/kotlin/
// MatMul.kt:460-486; M == 1 is multiplyQuantizedRow :494-536).
//
// The weights stream from HBM once, in the reference layout. The MFMA unit does the
// multiply-adds, so the vector ALU only unpacks (about one instruction per weight):
//
//   * v_mfma_f32_16x16x32_f16: lane l holds B[k = 8*(l/16) + i][n = l%16], i < 8. A lane
//     (cl = l%16, kb = l/16) loads rows r0 + 8*kb + i of an 8-byte column strip, so its
//     registers already hold, for each byte j of the strip, the 8 k-values of one
//     column -- a B fragment. 16 lanes cover 128 contiguous bytes of a row (one cache
//     line); a chunk is 32 rows (4 k-blocks);
//   * a weight becomes an exact fp16 without arithmetic: v_perm_b32 puts the byte j of
//     two consecutive rows into the low bytes of the two fp16 halves and a mask keeps
//     the nibble, giving the fp16 subnormal q * 2^-24 (low nibble), 16*q * 2^-24 (high
//     nibble) or, for INT8 after xor 0x80, (q + 128) * 2^-24 (bias folded into the zero);
//   * x is split into fp16 hi + lo parts after an exact power-of-two scaling per row
//     (largest |x| of the workgroup's K-range in [2^14, 2^15)), about 22 significant
//     bits; A_hi and A_lo both multiply the same B into one fp32 accumulator;
//   * rowSum for the zero-point term comes from the same MFMA against a constant B of
//     2^-24 (one extra pair of MFMAs per chunk), in exactly the units of the weights';
//   * per quantization group: res += scale * (acc - zero * rowSum) (the reference's
//     combineGroup form), then one exact power-of-two factor per row at the end;
//   * a workgroup is WAVES waves on one 128-byte column strip; its waves take the
//     groups of its K-slice round-robin and meet through LDS in a fixed order; K-slices
//     of one strip meet through the in-kernel counter reduction of kt_gemv.hip's
//     scheme or, for many slices, through a reduction kernel.
#include "kt_common.h"

namespace kt {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int MAX_JOBS = 4;
constexpr int CHUNK = 32;  // rows per MFMA k-step (4 lanes groups x 8 rows)
constexpr int STRIP = 128; // bytes of a row per wave (16 lanes x 8 bytes)

struct Job {
    const uint8_t* q;
    const float* s;
    const int8_t* z;
    float* out;
    const float* bias;
    float* partials;     // [slices x M x N] or nullptr
    uint32_t* counters;  // [tiles] for the in-kernel slice reduction, or nullptr
    int32_t N, bpr, tiles, slices, groups_per_slice, block_begin;
};

struct Jobs {
    Job job[MAX_JOBS];
    int32_t count;
};

__device__ __forceinline__ half8 as_half8(u32x4 v) { return __builtin_bit_cast(half8, v); }

// Byte j (0..3) of rows (a, b) into the low bytes of the two halves of a word.
__device__ __forceinline__ uint32_t pair_bytes(uint32_t a, uint32_t b, int j) {
    // v_perm_b32(S0 = b, S1 = a): selector bytes 0..3 pick a's bytes, 4..7 pick b's, 0x0c is 0.
    const uint32_t sel = 0x0c000c00u | (static_cast<uint32_t>(4 + j) << 16) | static_cast<uint32_t>(j);
    return __builtin_amdgcn_perm(b, a, sel);
}

// R: rows per lane of the 16x16 result (min(M, 4)); WAVES per workgroup.
template <int BITS, int R, int WAVES, bool ZP>
__global__ void __launch_bounds__(64 * WAVES)
    gemv_mfma_kernel(const float* __restrict__ x, int32_t M, int32_t K, int32_t g, Jobs jobs, float alpha,
                     int32_t accumulate) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    constexpr int NCOL = BITS == 4 ? 16 : 8;  // columns per lane

    int32_t ji = 0;
#pragma unroll
    for (int j = 1; j < MAX_JOBS; ++j)
        if (j < jobs.count && static_cast<int32_t>(blockIdx.x) >= jobs.job[j].block_begin) ji = j;
    const Job& jb = jobs.job[ji];
    const uint8_t* __restrict__ q = jb.q;
    const int32_t N = jb.N, bpr = jb.bpr, half = jb.bpr;
    const int32_t local = blockIdx.x - jb.block_begin;
    const int32_t tile = local % jb.tiles;
    const int32_t slice = local / jb.tiles;
    const int32_t G = K / g;
    const int32_t g_begin = slice * jb.groups_per_slice;
    const int32_t g_end = min(g_begin + jb.groups_per_slice, G);
    const int32_t ra = g_begin * g, nrows = (g_end - g_begin) * g;

    const int32_t t = threadIdx.x;
    const int32_t ln = t & 63;
    const int32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int32_t cl = ln & 15, kb = ln >> 4;
    const int32_t col_off = tile * STRIP + cl * 8;
    const bool active = col_off < bpr;
    const int32_t boff = active ? col_off : 0;  // lanes past the row end compute and discard

    // ---- x in LDS as fp16 hi/lo, per-row exponent ---------------------------------
    _Float16* xh = reinterpret_cast<_Float16*>(smem);
    _Float16* xl = xh + M * nrows;
    uint32_t* amax = reinterpret_cast<uint32_t*>(xl + M * nrows);  // [16]
    if (t < 16) amax[t] = 0u;
    __syncthreads();
    for (int32_t idx = t; idx < M * nrows; idx += 64 * WAVES) {
        const int32_t m = idx / nrows, k = idx - m * nrows;
        const float v = x[static_cast<size_t>(m) * K + ra + k];
        atomicMax(&amax[m], __float_as_uint(fabsf(v)));
    }
    __syncthreads();
    for (int32_t idx = t; idx < M * nrows; idx += 64 * WAVES) {
        const int32_t m = idx / nrows, k = idx - m * nrows;
        const float mx = __uint_as_float(amax[m]);
        int e = 0;
        if (mx > 0.0f && isfinite(mx)) {
            frexpf(mx, &e);
            e -= 15;
        }
        const float v = ldexpf(x[static_cast<size_t>(m) * K + ra + k], -e);
        const _Float16 h = static_cast<_Float16>(v);
        xh[idx] = h;
        xl[idx] = static_cast<_Float16>(v - static_cast<float>(h));
    }
    __syncthreads();

    // Per result row (m = 4*kb + i): the power of two that undoes the x scaling, read now
    // because the final reduction reuses this LDS.
    float rowf[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
        const int32_t m = 4 * kb + i;
        int e = 0;
        const float mx = m < M ? __uint_as_float(amax[m]) : 0.0f;
        if (mx > 0.0f && isfinite(mx)) {
            frexpf(mx, &e);
            e -= 15;
        }
        rowf[i] = ldexpf(1.0f, e);
    }

    // ---- main loop: this wave's groups, chunk by chunk, double-buffered ---------------
    // res[c][i]: column c of this lane, result row m = 4*kb + i.
    float res[NCOL][R];
#pragma unroll
    for (int c = 0; c < NCOL; ++c)
#pragma unroll
        for (int i = 0; i < R; ++i) res[c][i] = 0.0f;

    const int32_t chunks_per_group = g / CHUNK;
    const int32_t my_groups = g_end - g_begin > wave ? (g_end - g_begin - wave + WAVES - 1) / WAVES : 0;
    const int32_t my_chunks = my_groups * chunks_per_group;
    // k-th chunk of this wave -> absolute row of its first line
    auto chunk_row = [&](int32_t c) {
        const int32_t gg = c / chunks_per_group;
        return (g_begin + wave + gg * WAVES) * g + (c - gg * chunks_per_group) * CHUNK;
    };
    auto load = [&](uint2* v, int32_t c) {
        const int32_t r = chunk_row(c) + 8 * kb;
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const uint2*>(q + static_cast<size_t>(r + i) * bpr + boff);
    };
    const u32x4 ones = {0x00010001u, 0x00010001u, 0x00010001u, 0x00010001u};  // fp16 2^-24 in every half
    f32x4 acc[NCOL];
    f32x4 racc;
#pragma unroll
    for (int c = 0; c < NCOL; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
    racc = f32x4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](const uint2* v, int32_t c) {
        // A fragments: x rows m = cl (zero for m >= M), k = chunk rows 8*kb .. 8*kb+7.
        const int32_t krow = chunk_row(c) - ra + 8 * kb;
        half8 ah = {}, al = {};
        if (cl < M) {
            ah = *reinterpret_cast<const half8*>(xh + cl * nrows + krow);
            al = *reinterpret_cast<const half8*>(xl + cl * nrows + krow);
        }
        racc = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, as_half8(ones), racc, 0, 0, 0);
        racc = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, as_half8(ones), racc, 0, 0, 0);
#pragma unroll
        for (int w = 0; w < 2; ++w) {  // dword of the 8-byte strip
            // B fragments of the dword's 4 byte columns first, then the hi products of all
            // of them, then the lo ones: consecutive MFMAs write different accumulators.
            u32x4 p[4];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint32_t a = w ? v[2 * i].y : v[2 * i].x;
                    uint32_t b = w ? v[2 * i + 1].y : v[2 * i + 1].x;
                    if (BITS == 8) {
                        a ^= 0x80808080u;
                        b ^= 0x80808080u;
                    }
                    p[jj][i] = pair_bytes(a, b, jj);
                }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const half8 xa = h ? al : ah;
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int j = 4 * w + jj;
                    if (BITS == 8) {
                        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, as_half8(p[jj]), acc[j], 0, 0, 0);
                    } else {
                        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, as_half8(p[jj] & 0x000F000Fu), acc[j], 0, 0, 0);
                        acc[8 + j] =
                            __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, as_half8(p[jj] & 0x00F000F0u), acc[8 + j], 0, 0, 0);
                    }
                }
            }
        }
    };
    // res += scale * (acc - zero * rowSum) for group gi; then clear the accumulators.
    auto combine = [&](int32_t gi) {
        const float* srow = jb.s + static_cast<size_t>(gi) * N;
        float sc[NCOL];
        int32_t zr[NCOL];
#pragma unroll
        for (int side = 0; side < NCOL / 8; ++side) {
            const int32_t col = (side ? half : 0) + boff;
            const float4 s0 = *reinterpret_cast<const float4*>(srow + col);
            const float4 s1 = *reinterpret_cast<const float4*>(srow + col + 4);
            sc[8 * side + 0] = s0.x; sc[8 * side + 1] = s0.y; sc[8 * side + 2] = s0.z; sc[8 * side + 3] = s0.w;
            sc[8 * side + 4] = s1.x; sc[8 * side + 5] = s1.y; sc[8 * side + 6] = s1.z; sc[8 * side + 7] = s1.w;
            uint2 zz = make_uint2(0u, 0u);
            if constexpr (ZP) zz = *reinterpret_cast<const uint2*>(jb.z + static_cast<size_t>(gi) * N + col);
#pragma unroll
            for (int b = 0; b < 8; ++b)
                zr[8 * side + b] = static_cast<int8_t>(((b < 4 ? zz.x : zz.y) >> (8 * (b & 3))) & 0xFFu);
        }
#pragma unroll
        for (int c = 0; c < NCOL; ++c) {
            // low nibble / INT8 columns: acc and rowSum in units of 2^-24; high nibble
            // columns carry an extra 16 in acc, matched by 16 * zero.
            float zf = static_cast<float>(zr[c]) + (BITS == 8 ? 128.0f : 0.0f);
            if (BITS == 4 && c >= 8) zf *= 16.0f;
#pragma unroll
            for (int i = 0; i < R; ++i) res[c][i] = fmaf(sc[c], fmaf(-zf, racc[i], acc[c][i]), res[c][i]);
            acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
        racc = f32x4{0.f, 0.f, 0.f, 0.f};
    };

    if (my_chunks > 0) {
        uint2 va[8], vb[8];
        load(va, 0);
        int32_t c = 0;
        for (;;) {
            load(vb, c + 1 < my_chunks ? c + 1 : c);
            compute(va, c);
            if ((c + 1) % chunks_per_group == 0) combine(g_begin + wave + (c / chunks_per_group) * WAVES);
            if (++c >= my_chunks) break;
            load(va, c + 1 < my_chunks ? c + 1 : c);
            compute(vb, c);
            if ((c + 1) % chunks_per_group == 0) combine(g_begin + wave + (c / chunks_per_group) * WAVES);
            if (++c >= my_chunks) break;
        }
    }

    // ---- waves of the workgroup meet in LDS (reusing the x area), in wave order ---------
    // Results are in units of 2^-24 (low nibble, INT8) or 2^-20 (high nibble) times 2^-e_m.
    __syncthreads();
    float* red = reinterpret_cast<float*>(smem);  // [64 lanes][NCOL][R]
    for (int w = 0; w < WAVES; ++w) {
        if (wave == w) {
#pragma unroll
            for (int c = 0; c < NCOL; ++c)
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    float* slot = red + (ln * NCOL + c) * R + i;
                    *slot = w == 0 ? res[c][i] : *slot + res[c][i];
                }
        }
        __syncthreads();
    }
    if (wave != 0) return;
#pragma unroll
    for (int c = 0; c < NCOL; ++c)
#pragma unroll
        for (int i = 0; i < R; ++i) res[c][i] = red[(ln * NCOL + c) * R + i];

    // Back to real units: 2^(24 or 20) and 2^e_m per row.
#pragma unroll
    for (int c = 0; c < NCOL; ++c) {
        const float unit = (BITS == 4 && c >= 8) ? 1048576.0f : 16777216.0f;  // 2^20 : 2^24
#pragma unroll
        for (int i = 0; i < R; ++i) res[c][i] *= unit * rowf[i];
    }

    auto column = [&](int c) { return (c >= 8 ? half : 0) + boff + (c & 7); };
    if (jb.partials && jb.counters) {
        // In-kernel slice reduction (write-through sums + tile counter), as in kt_gemv.hip.
        float* part = jb.partials + static_cast<size_t>(slice) * M * N;
        if (active)
#pragma unroll
            for (int c = 0; c < NCOL; ++c)
#pragma unroll
                for (int i = 0; i < R; ++i) {
                    const int32_t m = 4 * kb + i;
                    if (m < M)
                        __hip_atomic_store(part + static_cast<size_t>(m) * N + column(c), res[c][i], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_SYSTEM);
                }
        __builtin_amdgcn_s_waitcnt(0);
        uint32_t old = 0;
        if (ln == 0) old = __hip_atomic_fetch_add(jb.counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __builtin_amdgcn_readfirstlane(old);
        if (old != static_cast<uint32_t>(jb.slices - 1)) return;
#pragma unroll
        for (int c = 0; c < NCOL; ++c)
#pragma unroll
            for (int i = 0; i < R; ++i) {
                const int32_t m = 4 * kb + i;
                float sum = 0.0f;
                if (active && m < M)
                    for (int32_t sp = 0; sp < jb.slices; ++sp) {
                        const float v = sp == slice ? res[c][i]
                                                    : __hip_atomic_load(jb.partials + (static_cast<size_t>(sp) * M + m) * N + column(c),
                                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                        sum = sp == 0 ? v : sum + v;
                    }
                res[c][i] = sum;
            }
        if (ln == 0) __hip_atomic_store(jb.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!active) return;
#pragma unroll
    for (int c = 0; c < NCOL; ++c) {
        const int32_t n = column(c);
#pragma unroll
        for (int i = 0; i < R; ++i) {
            const int32_t m = 4 * kb + i;
            if (m >= M) continue;
            if (jb.partials && !jb.counters) {
                jb.partials[(static_cast<size_t>(slice) * M + m) * N + n] = res[c][i];
            } else {
                float* dst = jb.out + static_cast<size_t>(m) * N + n;
                float o = accumulate ? *dst : 0.0f;
                o = fmaf(alpha, res[c][i], o);
                if (jb.bias) o += jb.bias[n];
                *dst = o;
            }
        }
    }
}

// Slice sums in slice order for jobs that were not reduced in the kernel.
__global__ void __launch_bounds__(256) gemv_mfma_reduce(Jobs jobs, int32_t M, float alpha, int32_t accumulate) {
    const int32_t idx = blockIdx.x * 256 + threadIdx.x;
#pragma unroll
    for (int j = 0; j < MAX_JOBS; ++j) {
        if (j >= jobs.count) break;
        const Job& jb = jobs.job[j];
        if (!jb.partials || jb.counters || idx >= M * jb.N) continue;
        float p[16];
        float t = 0.0f;
        for (int32_t s0 = 0; s0 < jb.slices; s0 += 16) {
#pragma unroll
            for (int u = 0; u < 16; ++u)
                p[u] = s0 + u < jb.slices ? jb.partials[static_cast<size_t>(s0 + u) * M * jb.N + idx] : 0.0f;
#pragma unroll
            for (int u = 0; u < 16; ++u)
                if (s0 + u < jb.slices) t = (s0 + u == 0) ? p[u] : t + p[u];
        }
        float o = accumulate ? jb.out[idx] : 0.0f;
        o = fmaf(alpha, t, o);
        if (jb.bias) o += jb.bias[idx % jb.N];
        jb.out[idx] = o;
    }
}

struct Forced {
    int slices = 0;
    int waves = 0;
    int reduce = 0;
    int disable = 0;
};
Forced g_forced;

constexpr size_t LDS_X_BYTES = 40 << 10;  // x hi/lo of a K-slice: 4 bytes per (row of x, k)

template <int BITS, int R, int WAVES, bool ZP>
void launch_kernel(dim3 grid, size_t lds, hipStream_t st, const float* a, int32_t M, int32_t K, int32_t g,
                   const Jobs& jobs, float alpha, int32_t accumulate) {
    gemv_mfma_kernel<BITS, R, WAVES, ZP><<<grid, dim3(64 * WAVES), lds, st>>>(a, M, K, g, jobs, alpha, accumulate);
}

template <int BITS, int R, int WAVES>
void launch_zp(bool zp, dim3 grid, size_t lds, hipStream_t st, const float* a, int32_t M, int32_t K, int32_t g,
               const Jobs& jobs, float alpha, int32_t accumulate) {
    if (BITS == 4 || zp) launch_kernel<BITS, R, WAVES, true>(grid, lds, st, a, M, K, g, jobs, alpha, accumulate);
    else launch_kernel<BITS, R, WAVES, false>(grid, lds, st, a, M, K, g, jobs, alpha, accumulate);
}

template <int BITS, int WAVES>
void launch_r(int r, bool zp, dim3 grid, size_t lds, hipStream_t st, const float* a, int32_t M, int32_t K, int32_t g,
              const Jobs& jobs, float alpha, int32_t accumulate) {
    if (r == 1) launch_zp<BITS, 1, WAVES>(zp, grid, lds, st, a, M, K, g, jobs, alpha, accumulate);
    else if (r == 2) launch_zp<BITS, 2, WAVES>(zp, grid, lds, st, a, M, K, g, jobs, alpha, accumulate);
    else launch_zp<BITS, 4, WAVES>(zp, grid, lds, st, a, M, K, g, jobs, alpha, accumulate);
}

}  // namespace

void set_gemv_mfma_config(int32_t slices, int32_t waves, int32_t reduce, int32_t disable) {
    g_forced.slices = slices > 0 ? slices : 0;
    g_forced.waves = (waves == 2 || waves == 4 || waves == 8) ? waves : 0;
    g_forced.reduce = (reduce == 1 || reduce == 2) ? reduce : 0;
    g_forced.disable = disable ? 1 : 0;
}

bool gemv_mfma_supported(const float* a, int32_t m, const WeightView& w, const float* c) {
    (void)a;
    (void)c;
    if (g_forced.disable) return false;
    if (m < 1 || m > 16) return false;
    if (w.g % CHUNK != 0 || w.K % w.g != 0) return false;  // whole 32-row chunks in whole groups
    if (w.bpr % 8 != 0 || !aligned(w.q, 8)) return false;  // 8-byte lane strips
    if (w.N % 8 != 0 || !aligned(w.s, 16) || (w.z && !aligned(w.z, 8))) return false;
    if (w.bits == 4 && w.N % 16 != 0) return false;        // high-nibble columns start 8-aligned
    return true;
}

int32_t launch_gemv_mfma(const float* a, int32_t M, const WeightView* ws, float* const* cs, const float* const* biases,
                         int32_t count, int32_t accumulate, float alpha, hipStream_t st) {
    const WeightView& w0 = ws[0];
    const int32_t G = w0.K / w0.g;
    bool zp = false;
    for (int32_t i = 0; i < count; ++i) zp = zp || ws[i].z != nullptr;
    if (zp)
        for (int32_t i = 0; i < count; ++i)
            if (!ws[i].z) return fail(KT_ERR_ARGUMENT, "grouped weights must all have zero points or none");

    int64_t tiles_total = 0;
    for (int32_t i = 0; i < count; ++i) tiles_total += ceil_div(ws[i].bpr, STRIP);
    const int32_t target_waves = cu_count() * 8;
    // Waves per workgroup (each takes whole groups), then K-slices until the GPU is
    // covered; the x area in LDS bounds the rows of a slice.
    int32_t waves = 4;
    if (G < 4) waves = G >= 2 ? 2 : 1;
    if (waves == 1) waves = 2;  // the smallest instantiation; an idle wave costs little
    int32_t slices = static_cast<int32_t>((target_waves + tiles_total * waves - 1) / (tiles_total * waves));
    const int32_t max_slices = G / waves > 1 ? G / waves : 1;
    if (slices > max_slices) slices = max_slices;
    if (slices < 1) slices = 1;
    const int32_t rows_cap = static_cast<int32_t>(LDS_X_BYTES / (4 * static_cast<size_t>(M)));
    const int32_t min_slices = ceil_div(w0.K, rows_cap > w0.g ? rows_cap - rows_cap % w0.g : w0.g);
    if (slices < min_slices) slices = min_slices;
    if (g_forced.waves) waves = g_forced.waves;
    if (g_forced.slices) slices = g_forced.slices > min_slices ? g_forced.slices : min_slices;
    if (slices > G) slices = G;
    constexpr int32_t MAX_INKERNEL_SLICES = 8;
    // A few more slices than the in-kernel limit buy less than the reduction kernel costs.
    if (!g_forced.slices && slices > MAX_INKERNEL_SLICES && slices < 2 * MAX_INKERNEL_SLICES &&
        min_slices <= MAX_INKERNEL_SLICES)
        slices = MAX_INKERNEL_SLICES;
    // Every slice takes gps whole groups; the last may take fewer.
    const int32_t gps = ceil_div(G, slices);
    slices = ceil_div(G, gps);
    const int32_t rows = gps * w0.g;
    size_t ws_floats = 0, n_counters = 0;
    if (slices > 1)
        for (int32_t i = 0; i < count; ++i) {
            ws_floats += static_cast<size_t>(slices) * M * ws[i].N;
            n_counters += ceil_div(ws[i].bpr, STRIP);
        }
    bool inkernel = slices > 1 && slices <= MAX_INKERNEL_SLICES && n_counters <= MAX_COUNTERS;
    if (g_forced.reduce == 1) inkernel = false;
    if (g_forced.reduce == 2 && slices > 1 && n_counters <= MAX_COUNTERS) inkernel = true;
    float* partials = nullptr;
    uint32_t* counters = nullptr;
    if (ws_floats) {
        void* p = nullptr;
        int32_t status = inkernel ? workspace_counters(st, ws_floats * sizeof(float), n_counters, &p, &counters)
                                  : workspace(st, ws_floats * sizeof(float), &p);
        if (status) return status;
        partials = static_cast<float*>(p);
    }
    Jobs jobs{};
    jobs.count = count;
    int32_t blocks = 0, widest = 0;
    size_t offset = 0, coffset = 0;
    for (int32_t i = 0; i < count; ++i) {
        Job& jb = jobs.job[i];
        jb.q = ws[i].q;
        jb.s = ws[i].s;
        jb.z = ws[i].z;
        jb.out = cs[i];
        jb.bias = biases ? biases[i] : nullptr;
        jb.N = ws[i].N;
        jb.bpr = ws[i].bpr;
        jb.tiles = ceil_div(ws[i].bpr, STRIP);
        jb.slices = slices;
        jb.groups_per_slice = gps;
        jb.block_begin = blocks;
        jb.partials = slices > 1 ? partials + offset : nullptr;
        jb.counters = inkernel ? counters + coffset : nullptr;
        offset += static_cast<size_t>(slices) * M * ws[i].N;
        coffset += jb.tiles;
        blocks += jb.tiles * slices;
        if (M * ws[i].N > widest) widest = M * ws[i].N;
    }
    // LDS: x hi/lo for the slice rows, the 16 row maxima; the wave reduction reuses it.
    const int r = M >= 3 ? 4 : M;
    const int ncol = ws[0].bits == 4 ? 16 : 8;
    const size_t lds_x = static_cast<size_t>(4) * M * rows + 16 * sizeof(uint32_t);
    const size_t lds_red = static_cast<size_t>(64) * ncol * r * sizeof(float);
    const size_t lds = lds_x > lds_red ? lds_x : lds_red;
    const dim3 grid(static_cast<uint32_t>(blocks));
    if (ws[0].bits == 4) {
        if (waves == 8) launch_r<4, 8>(r, zp, grid, lds, st, a, M, w0.K, w0.g, jobs, alpha, accumulate);
        else if (waves == 2) launch_r<4, 2>(r, zp, grid, lds, st, a, M, w0.K, w0.g, jobs, alpha, accumulate);
        else launch_r<4, 4>(r, zp, grid, lds, st, a, M, w0.K, w0.g, jobs, alpha, accumulate);
    } else {
        if (waves == 8) launch_r<8, 8>(r, zp, grid, lds, st, a, M, w0.K, w0.g, jobs, alpha, accumulate);
        else if (waves == 2) launch_r<8, 2>(r, zp, grid, lds, st, a, M, w0.K, w0.g, jobs, alpha, accumulate);
        else launch_r<8, 4>(r, zp, grid, lds, st, a, M, w0.K, w0.g, jobs, alpha, accumulate);
    }
    KT_LAUNCHED("qmatmul: mfma gemv kernel");
    if (slices > 1 && !inkernel) {
        gemv_mfma_reduce<<<ceil_div(widest, 256), 256, 0, st>>>(jobs, M, alpha, accumulate);
        KT_LAUNCHED("qmatmul: mfma gemv reduce");
    }
    return KT_OK;
}

}  // namespace kt
