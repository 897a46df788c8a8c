// kt_gemv_wide.hip -- the decode dequant-GEMV at M == 1 on gfx950 MFMA:
//   c[1 x N] = (accumulate ? c : 0) + alpha * x[1 x K] . deq(W) (+ bias),
// MatMul.multiplyQuantizedRow (Engine/kotensor/src/main/kotlin/MatMul.kt:494-536) for
// the reference layout of the weights.
//
// HBM is the bound, so the kernel is built around the load stream:
//
//   * a wave owns a 512-byte strip of the packed rows (a tile) and one load instruction
//     reads 512 contiguous bytes of one row: lane (cl = l % 16, kb = l / 16) reads bytes
//     128 kb + 8 cl .. + 7. A chunk is 8 rows (4 KB per wave); every wave keeps NB
//     chunks in flight and issues exactly the loads it needs;
//   * v_mfma_f32_16x16x32_f16 with a block-diagonal A: k-block kb of B (lanes kb) holds
//     the 8 rows of sub-strip kb, and A row block kb (rows 4 kb .. 4 kb + 3) holds x for
//     those 8 rows only, so one MFMA gives all four sub-strips at once, each in the
//     result rows of its own lanes;
//   * weight bytes become exact fp16 integers in two instructions per pair of rows
//     (v_perm_b32 pairs the byte of two rows, an and-or sets the exponent of 1024:
//     1024 + q, 1024 + 16 q for the high nibble, 1152 + q for INT8 after a bias of 128);
//   * x is split per 32-row unit into three fp16 parts on fixed grids (256 steps each,
//     the unit's largest |x| scaled into [2^14, 2^15), 24 bits below it); the three
//     parts are A rows 0..2 of the block. Every partial sum of part * (1024 + q) over a
//     unit is an integer multiple of the part's grid below 2^24 grids, so the MFMA sums
//     are exact, and so is sum(part * (q - z)) = fma(-(1024 + z), sum(part), that sum);
//   * per unit: res += scale * 2^e * (hi + mid + lo), on every lane (16 columns each);
//   * a workgroup is 2, 4 or 8 waves on one tile; its waves take the units of its
//     K-slice round-robin and meet in LDS. With several K-slices, every workgroup writes
//     its column sums to its slice's row of partial sums (written through to memory) and
//     counts in on a per-tile counter; the last one of the tile adds the slices' rows in
//     slice order and resets the counter. The result therefore does not depend on the
//     order in which the workgroups finish.
//
// Grid shape: one workgroup is one tile x one K-slice. A workgroup's bandwidth is
// limited (about 45 GB/s for 8 waves on MI355X), so the launcher takes as many K-slices
// as keep one round of 8-wave workgroups on the CUs with a unit for every wave.
#include "kt_common.h"

namespace kt {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int MAX_JOBS = 4;
constexpr int UNIT = 32;          // rows per x unit (exponent, parts, sums)
constexpr int CROWS = 8;          // rows per chunk
constexpr int CPU_ = UNIT / CROWS;  // chunks per unit
constexpr int TILE = 512;         // bytes of a row per wave
constexpr int MAX_WAVES = 8;      // waves per workgroup: 2, 4 or 8
constexpr int XB = 2;             // x load instructions per batch (2 units each)

struct Job {
    const uint8_t* q;
    const float* s;
    const int8_t* z;
    float* out;
    const float* bias;
    float* partial;      // [slices][N] the slices' column sums, when slices > 1
    uint32_t* counters;  // [tiles], zero on entry and exit, when slices > 1
    int32_t N, bpr, tiles, slices, units_per_slice;
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

// A constant held in a VGPR: (v & mask) | bits and (v ^ a) + b with such operands are
// one v_and_or_b32 / v_xad_u32 each. Only vector ALU instructions read the result.
__device__ __forceinline__ uint32_t in_vgpr(uint32_t c) {
    uint32_t r;
    asm("v_mov_b32 %0, %1" : "=v"(r) : "s"(c));
    return r;
}

// Max (or sum) over each 32-lane half of the wave, in every lane: a DPP butterfly in
// each 16-lane row, then the row results through scalar registers. The values reduced
// are exact (maxima, sums on one fixed-point grid), so the order does not matter.
template <bool MAX>
__device__ __forceinline__ float dpp_step(float v, int tag) {
    int o;
    switch (tag) {  // dpp_ctrl must be a constant
        case 0: o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false); break;   // quad [1,0,3,2]
        case 1: o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false); break;   // quad [2,3,0,1]
        case 2: o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false); break;  // row_half_mirror
        default: o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false); break; // row_mirror
    }
    return MAX ? fmaxf(v, __int_as_float(o)) : v + __int_as_float(o);
}
template <bool MAX>
__device__ __forceinline__ float half_reduce(float v, int32_t ln) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v = dpp_step<MAX>(v, i);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    const float a = MAX ? fmaxf(r0, r1) : r0 + r1;
    const float b = MAX ? fmaxf(r2, r3) : r2 + r3;
    return ln < 32 ? a : b;
}

// Scales and zero points of one unit's group for a lane's columns: for each nibble side
// (INT8: one), 8 consecutive columns.
template <int BITS>
struct UnitScales {
    float4 s[BITS == 4 ? 4 : 2];
    uint2 z[BITS == 4 ? 2 : 1];
};

// The input row, by XMODE:
//   X_PLAIN  x;
//   X_SWIGLU silu(x) * aux (the SwiGLU gate, computed as silu_mul_kernel does:
//            x / (1 + exp(-x)) with exp in double rounded to float, times up), so the
//            down projection needs no separate gate launch;
//   X_NORM   RMSNorm(x) with weight aux: the product takes x * aux and the result is
//            scaled by r = 1 / sqrt(mean(x^2) + eps), the sum of squares reduced as
//            rmsnorm_kernel does (norm_partial etc.), so the q/k/v and gate/up
//            projections need no separate RMSNorm launch. Every workgroup reads the
//            whole row for the sum (at most 32 KB, from L2) while its weights stream.
constexpr int X_PLAIN = 0, X_SWIGLU = 1, X_NORM = 2;

template <int BITS, int NB, bool ZP, int WAVES, int XMODE>
__global__ void __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2)))
    gemv_wide_kernel(const float* __restrict__ x, const float* __restrict__ aux, float eps, int32_t K, int32_t g,
                     Jobs jobs, float alpha, int32_t accumulate) {
    constexpr int THREADS = 64 * WAVES;
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    constexpr int SIDES = BITS == 4 ? 2 : 1;
    constexpr int NACC = 8 * SIDES;  // accumulators (columns) per lane
    constexpr float OFF = BITS == 4 ? 1024.0f : 1152.0f;
    constexpr float GRID0 = 128.0f, GRID1 = 0.5f, GRID2 = 1.0f / 512.0f;  // 256 steps each below 2^15
    static_assert(NB == CPU_, "the load ring is one unit");

    // The job is blockIdx.y; the empty asm makes the arguments of the load stream load in
    // one round (the output's are needed only at the end).
    Job jb = jobs.job[blockIdx.y];
    asm volatile("" ::"s"(jb.q), "s"(jb.s), "s"(jb.z), "s"(jb.N), "s"(jb.bpr), "s"(jb.tiles), "s"(jb.slices),
                 "s"(jb.units_per_slice), "s"(x), "s"(K), "s"(g));
    if (static_cast<int32_t>(blockIdx.x) >= jb.tiles * jb.slices) return;
    const int32_t N = jb.N, bpr = jb.bpr, half = jb.bpr;
    const int32_t tile = blockIdx.x % jb.tiles;
    const int32_t slice = blockIdx.x / jb.tiles;
    const int32_t units = K / UNIT;
    const int32_t u_begin = slice * jb.units_per_slice;
    const int32_t u_end = min(u_begin + jb.units_per_slice, units);

    const int32_t t = threadIdx.x;
    const int32_t ln = t & 63;
    const int32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int32_t cl = ln & 15, kb = ln >> 4;
    const int32_t col_off = tile * TILE + kb * 128 + cl * 8;  // first byte of this lane in a row
    const bool active = col_off < bpr;
    const int32_t boff = active ? col_off : 0;  // lanes past the row end compute and discard

    // This wave's units: u_begin + wave + k * WAVES, k < my_units.
    const int32_t my_units = u_end - u_begin > wave ? (u_end - u_begin - wave + WAVES - 1) / WAVES : 0;
    const int32_t wave_units = (jb.units_per_slice + WAVES - 1) / WAVES;

    // LDS: per wave, parts [wave_units][4][UNIT] fp16 (hi, mid, lo, zeros) and
    // [wave_units] x {sum hi, sum mid, sum lo, 2^e}; the cross-wave sums reuse it.
    const int32_t xw_bytes = wave_units * (4 * UNIT * 2 + 16);
    _Float16* xs = reinterpret_cast<_Float16*>(smem + wave * xw_bytes);
    float4* sums = reinterpret_cast<float4*>(smem + wave * xw_bytes + wave_units * 4 * UNIT * 2);
    // A role: row cl of the block-diagonal A is x-part cl % 4 for k-block cl / 4.
    const int32_t a_off = ((cl >> 2) == kb ? (cl & 3) : 3) * UNIT;

    const uint32_t mask_lo = in_vgpr(0x000F000Fu), mask_hi = in_vgpr(0x00F000F0u);
    const uint32_t flip = in_vgpr(0x00800080u), exp1024 = in_vgpr(0x64006400u);

    float res[NACC];
#pragma unroll
    for (int a = 0; a < NACC; ++a) res[a] = 0.0f;

    // X_NORM: the row for the sum of squares, loaded first (used after the first unit's
    // loads are out); threads past NORM_THREADS load in-bounds copies and ignore them.
    const int32_t n4 = K >> 2;
    norm_v4 nv[NORM_F4];
    float nsum = 0.0f;
    if constexpr (XMODE == X_NORM) {
#pragma unroll
        for (int i = 0; i < NORM_F4; ++i)
            nv[i] = reinterpret_cast<const norm_v4*>(x)[min(t + i * NORM_THREADS, n4 - 1)];
    }
    __builtin_amdgcn_sched_barrier(0);

    if (my_units > 0) {
        // ---- x: first batch of loads, before the weight loads --------------------------
        const int32_t sub = ln >> 5;  // two units per x instruction
        const int32_t kk = ln & 31;
        float xv[XB], uv[XB];
        auto load_x = [&](int32_t k0) {
#pragma unroll
            for (int b = 0; b < XB; ++b) {
                int32_t k = k0 + 2 * b + sub;
                k = k < my_units ? k : my_units - 1;
                const size_t i = static_cast<size_t>(u_begin + wave + k * WAVES) * UNIT + kk;
                xv[b] = x[i];
                if constexpr (XMODE != X_PLAIN) uv[b] = aux[i];
            }
        };
        // Every loaded slot is processed (slots past my_units only skip their stores): a
        // conditional use would let the compiler sink the load behind the weight loads.
        auto prep_x = [&](int32_t k0) {
#pragma unroll
            for (int b = 0; b < XB; ++b) {
                const int32_t k = k0 + 2 * b + sub;
                if constexpr (XMODE == X_SWIGLU) {
                    const float gv = xv[b];
                    xv[b] = gv / (1.0f + static_cast<float>(exp(-static_cast<double>(gv)))) * uv[b];
                } else if constexpr (XMODE == X_NORM) {
                    xv[b] *= uv[b];
                }
                const float mx = half_reduce<true>(fabsf(xv[b]), ln);
                int e = 0;
                if (mx > 0.0f && mx <= 3.402823466e38f) {
                    frexpf(mx, &e);
                    e -= 15;
                }
                const float xp = ldexpf(xv[b], -e);
                const float hi = rintf(xp * (1.0f / GRID0)) * GRID0;
                const float r1 = xp - hi;
                const float mid = rintf(r1 * (1.0f / GRID1)) * GRID1;
                const float lo = rintf((r1 - mid) * (1.0f / GRID2)) * GRID2;
                const float s0 = half_reduce<false>(hi, ln);
                const float s1 = half_reduce<false>(mid, ln);
                const float s2 = half_reduce<false>(lo, ln);
                if (k < my_units) {
                    _Float16* dst = xs + k * 4 * UNIT + kk;
                    dst[0] = static_cast<_Float16>(hi);
                    dst[UNIT] = static_cast<_Float16>(mid);
                    dst[2 * UNIT] = static_cast<_Float16>(lo);
                    dst[3 * UNIT] = static_cast<_Float16>(0.0f);
                    if (kk == 0) sums[k] = make_float4(s0, s1, s2, ldexpf(1.0f, e));
                }
            }
        };
        load_x(0);
        __builtin_amdgcn_sched_barrier(0);  // the x loads go out first: they are waited for first

        // ---- weight loads: the first unit (NB chunks) ---------------------------------
        // The first chunk goes out with x; the others follow once x is prepared, so the
        // x loads do not queue behind the whole unit.
        uint32_t roff[CROWS];
#pragma unroll
        for (int i = 0; i < CROWS; ++i) roff[i] = static_cast<uint32_t>(i * bpr + boff);
        auto load = [&](uint2* v, int32_t k, int32_t cc) {
            const uint8_t* base =
                jb.q + static_cast<size_t>((u_begin + wave + k * WAVES) * UNIT + cc * CROWS) * bpr;
#pragma unroll
            for (int i = 0; i < CROWS; ++i) v[i] = *reinterpret_cast<const uint2*>(base + roff[i]);
        };
        uint2 buf[NB][CROWS];
        load(buf[0], 0, 0);
        __builtin_amdgcn_sched_barrier(0);
        prep_x(0);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int b = 1; b < NB; ++b) load(buf[b], 0, b);
        if constexpr (XMODE == X_NORM) nsum = t < NORM_THREADS ? norm_partial(nv, t, n4) : 0.0f;

        const int32_t scol = tile * TILE + kb * 128 + cl * 8;  // first column of the lane, low side
        const int32_t scol_c = active ? scol : 0;
        auto load_scales = [&](int32_t k) {
            UnitScales<BITS> sc;
            const size_t gi = static_cast<size_t>((u_begin + wave + k * WAVES) * UNIT / g);
#pragma unroll
            for (int side = 0; side < SIDES; ++side) {
                const int32_t col = (side ? half : 0) + scol_c;
                sc.s[2 * side] = *reinterpret_cast<const float4*>(jb.s + gi * N + col);
                sc.s[2 * side + 1] = *reinterpret_cast<const float4*>(jb.s + gi * N + col + 4);
                if constexpr (ZP) sc.z[side] = *reinterpret_cast<const uint2*>(jb.z + gi * N + col);
                else sc.z[side] = make_uint2(0u, 0u);
            }
            return sc;
        };
        // A unit's scales go out with its first chunk computations and are used at its end.
        UnitScales<BITS> sc = load_scales(0);
        __builtin_amdgcn_sched_barrier(0);

        for (int32_t k0 = 2 * XB; k0 < my_units; k0 += 2 * XB) {
            load_x(k0);
            prep_x(k0);
        }

        // ---- main loop ----------------------------------------------------------------
        f32x4 acc[NACC];
        const f32x4 zero4 = {0.0f, 0.0f, 0.0f, 0.0f};
        // Chunk cc of unit k; the unit's first chunk starts the accumulators at zero.
        auto compute = [&](const uint2* v, int32_t k, int cc) {
            const half8 a = *reinterpret_cast<const half8*>(xs + k * 4 * UNIT + a_off + cc * CROWS);
#pragma unroll
            for (int w = 0; w < 2; ++w) {  // dword of the 8-byte strip
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int j = 4 * w + jj;
                    u32x4 p;
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        p[i] = pair_bytes(w ? v[2 * i].y : v[2 * i].x, w ? v[2 * i + 1].y : v[2 * i + 1].x, jj);
                    if (BITS == 8) {
                        u32x4 bq;
#pragma unroll
                        for (int i = 0; i < 4; ++i) bq[i] = (p[i] ^ flip) + exp1024;  // 1152 + q
                        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, as_half8(bq), cc ? acc[j] : zero4, 0, 0, 0);
                    } else {
                        u32x4 blo, bhi;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            blo[i] = (p[i] & mask_lo) | exp1024;  // 1024 + q
                            bhi[i] = (p[i] & mask_hi) | exp1024;  // 1024 + 16 q
                        }
                        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, as_half8(blo), cc ? acc[j] : zero4, 0, 0, 0);
                        acc[8 + j] =
                            __builtin_amdgcn_mfma_f32_16x16x32_f16(a, as_half8(bhi), cc ? acc[8 + j] : zero4, 0, 0, 0);
                    }
                }
            }
        };
        // res += scale * 2^e * sum over parts of (D_p - (OFF + zero) * S_p), each term exact.
        auto combine = [&](int32_t k, const UnitScales<BITS>& us) {
            const float4 sm = sums[k];
#pragma unroll
            for (int a = 0; a < NACC; ++a) {
                const int side = a >> 3, j = a & 7;
                const float4 s4 = us.s[2 * side + (j >> 2)];
                float scl = (j & 3) == 0 ? s4.x : (j & 3) == 1 ? s4.y : (j & 3) == 2 ? s4.z : s4.w;
                float off = OFF;
                if constexpr (ZP) {
                    const uint32_t zw = j < 4 ? us.z[side].x : us.z[side].y;
                    off += (side ? 16.0f : 1.0f) * static_cast<float>(static_cast<int8_t>((zw >> (8 * (j & 3))) & 0xFFu));
                }
                if (side) scl *= 0.0625f;  // high nibble columns carry 16 q
                const float d = (fmaf(-off, sm.x, acc[a][0]) + fmaf(-off, sm.y, acc[a][1])) + fmaf(-off, sm.z, acc[a][2]);
                res[a] = fmaf(scl * sm.w, d, res[a]);
            }
        };

        int32_t k = 0;
        // Every unit but the last loads the next unit behind its own chunks; the last
        // loads nothing, so no wave reads past its range.
        for (; k + 1 < my_units; ++k) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                compute(buf[b], k, b);
                load(buf[b], k + 1, b);
            }
            combine(k, sc);
            sc = load_scales(k + 1);
        }
#pragma unroll
        for (int b = 0; b < NB; ++b) compute(buf[b], k, b);
        combine(k, sc);
    }

    // ---- the workgroup's waves meet in LDS (reusing the x areas) ------------------------
    // red[wave][column] with column = side * 512 + (kb * 128 + cl * 8 + j) of the tile.
    float* red = reinterpret_cast<float*>(smem);
    __shared__ float npart[NORM_THREADS / 64];
    if constexpr (XMODE == X_NORM) {
        if (my_units == 0) nsum = t < NORM_THREADS ? norm_partial(nv, t, n4) : 0.0f;
        const float ws = norm_wave_sum(nsum);
        if (t < NORM_THREADS && (t & 63) == 0) npart[t >> 6] = ws;
    }
    __syncthreads();
#pragma unroll
    for (int a = 0; a < NACC; ++a) {
        const int side = a >> 3, j = a & 7;
        red[wave * (SIDES * TILE) + side * TILE + kb * 128 + cl * 8 + j] = res[a];
    }
    __syncthreads();
    // Thread t owns tile columns t and t + 512 (INT4) or t (INT8), summed in wave order.
    constexpr int PER_THREAD = SIDES * TILE / THREADS;
    float sum[PER_THREAD];
    int32_t colg[PER_THREAD];
    bool live[PER_THREAD];
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        const int c = t + i * THREADS;  // tile column: side = c / 512, byte = c % 512
        float v = red[c];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) v += red[w * (SIDES * TILE) + c];
        sum[i] = v;
        const int32_t byte = tile * TILE + (c & (TILE - 1));
        live[i] = byte < bpr;
        colg[i] = (c >= TILE ? half : 0) + (live[i] ? byte : 0);
    }

    if (jb.slices > 1) {
        // The slices of the tile meet through their rows of partial sums. The rows are
        // written with system-scope stores (written through the caches), and every
        // thread waits until its own stores are complete (s_waitcnt 0, behind a release
        // fence that keeps the compiler from sinking a store past it) before the
        // barrier, so the counter is taken only after the workgroup's row is in memory.
        // The last workgroup's reads are system-scope loads (past the caches), issued
        // after it has seen the count (a barrier and an acquire fence keep the compiler
        // from hoisting them), so they see every slice's row.
        float* row = jb.partial + static_cast<size_t>(slice) * N;
#pragma unroll
        for (int i = 0; i < PER_THREAD; ++i)
            if (live[i]) __hip_atomic_store(row + colg[i], sum[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        __shared__ uint32_t last;
        if (t == 0)
            last = __hip_atomic_fetch_add(jb.counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) ==
                   static_cast<uint32_t>(jb.slices - 1);
        __syncthreads();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        if (!last) return;
        // eight slices' loads per column in flight at once, then added in slice order
        constexpr int BATCH = 8;
#pragma unroll
        for (int i = 0; i < PER_THREAD; ++i) sum[i] = 0.0f;
        for (int32_t s0 = 0; s0 < jb.slices; s0 += BATCH) {
            float pv[PER_THREAD][BATCH];
#pragma unroll
            for (int i = 0; i < PER_THREAD; ++i)
#pragma unroll
                for (int j = 0; j < BATCH; ++j)
                    pv[i][j] = live[i] && s0 + j < jb.slices
                                   ? __hip_atomic_load(jb.partial + static_cast<size_t>(s0 + j) * N + colg[i],
                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM)
                                   : 0.0f;
#pragma unroll
            for (int i = 0; i < PER_THREAD; ++i)
#pragma unroll
                for (int j = 0; j < BATCH; ++j)
                    if (s0 + j < jb.slices) sum[i] = s0 + j == 0 ? pv[i][j] : sum[i] + pv[i][j];
        }
        if (t == 0) __hip_atomic_store(jb.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    const float al = XMODE == X_NORM ? alpha * norm_scale(npart, K, eps) : alpha;
#pragma unroll
    for (int i = 0; i < PER_THREAD; ++i) {
        if (!live[i]) continue;
        float* dst = jb.out + colg[i];
        float o = accumulate ? *dst : 0.0f;
        o = fmaf(al, sum[i], o);
        if (jb.bias) o += jb.bias[colg[i]];
        *dst = o;
    }
}

struct Forced {
    int slices = 0;
    int waves = 0;
};
Forced g_forced;

// x areas: 4 fp16 parts per x value plus 16 bytes per unit, per wave.
constexpr size_t LDS_X_BYTES = 96 << 10;
constexpr size_t X_UNIT_BYTES = 4 * UNIT * 2 + 16;

struct XInput {
    const float* x;
    const float* aux;  // up (X_SWIGLU) or the RMSNorm weight (X_NORM)
    float eps;
    int mode;
};

template <int BITS, bool ZP, int WAVES>
void launch_one(dim3 grid, size_t lds, hipStream_t st, const XInput& in, int32_t K, int32_t g, const Jobs& jobs,
                float alpha, int32_t accumulate) {
    const dim3 block(64 * WAVES);
    if (in.mode == X_SWIGLU)
        gemv_wide_kernel<BITS, CPU_, ZP, WAVES, X_SWIGLU><<<grid, block, lds, st>>>(in.x, in.aux, in.eps, K, g, jobs,
                                                                                  alpha, accumulate);
    else if (in.mode == X_NORM)
        gemv_wide_kernel<BITS, CPU_, ZP, WAVES, X_NORM><<<grid, block, lds, st>>>(in.x, in.aux, in.eps, K, g, jobs,
                                                                                alpha, accumulate);
    else
        gemv_wide_kernel<BITS, CPU_, ZP, WAVES, X_PLAIN><<<grid, block, lds, st>>>(in.x, in.aux, in.eps, K, g, jobs,
                                                                                 alpha, accumulate);
}

template <int BITS, bool ZP>
void launch_waves(int waves, dim3 grid, size_t lds, hipStream_t st, const XInput& in, int32_t K, int32_t g,
                  const Jobs& jobs, float alpha, int32_t accumulate) {
    if (waves == 8) launch_one<BITS, ZP, 8>(grid, lds, st, in, K, g, jobs, alpha, accumulate);
    else if (waves == 4) launch_one<BITS, ZP, 4>(grid, lds, st, in, K, g, jobs, alpha, accumulate);
    else launch_one<BITS, ZP, 2>(grid, lds, st, in, K, g, jobs, alpha, accumulate);
}

void launch_kernel(int bits, bool zp, int waves, dim3 grid, size_t lds, hipStream_t st, const XInput& in, int32_t K,
                   int32_t g, const Jobs& jobs, float alpha, int32_t accumulate) {
    if (bits == 4) launch_waves<4, true>(waves, grid, lds, st, in, K, g, jobs, alpha, accumulate);
    else if (zp) launch_waves<8, true>(waves, grid, lds, st, in, K, g, jobs, alpha, accumulate);
    else launch_waves<8, false>(waves, grid, lds, st, in, K, g, jobs, alpha, accumulate);
}

struct Plan {
    int32_t slices, waves, ups;
};

size_t lds_bytes(int32_t ups, int32_t waves, int sides) {
    const size_t lds_x = static_cast<size_t>(ceil_div(ups, waves)) * waves * X_UNIT_BYTES;
    const size_t lds_red = static_cast<size_t>(waves) * sides * TILE * sizeof(float);
    return lds_x > lds_red ? lds_x : lds_red;
}

// Eight waves per workgroup and the most K-slices that keep one round of workgroups
// (one per CU) with at least one unit for every wave: measured on MI355X, a second round
// or idle waves cost more than the longer slices.
Plan choose_plan(int64_t tiles, int32_t units) {
    constexpr int32_t W = MAX_WAVES;
    if (units < 1 || tiles < 1) return Plan{1, W, 1};  // no unit of 32 rows: the kernel does not apply
    const int64_t cus = cu_count();
    int32_t slices = static_cast<int32_t>(cus / tiles);
    if (slices > units / W) slices = units / W;
    if (slices < 1) slices = 1;
    int32_t ups = ceil_div(units, slices);
    if (static_cast<size_t>(ceil_div(ups, W)) * W * X_UNIT_BYTES > LDS_X_BYTES)
        ups = static_cast<int32_t>(LDS_X_BYTES / (W * X_UNIT_BYTES)) * W;
    return Plan{ceil_div(units, ups), W, ups};
}

}  // namespace

void set_gemv_wide_config(int32_t slices, int32_t waves) {
    g_forced.slices = slices > 0 ? slices : 0;
    g_forced.waves = waves == 2 || waves == 4 || waves == 8 ? waves : 0;
}

bool gemv_wide_preferred(const WeightView* ws, int32_t count) {
    // Measured on MI355X in graph replay, this kernel is at least as fast as the
    // row-block MFMA kernel (and its second reduction kernel) on every decode shape
    // tried, from 2048 -> 3072 INT4 (8.0 us against 9.0) and 8192 -> 2048 (9.2 against
    // 11.0) to the 4096 x 128256 head; it needs K >= 32.
    (void)count;
    return ws[0].K >= UNIT;
}

bool gemv_wide_supported(const float* a, int32_t m, const WeightView& w, const float* c) {
    (void)a;
    (void)c;
    if (m != 1) return false;
    if (w.g % UNIT != 0 || w.K % UNIT != 0) return false;  // units of 32 rows inside one group
    if (w.bpr % 8 != 0 || !aligned(w.q, 8)) return false;  // 8-byte lane strips
    if (w.N % 8 != 0 || !aligned(w.s, 16) || (w.z && !aligned(w.z, 8))) return false;
    if (w.bits == 4 && w.N % 16 != 0) return false;        // high-nibble scales and zeros stay aligned
    if (static_cast<int64_t>(CROWS) * w.bpr >= (static_cast<int64_t>(1) << 31)) return false;
    return true;
}

int32_t launch_gemv_wide(const float* a, const WeightView* ws, float* const* cs, const float* const* biases, int32_t count,
                         int32_t accumulate, float alpha, hipStream_t st, const float* up, const float* norm_weight,
                         float eps) {
    const WeightView& w0 = ws[0];
    const int32_t units = w0.K / UNIT;
    bool zp = false;
    for (int32_t i = 0; i < count; ++i) zp = zp || ws[i].z != nullptr;
    if (zp)
        for (int32_t i = 0; i < count; ++i)
            if (!ws[i].z) return fail(KT_ERR_ARGUMENT, "grouped weights must all have zero points or none");
    const int sides = w0.bits == 4 ? 2 : 1;

    int64_t tiles_total = 0;
    for (int32_t i = 0; i < count; ++i) tiles_total += ceil_div(ws[i].bpr, TILE);
    Plan plan = choose_plan(tiles_total, units);
    if (g_forced.slices || g_forced.waves) {
        const int32_t waves = g_forced.waves ? g_forced.waves : plan.waves;
        int32_t slices = g_forced.slices ? g_forced.slices : plan.slices;
        if (slices > units) slices = units;
        const int32_t ups = ceil_div(units, slices);
        plan = Plan{ceil_div(units, ups), waves, ups};
    }
    if (static_cast<size_t>(ceil_div(plan.ups, plan.waves)) * plan.waves * X_UNIT_BYTES > LDS_X_BYTES)
        return fail(KT_ERR_ARGUMENT, "wide gemv: K-slice of %d units too long for the x area", plan.ups);
    const int32_t slices = plan.slices;

    size_t n_partial = 0;  // floats: each weight's [slices][N]
    if (slices > 1)
        for (int32_t i = 0; i < count; ++i) n_partial += static_cast<size_t>(slices) * ws[i].N;
    float* partials = nullptr;
    uint32_t* counters = nullptr;
    if (slices > 1) {
        if (static_cast<size_t>(tiles_total) > MAX_COUNTERS)
            return fail(KT_ERR_ARGUMENT, "wide gemv: too many tiles for the counters");
        void* general = nullptr;
        const int32_t status = workspace_counters(st, n_partial * sizeof(float), static_cast<size_t>(tiles_total),
                                                  &general, &counters);
        if (status) return status;
        partials = static_cast<float*>(general);
    }
    Jobs jobs{};
    jobs.count = count;
    int32_t blocks = 0;
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
        jb.tiles = ceil_div(ws[i].bpr, TILE);
        jb.slices = slices;
        jb.units_per_slice = plan.ups;
        jb.partial = slices > 1 ? partials + offset : nullptr;
        jb.counters = slices > 1 ? counters + coffset : nullptr;
        offset += static_cast<size_t>(slices) * ws[i].N;
        coffset += jb.tiles;
        if (jb.tiles * slices > blocks) blocks = jb.tiles * slices;
    }
    const size_t lds = lds_bytes(plan.ups, plan.waves, sides);
    const dim3 grid(static_cast<uint32_t>(blocks), static_cast<uint32_t>(count));
    XInput in{a, up ? up : norm_weight, eps, up ? X_SWIGLU : norm_weight ? X_NORM : X_PLAIN};
    if (up && norm_weight) return fail(KT_ERR_ARGUMENT, "wide gemv: one input transform at a time");
    if (norm_weight && (w0.K % 4 != 0 || w0.K > NORM_F4 * 4 * NORM_THREADS || !aligned(a, 16)))
        return fail(KT_ERR_ARGUMENT, "wide gemv: the RMSNorm input needs a 16-byte aligned row of <= 8192 floats");
    launch_kernel(w0.bits, zp, plan.waves, grid, lds, st, in, w0.K, w0.g, jobs, alpha, accumulate);
    KT_LAUNCHED("qmatmul: wide gemv kernel");
    return KT_OK;
}

}  // namespace kt
