// kt_gemv_mfma.hip -- decode dequant-GEMV for M = 1, 2 rows on gfx950 MFMA:
//   c[M x N] = (accumulate ? c : 0) + alpha * x[M x K] . deq(W) (+ bias),
// the small-M case of MatMul.multiplyQuantized (Engine/kotensor/src/main/kotlin/
// MatMul.kt:460-486; M == 1 is multiplyQuantizedRow :494-536).
//
// The weights stream from HBM once, in the reference layout, and the matrix cores do
// all multiply-adds exactly, so the vector ALU spends under one instruction per weight:
//
//   * v_mfma_f32_16x16x32_f16: lane l holds B[k = 8*(l/16) + i][n = l%16], i < 8. A lane
//     (cl = l%16, kb = l/16) loads rows r0 + 8*kb + i of an 8-byte column strip, so for
//     each byte j of the strip its registers hold the 8 k-values of one column. 16 lanes
//     cover 128 contiguous bytes of a row; a chunk is 32 rows;
//   * weight bytes become fp16 in two instructions per pair of k-values: v_perm_b32
//     puts byte j of two consecutive rows into the low bytes of the two halves and an
//     and-or keeps the nibble under the exponent of 1024, giving the exact integers
//     1024 + q (low nibble), 1024 + 16q (high nibble) or, INT8 bytes biased by 128,
//     1152 + q;
//   * the constant 1024 (1152) and the zero point are removed exactly through the
//     accumulator: per quantization group, x is split into three fp16 parts on fixed
//     grids (hi + mid + lo, 2^13 / g steps each, about 21 bits below the group's
//     largest |x|, which is scaled into [2^14, 2^15)), each part is an A row, and each
//     accumulator starts the group at -(1024 + zero) * sum(part). Every partial sum of
//     the group is then an fp32 integer multiple of the part's grid with at most 24
//     bits, so the MFMA results are exact: sum(part * (q - zero)) per part;
//   * for M == 1 the 16 A rows hold four copies of the three parts in four row blocks;
//     the MFMA for column u uses block u % 4 only, so its result lands in lane group
//     u % 4 and four MFMAs share one accumulator. The per-group combine
//     res += scale * 2^e * (hi + mid + lo) then runs on all 64 lanes, four columns each
//     (two blocks of two x rows for M == 2);
//   * every wave prepares the x of its own groups in its own LDS area before its
//     weight loads, then keeps NB chunks (16 KB) of weight loads in flight;
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
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

constexpr int MAX_JOBS = 4;
constexpr int CHUNK = 32;  // rows per MFMA k-step (4 lanes groups x 8 rows)
constexpr int STRIP = 128; // bytes of a row per wave (16 lanes x 8 bytes)
constexpr int NB = 4;      // chunks of weight loads in flight per wave
constexpr int MAX_M = 2;   // x rows: three parts (and a zero row) of each take 4 A rows
constexpr int MAX_M_ROWS = 16;  // row mode: one A row per x row (in each of two MFMAs)
constexpr int XB = 4;      // groups of x loaded per batch

struct Job {
    const uint8_t* q;
    const float* s;
    const int8_t* z;
    float* out;
    const float* bias;
    float* partials;     // [slices x M x N] or nullptr
    uint32_t* counters;  // [tiles] for the in-kernel slice reduction, or nullptr
    int32_t N, bpr, tiles, slices, groups_per_slice;
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

// A constant the compiler keeps in a VGPR: (v & mask) | bits and (v ^ a) + b with such
// operands become one v_and_or_b32 / v_xad_u32 each instead of two instructions with
// literals. Only vector ALU instructions read the result.
__device__ __forceinline__ uint32_t in_vgpr(uint32_t c) {
    uint32_t r;
    asm("v_mov_b32 %0, %1" : "=v"(r) : "s"(c));
    return r;
}

// Max (or sum) over the SEG lanes of a segment (32 or 64), in every lane: a DPP
// butterfly inside each 16-lane row (quad swaps, then half-row and row mirrors), then
// the four row results through scalar registers. The values reduced here are exact
// (maxima, or sums of numbers on one fixed-point grid), so the order does not matter.
template <bool MAX>
__device__ __forceinline__ float dpp_step(float v, int ctrl_tag) {
    int o = 0;
    switch (ctrl_tag) {  // dpp_ctrl must be a constant
        case 0: o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false); break;   // quad [1,0,3,2]
        case 1: o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false); break;   // quad [2,3,0,1]
        case 2: o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false); break;  // row_half_mirror
        default: o = __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false); break; // row_mirror
    }
    return MAX ? fmaxf(v, __int_as_float(o)) : v + __int_as_float(o);
}
template <int SEG, bool MAX>
__device__ __forceinline__ float segment_reduce(float v, int32_t ln) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v = dpp_step<MAX>(v, i);
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    const float a = MAX ? fmaxf(r0, r1) : r0 + r1;
    const float b = MAX ? fmaxf(r2, r3) : r2 + r3;
    if (SEG == 64) return MAX ? fmaxf(a, b) : a + b;
    return ln < 32 ? a : b;
}

// Scales and zero points of one quantization group for a lane's NACC columns.
template <int NACC>
struct GroupScales {
    float s[NACC];
    int32_t z[NACC];
};

// MP: x rows per A row block (1 or 2; M <= MP); CPG: 32-row chunks per group.
template <int BITS, int MP, int WAVES, int CPG, bool ZP>
__global__ void __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2)))
    gemv_mfma_kernel(const float* __restrict__ x, int32_t M, int32_t K, Jobs jobs, int32_t wave_groups,
                     float alpha, int32_t accumulate) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    constexpr int g = CPG * CHUNK;
    constexpr int NCOL = BITS == 4 ? 16 : 8;  // columns per lane strip: (byte, nibble) pairs
    constexpr int NR = 4 / MP;                 // A row blocks
    constexpr int NACC = NCOL / NR;            // accumulators (columns) per lane
    constexpr float OFF = BITS == 4 ? 1024.0f : 1152.0f;
    // fixed-point parts: P steps each; grids 2^15 / P, 2^15 / P^2, 2^15 / P^3
    constexpr int P = 8192 / g;
    constexpr float GRID0 = 32768.0f / P, GRID1 = GRID0 / P, GRID2 = GRID1 / P;
    static_assert(NB % CPG == 0, "a ring of NB chunks holds whole groups");

    // The job is blockIdx.y: its fields load at an offset known at wave start. The empty
    // asm takes every argument the kernel uses, so all scalar loads go out in one round
    // instead of one round per use; then blocks past the job's own count leave.
    Job jb = jobs.job[blockIdx.y];
    asm volatile("" ::"s"(jb.q), "s"(jb.s), "s"(jb.z), "s"(jb.out), "s"(jb.bias), "s"(jb.partials), "s"(jb.counters),
                 "s"(jb.N), "s"(jb.bpr), "s"(jb.tiles), "s"(jb.slices), "s"(jb.groups_per_slice), "s"(x), "s"(M), "s"(K),
                 "s"(wave_groups), "s"(alpha), "s"(accumulate));
    const int32_t local = blockIdx.x;
    if (local >= jb.tiles * jb.slices) return;
    const int32_t N = jb.N, bpr = jb.bpr, half = jb.bpr;
    const int32_t tile = local % jb.tiles;
    const int32_t slice = local / jb.tiles;
    const int32_t G = K / g;
    const int32_t g_begin = slice * jb.groups_per_slice;
    const int32_t g_end = min(g_begin + jb.groups_per_slice, G);

    const int32_t t = threadIdx.x;
    const int32_t ln = t & 63;
    const int32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int32_t cl = ln & 15, kb = ln >> 4;
    const int32_t col_off = tile * STRIP + cl * 8;
    const bool active = col_off < bpr;
    const int32_t boff = active ? col_off : 0;  // lanes past the row end compute and discard

    // This wave's quantization groups: g_begin + wave + k * WAVES, k < my_groups.
    const int32_t my_groups = g_end - g_begin > wave ? (g_end - g_begin - wave + WAVES - 1) / WAVES : 0;
    const int32_t my_chunks = my_groups * CPG;

    // The wave's LDS area: parts [wave_groups][M][4][g] fp16 (hi, mid, lo, zeros), then
    // [wave_groups][M] x {sum hi, sum mid, sum lo, 2^e}.
    const int32_t parts_bytes = wave_groups * M * 8 * g;
    const int32_t xw_bytes = parts_bytes + wave_groups * M * 16;
    _Float16* xs = reinterpret_cast<_Float16*>(smem + wave * xw_bytes);
    float4* sums = reinterpret_cast<float4*>(smem + wave * xw_bytes + parts_bytes);

    // A role of this lane (A row cl): block cl / (4 MP), x row (cl / 4) % MP, part cl % 4.
    const int32_t a_block = cl / (4 * MP);
    const int32_t a_row = (cl >> 2) % MP;
    const int32_t a_part = a_row < M ? (cl & 3) : 3;  // rows past M read the zero part
    const int32_t a_off = ((a_row < M ? a_row : 0) * 4 + a_part) * g + 8 * kb;
    // D role (result rows 4 kb .. 4 kb + 3): block kb / MP, x row kb % MP, part i.
    const int32_t d_block = kb / MP;
    const int32_t d_row = kb % MP;
    const int32_t d_row_c = d_row < M ? d_row : 0;
    // Accumulator a holds column u = a * NR + d_block: byte u & 7, high nibble if u >= 8.
    int32_t col[NACC];
#pragma unroll
    for (int a = 0; a < NACC; ++a) {
        const int u = a * NR + d_block;
        col[a] = (u >= 8 ? half : 0) + boff + (u & 7);
    }

    float res[NACC];
#pragma unroll
    for (int a = 0; a < NACC; ++a) res[a] = 0.0f;
    const uint32_t mask_lo = in_vgpr(0x000F000Fu), mask_hi = in_vgpr(0x00F000F0u);
    const uint32_t flip = in_vgpr(0x00800080u), exp1024 = in_vgpr(0x64006400u);

    if (my_groups > 0) {
        // ---- x of this wave's groups as fixed-point fp16 parts ------------------------
        // The first batch of x loads goes out before the weight loads (a wave's loads
        // return in order), the parts are made while the weights are in flight.
        constexpr int SEG = CPG >= 2 ? 64 : 32;       // lanes per group
        constexpr int VPL = CPG >= 2 ? CPG / 2 : 1;   // x values per lane per group and row
        constexpr int GPI = 64 / SEG;                 // groups per wave instruction
        const int32_t sub = SEG == 32 ? (ln >> 5) : 0;
        const int32_t kk0 = ln & (SEG - 1);
        float xv[XB][MP][VPL];
        auto load_x = [&](int32_t k0) {
#pragma unroll
            for (int b = 0; b < XB; ++b) {
                int32_t k = k0 + b * GPI + sub;
                k = k < my_groups ? k : my_groups - 1;
                const float* px = x + static_cast<size_t>(g_begin + wave + k * WAVES) * g + kk0;
#pragma unroll
                for (int m = 0; m < MP; ++m)
#pragma unroll
                    for (int v = 0; v < VPL; ++v) xv[b][m][v] = px[static_cast<size_t>(m < M ? m : 0) * K + 64 * v];
            }
        };
        // Every loaded slot is processed (slots past my_groups only skip their stores):
        // a conditional use would let the compiler sink the slot's load behind the
        // weight loads, and waiting for it would then wait for all of them.
        auto prep_x = [&](int32_t k0) {
#pragma unroll
            for (int b = 0; b < XB; ++b) {
                const int32_t k = k0 + b * GPI + sub;
#pragma unroll
                for (int m = 0; m < MP; ++m) {  // MP == M
                    float mx = 0.0f;
#pragma unroll
                    for (int v = 0; v < VPL; ++v) mx = fmaxf(mx, fabsf(xv[b][m][v]));
                    mx = segment_reduce<SEG, true>(mx, ln);
                    int e = 0;
                    if (mx > 0.0f && mx <= 3.402823466e38f) {
                        frexpf(mx, &e);
                        e -= 15;
                    }
                    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f;
                    _Float16* dst = xs + (k * M + m) * 4 * g + kk0;
#pragma unroll
                    for (int v = 0; v < VPL; ++v) {
                        const float xp = ldexpf(xv[b][m][v], -e);
                        const float hi = rintf(xp * (1.0f / GRID0)) * GRID0;
                        const float r1 = xp - hi;
                        const float mid = rintf(r1 * (1.0f / GRID1)) * GRID1;
                        const float lo = rintf((r1 - mid) * (1.0f / GRID2)) * GRID2;
                        s0 += hi;
                        s1 += mid;
                        s2 += lo;
                        if (k < my_groups) {
                            dst[64 * v] = static_cast<_Float16>(hi);
                            dst[g + 64 * v] = static_cast<_Float16>(mid);
                            dst[2 * g + 64 * v] = static_cast<_Float16>(lo);
                            dst[3 * g + 64 * v] = static_cast<_Float16>(0.0f);
                        }
                    }
                    s0 = segment_reduce<SEG, false>(s0, ln);
                    s1 = segment_reduce<SEG, false>(s1, ln);
                    s2 = segment_reduce<SEG, false>(s2, ln);
                    if (k < my_groups && kk0 == 0) sums[k * M + m] = make_float4(s0, s1, s2, ldexpf(1.0f, e));
                }
            }
        };
        load_x(0);
        __builtin_amdgcn_sched_barrier(0);  // the x loads go out first: they are waited for first

        // ---- weight loads: NB chunks in flight -------------------------------------
        uint32_t roff[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) roff[i] = static_cast<uint32_t>((8 * kb + i) * bpr + boff);
        auto chunk_base = [&](int32_t c) {
            const int32_t k = c / CPG, cc = c - k * CPG;
            return jb.q + static_cast<size_t>((g_begin + wave + k * WAVES) * g + cc * CHUNK) * bpr;
        };
        auto load = [&](uint2* v, int32_t c) {
            const uint8_t* base = chunk_base(c < my_chunks ? c : my_chunks - 1);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const uint2*>(base + roff[i]);
        };
        uint2 buf[NB][8];
#pragma unroll
        for (int b = 0; b < NB; ++b) load(buf[b], b);

        auto load_scales = [&](int32_t k) {
            GroupScales<NACC> sc;
            const size_t gi = static_cast<size_t>(g_begin + wave + k * WAVES);
#pragma unroll
            for (int a = 0; a < NACC; ++a) {
                sc.s[a] = jb.s[gi * N + col[a]];
                sc.z[a] = ZP ? static_cast<int32_t>(jb.z[gi * N + col[a]]) : 0;
            }
            return sc;
        };
        // Scales of the next SR groups are in flight with the weights (slot = group % SR).
        constexpr int SR = NB / CPG >= 2 ? 2 : 1;
        GroupScales<NACC> scales[SR];
#pragma unroll
        for (int i = 0; i < SR; ++i) scales[i] = load_scales(i < my_groups ? i : my_groups - 1);
        __builtin_amdgcn_sched_barrier(0);

        prep_x(0);
        for (int32_t k0 = XB * GPI; k0 < my_groups; k0 += XB * GPI) {
            load_x(k0);
            prep_x(k0);
        }

        // ---- main loop --------------------------------------------------------------
        f32x4 acc[NACC];
        // Accumulators start group k at -(OFF + zero) * sum(part) for D rows (parts) 0..2.
        auto start_group = [&](int32_t k, const GroupScales<NACC>& gs) {
            const float4 sm = sums[k * M + d_row_c];
#pragma unroll
            for (int a = 0; a < NACC; ++a) {
                const int u = a * NR + d_block;
                const float zs = (BITS == 4 && u >= 8) ? 16.0f : 1.0f;
                const float off = -(OFF + zs * static_cast<float>(gs.z[a]));
                acc[a] = f32x4{off * sm.x, off * sm.y, off * sm.z, 0.0f};
            }
        };
        auto compute = [&](const uint2* v, int32_t c) {
            const int32_t k = c / CPG, cc = c - k * CPG;
            const half8 a = *reinterpret_cast<const half8*>(xs + k * M * 4 * g + a_off + cc * CHUNK);
            half8 ab[NR];
#pragma unroll
            for (int r = 0; r < NR; ++r) ab[r] = a_block == r ? a : half8{};
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
                        acc[j / NR] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ab[j % NR], as_half8(bq), acc[j / NR], 0, 0, 0);
                    } else {
                        u32x4 blo, bhi;
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            blo[i] = (p[i] & mask_lo) | exp1024;  // 1024 + q
                            bhi[i] = (p[i] & mask_hi) | exp1024;  // 1024 + 16 q
                        }
                        acc[j / NR] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ab[j % NR], as_half8(blo), acc[j / NR], 0, 0, 0);
                        acc[(8 + j) / NR] =
                            __builtin_amdgcn_mfma_f32_16x16x32_f16(ab[(8 + j) % NR], as_half8(bhi), acc[(8 + j) / NR], 0, 0, 0);
                    }
                }
            }
        };
        // res += scale * 2^e * (hi + mid + lo) of local group k.
        auto combine = [&](int32_t k, const GroupScales<NACC>& gs) {
            const float f = sums[k * M + d_row_c].w;
#pragma unroll
            for (int a = 0; a < NACC; ++a) {
                const int u = a * NR + d_block;
                const float sc = (BITS == 4 && u >= 8) ? gs.s[a] * 0.0625f : gs.s[a];
                res[a] = fmaf(sc * f, (acc[a][0] + acc[a][1]) + acc[a][2], res[a]);
            }
        };

        start_group(0, scales[0]);
        for (int32_t c0 = 0; c0 < my_chunks; c0 += NB) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int32_t c = c0 + b;
                if (c < my_chunks) {
                    compute(buf[b], c);
                    if (b % CPG == CPG - 1) {
                        const int32_t k = c / CPG;  // k % SR == (b / CPG) % SR: NB / CPG is a multiple of SR
                        const int slot = (b / CPG) % SR;  // a constant once the loop is unrolled
                        const int next = (slot + 1) % SR;
                        combine(k, scales[slot]);
                        scales[slot] = load_scales(k + SR < my_groups ? k + SR : my_groups - 1);
                        if (k + 1 < my_groups) start_group(k + 1, scales[next]);
                    }
                }
                load(buf[b], c + NB);
            }
        }
    }

    // ---- waves of the workgroup meet in LDS (reusing the x areas), in wave order -------
    float* red = reinterpret_cast<float*>(smem);  // [WAVES - 1][NACC][64 lanes]
    __syncthreads();
    if (wave > 0)
#pragma unroll
        for (int a = 0; a < NACC; ++a) red[((wave - 1) * NACC + a) * 64 + ln] = res[a];
    __syncthreads();
    if (wave != 0) return;
    for (int w = 1; w < WAVES; ++w)
#pragma unroll
        for (int a = 0; a < NACC; ++a) res[a] += red[((w - 1) * NACC + a) * 64 + ln];

    const bool live = active && d_row < M;
    if (jb.partials && jb.counters) {
        // In-kernel slice reduction (write-through sums + tile counter), as in kt_gemv.hip.
        float* part = jb.partials + (static_cast<size_t>(slice) * M + d_row_c) * N;
        if (live)
#pragma unroll
            for (int a = 0; a < NACC; ++a)
                __hip_atomic_store(part + col[a], res[a], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __builtin_amdgcn_s_waitcnt(0);
        uint32_t old = 0;
        if (ln == 0) old = __hip_atomic_fetch_add(jb.counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __builtin_amdgcn_readfirstlane(old);
        if (old != static_cast<uint32_t>(jb.slices - 1)) return;
        // The last workgroup of the strip: every slice's sums (write-through, read past
        // the caches), all loads in flight together, added in slice order.
        constexpr int MAXS = 8;  // the host takes this path for at most 8 slices
        float v[MAXS][NACC];
#pragma unroll
        for (int sp = 0; sp < MAXS; ++sp)
#pragma unroll
            for (int a = 0; a < NACC; ++a) {
                v[sp][a] = 0.0f;
                if (live && sp < jb.slices && sp != slice)
                    v[sp][a] = __hip_atomic_load(jb.partials + (static_cast<size_t>(sp) * M + d_row_c) * N + col[a],
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
#pragma unroll
        for (int a = 0; a < NACC; ++a) {
            float sum = 0.0f;
#pragma unroll
            for (int sp = 0; sp < MAXS; ++sp)
                if (sp < jb.slices) {
                    const float vv = sp == slice ? res[a] : v[sp][a];
                    sum = sp == 0 ? vv : sum + vv;
                }
            res[a] = sum;
        }
        if (ln == 0) __hip_atomic_store(jb.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (!live) return;
#pragma unroll
    for (int a = 0; a < NACC; ++a) {
        const int32_t n = col[a];
        if (jb.partials && !jb.counters) {
            jb.partials[(static_cast<size_t>(slice) * M + d_row) * N + n] = res[a];
        } else {
            float* dst = jb.out + static_cast<size_t>(d_row) * N + n;
            float o = accumulate ? *dst : 0.0f;
            o = fmaf(alpha, res[a], o);
            if (jb.bias) o += jb.bias[n];
            *dst = o;
        }
    }
}

// 3 <= M <= 16 x rows ("row mode"): the 16 A rows are the x rows themselves, scaled per
// (row, group) by a power of two so that the row's largest |x| in the group lies in
// [2^14, 2^15), and each value is split into fp16 hi = fp16(x) and lo = fp16(x - hi);
// two MFMAs (hi rows, then lo rows) share one accumulator. B is the exact fp16 integer
// q - zero (INT4 high nibble: 16 (q - zero)), made as in the M <= 2 kernel and then
// reduced by the packed fp16 difference with 1024 + zero (1152 + zero for INT8), which is
// exact; every product is exact in fp32, and the MFMA accumulates a group in fp32. Per
// group: res += scale * 2^e(row) * D. The error is that of x held to 22 significant bits
// (relative 2^-22 of each value) plus fp32 accumulation, so a row's result does not
// depend on the row count beyond fp32 rounding (the reference's rows do not: its tile
// kernel gives every row the single-row result, QuantizationTest.kt:110-134); the kernel
// is HBM-bound, so the second MFMA costs issue slots only. Lane (cl, kb) keeps D rows
// 4 kb .. 4 kb + 3 (x rows) of its own columns. An INT4 workgroup takes one nibble side
// of its strip (eight accumulators): the two workgroups of a strip are numbered 8 apart,
// so they run on one XCD and the second reads the strip's bytes from that XCD's L2.
template <int BITS, int WAVES, int CPG, bool ZP>
__global__ void __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(2)))
    gemv_rows_kernel(const float* __restrict__ x, int32_t M, int32_t K, Jobs jobs, int32_t wave_groups,
                     float alpha, int32_t accumulate) {
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    constexpr int g = CPG * CHUNK;
    constexpr int NACC = 8;  // byte positions of the lane strip (one nibble side for INT4)
    constexpr float OFF = BITS == 4 ? 1024.0f : 1152.0f;
    static_assert(NB % CPG == 0, "a ring of NB chunks holds whole groups");

    Job jb = jobs.job[blockIdx.y];
    asm volatile("" ::"s"(jb.q), "s"(jb.s), "s"(jb.z), "s"(jb.out), "s"(jb.bias), "s"(jb.partials), "s"(jb.N),
                 "s"(jb.bpr), "s"(jb.tiles), "s"(jb.slices), "s"(jb.groups_per_slice), "s"(x), "s"(M), "s"(K),
                 "s"(wave_groups), "s"(alpha), "s"(accumulate));
    const int32_t local = blockIdx.x;
    const int32_t side = BITS == 4 ? (local >> 3) & 1 : 0;
    const int32_t pair = BITS == 4 ? ((local >> 4) << 3) | (local & 7) : local;
    if (pair >= jb.tiles * jb.slices) return;
    const int32_t N = jb.N, bpr = jb.bpr, half = jb.bpr;
    const int32_t tile = pair % jb.tiles;
    const int32_t slice = pair / jb.tiles;
    const int32_t G = K / g;
    const int32_t g_begin = slice * jb.groups_per_slice;
    const int32_t g_end = min(g_begin + jb.groups_per_slice, G);

    const int32_t t = threadIdx.x;
    const int32_t ln = t & 63;
    const int32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int32_t cl = ln & 15, kb = ln >> 4;
    const int32_t col_off = tile * STRIP + cl * 8;
    const bool active = col_off < bpr;
    const int32_t boff = active ? col_off : 0;  // lanes past the row end compute and discard

    const int32_t my_groups = g_end - g_begin > wave ? (g_end - g_begin - wave + WAVES - 1) / WAVES : 0;
    const int32_t my_chunks = my_groups * CPG;

    // The wave's LDS area: x [wave_groups][hi, lo][16 rows][g] fp16, then [wave_groups][16] 2^e.
    const int32_t xs_bytes = wave_groups * 2 * 16 * 2 * g;
    const int32_t xw_bytes = xs_bytes + wave_groups * 16 * 4;
    _Float16* xs = reinterpret_cast<_Float16*>(smem + wave * xw_bytes);
    float* fw = reinterpret_cast<float*>(smem + wave * xw_bytes + xs_bytes);

    int32_t col[NACC];
#pragma unroll
    for (int a = 0; a < NACC; ++a) col[a] = (side ? half : 0) + boff + a;
    float res[NACC][4];
#pragma unroll
    for (int a = 0; a < NACC; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) res[a][r] = 0.0f;
    const uint32_t mask = in_vgpr(side ? 0x00F000F0u : 0x000F000Fu);
    const uint32_t flip = in_vgpr(0x00800080u), exp1024 = in_vgpr(0x64006400u);
    const float zs = side ? 16.0f : 1.0f;       // the high nibble carries 16 q
    const float ss = side ? 0.0625f : 1.0f;

    if (my_groups > 0) {
        // ---- x of this wave's groups ------------------------------------------------
        // Lane (row xm = ln / 4, quarter xq = ln % 4) loads g / 4 consecutive values of its
        // row's group: the row's group maximum is a quad maximum (two DPP steps), and the
        // lane writes its fp16 values as 16-byte LDS stores. Lanes of rows past M load
        // row 0 and store nothing: those A rows are zeroed at use.
        constexpr int VQ = g / 4;   // values per lane: 8, 16 or 32
        constexpr int F4 = VQ / 4;  // float4 loads per lane
        const int32_t xm = ln >> 2, xq = ln & 3;
        const int32_t xrow = xm < M ? xm : 0;
        float4 xv[F4];
        auto load_x = [&](int32_t k) {
            k = k < my_groups ? k : my_groups - 1;
            const float4* px = reinterpret_cast<const float4*>(
                x + static_cast<size_t>(xrow) * K + static_cast<size_t>(g_begin + wave + k * WAVES) * g + xq * VQ);
#pragma unroll
            for (int f = 0; f < F4; ++f) xv[f] = px[f];
        };
        auto prep_x = [&](int32_t k) {
            float mx = 0.0f;
#pragma unroll
            for (int f = 0; f < F4; ++f)
                mx = fmaxf(fmaxf(mx, fmaxf(fabsf(xv[f].x), fabsf(xv[f].y))), fmaxf(fabsf(xv[f].z), fabsf(xv[f].w)));
            mx = dpp_step<true>(mx, 0);  // quad [1,0,3,2]
            mx = dpp_step<true>(mx, 1);  // quad [2,3,0,1]
            int e = 0;
            if (mx > 0.0f && mx <= 3.402823466e38f) {
                frexpf(mx, &e);
                e -= 15;
            }
            if (xm < M) {
                // hi = fp16(x 2^-e), lo = fp16(x 2^-e - hi): 22 significant bits of every
                // value, so a row's result does not depend on how many rows share the call
                _Float16* dst = xs + (k * 32 + xm) * g + xq * VQ;
#pragma unroll
                for (int h = 0; h < VQ / 8; ++h) {
                    half8 hv, lv;
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        const float4& q4 = xv[(8 * h + i) / 4];
                        const int c = (8 * h + i) % 4;
                        const float v = ldexpf(c == 0 ? q4.x : c == 1 ? q4.y : c == 2 ? q4.z : q4.w, -e);
                        hv[i] = static_cast<_Float16>(v);
                        lv[i] = static_cast<_Float16>(v - static_cast<float>(hv[i]));
                    }
                    *reinterpret_cast<half8*>(dst + 8 * h) = hv;
                    *reinterpret_cast<half8*>(dst + 16 * g + 8 * h) = lv;
                }
                if (xq == 0) fw[k * 16 + xm] = ldexpf(1.0f, e);
            }
        };
        load_x(0);
        __builtin_amdgcn_sched_barrier(0);

        uint32_t roff[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) roff[i] = static_cast<uint32_t>((8 * kb + i) * bpr + boff);
        auto chunk_base = [&](int32_t c) {
            const int32_t k = c / CPG, cc = c - k * CPG;
            return jb.q + static_cast<size_t>((g_begin + wave + k * WAVES) * g + cc * CHUNK) * bpr;
        };
        auto load = [&](uint2* v, int32_t c) {
            const uint8_t* base = chunk_base(c < my_chunks ? c : my_chunks - 1);
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = *reinterpret_cast<const uint2*>(base + roff[i]);
        };
        uint2 buf[NB][8];
#pragma unroll
        for (int b = 0; b < NB; ++b) load(buf[b], b);

        auto load_scales = [&](int32_t k) {
            GroupScales<NACC> sc;
            const size_t gi = static_cast<size_t>(g_begin + wave + k * WAVES);
#pragma unroll
            for (int a = 0; a < NACC; ++a) {
                sc.s[a] = jb.s[gi * N + col[a]];
                sc.z[a] = ZP ? static_cast<int32_t>(jb.z[gi * N + col[a]]) : 0;
            }
            return sc;
        };
        constexpr int SR = NB / CPG >= 2 ? 2 : 1;
        GroupScales<NACC> scales[SR];
#pragma unroll
        for (int i = 0; i < SR; ++i) scales[i] = load_scales(i < my_groups ? i : my_groups - 1);
        __builtin_amdgcn_sched_barrier(0);

        prep_x(0);
        for (int32_t k = 1; k < my_groups; ++k) {
            load_x(k);
            prep_x(k);
        }

        // ---- main loop --------------------------------------------------------------
        f32x4 acc[NACC];
        h2 zh[NACC];  // (OFF + zs * zero) in both halves, per column of the group
        auto start_group = [&](const GroupScales<NACC>& gs) {
#pragma unroll
            for (int a = 0; a < NACC; ++a) {
                acc[a] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                const _Float16 o = static_cast<_Float16>(OFF + zs * static_cast<float>(gs.z[a]));
                zh[a] = h2{o, o};
            }
        };
        auto compute = [&](const uint2* v, int32_t c) {
            const int32_t k = c / CPG, cc = c - k * CPG;
            const _Float16* pa = xs + (k * 32 + cl) * g + cc * CHUNK + 8 * kb;
            const half8 xa = *reinterpret_cast<const half8*>(pa);
            const half8 xl = *reinterpret_cast<const half8*>(pa + 16 * g);
            const half8 a = cl < M ? xa : half8{};
            const half8 al = cl < M ? xl : half8{};
#pragma unroll
            for (int w = 0; w < 2; ++w) {
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int j = 4 * w + jj;
                    u32x4 bq;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint32_t p =
                            pair_bytes(w ? v[2 * i].y : v[2 * i].x, w ? v[2 * i + 1].y : v[2 * i + 1].x, jj);
                        const uint32_t e = BITS == 8 ? (p ^ flip) + exp1024 : (p & mask) | exp1024;
                        bq[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, e) - zh[j]);
                    }
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, as_half8(bq), acc[j], 0, 0, 0);
                    acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, as_half8(bq), acc[j], 0, 0, 0);
                }
            }
        };
        auto combine = [&](int32_t k, const GroupScales<NACC>& gs) {
            const float4 f = *reinterpret_cast<const float4*>(fw + k * 16 + 4 * kb);
#pragma unroll
            for (int a = 0; a < NACC; ++a) {
                const float sc = gs.s[a] * ss;
                res[a][0] = fmaf(sc * f.x, acc[a][0], res[a][0]);
                res[a][1] = fmaf(sc * f.y, acc[a][1], res[a][1]);
                res[a][2] = fmaf(sc * f.z, acc[a][2], res[a][2]);
                res[a][3] = fmaf(sc * f.w, acc[a][3], res[a][3]);
            }
        };

        start_group(scales[0]);
        for (int32_t c0 = 0; c0 < my_chunks; c0 += NB) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const int32_t c = c0 + b;
                if (c < my_chunks) {
                    compute(buf[b], c);
                    if (b % CPG == CPG - 1) {
                        const int32_t k = c / CPG;
                        const int slot = (b / CPG) % SR;
                        const int next = (slot + 1) % SR;
                        combine(k, scales[slot]);
                        scales[slot] = load_scales(k + SR < my_groups ? k + SR : my_groups - 1);
                        if (k + 1 < my_groups) start_group(scales[next]);
                    }
                }
                load(buf[b], c + NB);
            }
        }
    }

    // ---- waves of the workgroup meet in LDS (reusing the x areas), in wave order -------
    float* red = reinterpret_cast<float*>(smem);  // [WAVES - 1][NACC][4][64 lanes]
    __syncthreads();
    if (wave > 0)
#pragma unroll
        for (int a = 0; a < NACC; ++a)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[(((wave - 1) * NACC + a) * 4 + r) * 64 + ln] = res[a][r];
    __syncthreads();
    if (wave != 0) return;
    for (int w = 1; w < WAVES; ++w)
#pragma unroll
        for (int a = 0; a < NACC; ++a)
#pragma unroll
            for (int r = 0; r < 4; ++r) res[a][r] += red[(((w - 1) * NACC + a) * 4 + r) * 64 + ln];
    if (!active) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int32_t row = 4 * kb + r;
        if (row >= M) continue;
#pragma unroll
        for (int a = 0; a < NACC; ++a) {
            const int32_t n = col[a];
            if (jb.partials) {
                jb.partials[(static_cast<size_t>(slice) * M + row) * N + n] = res[a][r];
            } else {
                float* dst = jb.out + static_cast<size_t>(row) * N + n;
                float o = accumulate ? *dst : 0.0f;
                o = fmaf(alpha, res[a][r], o);
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

// x areas of a workgroup: every wave keeps four fp16 parts of its groups (8 bytes per x
// value and row) plus four floats per group and row.
constexpr size_t LDS_X_BYTES = 64 << 10;

template <int BITS, int MP, int WAVES, int CPG, bool ZP>
void launch_kernel(dim3 grid, size_t lds, hipStream_t st, const float* a, int32_t M, int32_t K, const Jobs& jobs,
                   int32_t wave_groups, float alpha, int32_t accumulate) {
    gemv_mfma_kernel<BITS, MP, WAVES, CPG, ZP>
        <<<grid, dim3(64 * WAVES), lds, st>>>(a, M, K, jobs, wave_groups, alpha, accumulate);
}

template <int BITS, int MP, int WAVES, int CPG>
void launch_zp(bool zp, dim3 grid, size_t lds, hipStream_t st, const float* a, int32_t M, int32_t K, const Jobs& jobs,
               int32_t wave_groups, float alpha, int32_t accumulate) {
    if (BITS == 4 || zp) launch_kernel<BITS, MP, WAVES, CPG, true>(grid, lds, st, a, M, K, jobs, wave_groups, alpha, accumulate);
    else launch_kernel<BITS, MP, WAVES, CPG, false>(grid, lds, st, a, M, K, jobs, wave_groups, alpha, accumulate);
}

template <int BITS, int MP, int WAVES>
void launch_cpg(int cpg, bool zp, dim3 grid, size_t lds, hipStream_t st, const float* a, int32_t M, int32_t K,
                const Jobs& jobs, int32_t wave_groups, float alpha, int32_t accumulate) {
    if (cpg == 1) launch_zp<BITS, MP, WAVES, 1>(zp, grid, lds, st, a, M, K, jobs, wave_groups, alpha, accumulate);
    else if (cpg == 2) launch_zp<BITS, MP, WAVES, 2>(zp, grid, lds, st, a, M, K, jobs, wave_groups, alpha, accumulate);
    else launch_zp<BITS, MP, WAVES, 4>(zp, grid, lds, st, a, M, K, jobs, wave_groups, alpha, accumulate);
}

template <int BITS, int MP>
void launch_waves(int waves, int cpg, bool zp, dim3 grid, size_t lds, hipStream_t st, const float* a, int32_t M,
                  int32_t K, const Jobs& jobs, int32_t wave_groups, float alpha, int32_t accumulate) {
    if (waves == 8) launch_cpg<BITS, MP, 8>(cpg, zp, grid, lds, st, a, M, K, jobs, wave_groups, alpha, accumulate);
    else launch_cpg<BITS, MP, 4>(cpg, zp, grid, lds, st, a, M, K, jobs, wave_groups, alpha, accumulate);
}

template <int BITS>
void launch_bits(int mp, int waves, int cpg, bool zp, dim3 grid, size_t lds, hipStream_t st, const float* a, int32_t M,
                 int32_t K, const Jobs& jobs, int32_t wave_groups, float alpha, int32_t accumulate) {
    if (mp == 1) launch_waves<BITS, 1>(waves, cpg, zp, grid, lds, st, a, M, K, jobs, wave_groups, alpha, accumulate);
    else launch_waves<BITS, 2>(waves, cpg, zp, grid, lds, st, a, M, K, jobs, wave_groups, alpha, accumulate);
}

template <int BITS, int WAVES, int CPG>
void launch_rows_zp(bool zp, dim3 grid, size_t lds, hipStream_t st, const float* a, int32_t M, int32_t K,
                    const Jobs& jobs, int32_t wave_groups, float alpha, int32_t accumulate) {
    if (BITS == 4 || zp)
        gemv_rows_kernel<BITS, WAVES, CPG, true>
            <<<grid, dim3(64 * WAVES), lds, st>>>(a, M, K, jobs, wave_groups, alpha, accumulate);
    else
        gemv_rows_kernel<BITS, WAVES, CPG, false>
            <<<grid, dim3(64 * WAVES), lds, st>>>(a, M, K, jobs, wave_groups, alpha, accumulate);
}

template <int BITS>
void launch_rows(int waves, int cpg, bool zp, dim3 grid, size_t lds, hipStream_t st, const float* a, int32_t M,
                 int32_t K, const Jobs& jobs, int32_t wave_groups, float alpha, int32_t accumulate) {
    // four waves: with eight the register budget of 2 waves per SIMD is exceeded
    (void)waves;
    if (cpg == 1) launch_rows_zp<BITS, 4, 1>(zp, grid, lds, st, a, M, K, jobs, wave_groups, alpha, accumulate);
    else if (cpg == 2) launch_rows_zp<BITS, 4, 2>(zp, grid, lds, st, a, M, K, jobs, wave_groups, alpha, accumulate);
    else launch_rows_zp<BITS, 4, 4>(zp, grid, lds, st, a, M, K, jobs, wave_groups, alpha, accumulate);
}

// LDS bytes of one quantization group of x per wave: M <= 2 keeps four fp16 parts per
// value and row plus four floats per row; row mode keeps 16 rows of fp16 hi and lo parts
// plus 2^e per row.
size_t x_group_bytes(int32_t m, int32_t g) {
    return m > MAX_M ? static_cast<size_t>(16) * (4 * g + 4) : static_cast<size_t>(m) * (8 * g + 16);
}

}  // namespace

void set_gemv_mfma_config(int32_t slices, int32_t waves, int32_t reduce, int32_t disable) {
    g_forced.slices = slices > 0 ? slices : 0;
    g_forced.waves = (waves == 4 || waves == 8) ? waves : 0;
    g_forced.reduce = (reduce == 1 || reduce == 2) ? reduce : 0;
    g_forced.disable = disable ? 1 : 0;
}

bool gemv_mfma_supported(const float* a, int32_t m, const WeightView& w, const float* c) {
    (void)a;
    (void)c;
    if (g_forced.disable) return false;
    if (m < 1 || m > MAX_M_ROWS) return false;
    if (w.g != 32 && w.g != 64 && w.g != 128) return false;  // whole 32-row chunks, up to 4 per group
    if (w.K % w.g != 0) return false;
    if (w.bpr % 8 != 0 || !aligned(w.q, 8)) return false;  // 8-byte lane strips
    if (w.N % 8 != 0 || !aligned(w.s, 16) || (w.z && !aligned(w.z, 8))) return false;
    if (w.bits == 4 && w.N % 16 != 0) return false;        // high-nibble columns start 8-aligned
    // lane row offsets within a chunk are 32-bit
    if (static_cast<int64_t>(CHUNK) * w.bpr >= (static_cast<int64_t>(1) << 31)) return false;
    // one x group of every row must fit a wave's LDS area (row mode runs four waves)
    if ((m > MAX_M ? 4 : 8) * x_group_bytes(m, w.g) > LDS_X_BYTES) return false;
    if (m > MAX_M && !aligned(a, 16)) return false;  // row mode reads x as float4
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

    // M > 2: row mode (gemv_rows_kernel); INT4 strips there take two workgroups (sides).
    const bool rows = M > MAX_M;
    const int32_t sides = rows && w0.bits == 4 ? 2 : 1;
    int64_t tiles_total = 0;
    for (int32_t i = 0; i < count; ++i) tiles_total += ceil_div(ws[i].bpr, STRIP);
    const int32_t target_waves = cu_count() * 8;
    // Waves per workgroup (each takes whole groups), then K-slices until the GPU is
    // covered; the x areas in LDS bound the groups of a slice.
    int32_t waves = g_forced.waves && !rows ? g_forced.waves : 4;
    const int64_t wg_waves = tiles_total * sides * waves;
    int32_t slices;
    if (rows) {
        // About one workgroup per CU, at least four K-slices, at most one group per slice
        // (measured on MI355X: 4096 x 4096 INT4 11.9 us at 8 slices against 13.1 at 16,
        // 896 x 4864 9.6 at 6 against 10.9 at 3; the 4096 x 14336 gate/up is best at 4).
        slices = static_cast<int32_t>(cu_count() / (tiles_total * sides));
        if (slices < 4) slices = 4;
        if (slices > 16) slices = 16;  // the most measured; 4096 -> 1024 INT4 is best there
        if (slices > G) slices = G;
    } else {
        slices = static_cast<int32_t>((target_waves + wg_waves - 1) / wg_waves);
        const int32_t max_slices = G / waves > 1 ? G / waves : 1;
        if (slices > max_slices) slices = max_slices;
    }
    if (slices < 1) slices = 1;
    const size_t per_group = x_group_bytes(M, w0.g);
    const int32_t cap_groups = static_cast<int32_t>(LDS_X_BYTES / (waves * per_group));  // per wave, >= 1
    const int32_t min_slices = ceil_div(G, cap_groups * waves);
    if (slices < min_slices) slices = min_slices;
    if (g_forced.slices) slices = g_forced.slices > min_slices ? g_forced.slices : min_slices;
    if (slices > G) slices = G;
    constexpr int32_t MAX_INKERNEL_SLICES = 8;
    // A few more slices than the in-kernel limit buy less than the reduction kernel costs.
    if (!rows && !g_forced.slices && slices > MAX_INKERNEL_SLICES && slices < 2 * MAX_INKERNEL_SLICES &&
        min_slices <= MAX_INKERNEL_SLICES)
        slices = MAX_INKERNEL_SLICES;
    // Every slice takes gps whole groups; the last may take fewer.
    const int32_t gps = ceil_div(G, slices);
    slices = ceil_div(G, gps);
    const int32_t wave_groups = ceil_div(gps, waves);
    size_t ws_floats = 0, n_counters = 0;
    if (slices > 1)
        for (int32_t i = 0; i < count; ++i) {
            ws_floats += static_cast<size_t>(slices) * M * ws[i].N;
            n_counters += ceil_div(ws[i].bpr, STRIP);
        }
    bool inkernel = !rows && slices > 1 && slices <= MAX_INKERNEL_SLICES && n_counters <= MAX_COUNTERS;
    if (g_forced.reduce == 1) inkernel = false;
    if (g_forced.reduce == 2 && !rows && slices > 1 && slices <= MAX_INKERNEL_SLICES && n_counters <= MAX_COUNTERS)
        inkernel = true;
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
    int32_t blocks = 0, widest = 0;  // blocks of the largest job: the grid is blocks x count
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
        jb.partials = slices > 1 ? partials + offset : nullptr;
        jb.counters = inkernel ? counters + coffset : nullptr;
        offset += static_cast<size_t>(slices) * M * ws[i].N;
        coffset += jb.tiles;
        // row mode INT4: workgroups b and b + 8 take the two sides of one (tile, slice)
        const int32_t jb_blocks = sides == 2 ? ceil_div(jb.tiles * slices, 8) * 16 : jb.tiles * slices;
        if (jb_blocks > blocks) blocks = jb_blocks;
        if (M * ws[i].N > widest) widest = M * ws[i].N;
    }
    // LDS: the waves' x areas; the cross-wave reduction reuses them.
    const int mp = M == 1 ? 1 : 2;
    const int ncol = ws[0].bits == 4 ? 16 : 8;
    const int nacc = ncol / (4 / mp);
    const size_t xw = static_cast<size_t>(wave_groups) * per_group;
    const size_t lds_x = waves * xw;
    // cross-wave sums: nacc values per lane, or (row mode) 8 columns x 4 rows
    const size_t lds_red = static_cast<size_t>(waves - 1) * (rows ? 8 * 4 : nacc) * 64 * sizeof(float);
    const size_t lds = lds_x > lds_red ? lds_x : lds_red;
    const int cpg = w0.g / CHUNK;
    const dim3 grid(static_cast<uint32_t>(blocks), static_cast<uint32_t>(count));
    if (rows) {
        if (ws[0].bits == 4) launch_rows<4>(waves, cpg, zp, grid, lds, st, a, M, w0.K, jobs, wave_groups, alpha, accumulate);
        else launch_rows<8>(waves, cpg, zp, grid, lds, st, a, M, w0.K, jobs, wave_groups, alpha, accumulate);
    } else if (ws[0].bits == 4) {
        launch_bits<4>(mp, waves, cpg, zp, grid, lds, st, a, M, w0.K, jobs, wave_groups, alpha, accumulate);
    } else {
        launch_bits<8>(mp, waves, cpg, zp, grid, lds, st, a, M, w0.K, jobs, wave_groups, alpha, accumulate);
    }
    KT_LAUNCHED("qmatmul: mfma gemv kernel");
    if (slices > 1 && !inkernel) {
        gemv_mfma_reduce<<<ceil_div(widest, 256), 256, 0, st>>>(jobs, M, alpha, accumulate);
        KT_LAUNCHED("qmatmul: mfma gemv reduce");
    }
    return KT_OK;
}

}  // namespace kt
