// kt_gemv_rows_packed.hip -- 2 to 16 rows on the column-run copy:
//   c[M x N] = (accumulate ? c : 0) + alpha * x[M x K] . deq(W) (+ bias),
// MatMul.multiplyQuantized's M > 1 branch (Engine/kotensor/src/main/kotlin/MatMul.kt:479-485,
// computeQuantizedTile :830-881) for the few-row products of batched or speculative decode.
//
// The weights stream exactly as in the one-row kernel (kt_gemv_packed.hip): a workgroup of
// eight waves owns 8 / ks column sets over ks K-parts, each wave streams its set's 1 KB
// (INT8 2 KB) chunks with four in flight (non-temporal loads) and reads its scales and
// zero points from rows staged in LDS; so a call moves the weight bytes once, whatever M.
//
// Arithmetic (exact products, fp32 sums, the reference's per-group combine):
//   * x: one launch before the product (rows_prep_kernel, a workgroup per row) scales each
//     row by a power of two, 2^s_m, so that its largest |x| lies in [2^14, 2^15), and
//     splits it into two fp16 parts, hi = fp16(x 2^s) and lo = fp16(x 2^s - hi): 22
//     significant bits, written as the MFMA's A operands, 16 bytes per (run, part, lane
//     group, row), which the product's workgroups copy into LDS. (Converting x inside
//     every workgroup instead repeats M K conversions per workgroup: slower at M = 8.)
//   * weights: the exact integers q - z as fp16 (the bits of 1024 + q from the nibble or
//     byte, minus 1024 + z in one packed fp16 add). The chunk's 16-byte lane pieces hold
//     one run each (lane group kb: run kb); four lane swaps across the lane groups
//     (v_permlane32_swap, v_permlane16_swap) transpose them so that lane group kb holds
//     k 8 kb .. 8 kb + 7 of every run, and each MFMA step covers one run, one group;
//   * v_mfma_f32_16x16x32_f16, hi then lo into one accumulator per run: every product is
//     exact in fp32 (11-bit x part times an integer of at most 9 bits); lane (kb, n) gets
//     rows 4 kb .. 4 kb + 3 of column n, and y += scale(group, n) * D per run
//     (combineGroup, MatMul.kt:804-828, per run); INT4 high nibbles enter as 16 (q - z),
//     so the prep divides x's parts at those positions by 16 (exact);
//   * K's sub-parts (kt_packed.h) are summed alone and added in a fixed tree, whatever
//     the K split; then y * 2^-s_m.
// A row's result therefore differs from the one-row kernel's only by the rounding of x to
// 22 bits and the order of fp32 sums (normwise near 1e-7 against the oracle), and does
// not depend on the other rows of the call (QuantizationTest.kt:110-134 asks 1e-4).
// The x tiles live in LDS for the whole K range a workgroup covers when they fit, else in
// phases: at a phase change the workgroup meets at a barrier and copies the next ones
// (their loads then queue behind the weight loads in flight).
#include "kt_common.h"
#include "kt_packed.h"

#include <algorithm>

namespace kt {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int W = 8;                  // waves per workgroup
constexpr int R = 4;                  // chunks in flight per wave
constexpr int MAX_ROWS = 16;

// Bytes of x tiles per run: two parts x four lane groups x M rows x 16 bytes.
__host__ __device__ constexpr int32_t run_tile_bytes(int32_t M) { return 2 * 4 * 16 * M; }
constexpr int PREP_THREADS = 256;
constexpr int MAX_PIECES = 16;  // 16-byte pieces of x tiles a thread moves per round

// x [M x K] -> the A tiles [K / 32 runs][part][lane group kb][row][8 halves] of MT rows
// (rows M .. MT - 1 zero) and the row shifts s_m (16 ints, zero past M): one workgroup per
// tile row, once per call, so that the product's workgroups only copy tiles. K % 32 == 0.
template <int BITS>
__global__ void __launch_bounds__(PREP_THREADS)
    rows_prep_kernel(const float* __restrict__ x, int32_t M, int32_t MT, int32_t K, _Float16* __restrict__ at,
                     int32_t* __restrict__ shifts) {
    __shared__ float red[PREP_THREADS / 64];
    const int32_t m = blockIdx.x, t = threadIdx.x;
    const int32_t units = K >> 3;  // 8 k per unit
    if (m >= M) {  // a padding row of the tiles
        for (int32_t u = t; u < units; u += PREP_THREADS) {
            _Float16* base = at + static_cast<size_t>(u >> 2) * (2 * 4 * 8 * MT);
            *reinterpret_cast<u32x4*>(base + (0 * 4 + (u & 3)) * MT * 8 + m * 8) = u32x4{0u, 0u, 0u, 0u};
            *reinterpret_cast<u32x4*>(base + (1 * 4 + (u & 3)) * MT * 8 + m * 8) = u32x4{0u, 0u, 0u, 0u};
        }
        if (t == 0) shifts[m] = 0;
        return;
    }
    const float* row = x + static_cast<size_t>(m) * K;
    // the row's largest |x| (a NaN or an infinity compares above every finite value)
    uint32_t mb = 0u;
    for (int32_t u = t; u < units; u += PREP_THREADS) {
        const float4 a = reinterpret_cast<const float4*>(row)[2 * u];
        const float4 b = reinterpret_cast<const float4*>(row)[2 * u + 1];
        mb = max(mb, max(max(max(__float_as_uint(fabsf(a.x)), __float_as_uint(fabsf(a.y))),
                             max(__float_as_uint(fabsf(a.z)), __float_as_uint(fabsf(a.w)))),
                         max(max(__float_as_uint(fabsf(b.x)), __float_as_uint(fabsf(b.y))),
                             max(__float_as_uint(fabsf(b.z)), __float_as_uint(fabsf(b.w))))));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mb = max(mb, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mb), o, 64)));
    if ((t & 63) == 0) red[t >> 6] = __uint_as_float(mb);
    __syncthreads();
    mb = max(max(__float_as_uint(red[0]), __float_as_uint(red[1])), max(__float_as_uint(red[2]), __float_as_uint(red[3])));
    // largest |x| into [2^14, 2^15); a zero or non-finite row is not scaled (non-finite
    // values then make non-finite outputs, as the reference's sums do)
    const int32_t s = mb == 0u || mb >= 0x7F800000u ? 0 : 15 - __builtin_amdgcn_frexp_expf(__uint_as_float(mb));
    for (int32_t u = t; u < units; u += PREP_THREADS) {
        const float4 a = reinterpret_cast<const float4*>(row)[2 * u];
        const float4 b = reinterpret_cast<const float4*>(row)[2 * u + 1];
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        half8 hv, lv;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float xs = ldexpf(v[j], s);
            const _Float16 h = static_cast<_Float16>(xs);
            // INT4: positions 4..7 of the 8 meet high nibbles, which enter as 16 (q - z)
            const float f = BITS == 4 && j >= 4 ? 0.0625f : 1.0f;
            hv[j] = static_cast<_Float16>(static_cast<float>(h) * f);
            lv[j] = static_cast<_Float16>((xs - static_cast<float>(h)) * f);  // the difference is exact
        }
        const int32_t run = u >> 2, kb = u & 3;
        _Float16* base = at + static_cast<size_t>(run) * (2 * 4 * 8 * MT);
        *reinterpret_cast<half8*>(base + (0 * 4 + kb) * MT * 8 + m * 8) = hv;
        *reinterpret_cast<half8*>(base + (1 * 4 + kb) * MT * 8 + m * 8) = lv;
    }
    if (t == 0) {
        shifts[m] = s;
        if (m == 0)
            for (int32_t r = MT; r < MAX_ROWS; ++r) shifts[r] = 0;
    }
}

// The workgroup's LDS: the x tiles of one phase [ks][cpp chunks][4 runs][tile], each tile
// [part][lane group kb][row][8 halves]; each wave's staged scale and zero-point rows; the
// meeting area [W][16 rows][16 columns] floats.
__host__ __device__ constexpr int32_t rows_lds_a(int32_t ks, int32_t cpp, int32_t M) {
    return ks * cpp * 4 * run_tile_bytes(M);
}
__host__ __device__ constexpr int32_t rows_lds_stage(int32_t ks, int32_t cpp, int32_t M) {
    return rows_lds_a(ks, cpp, M);
}
__host__ __device__ constexpr int32_t rows_lds_red(int32_t ks, int32_t cpp, int32_t M, int32_t rows) {
    return rows_lds_stage(ks, cpp, M) + W * rows * STAGE_ROW_BYTES;
}
__host__ __device__ constexpr int32_t rows_lds_bytes(int32_t ks, int32_t cpp, int32_t M, int32_t rows) {
    return rows_lds_red(ks, cpp, M, rows) + W * 16 * 16 * 4;
}

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}
__device__ __forceinline__ half2v as_h2(uint32_t v) { return __builtin_bit_cast(half2v, v); }
__device__ __forceinline__ uint32_t as_u(half2v v) { return __builtin_bit_cast(uint32_t, v); }
// (a & m) | o in one instruction (the compiler emits two)
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(o));
    return r;
}

// 4 x 4 transpose of dwords across the lane groups: on entry lane group r holds V[r][d]
// in v[d]; on exit lane group r holds V[d][r] in v[d].
__device__ __forceinline__ void transpose4(uint32_t (&v)[4]) {
    auto a = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
    auto b = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
    auto c = __builtin_amdgcn_permlane16_swap(a[0], b[0], false, false);
    auto d = __builtin_amdgcn_permlane16_swap(a[1], b[1], false, false);
    v[0] = c[0];
    v[1] = c[1];
    v[2] = d[0];
    v[3] = d[1];
}

// GS: the group size's class (0: g = 32, a group per run; 1: g = 64, a group per two
// runs; 2: g >= 128, one group per chunk), MT: rows of the x tiles (4, 8 or 16; rows M ..
// MT - 1 are zero).
template <int BITS, bool ZP, int GS, int MT>
__global__ void __launch_bounds__(64 * W)
    gemv_rows_packed_kernel(const uint8_t* __restrict__ packed, const _Float16* __restrict__ at,
                            const int32_t* __restrict__ shifts_m, int32_t M, int32_t N, int32_t K, int32_t shifts,
                            int32_t cpp, float alpha, float* out, int32_t accumulate, const float* bias) {
    constexpr int BB = block_bytes(BITS);
    constexpr int NB = BITS == 4 ? 1 : 2;  // 16-byte loads per lane and chunk
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int32_t kslog = shifts & 15, gshift = shifts >> 4;
    const int32_t ks = 1 << kslog;
    const int32_t sets = N >> 4, chunks = (K + CHUNK - 1) >> 7, G = (K + (RUN << gshift) - 1) >> (gshift + 5);
    const int32_t tid = threadIdx.x, ln = tid & 63;
    const int32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int32_t cslog = 3 - kslog;
    const int32_t set0 = blockIdx.x << cslog;
    if (set0 >= sets) return;
    const int32_t my_cs = wave & ((1 << cslog) - 1), kp = wave >> cslog;
    const int32_t my_set = set0 + my_cs;
    const bool set_live = my_set < sets;
    const int32_t set = set_live ? my_set : sets - 1;
    const int32_t nmax = (chunks + ks - 1) >> kslog;
    const int32_t c_begin = (kp * chunks) >> kslog;
    const int32_t n = (((kp + 1) * chunks) >> kslog) - c_begin;
    const int32_t k0 = c_begin * CHUNK;
    const int32_t nl = ln & 15, kb = ln >> 4;
    const int32_t col = set * SET + nl;
    const int32_t phases = (nmax + cpp - 1) / cpp;
    const int32_t rows = stage_rows(nmax, gshift);
    constexpr int32_t tile = run_tile_bytes(MT);

    // ---- loads, in the order they complete: the first phase's x tiles (16 bytes per
    // thread and step), the wave's scale and zero-point rows, the first R chunks of weights.
    const int32_t piece_count = ks * cpp * 4 * tile / 16;  // 16-byte pieces of a phase
    const __amdgpu_buffer_rsrc_t ar =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<_Float16*>(at), 0, (K >> 5) * tile, 0x00020000);
    // piece p of phase ph: part p / per_part, then that part's chunks [begin + ph cpp, ...)
    // in run order, contiguous in the prep's output; runs past K (the padding of the last
    // chunk) and chunks past the part read zeros
    auto piece_offset = [&](int32_t p, int32_t ph) -> int32_t {
        const int32_t per_part = cpp * 4 * tile / 16;
        const int32_t part = p / per_part, within = p - part * per_part;
        const int32_t cb = ((part * chunks) >> kslog) + ph * cpp;
        const int32_t ce = ((part + 1) * chunks) >> kslog;
        const int32_t off = cb * 4 * tile + within * 16;
        return off < ce * 4 * tile ? off : 0x7FFFFFF0;
    };
    const int32_t rounds = (piece_count + 64 * W * MAX_PIECES - 1) / (64 * W * MAX_PIECES);
    u32x4 ap[MAX_PIECES];
    auto load_round = [&](int32_t ph, int32_t rd) {
#pragma unroll
        for (int i = 0; i < MAX_PIECES; ++i) {
            const int32_t p = tid + 64 * W * (MAX_PIECES * rd + i);
            ap[i] = p < piece_count
                        ? __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ar, piece_offset(p, ph), 0, 0))
                        : u32x4{0u, 0u, 0u, 0u};
        }
    };
    auto store_round = [&](int32_t rd) {
#pragma unroll
        for (int i = 0; i < MAX_PIECES; ++i) {
            const int32_t p = tid + 64 * W * (MAX_PIECES * rd + i);
            if (p < piece_count) reinterpret_cast<u32x4*>(smem)[p] = ap[i];
        }
    };
    load_round(0, 0);

    const float* ps = reinterpret_cast<const float*>(packed + static_cast<int64_t>(sets) * chunks * BB);
    const int8_t* pz = reinterpret_cast<const int8_t*>(ps + static_cast<int64_t>(sets) * G * SET);
    const int32_t g0 = k0 >> (gshift + 5);
    const __amdgpu_buffer_rsrc_t sr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(ps), 0, G * N * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t zr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(ZP ? pz : reinterpret_cast<const int8_t*>(ps)), 0,
                                          G * N, 0x00020000);
    u32x4 sst[4];
    u32x4 zst;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int32_t r = g0 + 16 * i + (ln >> 2);
        const int32_t off = r < G ? ((set * G + r) * SET + 4 * (ln & 3)) * 4 : G * N * 4;
        sst[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(sr, off, 0, 0));
    }
    if constexpr (ZP) {
        const int32_t r = g0 + ln;
        zst = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(zr, r < G ? (set * G + r) * SET : G * N, 0, 0));
    }
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(packed + (static_cast<int64_t>(set) * chunks + c_begin) * BB), 0, n * BB, 0x00020000);
    u32x4 wb[R][NB];
    auto issue = [&](int slot, int32_t cc) {
#pragma unroll
        for (int h = 0; h < NB; ++h)
            wb[slot][h] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        wr, cc * BB + h * 1024 + 16 * ln, 0, NONTEMPORAL));
    };
#pragma unroll
    for (int s = 0; s < R; ++s) issue(s, s);
    const int4 rsh = *reinterpret_cast<const int4*>(shifts_m + 4 * kb);  // rows 4 kb .. 4 kb + 3

    // ---- into LDS: the x tiles, the wave's staged rows ---------------------------------
    store_round(0);
    for (int32_t rd = 1; rd < rounds; ++rd) {  // a phase larger than one round
        load_round(0, rd);
        store_round(rd);
    }
    unsigned char* stg = smem + rows_lds_stage(ks, cpp, MT) + wave * rows * STAGE_ROW_BYTES;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (16 * i + (ln >> 2) < rows) *reinterpret_cast<u32x4*>(stg + i * 1024 + 16 * ln) = sst[i];
    if constexpr (ZP)
        if (ln < rows) *reinterpret_cast<u32x4*>(stg + rows * SET * 4 + 16 * ln) = zst;
    __syncthreads();

    // lanes of rows past MT read row MT - 1's operand: an MFMA's output rows depend only
    // on their own A rows, and rows past M are never stored
    const int32_t a_lane = kb * MT * 16 + min(nl, MT - 1) * 16;
    float y[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    // sub-parts of K, each summed alone and added in a balanced tree in K order (the
    // one-row kernel's scheme): the result does not depend on ks
    const int32_t sp_count = SUB_PARTS >> kslog, sp0 = kp * sp_count;
    int32_t sp = 0;
    int32_t sp_end = (((sp0 + 1) * chunks) >> SUB_LOG) - c_begin;
    float tree[4][3] = {};
    float part[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto close_sub_part = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            part[i] = tree_push(tree[i], sp, y[i]);
            y[i] = 0.0f;
        }
        ++sp;
        sp_end = (((sp0 + sp + 1) * chunks) >> SUB_LOG) - c_begin;
    };
    const int32_t run0 = k0 >> 5;  // the wave's first run
    // the slot's weights, transposed: t[r] = k 8 kb .. 8 kb + 7 of run r of the chunk
    // (INT8: t2[r] the next 8 bytes) -- taken out of the ring so the slot refills at once
    auto take = [&](int s, uint32_t (&t)[4], uint32_t (&t2)[4]) {
        if constexpr (BITS == 4) {
            t[0] = wb[s][0][0];
            t[1] = wb[s][0][1];
            t[2] = wb[s][0][2];
            t[3] = wb[s][0][3];
            transpose4(t);
        } else {
            // 8-byte pieces p = k 8p .. 8p + 7: dwords (2p, 2p + 1) of the lane's 32 bytes
            t[0] = wb[s][0][0];
            t[1] = wb[s][0][2];
            t[2] = wb[s][1][0];
            t[3] = wb[s][1][2];
            t2[0] = wb[s][0][1];
            t2[1] = wb[s][0][3];
            t2[2] = wb[s][1][1];
            t2[3] = wb[s][1][3];
            transpose4(t);
            transpose4(t2);
        }
    };
    constexpr int NGC = GS == 0 ? 4 : GS == 1 ? 2 : 1;  // quantization groups a chunk touches
    constexpr int RPG = 4 / NGC;                        // runs per group
    auto process = [&](const uint32_t (&t)[4], const uint32_t (&t2)[4], int32_t cl, bool live, int32_t ph) {
        if (live)
            while (cl >= sp_end) close_sub_part();
        // a chunk past the wave's range adds nothing; its reads stay in the phase's tiles
        // and the wave's staged rows (the phase's first chunk is below nmax)
        const int32_t cc = live ? cl : ph * cpp;
        const unsigned char* tc = smem + (kp * cpp + (cc - ph * cpp)) * 4 * tile + a_lane;
        float sc[NGC];
        uint32_t zc[NGC];
        half8 ah[4], al[4];
#pragma unroll
        for (int gi = 0; gi < NGC; ++gi) {
            // the group row of runs gi RPG .. (a run past K, the padding of the last chunk,
            // takes the last group's; its x is zero)
            const int32_t gr = min((run0 + cc * 4 + gi * RPG) >> gshift, G - 1) - g0;
            sc[gi] = *reinterpret_cast<const float*>(stg + gr * (SET * 4) + nl * 4);
            zc[gi] = ZP ? stg[rows * SET * 4 + gr * SET + nl] : 0u;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            ah[r] = *reinterpret_cast<const half8*>(tc + r * tile);
            al[r] = *reinterpret_cast<const half8*>(tc + r * tile + 4 * MT * 16);
        }
        // the exact fp16 offsets of each group: 1024 + z (INT4 also 1024 + 16 z), 1152 + z
        half2v ol[NGC], oh[NGC];
#pragma unroll
        for (int gi = 0; gi < NGC; ++gi) {
            if constexpr (BITS == 4) {
                const uint32_t zz = zc[gi] | (zc[gi] << 16);
                ol[gi] = as_h2(zz | 0x64006400u);
                oh[gi] = as_h2((zz << 4) | 0x64006400u);
            } else {
                const uint32_t zz = (zc[gi] ^ 0x80u) | ((zc[gi] ^ 0x80u) << 16);
                ol[gi] = as_h2(zz | 0x64006400u);
                oh[gi] = ol[gi];
            }
        }
        half8 b[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            uint32_t bw[4];
            const half2v o_lo = ol[r / RPG], o_hi = oh[r / RPG];
            if constexpr (BITS == 4) {
                // halves 0..3: low nibbles, the bits of 1024 + q; 4..7: high nibbles, 1024 + 16 q;
                // minus 1024 + z and 1024 + 16 z (the bits 0x6400 | z, 0x6400 | z << 4)
                const half2v ol = o_lo, oh = o_hi;
                const uint32_t p01 = perm(0u, t[r], 0x0c010c00u), p23 = perm(0u, t[r], 0x0c030c02u);
                bw[0] = as_u(as_h2(and_or(p01, 0x000F000Fu, 0x64006400u)) - ol);
                bw[1] = as_u(as_h2(and_or(p23, 0x000F000Fu, 0x64006400u)) - ol);
                bw[2] = as_u(as_h2(and_or(p01, 0x00F000F0u, 0x64006400u)) - oh);
                bw[3] = as_u(as_h2(and_or(p23, 0x00F000F0u, 0x64006400u)) - oh);
            } else {
                // byte b: (b ^ 0x80) + 1024 = 1152 + q; minus 1152 + z, the bits 0x6400 | (z ^ 0x80)
                const half2v o = o_lo;
                bw[0] = as_u(as_h2(perm(0u, t[r], 0x0c010c00u) ^ 0x64806480u) - o);
                bw[1] = as_u(as_h2(perm(0u, t[r], 0x0c030c02u) ^ 0x64806480u) - o);
                bw[2] = as_u(as_h2(perm(0u, t2[r], 0x0c010c00u) ^ 0x64806480u) - o);
                bw[3] = as_u(as_h2(perm(0u, t2[r], 0x0c030c02u) ^ 0x64806480u) - o);
            }
            b[r] = __builtin_bit_cast(half8, u32x4{bw[0], bw[1], bw[2], bw[3]});
        }
        // one accumulator per group: its runs' hi and lo products in run order
        f32x4 acc[NGC];
#pragma unroll
        for (int gi = 0; gi < NGC; ++gi) acc[gi] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            acc[r / RPG] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[r], b[r], acc[r / RPG], 0, 0, 0);
            acc[r / RPG] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[r], b[r], acc[r / RPG], 0, 0, 0);
        }
        // a chunk past the wave's range may have read tiles no phase wrote: its whole
        // contribution is dropped by a select, never scaled by zero (0 * NaN)
        float cy[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            cy[i] = y[i];
#pragma unroll
            for (int gi = 0; gi < NGC; ++gi) cy[i] = fmaf(sc[gi], acc[gi][i], cy[i]);
            y[i] = live ? cy[i] : y[i];
        }
    };
    // The ring over each phase's chunks (refills cross the loop's back edge, as in the
    // one-row kernel; cpp is a multiple of R, so the ring's slots line up with phases).
    for (int32_t ph = 0; ph < phases; ++ph) {
        if (ph > 0) {
            __syncthreads();  // every wave is done with the previous phase's tiles
            for (int32_t rd = 0; rd < rounds; ++rd) {
                load_round(ph, rd);
                store_round(rd);
            }
            __syncthreads();
        }
        const int32_t c_end = min((ph + 1) * cpp, nmax);
#pragma nounroll
        for (int32_t c0 = ph * cpp; c0 < c_end; c0 += R) {
            static_for<0, R>([&](auto si) {
                constexpr int sl = decltype(si)::value;
                uint32_t t[4], t2[4];
                take(sl, t, t2);
                issue(sl, c0 + sl + R);  // the slot refills before its chunk is computed
                process(t, t2, c0 + sl, c0 + sl < n, ph);
                __builtin_amdgcn_sched_barrier(0);
            });
        }
    }

    // ---- the last sub-parts; the K-parts of each column set (the tree's top); the row
    // shifts; the stores
    while (sp < sp_count) close_sub_part();
    float* red = reinterpret_cast<float*>(smem + rows_lds_red(ks, cpp, MT, rows));  // [W][16 rows][16 cols]
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(wave * 16 + 4 * kb + i) * 16 + nl] = part[i];
    __syncthreads();
    if (kp != 0 || !set_live) return;
    const int32_t cs = 1 << cslog;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int32_t m = 4 * kb + i;
        if (m >= M) continue;
        const float sum = tree_top(red + (my_cs * 16 + m) * 16 + nl, cs * 256, kslog);
        float* dst = out + static_cast<size_t>(m) * N + col;
        float o = accumulate ? *dst : 0.0f;
        const int32_t sh[4] = {rsh.x, rsh.y, rsh.z, rsh.w};
        o = fmaf(alpha, ldexpf(sum, -sh[i]), o);
        if (bias) o += bias[col];
        *dst = o;
    }
}

}  // namespace

// The launch: the one-row kernel's K split (plan_packed), or the largest smaller one
// whose x tiles fit (the result does not depend on the split); the x tiles a phase holds
// (chunks per phase: a multiple of R, the wave's range rounded up to R when all of it
// fits in what LDS the staged rows and the meeting area leave); the LDS. ks = 0: none fits.
struct RowsPlan {
    int32_t ks = 0, cpp = 0;
    size_t lds = 0;
};
// Rows of the x tiles for M rows: 4, 8 or 16.
static int32_t tile_rows(int32_t M) { return M <= 4 ? 4 : M <= 8 ? 8 : 16; }

static RowsPlan rows_plan(int32_t M, int32_t K, int32_t g, int32_t sets) {
    RowsPlan r;
    const PackedPlan plan = plan_packed(K, g, sets);
    const int32_t gshift = log2_exact(g / RUN), chunks = ceil_div(K, CHUNK);
    M = tile_rows(M);
    const int32_t tile = run_tile_bytes(M);
    for (int32_t ks = plan.ks; ks >= 1; ks /= 2) {
        const int32_t nmax = ceil_div(chunks, ks);
        if (nmax > MAX_WAVE_CHUNKS) break;
        const int32_t rows = stage_rows(nmax, gshift);
        const int32_t fixed = rows_lds_bytes(ks, 0, M, rows);
        if (fixed >= static_cast<int32_t>(LDS_MAX)) continue;
        int32_t cpp = (static_cast<int32_t>(LDS_MAX) - fixed) / (ks * 4 * tile);
        cpp = std::min(cpp, (nmax + R - 1) / R * R) / R * R;
        if (cpp < R) continue;
        r.ks = ks;
        r.cpp = cpp;
        r.lds = static_cast<size_t>(rows_lds_bytes(ks, cpp, M, rows));
        return r;
    }
    return r;
}

// The automatic choice: wide weights only. With column sets at least 16 times the 128-k
// chunks (the 8B gate/up, the heads) this kernel is well ahead of the row-block kernel;
// for narrow ones (8192 -> 2048, 14336 -> 4096, 4096 -> 4096) its grid is small and its x
// tiles take several phases, and the row-block kernel is faster (measured at M = 2..16).
bool gemv_rows_packed_preferred(const WeightView& w) { return w.N / SET >= 16 * ceil_div(w.K, CHUNK); }

bool gemv_rows_packed_supported(const float* a, int32_t m, const WeightView& w, const float* c) {
    if (m < 2 || m > MAX_ROWS || !w.p) return false;
    if (w.K % RUN != 0 || w.K > 16384) return false;
    if (static_cast<int64_t>(w.K / RUN) * run_tile_bytes(m) > INT32_MAX) return false;
    if (w.g % RUN != 0 || log2_exact(w.g / RUN) < 0) return false;
    if (w.N % SET != 0) return false;
    if (static_cast<int64_t>(w.G) * w.N * 4 > INT32_MAX) return false;
    if (!aligned(w.p, 16) || !aligned(a, 16) || !aligned(c, 4)) return false;
    return rows_plan(m, w.K, w.g, w.N / SET).ks != 0;
}

template <int GS, int MT>
static int32_t launch_rows(int32_t bits, bool zp, dim3 grid, size_t lds, hipStream_t st, const uint8_t* p,
                           const _Float16* at, const int32_t* sh, int32_t m, int32_t N, int32_t K, int32_t shifts,
                           int32_t cpp, float alpha, float* c, int32_t accumulate, const float* bias) {
    if (bits == 4) {
        if (const int32_t ls = allow_lds<&gemv_rows_packed_kernel<4, true, GS, MT>>(lds)) return ls;
        gemv_rows_packed_kernel<4, true, GS, MT>
            <<<grid, 64 * W, lds, st>>>(p, at, sh, m, N, K, shifts, cpp, alpha, c, accumulate, bias);
    } else if (zp) {
        if (const int32_t ls = allow_lds<&gemv_rows_packed_kernel<8, true, GS, MT>>(lds)) return ls;
        gemv_rows_packed_kernel<8, true, GS, MT>
            <<<grid, 64 * W, lds, st>>>(p, at, sh, m, N, K, shifts, cpp, alpha, c, accumulate, bias);
    } else {
        if (const int32_t ls = allow_lds<&gemv_rows_packed_kernel<8, false, GS, MT>>(lds)) return ls;
        gemv_rows_packed_kernel<8, false, GS, MT>
            <<<grid, 64 * W, lds, st>>>(p, at, sh, m, N, K, shifts, cpp, alpha, c, accumulate, bias);
    }
    return KT_OK;
}

template <int MT>
static int32_t launch_rows_g(int32_t gshift, int32_t bits, bool zp, dim3 grid, size_t lds, hipStream_t st,
                             const uint8_t* p, const _Float16* at, const int32_t* sh, int32_t m, int32_t N, int32_t K,
                             int32_t shifts, int32_t cpp, float alpha, float* c, int32_t accumulate, const float* bias) {
    if (gshift == 0)
        return launch_rows<0, MT>(bits, zp, grid, lds, st, p, at, sh, m, N, K, shifts, cpp, alpha, c, accumulate, bias);
    if (gshift == 1)
        return launch_rows<1, MT>(bits, zp, grid, lds, st, p, at, sh, m, N, K, shifts, cpp, alpha, c, accumulate, bias);
    return launch_rows<2, MT>(bits, zp, grid, lds, st, p, at, sh, m, N, K, shifts, cpp, alpha, c, accumulate, bias);
}

int32_t launch_gemv_rows_packed(const float* a, int32_t m, const WeightView* ws, float* const* cs,
                                const float* const* biases, int32_t count, int32_t accumulate, float alpha,
                                hipStream_t st) {
    // one preparation of x for every weight of the call (same K, bits)
    const WeightView& w0 = ws[0];
    const int32_t mt = tile_rows(m);
    void* general = nullptr;
    const size_t tiles = static_cast<size_t>(w0.K / RUN) * run_tile_bytes(mt);
    if (const int32_t status = workspace(st, tiles + 64 + 256, &general)) return status;
    char* base = reinterpret_cast<char*>((reinterpret_cast<uintptr_t>(general) + 255) & ~uintptr_t{255});
    _Float16* at = reinterpret_cast<_Float16*>(base);
    int32_t* sh = reinterpret_cast<int32_t*>(base + tiles);
    if (w0.bits == 4)
        rows_prep_kernel<4><<<mt, PREP_THREADS, 0, st>>>(a, m, mt, w0.K, at, sh);
    else
        rows_prep_kernel<8><<<mt, PREP_THREADS, 0, st>>>(a, m, mt, w0.K, at, sh);
    KT_LAUNCHED("qmatmul: rows prep kernel");
    for (int32_t i = 0; i < count; ++i) {
        const WeightView& w = ws[i];
        const RowsPlan plan = rows_plan(m, w.K, w.g, w.N / SET);
        const int32_t gshift = log2_exact(w.g / RUN);
        if (!plan.ks) return fail(KT_ERR_ARGUMENT, "packed rows gemv: no work split fits K = %d, M = %d", w.K, m);
        const int32_t kslog = log2_exact(plan.ks);
        const dim3 grid(static_cast<uint32_t>(ceil_div(w.N / SET, W / plan.ks)));
        const int32_t shifts = kslog | gshift << 4;
        const float* bias = biases ? biases[i] : nullptr;
        int32_t status;
        if (mt == 4)
            status = launch_rows_g<4>(gshift, w.bits, w.z != nullptr, grid, plan.lds, st, w.p, at, sh, m, w.N, w.K,
                                      shifts, plan.cpp, alpha, cs[i], accumulate, bias);
        else if (mt == 8)
            status = launch_rows_g<8>(gshift, w.bits, w.z != nullptr, grid, plan.lds, st, w.p, at, sh, m, w.N, w.K,
                                      shifts, plan.cpp, alpha, cs[i], accumulate, bias);
        else
            status = launch_rows_g<16>(gshift, w.bits, w.z != nullptr, grid, plan.lds, st, w.p, at, sh, m, w.N, w.K,
                                       shifts, plan.cpp, alpha, cs[i], accumulate, bias);
        if (status) return status;
        KT_LAUNCHED("qmatmul: packed rows gemv kernel");
    }
    return KT_OK;
}

}  // namespace kt
