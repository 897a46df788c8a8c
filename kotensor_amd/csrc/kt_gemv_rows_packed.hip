// kt_gemv_rows_packed.hip -- 2 to 16 rows on the column-run copy:
//   c[M x N] = (accumulate ? c : 0) + alpha * x[M x K] . deq(W) (+ bias),
// MatMul.multiplyQuantized's M > 1 branch (Engine/kotensor/src/main/kotlin/MatMul.kt:479-485,
// computeQuantizedTile :830-881) for the few-row products of batched or speculative decode.
//
// The weights stream exactly as in the one-row kernel (kt_gemv_packed.hip): a workgroup of
// eight waves owns 8 / ks column sets over ks K-parts, each wave streams its set's 1 KB
// (INT8 2 KB) chunks with four in flight (non-temporal loads) and reads its scales and
// zero points from rows staged in LDS; so a call moves the weight bytes once, whatever M.
// One launch per weight: x is converted inside every workgroup.
//
// Arithmetic (exact products, fp32 sums, the reference's per-group combine):
//   * x: each row's 128-k chunk gets its own power of two, 2^s (its largest |x| into
//     [2^14, 2^15)), and x 2^s splits into two fp16 parts, hi = fp16(x 2^s) and
//     lo = fp16(x 2^s - hi): 22 significant bits. The parts of up to eight rows make the
//     16 rows of one MFMA A tile (rows 0..7 hi, 8..15 lo; four rows: 0..3 and 4..7), so one
//     MFMA per 32 k covers both parts; sixteen rows take an A tile per part, two MFMAs per
//     run into one accumulator. The workgroup converts the chunks of its K range into LDS
//     once for all its waves, or (sixteen rows, or more workgroups than CUs) copies them
//     from one conversion launch before the product;
//   * weights: the exact integers q - z as fp16 (the bits of 1024 + q from the nibble or
//     byte, minus 1024 + z in one packed fp16 add). The chunk's 16-byte lane pieces hold
//     one run each (lane group kb: run kb, dword j its 8-k slice j); each MFMA takes 8 k
//     per lane group of one quantization group only: g = 32 transposes the pieces with four
//     lane swaps (v_permlane32_swap, v_permlane16_swap: MFMA m = run m), g = 64 swaps halves
//     with two (MFMA m = two slices of each of the group's two runs), g >= 128 takes them as
//     they lie (MFMA m = slice m of every run); the A tiles hold x in the same places. INT4
//     takes the nibbles as they lie (low nibbles of bytes 0 and 2, high nibbles of 0 and 2,
//     then bytes 1 and 3 after a shift), so the A tiles hold x in that order: k 0, 2, 4, 6,
//     1, 3, 5, 7 of the eight;
//   * v_mfma_f32_16x16x32_f16, four per chunk and A tile into one accumulator per group:
//     every product is exact in fp32 (11-bit x part times an integer of at most 9 bits);
//     INT4 high nibbles enter as 16 (q - z), so x's parts at those positions carry 2^(s-4).
//     Lane (kb, n) gets A rows 4 kb .. 4 kb + 3 of column n, and per chunk
//     y += 2^-s (sum over the chunk's groups of scale(group, n) * D) (combineGroup,
//     MatMul.kt:804-828, per group and chunk);
//   * K's sub-parts (kt_packed.h) are summed alone and added in a fixed tree, whatever the
//     K split; with the parts in the rows, a row's result is its hi sum plus its lo sum.
// A row's result therefore differs from the one-row kernel's only by the rounding of x to
// 22 bits and the order of fp32 sums (normwise near 1e-7 against the oracle), and does
// not depend on the other rows of the call (QuantizationTest.kt:110-134 asks 1e-4): its
// bits are the same for every call of 2..8 rows, and for every call of 9..16 rows.
// The x tiles live in LDS for the whole K range a workgroup covers when they fit, else in
// phases: at a phase change the workgroup meets at a barrier and converts the next ones
// (their loads then queue behind the weight loads in flight).
#include "kt_common.h"
#include "kt_packed.h"

#include <algorithm>

namespace kt {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));

constexpr int W = 8;  // waves per workgroup
constexpr int R = 4;  // chunks in flight per wave (eight measured slower at 2..16 rows)
constexpr int MAX_ROWS = 16;
constexpr int MAX_PASSES = 8;  // x conversion tasks a wave takes per phase

// Two arrangements of x's parts. Up to eight rows: both parts in the rows of one A tile
// (rows 0..7 hi, 8..15 lo; four rows: 0..3 and 4..7), one MFMA per 32 k. Sixteen rows: an
// A tile per part, [part][lane group kb][row][8 halves], both MFMAs into one accumulator
// (half the values per lane to combine that two tiles of eight rows would hold).
__host__ __device__ constexpr bool parts_in_k(int32_t MT) { return MT == 16; }
// x rows per A tile.
__host__ __device__ constexpr int32_t tile_x_rows(int32_t MT) { return MT < 8 ? MT : MT == 8 ? 8 : 16; }
// Bytes of x tiles per run: MT rows x two parts x 32 k x 2 bytes; with the parts in the
// rows, per A tile [lane group kb][A row, swizzled][8 halves].
__host__ __device__ constexpr int32_t run_tile_bytes(int32_t MT) { return 2 * 4 * 16 * MT; }
// The 16-byte slot of (lane group kb, A row a) in an A tile of HR x rows: a ^ 4 kb (HR = 4:
// a ^ 4 (kb / 2)), so that the conversion's stores (lanes: four rows x the four lane
// groups) meet 16 different bank groups, as the MFMA's reads (lanes: the A rows of one lane
// group) do without it.
template <int HR>
__device__ __forceinline__ int32_t a_slot(int32_t kb, int32_t a) {
    return kb * (2 * HR) + (a ^ (HR == 8 ? 4 * kb : 4 * (kb >> 1)));
}

// The workgroup's LDS: the x tiles of one phase [ks][cpp chunks][4 runs][tile]; the
// chunks' factors 2^-s [ks][cpp][MT] floats; each wave's staged scale and zero-point rows.
// At the end the meeting area [W][A tiles][16 A rows][16 columns] floats takes the tiles'
// place (it is never larger).
__host__ __device__ constexpr int32_t rows_lds_p(int32_t ks, int32_t cpp, int32_t MT) {
    return ks * cpp * 4 * run_tile_bytes(MT);
}
__host__ __device__ constexpr int32_t rows_lds_stage(int32_t ks, int32_t cpp, int32_t MT) {
    return rows_lds_p(ks, cpp, MT) + ks * cpp * MT * 4;
}
__host__ __device__ constexpr int32_t rows_lds_bytes(int32_t ks, int32_t cpp, int32_t MT, int32_t rows) {
    return rows_lds_stage(ks, cpp, MT) + W * rows * STAGE_ROW_BYTES;
}

__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_perm(hi, lo, sel);
}
__device__ __forceinline__ half2v as_h2(uint32_t v) { return __builtin_bit_cast(half2v, v); }
__device__ __forceinline__ uint32_t as_u(half2v v) { return __builtin_bit_cast(uint32_t, v); }
// a b + c for a, b < 2^24 in one instruction
__device__ __forceinline__ uint32_t mad24(uint32_t a, uint32_t b, uint32_t c) {
    return __umul24(a, b) + c;  // (v_mad_u32_u24)
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

// A chunk's weights as the MFMAs take them: on exit v[m] feeds MFMA m, which must not mix
// quantization groups. On entry lane group r holds run r, v[j] its 8-k slice j. g = 32 (a
// group per run): the full transpose, MFMA m = run m, lane group kb its slice kb. g = 64:
// only the halves swap, MFMA m = runs 2 (m / 2) and 2 (m / 2) + 1 (one group), lane group kb
// run 2 (m / 2) + kb % 2, slice 2 (kb / 2) + m % 2. g >= 128 (one group per chunk): as they
// lie, MFMA m = slice m, lane group kb run kb.
template <int GS>
__device__ __forceinline__ void arrange(uint32_t (&v)[4]) {
    if constexpr (GS == 0) {
        transpose4(v);
    } else if constexpr (GS == 1) {
        auto a = __builtin_amdgcn_permlane32_swap(v[0], v[2], false, false);
        auto b = __builtin_amdgcn_permlane32_swap(v[1], v[3], false, false);
        v[0] = a[0];
        v[1] = b[0];
        v[2] = a[1];
        v[3] = b[1];
    }
}
// The run and the 8-k slice that MFMA m's lane group kb takes after arrange<GS>: what x's
// A tile m holds for lane group kb.
template <int GS>
__device__ __forceinline__ int32_t run_of(int32_t m, int32_t kb) {
    return GS == 0 ? m : GS == 1 ? 2 * (m >> 1) + (kb & 1) : kb;
}
template <int GS>
__device__ __forceinline__ int32_t slice_of(int32_t m, int32_t kb) {
    return GS == 0 ? kb : GS == 1 ? 2 * (kb >> 1) + (m & 1) : m;
}

// hi and lo fp16 parts of two floats (RNE; the differences are exact in fp32)
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
    const half2v h = __builtin_convertvector(f32x2{a, b}, half2v);
    const half2v l = __builtin_convertvector(f32x2{a - static_cast<float>(h[0]), b - static_cast<float>(h[1])}, half2v);
    hi = as_u(h);
    lo = as_u(l);
}

// x conversion, a task at a time: a task is four rows' one chunk, a wave's lane (row
// 4 q + (ln & 3); the run and 8-k slice that A tile ln / 16 holds for lane group
// (ln / 4) % 4) holding its 8 floats (zeros past M and K). Returns 2^-s of the lane's row and chunk and its hi and lo parts in the A order:
// INT4 k 0, 2, 4, 6, 1, 3, 5, 7 of the eight (4..7 meet high nibbles: 2^(s - 4)), INT8
// k 0..7.
template <int BITS>
__device__ __forceinline__ float convert_task(const float4& a, const float4& b, uint32_t (&hw)[4], uint32_t (&lw)[4]) {
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    float mx = fabsf(v[0]);
#pragma unroll
    for (int e = 1; e < 8; ++e) mx = fmaxf(mx, fabsf(v[e]));
    mx = rows4_max(row_stride4_max(mx));  // the row's 16 slices of the chunk
    // largest |x| into [2^14, 2^15); a zero or non-finite chunk is not scaled (non-finite
    // values then make non-finite outputs, as the reference's sums do); at most 2^126, so
    // that 2^-s stays a normal float
    const bool finite = mx <= 3.402823466e38f;
    const int32_t s = finite && mx > 0.0f ? min(15 - __builtin_amdgcn_frexp_expf(mx), 126) : 0;
    constexpr int ORD4[8] = {0, 2, 4, 6, 1, 3, 5, 7};
#pragma unroll
    for (int pr = 0; pr < 4; ++pr) {
        const int e0 = BITS == 4 ? ORD4[2 * pr] : 2 * pr, e1 = BITS == 4 ? ORD4[2 * pr + 1] : 2 * pr + 1;
        split2(ldexpf(v[e0], BITS == 4 && e0 >= 4 ? s - 4 : s), ldexpf(v[e1], BITS == 4 && e1 >= 4 ? s - 4 : s), hw[pr],
               lw[pr]);
    }
    return ldexpf(1.0f, -s);
}
// Byte offset of x row `row`'s part (0 hi, 1 lo) for lane group kb in a run's tiles.
template <int MT>
__device__ __forceinline__ int32_t tile_offset(int32_t row, int32_t kb, int32_t part) {
    constexpr int HR = tile_x_rows(MT);
    if constexpr (parts_in_k(MT)) return part * 1024 + (kb * 16 + row) * 16;
    return (row / HR) * (128 * HR) + a_slot<HR>(kb, part * HR + row % HR) * 16;
}

// x [M x K] -> the A tiles of every chunk [chunks][4 runs][tile], then their factors 2^-s
// [chunks][MT] floats: a task per wave, once per call, for the products that copy tiles
// instead of converting x themselves. Quads past M are not written (their A rows reach only
// output rows that are never stored).
template <int BITS, int MT, int GS>
__global__ void __launch_bounds__(64 * W)
    rows_prep_kernel(const float* __restrict__ x, int32_t M, int32_t K, unsigned char* __restrict__ xt) {
    constexpr int32_t tile = run_tile_bytes(MT);
    const int32_t chunks = (K + CHUNK - 1) >> 7, ln = threadIdx.x & 63;
    const int32_t j = blockIdx.x * W + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (j >= ((M + 3) >> 2) * chunks) return;
    const int32_t quad = j / chunks, c = j - quad * chunks;
    // lane: x row ln % 4 of the quad for A tile ln / 16, lane group (ln / 4) % 4
    const int32_t xrow = ln & 3, xkb = (ln >> 2) & 3, xm = ln >> 4;
    const int32_t row = 4 * quad + xrow, k = c * CHUNK + run_of<GS>(xm, xkb) * RUN + slice_of<GS>(xm, xkb) * 8;
    const int32_t xoob = M * K * 4;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(x), 0, xoob, 0x00020000);
    const int32_t off = row < M && k < K ? (row * K + k) * 4 : xoob;
    const float4 a = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
    const float4 b = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 16, 0));
    uint32_t hw[4], lw[4];
    const float f = convert_task<BITS>(a, b, hw, lw);
    unsigned char* d = xt + static_cast<size_t>(c * 4 + xm) * tile;
    *reinterpret_cast<u32x4*>(d + tile_offset<MT>(row, xkb, 0)) = u32x4{hw[0], hw[1], hw[2], hw[3]};
    *reinterpret_cast<u32x4*>(d + tile_offset<MT>(row, xkb, 1)) = u32x4{lw[0], lw[1], lw[2], lw[3]};
    if ((ln >> 2) == 0) reinterpret_cast<float*>(xt + static_cast<size_t>(chunks) * 4 * tile)[c * MT + row] = f;
}

// GS: the group size's class (0: g = 32, a group per run; 1: g = 64, a group per two
// runs; 2: g >= 128, one group per chunk), MT: rows of the x tiles (4, 8 or 16; rows
// M .. MT - 1 reach only output rows that are never stored). COPY: x is rows_prep_kernel's
// output, which the workgroup copies; otherwise the workgroup converts x itself.
// SPLIT: the ks K-parts of a column set are workgroups (blockIdx.y), each of eight column
// sets over one K-part, so a workgroup converts only its part of x; every wave writes its
// subtree of sums to `partials` (write-through), the workgroup counts itself in at
// counters[blockIdx.x], and the last of the ks workgroups adds the parts in the tree's
// fixed order: the same bits as the parts meeting inside one workgroup.
template <int BITS, bool ZP, int GS, int MT, bool COPY, bool SPLIT>
__global__ void __launch_bounds__(64 * W)
    gemv_rows_packed_kernel(const uint8_t* __restrict__ packed, const float* __restrict__ x, int32_t M, int32_t N,
                            int32_t K, int32_t shifts, float alpha, float* out, int32_t accumulate, const float* bias,
                            float* partials, uint32_t* counters) {
    static_assert(!(SPLIT && COPY), "split workgroups convert their own part of x");
    constexpr int BB = block_bytes(BITS);
    constexpr int NB = BITS == 4 ? 1 : 2;  // 16-byte loads per lane and chunk
    constexpr bool PK = parts_in_k(MT);
    // x rows per A tile, A tiles of x rows, A rows used, A operands per run
    constexpr int HR = tile_x_rows(MT), NT = MT / HR, AR = PK ? 16 : 2 * HR, NA = PK ? 2 : NT;
    constexpr int32_t tile = run_tile_bytes(MT);
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
    const int32_t kslog = shifts & 15, gshift = (shifts >> 4) & 15, cpplog = shifts >> 8;
    const int32_t ks = 1 << kslog, cpp = 1 << cpplog;
    const int32_t kinlog = SPLIT ? 0 : kslog, kin = 1 << kinlog;  // K-parts inside the workgroup
    const int32_t sets = N >> 4, chunks = (K + CHUNK - 1) >> 7, G = (K + (RUN << gshift) - 1) >> (gshift + 5);
    const int32_t tid = threadIdx.x, ln = tid & 63;
    const int32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int32_t cslog = 3 - kinlog;
    const int32_t set0 = blockIdx.x << cslog;
    if (set0 >= sets) return;  // (split: never, the grid's column-set groups all hold a set)
    const int32_t my_cs = wave & ((1 << cslog) - 1), kp = SPLIT ? static_cast<int32_t>(blockIdx.y) : wave >> cslog;
    const int32_t kpl = SPLIT ? 0 : kp;  // the K-part's place in the workgroup's tiles
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

    // ---- x into the phase's tiles. Converting: task j of a phase is quad j / (kin cpp),
    // phase chunk j % (kin cpp) (powers of two: shifts and masks), MAX_PASSES tasks per
    // wave at most. Copying: 16-byte pieces of the prep's tiles and factors, each part's
    // chunks of the phase contiguous there and here.
    const int32_t ppr = kin * cpp;              // a phase's chunks over the workgroup's K-parts
    const int32_t tasks = ((M + 3) >> 2) * ppr;  // quads past M are not converted
    // lane: x row ln % 4 of the task's quad for A tile ln / 16, lane group (ln / 4) % 4
    const int32_t xrow = ln & 3, xkb = (ln >> 2) & 3, xm = ln >> 4;
    const int32_t xk = run_of<GS>(xm, xkb) * RUN + slice_of<GS>(xm, xkb) * 8;  // its k in the chunk
    const int32_t xoob = COPY ? chunks * (4 * tile + MT * 4) : M * K * 4;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(x), 0, xoob, 0x00020000);
    float4 xv[MAX_PASSES][2];
    // the task's quad and phase chunk (wave-uniform), and the lane's byte offset in x
    // (rows past M, runs past K and chunks past the part read zeros without memory traffic)
    auto task_of = [&](int32_t j, int32_t ph, int32_t& quad, int32_t& ch) -> int32_t {
        quad = j >> (kinlog + cpplog);
        ch = j & (ppr - 1);
        const int32_t part = (SPLIT ? kp : 0) + (ch >> cpplog);
        const int32_t c = ph * cpp + (ch & (cpp - 1));
        const int32_t cg = ((part * chunks) >> kslog) + c;
        const int32_t ce = ((part + 1) * chunks) >> kslog;
        const int32_t row = 4 * quad + xrow, k = cg * CHUNK + xk;
        return cg < ce && row < M && k < K ? (row * K + k) * 4 : xoob;
    };
    // copy pieces: a part's phase is 2^(cpplog + 5 + log2 MT) pieces of tiles (32 MT per
    // chunk); the factors ks cpp MT / 4 pieces (MT / 4 per chunk)
    constexpr int MTLOG = MT == 4 ? 2 : MT == 8 ? 3 : 4;
    const int32_t tile_pieces = kin << (cpplog + 5 + MTLOG);
    auto piece_off = [&](int32_t q, int32_t ph) -> int32_t {  // the prep's byte offset of tile piece q, or xoob
        const int32_t part = q >> (cpplog + 5 + MTLOG), within = q & ((1 << (cpplog + 5 + MTLOG)) - 1);
        const int32_t cg = ((part * chunks) >> kslog) + ph * cpp + (within >> (5 + MTLOG));
        return cg < (((part + 1) * chunks) >> kslog) ? (cg << (5 + MTLOG)) * 16 + (within & ((32 << MTLOG) - 1)) * 16
                                                     : xoob;
    };
    // factor piece q (at most 128 of them: one per thread, with the first round)
    const int32_t factor_pieces = kin << (cpplog + MTLOG - 2);
    auto factor_off = [&](int32_t q, int32_t ph) -> int32_t {
        const int32_t part = q >> (cpplog + MTLOG - 2), within = q & ((1 << (cpplog + MTLOG - 2)) - 1);
        const int32_t cg = ((part * chunks) >> kslog) + ph * cpp + (within >> (MTLOG - 2));
        return cg < (((part + 1) * chunks) >> kslog)
                   ? chunks * 4 * tile + (cg * MT + (within & ((MT >> 2) - 1)) * 4) * 4
                   : xoob;
    };
    const int32_t copy_rounds = (tile_pieces + 2 * 64 * W * MAX_PASSES - 1) / (2 * 64 * W * MAX_PASSES);
    float4 fv;
    // passes i0 .. i1 - 1 of round rd (the factors go with the round's first passes)
    auto load_x = [&](int32_t ph, int32_t rd, int i0, int i1) {
        if constexpr (COPY)
            if (rd == 0 && i0 == 0 && tid < factor_pieces)
                fv = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, factor_off(tid, ph), 0, 0));
#pragma unroll
        for (int i = 0; i < MAX_PASSES; ++i) {
            if (i < i0 || i >= i1) continue;
            if constexpr (COPY) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int32_t q = tid + 64 * W * (2 * MAX_PASSES * rd + 2 * i + h);
                    if (q < tile_pieces)
                        xv[i][h] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, piece_off(q, ph), 0, 0));
                }
            } else {
                const int32_t j = i * W + wave;
                if (j < tasks) {
                    int32_t quad, ch;
                    const int32_t off = task_of(j, ph, quad, ch);
                    xv[i][0] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 0, 0));
                    xv[i][1] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, off, 16, 0));
                }
            }
        }
    };
    float* pl = reinterpret_cast<float*>(smem + rows_lds_p(kin, cpp, MT));  // [kin cpp][MT]: 2^-s
    auto store_x = [&](int32_t ph, int32_t rd) {
        if constexpr (COPY)
            if (rd == 0 && tid < factor_pieces) reinterpret_cast<float4*>(pl)[tid] = fv;
#pragma unroll
        for (int i = 0; i < MAX_PASSES; ++i) {
            if constexpr (COPY) {
                // the phase's tiles are contiguous in LDS as in the piece order
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int32_t q = tid + 64 * W * (2 * MAX_PASSES * rd + 2 * i + h);
                    if (q < tile_pieces) reinterpret_cast<float4*>(smem)[q] = xv[i][h];
                }
            } else {
                const int32_t j = i * W + wave;
                if (j >= tasks) break;
                int32_t quad, ch;
                task_of(j, ph, quad, ch);
                uint32_t hw[4], lw[4];
                const float f = convert_task<BITS>(xv[i][0], xv[i][1], hw, lw);
                const int32_t row = 4 * quad + xrow;  // < MT
                unsigned char* d = smem + (ch * 4 + xm) * tile;
                *reinterpret_cast<u32x4*>(d + tile_offset<MT>(row, xkb, 0)) = u32x4{hw[0], hw[1], hw[2], hw[3]};
                *reinterpret_cast<u32x4*>(d + tile_offset<MT>(row, xkb, 1)) = u32x4{lw[0], lw[1], lw[2], lw[3]};
                if ((ln >> 2) == 0) pl[ch * MT + row] = f;
            }
        }
    };
    const int32_t x_rounds = COPY ? copy_rounds : 1;

    // ---- loads, in the order they complete: the first half of the first phase's x, the
    // wave's scale and zero-point rows, two chunks of weights, the second half of x, two
    // more chunks. The first half converts while the weights are in flight; the second
    // waits for the first two chunks only (a wave's loads complete in issue order).
    // Measured at 4096 -> 14336 INT4, M = 2 / 8 / 16: x whole, then the weights 13.3 /
    // 16.9 / 22.5 us; this order 12.9 / 16.6 / 21.8; the weights first 13.8 / 17.9 / 22.7.
    load_x(0, 0, 0, MAX_PASSES / 2);
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
    u32x4 wb[R][NB], wb2[R][NB];
    auto issue_to = [&](u32x4 (&ring)[R][NB], int slot, int32_t cc) {
#pragma unroll
        for (int h = 0; h < NB; ++h)
            ring[slot][h] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        wr, cc * BB + h * 1024 + 16 * ln, 0, NONTEMPORAL));
    };
    auto issue = [&](int slot, int32_t cc) { issue_to(wb, slot, cc); };
#pragma unroll
    for (int s = 0; s < R / 2; ++s) issue(s, s);
    load_x(0, 0, MAX_PASSES / 2, MAX_PASSES);
#pragma unroll
    for (int s = R / 2; s < R; ++s) issue(s, s);

    // ---- into LDS: the first phase's x tiles, the wave's staged rows ----------------------
    store_x(0, 0);
    for (int32_t rd = 1; rd < x_rounds; ++rd) {  // a phase larger than one round of pieces
        load_x(0, rd, 0, MAX_PASSES);
        store_x(0, rd);
    }
    unsigned char* stg = smem + rows_lds_stage(kin, cpp, MT) + wave * rows * STAGE_ROW_BYTES;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (16 * i + (ln >> 2) < rows) *reinterpret_cast<u32x4*>(stg + i * 1024 + 16 * ln) = sst[i];
    if constexpr (ZP)
        if (ln < rows) *reinterpret_cast<u32x4*>(stg + rows * SET * 4 + 16 * ln) = zst;
    __syncthreads();

    // lanes of A rows past AR (four x rows) read A row AR - 1: an MFMA's output rows depend
    // only on their own A rows, and those are never stored
    const int32_t a_lane = PK ? (kb * 16 + nl) * 16 : a_slot<HR>(kb, min(nl, AR - 1)) * 16;
    const int32_t p_row = (4 * kb) % HR;  // the x row of the lane's first A row
    float y[NT][4] = {};
    // sub-parts of K, each summed alone and added in a balanced tree in K order (the
    // one-row kernel's scheme): the result does not depend on ks
    const int32_t sp_count = SUB_PARTS >> kslog, sp0 = kp * sp_count;
    int32_t sp = 0;
    int32_t sp_end = (((sp0 + 1) * chunks) >> SUB_LOG) - c_begin;
    float tree[NT][4][3] = {};
    float part[NT][4] = {};
    auto close_sub_part = [&]() {
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                part[tt][i] = tree_push(tree[tt][i], sp, y[tt][i]);
                y[tt][i] = 0.0f;
            }
        ++sp;
        sp_end = (((sp0 + sp + 1) * chunks) >> SUB_LOG) - c_begin;
    };
    const int32_t run0 = k0 >> 5;  // the wave's first run
    // the slot's weights as the MFMAs take them (arrange: t[m] feeds MFMA m; INT4 a slice's
    // 8 k, INT8 t[m] its first 4 k and t2[m] the next 4) -- taken out of the ring so the slot
    // refills at once
    // (the copies are forced: left to itself the compiler works on the ring's registers
    // and delays their refill until the chunk is converted, measured slower)
    auto take_from = [&](const u32x4 (&ring)[R][NB], int s, uint32_t (&t)[4], uint32_t (&t2)[4], bool copy) {
        if constexpr (BITS == 4) {
            t[0] = ring[s][0][0];
            t[1] = ring[s][0][1];
            t[2] = ring[s][0][2];
            t[3] = ring[s][0][3];
            if (copy)
#pragma unroll
                for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(t[i]));
            arrange<GS>(t);
        } else {
            // 8-byte pieces p = k 8p .. 8p + 7: dwords (2p, 2p + 1) of the lane's 32 bytes
            t[0] = ring[s][0][0];
            t[1] = ring[s][0][2];
            t[2] = ring[s][1][0];
            t[3] = ring[s][1][2];
            t2[0] = ring[s][0][1];
            t2[1] = ring[s][0][3];
            t2[2] = ring[s][1][1];
            t2[3] = ring[s][1][3];
            if (copy)
#pragma unroll
                for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(t[i]), "+v"(t2[i]));
            arrange<GS>(t);
            arrange<GS>(t2);
        }
    };
    auto take = [&](int s, uint32_t (&t)[4], uint32_t (&t2)[4]) { take_from(wb, s, t, t2, true); };
    constexpr int NGC = GS == 0 ? 4 : GS == 1 ? 2 : 1;  // quantization groups a chunk touches
    constexpr int RPG = 4 / NGC;                        // runs per group
    // the nibble masks and 1024's bits held in registers: with register operands the
    // compiler makes each (w & m) | o one v_and_or_b32 that it can schedule (literal
    // operands give two instructions; an inline-asm form cost hazard nops and SALU work)
    uint32_t k_lo = 0x000F000Fu, k_hi = 0x00F000F0u, k_or = 0x64006400u;
    asm volatile("" : "+v"(k_lo), "+v"(k_hi), "+v"(k_or));
    auto process = [&](const uint32_t (&t)[4], const uint32_t (&t2)[4], int32_t cl, bool live, int32_t ph) {
        if (live)
            while (cl >= sp_end) close_sub_part();
        // a chunk past the wave's range adds nothing; its reads stay in the phase's tiles
        // and the wave's staged rows (the phase's first chunk is below nmax)
        const int32_t cc = live ? cl : ph * cpp;
        const int32_t chl = kpl * cpp + (cc - ph * cpp);  // the chunk's place in the phase
        const unsigned char* tc = smem + chl * 4 * tile + a_lane;
        float sc[NGC];
        uint32_t zc[NGC];
        half8 a[NA][4];  // [A tile or part][run]
        f32x4 pf[NT];
        // the chunk's first group row; group gi is row gr + gi (the staged rows cover every
        // group of the wave's chunks, those past G, the padding of the last chunk, as zeros:
        // their x is zero, so they add nothing)
        const int32_t gr = ((run0 + cc * 4) >> gshift) - g0;
        const unsigned char* srow = stg + gr * (SET * 4) + nl * 4;
        const unsigned char* zrow = stg + rows * SET * 4 + gr * SET + nl;
#pragma unroll
        for (int gi = 0; gi < NGC; ++gi) {
            sc[gi] = *reinterpret_cast<const float*>(srow + gi * (SET * 4));
            zc[gi] = ZP ? zrow[gi * SET] : 0u;
        }
#pragma unroll
        for (int u = 0; u < NA; ++u)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                a[u][r] = *reinterpret_cast<const half8*>(tc + r * tile + u * (PK ? 1024 : 128 * HR));
#pragma unroll
        for (int tt = 0; tt < NT; ++tt) pf[tt] = *reinterpret_cast<const f32x4*>(pl + chl * MT + tt * HR + p_row);
        // the exact fp16 offsets of each group: 1024 + z (INT4 also 1024 + 16 z); INT8
        // 1152 + z (its bytes enter as 1152 + q)
        half2v ol[NGC], oh[NGC];
#pragma unroll
        for (int gi = 0; gi < NGC; ++gi) {
            // (z (2^16 + 1) + 0x64006400 in one 24-bit multiply-add: z <= 255 never carries
            // into the exponent bits)
            if constexpr (BITS == 4) {
                ol[gi] = as_h2(mad24(zc[gi], 0x00010001u, 0x64006400u));
                oh[gi] = as_h2(mad24(zc[gi], 0x00100010u, 0x64006400u));
            } else {
                ol[gi] = as_h2(mad24(zc[gi] ^ 0x80u, 0x00010001u, 0x64006400u));
                oh[gi] = ol[gi];
            }
        }
        half8 b[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            uint32_t bw[4];
            const half2v o_lo = ol[r / RPG], o_hi = oh[r / RPG];
            if constexpr (BITS == 4) {
                // halves: the bits of 1024 + q (low nibbles) or 1024 + 16 q (high nibbles),
                // minus 1024 + z or 1024 + 16 z: bytes 0 and 2, then 1 and 3
                const uint32_t w = t[r], w8 = t[r] >> 8;
                bw[0] = as_u(as_h2(((w & k_lo) | k_or)) - o_lo);   // k 0, 2
                bw[1] = as_u(as_h2(((w & k_hi) | k_or)) - o_hi);   // k 4, 6
                bw[2] = as_u(as_h2(((w8 & k_lo) | k_or)) - o_lo);  // k 1, 3
                bw[3] = as_u(as_h2(((w8 & k_hi) | k_or)) - o_hi);  // k 5, 7
            } else {
                // byte b (signed q): 0x64 above b ^ 0x80 is 1152 + q; minus 1152 + z
                const uint32_t u0 = t[r] ^ 0x80808080u, u1 = t2[r] ^ 0x80808080u;
                bw[0] = as_u(as_h2(perm(0x64646464u, u0, 0x04010400u)) - o_lo);
                bw[1] = as_u(as_h2(perm(0x64646464u, u0, 0x04030402u)) - o_lo);
                bw[2] = as_u(as_h2(perm(0x64646464u, u1, 0x04010400u)) - o_lo);
                bw[3] = as_u(as_h2(perm(0x64646464u, u1, 0x04030402u)) - o_lo);
            }
            b[r] = __builtin_bit_cast(half8, u32x4{bw[0], bw[1], bw[2], bw[3]});
        }
        // one accumulator per A tile and group: its runs' products in run order
        f32x4 acc[NT][NGC];
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
            for (int gi = 0; gi < NGC; ++gi) acc[tt][gi] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if constexpr (PK) {  // hi, then lo
                acc[0][r / RPG] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[0][r], b[r], acc[0][r / RPG], 0, 0, 0);
                acc[0][r / RPG] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[1][r], b[r], acc[0][r / RPG], 0, 0, 0);
            } else {
#pragma unroll
                for (int tt = 0; tt < NT; ++tt)
                    acc[tt][r / RPG] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[tt][r], b[r], acc[tt][r / RPG], 0, 0, 0);
            }
        }
        // a chunk past the wave's range may have read tiles no phase wrote: its whole
        // contribution is dropped by a select, never scaled by zero (0 * NaN)
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float cy = sc[0] * acc[tt][0][i];
#pragma unroll
                for (int gi = 1; gi < NGC; ++gi) cy = fmaf(sc[gi], acc[tt][gi][i], cy);
                const float yn = fmaf(pf[tt][i], cy, y[tt][i]);
                y[tt][i] = live ? yn : y[tt][i];
            }
    };
    // The ring over each phase's chunks (refills cross the loop's back edge, as in the
    // one-row kernel; cpp is a multiple of R, so the ring's slots line up with phases).
    bool two_sets = false;  // (not where x tiles are copied: their registers would spill)
    if constexpr (!COPY) two_sets = phases == 1 && nmax >= 4 * R;
    if (two_sets) {
        // one phase of at least 4 R chunks: two register sets, chunk c in set (c / R) % 2,
        // each refill going to the other set, so a chunk's registers are worked on in place
        // (no copies) while its refill is already in flight (8B FFN M = 8 14.4 -> 13.3 us;
        // with 8 chunks per wave, 4096 x 4096, it measured slower: 10.2 -> 10.9)
        const int32_t c_end = nmax, c_live = min(nmax, n);
        int32_t c0 = 0;
#pragma nounroll
        for (; c0 + 2 * R <= c_live; c0 += 2 * R) {
            static_for<0, 2 * R>([&](auto si) {
                constexpr int q = decltype(si)::value, sl = q % R;
                uint32_t t[4], t2[4];
                take_from(q < R ? wb : wb2, sl, t, t2, false);
                issue_to(q < R ? wb2 : wb, sl, c0 + q + R);
                process(t, t2, c0 + q, true, 0);
                __builtin_amdgcn_sched_barrier(0);
            });
        }
#pragma nounroll
        for (; c0 < c_end; c0 += 2 * R) {
            static_for<0, 2 * R>([&](auto si) {
                constexpr int q = decltype(si)::value, sl = q % R;
                uint32_t t[4], t2[4];
                take_from(q < R ? wb : wb2, sl, t, t2, false);
                issue_to(q < R ? wb2 : wb, sl, c0 + q + R);
                process(t, t2, c0 + q, c0 + q < n, 0);
                __builtin_amdgcn_sched_barrier(0);
            });
        }
    } else {
        for (int32_t ph = 0; ph < phases; ++ph) {
            if (ph > 0) {
                __syncthreads();  // every wave is done with the previous phase's tiles
                for (int32_t rd = 0; rd < x_rounds; ++rd) {
                    load_x(ph, rd, 0, MAX_PASSES);
                    store_x(ph, rd);
                }
                __syncthreads();
            }
            const int32_t c_end = min((ph + 1) * cpp, nmax);
            // groups of R chunks all below n first (no per-chunk select), then the rest
            const int32_t c_live = min(c_end, n);
            int32_t c0 = ph * cpp;
#pragma nounroll
            for (; c0 + R <= c_live; c0 += R) {
                static_for<0, R>([&](auto si) {
                    constexpr int sl = decltype(si)::value;
                    uint32_t t[4], t2[4];
                    take(sl, t, t2);
                    issue(sl, c0 + sl + R);  // the slot refills before its chunk is computed
                    process(t, t2, c0 + sl, true, ph);
                    __builtin_amdgcn_sched_barrier(0);
                });
            }
#pragma nounroll
            for (; c0 < c_end; c0 += R) {
                static_for<0, R>([&](auto si) {
                    constexpr int sl = decltype(si)::value;
                    uint32_t t[4], t2[4];
                    take(sl, t, t2);
                    issue(sl, c0 + sl + R);
                    process(t, t2, c0 + sl, c0 + sl < n, ph);
                    __builtin_amdgcn_sched_barrier(0);
                });
            }
        }
    }

    // ---- the last sub-parts; the K-parts of each column set (the tree's top), a row's
    // hi and lo sums; the stores. The meeting area takes the x tiles' place.
    while (sp < sp_count) close_sub_part();
    auto store_row = [&](int32_t m, float sum) {
        float* dst = out + static_cast<size_t>(m) * N + col;
        float o = accumulate ? *dst : 0.0f;
        o = fmaf(alpha, sum, o);
        if (bias) o += bias[col];
        *dst = o;
    };
    if constexpr (SPLIT) {
        // [K-part][column-set group][wave][NT][16 A rows][16 columns]: this wave's subtree,
        // written through the caches; once every wave's stores are complete the workgroup
        // counts itself in, and the last of the K-parts reads them all past the caches.
        const size_t stride = static_cast<size_t>(gridDim.x) * W * NT * 256;  // one K-part
        float* mine = partials + kp * stride + (static_cast<size_t>(blockIdx.x) * W + wave) * NT * 256 + nl;
#pragma unroll
        for (int tt = 0; tt < NT; ++tt)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                __hip_atomic_store(mine + (tt * 16 + 4 * kb + i) * 16, part[tt][i], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_SYSTEM);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();  // every wave's stores are in memory; the tiles are free
        uint32_t* flag = reinterpret_cast<uint32_t*>(smem);
        if (tid == 0) {
            const uint32_t before =
                __hip_atomic_fetch_add(counters + blockIdx.x, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const bool last = before == static_cast<uint32_t>(ks - 1);
            if (last) __hip_atomic_store(counters + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            *flag = last ? 1u : 0u;
        }
        __syncthreads();
        if (*flag == 0u || !set_live) return;
        const float* base = partials + (static_cast<size_t>(blockIdx.x) * W + wave) * NT * 256 + nl;
#pragma unroll
        for (int j = 0; j < MT / 4; ++j) {
            const int32_t m = 4 * j + kb;  // lane group kb stores rows kb, kb + 4, ...
            if (m >= M) continue;
            const int32_t ah = PK ? m : m % HR, al = HR + m % HR;  // the row's A rows (hi, lo)
            float vh[SUB_PARTS], vl[SUB_PARTS];
#pragma unroll
            for (int q = 0; q < SUB_PARTS; ++q) {
                vh[q] = vl[q] = 0.0f;
                if (q < ks) {
                    const float* pq = base + q * stride + (m / HR) * 256;
                    vh[q] = __hip_atomic_load(pq + ah * 16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                    if (!PK) vl[q] = __hip_atomic_load(pq + al * 16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                }
            }
            store_row(m, PK ? tree_top(vh, 1, kslog) : tree_top(vh, 1, kslog) + tree_top(vl, 1, kslog));
        }
        return;
    }
    __syncthreads();  // every wave is done with the tiles
    float* red = reinterpret_cast<float*>(smem);  // [W][NT][16 A rows][16 columns]
#pragma unroll
    for (int tt = 0; tt < NT; ++tt)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[((wave * NT + tt) * 16 + 4 * kb + i) * 16 + nl] = part[tt][i];
    __syncthreads();
    if (kp != 0 || !set_live) return;
    const int32_t cs = 1 << cslog;
#pragma unroll
    for (int j = 0; j < MT / 4; ++j) {
        const int32_t m = 4 * j + kb;  // lane group kb stores rows kb, kb + 4, ...
        if (m >= M) continue;
        const float* base = red + (my_cs * NT + m / HR) * 256 + nl;
        store_row(m, PK ? tree_top(base + m * 16, cs * NT * 256, kslog)
                        : tree_top(base + (m % HR) * 16, cs * NT * 256, kslog) +
                              tree_top(base + (HR + m % HR) * 16, cs * NT * 256, kslog));  // hi + lo
    }
}

}  // namespace

// The launch. Inside the workgroup (split = false): the one-row kernel's K split
// (plan_packed), or the largest smaller one whose x tiles fit. Across workgroups (split):
// the smallest power of two that keeps a wave's range within MAX_WAVE_CHUNKS, doubled up
// to SUB_PARTS while the workgroups (eight column sets each, one per K-part) number fewer
// than 4/5 of the CUs and every part keeps four chunks. The result does not depend on
// either. Then the x tiles a phase holds (chunks per phase: a power of two, at least R, at
// most what the waves convert in MAX_PASSES tasks each, no more than the wave's range
// needs, within what LDS the staged rows leave) and the LDS. ks = 0: none fits.
struct RowsPlan {
    int32_t ks = 0, cpp = 0;
    bool split = false;
    size_t lds = 0;
};
// Rows of the x tiles for M rows: 4, 8 or 16.
static int32_t tile_rows(int32_t M) { return M <= 4 ? 4 : M <= 8 ? 8 : 16; }

// The x tiles of one K-part per phase, for kin K-parts in the workgroup: false when none fits.
static bool rows_phase(int32_t M, int32_t chunks, int32_t gshift, int32_t ks, int32_t kin, RowsPlan& r) {
    const int32_t mt = tile_rows(M), quads = ceil_div(M, 4);
    const int32_t tile = run_tile_bytes(mt);
    const int32_t nmax = ceil_div(chunks, ks);
    if (nmax > MAX_WAVE_CHUNKS) return false;
    const int32_t rows = stage_rows(nmax, gshift);
    const int32_t fixed = rows_lds_bytes(kin, 0, mt, rows);
    if (fixed >= static_cast<int32_t>(LDS_MAX)) return false;
    int32_t cap = (static_cast<int32_t>(LDS_MAX) - fixed) / (kin * (4 * tile + mt * 4));
    cap = std::min(cap, W * MAX_PASSES / (quads * kin));
    int32_t cpp = R;
    while (cpp * 2 <= cap && cpp < nmax) cpp *= 2;
    if (cpp > cap) return false;
    r.ks = ks;
    r.cpp = cpp;
    r.lds = static_cast<size_t>(rows_lds_bytes(kin, cpp, mt, rows));
    return true;
}

static RowsPlan rows_plan(int32_t M, int32_t K, int32_t g, int32_t sets, bool split) {
    RowsPlan r;
    r.split = split;
    const int32_t gshift = log2_exact(g / RUN), chunks = ceil_div(K, CHUNK);
    if (split) {
        int32_t ks = 1;
        while (ks < SUB_PARTS && ceil_div(chunks, ks) > MAX_WAVE_CHUNKS) ks *= 2;
        const int64_t groups = ceil_div(sets, W);
        if (const int32_t f = packed_forced_ks()) {  // a forced split, where it covers K
            if (f < ks || f > chunks) return r;
            ks = f;
        } else {
            while (ks < SUB_PARTS && groups * ks * 5 < static_cast<int64_t>(cu_count()) * 4 && chunks >= 8 * ks)
                ks *= 2;
        }
        if (!rows_phase(M, chunks, gshift, ks, 1, r)) r.ks = 0;
        return r;
    }
    const PackedPlan plan = plan_packed(K, g, sets);
    for (int32_t ks = plan.ks; ks >= 1; ks /= 2) {
        if (ceil_div(chunks, ks) > MAX_WAVE_CHUNKS) break;
        if (rows_phase(M, chunks, gshift, ks, ks, r)) return r;
    }
    r.ks = 0;
    return r;
}

// How the K-parts meet: 0 automatic, 1 inside the workgroup, 2 across workgroups
// (kt_set_kernel_config's gemv_reduce).
static int32_t g_rows_reduce = 0;
void set_gemv_rows_packed_reduce(int32_t mode) { g_rows_reduce = mode; }
// Automatic: across workgroups from K = 4096 on (32 chunks), for the wide weights from 5
// rows on and for narrower ones of at least 256 column sets. A workgroup holding every
// K-part of its sets converts and reads all of x (M K floats: at M = 8 and K = 4096 as
// many bytes as its weights), and beyond K = 8192 its x tiles take several phases; split,
// each workgroup converts only its part, and the parts meet through memory, one more
// round trip. Measured (INT4 g64, us, M = 2 / 4 / 8 / 16): 14336 -> 4096 split 14.6 /
// 14.8 / 16.6 / 20.8, the row-block kernel 19.6 / 25.3 / 25.7 / 26.8; 4096 -> 14336
// split 13.5 / 13.8 / 15.4 / 18.8, inside 12.8 / 13.4 / 16.3 / 22.1; 4096 -> 4096 split
// 9.7 / - / 10.6 / 12.2, row-block 11.9 / - / 11.5 / 11.9; 8192 -> 2048 (128 sets) at
// M = 16 split 15.1, row-block 12.2.
static bool rows_wide(const WeightView& w) { return w.N / SET >= 16 * ceil_div(w.K, CHUNK); }
static bool rows_split_preferred(const WeightView& w, int32_t m) {
    if (ceil_div(w.K, CHUNK) < 32) return false;
    return rows_wide(w) ? m > 4 : w.N / SET >= 256;
}
static bool rows_split(const WeightView& w, int32_t m) {
    if (g_rows_reduce != 0) return g_rows_reduce == 2;
    return rows_split_preferred(w, m);
}

// The automatic choice: wide weights (column sets at least 16 times the 128-k chunks: the
// 8B gate/up, the heads), and the long-K weights of at least 256 column sets, which split
// across workgroups (14336 -> 4096, 4096 -> 4096). For the rest (fewer column sets,
// shorter K: 8192 -> 2048, 4864 -> 896) the row-block kernel is as fast or faster
// (measured at M = 2..16).
bool gemv_rows_packed_preferred(const WeightView& w) {
    return rows_wide(w) || (ceil_div(w.K, CHUNK) >= 32 && w.N / SET >= 256);
}

bool gemv_rows_packed_supported(const float* a, int32_t m, const WeightView& w, const float* c) {
    if (m < 2 || m > MAX_ROWS || !w.p) return false;
    if (w.K % RUN != 0 || w.K > 16384) return false;
    if (w.g % RUN != 0 || log2_exact(w.g / RUN) < 0) return false;
    if (w.N % SET != 0) return false;
    if (static_cast<int64_t>(w.G) * w.N * 4 > INT32_MAX) return false;
    if (!aligned(w.p, 16) || !aligned(a, 16) || !aligned(c, 4)) return false;
    return rows_plan(m, w.K, w.g, w.N / SET, rows_split(w, m)).ks != 0;
}

// What every launch of a call shares.
struct RowsLaunch {
    dim3 grid;
    size_t lds;
    hipStream_t st;
    const uint8_t* p;
    const float* a;
    int32_t m, N, K, shifts;
    float alpha;
    float* c;
    int32_t accumulate;
    const float* bias;
    float* partials;
    uint32_t* counters;
};

template <int BITS, bool ZP, int GS, int MT, bool COPY, bool SPLIT>
static int32_t launch_rows_kernel(const RowsLaunch& L) {
    if (const int32_t ls = allow_lds<&gemv_rows_packed_kernel<BITS, ZP, GS, MT, COPY, SPLIT>>(L.lds)) return ls;
    gemv_rows_packed_kernel<BITS, ZP, GS, MT, COPY, SPLIT><<<L.grid, 64 * W, L.lds, L.st>>>(
        L.p, L.a, L.m, L.N, L.K, L.shifts, L.alpha, L.c, L.accumulate, L.bias, L.partials, L.counters);
    return KT_OK;
}

template <int GS, int MT, bool COPY, bool SPLIT>
static int32_t launch_rows(int32_t bits, bool zp, const RowsLaunch& L) {
    if (bits == 4) return launch_rows_kernel<4, true, GS, MT, COPY, SPLIT>(L);
    if (zp) return launch_rows_kernel<8, true, GS, MT, COPY, SPLIT>(L);
    return launch_rows_kernel<8, false, GS, MT, COPY, SPLIT>(L);
}

template <int MT, bool COPY, bool SPLIT>
static int32_t launch_rows_g(int32_t gshift, int32_t bits, bool zp, const RowsLaunch& L) {
    if (gshift == 0) return launch_rows<0, MT, COPY, SPLIT>(bits, zp, L);
    if (gshift == 1) return launch_rows<1, MT, COPY, SPLIT>(bits, zp, L);
    return launch_rows<2, MT, COPY, SPLIT>(bits, zp, L);
}

// 16 rows copy prepared tiles unless the K-parts are split across workgroups (each then
// converts only its own part).
template <int MT>
static int32_t launch_rows_mt(bool copy, bool split, int32_t gshift, int32_t bits, bool zp, const RowsLaunch& L) {
    if (split) return launch_rows_g<MT, false, true>(gshift, bits, zp, L);
    if (MT == 16 || copy) return launch_rows_g<MT, true, false>(gshift, bits, zp, L);
    if constexpr (MT != 16) return launch_rows_g<MT, false, false>(gshift, bits, zp, L);
    return KT_OK;
}

// The group size's class: 0 g = 32, 1 g = 64, 2 g >= 128.
static int32_t gs_class(int32_t g) { return g == RUN ? 0 : g == 2 * RUN ? 1 : 2; }

template <int GS>
static void launch_rows_prep(int32_t bits, int32_t mt, uint32_t blocks, const float* a, int32_t m, int32_t K,
                             unsigned char* xt, hipStream_t st) {
    if (bits == 4) {
        if (mt == 4) rows_prep_kernel<4, 4, GS><<<blocks, 64 * W, 0, st>>>(a, m, K, xt);
        else if (mt == 8) rows_prep_kernel<4, 8, GS><<<blocks, 64 * W, 0, st>>>(a, m, K, xt);
        else rows_prep_kernel<4, 16, GS><<<blocks, 64 * W, 0, st>>>(a, m, K, xt);
    } else {
        if (mt == 4) rows_prep_kernel<8, 4, GS><<<blocks, 64 * W, 0, st>>>(a, m, K, xt);
        else if (mt == 8) rows_prep_kernel<8, 8, GS><<<blocks, 64 * W, 0, st>>>(a, m, K, xt);
        else rows_prep_kernel<8, 16, GS><<<blocks, 64 * W, 0, st>>>(a, m, K, xt);
    }
}

// Converting x in every workgroup saves the prep's launch; copying prepared tiles is
// cheaper for 16 rows (two phases of conversion per workgroup) and when the workgroups
// outnumber the CUs (the conversion repeats per round of workgroups).
int32_t launch_gemv_rows_packed(const float* a, int32_t m, const WeightView* ws, float* const* cs,
                                const float* const* biases, int32_t count, int32_t accumulate, float alpha,
                                hipStream_t st) {
    const WeightView& w0 = ws[0];
    const int32_t mt = tile_rows(m);
    bool split = true;  // every weight of the call meets its K-parts across workgroups
    for (int32_t i = 0; i < count; ++i) split = split && rows_split(ws[i], m);
    int64_t wgs = 0;
    size_t part_floats = 0;
    int64_t groups = 0;
    for (int32_t i = 0; i < count; ++i) {
        const RowsPlan plan = rows_plan(m, ws[i].K, ws[i].g, ws[i].N / SET, split);
        if (!plan.ks) continue;
        wgs = std::max<int64_t>(wgs, ceil_div(ws[i].N / SET, W / plan.ks));
        const int64_t gi = ceil_div(ws[i].N / SET, W);
        groups = std::max(groups, gi);
        part_floats = std::max(part_floats, static_cast<size_t>(plan.ks) * gi * W * 256);
    }
    const bool copy = !split && (mt == 16 || wgs > cu_count());
    float* partials = nullptr;
    uint32_t* counters = nullptr;
    if (split) {  // the K-parts' sums and one counter per column-set group (launches run in turn)
        void* general = nullptr;
        if (const int32_t status = workspace_counters(st, part_floats * sizeof(float), static_cast<size_t>(groups),
                                                      &general, &counters))
            return status;
        partials = static_cast<float*>(general);
    }
    // the x tiles are arranged as the weights' MFMAs take them, which depends on the group
    // size's class (arrange): copying, one preparation per class among the call's weights
    const float* srcs[3] = {a, a, a};
    if (copy) {
        const int32_t chunks = ceil_div(w0.K, CHUNK);
        const size_t bytes = (static_cast<size_t>(chunks) * (4 * run_tile_bytes(mt) + mt * 4) + 255) & ~size_t{255};
        bool used[3] = {false, false, false};
        for (int32_t i = 0; i < count; ++i) used[gs_class(ws[i].g)] = true;
        const size_t classes = static_cast<size_t>(used[0]) + used[1] + used[2];
        void* general = nullptr;
        if (const int32_t status = workspace(st, classes * bytes + 256, &general)) return status;
        unsigned char* xt =
            reinterpret_cast<unsigned char*>((reinterpret_cast<uintptr_t>(general) + 255) & ~uintptr_t{255});
        const uint32_t blocks = static_cast<uint32_t>(ceil_div(ceil_div(m, 4) * chunks, W));
        for (int32_t gc = 0; gc < 3; ++gc) {
            if (!used[gc]) continue;
            if (gc == 0) launch_rows_prep<0>(w0.bits, mt, blocks, a, m, w0.K, xt, st);
            else if (gc == 1) launch_rows_prep<1>(w0.bits, mt, blocks, a, m, w0.K, xt, st);
            else launch_rows_prep<2>(w0.bits, mt, blocks, a, m, w0.K, xt, st);
            KT_LAUNCHED("qmatmul: rows prep kernel");
            srcs[gc] = reinterpret_cast<const float*>(xt);
            xt += bytes;
        }
    }
    for (int32_t i = 0; i < count; ++i) {
        const WeightView& w = ws[i];
        const RowsPlan plan = rows_plan(m, w.K, w.g, w.N / SET, split);
        const int32_t gshift = log2_exact(w.g / RUN);
        const float* src = srcs[gs_class(w.g)];
        if (!plan.ks) return fail(KT_ERR_ARGUMENT, "packed rows gemv: no work split fits K = %d, M = %d", w.K, m);
        const int32_t kslog = log2_exact(plan.ks);
        const dim3 grid = split ? dim3(static_cast<uint32_t>(ceil_div(w.N / SET, W)), static_cast<uint32_t>(plan.ks))
                                : dim3(static_cast<uint32_t>(ceil_div(w.N / SET, W / plan.ks)));
        const int32_t shifts = kslog | gshift << 4 | log2_exact(plan.cpp) << 8;
        const RowsLaunch L{grid,  plan.lds, st,    w.p,        src, m,          w.N, w.K, shifts, alpha, cs[i],
                           accumulate, biases ? biases[i] : nullptr, partials, counters};
        const bool zp = w.z != nullptr;
        int32_t status;
        if (mt == 4) status = launch_rows_mt<4>(copy, split, gshift, w.bits, zp, L);
        else if (mt == 8) status = launch_rows_mt<8>(copy, split, gshift, w.bits, zp, L);
        else status = launch_rows_mt<16>(copy, split, gshift, w.bits, zp, L);
        if (status) return status;
        KT_LAUNCHED("qmatmul: packed rows gemv kernel");
    }
    return KT_OK;
}

}  // namespace kt
