// kt_gemm.hip -- prefill dequant-GEMM (M >= 3) on gfx950 MFMA:
//   c[M x N] = (accumulate ? c : 0) + alpha * a[M x K] . deq(W) (+ bias),
// the M > 1 branch of MatMul.multiplyQuantized (Engine/kotensor/src/main/kotlin/
// MatMul.kt:479-485 -> computeQuantizedTile :830-881).
//
// Numerics. The operands go to v_mfma_f32_32x32x16_f16 as fp16 with fp32
// accumulation. Two exact power-of-two rescalings keep fp16 in its normal range
// whatever the data: row m of a is multiplied by 2^-er[m] so its largest magnitude
// lies in [2^14, 2^15), and every scale of the weight by 2^-ew so that the largest
// scale lies in [2^6, 2^7) (so |q - zero| <= 255 times it stays below 2^15). A
// weight element enters the MFMA as (q - zero) * fp16(scale * 2^-ew) rounded once to
// fp16 (q - zero is an exact small integer), and the fp32 result is multiplied back
// by 2^(er[m] + ew). The roundings of a, of the scale and of the product to fp16
// (relative 2^-11 each) keep the normwise error far below the 2e-3 the path is held
// to; scales more than 2^20 below the largest one become fp16 subnormals and lose
// relative precision, but their products are that much below the largest ones.
//
// Pre-pass. One kernel writes the fp16 copy of a (zero-padded to whole tiles, so tile
// loads need no bounds checks) and er, one block per row reading the row once, and
// the largest scale magnitude of each slice of the scale array.
//
// GEMM. A 256-thread workgroup computes a 128 x 128 output tile (four waves in a
// 2 x 2 arrangement, 64 x 64 each as 2 x 2 MFMA 32x32 blocks) over K in steps of 64.
// Two LDS stages hold a and the dequantized weights of two steps; the global loads
// run two steps ahead in two register sets, so a step's data has two steps of MFMA
// time to arrive. Dequantization works on pairs of rows of one column: v_perm_b32
// puts the two bytes in the low bytes of the two halves of a word, and OR-ing (INT4
// nibble) or XOR-adding (INT8 byte + 128) the fp16 exponent of 1024 turns each half
// into the exact fp16 integer B + q; one packed fp16 add of -(B + zero) and one packed
// multiply by the scale give two weights, stored k-contiguous as the MFMA B operand
// reads them. INT8 tiles are 128 byte columns; INT4 tiles are 64 bytes = 64
// low-nibble plus 64 high-nibble columns, so every packed byte is read once per row
// tile. Workgroups that share a weight tile are numbered to land on one XCD (blocks
// are dealt to the eight XCDs round-robin), so the weight tile is fetched into one
// L2. When the tile grid is smaller than the GPU, K is split and a second kernel adds
// the slices in slice order.
#include <type_traits>

#include "kt_common.h"
#include "kt_packed.h"

namespace kt {
namespace {

typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 64;
constexpr int PITCH = BK + 8;  // halfs per LDS row (16-byte pad: conflict-free fragment reads)
constexpr int STAGE = BN * PITCH;  // halfs per weight stage (the dequantized weight tile)
constexpr int ASTAGE = BM * BK;    // halfs per a stage (rows of 128 bytes, chunks swizzled)
constexpr int ADEPTH = 4;          // a stages: K steps whose a tiles are loaded or in flight
constexpr int XCDS = 8;
constexpr int MAX_SPLITS = 8;
constexpr int DEPTH = 4;  // K steps whose weight loads are in flight
// LDS: the a stages and two weight stages; after the K loop the same array holds the
// exchange of the K halves (8 x 2 x 16 x 64 floats) and then the output tile
// (BM x (BN + 4) floats).
constexpr int LDS_HALFS = ADEPTH * ASTAGE + 2 * STAGE;
static_assert(LDS_HALFS >= 2 * 16384 && LDS_HALFS >= 2 * BM * (BN + 4), "LDS array holds the epilogue");

// s_waitcnt immediate that waits until at most n vector memory operations are
// outstanding (gfx9 encoding: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt at max).
constexpr int vmcnt_imm(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }
constexpr int ROW_CHUNKS = 16;       // float4 chunks of a row each pre-pass thread keeps in registers
constexpr int MAX_SCALE_BLOCKS = 256;  // pre-pass blocks over one weight's scales (one maximum each)
constexpr int MAX_GEMM_JOBS = 4;

// One weight of a launch (kt_qmatmul_group's q/k/v or gate/up share a and K): its column
// tiles are tile_begin .. tile_begin + tiles of the launch's tile row, its scale maxima
// smax[smax_begin .. smax_begin + nsb).
struct GemmJob {
    const uint8_t* q;
    const uint8_t* p;     // the column-run copy (gemm_packed_kernel)
    const float* pmax;    // its largest |scale| (the copy's trailer)
    const float* s;
    const int8_t* z;
    float* c;
    float* partials;  // [splits][M][N] when K is split
    const float* bias;
    int64_t scale_quads;
    int32_t N, bpr, tile_begin, smax_begin, nsb;
};
struct GemmJobs {
    GemmJob job[MAX_GEMM_JOBS];
    int32_t count;
};
__device__ __forceinline__ int32_t job_of_tile(const GemmJobs& jobs, int32_t tile_n) {
    int32_t j = 0;
#pragma unroll
    for (int32_t i = 1; i < MAX_GEMM_JOBS; ++i)
        if (i < jobs.count && tile_n >= jobs.job[i].tile_begin) j = i;
    return j;
}
__device__ __forceinline__ int32_t job_of_scale_block(const GemmJobs& jobs, int32_t sb) {
    int32_t j = 0;
#pragma unroll
    for (int32_t i = 1; i < MAX_GEMM_JOBS; ++i)
        if (i < jobs.count && sb >= jobs.job[i].smax_begin) j = i;
    return j;
}

// e such that max_abs * 2^-e lies in [2^(top-1), 2^top); 0 for zero or non-finite input.
__device__ __forceinline__ int32_t scale_exponent(float max_abs, int32_t top) {
    if (!(max_abs > 0.0f) || !isfinite(max_abs)) return 0;
    int e = 0;
    frexpf(max_abs, &e);  // max_abs = f * 2^e, f in [0.5, 1)
    return e - top;
}

__device__ __forceinline__ uint32_t pack_half2(float lo, float hi) {
    const half2v h = {static_cast<_Float16>(lo), static_cast<_Float16>(hi)};
    return __builtin_bit_cast(uint32_t, h);
}

// Maximum over the threads of a block of WAVES waves, returned to every thread.
template <int WAVES>
__device__ __forceinline__ float block_max(float v, float* red) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) v = fmaxf(v, __shfl_xor(v, o));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = red[0];
#pragma unroll
    for (int i = 1; i < WAVES; ++i) m = fmaxf(m, red[i]);
    return m;
}

// Chunk c (4 floats) of a row of K floats; zero past the end.
__device__ __forceinline__ f32x4 row_chunk(const float* row, int32_t c, int32_t K, bool vec) {
    const int32_t k = 4 * c;
    if (vec) return k < K ? *reinterpret_cast<const f32x4*>(row + k) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    f32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = k + i < K ? row[k + i] : 0.0f;
    return v;
}

// The largest |scale| over slice sb of the launch's scale slices, into smax[sb] (256
// threads). G * N is a multiple of 4 and s is 16-byte aligned (checked by the launchers).
__device__ __forceinline__ void scale_slice_max(const GemmJobs& jobs, int32_t sb, float* red, float* __restrict__ smax) {
    const int32_t t = threadIdx.x;
    const GemmJob& jb = jobs.job[job_of_scale_block(jobs, sb)];
    const float* s = jb.s;
    const int64_t scale_quads = jb.scale_quads;
    const int32_t nsb = jb.nsb;
    const int64_t per = (scale_quads + nsb - 1) / nsb;
    const int32_t sl = sb - jb.smax_begin;
    const int64_t begin = per * sl;
    const int64_t end = begin + per < scale_quads ? begin + per : scale_quads;
    float mx = 0.0f;
#pragma unroll 8
    for (int64_t i = begin + t; i < end; i += 256) {
        const f32x4 u = reinterpret_cast<const f32x4*>(s)[i];
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(u[0]), fabsf(u[1])), fmaxf(fabsf(u[2]), fabsf(u[3]))));
    }
    mx = block_max<4>(mx, red);
    if (t == 0) smax[sb] = mx;
}

// Blocks [0, Mp): row m of a as fp16 times 2^-er[m] (zeros for m >= M and k >= K).
// Blocks [Mp, Mp + sum of nsb): the largest |scale| over one slice of a job's G * N scales.
__global__ void __launch_bounds__(256)
    gemm_prep(const float* __restrict__ a, int32_t M, int32_t K, int32_t Kp, int32_t vec_rows, int32_t Mp,
              GemmJobs jobs, _Float16* __restrict__ a16,
              int32_t* __restrict__ er, float* __restrict__ smax) {
    __shared__ float red[4];
    const int32_t t = threadIdx.x;
    const int32_t b = blockIdx.x;
    if (b < Mp) {
        const int32_t m = b;
        const int32_t chunks = Kp / 4;
        uint2* row16 = reinterpret_cast<uint2*>(a16 + static_cast<size_t>(m) * Kp);
        auto dst = [&](int32_t cc) -> uint2& { return row16[cc]; };
        if (m >= M) {
            for (int32_t cc = t; cc < chunks; cc += 256) dst(cc) = make_uint2(0, 0);
            if (t == 0) er[m] = 0;
            return;
        }
        const float* row = a + static_cast<size_t>(m) * K;
        const bool vec = vec_rows != 0;  // K % 4 == 0 and a 16-byte aligned
        f32x4 v[ROW_CHUNKS];
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < ROW_CHUNKS; ++i) {
            const int32_t cc = t + 256 * i;
            v[i] = cc < chunks ? row_chunk(row, cc, K, vec) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i][0]), fabsf(v[i][1])), fmaxf(fabsf(v[i][2]), fabsf(v[i][3]))));
        }
        for (int32_t cc = t + 256 * ROW_CHUNKS; cc < chunks; cc += 256) {  // rows longer than 16384
            const f32x4 u = row_chunk(row, cc, K, vec);
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(u[0]), fabsf(u[1])), fmaxf(fabsf(u[2]), fabsf(u[3]))));
        }
        const int32_t e = scale_exponent(block_max<4>(mx, red), 15);
#pragma unroll
        for (int i = 0; i < ROW_CHUNKS; ++i) {
            const int32_t cc = t + 256 * i;
            if (cc < chunks)
                dst(cc) = make_uint2(pack_half2(ldexpf(v[i][0], -e), ldexpf(v[i][1], -e)),
                                     pack_half2(ldexpf(v[i][2], -e), ldexpf(v[i][3], -e)));
        }
        for (int32_t cc = t + 256 * ROW_CHUNKS; cc < chunks; cc += 256) {
            const f32x4 u = row_chunk(row, cc, K, vec);
            dst(cc) = make_uint2(pack_half2(ldexpf(u[0], -e), ldexpf(u[1], -e)),
                                 pack_half2(ldexpf(u[2], -e), ldexpf(u[3], -e)));
        }
        if (t == 0) er[m] = e;
        return;
    }
    scale_slice_max(jobs, b - Mp, red, smax);
}

// Work split of the 512 threads per K step: the weight tile is 64 rows x 32 lanes of
// column bytes (INT8: 4 bytes = 4 columns; INT4: 2 bytes = 2 low-nibble + 2
// high-nibble columns), each thread taking 4 consecutive rows of one lane's bytes,
// which lie in one scale group (g % 4 == 0).
constexpr int THREADS = 512;
constexpr int WROWS = 4;

template <int BITS>
struct WTile {
    static constexpr int BYTES = BITS == 8 ? 4 : 2;  // weight bytes per row and thread
    static constexpr int COLS = BITS == 8 ? 4 : 2;   // byte columns per thread
    static constexpr int SIDES = BITS == 8 ? 1 : 2;
};

// The weight data of one K step held by a thread.
template <int BITS>
struct WRegs {
    uint32_t w[WROWS];              // the thread's weight bytes of each row
    f32x4 s[WTile<BITS>::SIDES];    // scales of the thread's columns (per side)
    uint32_t z[WTile<BITS>::SIDES]; // zero points of the thread's columns (per side)
};

// Bytes j of words lo and hi in the low bytes of the two halves of a word.
__device__ __forceinline__ uint32_t pair_bytes(uint32_t lo, uint32_t hi, int j) {
    // v_perm_b32(S0 = hi, S1 = lo): selector bytes 0..3 pick lo's bytes, 4..7 hi's, 0x0c is 0.
    const uint32_t sel = 0x0c000c00u | (static_cast<uint32_t>(4 + j) << 16) | static_cast<uint32_t>(j);
    return __builtin_amdgcn_perm(hi, lo, sel);
}

// A constant held in a VGPR: (v & mask) | bits and (v ^ a) + b with such operands are
// one v_and_or_b32 / v_xad_u32 each. Only vector ALU instructions read the result.
__device__ __forceinline__ uint32_t in_vgpr(uint32_t c) {
    uint32_t r;
    asm("v_mov_b32 %0, %1" : "=v"(r) : "s"(c));
    return r;
}

__device__ __forceinline__ half2v as_h2(uint32_t v) { return __builtin_bit_cast(half2v, v); }

// One global_load_lds_dwordx4: lane l's 16 bytes at g land at LDS byte address lds + 16 l
// (lds wave-uniform). Written as inline assembly so the compiler neither reorders LDS
// accesses around it ("memory") nor waits for it on its own: the kernel waits for these
// loads itself with explicit vmcnt counts. The compiler's own waits for register loads
// stay correct, only stricter than needed, since it does not count these operations.
// Nothing else in the kernel uses m0.
__device__ __forceinline__ void lds_dma16(const void* g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(g), "s"(lds) : "memory");
}

template <int N_>
__device__ __forceinline__ f32x4 load_scales(const float* p) {
    if constexpr (N_ == 4) return *reinterpret_cast<const f32x4*>(p);
    const float2 v = *reinterpret_cast<const float2*>(p);
    return f32x4{v.x, v.y, 0.0f, 0.0f};
}

template <int N_>
__device__ __forceinline__ uint32_t load_bytes(const void* p) {
    if constexpr (N_ == 4) return *reinterpret_cast<const uint32_t*>(p);
    return *reinterpret_cast<const uint16_t*>(p);
}

// The 8 waves split each K step: waves 0-3 multiply k 0..31 of it, waves 4-7 k 32..63,
// each wave a 64 x 64 block of the tile (2 x 2 waves per half). The a tile of a step
// goes from global memory straight into an LDS stage (global_load_lds, 16 bytes per
// lane, no registers), ADEPTH steps ahead; the weights come through registers and are
// dequantized into LDS. The two halves' sums are added through LDS at the end. Two
// waves per SIMD let one wave's dequantization and waits overlap the other's MFMAs.
// FAST: K % BK == 0 and the group size divides BK or is a multiple of it, so every
// weight load of a step is a uniform base plus an offset fixed per lane (no per-step
// address arithmetic and no clamping); otherwise rows and groups are computed per step.
template <int BITS, bool ZP, bool FAST>
__global__ void __launch_bounds__(THREADS, 1)
    gemm_kernel(const _Float16* __restrict__ a16, int32_t Kp, const int32_t* __restrict__ er,
                const float* __restrict__ smax_all, GemmJobs jobs, int32_t M, int32_t K, int32_t g, int32_t tiles_m,
                int32_t tiles_n, int32_t splits, int32_t steps_per_split, float alpha, int32_t accumulate) {
    __shared__ __attribute__((aligned(16))) _Float16 lds[LDS_HALFS];
    __shared__ int32_t er_s[BM];
    __shared__ float red[THREADS / 64];
    _Float16* const wstage = lds + ADEPTH * ASTAGE;  // the two weight stages
    constexpr int BYTES = WTile<BITS>::BYTES;
    constexpr int COLS = WTile<BITS>::COLS;
    constexpr int SIDES = WTile<BITS>::SIDES;

    // Block -> (tile_n, tile_m, slice): blocks d, d + 8, d + 16, ... run on XCD d, and
    // consecutive ones of them take the row tiles and K slices of one weight tile.
    const int32_t pid = blockIdx.x;
    const int32_t j = pid / XCDS;
    const int32_t per_n = tiles_m * splits;
    const int32_t tile_n = (j / per_n) * XCDS + pid % XCDS;
    if (tile_n >= tiles_n) return;
    // the weight of this column tile
    const GemmJob& jb = jobs.job[job_of_tile(jobs, tile_n)];
    const uint8_t* __restrict__ q = jb.q;
    const float* __restrict__ s = jb.s;
    const int8_t* __restrict__ z = jb.z;
    float* __restrict__ c = jb.c;
    float* __restrict__ partials = jb.partials;
    const float* __restrict__ bias = jb.bias;
    const float* __restrict__ smax = smax_all + jb.smax_begin;
    const int32_t N = jb.N, bpr = jb.bpr, nsb = jb.nsb;
    const int32_t rem = j % per_n;
    const int32_t tile_m = rem % tiles_m;
    const int32_t sp = rem / tiles_m;
    const int32_t k_steps = (K + BK - 1) / BK;
    const int32_t ks0 = sp * steps_per_split;
    const int32_t n_steps = min(steps_per_split, k_steps - ks0);  // >= 1 by the host's split count

    const int32_t t = threadIdx.x;
    const int32_t ln = t & 63;
    const int32_t wave = t >> 6;
    const int32_t kh = __builtin_amdgcn_readfirstlane(wave >> 2);  // which half of each K step this wave multiplies
    const int32_t wm = (wave >> 1) & 1, wn = wave & 1;
    const int32_t m0 = tile_m * BM;
    const int32_t b0 = (tile_n - jb.tile_begin) * (BITS == 8 ? BN : BN / 2);  // first byte column of the tile

    // Lane l of wave w takes byte group cq = l % 16 + 16 (l / 32) of rows rg * 4 .. rg * 4 + 3,
    // rg = 2 w + (l / 16) % 2. Its column j of the group goes to row 32 j + cq of the
    // dequantized tile (64 + ... for INT4 high nibbles), so the 32 lanes of a half-wave
    // write 16 consecutive rows at two k offsets: the 64 LDS banks exactly once.
    const int32_t cq = (t & 15) + ((t >> 1) & 16);
    const int32_t rg = ((t >> 6) << 1) + ((t >> 4) & 1);
    const int32_t bcol = b0 + cq * BYTES < bpr ? b0 + cq * BYTES : 0;  // bpr % 4 == 0: byte groups are whole

    // Byte offsets fixed per lane.
    uint32_t w_off[WROWS];
#pragma unroll
    for (int i = 0; i < WROWS; ++i) w_off[i] = static_cast<uint32_t>(rg * WROWS + i) * bpr + bcol;
    const uint32_t s_idx = static_cast<uint32_t>(g < BK ? (rg * WROWS) / g : 0) * N + bcol;
    // a tile: row r of a stage is 128 bytes = 8 chunks of 16 bytes; chunk c of row r sits
    // in slot c ^ ((r / 2) % 8), so 16 lanes reading one chunk column of 16 rows hit all
    // 64 banks once. A load instruction fills 1 KiB = rows 8 b .. 8 b + 7 (b = 8 j + wave,
    // j = 0, 1), lane l writing slot l % 8 of row 8 b + l / 8: it loads the chunk that
    // belongs there.
    uint32_t a_off[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
        const int32_t r = (jj * 8 + wave) * 8 + (ln >> 3);
        a_off[jj] = static_cast<uint32_t>(r) * Kp + (((ln & 7) ^ ((r >> 1) & 7)) << 3);
    }
    const _Float16* a_tile = a16 + static_cast<size_t>(m0) * Kp;

    // Loads part `part` of a step's weight data: 0 rows 0-1, 1 rows 2-3, 2 scales and
    // zero points (-1: all), so the loads can be spread over a step.
    auto load_w = [&](WRegs<BITS>& r, int32_t step, int part = -1) {
        const int32_t k0 = (ks0 + step) * BK;
        const int32_t kr = k0 + rg * WROWS;
#pragma unroll
        for (int i = 0; i < WROWS; ++i) {
            if (part >= 0 && part != i / 2) continue;
            if constexpr (FAST) {
                r.w[i] = load_bytes<BYTES>(q + static_cast<size_t>(k0) * bpr + w_off[i]);
            } else {
                const int32_t row = kr + i < K ? kr + i : K - 1;  // a is zero on rows >= K
                r.w[i] = load_bytes<BYTES>(q + static_cast<size_t>(row) * bpr + bcol);
            }
        }
        if (part >= 0 && part != 2) return;
        const size_t at = FAST ? static_cast<size_t>(k0 / g) * N + s_idx
                               : static_cast<size_t>((kr < K ? kr : K - 1) / g) * N + bcol;
#pragma unroll
        for (int side = 0; side < SIDES; ++side) {
            r.s[side] = load_scales<COLS>(s + at + (side ? bpr : 0));
            if constexpr (ZP) r.z[side] = load_bytes<BYTES>(z + at + (side ? bpr : 0));
        }
    };
    auto load_a = [&](int32_t step) {
        const _Float16* ab = a_tile + static_cast<size_t>(ks0 + step) * BK;
        const uint32_t st = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds + (step % ADEPTH) * ASTAGE));
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
            lds_dma16(ab + a_off[jj], __builtin_amdgcn_readfirstlane(st + (jj * 8 + wave) * 1024));
    };
    // Vector memory operations a thread issues per step after its a loads: the weight
    // bytes, scales and zero points.
    constexpr int NW = WROWS + SIDES * (ZP ? 2 : 1);

    // The slice maxima of the scales and the row exponents are loaded first, then the
    // first steps: loads complete in order, so waiting for the former does not wait
    // for the latter.
    const float smx = t < nsb ? smax[t] : 0.0f;  // nsb <= 256
    const int32_t erv = t < BM && m0 + t < M ? er[m0 + t] : 0;
    __builtin_amdgcn_sched_barrier(0);
    WRegs<BITS> r[DEPTH];
    const int32_t last = n_steps - 1;
    static_assert(ADEPTH == DEPTH, "a stage and weight set indices both follow step % 4");
    // a tiles of steps 0..2 and weights of steps 0..3, a first in each pair.
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) {
        if (d < ADEPTH - 1) load_a(min(d, last));
        __builtin_amdgcn_sched_barrier(0);
        load_w(r[d], min(d, last));
        __builtin_amdgcn_sched_barrier(0);
    }
    if (t < BM) er_s[t] = erv;
    const int32_t ew = scale_exponent(block_max<THREADS / 64>(smx, red), 7);

    const uint32_t flip = in_vgpr(0x00800080u), exp1024 = in_vgpr(0x64006400u);
    const uint32_t mask_lo = in_vgpr(0x000F000Fu), mask_hi = in_vgpr(0x00F000F0u);

    // Dequantizes piece p (0..3) of the thread's weight bytes into a stage: INT8 column
    // p; INT4 byte column p / 2, low nibbles for even p and high nibbles for odd p.
    auto store_piece = [&](const WRegs<BITS>& rs, int32_t stage, int p) {
        _Float16* Bs = wstage + stage * STAGE;
        const int jq = BITS == 8 ? p : p >> 1;
        const int side = BITS == 8 ? 0 : p & 1;
        const uint32_t pr0 = pair_bytes(rs.w[0], rs.w[1], jq), pr1 = pair_bytes(rs.w[2], rs.w[3], jq);
        // INT4 high nibbles enter as 1024 + 16 q: the offset is -(1024 + 16 zero) and the
        // scale is divided by 16, which is exact, so the product is the same.
        const float sc = ldexpf(rs.s[side][jq], side ? -ew - 4 : -ew);
        const half2v scv = {static_cast<_Float16>(sc), static_cast<_Float16>(sc)};
        // -(B + zero) in both halves: the zero byte under the fp16 bits of -1024 (INT4,
        // zero in [0, 15]) or of -1024 - (zero + 128) (INT8, signed zero).
        uint32_t off;
        if constexpr (!ZP) {
            off = 0xE480E480u;  // -1152
        } else {
            const uint32_t zz = pair_bytes(rs.z[side], rs.z[side], jq);
            if constexpr (BITS == 8) off = (zz ^ flip) + 0xE400E400u;
            else off = side ? (zz << 4) | 0xE400E400u : zz | 0xE400E400u;
        }
        const half2v ofv = as_h2(off);
        uint32_t x0, x1;
        if constexpr (BITS == 8) {
            x0 = (pr0 ^ flip) + exp1024;
            x1 = (pr1 ^ flip) + exp1024;
        } else {
            x0 = (pr0 & (side ? mask_hi : mask_lo)) | exp1024;
            x1 = (pr1 & (side ? mask_hi : mask_lo)) | exp1024;
        }
        const uint32_t h0 = __builtin_bit_cast(uint32_t, (as_h2(x0) + ofv) * scv);
        const uint32_t h1 = __builtin_bit_cast(uint32_t, (as_h2(x1) + ofv) * scv);
        const int32_t nl = side * (BN / 2) + jq * 32 + cq;
        *reinterpret_cast<uint2*>(Bs + nl * PITCH + rg * WROWS) = make_uint2(h0, h1);
    };

    float16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][jj][e] = 0.0f;

    // One step: the MFMAs of a stage `as` and weight stage `cur` (this wave's half of
    // the step's K) alternate with the dequantization of the next step's weights into
    // weight stage `nxt`, in a fixed order (sched_barrier) so the matrix and vector
    // units work at the same time.
    // With loads (main loop), the a tile of step `la` goes into a stage `las` and the
    // weights of step `lw` into `rl` between the MFMA pairs, so the memory pipeline
    // works while the MFMAs run instead of after the barrier.
    auto step = [&](int32_t as, int32_t cur, const WRegs<BITS>& rs, int32_t nxt, auto dequant, auto loads,
                    WRegs<BITS>& rl, int32_t la, int32_t lw) {
        constexpr bool DQ = decltype(dequant)::value;
        constexpr bool LD = decltype(loads)::value;
        const _Float16* As = lds + as * ASTAGE;
        const _Float16* Bs = wstage + cur * STAGE;
        half8 af[2][2], bf[2][2];
#pragma unroll
        for (int kq = 0; kq < 2; ++kq) {
            const int32_t kk = kh * (BK / 2) + kq * 16 + (ln >> 5) * 8;
            const int32_t kc = kk >> 3;  // chunk of the a row
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int32_t ra = wm * 64 + i * 32 + (ln & 31);
                af[kq][i] = *reinterpret_cast<const half8*>(As + ra * BK + ((kc ^ ((ra >> 1) & 7)) << 3));
                bf[kq][i] = *reinterpret_cast<const half8*>(Bs + (wn * 64 + i * 32 + (ln & 31)) * PITCH + kk);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int kq = p >> 1, i = p & 1;
            acc[i][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[kq][i], bf[kq][0], acc[i][0], 0, 0, 0);
            acc[i][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[kq][i], bf[kq][1], acc[i][1], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (DQ) store_piece(rs, nxt, p);
            if constexpr (LD) {
                if (p == 0) load_a(la);
                else load_w(rl, lw, p - 1);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    // Pipeline: weight stage (step & 1) holds the weights of the step being multiplied
    // while the next step is dequantized into the other stage. During step s the a tile
    // of step s + 3 loads into the a stage step s - 1 used and the weights of step s + 4
    // into the register set step s - 1 dequantized. Loads past the last step repeat the
    // last step and are never used. sched_barrier(0) keeps the compiler from moving
    // loads across the phases. The compiler waits for register loads itself; the a loads
    // write LDS behind its back, so before the barrier that precedes reading a stage each
    // thread waits until only the loads issued after that stage's are outstanding: in
    // the steady state the weights of its own step and two later steps (3 NW + 4). The
    // main loop body has no branches, so the compiler's waits stay exact; the last (at
    // most DEPTH) steps, whose loads are all issued, run in the tail.
#pragma unroll
    for (int p = 0; p < 4; ++p) store_piece(r[0], 0, p);
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(4 * NW + 4));  // a tile of step 0
    __syncthreads();
    int32_t i = 0;
    for (; i + DEPTH < n_steps; i += DEPTH) {
#pragma unroll
        for (int u = 0; u < DEPTH; ++u) {
            // step i + u
            step(u, u & 1, r[(u + 1) % DEPTH], (u + 1) & 1, std::true_type{}, std::true_type{}, r[u],
                 min(i + u + ADEPTH - 1, last), min(i + u + DEPTH, last));
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(3 * NW + 4));  // a tile of step i + u + 1
            __syncthreads();
        }
    }
    // The tail issues the same loads (the a tile of step i + 3 may not be loaded yet) and
    // waits for all of them before each barrier.
#pragma unroll
    for (int u = 0; u < DEPTH; ++u) {
        if (i + u < n_steps) {
            if (i + u + 1 < n_steps)
                step(u, u & 1, r[(u + 1) % DEPTH], (u + 1) & 1, std::true_type{}, std::true_type{}, r[u],
                     min(i + u + ADEPTH - 1, last), min(i + u + DEPTH, last));
            else
                step(u, u & 1, r[0], 0, std::false_type{}, std::false_type{}, r[0], 0, 0);
            __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
            __syncthreads();
        }
    }

    // The two K halves meet: wave (kh, quad) hands its sums of row block 1 - kh to its
    // partner (1 - kh, quad) through LDS and adds the partner's sums of row block kh,
    // so each wave ends with the full sums of 32 rows x 64 columns.
    float16v fin[2];
    {
        float* xch = reinterpret_cast<float*>(lds);  // 8 regions of 2 x 16 x 64 floats = 64 KiB
        const int32_t quad = wave & 3;
        float* mine = xch + (quad * 2 + (1 - kh)) * 2 * 16 * 64;
        const float* theirs = xch + (quad * 2 + kh) * 2 * 16 * 64;
        if (kh == 0) {
            fin[0] = acc[1][0];
            fin[1] = acc[1][1];
        } else {
            fin[0] = acc[0][0];
            fin[1] = acc[0][1];
        }
#pragma unroll
        for (int jb = 0; jb < 2; ++jb)
#pragma unroll
            for (int e = 0; e < 16; ++e) mine[(jb * 16 + e) * 64 + ln] = fin[jb][e];
        if (kh == 0) {
            fin[0] = acc[0][0];
            fin[1] = acc[0][1];
        } else {
            fin[0] = acc[1][0];
            fin[1] = acc[1][1];
        }
        __syncthreads();
#pragma unroll
        for (int jb = 0; jb < 2; ++jb)
#pragma unroll
            for (int e = 0; e < 16; ++e) fin[jb][e] += theirs[(jb * 16 + e) * 64 + ln];
    }

    // Epilogue: the tile goes through LDS in output-column order and leaves in rows of
    // 16-byte stores. Element (i, j) of a 32x32 MFMA block sits in lane
    // j + 32 * ((i / 4) % 2), register (i / 8) * 4 + i % 4; tile row nl holds byte column
    // COLS (nl % 32) + (nl / 32) % COLS of the tile (INT4: high nibbles when nl >= 64).
    constexpr int OPITCH = BN + 4;  // floats per staged row
    float* tile_out = reinterpret_cast<float*>(lds);  // BM x OPITCH floats
    __syncthreads();                                  // the exchange area is read
    {
        const int32_t mrow = wm * 64 + kh * 32 + (ln >> 5) * 4;  // tile row of register 0
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) {
            const int32_t nl = wn * 64 + jb * 32 + (ln & 31);
            const int32_t col = (nl & BN / 2) * (BITS == 4) + COLS * (nl & 31) + ((nl >> 5) & (COLS - 1));
#pragma unroll
            for (int e = 0; e < 16; ++e) tile_out[(mrow + (e >> 2) * 8 + (e & 3)) * OPITCH + col] = fin[jb][e];
        }
    }
    __syncthreads();
    float* out = partials ? partials + static_cast<size_t>(sp) * M * N : c;
    const bool add = !partials && accumulate;
    const float* bs = partials ? nullptr : bias;
    const float al = partials ? 1.0f : alpha;
#pragma unroll
    for (int it = 0; it < BM * BN / 4 / THREADS; ++it) {
        const int32_t idx = t + THREADS * it;
        const int32_t ml = idx / (BN / 4), cv = (idx % (BN / 4)) * 4;  // tile row, first tile column
        const int32_t tc = BITS == 4 && cv >= BN / 2 ? cv - BN / 2 : cv;  // byte column within the tile
        const int32_t n = (BITS == 4 && cv >= BN / 2 ? bpr : 0) + b0 + tc;
        if (m0 + ml >= M || b0 + tc >= bpr) continue;  // bpr % 4 == 0: the 4 columns are valid together
        f32x4 v = *reinterpret_cast<const f32x4*>(tile_out + ml * OPITCH + cv);
        const int32_t e = er_s[ml] + ew;
        f32x4* dst = reinterpret_cast<f32x4*>(out + static_cast<size_t>(m0 + ml) * N + n);
        const f32x4 old = add ? *dst : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        const f32x4 bv = bs ? *reinterpret_cast<const f32x4*>(bs + n) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) v[q4] = fmaf(al, ldexpf(v[q4], e), old[q4]) + bv[q4];
        *dst = v;
    }
}

// Adds the K slices of every output in slice order, then alpha, accumulate, bias.
__global__ void __launch_bounds__(256)
    gemm_reduce(const float* __restrict__ partials, int32_t splits, int32_t M, int32_t N, float* __restrict__ c,
                const float* __restrict__ bias, float alpha, int32_t accumulate) {
    const size_t idx = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    const size_t total = static_cast<size_t>(M) * N;
    if (idx >= total) return;
    float v[MAX_SPLITS];
#pragma unroll
    for (int i = 0; i < MAX_SPLITS; ++i) v[i] = i < splits ? partials[i * total + idx] : 0.0f;
    float sum = v[0];
#pragma unroll
    for (int i = 1; i < MAX_SPLITS; ++i)
        if (i < splits) sum += v[i];
    const float o = fmaf(alpha, sum, accumulate ? c[idx] : 0.0f);
    c[idx] = bias ? o + bias[idx % N] : o;
}


// ---- prefill GEMM on the column-run copy ------------------------------------------------
// With the weight's column-run copy (kt_qweight_pack) and g a multiple of 32, each of the
// four waves of a workgroup computes the whole 128 x 128 output tile over its own quarter
// of K: slabs of 32 k, wave w taking slabs w, w + 4, ... of the workgroup's range. A wave
// shares no operand with another, so the K loop has no LDS traffic and no barrier: every
// operand goes from memory straight into registers in the MFMA layout (16-byte lanes for
// a, 16 or 8 contiguous bytes of one column for the weights), PDEPTH slabs ahead, and the
// 128 x 128 fp32 sums (16 blocks of v_mfma_f32_32x32x16_f16) sit in the accumulation
// registers. The four waves' sums meet once, through LDS, at the end, added in wave order.
//
// MFMA k order. In slab s, lane l (row or column l % 32, hl = l / 32) supplies elements
// e = 0..7 of sub-product i = 0, 1 at k =
//   INT8: 32 s + 16 hl + 8 i + e      (column-run bytes 8 i + e of piece hl of run s),
//   INT4: 64 (s / 2) + 32 hl + 16 (s % 2) + 8 i + e   (dword 2 (s % 2) + i of the lane's
//         16 bytes of run 2 (s / 2) + hl: low nibbles e = 0..3, high nibbles e = 4..7),
// so a lane's weight bytes are contiguous in the copy. The fp16 copy of a is written in
// the same order by gemm_prep_tiled: per (row tile, slab) 8 KiB, piece (row block rb,
// sub i) of 1 KiB holding lane l's 16 bytes at 16 l. With g % 32 == 0 a lane's 16 or 32 k
// of a column lie in one scale group.
// Dequantization and scaling are those of gemm_kernel (same fp16 values of the weights and
// of a, the same powers of two); only the order of the fp32 sums differs.
// Tiles are TM x TN with TM, TN in {64, 128}: 128 x 128 when the tiles fill the CUs,
// 64-row tiles for M <= 64 (no padded rows), 64-column tiles when 128-column ones leave
// CUs idle (narrow M).
constexpr int PTHREADS = 256;
__host__ __device__ constexpr int pslab_bytes(int tm) { return tm * 32 * 2; }  // fp16 a per (row tile, slab)
__host__ __device__ constexpr int mpitch(int tn) { return tn + 4; }            // floats per row of the meet
// the epilogue's meet: four waves x 64 rows (132 KiB at TN = 128)
__host__ __device__ constexpr size_t plds_bytes(int tn) { return 4 * 64 * mpitch(tn) * sizeof(float); }

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Rows of a in the tiled fp16 order above (row tiles of TM rows), one wave per row
// (Mp / 4 blocks; the weights' scale maxima come from their copies). S = slabs (K rounded
// up to 128, over 32).
template <int BITS, int TM>
__global__ void __launch_bounds__(256)
    gemm_prep_tiled(const float* __restrict__ a, int32_t M, int32_t K, int32_t S, int32_t vec_rows, int32_t Mp,
                    _Float16* __restrict__ a16t, int32_t* __restrict__ er) {
    (void)Mp;
    const int32_t m = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int32_t ln = threadIdx.x & 63;
    const int32_t tm = m / TM, r = m % TM, rb = r / 32, rl = r % 32;
    // the piece holding k = 32 sp + 8 o8 .. + 8 of this row
    auto piece = [&](int32_t sp, int32_t o8) -> u32x4* {
        const int32_t q = o8 >> 1, i = o8 & 1;
        const int32_t slab = BITS == 8 ? sp : 2 * (sp >> 1) + q;
        const int32_t hl = BITS == 8 ? q : (sp & 1);
        return reinterpret_cast<u32x4*>(a16t) + ((static_cast<size_t>(tm) * S + slab) * (TM / 16) + rb * 2 + i) * 64 +
               rl + 32 * hl;
    };
    if (m >= M) {
        for (int32_t sp = ln; sp < S; sp += 64)
#pragma unroll
            for (int o8 = 0; o8 < 4; ++o8) *piece(sp, o8) = u32x4{0u, 0u, 0u, 0u};
        if (ln == 0) er[m] = 0;
        return;
    }
    const float* row = a + static_cast<size_t>(m) * K;
    const bool vec = vec_rows != 0;
    auto absmax = [](const f32x4& v) { return fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))); };
    // float4 f of the row (lanes take f = ln + 64 j: each load a contiguous KiB) holds
    // elements 4 (f % 8) .. + 3 of span f / 8: half f % 2 of piece (f / 8, (f % 8) / 2)
    auto put_half = [&](int32_t f, const f32x4& v, int32_t e) {
        *reinterpret_cast<u32x2*>(reinterpret_cast<char*>(piece(f >> 3, (f & 7) >> 1)) + 8 * (f & 1)) =
            u32x2{pack_half2(ldexpf(v[0], -e), ldexpf(v[1], -e)), pack_half2(ldexpf(v[2], -e), ldexpf(v[3], -e))};
    };
    float mx = 0.0f;
    if (S <= 2 * 64) {
        // K <= 4096: the row read once, into registers
        f32x4 v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int32_t f = ln + 64 * j;
            v[j] = f < 8 * S ? row_chunk(row, f, K, vec) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            mx = fmaxf(mx, absmax(v[j]));
        }
        mx = wave_max64(mx);
        const int32_t e = scale_exponent(mx, 15);
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (ln + 64 * j < 8 * S) put_half(ln + 64 * j, v[j], e);
        if (ln == 0) er[m] = e;
        return;
    }
    // longer rows: read twice (the maximum, then the halves), 16 loads in flight per lane
    for (int32_t f0 = 0; f0 < 8 * S; f0 += 16 * 64) {
        f32x4 v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int32_t f = f0 + ln + 64 * j;
            v[j] = f < 8 * S ? row_chunk(row, f, K, vec) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) mx = fmaxf(mx, absmax(v[j]));
    }
    mx = wave_max64(mx);
    const int32_t e = scale_exponent(mx, 15);
    for (int32_t f0 = 0; f0 < 8 * S; f0 += 16 * 64) {
        f32x4 v[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int32_t f = f0 + ln + 64 * j;
            v[j] = f < 8 * S ? row_chunk(row, f, K, vec) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int j = 0; j < 16; ++j)
            if (f0 + ln + 64 * j < 8 * S) put_half(f0 + ln + 64 * j, v[j], e);
    }
    if (ln == 0) er[m] = e;
}

// The same for rows of 4096 < K <= 16384: a workgroup of four waves per row, each wave a
// quarter of it in registers (float4 f = 1024 w + ln + 64 j), the row's maximum through
// LDS, so the row is read once and in one round trip. (One wave per row read such a row
// twice, in rounds of 16 loads per lane: 22 us for 64 rows of 14336 against 4 at 4096.)
template <int BITS, int TM>
__global__ void __launch_bounds__(256)
    gemm_prep_tiled_long(const float* __restrict__ a, int32_t M, int32_t K, int32_t S, int32_t vec_rows,
                         _Float16* __restrict__ a16t, int32_t* __restrict__ er) {
    __shared__ float red[4];
    const int32_t m = blockIdx.x, t = threadIdx.x, ln = t & 63, w = t >> 6;
    const int32_t tm = m / TM, r = m % TM, rb = r / 32, rl = r % 32;
    auto piece = [&](int32_t sp, int32_t o8) -> u32x4* {
        const int32_t q = o8 >> 1, i = o8 & 1;
        const int32_t slab = BITS == 8 ? sp : 2 * (sp >> 1) + q;
        const int32_t hl = BITS == 8 ? q : (sp & 1);
        return reinterpret_cast<u32x4*>(a16t) + ((static_cast<size_t>(tm) * S + slab) * (TM / 16) + rb * 2 + i) * 64 +
               rl + 32 * hl;
    };
    if (m >= M) {
        for (int32_t sp = t; sp < S; sp += 256)
#pragma unroll
            for (int o8 = 0; o8 < 4; ++o8) *piece(sp, o8) = u32x4{0u, 0u, 0u, 0u};
        if (t == 0) er[m] = 0;
        return;
    }
    const float* row = a + static_cast<size_t>(m) * K;
    const bool vec = vec_rows != 0;
    auto absmax = [](const f32x4& v) { return fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))); };
    f32x4 v[16];
    float mx = 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int32_t f = 1024 * w + ln + 64 * j;
        v[j] = f < 8 * S ? row_chunk(row, f, K, vec) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        mx = fmaxf(mx, absmax(v[j]));
    }
    const int32_t e = scale_exponent(block_max<4>(mx, red), 15);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int32_t f = 1024 * w + ln + 64 * j;
        if (f < 8 * S)
            *reinterpret_cast<u32x2*>(reinterpret_cast<char*>(piece(f >> 3, (f & 7) >> 1)) + 8 * (f & 1)) =
                u32x2{pack_half2(ldexpf(v[j][0], -e), ldexpf(v[j][1], -e)),
                      pack_half2(ldexpf(v[j][2], -e), ldexpf(v[j][3], -e))};
    }
    if (t == 0) er[m] = e;
}

// One slab of a wave: a pieces (2 rb + i), the weight bytes of its CB column blocks, and
// their scales and zero points.
template <int BITS, int RB, int CB>
struct PSlab {
    u32x4 a[2 * RB];
    typename std::conditional<BITS == 8, u32x4, u32x2>::type w[CB];
    float s[CB];
    uint32_t z[CB];  // the dword holding the column's zero byte
};

// v_perm_b32 selectors: bytes (0, 1) or (2, 3) of a word into the low bytes of its halves.
constexpr uint32_t SEL01 = 0x0c010c00u, SEL23 = 0x0c030c02u;

// PDEPTH: slabs a wave holds or has in flight (3 for the larger tiles; the 64 x 64 tile of
// narrow M, whose waves have few registers of sums and a long K range each, holds 8).
template <int BITS, bool ZP, int TM, int TN, int PDEPTH>
__global__ void __launch_bounds__(PTHREADS, 1)
    gemm_packed_kernel(const _Float16* __restrict__ a16t, const int32_t* __restrict__ er, GemmJobs jobs, int32_t M,
                       int32_t K, int32_t S, int32_t g,
                       int32_t tiles_m, int32_t tiles_n, int32_t splits, int32_t slabs_per_split, float alpha,
                       int32_t accumulate) {
    constexpr int RB = TM / 32, CB = TN / 32;  // 32 x 32 row and column blocks
    constexpr int PSLAB = pslab_bytes(TM), MPITCH = mpitch(TN);
    extern __shared__ f32x4 meet[];  // the epilogue's meet, plds_bytes(TN)
    __shared__ int32_t er_s[TM];

    // Block -> (tile_n, tile_m, slice) as gemm_kernel: the workgroups of one weight tile on one XCD.
    const int32_t pid = blockIdx.x;
    const int32_t jx = pid / XCDS;
    const int32_t per_n = tiles_m * splits;
    const int32_t tile_n = (jx / per_n) * XCDS + pid % XCDS;
    if (tile_n >= tiles_n) return;
    const GemmJob& jb = jobs.job[job_of_tile(jobs, tile_n)];
    const int32_t N = jb.N;
    const int32_t sets = (N + 15) / 16, chunks = S / 4, G = (K + g - 1) / g;
    const int32_t gsh = __builtin_ctz(static_cast<uint32_t>(g));  // g = 32 << k
    const int32_t rem = jx % per_n;
    const int32_t tile_m = rem % tiles_m;
    const int32_t sp = rem / tiles_m;
    const int32_t col0 = (tile_n - jb.tile_begin) * TN;
    const int32_t m0 = tile_m * TM;
    const int32_t t = threadIdx.x, ln = t & 63, hl = ln >> 5;
    const int32_t wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int32_t s_begin = sp * slabs_per_split;
    const int32_t n_mine = (min(S, s_begin + slabs_per_split) - s_begin) / 4;  // >= 1: the host keeps slices whole

    const float smx = *jb.pmax;  // the weight's largest |scale|, from its copy
    const int32_t erv = t < TM && m0 + t < M ? er[m0 + t] : 0;

    const __amdgpu_buffer_rsrc_t ar = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(a16t) + static_cast<size_t>(tile_m) * S * (PSLAB / 2), 0, S * PSLAB, 0x00020000);
    const uint32_t wbytes = static_cast<uint32_t>(sets) * chunks * (BITS == 8 ? 2048u : 1024u);
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(jb.p), 0, wbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t sr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(jb.s), 0, static_cast<uint32_t>(G) * N * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t zr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(ZP ? jb.z : nullptr), 0, ZP ? static_cast<uint32_t>(G) * N : 0u, 0x00020000);

    // Lane offsets fixed for the whole loop.
    uint32_t w_off[CB], z_shift[CB];
    int32_t col_c[CB];
#pragma unroll
    for (int j = 0; j < CB; ++j) {
        const int32_t col = col0 + 32 * j + (ln & 31);
        const int32_t set = min(col >> 4, sets - 1);  // past the last column: any valid bytes, outputs dropped
        w_off[j] = static_cast<uint32_t>(set) * chunks * (BITS == 8 ? 2048u : 1024u) +
                   (BITS == 8 ? hl * 1024u : hl * 256u) + (ln & 15) * 16u;
        col_c[j] = min(col, N - 1);
        z_shift[j] = 8u * (col_c[j] & 3);
    }
    auto load = [&](PSlab<BITS, RB, CB>& d, int32_t x) {
        const int32_t s = s_begin + wave + 4 * min(x, n_mine - 1);
#pragma unroll
        for (int pc = 0; pc < 2 * RB; ++pc)
            d.a[pc] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(ar, (pc * 64 + ln) * 16, s * PSLAB, 0));
        const int32_t wso = BITS == 8 ? (s >> 2) * 2048 + (s & 3) * 256 : (s >> 2) * 1024 + ((s >> 1) & 1) * 512 + (s & 1) * 8;
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            if constexpr (BITS == 8)
                d.w[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wr, w_off[j], wso, 0));
            else
                d.w[j] = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(wr, w_off[j], wso, 0));
        }
        // the group row of the lane's run (first k: 64 (s / 2) + 32 hl; INT8 32 s), offset
        // into the [G x N] arrays: scalars for the two lane halves (g a power of two), one
        // select per lane
        const int32_t kg0 = BITS == 8 ? 32 * s : 64 * (s >> 1);
        const uint32_t row0 = static_cast<uint32_t>(min(kg0 >> gsh, G - 1)) * N;
        const uint32_t row1 = BITS == 8 ? row0 : static_cast<uint32_t>(min((kg0 + 32) >> gsh, G - 1)) * N;
        const uint32_t row_off = hl ? row1 : row0;
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            const uint32_t at = row_off + col_c[j];
            d.s[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(sr, at * 4, 0, 0));
            // the dword holding the zero byte (N % 4 == 0: it lies inside the array); a byte
            // load's extension would be placed ahead of the loop and wait for every load
            if constexpr (ZP) d.z[j] = __builtin_amdgcn_raw_buffer_load_b32(zr, at & ~3u, 0, 0);
        }
    };

    PSlab<BITS, RB, CB> sl[PDEPTH];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 0; d + 1 < PDEPTH; ++d) {
        load(sl[d], d);  // in slab order: the loop's waits count on it
        __builtin_amdgcn_sched_barrier(0);
    }
    if (t < TM) er_s[t] = erv;
    const int32_t ew = scale_exponent(smx, 7);
    __builtin_amdgcn_sched_barrier(0);

    float16v acc[RB][CB];
#pragma unroll
    for (int i = 0; i < RB; ++i)
#pragma unroll
        for (int j = 0; j < CB; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;

    // Dequantizes sub-product i of one slab's weights (the fp16 values gemm_kernel's
    // store_piece makes): column block j's operand into b[j]. Sub-product 0 also turns the
    // slab's scales and zero points into their fp16 forms, kept in s and z for sub-product 1.
    auto dequant = [&](PSlab<BITS, RB, CB>& d, int i, half8 (&b)[CB]) {
#pragma unroll
        for (int j = 0; j < CB; ++j) {
            if constexpr (BITS == 8) {
                if (i == 0) {
                    const float sc = ldexpf(d.s[j], -ew);
                    const half2v scv = {static_cast<_Float16>(sc), static_cast<_Float16>(sc)};
                    uint32_t off = 0xE480E480u;  // -1152
                    if constexpr (ZP) {
                        const uint32_t zz = ((d.z[j] >> z_shift[j]) & 0xFFu) * 0x00010001u;
                        off = (zz ^ 0x00800080u) + 0xE400E400u;
                    }
                    d.s[j] = __builtin_bit_cast(float, scv);
                    d.z[j] = off;
                }
                const half2v scv = __builtin_bit_cast(half2v, d.s[j]);
                const half2v ofv = as_h2(d.z[j]);
                uint32_t h[4];
#pragma unroll
                for (int dw = 0; dw < 2; ++dw) {
                    // the bytes b ^ 0x80 under 0x64: the halves 1152 + q (one XOR for four bytes,
                    // then one permute a pair)
                    const uint32_t wv = d.w[j][2 * i + dw] ^ 0x80808080u;
                    const uint32_t p0 = __builtin_amdgcn_perm(0x64646464u, wv, 0x04010400u);
                    const uint32_t p1 = __builtin_amdgcn_perm(0x64646464u, wv, 0x04030402u);
                    h[2 * dw] = __builtin_bit_cast(uint32_t, (as_h2(p0) + ofv) * scv);
                    h[2 * dw + 1] = __builtin_bit_cast(uint32_t, (as_h2(p1) + ofv) * scv);
                }
                b[j] = __builtin_bit_cast(half8, u32x4{h[0], h[1], h[2], h[3]});
            } else {
                if (i == 0) {
                    const float sc = ldexpf(d.s[j], -ew);
                    const float sh = ldexpf(d.s[j], -ew - 4);  // high nibbles enter as 1024 + 16 q
                    const half2v lh = {static_cast<_Float16>(sc), static_cast<_Float16>(sh)};
                    d.s[j] = __builtin_bit_cast(float, lh);
                    d.z[j] = ((d.z[j] >> z_shift[j]) & 0xFFu) * 0x00010001u;
                }
                const half2v lh = __builtin_bit_cast(half2v, d.s[j]);
                const half2v scl = {lh[0], lh[0]}, sch = {lh[1], lh[1]};
                const uint32_t zz = d.z[j];
                const uint32_t mlo = in_vgpr(0x000F000Fu), mhi = in_vgpr(0x00F000F0u), e1024 = in_vgpr(0x64006400u);
                const half2v ofl = as_h2(zz | 0xE400E400u), ofh = as_h2((zz << 4) | 0xE400E400u);
                const uint32_t wv = d.w[j][i];
                const uint32_t p01 = __builtin_amdgcn_perm(0u, wv, SEL01), p23 = __builtin_amdgcn_perm(0u, wv, SEL23);
                const uint32_t h0 = __builtin_bit_cast(uint32_t, (as_h2((p01 & mlo) | e1024) + ofl) * scl);
                const uint32_t h1 = __builtin_bit_cast(uint32_t, (as_h2((p23 & mlo) | e1024) + ofl) * scl);
                const uint32_t h2 = __builtin_bit_cast(uint32_t, (as_h2((p01 & mhi) | e1024) + ofh) * sch);
                const uint32_t h3 = __builtin_bit_cast(uint32_t, (as_h2((p23 & mhi) | e1024) + ofh) * sch);
                b[j] = __builtin_bit_cast(half8, u32x4{h0, h1, h2, h3});
            }
        }
    };
    // The RB x CB products of sub-product i of one slab.
    auto multiply = [&](const PSlab<BITS, RB, CB>& d, int i, const half8 (&b)[CB]) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const half8 av = __builtin_bit_cast(half8, d.a[rb * 2 + i]);
#pragma unroll
            for (int j = 0; j < CB; ++j)
                acc[rb][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, b[j], acc[rb][j], 0, 0, 0);
        }
    };
    // Software pipeline. Step u multiplies slab set u: its first sub-product's MFMAs run while
    // the second sub-product is dequantized and the loads that refill the set freed by the
    // step before are issued; its second sub-product's MFMAs run while the next set's first
    // sub-product is dequantized. One MFMA, then a few vector ALU and memory instructions, in
    // turn (sched_group_barrier), so the matrix unit is not left idle while operands are
    // prepared and the loads go out spread over the step.
    half8 b0[CB], b1[CB];
    constexpr int NLOADS = 2 * RB + 2 * CB + (ZP ? CB : 0);  // vector memory instructions per slab
    constexpr int NMF = RB * CB;                             // MFMAs per sub-product
    constexpr int VPER = (20 * CB + NMF - 1) / NMF;          // dequantization VALU per MFMA (about)
    auto step = [&](PSlab<BITS, RB, CB>& d, PSlab<BITS, RB, CB>& nx, PSlab<BITS, RB, CB>& refill, int32_t refill_x) {
        multiply(d, 0, b0);
        dequant(d, 1, b1);
        load(refill, refill_x);  // past the end: the last slab again, never used
        static_for<0, NMF>([&](auto kc) {
            constexpr int k = decltype(kc)::value;
            constexpr int nl = NLOADS / NMF + (k < NLOADS % NMF ? 1 : 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                 // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, VPER - 1, 0);          // vector ALU
            if constexpr (nl > 0) __builtin_amdgcn_sched_group_barrier(0x020, nl, 0);  // loads
        });
        __builtin_amdgcn_sched_barrier(0);
        multiply(d, 1, b1);
        dequant(nx, 0, b0);
        static_for<0, NMF>([&](auto) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x002, VPER, 0);
        });
        __builtin_amdgcn_sched_barrier(0);
    };

    // Sets 0 .. PDEPTH - 2 are loaded here; step u loads set (u + PDEPTH - 1) % PDEPTH (the
    // one step u - 1 finished) with slab x + u + PDEPTH - 1.
    dequant(sl[0], 0, b0);
    __builtin_amdgcn_sched_barrier(0);
    int32_t x = 0;
    for (; x + PDEPTH <= n_mine; x += PDEPTH) {
#pragma unroll
        for (int u = 0; u < PDEPTH; ++u)
            step(sl[u], sl[(u + 1) % PDEPTH], sl[(u + PDEPTH - 1) % PDEPTH], x + u + PDEPTH - 1);
    }
    // the last slabs; the dequantization after the last one reads a loaded set and is not used
#pragma unroll
    for (int u = 0; u < PDEPTH; ++u)
        if (x + u < n_mine) step(sl[u], sl[(u + 1) % PDEPTH], sl[(u + PDEPTH - 1) % PDEPTH], x + u + PDEPTH - 1);

    // The waves' sums meet in LDS, a half of the tile (64 rows) at a time: each wave writes
    // its sums row-major (element (r, c) of a 32 x 32 block is in lane c + 32 ((r / 4) % 2),
    // register (r / 8) * 4 + r % 4), then each thread adds four consecutive columns of a row
    // over the waves in wave order and stores them with one 16-byte store. Any loads of old
    // outputs and biases are all issued before the first store (on gfx9 a wait for a load
    // also waits for every earlier store), and the copy without them has no load at all.
    // Buffer operations on the tile's rows: an element outside [M x N] (N % 4 == 0, so a
    // quad is inside or outside whole) gets an offset past the buffer, where loads read 0
    // and stores are dropped.
    float* out = jb.partials ? jb.partials + static_cast<size_t>(sp) * M * N : jb.c;
    const bool add = !jb.partials && accumulate;
    const float* bs = jb.partials ? nullptr : jb.bias;
    const float al = jb.partials ? 1.0f : alpha;
    const __amdgpu_buffer_rsrc_t orr = __builtin_amdgcn_make_buffer_rsrc(
        out + static_cast<size_t>(m0) * N, 0, static_cast<uint32_t>(min(M - m0, TM)) * N * 4, 0x00020000);
    float* mt = reinterpret_cast<float*>(meet);  // [wave][64 rows][MPITCH]
    constexpr int QPR = TN / 4, RPI = PTHREADS / QPR, ITEMS = 64 / RPI;  // quads a row, rows an item, items
    const int32_t c4 = t % QPR, rsub = t / QPR;  // this thread's column quad and row within RPI
#pragma unroll
    for (int half = 0; half < TM / 64; ++half) {
        __syncthreads();  // er_s written; the previous half's meet read
#pragma unroll
        for (int rl = 0; rl < 2; ++rl)
#pragma unroll
            for (int j = 0; j < CB; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int32_t r = rl * 32 + (e >> 2) * 8 + (ln >> 5) * 4 + (e & 3);
                    mt[(wave * 64 + r) * MPITCH + j * 32 + (ln & 31)] = acc[half * 2 + rl][j][e];
                }
        __syncthreads();
        // item it: row it * RPI + rsub of the half, columns 4 c4 .. 4 c4 + 3
        auto offset = [&](int it) -> uint32_t {
            const int32_t rt = half * 64 + it * RPI + rsub;  // tile row
            return m0 + rt < M && col0 + 4 * c4 < N ? static_cast<uint32_t>(rt * N + col0 + 4 * c4) * 4u : 0x80000000u;
        };
        auto total = [&](int it) -> f32x4 {
            const int32_t r = it * RPI + rsub;
            const int32_t idx = r * MPITCH + 4 * c4;
            f32x4 v = *reinterpret_cast<const f32x4*>(mt + idx);
#pragma unroll
            for (int w = 1; w < 4; ++w) v += *reinterpret_cast<const f32x4*>(mt + w * 64 * MPITCH + idx);
            return v * ldexpf(1.0f, er_s[half * 64 + r] + ew);
        };
        auto store = [&](auto loads) {
            constexpr bool LOADS = decltype(loads)::value;
            f32x4 old[ITEMS];
            f32x4 bv = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            if constexpr (LOADS) {
                if (bs) bv = *reinterpret_cast<const f32x4*>(bs + min(col0 + 4 * c4, N - 4));
#pragma unroll
                for (int it = 0; it < ITEMS; ++it)
                    old[it] = add ? __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(orr, offset(it), 0, 0))
                                  : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
#pragma unroll
            for (int it = 0; it < ITEMS; ++it) {
                const f32x4 sm = total(it);
                f32x4 v;
#pragma unroll
                for (int c = 0; c < 4; ++c) v[c] = LOADS ? fmaf(al, sm[c], old[it][c]) + bv[c] : al * sm[c];
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), orr, offset(it), 0, 0);
            }
        };
        if (add || bs) store(std::true_type{});
        else store(std::false_type{});
    }
}
}  // namespace

bool gemm_supported(const float* a, int32_t m, const WeightView& w, const float* c) {
    (void)a;
    (void)m;
    if (w.g % WROWS != 0) return false;  // a thread's weight rows share one group
    if (w.N % (w.bits == 4 ? 8 : 4) != 0) return false;  // whole 4-byte column quads
    return aligned(w.q, 4) && aligned(w.s, 16) && (!w.z || aligned(w.z, 4)) && aligned(c, 16);
}

// The job table of a launch: column tiles of `tile_cols` columns (value columns for the
// column-run kernel, byte columns for gemm_kernel), scale slices for the maxima.
static void fill_jobs(GemmJobs& jobs, const WeightView* ws, float* const* cs, const float* const* biases, int32_t count,
                      int32_t tile_cols, bool value_columns, int32_t splits, int32_t m, int32_t* nsb_total,
                      size_t* part_elems) {
    jobs = GemmJobs{};
    jobs.count = count;
    int32_t tile_begin = 0;
    *nsb_total = 0;
    *part_elems = 0;
    for (int32_t i = 0; i < count; ++i) {
        GemmJob& jb = jobs.job[i];
        jb.q = ws[i].q;
        jb.p = ws[i].p;
        jb.pmax = ws[i].p ? packed_scale_max(ws[i]) : nullptr;
        jb.s = ws[i].s;
        jb.z = ws[i].z;
        jb.c = cs[i];
        jb.bias = biases ? biases[i] : nullptr;
        jb.N = ws[i].N;
        jb.bpr = ws[i].bpr;
        jb.tile_begin = tile_begin;
        tile_begin += ceil_div(value_columns ? ws[i].N : ws[i].bpr, tile_cols);
        jb.scale_quads = static_cast<int64_t>(ws[i].G) * ws[i].N / 4;
        int64_t nsb64 = (jb.scale_quads + 2047) / 2048;  // at least 8 quads per thread
        if (nsb64 < 1) nsb64 = 1;
        if (nsb64 > MAX_SCALE_BLOCKS) nsb64 = MAX_SCALE_BLOCKS;
        jb.nsb = static_cast<int32_t>(nsb64);
        jb.smax_begin = *nsb_total;
        *nsb_total += jb.nsb;
        if (splits > 1) *part_elems += static_cast<size_t>(splits) * m * ws[i].N;
    }
}

// The column-run kernel: every weight of the group has its copy, g % 32 == 0, and INT4
// weights have zero points (as every INT4 quantization does); the copy and the scales are
// addressed with 32-bit buffer offsets, so each stays below 4 GiB.
static bool gemm_packed_usable(const WeightView* ws, int32_t count) {
    for (int32_t i = 0; i < count; ++i) {
        if (!ws[i].p || ws[i].g % 32 != 0 || log2_exact(ws[i].g / 32) < 0 || (ws[i].bits == 4 && !ws[i].z)) return false;
        if (packed_weight_bytes(ws[i].K, ws[i].N, ws[i].bits) > 0xFFFFFFFFll) return false;
        if (static_cast<int64_t>(ws[i].G) * ws[i].N * 4 > 0xFFFFFFFFll) return false;
    }
    return true;
}

// The launch of one tile shape: the prep (a in the tiled fp16 order of TM-row tiles, the
// scale maxima), the kernel, and the slices' reduction when K is split.
template <int TM, int TN, int PD>
static int32_t launch_gemm_packed_tiles(const float* a, int32_t m, const WeightView* ws, float* const* cs,
                                        const float* const* biases, int32_t count, int32_t accumulate, float alpha,
                                        hipStream_t st) {
    const WeightView& w = ws[0];
    const int32_t Mp = ceil_div(m, TM) * TM;
    const int32_t chunks = ceil_div(w.K, 128);
    const int32_t S = chunks * 4;
    int32_t tiles_n = 0;
    for (int32_t i = 0; i < count; ++i) tiles_n += ceil_div(ws[i].N, TN);
    const int32_t tiles_m = Mp / TM;
    // Split K (in whole 128-k chunks, at least two per slice) when the tiles leave CUs
    // idle, into as many slices as keep one round of workgroups (one per CU).
    int32_t splits = 1;
    const int64_t tiles = static_cast<int64_t>(tiles_m) * tiles_n;
    const int32_t cus = cu_count();
    if (tiles < cus) splits = static_cast<int32_t>(cus / tiles);
    const int32_t cap = chunks / 2 > 1 ? chunks / 2 : 1;
    if (splits > cap) splits = cap;
    if (splits > MAX_SPLITS) splits = MAX_SPLITS;
    const int32_t chunks_per_split = ceil_div(chunks, splits);
    splits = ceil_div(chunks, chunks_per_split);

    GemmJobs jobs;
    int32_t nsb_total = 0;  // the scale maxima come from the copies' trailers: no scale blocks
    size_t part_elems = 0;
    fill_jobs(jobs, ws, cs, biases, count, TN, true, splits, m, &nsb_total, &part_elems);
    auto round256 = [](size_t b) { return (b + 255) & ~size_t(255); };
    const size_t a16_bytes = round256(static_cast<size_t>(Mp) * S * 64);
    const size_t er_bytes = round256(static_cast<size_t>(Mp) * 4);
    void* wsp = nullptr;
    int32_t status = workspace(st, a16_bytes + er_bytes + part_elems * sizeof(float), &wsp);
    if (status) return status;
    char* base = static_cast<char*>(wsp);
    _Float16* a16t = reinterpret_cast<_Float16*>(base);
    int32_t* er = reinterpret_cast<int32_t*>(base + a16_bytes);
    float* part = reinterpret_cast<float*>(base + a16_bytes + er_bytes);
    for (int32_t i = 0; i < count && splits > 1; ++i) {
        jobs.job[i].partials = part;
        part += static_cast<size_t>(splits) * m * ws[i].N;
    }
    const int32_t vec_rows = (w.K % 4 == 0 && aligned(a, 16)) ? 1 : 0;
    if (S > 128 && S <= 512) {  // a workgroup per row
        if (w.bits == 4) gemm_prep_tiled_long<4, TM><<<Mp, 256, 0, st>>>(a, m, w.K, S, vec_rows, a16t, er);
        else gemm_prep_tiled_long<8, TM><<<Mp, 256, 0, st>>>(a, m, w.K, S, vec_rows, a16t, er);
    } else {
        const uint32_t prep_blocks = static_cast<uint32_t>(Mp / 4);
        if (w.bits == 4)
            gemm_prep_tiled<4, TM><<<prep_blocks, 256, 0, st>>>(a, m, w.K, S, vec_rows, Mp, a16t, er);
        else
            gemm_prep_tiled<8, TM><<<prep_blocks, 256, 0, st>>>(a, m, w.K, S, vec_rows, Mp, a16t, er);
    }
    KT_LAUNCHED("qmatmul: tiled gemm prep");
    constexpr size_t lds = plds_bytes(TN);
    static bool raised = false;
    if (!raised && lds > LDS_DEFAULT) {  // the meet is beyond the default dynamic LDS limit (exactly
        // what it needs: the kernel's static LDS comes on top)
        KT_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_packed_kernel<4, true, TM, TN, PD>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
        KT_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_packed_kernel<8, true, TM, TN, PD>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
        KT_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_packed_kernel<8, false, TM, TN, PD>),
                                   hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));
        raised = true;
    }
    const uint32_t blocks = static_cast<uint32_t>(ceil_div(tiles_n, XCDS) * XCDS * tiles_m * splits);
#define KT_GEMM_ARGS a16t, er, jobs, m, w.K, S, w.g, tiles_m, tiles_n, splits, chunks_per_split * 4, alpha, accumulate
    if (w.bits == 4) gemm_packed_kernel<4, true, TM, TN, PD><<<blocks, PTHREADS, lds, st>>>(KT_GEMM_ARGS);
    else if (w.z) gemm_packed_kernel<8, true, TM, TN, PD><<<blocks, PTHREADS, lds, st>>>(KT_GEMM_ARGS);
    else gemm_packed_kernel<8, false, TM, TN, PD><<<blocks, PTHREADS, lds, st>>>(KT_GEMM_ARGS);
#undef KT_GEMM_ARGS
    KT_LAUNCHED("qmatmul: packed gemm kernel");
    for (int32_t i = 0; i < count && splits > 1; ++i) {
        const size_t total = static_cast<size_t>(m) * ws[i].N;
        gemm_reduce<<<static_cast<uint32_t>((total + 255) / 256), 256, 0, st>>>(
            jobs.job[i].partials, splits, m, ws[i].N, cs[i], biases ? biases[i] : nullptr, alpha, accumulate);
        KT_LAUNCHED("qmatmul: gemm reduce");
    }
    return KT_OK;
}

constexpr int GEMM_NARROW_DEPTH = 5;  // the 64 x 64 tile's ring (3, 5, 8 measured alike; 5 a little ahead)
// Tile shape: 64-row tiles when M <= 64 (a 128-row tile would be half padding), and up to
// M = 128 while 64 x 64 tiles make one round of workgroups with K <= 8192 (2048 -> 8192
// INT8 g32 M = 128: 20.5 -> 15.6 us, 128-row tiles needing a K split there; 4096 -> 4096
// 20.9 -> 19.9; two rounds, 4096 -> 14336, 31.5 -> 35.4, and K = 14336, 35.4 -> 36.2,
// stay with 128 rows); 64-column tiles when 128-column ones number fewer than the CUs.
static int32_t launch_gemm_packed(const float* a, int32_t m, const WeightView* ws, float* const* cs,
                                  const float* const* biases, int32_t count, int32_t accumulate, float alpha,
                                  hipStream_t st) {
    int64_t tiles64 = 0;
    for (int32_t i = 0; i < count; ++i) tiles64 += ceil_div(ws[i].N, 64);
    tiles64 *= ceil_div(m, 64);
    const bool rows64 = m <= 64 || (m <= 128 && tiles64 <= cu_count() && ws[0].K <= 8192);
    int64_t tiles128 = 0;
    for (int32_t i = 0; i < count; ++i) tiles128 += ceil_div(ws[i].N, 128);
    tiles128 *= ceil_div(m, rows64 ? 64 : 128);
    const bool cols64 = tiles128 < cu_count();
    if (rows64 && cols64)
        return launch_gemm_packed_tiles<64, 64, GEMM_NARROW_DEPTH>(a, m, ws, cs, biases, count, accumulate, alpha, st);
    if (rows64) return launch_gemm_packed_tiles<64, 128, 3>(a, m, ws, cs, biases, count, accumulate, alpha, st);
    if (cols64) return launch_gemm_packed_tiles<128, 64, 3>(a, m, ws, cs, biases, count, accumulate, alpha, st);
    return launch_gemm_packed_tiles<128, 128, 3>(a, m, ws, cs, biases, count, accumulate, alpha, st);
}

int32_t launch_gemm_group(const float* a, int32_t m, const WeightView* ws, float* const* cs, const float* const* biases,
                          int32_t count, int32_t accumulate, float alpha, hipStream_t st) {
    if (count < 1 || count > MAX_GEMM_JOBS) return fail(KT_ERR_ARGUMENT, "gemm: 1 to %d weights, got %d", MAX_GEMM_JOBS, count);
    const WeightView& w = ws[0];
    for (int32_t i = 1; i < count; ++i)
        if (ws[i].K != w.K || ws[i].bits != w.bits || ws[i].g != w.g || (ws[i].z != nullptr) != (w.z != nullptr))
            return fail(KT_ERR_ARGUMENT, "gemm: grouped weights must share rows, bits, group size and zero points");
    if (gemm_packed_usable(ws, count)) return launch_gemm_packed(a, m, ws, cs, biases, count, accumulate, alpha, st);
    const int32_t Mp = ceil_div(m, BM) * BM;
    const int32_t Kp = ceil_div(w.K, BK) * BK;
    const int32_t tile_bytes = w.bits == 8 ? BN : BN / 2;
    int32_t tiles_n = 0;
    for (int32_t i = 0; i < count; ++i) tiles_n += ceil_div(ws[i].bpr, tile_bytes);
    const int32_t tiles_m = Mp / BM;
    const int32_t k_steps = Kp / BK;
    // Split K when the tile grid leaves CUs idle, keeping at least 4 steps per slice.
    int32_t splits = 1;
    const int64_t tiles = static_cast<int64_t>(tiles_m) * tiles_n;
    const int32_t cus = cu_count();
    if (tiles < cus) splits = static_cast<int32_t>((cus + tiles - 1) / tiles);
    const int32_t cap = k_steps / 4 > 1 ? k_steps / 4 : 1;
    if (splits > cap) splits = cap;
    if (splits > MAX_SPLITS) splits = MAX_SPLITS;
    const int32_t steps_per_split = ceil_div(k_steps, splits);
    splits = ceil_div(k_steps, steps_per_split);  // every slice has at least one step

    GemmJobs jobs;
    int32_t nsb_total = 0;
    size_t part_elems = 0;
    fill_jobs(jobs, ws, cs, biases, count, tile_bytes, false, splits, m, &nsb_total, &part_elems);

    auto round256 = [](size_t b) { return (b + 255) & ~size_t(255); };
    const size_t a16_bytes = round256(static_cast<size_t>(Mp) * Kp * sizeof(_Float16));
    const size_t er_bytes = round256(static_cast<size_t>(Mp) * 4);
    const size_t smax_bytes = round256(static_cast<size_t>(nsb_total) * 4);
    const size_t part_bytes = part_elems * sizeof(float);
    void* wsp = nullptr;
    int32_t status = workspace(st, a16_bytes + er_bytes + smax_bytes + part_bytes, &wsp);
    if (status) return status;
    char* base = static_cast<char*>(wsp);
    _Float16* a16 = reinterpret_cast<_Float16*>(base);
    int32_t* er = reinterpret_cast<int32_t*>(base + a16_bytes);
    float* smax = reinterpret_cast<float*>(base + a16_bytes + er_bytes);
    float* part = reinterpret_cast<float*>(base + a16_bytes + er_bytes + smax_bytes);
    for (int32_t i = 0; i < count && splits > 1; ++i) {
        jobs.job[i].partials = part;
        part += static_cast<size_t>(splits) * m * ws[i].N;
    }

    const int32_t vec_rows = (w.K % 4 == 0 && aligned(a, 16)) ? 1 : 0;
    gemm_prep<<<Mp + nsb_total, 256, 0, st>>>(a, m, w.K, Kp, vec_rows, Mp, jobs, a16, er, smax);
    KT_LAUNCHED("qmatmul: gemm prep");
    // Weight tiles dealt to the XCDs (padded to a multiple of 8), each with its row tiles
    // and K slices.
    const uint32_t blocks = static_cast<uint32_t>(ceil_div(tiles_n, XCDS) * XCDS * tiles_m * splits);
#define KT_GEMM_ARGS a16, Kp, er, smax, jobs, m, w.K, w.g, tiles_m, tiles_n, splits, steps_per_split, alpha, accumulate
    const bool fast = w.K % BK == 0 && (BK % w.g == 0 || w.g % BK == 0);
    if (w.bits == 4)
        fast ? gemm_kernel<4, true, true><<<blocks, THREADS, 0, st>>>(KT_GEMM_ARGS)
             : gemm_kernel<4, true, false><<<blocks, THREADS, 0, st>>>(KT_GEMM_ARGS);
    else if (w.z)
        fast ? gemm_kernel<8, true, true><<<blocks, THREADS, 0, st>>>(KT_GEMM_ARGS)
             : gemm_kernel<8, true, false><<<blocks, THREADS, 0, st>>>(KT_GEMM_ARGS);
    else
        fast ? gemm_kernel<8, false, true><<<blocks, THREADS, 0, st>>>(KT_GEMM_ARGS)
             : gemm_kernel<8, false, false><<<blocks, THREADS, 0, st>>>(KT_GEMM_ARGS);
#undef KT_GEMM_ARGS
    KT_LAUNCHED("qmatmul: gemm kernel");
    for (int32_t i = 0; i < count && splits > 1; ++i) {
        const size_t total = static_cast<size_t>(m) * ws[i].N;
        gemm_reduce<<<static_cast<uint32_t>((total + 255) / 256), 256, 0, st>>>(
            jobs.job[i].partials, splits, m, ws[i].N, cs[i], biases ? biases[i] : nullptr, alpha, accumulate);
        KT_LAUNCHED("qmatmul: gemm reduce");
    }
    return KT_OK;
}

int32_t launch_gemm(const float* a, int32_t m, const WeightView& w, float* c, int32_t accumulate, float alpha,
                    const float* bias, hipStream_t st) {
    const float* biases[1] = {bias};
    return launch_gemm_group(a, m, &w, &c, biases, 1, accumulate, alpha, st);
}

}  // namespace kt
