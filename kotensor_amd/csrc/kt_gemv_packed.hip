// kt_gemv_packed.hip -- the one-row dequant-GEMV on a device-native copy of the packed
// weights, and the kernel that writes that copy:
//   c[1 x N] = (accumulate ? c : 0) + alpha * x[1 x K] . deq(W) (+ bias),
// MatMul.multiplyQuantizedRow (Engine/kotensor/src/main/kotlin/MatMul.kt:494-536).
//
// Why a second layout. In the reference layout ([K x bytesPerRow], a row of the weight
// is contiguous) a workgroup that owns a strip of columns must read all K rows of it,
// and at shapes like 4096 -> 14336 there are too few strips to occupy 256 CUs: the K
// range has to be split over workgroups whose partial sums then meet through memory,
// several dependent round trips after the last load. In the column-run layout a column's
// K values are contiguous, so a workgroup owns whole columns over all of K: no sums
// leave it, every load instruction reads 1 KB of consecutive bytes, and the number of
// workgroups is set by N alone. The copy is made once per weight (kt_qweight_pack) next
// to the reference bytes, which stay the format of record (quantize, files, accessors
// and the M > 1 kernels read them).
//
// Layout (a column set is 16 columns, a chunk 128 k; block = column set x chunk):
//   blocks are ordered [column set][chunk]; INT4 blocks are 1 KB, INT8 blocks 2 KB;
//   within a block, lane l = 16 kb + n of the reading wave owns the 16 bytes at
//   16 l (INT8: and at 1024 + 16 l): column 16 set + n, the 32 k of run
//   [128 chunk + 32 kb, + 32). INT8: byte b of the first 16 is k = run + b, of the
//   second k = run + 16 + b. INT4: dword d = 2 m + h of the 16 bytes holds, in byte t,
//   k = run + 16 m + 8 h + t in the low nibble and k = run + 16 m + 8 h + 4 + t in the
//   high one, so that (d & 0x0F0F0F0F) and (d >> 4) & 0x0F0F0F0F are the int8 values
//   of k = run + 16 m + 8 h + 0..3 and + 4..7. Padding (k >= K, columns >= N) is 0.
//
// Arithmetic (integer-exact products, then the reference's per-group combine):
//   * x is cut into runs of 32 k. With E the binary exponent of the run's largest |x|
//     (largest |x| < 2^E), X = (int)(x * 2^(30 - E)) holds x to 2^-30 of that maximum,
//     and X = d0 + 2^8 d1 + 2^16 d2 + 2^24 d3 with signed byte digits (the bytes of
//     ((X + 0x808080) ^ 0x808080)). The four digit rows of every run go to LDS;
//   * v_mfma_i32_16x16x64_i8 with a block-diagonal A: lane group kb of B holds its own
//     run's 16 k of 16 columns, A row 4 kb + p holds digit p of that run's x (rows of
//     other lane groups' runs are 0), so one MFMA gives every lane group the four digit
//     sums of its own run: D_p = sum d_p q, exact in int32 (two MFMAs per run);
//   * per run: u = (D_2 + 256 D_3) + (D_0 + 256 D_1) / 2^16 (digit pairs added in int32,
//     then one fp32 fma), sum x q = u * 2^(E - 14), and y += scale * (sum x q - zero *
//     sum x): the reference's combineGroup, scale * (acc - zero * rowSum)
//     (MatMul.kt:804-828), applied per run;
//   * K is cut into eight fixed sub-parts (kt_packed.h); a sub-part's sum is its lanes'
//     runs in K order, then the column's four lanes, and the sub-parts add in a fixed
//     balanced tree, whose lower levels the wave covering them forms and whose top the
//     waves that split K form in LDS.
// A column's result therefore depends only on x and that column's weights, never on
// how the columns or the K range are divided among waves.
#include "kt_common.h"
#include "kt_packed.h"
#include <algorithm>
#include <atomic>
#include <type_traits>

namespace kt {
namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int MAX_JOBS = 4;
constexpr int MAX_K = 16384;  // eight waves of at most 2048 k each
constexpr int ZERO_BYTES = 32;


// The s_waitcnt immediate that waits until at most n vector memory operations are
// outstanding (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt and lgkmcnt left at
// their maxima so they do not wait).
__host__ __device__ constexpr int vmcnt_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

struct PJob {
    const uint8_t* packed;
    const float* s;   // the copy's scale rows [set][group][16]
    const int8_t* z;  // the copy's zero-point rows (null: no zero points)
    float* out;
    const float* bias;
    int32_t N, sets;
};

struct PJobs {
    PJob job[MAX_JOBS];
    int32_t count;
};

// Writes the column-run copy: one thread per output dword.
__global__ void __launch_bounds__(256)
    pack_kernel(const uint8_t* __restrict__ q, int32_t K, int32_t N, int32_t bits, int32_t bpr, int32_t chunks,
                int64_t dwords, uint32_t* __restrict__ out) {
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < dwords;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const int dw_per_block = block_bytes(bits) / 4;
        const int64_t blk = i / dw_per_block;
        const int within = static_cast<int>(i - blk * dw_per_block);
        const int32_t set = static_cast<int32_t>(blk / chunks);
        const int32_t chunk = static_cast<int32_t>(blk - static_cast<int64_t>(set) * chunks);
        uint32_t v = 0;
        if (bits == 4) {
            const int lane = within >> 2, d = within & 3;
            const int32_t col = set * SET + (lane & 15);
            const int32_t k0 = chunk * CHUNK + (lane >> 4) * RUN + 16 * (d >> 1) + 8 * (d & 1);
            if (col < N) {
                const int32_t byte_col = col < bpr ? col : col - bpr;
                const int shift = col < bpr ? 0 : 4;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int32_t kl = k0 + t, kh = k0 + 4 + t;
                    const uint32_t lo = kl < K ? (q[static_cast<int64_t>(kl) * bpr + byte_col] >> shift) & 15u : 0u;
                    const uint32_t hi = kh < K ? (q[static_cast<int64_t>(kh) * bpr + byte_col] >> shift) & 15u : 0u;
                    v |= (lo | (hi << 4)) << (8 * t);
                }
            }
        } else {
            const int h = within >> 8, lane = (within >> 2) & 63, d = within & 3;
            const int32_t col = set * SET + (lane & 15);
            const int32_t k0 = chunk * CHUNK + (lane >> 4) * RUN + 16 * h + 4 * d;
            if (col < N) {
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int32_t k = k0 + t;
                    const uint32_t b = k < K ? q[static_cast<int64_t>(k) * bpr + col] : 0u;
                    v |= b << (8 * t);
                }
            }
        }
        out[i] = v;
    }
}

// Writes the copy's scale and zero-point rows: [column set][group][16] fp32 scales, then
// [column set][group][16] zero points (0 without zero points, and past the last column);
// and the largest |scale| into the trailer word smax (zero beforehand): fmaxf's maximum
// (NaNs ignored, infinities kept), as the bits of a non-negative float, whose unsigned
// order is the float order, by one atomic maximum per workgroup (order-free).
__global__ void __launch_bounds__(256)
    pack_scales_kernel(const float* __restrict__ s, const int8_t* __restrict__ z, int32_t G, int32_t N, int64_t rows,
                       float* __restrict__ ps, int8_t* __restrict__ pz, uint32_t* smax) {
    __shared__ uint32_t red[4];
    uint32_t mx = 0u;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < rows;
         i += static_cast<int64_t>(gridDim.x) * 256) {
        const int64_t set_group = i / SET;
        const int32_t n = static_cast<int32_t>(i - set_group * SET);
        const int32_t set = static_cast<int32_t>(set_group / G);
        const int32_t grp = static_cast<int32_t>(set_group - static_cast<int64_t>(set) * G);
        const int32_t col = set * SET + n;
        const int64_t at = static_cast<int64_t>(grp) * N + col;
        const float v = col < N ? s[at] : 0.0f;
        ps[i] = v;
        pz[i] = z && col < N ? z[at] : static_cast<int8_t>(0);
        const uint32_t b = __float_as_uint(fabsf(v));
        mx = b <= 0x7F800000u ? max(mx, b) : mx;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = max(mx, static_cast<uint32_t>(__shfl_xor(static_cast<int>(mx), o, 64)));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
    __syncthreads();
    if (threadIdx.x == 0) {
        mx = max(max(red[0], red[1]), max(red[2], red[3]));
        __hip_atomic_fetch_max(smax, mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Zeroes the copy's 16-byte trailer before the maximum is taken into its first word.
__global__ void zero_trailer(uint32_t* w) {
    if (threadIdx.x < PACKED_TRAILER_BYTES / 4) w[threadIdx.x] = 0u;
}

// Max over the 8 lanes of an aligned group (quad swaps, then the half-row mirror).
__device__ __forceinline__ float max8(float v) {
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false)));
    v = fmaxf(v, __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false)));
    return v;
}
// Sum over the same 8 lanes, in the same fixed pattern (lane 8 q's value is the one used).
__device__ __forceinline__ float sum8(float v) {
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
    v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
    return v;
}

// The input row: X_PLAIN x; X_SWIGLU silu(x) * aux (the SwiGLU gate computed as
// silu_mul_kernel does, x / (1 + exp(-x)) with exp in double rounded to float, times up);
// X_NORM x * aux with the result scaled by r = 1 / sqrt(mean(x^2) + eps), RMSNorm with
// weight aux (K/RMSNorm.kt:71-90), the sum of squares taken by the waves that split K
// and added in K-part order (fp32 rounding apart from rmsnorm_kernel's order).
constexpr int X_PLAIN = 0, X_SWIGLU = 1, X_NORM = 2;


// A workgroup of W = 8 waves owns W / ks column sets over all of K; each wave streams
// one column set over one of the ks K-parts. The workgroup first turns all of x into
// digits together (every wave a slice of K, the loads ahead of the weights), meets once
// at a barrier, and from then on every wave streams its own chunks without waiting for
// another; the K-parts of a column set add in fixed order in LDS at the end. (Digits made
// by each wave for its own K-part alone, or units of one wave meeting through memory,
// were measured slower: more x traffic ahead of the first weights, or a memory round trip
// after the last.)

constexpr int W = 8;                  // waves per workgroup
constexpr int X_SLOTS = MAX_K / (256 * W);  // float4s of x per thread

// The workgroup's LDS: digit rows [4][kp] (kp = 128 chunks bytes), 32 zero bytes, run
// records [4 chunks] x 8 bytes, the meeting area: [W][16] sums and [W] sums of squares,
// then each wave's staged scales and zero points: rows [stage_rows][16] fp32, then
// [stage_rows][16] bytes (the quantization groups its K range touches, its 16 columns).
__host__ __device__ constexpr int32_t lds_rec_offset(int32_t chunks) { return 4 * chunks * CHUNK + ZERO_BYTES; }
__host__ __device__ constexpr int32_t lds_red_offset(int32_t chunks) { return lds_rec_offset(chunks) + chunks * (CHUNK / RUN) * 8; }
__host__ __device__ constexpr int32_t lds_stage_offset(int32_t chunks) {
    return (lds_red_offset(chunks) + W * (SET + 1) * 4 + 15) & ~15;
}
__host__ __device__ constexpr int32_t lds_bytes(int32_t chunks, int32_t nmax, int32_t gshift) {
    return lds_stage_offset(chunks) + W * stage_rows(nmax, gshift) * STAGE_ROW_BYTES;
}

// A stage of a chained launch (gemv_chain_kernel): the workgroup issues its first weight
// loads, waits until every partition of the previous stage has raised its flag (the first
// stage waits for nothing), then reads its input row; when its outputs are stored it
// counts itself in. Device-scope atomics on one address run one at a time (tens of ns
// each), so a stage's workgroups count in CHAIN_PARTS partition counters, each on its own
// line; the last workgroup of a partition returns the counter to zero and raises the
// partition's flag, and waiting workgroups read the flags (one lane each). A stage's flags
// are lowered two stages on, by the first workgroup of stage s + 2 once it is past its own
// wait (every workgroup of stage s + 1 is then past the flags). The last stage has no
// waiters: its partitions' last workgroups count into one stage counter instead, and the
// last of those lowers the previous stage's flags. Every word is zero when the launch ends.
constexpr int CHAIN_PARTS = 16;
constexpr int CHAIN_STRIDE = 32;  // words between counters and flags: one 128-byte line each
constexpr int CHAIN_WORDS = (2 * CHAIN_PARTS + 1) * CHAIN_STRIDE;  // per stage
constexpr int CHAIN_BASE = 8192;  // the chain's words start here in the stream's counters
constexpr uint32_t CHAIN_SPIN_LIMIT = 1u << 22;  // polls before a wait gives up (a fault, not a schedule)

struct ChainLink {
    int32_t* fault;         // the stream's fault word (or null): set when the wait gives up
    uint32_t spin_limit;    // polls before the wait gives up
    int32_t withhold;       // test hook: never raise the partition flags
    uint32_t* wait_flags;   // the previous stage's partition flags (null: the first stage)
    uint32_t* lower_flags;  // stage s - 2's flags, lowered by the stage's first workgroup (or null)
    uint32_t* part_count;   // this workgroup's partition counter
    uint32_t* part_flag;    // its flag (null: the last stage)
    uint32_t* stage_count;  // the last stage's counter
    uint32_t* last_lower;   // the last stage: the previous stage's flags, lowered at the end
    uint32_t wait_parts, lower_parts, last_lower_parts;
    uint32_t part_size, parts;  // workgroups in this partition; partitions of this stage
};

__device__ __forceinline__ void lower_chain_flags(uint32_t* flags, uint32_t parts) {
    for (uint32_t p = 0; p < parts; ++p)
        __hip_atomic_store(flags + p * CHAIN_STRIDE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Ordering. What one stage hands the next (its output row) is written with system-scope
// stores, which write through the caches; chain_signal makes every wave wait until its
// own stores are complete (s_waitcnt 0, behind a release fence that keeps the compiler
// from sinking a store past it) before the workgroup barrier, so the partition counter
// is incremented, and the flag raised, only after every output store of the partition
// is in memory. The waiter's flag loads are system-scope (past the caches); its input
// loads are issued only after the flags' values were seen (the loop's exit depends on
// them, then a barrier and an acquire fence keep the compiler from hoisting a load),
// and those loads read past the caches too, so they see the stored row.
__device__ __forceinline__ void chain_wait(const ChainLink& link) {
    if (!link.wait_flags) return;
    if (threadIdx.x < 64) {  // wave 0: lane p reads partition p's flag
        const uint32_t ln = threadIdx.x;
        uint32_t spins = 0;
        bool gave_up = false;
        while (true) {
            const uint32_t v = ln < link.wait_parts ? __hip_atomic_load(link.wait_flags + ln * CHAIN_STRIDE,
                                                                        __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM)
                                                    : 1u;
            if (__all(v != 0u)) break;
            if (++spins >= link.spin_limit) {
                gave_up = true;
                break;
            }
            __builtin_amdgcn_s_sleep(2);
        }
        if (gave_up && threadIdx.x == 0 && link.fault)
            __hip_atomic_store(link.fault, FAULT_CHAIN_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        if (threadIdx.x == 0 && link.lower_flags) lower_chain_flags(link.lower_flags, link.lower_parts);
    }
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

__device__ __forceinline__ void chain_signal(const ChainLink& link) {
    // this wave's write-through output stores are complete before the workgroup counts in
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x != 0) return;
    if (__hip_atomic_fetch_add(link.part_count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) != link.part_size - 1)
        return;
    __hip_atomic_store(link.part_count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (link.part_flag) {
        if (!link.withhold) __hip_atomic_store(link.part_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        return;
    }
    if (__hip_atomic_fetch_add(link.stage_count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) != link.parts - 1)
        return;
    __hip_atomic_store(link.stage_count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    if (link.last_lower) lower_chain_flags(link.last_lower, link.last_lower_parts);
}

// What crosses stages of a chain goes past the caches, so that no cache-wide write-back
// or invalidation is needed: outputs are written through (system-scope stores), and the
// input row and accumulated outputs are read from the coherence point (system-scope loads;
// the buffer loads' cache policy sc0 sc1).
constexpr int COHERENT = 1 | 16;
template <bool CHAIN>
__device__ __forceinline__ float load_out(const float* p) {
    if constexpr (CHAIN) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    else return *p;
}
template <bool CHAIN>
__device__ __forceinline__ void store_out(float* p, float v) {
    if constexpr (CHAIN) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    else *p = v;
}

// GLU: jobs 0 and 1 are SwiGLU's gate and up weights (same N); a workgroup's column sets
// are pairs (gate set s, up set s), and the gate wave's epilogue writes
// silu(gate) * up to job 0's output (silu_mul_kernel's expression) and up to job 1's.
// (bx, by) is the workgroup's place in the launch's own grid; CHAIN adds the hooks above.
template <int BITS, int R, bool ZP, int XMODE, bool GLU, bool CHAIN, int XS = X_SLOTS>
__device__ __forceinline__ void gemv_packed_body(const float* __restrict__ x, const float* __restrict__ aux, float eps,
                                                 int32_t K, int32_t gshift, const PJobs& jobs, int32_t kslog,
                                                 float alpha, int32_t accumulate, int32_t bx, int32_t by,
                                                 const ChainLink& link, int32_t out_row = 0) {
    constexpr int BB = block_bytes(BITS);
    constexpr int NB = BITS == 4 ? 1 : 2;  // 16-byte loads per lane and chunk
    extern __shared__ __attribute__((aligned(16))) unsigned char smem[];

    // Everything below is shifts and masks of the arguments (K-parts and group sizes are
    // powers of two), so the first loads go out one argument fetch after the start.
    // GLU: set slot my_cs holds weight my_cs % 2, column set my_cs / 2 of the pair range.
    // The job's fields are the first loads (first in the source: otherwise they wait for
    // kslog and the start costs a second scalar round trip).
    PJob jb = jobs.job[GLU ? (__builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & ((1 << (3 - kslog)) - 1) & 1)
                           : by];
    jb.out += static_cast<size_t>(out_row) * jb.N;  // (row out_row of a call's outputs)
    const int32_t tid = threadIdx.x, ln = tid & 63;
    const int32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int32_t cslog = 3 - kslog;  // column sets per workgroup: 1 << cslog
    const int32_t set0 = GLU ? bx << (cslog - 1) : bx << cslog;
    if (set0 >= jb.sets) {
        if constexpr (CHAIN) {
            chain_wait(link);
            chain_signal(link);
        }
        return;
    }
    const int32_t my_cs = wave & ((1 << cslog) - 1), kp = wave >> cslog;
    const int32_t my_set = set0 + (GLU ? my_cs >> 1 : my_cs);
    const bool set_live = my_set < jb.sets;
    const int32_t set = set_live ? my_set : jb.sets - 1;  // a dead wave computes a copy, never writes
    const int32_t chunks = (K + CHUNK - 1) >> 7;
    const int32_t G = (K + (RUN << gshift) - 1) >> (gshift + 5);  // quantization groups
    const int32_t c_begin = (kp * chunks) >> kslog;
    const int32_t n = (((kp + 1) * chunks) >> kslog) - c_begin;  // chunks of this wave, 1 .. nmax
    const int32_t k0 = c_begin * CHUNK;
    const int32_t nl = ln & 15, kb = ln >> 4;
    const int32_t col = set * SET + nl;
    const int32_t kpad = chunks * CHUNK;  // digit row stride

    // ---- loads, in the order they complete: this thread's share of x (buffer loads:
    // slots past the row read zeros without memory traffic), the wave's scales and zero
    // points, then the first R chunks of weights.
    const int32_t n4 = K >> 2, kp4 = kpad >> 2;
    const int32_t used = (kp4 + 64 * W - 1) / (64 * W);  // slots that reach into the digit rows
    float4 xv[XS];
    float4 uv[XMODE == X_PLAIN ? 1 : XS];
    auto load_x = [&]() {
        const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(x), 0, K * 4, 0x00020000);
        const __amdgpu_buffer_rsrc_t ur =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(XMODE == X_PLAIN ? x : aux), 0, K * 4, 0x00020000);
        static_for<0, XS>([&](auto jc) {
            constexpr int j = decltype(jc)::value;
            if (j < used) {
                xv[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(xr, (tid + 64 * W * j) * 16, 0,
                                                                                         CHAIN ? COHERENT : 0));
                if constexpr (XMODE != X_PLAIN)  // up (SwiGLU input) may come from the chain too
                    uv[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                           ur, (tid + 64 * W * j) * 16, 0,
                                                           CHAIN && XMODE == X_SWIGLU ? COHERENT : 0));
            } else {
                xv[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if constexpr (XMODE != X_PLAIN) uv[j] = xv[j];
            }
        });
    };
    if constexpr (!CHAIN) load_x();  // chained: after the weights and the wait

    int8_t* xd = reinterpret_cast<int8_t*>(smem);
    const int32_t zoff = 4 * kpad;
    int2* rec = reinterpret_cast<int2*>(smem + lds_rec_offset(chunks));

    // The wave's scales and zero points: group rows g0 .. g0 + rows - 1 of its column
    // set in the copy's [set][group][16] rows (contiguous: 64 bytes of scales and 16 of
    // zero points a row), in a few 16-byte loads per lane (sixteen rows of scales per
    // load: four lanes a row; a row of zero points per lane); rows past the wave's range or
    // past G read zeros without memory traffic, and the last two loads go out only for a
    // range of more than 32 rows (measured at 14336 -> 4096 INT4: 9.4 -> 9.0 us against
    // reading the next wave's rows too). They go to the wave's rows in LDS with the digit
    // pass, and each chunk reads its lane's pair there. Measured at 4096 -> 14336 /
    // 14336 -> 4096 INT4: one 4-byte and one 1-byte load per chunk from the [G x N] arrays
    // 7.9 / 10.7 us, these rows gathered from the [G x N] arrays 8.2-8.5 / 10.3-11.0, from
    // the copy's contiguous rows 8.0 / 8.8.
    const int32_t g0 = k0 >> (gshift + 5);
    const int32_t rows = stage_rows((chunks + (1 << kslog) - 1) >> kslog, gshift);
    const __amdgpu_buffer_rsrc_t sr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(jb.s), 0, G * jb.N * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t zr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(ZP ? jb.z : reinterpret_cast<const int8_t*>(jb.s)), 0, G * jb.N, 0x00020000);
    u32x4 sst[4];
    u32x4 zst;
    const int32_t rlim = min(G, g0 + rows);
    auto issue_stage = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int32_t r = g0 + 16 * i + (ln >> 2);
            const int32_t off = r < rlim ? ((set * G + r) * SET + 4 * (ln & 3)) * 4 : G * jb.N * 4;
            if (i < 2 || 16 * i < rows)  // (the first two unconditional: measured faster)
                sst[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(sr, off, 0, 0));
            else
                sst[i] = u32x4{0u, 0u, 0u, 0u};
        }
        if constexpr (ZP) {
            const int32_t r = g0 + ln;
            zst = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                zr, r < rlim ? (set * G + r) * SET : G * jb.N, 0, 0));
        }
    };
    if constexpr (!CHAIN) issue_stage();

    // the wave's blocks are contiguous; chunks past its range read as zeros without
    // touching memory. Weights are read once: non-temporal loads (measured 8.7 -> 7.9 us
    // at 4096 x 14336 before the staging above; a plain read of the same bytes 7.1 -> 6.5).
    const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(jb.packed + (static_cast<int64_t>(set) * chunks + c_begin) * BB), 0, n * BB, 0x00020000);
    const int32_t run_base = (k0 >> 5) + kb;  // this lane's run in chunk 0 of its range
    u32x4 wb[R][NB];
    auto issue = [&](int slot, int32_t cc) {
#pragma unroll
        for (int h = 0; h < NB; ++h)
            wb[slot][h] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                        wr, cc * BB + h * 1024 + 16 * ln, 0, NONTEMPORAL));
    };
    if constexpr (CHAIN) issue_stage();
#pragma unroll
    for (int s = 0; s < R; ++s) issue(s, s);
    __builtin_amdgcn_sched_barrier(0);
    // chained and accumulating: this lane's old output (an earlier stage may have written
    // it) goes out with the row
    float old_out = 0.0f;
    if constexpr (CHAIN) {
        chain_wait(link);
        load_x();
        if constexpr (!GLU)
            if (accumulate && kp == 0 && ln < SET && set_live) old_out = load_out<true>(jb.out + col);
    }

    // ---- x to digits and run records, the whole row by the whole workgroup --------------
    // (float4 slot j of thread t is float4 t + 64 W j of the row; a run's 8 float4s are 8
    // lanes of one wave). Float4s past the row give zero digits.
    if (tid < ZERO_BYTES / 4) reinterpret_cast<uint32_t*>(smem + zoff)[tid] = 0u;
    float nsum = 0.0f;  // X_NORM: this thread's share of sum x^2
    static_for<0, XS>([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        const int32_t i = tid + 64 * W * j;
        if (j >= used) return;
        float v[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
        const bool in_row = i < n4;
        if constexpr (XMODE == X_SWIGLU) {
            const float u[4] = {uv[j].x, uv[j].y, uv[j].z, uv[j].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = v[e] / (1.0f + static_cast<float>(exp(-static_cast<double>(v[e])))) * u[e];
        } else if constexpr (XMODE == X_NORM) {
            const float u[4] = {uv[j].x, uv[j].y, uv[j].z, uv[j].w};
            nsum = fmaf(v[0], v[0], fmaf(v[1], v[1], fmaf(v[2], v[2], fmaf(v[3], v[3], nsum))));
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] *= u[e];
        }
        if (!in_row) v[0] = v[1] = v[2] = v[3] = 0.0f;
        const float mx = max8(fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
        const bool finite = mx <= 3.402823466e38f;
        const int e = finite && mx > 0.0f ? __builtin_amdgcn_frexp_expf(mx) : 0;
        uint32_t dg[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int32_t X = finite ? static_cast<int32_t>(ldexpf(v[q], 30 - e)) : 0;
            dg[q] = (static_cast<uint32_t>(X) + 0x808080u) ^ 0x808080u;
        }
        // 4 x 4 byte transpose: digit p of the four values into one dword
        const uint32_t t01l = __builtin_amdgcn_perm(dg[1], dg[0], 0x05010400u);
        const uint32_t t01h = __builtin_amdgcn_perm(dg[1], dg[0], 0x07030602u);
        const uint32_t t23l = __builtin_amdgcn_perm(dg[3], dg[2], 0x05010400u);
        const uint32_t t23h = __builtin_amdgcn_perm(dg[3], dg[2], 0x07030602u);
        const float sx = sum8((v[0] + v[1]) + (v[2] + v[3]));
        if (i < kp4) {
            uint32_t* xw = reinterpret_cast<uint32_t*>(xd) + i;
            xw[0] = __builtin_amdgcn_perm(t23l, t01l, 0x05040100u);
            xw[kp4] = __builtin_amdgcn_perm(t23l, t01l, 0x07060302u);
            xw[2 * kp4] = __builtin_amdgcn_perm(t23h, t01h, 0x05040100u);
            xw[3 * kp4] = __builtin_amdgcn_perm(t23h, t01h, 0x07060302u);
            if ((ln & 7) == 0) rec[i >> 3] = make_int2(e - 14, __float_as_int(finite ? sx : __builtin_nanf("")));
        }
    });
    float* red = reinterpret_cast<float*>(smem + lds_red_offset(chunks));  // [W][16], then [W] x^2
    if constexpr (XMODE == X_NORM) {
        const float w2 = norm_wave_sum(nsum);
        if (ln == 0) red[W * SET + wave] = w2;
    }
    // the staged rows (only this wave reads them)
    unsigned char* stg = smem + lds_stage_offset(chunks) + wave * rows * STAGE_ROW_BYTES;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (16 * i + (ln >> 2) < rows) *reinterpret_cast<u32x4*>(stg + i * 1024 + 16 * ln) = sst[i];
    if constexpr (ZP)
        if (ln < rows) *reinterpret_cast<u32x4*>(stg + rows * SET * 4 + 16 * ln) = zst;
    __syncthreads();

    // ---- main loop: R chunks in flight ----------------------------------------------
    // A: lane (row i = ln % 16, lane group kb) reads digit i % 4 of its own group's run
    // when i / 4 == kb, the zero bytes otherwise.
    const bool diag = (nl >> 2) == kb;
    const int32_t a_base = diag ? (nl & 3) * kpad + k0 + kb * RUN : zoff;
    const int32_t a_step = diag ? CHUNK : 0;
    const uint32_t mask = 0x0F0F0F0Fu;
    float y = 0.0f;
    // K is cut into SUB_PARTS sub-parts at chunk (j chunks) / SUB_PARTS, j = 0 .. SUB_PARTS;
    // a wave's range is SUB_PARTS / ks of them. A sub-part's sum (each lane's runs in K
    // order, then the column's four lanes, (l0 + l1) + (l2 + l3), by two lane swaps)
    // enters a balanced tree over the sub-parts in K order: the wave completes the
    // subtree of its range, the meet adds the top levels. So the result does not depend
    // on ks, only on K.
    const int32_t sp_count = SUB_PARTS >> kslog, sp0 = kp * sp_count;
    int32_t sp = 0;                                                   // the current sub-part
    int32_t sp_end = (((sp0 + 1) * chunks) >> SUB_LOG) - c_begin;    // its end (wave's chunks)
    float tree[3] = {0.0f, 0.0f, 0.0f};
    float part = 0.0f;
    auto close_sub_part = [&]() {
        part = tree_push(tree, sp, lanes4_sum(y));
        y = 0.0f;
        ++sp;
        sp_end = (((sp0 + sp + 1) * chunks) >> SUB_LOG) - c_begin;
    };
    // live = false: a chunk past the wave's range (its weights read as zeros), which adds
    // nothing; its LDS reads stay inside the wave's rows
    auto process = [&](int s, int32_t cc, bool live) {
        if (live)
            while (cc >= sp_end) close_sub_part();
        cc = live ? cc : n - 1;
        const int8_t* pa = xd + a_base + cc * a_step;
        const i32x4 a0 = *reinterpret_cast<const i32x4*>(pa);
        const i32x4 a1 = *reinterpret_cast<const i32x4*>(pa + 16);
        i32x4 b0, b1;
        if constexpr (BITS == 4) {
            const u32x4 d = wb[s][0];
            b0 = i32x4{static_cast<int32_t>(d[0] & mask), static_cast<int32_t>((d[0] >> 4) & mask),
                       static_cast<int32_t>(d[1] & mask), static_cast<int32_t>((d[1] >> 4) & mask)};
            b1 = i32x4{static_cast<int32_t>(d[2] & mask), static_cast<int32_t>((d[2] >> 4) & mask),
                       static_cast<int32_t>(d[3] & mask), static_cast<int32_t>((d[3] >> 4) & mask)};
        } else {
            b0 = __builtin_bit_cast(i32x4, wb[s][0]);
            b1 = __builtin_bit_cast(i32x4, wb[s][1]);
        }
        i32x4 acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, i32x4{0, 0, 0, 0}, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, acc, 0, 0, 0);
        const int2 rc = rec[run_base + cc * (CHUNK / RUN)];
        // the lane's group row (a run past K, padding of the last chunk, takes the last
        // group's: its digits are zero, so it adds nothing)
        const int32_t r = min((run_base + cc * (CHUNK / RUN)) >> gshift, G - 1) - g0;
        const float scale = *reinterpret_cast<const float*>(stg + r * (SET * 4) + nl * 4);
        const float zero = ZP ? static_cast<float>(static_cast<int8_t>(stg[rows * SET * 4 + r * SET + nl])) : 0.0f;
        // digit pairs in integer (exact: |D_p| < 2^16 for INT4, so D_0 + 256 D_1 < 2^24;
        // INT8 sums round once in the conversion), then one fma: u = D_23 + D_01 / 2^16
        // with D_23 = D_2 + 256 D_3, D_01 = D_0 + 256 D_1; the run record holds E - 14
        const int32_t d01 = acc[0] + (acc[1] << 8), d23 = acc[2] + (acc[3] << 8);
        const float u = fmaf(static_cast<float>(d01), 1.0f / 65536.0f, static_cast<float>(d23));
        const float v = fmaf(-zero, __int_as_float(rc.y), ldexpf(u, rc.x));
        const float yn = fmaf(scale, v, y);
        y = live ? yn : y;
    };
    // The ring: a loop over groups of R chunks, each slot's refill (chunk c + R) issued
    // right behind its use. The refills cross the loop's back edge, so the compiler
    // cannot sink them to their uses: with the chunks unrolled under per-chunk range
    // tests it did exactly that in some instantiations (each load then waited for at
    // once, one chunk in flight: 4096 x 14336 INT4 11.4 us instead of 8.0). Refills past
    // the range read zeros without memory traffic; chunks past it are masked.
    auto ring_loop = [&]() {
#pragma nounroll
        for (int32_t c0 = 0; c0 < n; c0 += R) {
            static_for<0, R>([&](auto si) {
                constexpr int sl = decltype(si)::value;
                process(sl, c0 + sl, c0 + sl < n);
                issue(sl, c0 + sl + R);
                __builtin_amdgcn_sched_barrier(0);  // keep each refill right behind its use
            });
        }
    };
    if constexpr (CHAIN) {
        // a chained stage whose whole range is already in the ring: no refills, so the
        // chunks' reads and products may interleave
        if (n <= R)
            static_for<0, R>([&](auto ci) {
                constexpr int c = decltype(ci)::value;
                if (c < n) process(c, c, true);
            });
        else
            ring_loop();
    } else {
        ring_loop();
    }

    // ---- the last sub-parts, then the K-parts of the column set (the tree's top) --------
    while (sp < sp_count) close_sub_part();
    if (ln < SET) red[wave * SET + ln] = part;
    __syncthreads();
    [&]() {
        if (kp != 0 || ln >= SET || !set_live) return;
        const int32_t cs = 1 << cslog;
        const float sum = tree_top(red + my_cs * SET + ln, cs * SET, kslog);
        float al = alpha;
        if constexpr (XMODE == X_NORM) {
            float sq = red[W * SET];
            for (int32_t w = 1; w < W; ++w) sq += red[W * SET + w];
            al = alpha * (1.0f / sqrtf(sq / static_cast<float>(K) + eps));
        }
        if constexpr (GLU) {
            // the gate wave of the pair: its partner (slot my_cs + 1) holds up's sums
            if (my_cs & 1) return;
            const float usum = tree_top(red + (my_cs + 1) * SET + ln, cs * SET, kslog);
            float g = fmaf(al, sum, 0.0f);
            if (jb.bias) g += jb.bias[col];
            const PJob& ju = jobs.job[1];
            float u = fmaf(al, usum, 0.0f);
            if (ju.bias) u += ju.bias[col];
            store_out<CHAIN>(ju.out + col, u);
            store_out<CHAIN>(jb.out + col, g / (1.0f + static_cast<float>(exp(-static_cast<double>(g)))) * u);
            return;
        }
        float* dst = jb.out + col;
        float o = accumulate ? (CHAIN ? old_out : *dst) : 0.0f;
        o = fmaf(al, sum, o);
        if (jb.bias) o += jb.bias[col];
        store_out<CHAIN>(dst, o);
    }();
    if constexpr (CHAIN) chain_signal(link);
}

template <int BITS, int R, bool ZP, int XMODE, bool GLU>
__global__ void __launch_bounds__(64 * W)
    gemv_packed_kernel(const float* __restrict__ x, const float* __restrict__ aux, float eps, int32_t K, int32_t gshift,
                       PJobs jobs, int32_t kslog, int32_t nmax, float alpha, int32_t accumulate) {
    (void)nmax;
    gemv_packed_body<BITS, R, ZP, XMODE, GLU, false>(x, aux, eps, K, gshift, jobs, kslog, alpha, accumulate, blockIdx.x,
                                                     blockIdx.y, ChainLink{});
}


// One weight (the common call): everything the first loads depend on is in the first
// 16 dwords of the arguments, which arrive in scalar registers with the wave, and the
// copy's scale and zero-point rows are found from its size, so no wave waits for an
// argument fetch before its first loads (a job table indexed by blockIdx.y, and the
// K-part shift after it, are read from memory). shifts = kslog | gshift << 4.
template <int BITS, int R, bool ZP, int XMODE>
__global__ void __launch_bounds__(64 * W)
    gemv_packed_single(const uint8_t* __restrict__ packed, const float* __restrict__ x, int32_t N, int32_t K,
                       int32_t shifts, float alpha, float* out, int32_t accumulate, const float* bias,
                       const float* __restrict__ aux, float eps) {
    const int32_t kslog = shifts & 15, gshift = shifts >> 4;
    const int32_t sets = N >> 4, chunks = (K + CHUNK - 1) >> 7, G = (K + (RUN << gshift) - 1) >> (gshift + 5);
    PJobs jobs;
    jobs.count = 1;
    PJob& jb = jobs.job[0];
    jb.packed = packed;
    jb.s = reinterpret_cast<const float*>(packed + static_cast<int64_t>(sets) * chunks * block_bytes(BITS));
    jb.z = ZP ? reinterpret_cast<const int8_t*>(jb.s + static_cast<int64_t>(sets) * G * SET) : nullptr;
    jb.out = out;
    jb.bias = bias;
    jb.N = N;
    jb.sets = sets;
    gemv_packed_body<BITS, R, ZP, XMODE, false, false>(x, aux, eps, K, gshift, jobs, kslog, alpha, accumulate,
                                                       blockIdx.x, 0, ChainLink{});
}

// 2..16 rows of a small weight as one-row products in one launch: workgroup row
// blockIdx.y takes x row y and writes output row y, so each row's result is its one-row
// result bit for bit. The weight is read once per row (the later reads mostly from the
// caches); this pays where the rows' reads and workgroups cost less than the row kernels'
// fixed costs (the rule is gemv_packed_rows_rep_preferred).
template <int BITS, int R, bool ZP>
__global__ void __launch_bounds__(64 * W)
    gemv_packed_rows_rep(const uint8_t* __restrict__ packed, const float* __restrict__ x, int32_t N, int32_t K,
                         int32_t shifts, float alpha, float* out, int32_t accumulate, const float* bias) {
    const int32_t kslog = shifts & 15, gshift = shifts >> 4;
    const int32_t sets = N >> 4, chunks = (K + CHUNK - 1) >> 7, G = (K + (RUN << gshift) - 1) >> (gshift + 5);
    PJobs jobs;
    jobs.count = 1;
    PJob& jb = jobs.job[0];
    jb.packed = packed;
    jb.s = reinterpret_cast<const float*>(packed + static_cast<int64_t>(sets) * chunks * block_bytes(BITS));
    jb.z = ZP ? reinterpret_cast<const int8_t*>(jb.s + static_cast<int64_t>(sets) * G * SET) : nullptr;
    jb.out = out + static_cast<size_t>(blockIdx.y) * N;
    jb.bias = bias;
    jb.N = N;
    jb.sets = sets;
    gemv_packed_body<BITS, R, ZP, X_PLAIN, false, false>(x + static_cast<size_t>(blockIdx.y) * K, nullptr, 0.0f, K,
                                                         gshift, jobs, kslog, alpha, accumulate, blockIdx.x, 0,
                                                         ChainLink{});
}

// The same for up to four weights sharing x (blockIdx.y the weight, blockIdx.z the row).
template <int BITS, int R, bool ZP>
__global__ void __launch_bounds__(64 * W)
    gemv_packed_group_rep(const float* __restrict__ x, int32_t K, int32_t gshift, PJobs jobs, int32_t kslog, float alpha,
                          int32_t accumulate) {
    gemv_packed_body<BITS, R, ZP, X_PLAIN, false, false>(x + static_cast<size_t>(blockIdx.z) * K, nullptr, 0.0f, K,
                                                         gshift, jobs, kslog, alpha, accumulate, blockIdx.x,
                                                         blockIdx.y, ChainLink{}, blockIdx.z);
}

struct Forced {
    int ks = 0;
    int ring = 0;  // 1: 4 KB of weights in flight per wave, 2: 8 KB, 0: automatic
};
Forced g_forced;

template <int BITS, int R, bool ZP, int XMODE, bool GLU>
int32_t launch_k(dim3 grid, size_t lds, hipStream_t st, const float* x, const float* aux, float eps, int32_t K,
                 int32_t gshift, const PJobs& jobs, int32_t kslog, float alpha, int32_t accumulate, int32_t nmax) {
    if constexpr (!GLU) {
        if (jobs.count == 1) {
            if (const int32_t status = allow_lds<&gemv_packed_single<BITS, R, ZP, XMODE>>(lds)) return status;
            const PJob& jb = jobs.job[0];
            gemv_packed_single<BITS, R, ZP, XMODE><<<grid, dim3(64 * W), lds, st>>>(
                jb.packed, x, jb.N, K, kslog | gshift << 4, alpha, jb.out, accumulate, jb.bias, aux, eps);
            return KT_OK;
        }
    }
    if (const int32_t status = allow_lds<&gemv_packed_kernel<BITS, R, ZP, XMODE, GLU>>(lds)) return status;
    gemv_packed_kernel<BITS, R, ZP, XMODE, GLU>
        <<<grid, dim3(64 * W), lds, st>>>(x, aux, eps, K, gshift, jobs, kslog, nmax, alpha, accumulate);
    return KT_OK;
}

template <int BITS, bool ZP, int XMODE, bool GLU>
int32_t launch_g(dim3 grid, size_t lds, hipStream_t st, const float* x, const float* aux, float eps, int32_t K,
                 int32_t gshift, const PJobs& jobs, int32_t kslog, float alpha, int32_t accumulate, int32_t nmax) {
    // the ring: 4 KB of weights in flight per wave (8 KB when forced, 2 KB for short
    // ranges); INT8 ranges of 8 chunks or more take 8 KB (measured: 4096 -> 14336 g64 /
    // g32 12.8 / 14.3 -> 12.5 / 13.4 us, 4096 -> 128256 g32 95.3 -> 91.8; INT4 slower with
    // 8 KB, 8.4 -> 9.0; 2048 -> 8192 INT8, 4-chunk ranges, 5.4 -> 5.5)
    constexpr int RS = BITS == 4 ? 4 : 2;
    if (g_forced.ring == 2 || (g_forced.ring == 0 && BITS == 8 && nmax >= 8))
        return launch_k<BITS, 2 * RS, ZP, XMODE, GLU>(grid, lds, st, x, aux, eps, K, gshift, jobs, kslog, alpha,
                                                      accumulate, nmax);
    if (g_forced.ring == 1 || nmax > RS / 2)
        return launch_k<BITS, RS, ZP, XMODE, GLU>(grid, lds, st, x, aux, eps, K, gshift, jobs, kslog, alpha,
                                                  accumulate, nmax);
    return launch_k<BITS, RS / 2, ZP, XMODE, GLU>(grid, lds, st, x, aux, eps, K, gshift, jobs, kslog, alpha,
                                                  accumulate, nmax);
}

// The paired gate/up form exists for the plain and RMSNorm inputs only.
template <int BITS, bool ZP, int XMODE>
int32_t launch_r(dim3 grid, size_t lds, hipStream_t st, const float* x, const float* aux, float eps, int32_t K,
                 int32_t gshift, const PJobs& jobs, int32_t kslog, float alpha, int32_t accumulate, int32_t nmax,
                 int32_t glu) {
    if constexpr (XMODE != X_SWIGLU)
        if (glu)
            return launch_g<BITS, ZP, XMODE, true>(grid, lds, st, x, aux, eps, K, gshift, jobs, kslog, alpha,
                                                   accumulate, nmax);
    return launch_g<BITS, ZP, XMODE, false>(grid, lds, st, x, aux, eps, K, gshift, jobs, kslog, alpha, accumulate,
                                            nmax);
}

template <int BITS, bool ZP>
int32_t launch_mode(int mode, dim3 grid, size_t lds, hipStream_t st, const float* x, const float* aux, float eps,
                    int32_t K, int32_t gshift, const PJobs& jobs, int32_t kslog, float alpha, int32_t accumulate,
                    int32_t nmax, int32_t glu) {
    if (mode == X_SWIGLU)
        return launch_r<BITS, ZP, X_SWIGLU>(grid, lds, st, x, aux, eps, K, gshift, jobs, kslog, alpha, accumulate,
                                            nmax, glu);
    if (mode == X_NORM)
        return launch_r<BITS, ZP, X_NORM>(grid, lds, st, x, aux, eps, K, gshift, jobs, kslog, alpha, accumulate, nmax,
                                          glu);
    return launch_r<BITS, ZP, X_PLAIN>(grid, lds, st, x, aux, eps, K, gshift, jobs, kslog, alpha, accumulate, nmax,
                                       glu);
}


}  // namespace

int64_t packed_weight_bytes(int32_t rows, int32_t columns, int32_t bits) {
    const int64_t sets = ceil_div(columns, SET), chunks = ceil_div(rows, CHUNK);
    return sets * chunks * block_bytes(bits);
}

int64_t packed_bytes(int32_t rows, int32_t columns, int32_t bits, int32_t group_size) {
    const int64_t sets = ceil_div(columns, SET), groups = ceil_div(rows, group_size);
    return packed_weight_bytes(rows, columns, bits) + sets * groups * STAGE_ROW_BYTES + PACKED_TRAILER_BYTES;
}

const float* packed_scale_max(const WeightView& w) {
    return reinterpret_cast<const float*>(static_cast<const uint8_t*>(w.p) + packed_bytes(w.K, w.N, w.bits, w.g) -
                                          PACKED_TRAILER_BYTES);
}

int32_t launch_pack(const WeightView& w, void* packed, hipStream_t st) {
    const int32_t chunks = ceil_div(w.K, CHUNK);
    const int64_t wbytes = packed_weight_bytes(w.K, w.N, w.bits);
    const int64_t dwords = wbytes / 4;
    int64_t blocks = (dwords + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    pack_kernel<<<static_cast<uint32_t>(blocks), 256, 0, st>>>(w.q, w.K, w.N, w.bits, w.bpr, chunks, dwords,
                                                               static_cast<uint32_t*>(packed));
    KT_LAUNCHED("qweight pack kernel");
    const int32_t sets = ceil_div(w.N, SET);
    const int64_t rows = static_cast<int64_t>(sets) * w.G * SET;
    float* ps = reinterpret_cast<float*>(static_cast<uint8_t*>(packed) + wbytes);
    int8_t* pz = reinterpret_cast<int8_t*>(ps + rows);
    uint32_t* smax = reinterpret_cast<uint32_t*>(pz + rows);  // the trailer: 16-byte aligned (rows % 16 == 0)
    zero_trailer<<<1, 64, 0, st>>>(smax);
    KT_LAUNCHED("qweight pack kernel (trailer)");
    blocks = std::min<int64_t>((rows + 255) / 256, 65536);
    pack_scales_kernel<<<static_cast<uint32_t>(blocks), 256, 0, st>>>(w.s, w.z, w.G, w.N, rows, ps, pz, smax);
    KT_LAUNCHED("qweight pack kernel (scales)");
    return KT_OK;
}

void set_gemv_packed_config(int32_t ks, int32_t waves, int32_t ring) {
    g_forced.ks = ks == 1 || ks == 2 || ks == 4 || ks == 8 ? ks : 0;
    (void)waves;  // eight per workgroup
    g_forced.ring = ring == 4 ? 1 : ring == 8 ? 2 : 0;
}
int32_t packed_forced_ks() { return g_forced.ks; }




// K-parts per column set for a launch over weights with K rows, groups of g and
// sets_total column sets in all: the smallest power of two that keeps a wave's range
// within 2048 k, doubled while the workgroups (8 / ks column sets each) number fewer than
// 4/5 of the CUs and every part keeps at least two chunks (measured: at 4096 -> 14336,
// 224 workgroups of 16-chunk waves beat 448 of 8-chunk ones; at 2048 -> 8192, 256 of
// 4-chunk waves beat 128 of 8-chunk ones). ks = 0 when nothing fits.
PackedPlan plan_packed(int32_t K, int32_t g, int64_t sets_total) {
    PackedPlan p;
    if (g % RUN != 0 || log2_exact(g / RUN) < 0) return p;
    const int32_t chunks = ceil_div(K, CHUNK);
    int32_t ks = 1;
    while (ks < W && ceil_div(chunks, ks) > MAX_WAVE_CHUNKS) ks *= 2;
    if (ceil_div(chunks, ks) > MAX_WAVE_CHUNKS) return p;
    if (g_forced.ks) {
        if (g_forced.ks < ks || g_forced.ks > chunks) return p;
        ks = g_forced.ks;
    } else {
        while (ks < W && 2 * ks <= chunks && 5 * ((sets_total * ks + W - 1) / W) < 4 * cu_count()) ks *= 2;
    }
    const int32_t nmax = ceil_div(chunks, ks);
    const size_t lds = static_cast<size_t>(lds_bytes(chunks, nmax, log2_exact(g / RUN)));
    if (lds > LDS_MAX) return p;
    p.ks = ks;
    p.nmax = nmax;
    p.lds = lds;
    return p;
}



bool gemv_packed_supported(const float* a, int32_t m, const WeightView& w, const float* c) {
    (void)c;
    if (m != 1 || !w.p) return false;
    if (w.K % RUN != 0 || w.K > MAX_K) return false;             // whole runs; the digits fit LDS
    if (w.g % RUN != 0 || log2_exact(w.g / RUN) < 0) return false;  // a run lies in one group
    if (w.N % SET != 0) return false;                             // whole column sets
    if (static_cast<int64_t>(w.G) * w.N * 4 > INT32_MAX) return false;  // scale offsets in 32 bits
    if (!aligned(w.p, 16) || !aligned(a, 16) || !aligned(w.s, 16) || (w.z && !aligned(w.z, 16))) return false;
    return plan_packed(w.K, w.g, w.N / SET).ks != 0;
}

bool gemv_packed_pair_supported(const float* a, const WeightView* ws, float* const* cs) {
    if (!gemv_packed_supported(a, 1, ws[0], cs[0]) || !gemv_packed_supported(a, 1, ws[1], cs[1])) return false;
    if (ws[0].N != ws[1].N || ws[0].K != ws[1].K || ws[0].bits != ws[1].bits || ws[0].g != ws[1].g ||
        (ws[0].z != nullptr) != (ws[1].z != nullptr))
        return false;
    const PackedPlan plan = plan_packed(ws[0].K, ws[0].g, 2 * (ws[0].N / SET));
    return plan.ks != 0 && plan.ks <= W / 2;  // two column sets per workgroup at least
}

namespace {

// One launch of the column-run GEMV, as launch_gemv_packed checks and shapes it.
struct PackedLaunch {
    PJobs jobs{};
    dim3 grid;
    size_t lds = 0;
    int mode = X_PLAIN;
    int32_t kslog = 0, nmax = 0, gshift = 0, bits = 0;
    bool zp = false, glu = false;
    const float* x = nullptr;
    const float* aux = nullptr;
    float eps = 0.0f, alpha = 1.0f;
    int32_t K = 0, accumulate = 0;
};

int32_t prepare_gemv_packed(const float* a, const WeightView* ws, float* const* cs, const float* const* biases,
                            int32_t count, int32_t accumulate, float alpha, const float* up, const float* norm_weight,
                            float eps, bool glu, PackedLaunch* out) {
    const WeightView& w0 = ws[0];
    bool zp = false;
    for (int32_t i = 0; i < count; ++i) zp = zp || ws[i].z != nullptr;
    if (zp)
        for (int32_t i = 0; i < count; ++i)
            if (!ws[i].z) return fail(KT_ERR_ARGUMENT, "grouped weights must all have zero points or none");
    if (up && norm_weight) return fail(KT_ERR_ARGUMENT, "packed gemv: one input transform at a time");
    const int mode = up ? X_SWIGLU : norm_weight ? X_NORM : X_PLAIN;
    if (mode != X_PLAIN && !aligned(up ? up : norm_weight, 16))
        return fail(KT_ERR_ARGUMENT, "packed gemv: the gate's up row or the RMSNorm weight must be 16-byte aligned");
    int64_t sets_total = 0, sets_max = 0;
    for (int32_t i = 0; i < count; ++i) {
        sets_total += ws[i].N / SET;
        sets_max = std::max<int64_t>(sets_max, ws[i].N / SET);
    }
    const PackedPlan plan = plan_packed(w0.K, w0.g, sets_total);
    if (!plan.ks) return fail(KT_ERR_ARGUMENT, "packed gemv: no work split fits K = %d, g = %d", w0.K, w0.g);
    if (glu && (count != 2 || ws[0].N != ws[1].N || plan.ks > W / 2 || accumulate || up))
        return fail(KT_ERR_ARGUMENT, "packed gemv: the paired gate/up form needs two weights of one shape");
    PackedLaunch& L = *out;
    L.jobs = PJobs{};
    L.jobs.count = count;
    for (int32_t i = 0; i < count; ++i) {
        PJob& jb = L.jobs.job[i];
        jb.packed = ws[i].p;
        // the copy's scale and zero-point rows follow its weight blocks
        jb.s = reinterpret_cast<const float*>(ws[i].p + packed_weight_bytes(ws[i].K, ws[i].N, ws[i].bits));
        jb.z = ws[i].z ? reinterpret_cast<const int8_t*>(jb.s + static_cast<int64_t>(ws[i].N / SET) * ws[i].G * SET)
                       : nullptr;
        jb.out = cs[i];
        jb.bias = biases ? biases[i] : nullptr;
        jb.N = ws[i].N;
        jb.sets = ws[i].N / SET;
    }
    const int32_t per_wg = glu ? W / plan.ks / 2 : W / plan.ks;  // column sets (of each weight, glu) per workgroup
    L.grid = dim3(static_cast<uint32_t>(ceil_div(static_cast<int32_t>(sets_max), per_wg)),
                  static_cast<uint32_t>(glu ? 1 : count));
    L.lds = plan.lds;
    L.mode = mode;
    L.kslog = log2_exact(plan.ks);
    L.nmax = plan.nmax;
    L.gshift = log2_exact(w0.g / RUN);
    L.bits = w0.bits;
    L.zp = zp;
    L.glu = glu;
    L.x = a;
    L.aux = up ? up : norm_weight;
    L.eps = eps;
    L.alpha = alpha;
    L.K = w0.K;
    L.accumulate = accumulate;
    return KT_OK;
}

// ---- chained launches ---------------------------------------------------------------
// Dependent one-row products (each step's input row may be an earlier step's output) as
// one launch: stage s is the workgroups [begin[s], begin[s + 1]), in dispatch order after
// every earlier stage, so its first weight loads overlap the earlier stages and only the
// input row waits (ChainLink). A stage never waits for a later one and the workgroups of
// a launch are dispatched in order, so every wait ends.
constexpr int MAX_STAGES = 6;

struct ChainStage {
    PJobs jobs;
    const float* x;
    const float* aux;
    float eps, alpha;
    int32_t K, gshift, kslog, accumulate;
    int32_t gx;    // the stage's own grid is gx x (workgroups / gx)
    int32_t kind;  // 3 x the form (plain, RMSNorm, RMSNorm paired gate/up, plain paired, SwiGLU input) + ring
};
// A chained stage's wave takes its ring as deep as its chunk range where it can (RS / 2,
// RS or 2 RS chunks: all of the range in flight before the input row is there) and holds
// at most CHAIN_XS float4s of the row per thread (K <= 8192).
constexpr int CHAIN_XS = 4;

struct ChainArgs {
    int32_t begin[MAX_STAGES + 1];  // first workgroup of each stage, then the launch's total
    int32_t stages;
    uint32_t* counters;  // the stream's counters; the chain's words from CHAIN_BASE
    int32_t* fault;      // the stream's fault word
    uint32_t spin_limit;
    int32_t withhold;
    ChainStage st[MAX_STAGES];
};

template <int BITS, bool ZP>
__global__ void __launch_bounds__(64 * W) gemv_chain_kernel(ChainArgs c) {
    const int32_t b = blockIdx.x;
    int32_t s = 0;
#pragma unroll
    for (int i = 1; i < MAX_STAGES; ++i) s += (i < c.stages && b >= c.begin[i]) ? 1 : 0;
    const ChainStage& a = c.st[s];
    const int32_t local = b - c.begin[s];
    const int32_t by = local / a.gx, bx = local - by * a.gx;
    // stage s's words: CHAIN_PARTS partition counters, CHAIN_PARTS flags, the stage counter
    auto words = [&](int32_t t) { return c.counters + CHAIN_BASE + t * CHAIN_WORDS; };
    auto parts = [&](int32_t t) { return static_cast<uint32_t>(min(c.begin[t + 1] - c.begin[t], CHAIN_PARTS)); };
    const int32_t n = c.begin[s + 1] - c.begin[s], part = local % CHAIN_PARTS;
    const bool last = s + 1 == c.stages;
    ChainLink link;
    link.fault = c.fault;
    link.spin_limit = c.spin_limit;
    link.withhold = c.withhold;
    link.wait_flags = s > 0 ? words(s - 1) + CHAIN_PARTS * CHAIN_STRIDE : nullptr;
    link.wait_parts = s > 0 ? parts(s - 1) : 0u;
    link.lower_flags = s > 1 && local == 0 ? words(s - 2) + CHAIN_PARTS * CHAIN_STRIDE : nullptr;
    link.lower_parts = s > 1 ? parts(s - 2) : 0u;
    link.part_count = words(s) + part * CHAIN_STRIDE;
    link.part_flag = last ? nullptr : words(s) + (CHAIN_PARTS + part) * CHAIN_STRIDE;
    link.stage_count = words(s) + 2 * CHAIN_PARTS * CHAIN_STRIDE;
    link.last_lower = last && s > 0 ? link.wait_flags : nullptr;
    link.last_lower_parts = link.wait_parts;
    link.part_size = static_cast<uint32_t>((n - part + CHAIN_PARTS - 1) / CHAIN_PARTS);
    link.parts = parts(s);
    constexpr int RS = BITS == 4 ? 4 : 2;
#define KT_CHAIN_BODY(RING, XM, GL)                                                                                    \
    gemv_packed_body<BITS, RING, ZP, XM, GL, true, CHAIN_XS>(a.x, a.aux, a.eps, a.K, a.gshift, a.jobs, a.kslog,        \
                                                             a.alpha, a.accumulate, bx, by, link)
#define KT_CHAIN_FORM(F, XM, GL)                                                                                       \
    case 3 * F: KT_CHAIN_BODY(RS / 2, XM, GL); break;                                                                  \
    case 3 * F + 1: KT_CHAIN_BODY(RS, XM, GL); break;                                                                  \
    case 3 * F + 2: KT_CHAIN_BODY(2 * RS, XM, GL); break;
    switch (a.kind) {
        KT_CHAIN_FORM(0, X_PLAIN, false)
        KT_CHAIN_FORM(1, X_NORM, false)
        KT_CHAIN_FORM(2, X_NORM, true)
        KT_CHAIN_FORM(3, X_PLAIN, true)
        KT_CHAIN_FORM(4, X_SWIGLU, false)
        default: break;
    }
#undef KT_CHAIN_FORM
#undef KT_CHAIN_BODY
}

int32_t chain_kind(const PackedLaunch& L) {
    const int RS = L.bits == 4 ? 4 : 2;
    const int ring = L.nmax <= RS / 2 ? 0 : L.nmax <= RS ? 1 : 2;
    int form = 0;
    if (L.mode == X_SWIGLU) form = 4;
    else if (L.mode == X_NORM) form = L.glu ? 2 : 1;
    else form = L.glu ? 3 : 0;
    return 3 * form + ring;
}

}  // namespace

int32_t launch_gemv_packed(const float* a, const WeightView* ws, float* const* cs, const float* const* biases,
                           int32_t count, int32_t accumulate, float alpha, hipStream_t st, const float* up,
                           const float* norm_weight, float eps, bool glu) {
    PackedLaunch L;
    const int32_t status = prepare_gemv_packed(a, ws, cs, biases, count, accumulate, alpha, up, norm_weight, eps, glu, &L);
    if (status) return status;
    int32_t launched = KT_OK;
    if (L.bits == 4)
        launched = launch_mode<4, true>(L.mode, L.grid, L.lds, st, L.x, L.aux, L.eps, L.K, L.gshift, L.jobs, L.kslog,
                                        L.alpha, L.accumulate, L.nmax, L.glu ? 1 : 0);
    else if (L.zp)
        launched = launch_mode<8, true>(L.mode, L.grid, L.lds, st, L.x, L.aux, L.eps, L.K, L.gshift, L.jobs, L.kslog,
                                        L.alpha, L.accumulate, L.nmax, L.glu ? 1 : 0);
    else
        launched = launch_mode<8, false>(L.mode, L.grid, L.lds, st, L.x, L.aux, L.eps, L.K, L.gshift, L.jobs, L.kslog,
                                         L.alpha, L.accumulate, L.nmax, L.glu ? 1 : 0);
    if (launched) return launched;
    KT_LAUNCHED("qmatmul: packed gemv kernel");
    return KT_OK;
}

// Rows as one-row products where the extra rows cost little: (m - 1) times the larger of
// a row's workgroups that hold column sets at 5 ns each and its weight bytes at 10 TB/s
// (the extra rows' reads come mostly from the caches) within 5 us, or within 3 us per
// weight for the wide weights (their row kernel, one launch per weight, is nearer its
// one-row cost). Measured (INT4 g64, us, against the kernel taken before): 4096 -> 1024
// M = 2 / 4 / 8 / 16 4.1 / 4.3 / 5.6 / 8.5 (10.6 / 9.0 / 9.2 / 9.5); 2048 -> 2048 M = 3 / 8
// 5.0 / 7.5 (7.9 / 8.6), M = 16 12.7 (9.2, not taken); 8192 -> 2048 M = 2 / 4 5.6 / 7.8
// (12.8 / 11.3), M = 8 12.9 (11.7, not taken); 4096 -> 4096 M = 2 / 4 6.2 / 8.9 (9.7 /
// 9.8); 14336 -> 4096 M = 2 12.9 (15.1); 896 -> 896 M = 8 / 16 4.0 / 4.9 (7.9 / 8.0); wide:
// 2048 -> 8192 M = 2 / 3 5.9 / 7.0 (7.0 / 7.2), M = 4 8.6 (7.2, not taken); 896 -> 4864
// M = 2 / 4 4.7 / 5.8 (6.4 / 6.6); 4096 -> 14336 M = 2 11.4 (12.8); gate/up pairs 2048 ->
// 8192 M = 2 7.8 (13.4), 896 -> 4864 M = 3 7.4 (12.7).
bool gemv_packed_rows_rep_preferred(int32_t m, const WeightView* ws, int32_t count) {
    if (m < 2 || m > 16) return false;
    int64_t sets_total = 0;
    double bytes = 0.0;
    bool wide = false;
    for (int32_t i = 0; i < count; ++i) {
        const int64_t sets = ws[i].N / SET;
        wide = wide || sets >= 16 * ceil_div(ws[i].K, CHUNK);
        sets_total += sets;
        bytes += static_cast<double>(packed_weight_bytes(ws[i].K, ws[i].N, ws[i].bits));
    }
    const PackedPlan plan = plan_packed(ws[0].K, ws[0].g, sets_total);
    if (!plan.ks) return false;
    double wgs = 0.0;  // the workgroups that hold column sets (a grouped launch's others exit at once)
    for (int32_t i = 0; i < count; ++i) wgs += static_cast<double>(ceil_div(ws[i].N / SET, static_cast<int64_t>(W / plan.ks)));
    const double per_row_us = std::max(wgs * 0.005, bytes / 10.0e6);
    return (m - 1) * per_row_us <= (wide ? 3.0 * count : 5.0);
}

int32_t launch_gemv_packed_group_rep(const float* a, int32_t m, const WeightView* ws, float* const* cs,
                                     const float* const* biases, int32_t count, int32_t accumulate, float alpha,
                                     hipStream_t st) {
    PackedLaunch L;
    const int32_t status = prepare_gemv_packed(a, ws, cs, biases, count, accumulate, alpha, nullptr, nullptr, 0.0f,
                                               false, &L);
    if (status) return status;
    const dim3 grid(L.grid.x, static_cast<uint32_t>(count), static_cast<uint32_t>(m));
    if (L.bits == 4) {
        if (const int32_t ls = allow_lds<&gemv_packed_group_rep<4, 4, true>>(L.lds)) return ls;
        gemv_packed_group_rep<4, 4, true>
            <<<grid, dim3(64 * W), L.lds, st>>>(a, L.K, L.gshift, L.jobs, L.kslog, alpha, accumulate);
    } else if (L.zp) {
        if (const int32_t ls = allow_lds<&gemv_packed_group_rep<8, 2, true>>(L.lds)) return ls;
        gemv_packed_group_rep<8, 2, true>
            <<<grid, dim3(64 * W), L.lds, st>>>(a, L.K, L.gshift, L.jobs, L.kslog, alpha, accumulate);
    } else {
        if (const int32_t ls = allow_lds<&gemv_packed_group_rep<8, 2, false>>(L.lds)) return ls;
        gemv_packed_group_rep<8, 2, false>
            <<<grid, dim3(64 * W), L.lds, st>>>(a, L.K, L.gshift, L.jobs, L.kslog, alpha, accumulate);
    }
    KT_LAUNCHED("qmatmul: packed grouped rows as one-row products");
    return KT_OK;
}

int32_t launch_gemv_packed_rows_rep(const float* a, int32_t m, const WeightView& w, float* c, const float* bias,
                                    int32_t accumulate, float alpha, hipStream_t st) {
    const float* biases[1] = {bias};
    PackedLaunch L;
    const int32_t status = prepare_gemv_packed(a, &w, &c, biases, 1, accumulate, alpha, nullptr, nullptr, 0.0f, false, &L);
    if (status) return status;
    const dim3 grid(L.grid.x, static_cast<uint32_t>(m));
    const int32_t shifts = L.kslog | L.gshift << 4;
    if (L.bits == 4) {
        if (const int32_t ls = allow_lds<&gemv_packed_rows_rep<4, 4, true>>(L.lds)) return ls;
        gemv_packed_rows_rep<4, 4, true>
            <<<grid, dim3(64 * W), L.lds, st>>>(w.p, a, w.N, L.K, shifts, alpha, c, accumulate, bias);
    } else if (L.zp) {
        if (const int32_t ls = allow_lds<&gemv_packed_rows_rep<8, 2, true>>(L.lds)) return ls;
        gemv_packed_rows_rep<8, 2, true>
            <<<grid, dim3(64 * W), L.lds, st>>>(w.p, a, w.N, L.K, shifts, alpha, c, accumulate, bias);
    } else {
        if (const int32_t ls = allow_lds<&gemv_packed_rows_rep<8, 2, false>>(L.lds)) return ls;
        gemv_packed_rows_rep<8, 2, false>
            <<<grid, dim3(64 * W), L.lds, st>>>(w.p, a, w.N, L.K, shifts, alpha, c, accumulate, bias);
    }
    KT_LAUNCHED("qmatmul: packed rows as one-row products");
    return KT_OK;
}

int32_t gemv_chain_max_steps() { return MAX_STAGES; }
int32_t gemv_chain_max_k() { return CHAIN_XS * 4 * 64 * W; }

int32_t launch_gemv_chain(const ChainStep* steps, int32_t n, hipStream_t st) {
    if (n < 1 || n > MAX_STAGES) return fail(KT_ERR_ARGUMENT, "a chain holds 1 to %d steps, got %d", MAX_STAGES, n);
    ChainArgs c{};
    c.stages = n;
    size_t lds = 0;
    int32_t bits = 0;
    bool zp = false;
    int64_t total = 0;
    for (int32_t i = 0; i < n; ++i) {
        const ChainStep& p = steps[i];
        PackedLaunch L;
        const int32_t status = prepare_gemv_packed(p.a, p.ws, p.cs, p.biases, p.count, p.accumulate, p.alpha, p.up,
                                                   p.norm_weight, p.eps, p.glu, &L);
        if (status) return status;
        if (L.K > CHAIN_XS * 4 * 64 * W)
            return fail(KT_ERR_ARGUMENT, "a chained step's row holds at most %d values, got %d", CHAIN_XS * 4 * 64 * W, L.K);
        if (i == 0) {
            bits = L.bits;
            zp = L.zp;
        } else if (L.bits != bits || L.zp != zp) {
            return fail(KT_ERR_ARGUMENT, "a chain's weights must share one width and zero-point form");
        }
        ChainStage& a = c.st[i];
        a.jobs = L.jobs;
        a.x = L.x;
        a.aux = L.aux;
        a.eps = L.eps;
        a.alpha = L.alpha;
        a.K = L.K;
        a.gshift = L.gshift;
        a.kslog = L.kslog;
        a.accumulate = L.accumulate;
        a.gx = static_cast<int32_t>(L.grid.x);
        a.kind = chain_kind(L);
        c.begin[i] = static_cast<int32_t>(total);
        total += static_cast<int64_t>(L.grid.x) * L.grid.y;
        lds = std::max(lds, L.lds);
    }
    if (total > INT32_MAX) return fail(KT_ERR_SHAPE, "chain too large");
    for (int32_t i = n; i <= MAX_STAGES; ++i) c.begin[i] = static_cast<int32_t>(total);
    void* general = nullptr;
    const int32_t status =
        workspace_counters(st, 0, CHAIN_BASE + static_cast<size_t>(n) * CHAIN_WORDS, &general, &c.counters);
    if (status) return status;
    if (const int32_t fs = stream_fault_word(st, &c.fault)) return fs;
    const WaitLimits limits = wait_limits();
    c.spin_limit = limits.spin_limit ? limits.spin_limit : CHAIN_SPIN_LIMIT;
    c.withhold = limits.withhold;
    const dim3 grid(static_cast<uint32_t>(total));
    if (bits == 4) {
        if (const int32_t ls = allow_lds<&gemv_chain_kernel<4, true>>(lds)) return ls;
        gemv_chain_kernel<4, true><<<grid, dim3(64 * W), lds, st>>>(c);
    } else if (zp) {
        if (const int32_t ls = allow_lds<&gemv_chain_kernel<8, true>>(lds)) return ls;
        gemv_chain_kernel<8, true><<<grid, dim3(64 * W), lds, st>>>(c);
    } else {
        if (const int32_t ls = allow_lds<&gemv_chain_kernel<8, false>>(lds)) return ls;
        gemv_chain_kernel<8, false><<<grid, dim3(64 * W), lds, st>>>(c);
    }
    KT_LAUNCHED("qmatmul chain kernel");
    return KT_OK;
}

}  // namespace kt
