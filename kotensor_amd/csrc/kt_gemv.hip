// kt_gemv.hip -- decode dequant-GEMV (M == 1) for gfx950:
//   c[N] = (accumulate ? c : 0) + alpha * x[K] . deq(W) (+ bias),
// the M == 1 branch of MatMul.multiplyQuantized (Engine/kotensor/src/main/kotlin/
// MatMul.kt:475-477 -> multiplyQuantizedRow :494-536 / rowUnitInto :599-682).
//
// HBM-bound: every packed weight byte, scale and zero is read once. Work layout
// (reference layout, no repack):
//   * a lane owns VEC contiguous bytes of every row (VEC = 16, 8 or 4), so a wave
//     reads 64*VEC contiguous bytes of a row per load; for INT4 those bytes hold VEC
//     low-nibble columns b.. and VEC high-nibble columns half+b.. (split-half
//     packing), for INT8 VEC columns;
//   * K is cut into chunks of up to CH rows that never straddle a quantization
//     group. A wave issues all CH row loads of a chunk before using any (CH*VEC
//     bytes in flight per lane), accumulates acc = sum x[k]*q[k] and
//     rowSum = sum x[k] over the chunk, then applies the group's scale and zero:
//     res += scale * (acc - zero * rowSum) (the reference's combineGroup form,
//     which is linear, so chunks of one group may be combined separately);
//   * x[k] is uniform across the wave and lives in scalar registers, so the inner
//     loop is one v_cvt_f32_ubyte + one v_fma per weight; the signed INT8 byte is
//     biased by 128 (xor 0x80) and the bias folded into the zero-point term; the
//     INT4 high nibble is used in place (value 16*n) and rescaled by 1/16 exactly;
//   * a workgroup is WAVES (4 or 8) waves over one column tile; its waves take the
//     chunks of its K-slice round-robin and are summed through LDS in a fixed order
//     (16 waves would leave too few registers for two chunks in flight);
//   * with more than one K-slice per tile the slice sums go to a workspace and a
//     second kernel adds them in slice order (a fence-and-counter reduction inside
//     one kernel measured several microseconds slower on MI355X);
//   * one launch may serve up to four weights that share the input (q/k/v,
//     gate/up): the grid is the concatenation of their workgroups.
// Every reduction has a fixed order, so results are bit-reproducible run to run.
#include "kt_common.h"

namespace kt {
namespace {

constexpr int MAX_JOBS = 4;

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

struct Job {
    const uint8_t* q;
    const float* s;
    const int8_t* z;
    float* out;
    const float* bias;
    float* partials;      // [slices x N] or nullptr when slices == 1
    uint32_t* counters;   // [tiles], zero on entry, for the in-kernel slice reduction; or nullptr
    int32_t N, bpr;
    int32_t tiles, slices, chunks_per_slice;
    int32_t block_begin;  // first workgroup of this job in the grid
};

struct Jobs {
    Job job[MAX_JOBS];
    int32_t count;
};

// CH > 0: every chunk has exactly CH rows (the host checks K % g == 0 and g % CH == 0)
// and runs the double-buffered path; CH == 0: chunks of up to `chunk` rows run the
// bounds-checked row loop.
template <int BITS, int VEC, int CH, int WAVES, bool ZP>
__global__ void __launch_bounds__(64 * WAVES)
    gemv_kernel(const float* __restrict__ x, int32_t K, int32_t g, int32_t chunk, int32_t chunks_per_group,
                int32_t total_chunks, Jobs jobs, float alpha, int32_t accumulate) {
    using CT = typename Chunk<VEC>::T;
    constexpr int NC = BITS == 4 ? 2 * VEC : VEC;  // columns per lane
    __shared__ float red[WAVES][NC][64];

    // Select the job (scalar: blockIdx is uniform).
    // The job of this block: every job is read at a constant kernarg offset and selected,
    // so the scalar loads go out together instead of after a first dependent load.
    Job jb = jobs.job[0];
#pragma unroll
    for (int j = 1; j < MAX_JOBS; ++j)
        if (j < jobs.count && static_cast<int32_t>(blockIdx.x) >= jobs.job[j].block_begin) jb = jobs.job[j];
    const uint8_t* __restrict__ q = jb.q;
    const int32_t N = jb.N, bpr = jb.bpr, half = jb.bpr;
    const int32_t local = blockIdx.x - jb.block_begin;
    const int32_t tile = local % jb.tiles;
    const int32_t slice = local / jb.tiles;

    const int32_t ln = threadIdx.x & 63;
    const int32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int32_t col_off = tile * 64 * VEC + ln * VEC;
    const bool active = col_off < bpr;
    // Lanes past the end of the row run the loop on a valid offset and discard their
    // result: the whole wave must execute it, since x values are broadcast across
    // lanes (readlane, shuffles) within it.
    const int32_t boff = active ? col_off : 0;
    const int32_t c_begin = slice * jb.chunks_per_slice;
    const int32_t c_end = min(c_begin + jb.chunks_per_slice, total_chunks);

    float res[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) res[c] = 0.0f;

    // Chunk geometry: group gi, rows [r0, r1).
    auto rows_of = [&](int32_t ch, int32_t& gi, int32_t& r0, int32_t& r1) {
        gi = ch / chunks_per_group;
        r0 = gi * g + (ch - gi * chunks_per_group) * chunk;
        r1 = min(min(r0 + chunk, gi * g + g), K);
    };
    constexpr int CHB = CH > 0 ? CH : 1;
    // The scale and zero words of this lane's columns for group gi.
    constexpr int SV = BITS == 4 ? VEC / 2 : VEC / 4;  // float4 scale vectors per lane
    auto load_scales = [&](float4* sc, uint32_t* zw, int32_t gi) {
        const float* srow = jb.s + static_cast<size_t>(gi) * N;
#pragma unroll
        for (int v = 0; v < SV; ++v) {
            const int32_t col = (v < VEC / 4 ? boff : half + boff - VEC) + 4 * v;
            sc[v] = *reinterpret_cast<const float4*>(srow + col);
            // ZP is a template flag so no branch sits between the loads: a join there
            // would make the compiler wait for every outstanding load.
            if constexpr (ZP) zw[v] = *reinterpret_cast<const uint32_t*>(jb.z + static_cast<size_t>(gi) * N + col);
            else zw[v] = 0u;
        }
    };
    // res += scale * (acc - zero * rowSum), per column of this lane.
    auto combine = [&](const float* acc, float rsum, const float4* sc, const uint32_t* zw) {
#pragma unroll
        for (int v = 0; v < SV; ++v) {
            const float unit = v < VEC / 4 ? 1.0f : 0.0625f;
            const float scv[4] = {sc[v].x, sc[v].y, sc[v].z, sc[v].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float zero = static_cast<float>(static_cast<int8_t>((zw[v] >> (8 * j)) & 0xFFu));
                if (BITS == 8) zero += 128.0f;
                const int c = 4 * v + j;
                res[c] = fmaf(scv[j], fmaf(-zero, rsum, acc[c] * unit), res[c]);
            }
        }
    };
    // Accumulates one chunk whose rows (v) and x values (xv: lane u holds x[r0 + u])
    // are already in registers. x[r0 + u] is broadcast to a scalar register per row;
    // the row sum is a cross-lane reduction of xv.
    auto compute_loaded = [&](const CT* v, float xv, int32_t gi, const float4* sc, const uint32_t* zw) {
        float acc[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[c] = 0.0f;
#pragma unroll
        for (int u = 0; u < CHB; ++u) {
            const float xk = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(xv), u));
            accumulate_row<BITS, VEC>(v[u], xk, acc);
        }
        float rs = ln < CHB ? xv : 0.0f;
#pragma unroll
        for (int off = 1; off < CHB; off <<= 1) rs += __shfl_xor(rs, off);
        const float rsum = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(rs)));
        (void)gi;
        combine(acc, rsum, sc, zw);
    };
    // A chunk shorter than CH rows (group or K tail): row by row.
    auto compute_checked = [&](int32_t ch, const float4* sc, const uint32_t* zw) {
        int32_t gi, r0, r1;
        rows_of(ch, gi, r0, r1);
        float acc[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[c] = 0.0f;
        float rsum = 0.0f;
        for (int32_t l = r0; l < r1; ++l) {
            const CT v = *reinterpret_cast<const CT*>(q + static_cast<size_t>(l) * bpr + boff);
            const float xk = x[l];
            rsum += xk;
            accumulate_row<BITS, VEC>(v, xk, acc);
        }
        combine(acc, rsum, sc, zw);
    };

    {
        if constexpr (CH > 0) {
            // Every chunk has exactly CH rows. Double-buffered: while one chunk is
            // accumulated, the next chunk's rows and x values load into the other
            // register set. The current chunk's scales are requested before the next
            // chunk's rows (loads retire in order), and the next load is issued even past
            // the wave's last chunk (it re-reads the current one) so every iteration
            // waits for the same number of loads.
            auto load_chunk = [&](CT* v, float& xv, int32_t c) {
                const int32_t gi = c / chunks_per_group;
                const int32_t r0 = gi * g + (c - gi * chunks_per_group) * CH;
#pragma unroll
                for (int u = 0; u < CH; ++u) v[u] = *reinterpret_cast<const CT*>(q + static_cast<size_t>(r0 + u) * bpr + boff);
                xv = x[r0 + (ln < CH ? ln : 0)];
            };
            const int32_t first = c_begin + wave;
            if (first < c_end) {
                CT va[CH], vb[CH];
                float xa, xb;
                load_chunk(va, xa, first);
                int32_t c = first;
                for (;;) {
                    int32_t nx = c + WAVES;
                    float4 sc[SV];
                    uint32_t zw[SV];
                    int32_t gi = c / chunks_per_group;
                    load_scales(sc, zw, gi);
                    load_chunk(vb, xb, nx < c_end ? nx : c);
                    compute_loaded(va, xa, gi, sc, zw);
                    if (nx >= c_end) break;
                    c = nx;
                    nx = c + WAVES;
                    gi = c / chunks_per_group;
                    load_scales(sc, zw, gi);
                    load_chunk(va, xa, nx < c_end ? nx : c);
                    compute_loaded(vb, xb, gi, sc, zw);
                    if (nx >= c_end) break;
                    c = nx;
                }
            }
        } else {
            for (int32_t c = c_begin + wave; c < c_end; c += WAVES) {
                int32_t gi, r0, r1;
                rows_of(c, gi, r0, r1);
                float4 sc[SV];
                uint32_t zw[SV];
                load_scales(sc, zw, gi);
                compute_checked(c, sc, zw);
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
    auto column_of = [&](int c) { return (c < VEC ? boff : half + boff - VEC) + c; };
    if (jb.partials && jb.counters) {
        // In-kernel slice reduction. Every slice stores its sums with write-through
        // (system-scope) stores and waits for them to complete; the workgroup that
        // then takes the tile counter to slices-1 is the last one: it reads the other
        // slices' sums back past the caches, adds all slices in slice order, writes the
        // output and returns the counter to zero. No fence and no waiting on other
        // workgroups; the sum order, and so the result, does not depend on timing.
        float* part = jb.partials + static_cast<size_t>(slice) * N;
#pragma unroll
        for (int c = 0; c < NC; ++c) __hip_atomic_store(part + column_of(c), res[c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        __builtin_amdgcn_s_waitcnt(0);
        uint32_t old = 0;
        if (ln == 0)
            old = __hip_atomic_fetch_add(jb.counters + tile, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        old = __builtin_amdgcn_readfirstlane(old);
        if (old != static_cast<uint32_t>(jb.slices - 1)) return;
        float sum[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) sum[c] = 0.0f;
        for (int32_t sp = 0; sp < jb.slices; ++sp) {
            const float* other = jb.partials + static_cast<size_t>(sp) * N;
            float v[NC];
#pragma unroll
            for (int c = 0; c < NC; ++c)
                v[c] = sp == slice ? res[c] : __hip_atomic_load(other + column_of(c), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
#pragma unroll
            for (int c = 0; c < NC; ++c) sum[c] = sp == 0 ? v[c] : sum[c] + v[c];
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) res[c] = sum[c];
        if (ln == 0) __hip_atomic_store(jb.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int side = 0; side < (BITS == 4 ? 2 : 1); ++side) {
        const int32_t col0 = side ? half + boff : boff;
#pragma unroll
        for (int i = 0; i < VEC / 4; ++i) {
            const int32_t col = col0 + 4 * i;
            const int c = side * VEC + 4 * i;
            float4 r = make_float4(res[c], res[c + 1], res[c + 2], res[c + 3]);
            if (jb.partials && !jb.counters) {
                *reinterpret_cast<float4*>(jb.partials + static_cast<size_t>(slice) * N + col) = r;
            } else {
                float* out = jb.out;
                float4 o = accumulate ? *reinterpret_cast<const float4*>(out + col) : make_float4(0.f, 0.f, 0.f, 0.f);
                o.x = fmaf(alpha, r.x, o.x);
                o.y = fmaf(alpha, r.y, o.y);
                o.z = fmaf(alpha, r.z, o.z);
                o.w = fmaf(alpha, r.w, o.w);
                if (jb.bias) {
                    const float4 b = *reinterpret_cast<const float4*>(jb.bias + col);
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

// Adds the slice sums in slice order: out = (accumulate ? out : 0) + alpha * sum (+ bias),
// for every job of the launch that was split (grid covers the widest such job).
__global__ void __launch_bounds__(256)
    gemv_reduce(Jobs jobs, float alpha, int32_t accumulate) {
    const int32_t col = blockIdx.x * 256 + threadIdx.x;
#pragma unroll
    for (int j = 0; j < MAX_JOBS; ++j) {
        if (j >= jobs.count) break;
        const Job& jb = jobs.job[j];
        if (!jb.partials || jb.counters || col >= jb.N) continue;
        // All slice loads are issued before the first add (the sum itself stays in
        // slice order).
        float t = 0.0f;
        for (int32_t s0 = 0; s0 < jb.slices; s0 += 16) {
            float p[16];
#pragma unroll
            for (int u = 0; u < 16; ++u)
                p[u] = s0 + u < jb.slices ? jb.partials[static_cast<size_t>(s0 + u) * jb.N + col] : 0.0f;
#pragma unroll
            for (int u = 0; u < 16; ++u)
                if (s0 + u < jb.slices) t = (s0 + u == 0) ? p[u] : t + p[u];
        }
        float o = accumulate ? jb.out[col] : 0.0f;
        o = fmaf(alpha, t, o);
        if (jb.bias) o += jb.bias[col];
        jb.out[col] = o;
    }
}

struct Forced {
    int vec = 0;
    int slices = 0;
    int waves = 0;
    int reduce = 0;  // 0 automatic, 1 reduction kernel, 2 in-kernel
};
Forced g_forced;

}  // namespace

bool gemv_supported(const float* a, const WeightView& w, const float* c) {
    // Lanes need 4-column scale/zero vectors and 16-byte-aligned output quads.
    if (w.N % (w.bits == 4 ? 8 : 4) != 0) return false;
    if (!aligned(w.q, 4) || !aligned(w.s, 16) || (w.z && !aligned(w.z, 4)) || !aligned(c, 16)) return false;
    return aligned(a, 4);
}

void set_gemv_reduce_mode(int32_t mode) { g_forced.reduce = (mode == 1 || mode == 2) ? mode : 0; }

void set_gemv_config(int32_t vec, int32_t splits, int32_t waves) {
    g_forced.vec = (vec == 4 || vec == 8) ? vec : 0;
    g_forced.slices = splits > 0 ? splits : 0;
    g_forced.waves = (waves == 4 || waves == 8) ? waves : 0;
}

namespace {

// Rows per chunk (never more than a group): 32 for 4-byte lanes, 16 for wider
// ones, so two chunks of rows in flight fit in about 64 VGPRs.
constexpr int chunk_rows(int vec) { return vec == 4 ? 32 : 16; }

template <int BITS, int VEC>
int32_t launch_vec(const float* a, const WeightView* ws, float* const* cs, const float* const* biases, int32_t count,
                   int32_t accumulate, float alpha, hipStream_t st) {
    constexpr int CHMAX = chunk_rows(VEC);
    const WeightView& w0 = ws[0];
    // A chunk never straddles a group: CH = min(CHMAX, g); the shorter tail of a group
    // (g % CH) and of K take the bounds-checked path.
    const int32_t ch = w0.g < CHMAX ? w0.g : CHMAX;
    const int32_t chunks_per_group = ceil_div(w0.g, ch);
    const int32_t total_chunks = w0.G * chunks_per_group;
    const int32_t target_waves = cu_count() * 8;

    Jobs jobs{};
    jobs.count = count;
    int64_t tiles_total = 0;
    for (int32_t i = 0; i < count; ++i) tiles_total += ceil_div(ws[i].bpr, 64 * VEC);
    // Waves per workgroup and K-slices per tile. Waves of one workgroup split a
    // tile's chunks and meet in LDS; slices split them across workgroups and need the
    // reduction kernel, which costs a few microseconds, so slices are added only when
    // 16 waves per tile still leave the GPU short of waves.
    int32_t waves = 4;
    if (tiles_total * waves < target_waves && total_chunks >= 2 * 8) waves = 8;
    int32_t slices = 1;
    if (tiles_total * waves < target_waves / 2)
        slices = static_cast<int32_t>((target_waves + tiles_total * waves - 1) / (tiles_total * waves));
    const int32_t max_slices = total_chunks / waves > 1 ? total_chunks / waves : 1;
    if (slices > max_slices) slices = max_slices;
    if (g_forced.waves) waves = g_forced.waves;
    if (g_forced.slices) slices = g_forced.slices < total_chunks ? g_forced.slices : total_chunks;
    const int32_t cps = ceil_div(total_chunks, slices);
    slices = ceil_div(total_chunks, cps);

    // Up to MAX_INKERNEL_SLICES slices reduce inside the kernel (write-through sums and a
    // tile counter); more slices contend on the counters and use the reduction kernel.
    constexpr int32_t MAX_INKERNEL_SLICES = 8;
    size_t ws_floats = 0, n_counters = 0;
    if (slices > 1)
        for (int32_t i = 0; i < count; ++i) {
            ws_floats += static_cast<size_t>(slices) * ws[i].N;
            n_counters += ceil_div(ws[i].bpr, 64 * VEC);
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
        jb.tiles = ceil_div(ws[i].bpr, 64 * VEC);
        jb.slices = slices;
        jb.chunks_per_slice = cps;
        jb.block_begin = blocks;
        jb.partials = slices > 1 ? partials + offset : nullptr;
        jb.counters = inkernel ? counters + coffset : nullptr;
        offset += static_cast<size_t>(slices) * ws[i].N;
        coffset += jb.tiles;
        blocks += jb.tiles * slices;
        if (ws[i].N > widest) widest = ws[i].N;
    }
    const dim3 grid(static_cast<uint32_t>(blocks));
    // The pipelined path needs every chunk to be exactly CH rows (K a multiple of the
    // group size, the group size a multiple of CH); anything else runs the row loop.
    const bool all_full = w0.K % w0.g == 0 && w0.g % ch == 0;
    const int chk = !all_full ? 0 : (ch == CHMAX ? CHMAX : (ch == 16 ? 16 : 0));
    bool zp = false;
    for (int32_t i = 0; i < count; ++i) zp = zp || ws[i].z != nullptr;
    if (zp)
        for (int32_t i = 0; i < count; ++i)
            if (!ws[i].z) return fail(KT_ERR_ARGUMENT, "grouped weights must all have zero points or none");
#define KT_GEMV_LAUNCH(C, W)                                                                                              \
    if (BITS == 4 || zp)                                                                                                  \
        gemv_kernel<BITS, VEC, C, W, true><<<grid, dim3(64 * W), 0, st>>>(a, w0.K, w0.g, ch, chunks_per_group,           \
                                                                          total_chunks, jobs, alpha, accumulate);        \
    else                                                                                                                  \
        gemv_kernel<BITS, VEC, C, W, false><<<grid, dim3(64 * W), 0, st>>>(a, w0.K, w0.g, ch, chunks_per_group,          \
                                                                           total_chunks, jobs, alpha, accumulate)
#define KT_GEMV_WAVES(C)            \
    switch (waves) {                \
        case 8: KT_GEMV_LAUNCH(C, 8); break;   \
        default: KT_GEMV_LAUNCH(C, 4); break;  \
    }
    if (chk == CHMAX) {
        KT_GEMV_WAVES(CHMAX)
    } else if (chk == 16) {
        KT_GEMV_WAVES(16)
    } else {
        KT_GEMV_WAVES(0)
    }
#undef KT_GEMV_WAVES
#undef KT_GEMV_LAUNCH
    KT_LAUNCHED("qmatmul: gemv kernel");
    if (slices > 1 && !inkernel) {
        gemv_reduce<<<ceil_div(widest, 256), 256, 0, st>>>(jobs, alpha, accumulate);
        KT_LAUNCHED("qmatmul: gemv reduce");
    }
    return KT_OK;
}

template <int BITS>
int32_t launch_bits(const float* a, const WeightView* ws, float* const* cs, const float* const* biases, int32_t count,
                    int32_t accumulate, float alpha, hipStream_t st) {
    // Widest lane vector every weight's row pitch and alignment allow, then narrower
    // while the launch would have too few column tiles to fill the GPU.
    int vec = 8;
    for (int32_t i = 0; i < count; ++i) {
        while (vec > 4 && (ws[i].bpr % vec != 0 || !aligned(ws[i].q, vec))) vec /= 2;
    }
    const int32_t cus = cu_count();
    auto tiles_for = [&](int v) {
        int64_t t = 0;
        for (int32_t i = 0; i < count; ++i) t += ceil_div(ws[i].bpr, 64 * v);
        return t;
    };
    while (vec > 4 && tiles_for(vec) < cus / 2) vec /= 2;
    if (g_forced.vec) {
        bool ok = true;
        for (int32_t i = 0; i < count; ++i) ok = ok && ws[i].bpr % g_forced.vec == 0 && aligned(ws[i].q, g_forced.vec);
        if (ok) vec = g_forced.vec;
    }
    switch (vec) {
        case 8: return launch_vec<BITS, 8>(a, ws, cs, biases, count, accumulate, alpha, st);
        default: return launch_vec<BITS, 4>(a, ws, cs, biases, count, accumulate, alpha, st);
    }
}

}  // namespace

int32_t launch_gemv_group(const float* a, const WeightView* ws, float* const* cs, const float* const* biases,
                          int32_t count, int32_t accumulate, float alpha, hipStream_t st) {
    for (int32_t i = 0; i < count; ++i)
        if (biases && biases[i] && !aligned(biases[i], 16))
            return fail(KT_ERR_ARGUMENT, "bias must be 16-byte aligned for the grouped GEMV");
    return ws[0].bits == 4 ? launch_bits<4>(a, ws, cs, biases, count, accumulate, alpha, st)
                           : launch_bits<8>(a, ws, cs, biases, count, accumulate, alpha, st);
}

int32_t launch_gemv(const float* a, const WeightView& w, float* c, int32_t accumulate, float alpha, const float* bias,
                    hipStream_t st) {
    if (bias && !aligned(bias, 16)) return launch_generic(a, 1, w, c, accumulate, alpha, bias, st);
    const float* biases[1] = {bias};
    return launch_gemv_group(a, &w, &c, biases, 1, accumulate, alpha, st);
}

}  // namespace kt
