// kt_decoder.hip -- the rest of the decode/prefill step around the quantized
// projections, on the device: RMSNorm, RoPE with the KV-cache append, cached GQA
// attention, the SwiGLU gate, the greedy argmax and the cache position.
//
// Reference semantics (Engine/kotensor/src/main/kotlin/, K/):
//   RMSNorm.forwardInto          K/RMSNorm.kt:71-90
//   RoPE.invFreq, RoPEScaling     K/RoPE.kt:18-46
//   RoPE.applyRowsInPlace         K/RoPE.kt:139-164 (applyInPlace :117-137 is one row)
//   Attention.prefillInto/decodeInto's cache writes  K/Attention.kt:220-233, 254-270
//   Attention.attendCached/attendHead/dot            K/Attention.kt:277-349
//   SwiGLU gate: siluInPlace, mulInPlace             K/SwiGLU.kt:19-25, K/Tensor.kt:223-237
//   Transformer.argmaxOfLastToken                    K/Transformer.kt:253-266
//   KVCache layout ((layer * kv_heads + head) * max_seq + position) * head_dim,
//   K/KVCache.kt:25-27.
//
// The cache position is a device int32 (the cache length), read by the kernels and
// advanced by kt_position_add, so a whole decode step can be recorded in a HIP graph
// and replayed token after token.
//
// Numerics: the reference's transcendental functions are double-precision results
// rounded to float; the RoPE angles use double cos/sin the same way, and the RoPE
// rotation is computed without contraction, so q and k come out as the reference's.
// RMSNorm, attention and the gate use the GPU's fp32 reductions and expf, which
// differ from the reference's sequential sums by fp32 rounding only.
#include <math.h>

#include "kt_common.h"

namespace kt {
namespace {

constexpr int THREADS = 256;
constexpr int KT = 64;        // keys per attention tile
constexpr int MAX_SPLITS = 64;  // key splits of one (token, kv head); the merge holds one weight per lane
constexpr int MAX_NACC = 4;   // query floats per thread: heads per kv head x head_dim <= 1024
constexpr int ACC_REGS = 8;   // per lane: query heads of its wave x dims of its lane (head_dim / 64 rounded up)
constexpr int MAX_HD = 256;

// Sum and maximum over a wave without LDS round trips: inside each row of 16 lanes by DPP
// exchanges (quad xor 1, quad xor 2, half-row mirror, row mirror: every lane of a row ends
// with the same row total, the two operands of each add being the same pair), then the
// four row totals read into scalars and combined in one fixed order, so every lane holds
// the same bits. Needs every lane of the wave active.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float lane_value(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v += dpp_move<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_move<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_move<0x141>(v);  // row_half_mirror
    v += dpp_move<0x140>(v);  // row_mirror
    return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
}
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = fmaxf(v, dpp_move<0xB1>(v));
    v = fmaxf(v, dpp_move<0x4E>(v));
    v = fmaxf(v, dpp_move<0x141>(v));
    v = fmaxf(v, dpp_move<0x140>(v));
    return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)), fmaxf(lane_value(v, 32), lane_value(v, 48)));
}

// ---- RMSNorm ---------------------------------------------------------------------
// One workgroup per row: out = (x * (1 / sqrt(mean(x^2) + eps))) * weight, the sum of
// squares as norm_partial / norm_wave_sum / norm_scale define it. Rows of up to 8192
// floats (a multiple of 4) stay in registers: one load round trip per row.
static_assert(THREADS == NORM_THREADS, "one thread per norm_partial slot");

__global__ void __launch_bounds__(THREADS) rmsnorm_kernel(const float* __restrict__ x, int32_t dim,
                                                          const float* __restrict__ w, float eps,
                                                          float* __restrict__ out, int32_t aligned16) {
    __shared__ float part[THREADS / 64];
    const float* row = x + static_cast<size_t>(blockIdx.x) * dim;
    float* orow = out + static_cast<size_t>(blockIdx.x) * dim;
    const int32_t tid = threadIdx.x;
    const bool vec = aligned16 && (dim & 3) == 0 && dim <= NORM_F4 * 4 * THREADS;
    norm_v4 v[NORM_F4];
    float s = 0.0f;
    if (vec) {
        const int32_t n4 = dim >> 2;
#pragma unroll
        for (int i = 0; i < NORM_F4; ++i)  // in-bounds unconditional loads, masked in norm_partial
            v[i] = reinterpret_cast<const norm_v4*>(row)[min(tid + i * THREADS, n4 - 1)];
        s = norm_partial(v, tid, n4);
    } else {
        for (int32_t d = tid; d < dim; d += THREADS) s = fmaf(row[d], row[d], s);
    }
    s = norm_wave_sum(s);
    if ((tid & 63) == 0) part[tid >> 6] = s;
    __syncthreads();
    const float r = norm_scale(part, dim, eps);
    if (vec) {
        const int32_t n4 = dim >> 2;
#pragma unroll
        for (int i = 0; i < NORM_F4; ++i) {
            const int32_t e = tid + i * THREADS;
            if (e < n4) {
                const float4 wv = reinterpret_cast<const float4*>(w)[e];
                reinterpret_cast<float4*>(orow)[e] =
                    make_float4(v[i][0] * r * wv.x, v[i][1] * r * wv.y, v[i][2] * r * wv.z, v[i][3] * r * wv.w);
            }
        }
    } else {
        for (int32_t d = tid; d < dim; d += THREADS) orow[d] = row[d] * r * w[d];
    }
}

// ---- RoPE + cache append -----------------------------------------------------------
// Thread (token t, unit u): u < num_heads * half rotates pair i of q head u / half;
// the next num_kv_heads * half units rotate k and write k and v to the cache.
#pragma clang fp contract(off)
// RoPE.applyInPlace's rotation of pair (x1, x2) = (row[i], row[i + half]) at pos:
// theta = pos * invFreq[i] in fp32, cos and sin in double rounded to float, no
// contraction (the whole region is compiled with fp contract off).
__device__ __forceinline__ void rope_cos_sin(int32_t pos, float inv_freq_i, float& c, float& s) {
    const float theta = static_cast<float>(pos) * inv_freq_i;
    c = static_cast<float>(cos(static_cast<double>(theta)));
    s = static_cast<float>(sin(static_cast<double>(theta)));
}
__device__ __forceinline__ void rope_apply(float x1, float x2, float c, float s, float& y1, float& y2) {
    y1 = x1 * c - x2 * s;
    y2 = x1 * s + x2 * c;
}
__device__ __forceinline__ void rope_rotate(float x1, float x2, int32_t pos, float inv_freq_i, float& y1, float& y2) {
    float c, s;
    rope_cos_sin(pos, inv_freq_i, c, s);
    rope_apply(x1, x2, c, s, y1, y2);
}
__global__ void __launch_bounds__(THREADS) rope_kv_kernel(float* __restrict__ q, float* __restrict__ k,
                                                          const float* __restrict__ v, int32_t num_heads,
                                                          int32_t num_kv_heads, int32_t head_dim,
                                                          const float* __restrict__ inv_freq,
                                                          const int32_t* __restrict__ position,
                                                          float* __restrict__ cache_k, float* __restrict__ cache_v,
                                                          int32_t layer, int32_t max_seq) {
    const int32_t half = head_dim >> 1;
    const int32_t t = blockIdx.y;
    const int32_t u = blockIdx.x * THREADS + threadIdx.x;
    const int32_t q_units = num_heads * half, units = q_units + num_kv_heads * half;
    if (u >= units) return;
    const int32_t pos = *position + t;
    if (pos < 0 || pos >= max_seq) return;  // the host checks capacity; never write outside the cache
    const bool is_q = u < q_units;
    const int32_t h = (is_q ? u : u - q_units) / half;
    const int32_t i = (is_q ? u : u - q_units) % half;
    float* row = is_q ? q + static_cast<size_t>(t) * num_heads * head_dim
                      : k + static_cast<size_t>(t) * num_kv_heads * head_dim;
    const int32_t i1 = h * head_dim + i, i2 = i1 + half;
    float y1, y2;
    rope_rotate(row[i1], row[i2], pos, inv_freq[i], y1, y2);
    row[i1] = y1;
    row[i2] = y2;
    if (!is_q) {
        const size_t base = ((static_cast<size_t>(layer) * num_kv_heads + h) * max_seq + pos) * head_dim;
        const float* vrow = v + static_cast<size_t>(t) * num_kv_heads * head_dim;
        cache_k[base + i] = y1;
        cache_k[base + i + half] = y2;
        cache_v[base + i] = vrow[i1];
        cache_v[base + i + half] = vrow[i2];
    }
}
#pragma clang fp contract(on)

// ---- cached attention ------------------------------------------------------------------
struct AttnArgs {
    const float* q;          // [tokens x num_heads * head_dim]
    const int32_t* position;  // cache length before these tokens
    const float* ck;
    const float* cv;
    float* context;          // [tokens x num_heads * head_dim]
    // several splits: each split's sum of weighted values [tokens][num_heads][splits][head_dim]
    // and its (max, sum) as tagged words [tokens][num_heads][splits][2] (zero between launches)
    float* partials;
    uint64_t* stats;
    int32_t layer, max_seq, num_heads, num_kv_heads, head_dim, splits, span;
    float scale;
    // one decode token with RoPE and the cache append inside: q, k_new, v_new are the
    // projections before RoPE (rope_kv_kernel's inputs)
    const float* k_new;
    const float* v_new;
    const float* inv_freq;
    int32_t rope;
    // one decode token: per frequency i, words 4i .. 4i + 3 = (position + 1, inv_freq[i]'s
    // bits, cos, sin) as layer 0's launch computed them; layer 0 writes them, later
    // layers' launches use an entry whose position and frequency match (or null: none)
    uint32_t* rope_cache;
    // the merge's bounded wait: the stream's fault word (set when it gives up), its poll
    // budget, and the test hook that makes the other splits withhold their tagged words
    int32_t* fault;
    uint32_t spin_limit;
    int32_t withhold;
};

// Workgroup (kv head g, key split s, token t): the G = num_heads / num_kv_heads query
// heads of kv head g over keys [s * span, min((s + 1) * span, position + t + 1)), in
// tiles of 64 keys with a running maximum and sum (scores, then exp(score - max),
// then the weighted values). With one split the workgroup writes the context; with
// several the last split in dispatch order merges every split's (sum of weighted values,
// max, sum) and writes the context.
// Wave w owns query heads w, w + 4, ...: for the scores lane l is key l of the tile (its
// key row read from LDS 16 bytes at a time, the query row a broadcast), so the running
// maximum and sum are wave reductions on registers; for the weighted values lane l holds
// dims l, l + 64, ... and reads the wave's own row of exponentials back from LDS. The
// tile is the only thing the waves share: one barrier after it lands, one before the next.
// Every global load of a tile is issued before the first is used (unrolled, predicated
// float4 loads into registers, then LDS), so a tile costs one memory round trip.
// TF4: float4 per thread for a full tile (4, 8, 16 for head_dim up to 64, 128, 256).
// Unconditional loads of in-bounds addresses (indices past the tile repeat its last
// float4; the stores are masked): no branch around a load, so all go out together.
// (native 4-vectors: the registers of a tile stay registers across the loop)
typedef float f4 __attribute__((ext_vector_type(4)));
template <int TF4>
__device__ __forceinline__ void load_tile(f4 (&r)[TF4], const float* src, int32_t n4) {
#pragma unroll
    for (int i = 0; i < TF4; ++i) {
        const int32_t e = min(static_cast<int32_t>(threadIdx.x) + i * THREADS, n4 - 1);
        r[i] = reinterpret_cast<const f4*>(src)[e];
    }
}

// A split's max or sum word for the merge: the float's bits, the tag 1 above them.
__device__ __forceinline__ uint64_t tagged(float v) {
    return (uint64_t{1} << 32) | __builtin_bit_cast(uint32_t, v);
}
constexpr int MERGE_BATCH = 8;             // 16-byte loads of other splits' values a merging lane has in flight
constexpr int COHERENT_AUX = 1 | 16;       // buffer-load cache bits sc0 sc1: read past the caches
constexpr uint32_t MERGE_SPIN_LIMIT = 1u << 20;  // polls per merging lane, over all its waits
__device__ __forceinline__ bool is_tagged(uint64_t w) { return (w >> 32) == 1u; }
// Words w[u] = *(base + min(u, count - 1) * stride) (each already loaded once) until
// every tag of u < count is 1: each round reloads all N words, unconditionally (a load
// under a branch is waited for at the branch's end), so a round costs one memory round
// trip whatever the count; a word stays tagged once it is. The rounds of a lane share
// one budget, so that a fault shows as a wrong result within about a second rather than
// as a hang.
// Returns whether every word is tagged (false: the budget ran out first).
template <int N>
__device__ __forceinline__ bool await_tagged(uint64_t (&w)[N], uint64_t* base, int32_t stride, int32_t count,
                                             uint32_t& budget) {
    for (;;) {
        bool all = true;
#pragma unroll
        for (int u = 0; u < N; ++u) all = all && (u >= count || is_tagged(w[u]));
        if (all) return true;
        if (budget == 0) return false;
        --budget;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int u = 0; u < N; ++u)
            w[u] = __hip_atomic_load(base + min(u, count - 1) * stride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

template <int TF4>
__global__ void __launch_bounds__(THREADS) attention_kernel(AttnArgs a) {
    extern __shared__ float smem[];
    const int32_t g = blockIdx.x, s = blockIdx.y, t = blockIdx.z;
    const int32_t HD = a.head_dim, G = a.num_heads / a.num_kv_heads;
    const int32_t dim = a.num_heads * HD;
    const int32_t KP = HD + 4;  // padded key row: 16-byte reads of consecutive rows hit distinct banks
    float* qs = smem;                  // [G][HD]
    float* ks = qs + G * HD;           // [KT][HD + 4]
    float* vs = ks + KT * KP;          // [KT][HD]
    float* sc = vs + KT * HD;          // [G][KT] each wave's exponentials of its heads
    float* st = sc + G * KT;           // [G] x {m, l, alpha}
    float* kn_s = st + 3 * G;          // [HD] the new key after RoPE (the workgroup holding it), then one word
    const int32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

    const int32_t k_begin = s * a.span;
    const size_t base = (static_cast<size_t>(a.layer) * a.num_kv_heads + g) * a.max_seq;  // row of key 0
    // q of the G heads (G * HD <= 1024 floats: at most one float4 per thread)
    const int32_t q4 = G * HD / 4;
    float4 qv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (tid < q4) qv = reinterpret_cast<const float4*>(a.q + static_cast<size_t>(t) * dim + g * G * HD)[tid];
    // RoPE inputs (a decode token): this thread's frequency and, for the workgroup that
    // turns out to hold the new position, its pair of the new key and value. Issued ahead
    // of the tiles, so that the rotation below waits for them and not for the tiles.
    const int32_t half = HD >> 1;
    float ifr = 0.0f, kn1 = 0.0f, kn2 = 0.0f, vn1 = 0.0f, vn2 = 0.0f;
    // layers after the first take cos and sin of their position from the cache layer 0's
    // launch wrote (read past the caches: that launch wrote them through)
    const bool cache_read = a.rope_cache && a.layer != 0;
    uint32_t ce[4] = {0u, 0u, 0u, 0u};
    if (a.rope && tid < half) {
        const float* kn = a.k_new + static_cast<size_t>(g) * HD;
        const float* vn = a.v_new + static_cast<size_t>(g) * HD;
        ifr = a.inv_freq[tid];
        kn1 = kn[tid];
        kn2 = kn[tid + half];
        vn1 = vn[tid];
        vn2 = vn[tid + half];
        if (cache_read) {
#pragma unroll
            for (int w = 0; w < 4; ++w)
                ce[w] = __hip_atomic_load(a.rope_cache + 4 * tid + w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
    // The first tile's keys and values go out with q and the position, before anything
    // waits: a whole tile from k_begin (rows of the cache, k_begin < max_seq), so the
    // addresses do not wait for the position; rows past the key range are never used.
    constexpr bool TOGETHER = TF4 <= 8;
    f4 kr[TF4], vr[TOGETHER ? TF4 : 1];
    {
        const int32_t n4 = min(KT, a.max_seq - k_begin) * HD / 4;
        load_tile<TF4>(kr, a.ck + (base + k_begin) * HD, n4);
        if constexpr (TOGETHER) load_tile<TF4>(vr, a.cv + (base + k_begin) * HD, n4);
    }
    const int32_t pos = *a.position + t;
    const int32_t k_end = min(min(k_begin + a.span, pos + 1), a.max_seq);  // never read outside the cache
    // With RoPE inside, the workgroup whose key range holds the new position appends the
    // rotated key and the value to the cache for later steps and uses them from LDS in
    // its own tile (its tile load may see the row before or after the append; the LDS copy
    // replaces it), so no fence or second read of the row is needed.
    const bool holder = a.rope && pos >= k_begin && pos < k_end;
    constexpr int NW = THREADS / 64;
    constexpr int DPL = (TF4 + 3) / 4;     // dims per lane: head_dim <= 64 DPL
    constexpr int MAXH = ACC_REGS / DPL;   // query heads per wave
    float acc[MAXH][DPL], mrun[MAXH], lrun[MAXH];
#pragma unroll
    for (int h = 0; h < MAXH; ++h) {
        mrun[h] = -INFINITY;
        lrun[h] = 0.0f;
#pragma unroll
        for (int dd = 0; dd < DPL; ++dd) acc[h][dd] = 0.0f;
    }

    if (a.rope) {
        // one decode token: the G query heads are rotated in LDS; the holder rotates the
        // new key into LDS and appends it and the value to the cache
        if (tid < q4) reinterpret_cast<float4*>(qs)[tid] = qv;
        float* fc = vs;         // cos and sin of each frequency, until the first tile lands in vs
        float* fsn = vs + half;
        float cf = 0.0f, sf = 0.0f;
        if (tid < half) {
            if (cache_read && ce[0] == static_cast<uint32_t>(pos) + 1u && ce[1] == __builtin_bit_cast(uint32_t, ifr)) {
                cf = __builtin_bit_cast(float, ce[2]);
                sf = __builtin_bit_cast(float, ce[3]);
            } else {
                rope_cos_sin(pos, ifr, cf, sf);
            }
            fc[tid] = cf;
            fsn[tid] = sf;
            if (a.rope_cache && a.layer == 0 && g == 0 && s == 0) {
                uint32_t* e = a.rope_cache + 4 * tid;
                __hip_atomic_store(e, static_cast<uint32_t>(pos) + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                __hip_atomic_store(e + 1, __builtin_bit_cast(uint32_t, ifr), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                __hip_atomic_store(e + 2, __builtin_bit_cast(uint32_t, cf), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                __hip_atomic_store(e + 3, __builtin_bit_cast(uint32_t, sf), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
        }
        __syncthreads();
        for (int32_t e = tid; e < G * half; e += THREADS) {
            const int32_t i = e % half, hh = e / half;
            float y1, y2;
            rope_apply(qs[hh * HD + i], qs[hh * HD + i + half], fc[i], fsn[i], y1, y2);
            qs[hh * HD + i] = y1;
            qs[hh * HD + i + half] = y2;
        }
        if (holder && tid < half) {  // half <= THREADS: one pair per thread
            float* ckw = const_cast<float*>(a.ck) + (base + pos) * HD;
            float* cvw = const_cast<float*>(a.cv) + (base + pos) * HD;
            float y1, y2;
            rope_apply(kn1, kn2, cf, sf, y1, y2);
            kn_s[tid] = y1;
            kn_s[tid + half] = y2;
            ckw[tid] = y1;
            ckw[tid + half] = y2;
            cvw[tid] = vn1;
            cvw[tid + half] = vn2;
        }
        __syncthreads();
    }

    // K and V tiles in registers together (one round trip) up to head_dim 128; wider
    // heads load them one after the other to keep the registers in bounds.
    for (int32_t k0 = k_begin; k0 < k_end; k0 += KT) {
        const int32_t n = min(KT, k_end - k0);
        const int32_t n4 = n * HD / 4;
        if (k0 != k_begin) {
            load_tile<TF4>(kr, a.ck + (base + k0) * HD, n4);
            if constexpr (TOGETHER) load_tile<TF4>(vr, a.cv + (base + k0) * HD, n4);
        }
        if (!a.rope && k0 == k_begin && tid < q4) reinterpret_cast<float4*>(qs)[tid] = qv;
#pragma unroll
        for (int i = 0; i < TF4; ++i) {
            const int32_t e = tid + i * THREADS;
            if (e < n4) {
                const int32_t j = (4 * e) / HD, d = (4 * e) % HD;
                *reinterpret_cast<f4*>(ks + j * KP + d) = kr[i];
                if constexpr (TOGETHER) reinterpret_cast<f4*>(vs)[e] = vr[i];
            }
        }
        if constexpr (!TOGETHER) {
            load_tile<TF4>(kr, a.cv + (base + k0) * HD, n4);
#pragma unroll
            for (int i = 0; i < TF4; ++i) {
                const int32_t e = tid + i * THREADS;
                if (e < n4) reinterpret_cast<f4*>(vs)[e] = kr[i];
            }
        }
        if (holder && pos >= k0 && pos < k0 + n) {
            // the new row from LDS and the projection, whatever the tile load saw (each
            // thread replaces elements it did not write, so the tile writes come first)
            __syncthreads();
            const int32_t j = pos - k0;
            if (tid < half) {
                ks[j * KP + tid] = kn_s[tid];
                ks[j * KP + tid + half] = kn_s[tid + half];
                vs[j * HD + tid] = vn1;
                vs[j * HD + tid + half] = vn2;
            }
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < MAXH; ++h) {
            const int32_t hh = wave + h * NW;
            if (hh >= G) break;
            // score of key `lane` (four interleaved sums over the head's dims)
            // (eight 16-byte pairs in flight per group: indices past the row repeat its last
            // float4 and add nothing)
            float score = -INFINITY;
            if (lane < n) {
                const f4* qi = reinterpret_cast<const f4*>(qs + hh * HD);
                const f4* kj = reinterpret_cast<const f4*>(ks + lane * KP);
                const int32_t HD4 = HD >> 2;
                float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
                for (int32_t g0 = 0; g0 < HD4; g0 += 8) {
                    f4 qv4[8], kv4[8];
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        const int32_t d4 = min(g0 + u, HD4 - 1);
                        qv4[u] = qi[d4];
                        kv4[u] = kj[d4];
                    }
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        if (g0 + u < HD4) {
                            s0 = fmaf(qv4[u].x, kv4[u].x, s0);
                            s1 = fmaf(qv4[u].y, kv4[u].y, s1);
                            s2 = fmaf(qv4[u].z, kv4[u].z, s2);
                            s3 = fmaf(qv4[u].w, kv4[u].w, s3);
                        }
                    }
                }
                score = ((s0 + s1) + (s2 + s3)) * a.scale;
            }
            // running max and sum of the head
            const float m_old = mrun[h];
            const float m_new = fmaxf(m_old, wave_max_dpp(score));
            const float ex = lane < n ? expf(score - m_new) : 0.0f;
            const float sum = wave_sum_dpp(ex);
            const float alpha = m_old == -INFINITY ? 0.0f : expf(m_old - m_new);
            mrun[h] = m_new;
            lrun[h] = lrun[h] * alpha + sum;
            // weighted values: the wave's row of exponentials goes through LDS (a wave's
            // LDS accesses complete in order; the wave barrier keeps the compiler from
            // moving the reads above the write)
            float* ep = sc + hh * KT;
            ep[lane] = ex;
            __builtin_amdgcn_wave_barrier();
#pragma unroll
            for (int dd = 0; dd < DPL; ++dd) {
                const int32_t d = lane + 64 * dd;
                if (d < HD) {
                    float x = acc[h][dd] * alpha;
                    const float* vp = vs + d;
                    int32_t j = 0;
                    for (; j + 16 <= n; j += 16) {  // 20 reads in flight, then the 16 in order
                        f4 e4[4];
                        float vv[16];
#pragma unroll
                        for (int u = 0; u < 4; ++u) e4[u] = *reinterpret_cast<const f4*>(ep + j + 4 * u);
#pragma unroll
                        for (int u = 0; u < 16; ++u) vv[u] = vp[(j + u) * HD];
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            x = fmaf(e4[u].x, vv[4 * u], x);
                            x = fmaf(e4[u].y, vv[4 * u + 1], x);
                            x = fmaf(e4[u].z, vv[4 * u + 2], x);
                            x = fmaf(e4[u].w, vv[4 * u + 3], x);
                        }
                    }
                    for (; j + 4 <= n; j += 4) {
                        const f4 e4 = *reinterpret_cast<const f4*>(ep + j);
                        x = fmaf(e4.x, vp[j * HD], x);
                        x = fmaf(e4.y, vp[(j + 1) * HD], x);
                        x = fmaf(e4.z, vp[(j + 2) * HD], x);
                        x = fmaf(e4.w, vp[(j + 3) * HD], x);
                    }
                    for (; j < n; ++j) x = fmaf(ep[j], vp[j * HD], x);
                    acc[h][dd] = x;
                }
            }
            __builtin_amdgcn_wave_barrier();
        }
        __syncthreads();
    }

    if (a.splits == 1) {
#pragma unroll
        for (int h = 0; h < MAXH; ++h) {
            const int32_t hh = wave + h * NW;
            if (hh >= G) break;
#pragma unroll
            for (int dd = 0; dd < DPL; ++dd) {
                const int32_t d = lane + 64 * dd;
                if (d < HD) a.context[static_cast<size_t>(t) * dim + (g * G + hh) * HD + d] = acc[h][dd] * (1.0f / lrun[h]);
            }
        }
        return;
    }
    // Several splits: each split but the last writes its sums of weighted values through
    // to memory, waits until they are there, then writes its (max, sum) as 64-bit words,
    // the float's bits under the tag 1, and is done (no counter). The last split of the
    // (token, kv head), dispatched after the others, merges: it polls the (max, sum) words
    // past the caches (a word is ready when its tag is 1; the 64-bit store is single-copy
    // atomic), whereupon that split's values are in memory, and reads those 16 bytes at a
    // time, several splits per load instruction. It merges every split with its own from
    // registers, as attn_combine_kernel does (each lane a strided share of the splits, the
    // shares added in a fixed order), and returns the (max, sum) words to zero, so their
    // region (the workspace's zeroed area) is zero again when the launch ends. It waits
    // only for workgroups dispatched before it; the polls are bounded all the same. (In
    // decode the last split usually holds no keys, the key bound being the cache's
    // capacity, so it is free to wait from the start.)
    const int32_t S = a.splits;
    const size_t pbase = (static_cast<size_t>(t) * a.num_heads + g * G) * S;  // (head g G, split 0)
    if (s != S - 1) {
#pragma unroll
        for (int h = 0; h < MAXH; ++h) {
            const int32_t hh = wave + h * NW;
            if (hh >= G) break;
            float* pv = a.partials + (pbase + static_cast<size_t>(hh) * S + s) * HD;
#pragma unroll
            for (int dd = 0; dd < DPL; ++dd) {
                const int32_t d = lane + 64 * dd;
                if (d < HD) __hip_atomic_store(pv + d, acc[h][dd], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
            // this wave's values are in memory before its (max, sum) words go out
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_s_waitcnt(0);
            if (lane == 0 && !a.withhold) {
                uint64_t* ps = a.stats + (pbase + static_cast<size_t>(hh) * S + s) * 2;
                __hip_atomic_store(ps, tagged(mrun[h]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
                __hip_atomic_store(ps + 1, tagged(lrun[h]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            }
        }
        return;
    }
    float* ws = sc;  // [G][KT] each wave's weights of its heads (S <= MAX_SPLITS <= KT)
    float* red = ks + wave * 256;  // this wave's shares of the merged values, [phases][HD]
    const int32_t others = S - 1;
    uint32_t budget = a.spin_limit;
    // values: lane = (phase q, float4 r of the row); a load instruction covers `phases`
    // splits' rows (HD / 4 lanes each)
    const int32_t quads = HD >> 2, phases = 64 / quads;
    const int32_t q = lane / quads, r = lane - q * quads;
    const size_t vbytes = static_cast<size_t>(gridDim.z) * a.num_heads * S * HD * sizeof(float);
    const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(a.partials, 0, static_cast<int32_t>(vbytes),
                                                                        0x00020000);
#pragma unroll
    for (int h = 0; h < MAXH; ++h) {
        const int32_t hh = wave + h * NW;
        if (hh >= G) break;
        // split `lane`'s max and sum (this workgroup's own in lane S - 1)
        uint64_t* ps = a.stats + (pbase + static_cast<size_t>(hh) * S) * 2;  // split 0 of head hh
        uint64_t ml[2] = {0, 0};
        float ms = -INFINITY, ls = 0.0f;
        if (lane < others) {
            ml[0] = __hip_atomic_load(ps + 2 * lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            ml[1] = __hip_atomic_load(ps + 2 * lane + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            if (!await_tagged(ml, ps + 2 * lane, 1, 2, budget) && a.fault)
                __hip_atomic_store(a.fault, FAULT_MERGE_WAIT, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            ms = __builtin_bit_cast(float, static_cast<uint32_t>(ml[0]));
            ls = __builtin_bit_cast(float, static_cast<uint32_t>(ml[1]));
            __hip_atomic_store(ps + 2 * lane, uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(ps + 2 * lane + 1, uint64_t{0}, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        } else if (lane == others) {
            ms = mrun[h];
            ls = lrun[h];
        }
        const float m = wave_max_dpp(ms);
        const float w = ms == -INFINITY ? 0.0f : expf(ms - m);
        const float l = wave_sum_dpp(w * ls);
        ws[hh * KT + lane] = w;
        // every split's (max, sum) seen: their values are in memory; no read below may
        // move above the polls
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        // this lane's share: splits q, q + phases, ... of float4 r, in that order
        f4 x4 = {0.0f, 0.0f, 0.0f, 0.0f};
        const size_t row0 = (pbase + static_cast<size_t>(hh) * S) * HD;  // split 0's row of head hh
        for (int32_t b0 = 0; b0 < others; b0 += MERGE_BATCH * phases) {
            f4 vv[MERGE_BATCH];
#pragma unroll
            for (int u = 0; u < MERGE_BATCH; ++u) {
                const int32_t sp = min(b0 + q + u * phases, others - 1);
                vv[u] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(
                                                   pr, static_cast<int32_t>((row0 + static_cast<size_t>(sp) * HD + 4 * r) * 4),
                                                   0, COHERENT_AUX));
            }
#pragma unroll
            for (int u = 0; u < MERGE_BATCH; ++u) {
                const int32_t sp = b0 + q + u * phases;
                if (q < phases && sp < others) {
                    const float wsp = ws[hh * KT + sp];
                    x4.x = fmaf(vv[u].x, wsp, x4.x);
                    x4.y = fmaf(vv[u].y, wsp, x4.y);
                    x4.z = fmaf(vv[u].z, wsp, x4.z);
                    x4.w = fmaf(vv[u].w, wsp, x4.w);
                }
            }
        }
        if (q < phases) *reinterpret_cast<f4*>(red + q * HD + 4 * r) = x4;
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int dd = 0; dd < DPL; ++dd) {
            const int32_t d = lane + 64 * dd;
            if (d >= HD) continue;
            float x = 0.0f;
            for (int32_t p = 0; p < phases; ++p) x += red[p * HD + d];
            x = fmaf(acc[h][dd], ws[hh * KT + others], x);
            a.context[static_cast<size_t>(t) * dim + (g * G + hh) * HD + d] = x * (1.0f / l);
        }
        __builtin_amdgcn_wave_barrier();
    }
}

// ---- prefill attention: blocked over queries, fp32 MFMA ---------------------------------
// Workgroup (kv head g, block of QB = 128 / G consecutive tokens): the query rows
// r = (token t0 + r / G, head g G + r % G), r < QB G, over keys 0 .. position + token,
// 64 keys at a time; K and V tiles in LDS serve the four waves (32 rows each), so a key
// row is read once per workgroup instead of once per token. Both products run on
// v_mfma_f32_32x32x2_f32 (fp32 operands, fp32 sums; the reference's arithmetic up to
// summation order):
//   S^T = K Q^T: lane l ends with the scores of query row l % 32 against the 16 keys
//     8 (e / 4) + 4 (l / 32) + e % 4 of each 32-key block (register e), so the running
//     maximum, the exponentials and the rescaling of a row stay inside lanes l, l ^ 32;
//   O^T += V^T P^T, taking the keys of each block in that same order: the B operand of
//     step e is register e of the scores, as they lie.
// Blocks go out longest first (the last tokens see the most keys).
constexpr int PQ_ROWS = 128;  // query rows per workgroup
constexpr int PKT = 64;       // keys per tile
constexpr int PREFILL_MIN_TOKENS = 16;  // fewer tokens: the per-token kernel with key splits
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));

template <int HD>
__global__ void __launch_bounds__(THREADS) attention_prefill_kernel(AttnArgs a, int32_t tokens, int32_t qb_tokens,
                                                                    int32_t nqb) {
    extern __shared__ float smem[];
    constexpr int KP = HD + 1;  // K row stride: 32 lanes on 32 rows hit distinct banks
    constexpr int VP = HD + 8;  // V row stride: the two half-waves read rows 4 apart on other banks
    constexpr int DB = HD / 32;
    constexpr int QS = HD / 2;
    constexpr int TF = PKT * HD / 4 / THREADS;  // float4 of a K (V) tile per thread
    const int32_t g = blockIdx.x;
    const int32_t qb = nqb - 1 - static_cast<int32_t>(blockIdx.y);
    const int32_t G = a.num_heads / a.num_kv_heads;
    const int32_t dim = a.num_heads * HD;
    const int32_t t0 = qb * qb_tokens;
    const int32_t t_end = min(t0 + qb_tokens, tokens);
    const int32_t P0 = *a.position;
    const int32_t n_keys = min(P0 + t_end, a.max_seq);  // never read outside the cache
    const size_t base = (static_cast<size_t>(a.layer) * a.num_kv_heads + g) * a.max_seq;  // row of key 0
    const int32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int32_t rl = lane & 31, h = lane >> 5;

    const int32_t r = wave * 32 + rl;  // this lane's query row
    const int32_t tl = r / G;
    const int32_t tok = t0 + tl;
    const bool row_ok = tl < qb_tokens && tok < t_end;
    const int32_t head = g * G + r % G;
    const int32_t p_r = row_ok ? min(P0 + tok, a.max_seq - 1) : -1;  // last key of the row

    // the query rows through LDS into each lane's MFMA fragment: Q[r][2 s + h]
    float qf[QS];
    {
        float* qs = smem;  // [PQ_ROWS][KP]
        for (int32_t e = tid; e < PQ_ROWS * HD / 4; e += THREADS) {
            const int32_t rr = e / (HD / 4), c4 = e % (HD / 4);
            const int32_t tt = t0 + rr / G;
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (rr / G < qb_tokens && tt < t_end)
                v = *reinterpret_cast<const float4*>(a.q + static_cast<size_t>(tt) * dim + (g * G + rr % G) * HD + 4 * c4);
            float* d = qs + rr * KP + 4 * c4;
            d[0] = v.x;
            d[1] = v.y;
            d[2] = v.z;
            d[3] = v.w;
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < QS; ++s) qf[s] = qs[r * KP + 2 * s + h];
        __syncthreads();  // the area becomes the K and V tiles
    }

    float* ks = smem;             // [PKT][KP]
    float* vs = smem + PKT * KP;  // [PKT][VP]
    f32x16 oacc[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int e = 0; e < 16; ++e) oacc[db][e] = 0.0f;
    float m = -INFINITY, l = 0.0f;

    // a tile's K and V rows, all loads out before the first is used; rows past n_keys
    // repeat the last key and are masked, and the tile after the last one repeats it
    // (unconditional loads: no branch, and the arrays stay in registers)
    v4f kr[TF], vr[TF];  // (native vectors: the HIP float4 struct keeps the arrays in scratch)
#pragma unroll
    for (int i = 0; i < TF; ++i) {
        const int32_t e = tid + i * THREADS;
        const int32_t j = e / (HD / 4), c4 = e % (HD / 4);
        const size_t row = base + min(j, n_keys - 1);
        kr[i] = *reinterpret_cast<const v4f*>(a.ck + row * HD + 4 * c4);
        vr[i] = *reinterpret_cast<const v4f*>(a.cv + row * HD + 4 * c4);
    }
    for (int32_t k0 = 0; k0 < n_keys; k0 += PKT) {
#pragma unroll
        for (int i = 0; i < TF; ++i) {
            const int32_t e = tid + i * THREADS;
            const int32_t j = e / (HD / 4), c4 = e % (HD / 4);
            float* kd = ks + j * KP + 4 * c4;
            kd[0] = kr[i][0];
            kd[1] = kr[i][1];
            kd[2] = kr[i][2];
            kd[3] = kr[i][3];
            *reinterpret_cast<v4f*>(vs + j * VP + 4 * c4) = vr[i];
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < TF; ++i) {
            const int32_t e = tid + i * THREADS;
            const int32_t j = e / (HD / 4), c4 = e % (HD / 4);
            const size_t row = base + min(k0 + PKT + j, n_keys - 1);
            kr[i] = *reinterpret_cast<const v4f*>(a.ck + row * HD + 4 * c4);
            vr[i] = *reinterpret_cast<const v4f*>(a.cv + row * HD + 4 * c4);
        }

        // S^T = K Q^T for the two 32-key blocks
        f32x16 sacc[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
            for (int e = 0; e < 16; ++e) sacc[kb][e] = 0.0f;
#pragma unroll
            for (int s = 0; s < QS; ++s)
                sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(ks[(kb * 32 + rl) * KP + 2 * s + h], qf[s], sacc[kb], 0,
                                                                0, 0);
        }
        // scale, causal mask, running max and sum of the row (lanes l and l ^ 32)
        float tmax = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int32_t j = k0 + kb * 32 + 8 * (e >> 2) + 4 * h + (e & 3);
                const float v = j <= p_r ? sacc[kb][e] * a.scale : -INFINITY;
                sacc[kb][e] = v;
                tmax = fmaxf(tmax, v);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float m_new = fmaxf(m, tmax);
        const bool none = m_new == -INFINITY;  // no key of the row yet (a padding row)
        const float alpha = none || m == -INFINITY ? (none ? 1.0f : 0.0f) : expf(m - m_new);
        float psum = 0.0f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float p = none ? 0.0f : expf(sacc[kb][e] - m_new);
                sacc[kb][e] = p;
                psum += p;
            }
        psum += __shfl_xor(psum, 32);
        l = l * alpha + psum;
        m = m_new;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int e = 0; e < 16; ++e) oacc[db][e] *= alpha;
        // O^T += V^T P^T, the keys of block kb in the order of the score registers
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const float* vrow = vs + (kb * 32 + 8 * (e >> 2) + 4 * h + (e & 3)) * VP + rl;
#pragma unroll
                for (int db = 0; db < DB; ++db)
                    oacc[db] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[db * 32], sacc[kb][e], oacc[db], 0, 0, 0);
            }
        __syncthreads();  // the tiles are read before the next store
    }

    // O^T element (d, r) of block db: lane r + 32 ((d / 4) % 2), register (d / 8) * 4 + d % 4
    if (row_ok) {
        const float inv = 1.0f / l;
        float* dst = a.context + static_cast<size_t>(tok) * dim + head * HD;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int c = 0; c < 4; ++c)
                *reinterpret_cast<float4*>(dst + db * 32 + 8 * c + 4 * h) =
                    make_float4(oacc[db][4 * c] * inv, oacc[db][4 * c + 1] * inv, oacc[db][4 * c + 2] * inv,
                                oacc[db][4 * c + 3] * inv);
    }
}

size_t attention_prefill_lds(int32_t head_dim) {
    const size_t q = static_cast<size_t>(PQ_ROWS) * (head_dim + 1);
    const size_t kv = static_cast<size_t>(PKT) * (head_dim + 1) + static_cast<size_t>(PKT) * (head_dim + 8);
    return (q > kv ? q : kv) * sizeof(float);
}

// ---- SwiGLU gate -----------------------------------------------------------------------
__global__ void __launch_bounds__(THREADS) silu_mul_kernel(float* __restrict__ gate, const float* __restrict__ up,
                                                           int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * THREADS + threadIdx.x;
    if (i >= n) return;
    const float x = gate[i];
    const float silu = x / (1.0f + static_cast<float>(exp(-static_cast<double>(x))));
    gate[i] = silu * up[i];
}

// ---- argmax ----------------------------------------------------------------------------
// Key of a candidate logit: larger value first, then smaller index. Logits not above
// -1e9 (and NaNs) are not candidates; with none the key stays 0 and the index is 0.
__device__ __forceinline__ uint64_t argmax_key(float v, int32_t idx) {
    if (!(v > -1e9f)) return 0;
    uint32_t b = __float_as_uint(v);
    b = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return (static_cast<uint64_t>(b) << 32) | static_cast<uint32_t>(0xFFFFFFFFu - static_cast<uint32_t>(idx));
}
__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const uint64_t w = (static_cast<uint64_t>(__shfl_xor(static_cast<uint32_t>(v >> 32), o, 64)) << 32) |
                           __shfl_xor(static_cast<uint32_t>(v), o, 64);
        v = max_u64(v, w);
    }
    return v;
}

// Each workgroup reduces a stride of the logits into partials[block]; the last one to
// finish (counter) reduces the partials, writes the index and resets the counter.
// advance > 0 (one greedy decode step's bookkeeping): the last workgroup also adds advance
// to *position and records the token at the new position (position_add_kernel, then
// record_token_kernel; the argmax does not read the position).
__global__ void __launch_bounds__(THREADS) argmax_kernel(const float* __restrict__ logits, int32_t n,
                                                         int32_t* __restrict__ index, uint64_t* partials,
                                                         uint32_t* counter, int32_t* position, int32_t advance,
                                                         int32_t* generated, int32_t capacity) {
    __shared__ uint64_t part[THREADS / 64];
    __shared__ uint32_t last;
    uint64_t best = 0;
    for (int32_t i = blockIdx.x * THREADS + threadIdx.x; i < n; i += gridDim.x * THREADS)
        best = max_u64(best, argmax_key(logits[i], i));
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t b = part[0];
        for (int i = 1; i < THREADS / 64; ++i) b = max_u64(b, part[i]);
        __hip_atomic_store(partials + blockIdx.x, b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
        last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
    }
    __syncthreads();
    if (!last) return;
    uint64_t b = 0;
    for (int32_t i = threadIdx.x; i < static_cast<int32_t>(gridDim.x); i += THREADS)
        b = max_u64(b, __hip_atomic_load(partials + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    b = wave_max_u64(b);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = b;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < THREADS / 64; ++i) b = max_u64(b, part[i]);
        b = max_u64(b, part[0]);
        const int32_t token = b == 0 ? 0 : static_cast<int32_t>(0xFFFFFFFFu - static_cast<uint32_t>(b));
        *index = token;
        if (advance) {
            const int32_t p = *position + advance;
            *position = p;
            if (generated && p >= 0 && p < capacity) generated[p] = token;
        }
        __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// ---- residual add and synthetic weights ---------------------------------------------
__global__ void __launch_bounds__(THREADS) add_kernel(float* __restrict__ x, const float* __restrict__ y, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * THREADS + threadIdx.x;
    if (i < n) x[i] = x[i] + y[i];
}

// SplitMix64 of (seed, index): the same value for an element whatever the launch shape.
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
// Element i: Box-Muller on two 53-bit uniforms drawn from (seed, i).
__global__ void __launch_bounds__(THREADS) fill_normal_kernel(float* __restrict__ out, int64_t n, uint64_t seed,
                                                              float mean, float stddev) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * THREADS + threadIdx.x;
    if (i >= n) return;
    const uint64_t a = splitmix64(seed ^ splitmix64(2 * static_cast<uint64_t>(i)));
    const uint64_t b = splitmix64(seed ^ splitmix64(2 * static_cast<uint64_t>(i) + 1));
    const double u1 = (static_cast<double>(a >> 11) + 1.0) * 0x1.0p-53;  // (0, 1]
    const double u2 = static_cast<double>(b >> 11) * 0x1.0p-53;          // [0, 1)
    const double z = sqrt(-2.0 * log(u1)) * cos(2.0 * 3.141592653589793 * u2);
    out[i] = static_cast<float>(static_cast<double>(mean) + static_cast<double>(stddev) * z);
}

__global__ void position_add_kernel(int32_t* position, int32_t count) {
    if (threadIdx.x == 0) *position += count;
}

// generated[*position] = *token, when the position lies inside [0, capacity).
__global__ void record_token_kernel(const int32_t* token, const int32_t* position, int32_t* generated, int32_t capacity) {
    if (threadIdx.x == 0) {
        const int32_t p = *position;
        if (p >= 0 && p < capacity) generated[p] = *token;
    }
}

constexpr int32_t ARGMAX_BLOCKS = 64;

size_t attention_lds(int32_t G, int32_t HD) {
    return sizeof(float) * (static_cast<size_t>(G) * HD + static_cast<size_t>(KT) * (HD + 4) +
                            static_cast<size_t>(KT) * HD + static_cast<size_t>(G) * KT + 3 * static_cast<size_t>(G) +
                            static_cast<size_t>(HD) + 1);
}

}  // namespace
}  // namespace kt

using namespace kt;

extern "C" {

int32_t kt_rope_inv_freq(int32_t head_dim, float base, float factor, float low, float high, int32_t original_max,
                         float* out) {
    if (head_dim <= 0 || head_dim % 2 != 0) return fail(KT_ERR_ARGUMENT, "RoPE dimension must be even");
    if (!out) return fail(KT_ERR_ARGUMENT, "out is NULL");
    if (factor > 0.0f) {
        if (original_max <= 0) return fail(KT_ERR_ARGUMENT, "Invalid RoPE scaling");
        if (!(high > low)) return fail(KT_ERR_ARGUMENT, "highFrequencyFactor must exceed lowFrequencyFactor");
    }
    const double java_pi = 3.141592653589793;
    for (int32_t i = 0; i < head_dim / 2; ++i) {
        const float exponent = static_cast<float>(2 * i) / static_cast<float>(head_dim);
        float f = 1.0f / static_cast<float>(pow(static_cast<double>(base), static_cast<double>(exponent)));
        if (factor > 0.0f) {
            const float low_wl = static_cast<float>(original_max) / low;
            const float high_wl = static_cast<float>(original_max) / high;
            const float wl = static_cast<float>(2.0 * java_pi / static_cast<double>(f));
            if (wl < high_wl) {
            } else if (wl > low_wl) {
                f = f / factor;
            } else {
                const float smooth = (static_cast<float>(original_max) / wl - low) / (high - low);
                f = (1.0f - smooth) * f / factor + smooth * f;
            }
        }
        out[i] = f;
    }
    return KT_OK;
}

int32_t kt_rmsnorm(const float* x, int32_t rows, int32_t dim, const float* weight, float eps, float* out,
                   void* stream) {
    if (!x || !weight || !out) return fail(KT_ERR_ARGUMENT, "x, weight or out is NULL");
    if (rows < 0 || dim <= 0) return fail(KT_ERR_SHAPE, "RMSNorm needs rows >= 0 and dimension > 0, got %d x %d", rows, dim);
    if (rows == 0) return KT_OK;
    const int32_t al = aligned(x, 16) && aligned(weight, 16) && aligned(out, 16);
    rmsnorm_kernel<<<rows, THREADS, 0, static_cast<hipStream_t>(stream)>>>(x, dim, weight, eps, out, al);
    KT_LAUNCHED("rmsnorm kernel");
    return KT_OK;
}

int32_t kt_rope_kv(float* q, float* k, const float* v, int32_t tokens, int32_t num_heads, int32_t num_kv_heads,
                   int32_t head_dim, const float* inv_freq, const int32_t* position, float* cache_k, float* cache_v,
                   int32_t layer, int32_t max_seq, void* stream) {
    if (!q || !k || !v || !inv_freq || !position || !cache_k || !cache_v)
        return fail(KT_ERR_ARGUMENT, "a pointer argument is NULL");
    if (head_dim <= 0 || head_dim % 2 != 0) return fail(KT_ERR_ARGUMENT, "RoPE dimension must be even");
    if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
        return fail(KT_ERR_ARGUMENT, "numHeads %d must be a multiple of numKeyValueHeads %d", num_heads, num_kv_heads);
    if (tokens < 0 || layer < 0 || max_seq <= 0) return fail(KT_ERR_ARGUMENT, "bad tokens, layer or maxSequenceLength");
    if (tokens == 0) return KT_OK;
    const int32_t units = (num_heads + num_kv_heads) * (head_dim / 2);
    const dim3 grid(static_cast<uint32_t>(ceil_div(units, THREADS)), static_cast<uint32_t>(tokens));
    rope_kv_kernel<<<grid, THREADS, 0, static_cast<hipStream_t>(stream)>>>(q, k, v, num_heads, num_kv_heads, head_dim,
                                                                         inv_freq, position, cache_k, cache_v, layer,
                                                                         max_seq);
    KT_LAUNCHED("rope/kv kernel");
    return KT_OK;
}

static int32_t attention_launch(const float* q, int32_t tokens, const int32_t* position, int32_t key_bound,
                                const float* cache_k, const float* cache_v, int32_t layer, int32_t max_seq,
                                int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float* context,
                                const float* k_new, const float* v_new, const float* inv_freq, void* stream) {
    if (!q || !position || !cache_k || !cache_v || !context) return fail(KT_ERR_ARGUMENT, "a pointer argument is NULL");
    if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
        return fail(KT_ERR_ARGUMENT, "numHeads %d must be a multiple of numKeyValueHeads %d", num_heads, num_kv_heads);
    const int32_t G = num_heads / num_kv_heads;
    if (head_dim < 8 || head_dim % 4 != 0 || head_dim > MAX_HD)
        return fail(KT_ERR_ARGUMENT, "head dimension %d: a multiple of 4 from 8 to %d", head_dim, MAX_HD);
    if (G * head_dim > MAX_NACC * THREADS || ceil_div(G, THREADS / 64) * ceil_div(head_dim, 64) > ACC_REGS)
        return fail(KT_ERR_ARGUMENT, "%d query heads per key/value head of %d dims: more than %d floats, or more than %d "
                    "heads per wave", G, head_dim, MAX_NACC * THREADS, (THREADS / 64) * ACC_REGS / ceil_div(head_dim, 64));
    if (tokens < 0 || key_bound < tokens || key_bound > max_seq || layer < 0)
        return fail(KT_ERR_ARGUMENT, "key bound %d must cover the %d tokens and fit maxSequenceLength %d", key_bound,
                    tokens, max_seq);
    if (!aligned(q, 16) || !aligned(cache_k, 16) || !aligned(cache_v, 16))
        return fail(KT_ERR_ARGUMENT, "attention: q and the caches must be 16-byte aligned");
    if (tokens == 0) return KT_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (!k_new && tokens >= PREFILL_MIN_TOKENS && (head_dim == 64 || head_dim == 128) && G <= PQ_ROWS) {
        // many tokens: the query-blocked MFMA kernel
        AttnArgs a{};
        a.q = q;
        a.position = position;
        a.ck = cache_k;
        a.cv = cache_v;
        a.context = context;
        a.layer = layer;
        a.max_seq = max_seq;
        a.num_heads = num_heads;
        a.num_kv_heads = num_kv_heads;
        a.head_dim = head_dim;
        a.scale = 1.0f / sqrtf(static_cast<float>(head_dim));
        a.splits = 1;
        const int32_t qb_tokens = PQ_ROWS / G;
        const int32_t nqb = ceil_div(tokens, qb_tokens);
        const dim3 grid(static_cast<uint32_t>(num_kv_heads), static_cast<uint32_t>(nqb));
        const size_t lds = attention_prefill_lds(head_dim);
        if (head_dim == 64) {
            attention_prefill_kernel<64><<<grid, THREADS, lds, st>>>(a, tokens, qb_tokens, nqb);
        } else {
            static bool raised = false;
            if (!raised) {  // beyond the default dynamic LDS limit (160 KB per CU on gfx950)
                KT_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_prefill_kernel<128>),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, 160 << 10));
                raised = true;
            }
            attention_prefill_kernel<128><<<grid, THREADS, lds, st>>>(a, tokens, qb_tokens, nqb);
        }
        KT_LAUNCHED("prefill attention kernel");
        return KT_OK;
    }
    // Key splits: enough workgroups to fill the GPU when few tokens attend.
    int32_t splits = 1;
    const int32_t tiles = ceil_div(key_bound, KT);
    const int64_t wgs = static_cast<int64_t>(tokens) * num_kv_heads;
    if (wgs < 2 * cu_count()) {
        splits = static_cast<int32_t>((2 * cu_count() + wgs - 1) / wgs);
        if (splits > tiles) splits = tiles;
        if (splits > MAX_SPLITS) splits = MAX_SPLITS;
    }
    AttnArgs a{};
    a.q = q;
    a.position = position;
    a.ck = cache_k;
    a.cv = cache_v;
    a.context = context;
    a.layer = layer;
    a.max_seq = max_seq;
    a.num_heads = num_heads;
    a.num_kv_heads = num_kv_heads;
    a.head_dim = head_dim;
    a.scale = 1.0f / sqrtf(static_cast<float>(head_dim));
    a.k_new = k_new;
    a.v_new = v_new;
    a.inv_freq = inv_freq;
    a.rope = k_new != nullptr ? 1 : 0;
    a.span = ceil_div(tiles, splits) * KT;
    a.splits = ceil_div(key_bound, a.span);
    if (a.splits > 1) {
        // the tagged (max, sum) words live in the workspace's zeroed region (zero on entry,
        // zero again when the launch ends), the values in its general area
        uint32_t* counters = nullptr;
        double* zeroed = nullptr;
        void* general = nullptr;
        const size_t rows = static_cast<size_t>(tokens) * num_heads * a.splits;
        const int32_t status = workspace_regions(st, 2 * rows, rows * head_dim * sizeof(float), &counters, &zeroed,
                                                 &general);
        if (status) return status;
        a.stats = reinterpret_cast<uint64_t*>(zeroed);
        a.partials = static_cast<float*>(general);
        // the RoPE cache sits in the same workspace (with one split the launch needs none
        // and computes cos and sin itself)
        if (a.rope) a.rope_cache = counters + ROPE_CACHE_WORD;
        if (const int32_t fs = stream_fault_word(st, &a.fault)) return fs;
        const WaitLimits limits = wait_limits();
        a.spin_limit = limits.spin_limit ? limits.spin_limit : MERGE_SPIN_LIMIT;
        a.withhold = limits.withhold;
    }
    const dim3 grid(static_cast<uint32_t>(num_kv_heads), static_cast<uint32_t>(a.splits), static_cast<uint32_t>(tokens));
    const size_t lds = attention_lds(G, head_dim);
    if (lds > (64u << 10)) {  // beyond the default dynamic LDS limit (160 KB per CU on gfx950)
        static bool raised = false;
        if (!raised) {
            KT_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_kernel<8>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 << 10));
            KT_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&attention_kernel<16>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, 160 << 10));
            raised = true;
        }
    }
    if (head_dim <= 64) attention_kernel<4><<<grid, THREADS, lds, st>>>(a);
    else if (head_dim <= 128) attention_kernel<8><<<grid, THREADS, lds, st>>>(a);
    else attention_kernel<16><<<grid, THREADS, lds, st>>>(a);
    KT_LAUNCHED("attention kernel");
    return KT_OK;
}

int32_t kt_attention(const float* q, int32_t tokens, const int32_t* position, int32_t key_bound, const float* cache_k,
                     const float* cache_v, int32_t layer, int32_t max_seq, int32_t num_heads, int32_t num_kv_heads,
                     int32_t head_dim, float* context, void* stream) {
    return attention_launch(q, tokens, position, key_bound, cache_k, cache_v, layer, max_seq, num_heads, num_kv_heads,
                            head_dim, context, nullptr, nullptr, nullptr, stream);
}

int32_t kt_rope_attention(float* q, float* k, const float* v, const float* inv_freq, int32_t tokens,
                          const int32_t* position, int32_t key_bound, float* cache_k, float* cache_v, int32_t layer,
                          int32_t max_seq, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float* context,
                          void* stream) {
    if (!q || !k || !v || !inv_freq || !position || !cache_k || !cache_v || !context)
        return fail(KT_ERR_ARGUMENT, "a pointer argument is NULL");
    if (head_dim <= 0 || head_dim % 2 != 0) return fail(KT_ERR_ARGUMENT, "RoPE dimension must be even");
    if (tokens == 1)  // the decode step: RoPE and the cache append inside the attention kernel
        return attention_launch(q, 1, position, key_bound, cache_k, cache_v, layer, max_seq, num_heads, num_kv_heads,
                                head_dim, context, k, v, inv_freq, stream);
    const int32_t status = kt_rope_kv(q, k, v, tokens, num_heads, num_kv_heads, head_dim, inv_freq, position, cache_k,
                                      cache_v, layer, max_seq, stream);
    if (status) return status;
    return kt_attention(q, tokens, position, key_bound, cache_k, cache_v, layer, max_seq, num_heads, num_kv_heads,
                        head_dim, context, stream);
}

int32_t kt_silu_mul(float* gate, const float* up, int64_t n, void* stream) {
    if (!gate || !up) return fail(KT_ERR_ARGUMENT, "gate or up is NULL");
    if (n < 0) return fail(KT_ERR_SHAPE, "negative element count %lld", static_cast<long long>(n));
    if (n == 0) return KT_OK;
    const int64_t blocks = (n + THREADS - 1) / THREADS;
    if (blocks > 0x7FFFFFFF) return fail(KT_ERR_SHAPE, "too many elements");
    silu_mul_kernel<<<static_cast<uint32_t>(blocks), THREADS, 0, static_cast<hipStream_t>(stream)>>>(gate, up, n);
    KT_LAUNCHED("silu*mul kernel");
    return KT_OK;
}

int32_t kt_rmsnorm_qmatmul_group(const float* x, const float* norm_weight, float eps, float* normed, int32_t m,
                                 const kt_qweight* weights, int32_t count, float* const* outputs,
                                 const float* const* biases, int32_t accumulate, float alpha, void* stream) {
    if (!x || !norm_weight || !normed || !weights || !outputs)
        return fail(KT_ERR_ARGUMENT, "x, the norm weight, normed, weights or outputs is NULL");
    if (m < 0) return fail(KT_ERR_ARGUMENT, "Negative row count %d", m);
    if (count <= 0) return fail(KT_ERR_ARGUMENT, "rmsnorm group needs at least one weight, got %d", count);
    WeightView views[4];
    int32_t status = view_weight(&weights[0], &views[0]);
    if (status) return status;
    const int32_t K = views[0].K;
    if (m == 0) return KT_OK;
    // one row, at most four weights the column-run or wide GEMV takes: RMSNorm inside
    // the product
    bool fused = m == 1 && count <= 4 && aligned(x, 16) && aligned(norm_weight, 4) && K % 4 == 0 &&
                 K <= NORM_F4 * 4 * NORM_THREADS;
    bool packed = fused && (gemv_kind() == 0 || gemv_kind() == 5) && aligned(norm_weight, 16);
    fused = fused && (gemv_kind() == 0 || gemv_kind() == 3);
    for (int32_t i = 0; (fused || packed) && i < count; ++i) {
        if (i > 0) {
            status = view_weight(&weights[i], &views[i]);
            if (status) return status;
        }
        const WeightView& v = views[i];
        const bool same = outputs[i] && v.K == K && v.bits == views[0].bits && v.g == views[0].g &&
                          (v.z != nullptr) == (views[0].z != nullptr);
        packed = packed && same && gemv_packed_supported(x, 1, v, outputs[i]);
        fused = fused && same && gemv_wide_supported(x, 1, v, outputs[i]);
    }
    if (packed)
        return launch_gemv_packed(x, views, outputs, biases, count, accumulate, alpha, static_cast<hipStream_t>(stream),
                                  nullptr, norm_weight, eps);
    fused = fused && gemv_wide_preferred(views, count);
    if (fused)
        return launch_gemv_wide(x, views, outputs, biases, count, accumulate, alpha, static_cast<hipStream_t>(stream),
                                nullptr, norm_weight, eps);
    status = kt_rmsnorm(x, m, K, norm_weight, eps, normed, stream);
    if (status) return status;
    return kt_qmatmul_group(normed, m, weights, count, outputs, biases, accumulate, alpha, stream);
}

int32_t kt_rmsnorm_swiglu_gate(const float* x, const float* norm_weight, float eps, float* normed, int32_t m,
                               const kt_qweight* w_gate, const kt_qweight* w_up, const float* bias_gate,
                               const float* bias_up, float* gate, float* up, void* stream) {
    if (!x || !w_gate || !w_up || !gate || !up) return fail(KT_ERR_ARGUMENT, "x, a weight, gate or up is NULL");
    if (norm_weight && !normed) return fail(KT_ERR_ARGUMENT, "normed is NULL");
    if (m < 0) return fail(KT_ERR_ARGUMENT, "Negative row count %d", m);
    WeightView views[2];
    int32_t status = view_weight(w_gate, &views[0]);
    if (status) return status;
    if ((status = view_weight(w_up, &views[1]))) return status;
    if (views[0].K != views[1].K || views[0].N != views[1].N)
        return fail(KT_ERR_SHAPE, "gate and up weights must have the same shape");
    if (m == 0) return KT_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    float* outs[2] = {gate, up};
    const float* biases[2] = {bias_gate, bias_up};
    // one row on column-run copies: one launch, the gate computed in the product's epilogue
    if (m == 1 && (gemv_kind() == 0 || gemv_kind() == 5) && (!norm_weight || aligned(norm_weight, 16)) &&
        (!norm_weight || views[0].K <= NORM_F4 * 4 * NORM_THREADS) && gemv_packed_pair_supported(x, views, outs))
        return launch_gemv_packed(x, views, outs, biases, 2, 0, 1.0f, st, nullptr, norm_weight, eps, true);
    kt_qweight ws[2] = {*w_gate, *w_up};
    status = norm_weight ? kt_rmsnorm_qmatmul_group(x, norm_weight, eps, normed, m, ws, 2, outs, biases, 0, 1.0f, stream)
                         : kt_qmatmul_group(x, m, ws, 2, outs, biases, 0, 1.0f, stream);
    if (status) return status;
    return kt_silu_mul(gate, up, static_cast<int64_t>(m) * views[0].N, stream);
}

// One step of kt_qmatmul_chain as the call it stands for.
static int32_t chain_step_call(const kt_qmatmul_step& p, void* stream) {
    if (p.swiglu_gate)
        return kt_rmsnorm_swiglu_gate(p.x, p.norm_weight, p.eps, p.normed, 1, &p.weights[0], &p.weights[1],
                                      p.biases ? p.biases[0] : nullptr, p.biases ? p.biases[1] : nullptr,
                                      p.outputs[0], p.outputs[1], stream);
    if (p.norm_weight)
        return kt_rmsnorm_qmatmul_group(p.x, p.norm_weight, p.eps, p.normed, 1, p.weights, p.count, p.outputs,
                                        p.biases, p.accumulate, p.alpha, stream);
    return kt_qmatmul_group(p.x, 1, p.weights, p.count, p.outputs, p.biases, p.accumulate, p.alpha, stream);
}

int32_t kt_qmatmul_chain(const kt_qmatmul_step* steps, int32_t count, void* stream) {
    if (!steps) return fail(KT_ERR_ARGUMENT, "steps is NULL");
    if (count < 1 || count > gemv_chain_max_steps())
        return fail(KT_ERR_ARGUMENT, "a chain holds 1 to %d steps, got %d", gemv_chain_max_steps(), count);
    WeightView views[8][4];
    ChainStep cs[8];
    bool chain = gemv_kind() == 0 || gemv_kind() == 5;
    for (int32_t i = 0; i < count; ++i) {
        const kt_qmatmul_step& p = steps[i];
        if (!p.x || !p.weights || !p.outputs) return fail(KT_ERR_ARGUMENT, "step %d: x, weights or outputs is NULL", i);
        if (p.count < 1 || p.count > 4 || (p.swiglu_gate && p.count != 2))
            return fail(KT_ERR_ARGUMENT, "step %d: %d weights (1 to 4; the SwiGLU gate pair takes 2)", i, p.count);
        if (p.norm_weight && !p.normed) return fail(KT_ERR_ARGUMENT, "step %d: normed is NULL", i);
        for (int32_t j = 0; j < p.count; ++j) {
            if (!p.outputs[j]) return fail(KT_ERR_ARGUMENT, "step %d: output %d is NULL", i, j);
            const int32_t status = view_weight(&p.weights[j], &views[i][j]);
            if (status) return status;
            const WeightView& v = views[i][j];
            if (v.K != views[i][0].K) return fail(KT_ERR_SHAPE, "step %d: the weights must share K", i);
            chain = chain && v.bits == views[i][0].bits && v.g == views[i][0].g &&
                    (v.z != nullptr) == (views[i][0].z != nullptr) && gemv_packed_supported(p.x, 1, v, p.outputs[j]);
        }
        if (p.swiglu_gate) {
            if (views[i][0].N != views[i][1].N) return fail(KT_ERR_SHAPE, "step %d: gate and up differ in shape", i);
            chain = chain && !p.accumulate && p.alpha == 1.0f && gemv_packed_pair_supported(p.x, views[i], p.outputs);
        }
        if (p.norm_weight)
            chain = chain && aligned(p.norm_weight, 16) && views[i][0].K <= NORM_F4 * 4 * NORM_THREADS;
        chain = chain && views[i][0].K <= gemv_chain_max_k();
        chain = chain && views[i][0].bits == views[0][0].bits &&
                (views[i][0].z != nullptr) == (views[0][0].z != nullptr);
        cs[i] = ChainStep{p.x, views[i], p.outputs, p.biases, p.count, p.accumulate, p.alpha, nullptr,
                          p.norm_weight, p.eps, p.swiglu_gate != 0};
    }
    if (chain) return launch_gemv_chain(cs, count, static_cast<hipStream_t>(stream));
    for (int32_t i = 0; i < count; ++i) {
        const int32_t status = chain_step_call(steps[i], stream);
        if (status) return status;
    }
    return KT_OK;
}

int32_t kt_swiglu_qmatmul(float* gate, const float* up, int32_t m, const kt_qweight* w, float* c, int32_t accumulate,
                          float alpha, const float* bias, void* stream) {
    if (!gate || !up || !c) return fail(KT_ERR_ARGUMENT, "gate, up or the output is NULL");
    WeightView v;
    int32_t status = view_weight(w, &v);
    if (status) return status;
    if (m < 0) return fail(KT_ERR_ARGUMENT, "Negative row count %d", m);
    if (m == 0) return KT_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const float* biases[1] = {bias};
    // one row: the column-run or wide GEMV computes the gate while it loads its input
    // (and leaves the gate row as it was)
    if (m == 1 && (gemv_kind() == 0 || gemv_kind() == 5) && aligned(up, 16) && gemv_packed_supported(gate, 1, v, c))
        return launch_gemv_packed(gate, &v, &c, biases, 1, accumulate, alpha, st, up);
    if (m == 1 && (gemv_kind() == 0 || gemv_kind() == 3) && gemv_wide_preferred(&v, 1) &&
        gemv_wide_supported(gate, 1, v, c))
        return launch_gemv_wide(gate, &v, &c, biases, 1, accumulate, alpha, st, up);
    // otherwise the gate in place, then the product
    status = kt_silu_mul(gate, up, static_cast<int64_t>(m) * v.K, stream);
    if (status) return status;
    return qmatmul(gate, m, w, c, accumulate, alpha, bias, stream);
}

static int32_t launch_argmax(const float* logits, int32_t n, int32_t* index, int32_t* position, int32_t advance,
                             int32_t* generated, int32_t capacity, hipStream_t st) {
    int32_t blocks = ceil_div(n, 4 * THREADS);
    if (blocks > ARGMAX_BLOCKS) blocks = ARGMAX_BLOCKS;
    void* ws = nullptr;
    uint32_t* counters = nullptr;
    const int32_t status = workspace_counters(st, ARGMAX_BLOCKS * sizeof(uint64_t), 1, &ws, &counters);
    if (status) return status;
    argmax_kernel<<<blocks, THREADS, 0, st>>>(logits, n, index, static_cast<uint64_t*>(ws), counters, position, advance,
                                             generated, capacity);
    KT_LAUNCHED("argmax kernel");
    return KT_OK;
}

int32_t kt_argmax(const float* logits, int32_t n, int32_t* index, void* stream) {
    if (!logits || !index) return fail(KT_ERR_ARGUMENT, "logits or index is NULL");
    if (n <= 0) return fail(KT_ERR_SHAPE, "argmax needs at least one logit");
    return launch_argmax(logits, n, index, nullptr, 0, nullptr, 0, static_cast<hipStream_t>(stream));
}

int32_t kt_argmax_advance(const float* logits, int32_t n, int32_t* token, int32_t* position, int32_t* generated,
                          int32_t capacity, void* stream) {
    if (!logits || !token || !position) return fail(KT_ERR_ARGUMENT, "logits, token or position is NULL");
    if (n <= 0) return fail(KT_ERR_SHAPE, "argmax needs at least one logit");
    return launch_argmax(logits, n, token, position, 1, generated, capacity, static_cast<hipStream_t>(stream));
}

int32_t kt_add_inplace(float* x, const float* y, int64_t n, void* stream) {
    if (!x || !y) return fail(KT_ERR_ARGUMENT, "x or y is NULL");
    if (n < 0) return fail(KT_ERR_SHAPE, "negative element count %lld", static_cast<long long>(n));
    if (n == 0) return KT_OK;
    const int64_t blocks = (n + THREADS - 1) / THREADS;
    if (blocks > 0x7FFFFFFF) return fail(KT_ERR_SHAPE, "too many elements");
    add_kernel<<<static_cast<uint32_t>(blocks), THREADS, 0, static_cast<hipStream_t>(stream)>>>(x, y, n);
    KT_LAUNCHED("add kernel");
    return KT_OK;
}

int32_t kt_fill_normal(float* out, int64_t n, uint64_t seed, float mean, float stddev, void* stream) {
    if (!out) return fail(KT_ERR_ARGUMENT, "out is NULL");
    if (n < 0) return fail(KT_ERR_SHAPE, "negative element count %lld", static_cast<long long>(n));
    if (n == 0) return KT_OK;
    const int64_t blocks = (n + THREADS - 1) / THREADS;
    if (blocks > 0x7FFFFFFF) return fail(KT_ERR_SHAPE, "too many elements");
    fill_normal_kernel<<<static_cast<uint32_t>(blocks), THREADS, 0, static_cast<hipStream_t>(stream)>>>(out, n, seed,
                                                                                                    mean, stddev);
    KT_LAUNCHED("fill kernel");
    return KT_OK;
}

int32_t kt_record_token(const int32_t* token, const int32_t* position, int32_t* generated, int32_t capacity,
                        void* stream) {
    if (!token || !position || !generated) return fail(KT_ERR_ARGUMENT, "token, position or generated is NULL");
    if (capacity < 0) return fail(KT_ERR_ARGUMENT, "negative capacity");
    record_token_kernel<<<1, 64, 0, static_cast<hipStream_t>(stream)>>>(token, position, generated, capacity);
    KT_LAUNCHED("record kernel");
    return KT_OK;
}

int32_t kt_position_add(int32_t* position, int32_t count, void* stream) {
    if (!position) return fail(KT_ERR_ARGUMENT, "position is NULL");
    position_add_kernel<<<1, 64, 0, static_cast<hipStream_t>(stream)>>>(position, count);
    KT_LAUNCHED("position kernel");
    return KT_OK;
}

}  // extern "C"
