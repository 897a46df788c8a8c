// kt_packed.h -- the column-run copy's layout constants and helpers, shared by the
// kernels that read it (kt_gemv_packed.hip: one row; kt_gemv_rows_packed.hip: 2 to 16).
// Layout: blocks of one 16-column set x one 128-k chunk, ordered [set][chunk] (INT4 1 KB,
// INT8 2 KB), lane l = 16 kb + n of a reading wave owning column 16 set + n over the
// 32-k run [128 chunk + 32 kb, + 32); after the blocks, the scale and zero-point rows
// [set][group][16] (fp32, then bytes).
#pragma once

#include <atomic>
#include <type_traits>

#include "kt_common.h"

namespace kt {

constexpr int SET = 16;         // columns per column set
constexpr int CHUNK = 128;      // k per chunk
constexpr int RUN = 32;         // k per lane run
constexpr int NONTEMPORAL = 2;  // buffer-load cache policy: streamed data, read once
constexpr int MAX_WAVE_CHUNKS = 16;  // a wave's K range: at most 2048 (its staged group rows fit 64)
__host__ __device__ constexpr int block_bytes(int bits) { return bits == 4 ? 1024 : 2048; }

// Calls f(std::integral_constant<int, I>) for I = B .. E - 1, so register arrays indexed by
// I stay in registers.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// Sums that do not depend on how K is split: K's chunks are cut into SUB_PARTS sub-parts
// (sub-part j: chunks [j chunks / SUB_PARTS, (j + 1) chunks / SUB_PARTS)), every
// sub-part's sum is formed alone, and the sub-parts add as a balanced binary tree in K
// order. A wave that covers an aligned block of 2^b sub-parts pushes them in order
// (tree_push) and holds that block's subtree at the end; the K-parts' subtrees then meet
// in the tree's top levels (tree_top).
constexpr int SUB_LOG = 3;
constexpr int SUB_PARTS = 1 << SUB_LOG;  // the largest K split

// Pushes sub-part i's sum v (i: index within the wave's block); t holds the pending left
// subtrees of sizes 1, 2 and 4. Returns the subtree that v completes (after the block's
// last push: the block's sum).
__device__ __forceinline__ float tree_push(float (&t)[3], int32_t i, float v) {
    if (i & 1) {
        v = t[0] + v;
        if (i & 2) {
            v = t[1] + v;
            if (i & 4) v = t[2] + v;
            else t[2] = v;
        } else {
            t[1] = v;
        }
    } else {
        t[0] = v;
    }
    return v;
}

// (v_l + v_l^16) + (v_l^32 + v_l^48), the same value in the four lanes: the lane groups'
// sum in a fixed order by two lane swaps (no LDS path).
__device__ __forceinline__ float lanes4_sum(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const float s = __uint_as_float(a[0]) + __uint_as_float(a[1]);  // rows (0, 1) and (2, 3)
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(s), __float_as_uint(s), false, false);
    return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

#define KT_DPP(x, ctrl) __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), ctrl, 0xF, 0xF, false))
// The largest value over each row of 16 lanes, in every lane of the row: DPP quad swaps,
// then the half-row and row mirrors.
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, KT_DPP(v, 0xB1));   // quad_perm [1, 0, 3, 2]
    v = fmaxf(v, KT_DPP(v, 0x4E));   // quad_perm [2, 3, 0, 1]
    v = fmaxf(v, KT_DPP(v, 0x141));  // row_half_mirror: 8 lanes
    return fmaxf(v, KT_DPP(v, 0x140));  // row_mirror: 16 lanes
}
// The largest value over lanes l, l ^ 4, l ^ 8, l ^ 12 of each row of 16 (the lanes that
// agree in bits 0 and 1), in each of them: two row rotations.
__device__ __forceinline__ float row_stride4_max(float v) {
    v = fmaxf(v, KT_DPP(v, 0x124));     // row_ror:4
    return fmaxf(v, KT_DPP(v, 0x128));  // row_ror:8
}
#undef KT_DPP
// The largest value over the four rows of 16 (lanes l, l ^ 16, l ^ 32, l ^ 48), in each of
// them: the two lane swaps.
__device__ __forceinline__ float rows4_max(float v) {
    const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    v = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
    const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// The largest value over the wave's 64 lanes, in every lane, without the LDS path.
__device__ __forceinline__ float wave_max64(float v) { return rows4_max(row16_max(v)); }

// The top levels: the 2^kslog K-parts' subtrees p[0], p[stride], ... added pairwise.
__device__ __forceinline__ float tree_top(const float* p, int32_t stride, int32_t kslog) {
    float v[SUB_PARTS];
#pragma unroll
    for (int q = 0; q < SUB_PARTS; ++q) v[q] = q < (1 << kslog) ? p[q * stride] : 0.0f;
#pragma unroll
    for (int l = 0; l < SUB_LOG; ++l)
        if (l < kslog)
#pragma unroll
            for (int q = 0; q < SUB_PARTS; q += 2 << l) v[q] = v[q] + v[q + (1 << l)];
    return v[0];
}

// Groups a wave's range of at most nmax chunks touches (g = 32 << gshift): whole groups
// per chunk up to g = 128; beyond that a range may start inside a group, one row more.
__host__ __device__ constexpr int32_t stage_rows(int32_t nmax, int32_t gshift) {
    return gshift <= 2 ? nmax << (2 - gshift) : (((nmax << 2) + (1 << gshift) - 1) >> gshift) + 1;
}
constexpr int32_t STAGE_ROW_BYTES = SET * 4 + SET;  // scales and zero points of one group row

// gfx950 gives a workgroup up to 160 KB of LDS; a kernel asks for more than 64 KB of
// dynamic LDS by raising its attribute first (allow_lds).
constexpr size_t LDS_DEFAULT = 64 << 10, LDS_MAX = 160 << 10;
// Raises the dynamic-LDS attribute of kernel KERN to LDS_MAX once, when a launch needs
// more than the default.
template <auto KERN>
int32_t allow_lds(size_t lds) {
    static std::atomic<bool> raised{false};
    if (lds <= LDS_DEFAULT || raised.load(std::memory_order_acquire)) return KT_OK;
    KT_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(KERN), hipFuncAttributeMaxDynamicSharedMemorySize,
                               static_cast<int>(LDS_MAX)));
    raised.store(true, std::memory_order_release);
    return KT_OK;
}

inline int32_t log2_exact(int32_t v) {
    int32_t s = 0;
    while ((1 << s) < v) ++s;
    return (1 << s) == v ? s : -1;
}

// The work split of a launch over weights with K rows, groups of g and sets_total column
// sets: ks K-parts per column set (a workgroup of eight waves holds 8 / ks sets), nmax
// chunks at most per wave, and the one-row kernel's LDS (kt_gemv_packed.hip).
struct PackedPlan {
    int32_t ks = 0, nmax = 0;
    size_t lds = 0;
};
PackedPlan plan_packed(int32_t K, int32_t g, int64_t sets_total);

}  // namespace kt
