// kt_gemm.hip -- prefill dequant-GEMM (M >= 2) on gfx950 MFMA:
//   c[M x N] = (accumulate ? c : 0) + alpha * a[M x K] . deq(W) (+ bias),
// the M > 1 branch of MatMul.multiplyQuantized (Engine/kotensor/src/main/kotlin/
// MatMul.kt:479-485 -> computeQuantizedTile :830-881).
//
// Numerics. The operands go to v_mfma_f32_32x32x16_f16 as fp16 with fp32
// accumulation. Two exact power-of-two rescalings keep fp16 in its normal range
// whatever the data: row m of a is multiplied by 2^-er[m] so its largest magnitude
// lies in [2^14, 2^15), and column n of the weight by 2^-ec[n] so its largest
// group scale lies in [1/2, 1). A weight element enters the MFMA as
// fp16((q - zero) * scale * 2^-ec[n]) (q and zero exact integers), and the fp32
// result is multiplied back by 2^(er[m] + ec[n]). The rounding of a and of the
// dequantized weight to fp16 (relative 2^-11 each) keeps the normwise error far
// below the 2e-3 the path is held to.
//
// Work layout. A pre-pass kernel writes the fp16 copy of a (zero-padded to whole
// tiles, so tile loads need no bounds checks) and the two exponent vectors. The
// GEMM kernel computes a 128 x 128 output tile per 256-thread workgroup (four waves
// in a 2 x 2 arrangement, 64 x 64 each as 2 x 2 MFMA 32x32 blocks) over K in steps
// of 32: a's tile is copied to LDS; the weight tile's packed bytes are loaded
// (INT8: 128 bytes x 32 rows; INT4: 64 bytes x 32 rows = 64 low-nibble plus 64
// high-nibble columns, so every packed byte is read once per row tile),
// dequantized in registers and stored to LDS transposed (k contiguous) in the
// order the MFMA B operand reads it.
#include "kt_common.h"

namespace kt {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));

constexpr int BM = 128;
constexpr int BN = 128;
constexpr int BK = 32;
constexpr int PITCH = BK + 8;  // halfs per LDS row (16-byte pad)

// Largest-magnitude based exponent: returns e with max * 2^-e in [2^(top-1), 2^top).
__device__ __forceinline__ int32_t scale_exponent(float max_abs, int32_t top) {
    if (!(max_abs > 0.0f) || !isfinite(max_abs)) return 0;
    int e = 0;
    frexpf(max_abs, &e);  // max_abs = f * 2^e, f in [0.5, 1)
    return e - top;
}

// Blocks [0, Mp): fp16 rows of a. Blocks [Mp, Mp + ceil(N/256)): column exponents.
__global__ void __launch_bounds__(256)
    gemm_prep(const float* __restrict__ a, int32_t M, int32_t K, int32_t Mp, int32_t Kp, const float* __restrict__ s,
              int32_t G, int32_t N, _Float16* __restrict__ a16, int32_t* __restrict__ er, int32_t* __restrict__ ec) {
    __shared__ float red[256];
    const int32_t t = threadIdx.x;
    if (static_cast<int32_t>(blockIdx.x) < Mp) {
        const int32_t m = blockIdx.x;
        _Float16* dst = a16 + static_cast<size_t>(m) * Kp;
        if (m >= M) {
            for (int32_t k = t; k < Kp; k += 256) dst[k] = static_cast<_Float16>(0.0f);
            if (t == 0) er[m] = 0;
            return;
        }
        const float* row = a + static_cast<size_t>(m) * K;
        float mx = 0.0f;
        for (int32_t k = t; k < K; k += 256) mx = fmaxf(mx, fabsf(row[k]));
        red[t] = mx;
        __syncthreads();
        for (int32_t w = 128; w > 0; w >>= 1) {
            if (t < w) red[t] = fmaxf(red[t], red[t + w]);
            __syncthreads();
        }
        const int32_t e = scale_exponent(red[0], 15);
        const float mul = ldexpf(1.0f, -e);
        for (int32_t k = t; k < Kp; k += 256) dst[k] = static_cast<_Float16>(k < K ? row[k] * mul : 0.0f);
        if (t == 0) er[m] = e;
        return;
    }
    const int32_t n = (blockIdx.x - Mp) * 256 + t;
    if (n >= N) return;
    float mx = 0.0f;
    for (int32_t gi = 0; gi < G; ++gi) mx = fmaxf(mx, fabsf(s[static_cast<size_t>(gi) * N + n]));
    ec[n] = scale_exponent(mx, 0);
}

template <int BITS>
__global__ void __launch_bounds__(256)
    gemm_kernel(const _Float16* __restrict__ a16, int32_t Kp, const int32_t* __restrict__ er,
                const int32_t* __restrict__ ec, const uint8_t* __restrict__ q, const float* __restrict__ s,
                const int8_t* __restrict__ z, int32_t M, int32_t K, int32_t N, int32_t bpr, int32_t g,
                int32_t tiles_n, float* __restrict__ c, const float* __restrict__ bias, float alpha,
                int32_t accumulate) {
    __shared__ __attribute__((aligned(16))) _Float16 As[BM * PITCH];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[BN * PITCH];

    const int32_t t = threadIdx.x;
    const int32_t ln = t & 63;
    const int32_t wave = t >> 6;
    const int32_t wm = wave >> 1, wn = wave & 1;
    const int32_t tile_m = blockIdx.x / tiles_n;
    const int32_t tile_n = blockIdx.x % tiles_n;
    const int32_t m0 = tile_m * BM;
    const int32_t half = bpr;
    // Byte columns of this tile: INT8 [b0, b0 + 128); INT4 [b0, b0 + 64) holding
    // low-nibble columns b0.. and high-nibble columns half + b0.. .
    const int32_t b0 = tile_n * (BITS == 8 ? BN : BN / 2);

    // Weight-tile assignment: INT8 thread -> 4 byte columns x 4 rows; INT4 -> 4 bytes x 2 rows.
    constexpr int ROWS_PER_T = BITS == 8 ? 4 : 2;
    constexpr int COLQ = BITS == 8 ? 32 : 16;  // 4-byte column quads per tile row
    const int32_t cq = t % COLQ;
    const int32_t rg = t / COLQ;
    const int32_t bcol = b0 + cq * 4;  // first byte column of this thread
    const bool bvalid = bcol < bpr;

    float16v acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

    for (int32_t k0 = 0; k0 < K; k0 += BK) {
        // a tile: 128 rows x 32 halfs; thread -> row t/2, 16 halfs at (t&1)*16.
        {
            const int32_t r = t >> 1;
            const int32_t kc = (t & 1) * 16;
            const uint4* src = reinterpret_cast<const uint4*>(a16 + static_cast<size_t>(m0 + r) * Kp + k0 + kc);
            uint4 v0 = src[0], v1 = src[1];
            uint4* dst = reinterpret_cast<uint4*>(As + r * PITCH + kc);
            dst[0] = v0;
            dst[1] = v1;
        }
        // weight tile: load, dequantize, store transposed.
        {
            const int32_t kr = k0 + rg * ROWS_PER_T;  // all ROWS_PER_T rows share one group (g % 4 == 0)
            uint32_t w[ROWS_PER_T];
#pragma unroll
            for (int i = 0; i < ROWS_PER_T; ++i)
                w[i] = (bvalid && kr + i < K) ? *reinterpret_cast<const uint32_t*>(q + static_cast<size_t>(kr + i) * bpr + bcol) : 0u;
            const int32_t gi = (kr < K ? kr : K - 1) / g;
            const float* srow = s + static_cast<size_t>(gi) * N;
            const int8_t* zrow = z ? z + static_cast<size_t>(gi) * N : nullptr;
#pragma unroll
            for (int side = 0; side < (BITS == 4 ? 2 : 1); ++side) {
                const int32_t col = side ? half + bcol : bcol;
                float sc[4] = {0.f, 0.f, 0.f, 0.f};
                int32_t zr[4] = {0, 0, 0, 0};
                if (bvalid && kr < K) {
                    const float4 s4 = *reinterpret_cast<const float4*>(srow + col);
                    const int4 e4 = *reinterpret_cast<const int4*>(ec + col);
                    sc[0] = ldexpf(s4.x, -e4.x);
                    sc[1] = ldexpf(s4.y, -e4.y);
                    sc[2] = ldexpf(s4.z, -e4.z);
                    sc[3] = ldexpf(s4.w, -e4.w);
                    if (zrow) {
                        const uint32_t zw = *reinterpret_cast<const uint32_t*>(zrow + col);
#pragma unroll
                        for (int j = 0; j < 4; ++j) zr[j] = static_cast<int8_t>((zw >> (8 * j)) & 0xFFu);
                    }
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    _Float16 hv[ROWS_PER_T];
#pragma unroll
                    for (int i = 0; i < ROWS_PER_T; ++i) {
                        const uint32_t byte = (w[i] >> (8 * j)) & 0xFFu;
                        int32_t qv;
                        if (BITS == 8) qv = static_cast<int8_t>(byte);
                        else qv = side ? static_cast<int32_t>(byte >> 4) : static_cast<int32_t>(byte & 0xFu);
                        hv[i] = static_cast<_Float16>(static_cast<float>(qv - zr[j]) * sc[j]);
                    }
                    const int32_t nl = (BITS == 8 ? 0 : side * (BN / 2)) + cq * 4 + j;
                    _Float16* dst = Bs + nl * PITCH + rg * ROWS_PER_T;
                    if constexpr (ROWS_PER_T == 4) {
                        half4 hv4 = {hv[0], hv[1], hv[2], hv[3]};
                        *reinterpret_cast<half4*>(dst) = hv4;
                    } else {
                        half2v hv2 = {hv[0], hv[1]};
                        *reinterpret_cast<half2v*>(dst) = hv2;
                    }
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            half8 af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int32_t row = wm * 64 + i * 32 + (ln & 31);
                af[i] = *reinterpret_cast<const half8*>(As + row * PITCH + kk + (ln >> 5) * 8);
                const int32_t col = wn * 64 + i * 32 + (ln & 31);
                bf[i] = *reinterpret_cast<const half8*>(Bs + col * PITCH + kk + (ln >> 5) * 8);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
    }

    // Epilogue: D[i][j] of a 32x32 block sits in lane j + 32*((i/4)%2), register (i/8)*4 + i%4.
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
        const int32_t nl = wn * 64 + jb * 32 + (ln & 31);
        int32_t n;
        if (BITS == 8) n = b0 + nl;
        else n = nl < BN / 2 ? b0 + nl : half + b0 + (nl - BN / 2);
        const bool nvalid = BITS == 8 ? n < N : ((nl < BN / 2 ? b0 + nl : b0 + nl - BN / 2) < bpr && n < N);
        if (!nvalid) continue;
        const int32_t en = ec[n];
        const float bn = bias ? bias[n] : 0.0f;
#pragma unroll
        for (int ib = 0; ib < 2; ++ib) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int32_t i = (r >> 2) * 8 + (ln >> 5) * 4 + (r & 3);
                const int32_t m = m0 + wm * 64 + ib * 32 + i;
                if (m >= M) continue;
                float* dst = c + static_cast<size_t>(m) * N + n;
                const float v = ldexpf(acc[ib][jb][r], er[m] + en);
                float o = accumulate ? *dst : 0.0f;
                o = fmaf(alpha, v, o);
                if (bias) o += bn;
                *dst = o;
            }
        }
    }
}

}  // namespace

bool gemm_supported(const float* a, int32_t m, const WeightView& w, const float* c) {
    (void)a;
    (void)m;
    (void)c;
    if (w.g % 4 != 0) return false;  // a thread's 2 or 4 weight rows share one group
    if (w.N % (w.bits == 4 ? 8 : 4) != 0) return false;
    return aligned(w.q, 4) && aligned(w.s, 16) && (!w.z || aligned(w.z, 4));
}

int32_t launch_gemm(const float* a, int32_t m, const WeightView& w, float* c, int32_t accumulate, float alpha,
                    const float* bias, hipStream_t st) {
    const int32_t Mp = ceil_div(m, BM) * BM;
    const int32_t Kp = ceil_div(w.K, BK) * BK;
    const size_t a16_bytes = (static_cast<size_t>(Mp) * Kp * sizeof(_Float16) + 255) & ~size_t(255);
    const size_t er_bytes = (static_cast<size_t>(Mp) * 4 + 255) & ~size_t(255);
    const size_t ec_bytes = (static_cast<size_t>(w.N) * 4 + 255) & ~size_t(255);
    void* ws = nullptr;
    int32_t status = workspace(st, a16_bytes + er_bytes + ec_bytes, &ws);
    if (status) return status;
    _Float16* a16 = static_cast<_Float16*>(ws);
    int32_t* er = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + a16_bytes);
    int32_t* ec = reinterpret_cast<int32_t*>(static_cast<char*>(ws) + a16_bytes + er_bytes);
    gemm_prep<<<Mp + ceil_div(w.N, 256), 256, 0, st>>>(a, m, w.K, Mp, Kp, w.s, w.G, w.N, a16, er, ec);
    KT_LAUNCHED("qmatmul: gemm prep");
    const int32_t tiles_n = ceil_div(w.bpr, w.bits == 8 ? BN : BN / 2);
    const int32_t tiles_m = Mp / BM;
    const dim3 grid(static_cast<uint32_t>(tiles_m * tiles_n));
    if (w.bits == 8)
        gemm_kernel<8><<<grid, 256, 0, st>>>(a16, Kp, er, ec, w.q, w.s, w.z, m, w.K, w.N, w.bpr, w.g, tiles_n, c,
                                             bias, alpha, accumulate);
    else
        gemm_kernel<4><<<grid, 256, 0, st>>>(a16, Kp, er, ec, w.q, w.s, w.z, m, w.K, w.N, w.bpr, w.g, tiles_n, c,
                                             bias, alpha, accumulate);
    KT_LAUNCHED("qmatmul: gemm kernel");
    return KT_OK;
}

}  // namespace kt
