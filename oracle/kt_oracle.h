/*
 * kt_oracle.h -- CPU restatement of Kotensor's group-wise INT8/INT4 weight-only
 * quantization path (quantize + split-half pack, dequant accessors, the
 * dequantizing matmul and its transposed product).
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the HIP path is compared
 * against and the CPU baseline the benchmark reports beside the GPU figure. No
 * product code links it; the product (libkotensor_hip.so) never falls back to it.
 *
 * All reference citations are relative to the Kotensor source tree, with
 * Engine/kotensor/src/main/kotlin/ shortened to K/.
 *
 * Pinning status (how each function is checked, see tests/test_oracle_*.py):
 *   ko_java_round, ko_quantize ........ pinned: hand-derived known answers (ties,
 *       0.49999997f, split-half layout, pad nibble, zero clamps, maxAbs = 0,
 *       reciprocal-vs-divide, NaN/inf), the structural known answers of
 *       QuantizationTest.kt:37-74, and an independent numpy restatement.
 *   ko_raw_value/ko_value/ko_dequantize_row/ko_dequantize_column ... pinned:
 *       hand-derived known answers and the error bounds of QuantizationTest.kt:49-59.
 *   ko_multiply_quantized ............. pinned to fp64 brute force on the
 *       dequantized weights (QuantizationTest.kt:76-108 and DecodeKernelTest.kt:47-90
 *       shapes and tolerances) and to the reference's bit-for-bit invariants
 *       (thread-count independence). Its exact fp32 summation order follows
 *       K/MatMul.kt:494-536,599-682,830-881 by reading; that order is
 *       "parity unpinned" at the bit level (no JVM exists to produce the bits),
 *       which is below the 2e-3 normwise criterion the GPU path is held to.
 *   ko_multiply_by_quantized_transposed  pinned to fp64 brute force
 *       (QuantizationTest.kt:98-105 tolerance 1e-3); bit order unpinned as above.
 *
 * Decoder pieces (kt_oracle_decoder.c, tests/test_oracle_decoder.py):
 *   ko_rope_inv_freq ... pinned: closed form 1/base^(2i/d) in fp64, and the scaled
 *       frequencies' three regimes worked by hand (unchanged, divided by the factor,
 *       the smooth blend at its two ends).
 *   ko_rmsnorm ......... pinned: fp64 closed form, zero rows, a constant row (exact
 *       answer 1/sqrt(1+eps) per unit weight), scaling invariance.
 *   ko_rope_rows ....... pinned: position 0 is the identity, each pair keeps its norm,
 *       fp64 closed form, rotating by p1 then p2 equals p1 + p2, every head rotates
 *       alike (RegressionTest.kt:57-76), rows agree with one row at a time.
 *   ko_attend .......... pinned: fp64 brute-force softmax attention (causal, GQA
 *       head mapping), one position gives v, equal scores give the mean of v.
 *   ko_silu_mul, ko_argmax  pinned: fp64 closed form; first index of the maximum,
 *       the -1e9 floor and NaN skipping by hand.
 *   The summation orders follow the reference loops by reading; their bits are
 *   "parity unpinned" (no JVM), far below the tolerances the GPU path is held to.
 */
#ifndef KT_ORACLE_H
#define KT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes shared with the product ABI (include/kotensor_hip.h). */
#define KO_OK 0
#define KO_ERR_ARG (-1)
#define KO_ERR_NAN (-3)

typedef struct ko_qweight {
    const uint8_t* qdata;   /* [rows x bytes_per_row] */
    const float* scales;    /* [groups x columns] */
    const int8_t* zeros;    /* [groups x columns] or NULL (K/QuantizedTensor.kt:43) */
    int32_t rows;           /* K: input features  (K/QuantizedTensor.kt:45) */
    int32_t columns;        /* N: output features (K/QuantizedTensor.kt:46) */
    int32_t bits;           /* 4 or 8 */
    int32_t group_size;
} ko_qweight;

int32_t ko_groups(int32_t rows, int32_t group_size);
int32_t ko_bytes_per_row(int32_t columns, int32_t bits);

/* kotlin.math.roundToInt == java.lang.Math.round: nearest, ties toward +inf,
 * saturating at the int range; NaN sets *nan_seen (Kotlin throws). */
int32_t ko_java_round(float x, int32_t* nan_seen);

/* QuantizedTensor.quantize(data, rows, columns, Quantization(bits, group)),
 * K/QuantizedTensor.kt:261-324. qdata/scales/zeros are fully written; zeros may
 * be NULL only for bits == 8. Returns KO_ERR_NAN where Kotlin would throw. */
int32_t ko_quantize(const float* data, int32_t rows, int32_t columns, int32_t bits,
                    int32_t group_size, uint8_t* qdata, float* scales, int8_t* zeros);

/* Accessors, K/QuantizedTensor.kt:172-241. */
int32_t ko_raw_value(const ko_qweight* w, int32_t row, int32_t column);
float ko_value(const ko_qweight* w, int32_t row, int32_t column);
void ko_dequantize_row(const ko_qweight* w, int32_t row, float* dest);
void ko_dequantize_column(const ko_qweight* w, int32_t column, float* dest);

/* MatMul.multiplyQuantized(a, weight, c, m, accumulate, alpha), K/MatMul.kt:460-486.
 * threads <= 1 runs serially; the result does not depend on it. */
int32_t ko_multiply_quantized(const float* a, const ko_qweight* w, float* c, int32_t m,
                              int32_t accumulate, float alpha, int32_t threads);

/* MatMul.multiplyByQuantizedTransposed(dy, weight, dx, m, accumulate),
 * K/MatMul.kt:954-1003 (scalar dot). */
int32_t ko_multiply_by_quantized_transposed(const float* dy, const ko_qweight* w, float* dx,
                                            int32_t m, int32_t accumulate, int32_t threads);

/* The M == 1 unit decomposition of K/MatMul.kt:494-512, exposed for tests:
 * out[0..5] = {target_units, rows_per_unit, row_units, column_units, block_bytes, blocks}. */
void ko_row_units(const ko_qweight* w, int32_t* out6);

/* ---- decoder pieces (kt_oracle_decoder.c) ---------------------------------------- */
/* RoPE.invFreq (K/RoPE.kt:42-46) with RoPEScaling.scale (:18-30) when factor > 0. */
void ko_rope_inv_freq(int32_t head_dim, float base, float factor, float low, float high, int32_t original_max,
                      float* out);
/* RMSNorm.forwardInto (K/RMSNorm.kt:71-90). */
void ko_rmsnorm(const float* x, int32_t rows, int32_t dim, const float* weight, float eps, float* out);
/* RoPE.applyRowsInPlace (K/RoPE.kt:139-164). */
void ko_rope_rows(float* rows, int32_t tokens, int32_t width, int32_t head_dim, const float* inv_freq, int32_t start);
/* Attention.attendCached/attendHead/dot (K/Attention.kt:277-349); scores: start+tokens floats. */
void ko_attend(const float* q, int32_t tokens, int32_t start, const float* keys, const float* values, int32_t layer,
               int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t max_seq, float* context,
               float* scores);
/* gate = silu(gate) * up (K/SwiGLU.kt:19-25, K/Tensor.kt:223-237). */
void ko_silu_mul(float* gate, const float* up, int32_t n);
/* Transformer.argmaxOfLastToken (K/Transformer.kt:253-266). */
int32_t ko_argmax(const float* logits, int32_t n);

/* ---- the fused loss (kt_oracle_loss.c) -------------------------------------------- */
/* fusedCrossEntropyLoss(hidden, QuantizedLinear(w, bias), targets, ignoreIndex),
 * K/Loss.kt:114-219: *loss = mean over the rows whose target is not ignore_index of
 * max + ln(sum exp(l - max)) - l[target], logits l = hidden . deq(w) + bias (bias may be
 * NULL: zeros). hidden_grad [rows x K] and bias_grad [N] (each may be NULL) receive, added
 * to what they hold, the gradients the backward closure adds for an upstream gradient of
 * 1 (ignored rows get nothing). KO_ERR_ARG for no rows or a target outside [0, N). */
int32_t ko_fused_cross_entropy(const float* hidden, int32_t rows, const ko_qweight* w, const float* bias,
                               const int32_t* targets, int32_t ignore_index, float* loss, float* hidden_grad,
                               float* bias_grad, int32_t threads);

#ifdef __cplusplus
}
#endif
#endif
