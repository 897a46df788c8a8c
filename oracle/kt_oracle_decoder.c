/*
 * kt_oracle_decoder.c -- CPU restatement of the decoder pieces around the quantized
 * projections: RMSNorm, RoPE (frequencies, rotate-half), cached GQA attention, the
 * SwiGLU gate and the greedy argmax.
 *
 * TEST INFRASTRUCTURE ONLY (the checker of the HIP decoder kernels); no product code
 * links it. Reference citations are relative to Engine/kotensor/src/main/kotlin/ (K/).
 *
 * The JVM evaluates kotlin.math.exp/cos/sin/pow/sqrt on a Float argument in double
 * precision and rounds the result to float; the functions below do the same. Every
 * product and sum is a separate fp32 operation (built with -ffp-contract=off), in the
 * reference's loop order.
 */
#include <math.h>
#include <stdint.h>

#include "kt_oracle.h"

/* java.lang.Math.PI */
static const double JAVA_PI = 3.141592653589793;

/* RoPEScaling.scale (K/RoPE.kt:18-30). */
static float rope_scale(float inv_freq, float factor, float low, float high, int32_t original_max) {
    const float low_wavelength = (float)original_max / low;
    const float high_wavelength = (float)original_max / high;
    const float wavelength = (float)(2.0 * JAVA_PI / (double)inv_freq);
    if (wavelength < high_wavelength) return inv_freq;
    if (wavelength > low_wavelength) return inv_freq / factor;
    const float smooth = ((float)original_max / wavelength - low) / (high - low);
    return (1.0f - smooth) * inv_freq / factor + smooth * inv_freq;
}

/* RoPE.invFreq (K/RoPE.kt:42-46): 1 / base^((2i)/dimension), optionally scaled. */
void ko_rope_inv_freq(int32_t head_dim, float base, float factor, float low, float high, int32_t original_max,
                      float* out) {
    const int32_t half = head_dim / 2;
    for (int32_t i = 0; i < half; ++i) {
        const float exponent = (float)(2 * i) / (float)head_dim;
        const float raw = 1.0f / (float)pow((double)base, (double)exponent);
        out[i] = factor > 0.0f ? rope_scale(raw, factor, low, high, original_max) : raw;
    }
}

/* RMSNorm.forwardInto (K/RMSNorm.kt:71-90). */
void ko_rmsnorm(const float* x, int32_t rows, int32_t dim, const float* weight, float eps, float* out) {
    for (int32_t r = 0; r < rows; ++r) {
        const float* row = x + (int64_t)r * dim;
        float sum_sq = 0.0f;
        for (int32_t d = 0; d < dim; ++d) sum_sq += row[d] * row[d];
        const float r_rms = 1.0f / (float)sqrt((double)(sum_sq / (float)dim + eps));
        for (int32_t d = 0; d < dim; ++d) out[(int64_t)r * dim + d] = row[d] * r_rms * weight[d];
    }
}

/* RoPE.applyRowsInPlace (K/RoPE.kt:139-164): rows [tokens x width], width a multiple
 * of head_dim, token t at position start + t. */
void ko_rope_rows(float* rows, int32_t tokens, int32_t width, int32_t head_dim, const float* inv_freq, int32_t start) {
    const int32_t half = head_dim / 2, heads = width / head_dim;
    for (int32_t t = 0; t < tokens; ++t) {
        const int32_t position = start + t;
        float* row = rows + (int64_t)t * width;
        for (int32_t i = 0; i < half; ++i) {
            const float theta = (float)position * inv_freq[i];
            const float c = (float)cos((double)theta);
            const float s = (float)sin((double)theta);
            for (int32_t h = 0; h < heads; ++h) {
                const int32_t i1 = h * head_dim + i, i2 = i1 + half;
                const float x1 = row[i1], x2 = row[i2];
                row[i1] = x1 * c - x2 * s;
                row[i2] = x1 * s + x2 * c;
            }
        }
    }
}

/* Attention.dot (K/Attention.kt:330-349): four running sums, then the tail. */
static float attention_dot(const float* a, const float* b, int32_t n) {
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    int32_t d = 0;
    for (; d + 4 <= n; d += 4) {
        s0 += a[d] * b[d];
        s1 += a[d + 1] * b[d + 1];
        s2 += a[d + 2] * b[d + 2];
        s3 += a[d + 3] * b[d + 3];
    }
    float sum = (s0 + s1) + (s2 + s3);
    for (; d < n; ++d) sum += a[d] * b[d];
    return sum;
}

/* Attention.attendCached / attendHead (K/Attention.kt:277-328) over the KVCache layout
 * ((layer * kv_heads + head) * max_seq + position) * head_dim (K/KVCache.kt:25-27).
 * q [tokens x num_heads*head_dim]; token t at position start + t attends to 0..position.
 * scores needs start + tokens floats. */
void ko_attend(const float* q, int32_t tokens, int32_t start, const float* keys, const float* values, int32_t layer,
               int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t max_seq, float* context,
               float* scores) {
    const int32_t dimension = num_heads * head_dim, group = num_heads / num_kv_heads;
    const float scale = 1.0f / (float)sqrt((double)(float)head_dim);
    for (int32_t h = 0; h < num_heads; ++h) {
        for (int32_t t = 0; t < tokens; ++t) {
            const int32_t position = start + t;
            const float* qh = q + (int64_t)t * dimension + h * head_dim;
            const int64_t base = ((int64_t)(layer * num_kv_heads + h / group) * max_seq) * head_dim;
            float max_score = -1e9f;
            for (int32_t j = 0; j <= position; ++j) {
                const float score = attention_dot(qh, keys + base + (int64_t)j * head_dim, head_dim) * scale;
                scores[j] = score;
                if (score > max_score) max_score = score;
            }
            float sum_exp = 0.0f;
            for (int32_t j = 0; j <= position; ++j) {
                const float e = (float)exp((double)(scores[j] - max_score));
                scores[j] = e;
                sum_exp += e;
            }
            const float inv_sum = 1.0f / sum_exp;
            float* ctx = context + (int64_t)t * dimension + h * head_dim;
            for (int32_t d = 0; d < head_dim; ++d) ctx[d] = 0.0f;
            for (int32_t j = 0; j <= position; ++j) {
                const float w = scores[j] * inv_sum;
                const float* v = values + base + (int64_t)j * head_dim;
                for (int32_t d = 0; d < head_dim; ++d) ctx[d] += w * v[d];
            }
        }
    }
}

/* SwiGLU.forwardInto's gate (K/SwiGLU.kt:19-25 -> K/Tensor.kt:223-237):
 * gate = silu(gate) then gate *= up, with silu(x) = x / (1 + exp(-x)). */
void ko_silu_mul(float* gate, const float* up, int32_t n) {
    for (int32_t i = 0; i < n; ++i) {
        const float x = gate[i];
        const float silu = x / (1.0f + (float)exp((double)(-x)));
        gate[i] = silu * up[i];
    }
}

/* Transformer.argmaxOfLastToken (K/Transformer.kt:253-266): the first index whose
 * logit exceeds every earlier one, starting from -1e9; 0 when none does. */
int32_t ko_argmax(const float* logits, int32_t n) {
    int32_t best = 0;
    float max_logit = -1e9f;
    for (int32_t v = 0; v < n; ++v) {
        if (logits[v] > max_logit) {
            max_logit = logits[v];
            best = v;
        }
    }
    return best;
}
