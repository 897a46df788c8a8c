/* kt_oracle_loss.c -- the oracle's restatement of fusedCrossEntropyLoss with a quantized
 * head (TEST INFRASTRUCTURE ONLY: the checker of kt_fused_cross_entropy, never part of
 * the product). Follows K/Loss.kt:114-219 (the loop and the backward closure),
 * activeRows (:236-251), projectRows (:253-273) and logitGradients (:275-291), with
 * Kotlin's Float exp/ln (kotlin.math on the JVM: the double function rounded to float).
 * Pinning: tests/test_oracle_loss.py (an fp64 softmax cross-entropy on the dequantized
 * weights, closed forms for uniform logits and single-class rows, ignored rows, empty
 * and out-of-range targets, and a planted mistake). */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "kt_oracle.h"

#define FUSED_CHUNK_ELEMENTS (1 << 22) /* K/Loss.kt:8 */

int32_t ko_fused_cross_entropy(const float* hidden, int32_t rows, const ko_qweight* w, const float* bias,
                               const int32_t* targets, int32_t ignore_index, float* loss, float* hidden_grad,
                               float* bias_grad, int32_t threads) {
    if (!hidden || !w || !targets || !loss || rows <= 0) return KO_ERR_ARG; /* targets cannot be empty */
    const int32_t dimension = w->rows, vocabulary = w->columns;
    /* activeRows (:236-251): every target is ignore_index or in [0, vocabulary) */
    int32_t active = 0;
    for (int32_t i = 0; i < rows; ++i) {
        if (targets[i] == ignore_index) continue;
        if (targets[i] < 0 || targets[i] >= vocabulary) return KO_ERR_ARG;
        ++active;
    }
    if (active == 0) { /* emptyLoss() */
        *loss = 0.0f;
        return KO_OK;
    }
    int32_t* act = malloc(sizeof(int32_t) * (size_t)active);
    for (int32_t i = 0, next = 0; i < rows; ++i)
        if (targets[i] != ignore_index) act[next++] = i;

    int32_t chunk_rows = FUSED_CHUNK_ELEMENTS / vocabulary;
    if (chunk_rows < 1) chunk_rows = 1;
    if (chunk_rows > active) chunk_rows = active;
    float* inputs = malloc(sizeof(float) * (size_t)chunk_rows * dimension);
    float* logits = malloc(sizeof(float) * (size_t)chunk_rows * vocabulary);
    float* row_max = malloc(sizeof(float) * (size_t)active);
    float* row_sum = malloc(sizeof(float) * (size_t)active);
    const float scale = 1.0f / (float)active;
    float* hgrad = hidden_grad ? calloc((size_t)active * dimension, sizeof(float)) : NULL;
    float* chunk_grad = hidden_grad ? malloc(sizeof(float) * (size_t)chunk_rows * dimension) : NULL;
    float* bgrad = bias_grad ? calloc((size_t)vocabulary, sizeof(float)) : NULL;
    float total = 0.0f;
    int32_t status = KO_OK;

    for (int32_t start = 0; start < active && status == KO_OK; start += chunk_rows) {
        const int32_t count = active - start < chunk_rows ? active - start : chunk_rows;
        /* projectRows (:253-273) */
        for (int32_t r = 0; r < count; ++r)
            memcpy(inputs + (size_t)r * dimension, hidden + (size_t)act[start + r] * dimension,
                   sizeof(float) * dimension);
        status = ko_multiply_quantized(inputs, w, logits, count, 0, 1.0f, threads);
        if (status) break;
        for (int32_t r = 0; r < count; ++r)
            for (int32_t v = 0; v < vocabulary; ++v) logits[(size_t)r * vocabulary + v] += bias ? bias[v] : 0.0f;
        /* the loss of each row (:146-164) */
        for (int32_t r = 0; r < count; ++r) {
            const float* l = logits + (size_t)r * vocabulary;
            float max_logit = -1e9f;
            for (int32_t v = 0; v < vocabulary; ++v)
                if (l[v] > max_logit) max_logit = l[v];
            float sum_exp = 0.0f;
            for (int32_t v = 0; v < vocabulary; ++v) sum_exp += (float)exp((double)(l[v] - max_logit));
            row_max[start + r] = max_logit;
            row_sum[start + r] = sum_exp;
            total += max_logit + (float)log((double)sum_exp) - l[targets[act[start + r]]];
        }
        if (hgrad || bgrad) {
            /* logitGradients (:275-291) */
            for (int32_t r = 0; r < count; ++r) {
                float* l = logits + (size_t)r * vocabulary;
                const float max_logit = row_max[start + r];
                const float inv_sum = 1.0f / row_sum[start + r];
                const int32_t target = targets[act[start + r]];
                for (int32_t v = 0; v < vocabulary; ++v) {
                    const float prob = (float)exp((double)(l[v] - max_logit)) * inv_sum;
                    const float indicator = v == target ? 1.0f : 0.0f;
                    l[v] = scale * (prob - indicator);
                }
            }
            if (bgrad)
                for (int32_t r = 0; r < count; ++r)
                    for (int32_t v = 0; v < vocabulary; ++v) bgrad[v] += logits[(size_t)r * vocabulary + v];
            if (hgrad) {
                status = ko_multiply_by_quantized_transposed(logits, w, chunk_grad, count, 0, threads);
                if (status) break;
                memcpy(hgrad + (size_t)start * dimension, chunk_grad, sizeof(float) * (size_t)count * dimension);
            }
        }
    }
    if (status == KO_OK) {
        *loss = total / (float)active;
        /* the backward closure (:189-205) with an upstream gradient of 1 */
        if (hgrad)
            for (int32_t r = 0; r < active; ++r)
                for (int32_t d = 0; d < dimension; ++d)
                    hidden_grad[(size_t)act[r] * dimension + d] += 1.0f * hgrad[(size_t)r * dimension + d];
        if (bgrad)
            for (int32_t v = 0; v < vocabulary; ++v) bias_grad[v] += 1.0f * bgrad[v];
    }
    free(act); free(inputs); free(logits); free(row_max); free(row_sum); free(hgrad); free(chunk_grad); free(bgrad);
    return status;
}
