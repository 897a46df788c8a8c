/*
 * kotensor_hip.h -- C ABI of libkotensor_hip.so, the MI355X (gfx950) implementation
 * of Kotensor's group-wise INT8/INT4 weight-only quantization path.
 *
 * Binding rules (what a JDK Foreign Function & Memory downcall needs):
 *   - C linkage, fixed-width integer and float arguments, plain pointers, no C++ or
 *     HIP types. A stream is an opaque pointer (a hipStream_t); NULL is the null stream.
 *   - Every data pointer passed to a compute entry point is a DEVICE pointer owned
 *     by the caller (kt_dev_alloc / kt_dev_free). The library never frees them.
 *   - Entry points are stateless and reentrant. Compute entry points enqueue work on
 *     the given stream and return before it finishes, except kt_quantize (see there).
 *     The library keeps one internal workspace per (device, stream); calls that
 *     share a stream are ordered by it, and calls on different streams never share
 *     one, with one exception: every kt_qmatmul_noalloc call on a device uses that
 *     device's single fixed array (see there), so such calls must not overlap.
 *   - Return value: KT_OK (0) on success; a negative KT_ERR_* for an argument error
 *     (the reference raises IllegalArgumentException for the same cases) except
 *     KT_ERR_STATE; a positive value is a HIP runtime error code (the reference has no
 *     counterpart). A binding maps KT_ERR_STATE and positive values to
 *     IllegalStateException. kt_last_error() returns the message of the last failure
 *     on the calling thread.
 *
 * Weight layout is the reference's; every entry point reads it as it lies, and the
 * optional device-native copy (kt_qweight.packed, written by kt_qweight_pack from these
 * bytes) only adds a faster read path for some products:
 *   qdata  [rows x bytes_per_row], row-major. 8-bit: bytes_per_row = columns, each
 *          byte a two's-complement int8. 4-bit: bytes_per_row = (columns + columns%2)/2
 *          and split-half packing: column c < bytes_per_row is the LOW nibble of byte c,
 *          column c >= bytes_per_row the HIGH nibble of byte c - bytes_per_row; the
 *          high nibble of the last byte is 0 when columns is odd.
 *   scales [groups x columns] fp32, groups = ceil(rows / group_size).
 *   zeros  [groups x columns] bytes read as signed int8 (a Kotlin ByteArray), required
 *          for 4-bit, optional (NULL) for 8-bit.
 * Reference: Engine/kotensor/src/main/kotlin/QuantizedTensor.kt:27-98 (K/ below).
 */
#ifndef KOTENSOR_HIP_H
#define KOTENSOR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KT_ABI_VERSION 4

/* Status codes. */
#define KT_OK 0
#define KT_ERR_ARGUMENT (-1)   /* bad bits / group size / count / null pointer */
#define KT_ERR_SHAPE (-2)      /* size or shape mismatch */
#define KT_ERR_NAN (-3)        /* quantize met a value Float.roundToInt() rejects */
#define KT_ERR_ZEROS (-4)      /* 4-bit tensor without zero points (K/QuantizedTensor.kt:69) */
#define KT_ERR_RANGE (-5)      /* index out of range (row / column / token) */
#define KT_ERR_STATE (-6)      /* not possible in the current state: a binding maps it to
                                  IllegalStateException (e.g. a recorded call whose stream
                                  has no workspace of the size it needs yet) */

/* A quantized weight held in device memory. Mirrors the fields of
 * QuantizedTensor (K/QuantizedTensor.kt:27-49): rows = K (in), columns = N (out).
 * packed is optional (NULL or a copy written by kt_qweight_pack): a second, device-native
 * arrangement of qdata that the one-row products read instead when it is present, and
 * the prefill GEMM too when group_size is a multiple of 32. */
typedef struct kt_qweight {
    const void* qdata;
    const float* scales;
    const uint8_t* zeros;  /* NULL iff the tensor has no zero points */
    int32_t rows;
    int32_t columns;
    int32_t bits;          /* 4 or 8 (Quantization.bits, K/QuantizedTensor.kt:10-17) */
    int32_t group_size;    /* > 0 (Quantization.groupSize) */
    const void* packed;    /* NULL, or kt_qweight_packed_bytes bytes from kt_qweight_pack */
} kt_qweight;

/* ---- library / errors --------------------------------------------------------- */
int32_t kt_abi_version(void);
/* Copies the calling thread's last error message (NUL-terminated, truncated to len). */
int32_t kt_last_error(char* buf, size_t len);
int32_t kt_device_count(int32_t* count);
int32_t kt_set_device(int32_t device);

/* Kernel selection knobs, the counterpart of MatMul's runtime knobs
 * (K/MatMul.kt:30-82: numThreads, parallelThreshold, lookupInt4): they choose how the
 * small-M kernels split their work, never their result beyond fp32 rounding order.
 * gemv_kind: 0 = automatic (the column-run kernel for one row when the weight has a
 *            packed copy; for 2 to 16 rows of small weights that are not wide, the
 *            one-row kernel once per row in one launch (each row's bits its one-row
 *            result); for 2 to 16 rows when the weight also has at least 16 column sets
 *            of 16 per 128 rows of K, or K >= 4096 and at least 256 column sets, the
 *            column-run rows kernel; otherwise for one row the column-strip kernel up to
 *            a size and the wide-strip MFMA kernel above it, and the row-block MFMA kernel
 *            for 2 to 16 rows, where the layout allows), 1 = vector-ALU kernel for M == 1 (and no MFMA
 *            GEMV for M > 1: those go to the GEMM), 2 = row-block MFMA kernel for M <= 16,
 *            3 = wide-strip MFMA kernel for M == 1, 4 = column-strip kernel for M == 1,
 *            5 = column-run kernels for M <= 16 (need the packed copy);
 * gemv_vec: vector-ALU kernel bytes per lane per row (4 or 8; 0 = automatic); for the
 *            column-run kernel, the KB of weights in flight per wave (4 or 8);
 * gemv_splits: workgroups along K per column tile (0 = automatic); for the column-run
 *            kernel, the waves that split the K range of a column set (1, 2, 4 or 8);
 * gemv_waves: waves per workgroup (2, 4 or 8; 0 = automatic; the column-run kernel
 *            always runs eight);
 * gemv_reduce: how split sums meet (0 = automatic, 1 = a second kernel, 2 = inside the
 *            kernel); for the column-run kernel at 2 to 16 rows, how the K-parts of a
 *            column set meet (1 = inside one workgroup, 2 = across workgroups, through
 *            memory; the same bits either way). Process-wide. */
int32_t kt_set_kernel_config(int32_t gemv_kind, int32_t gemv_vec, int32_t gemv_splits,
                             int32_t gemv_waves, int32_t gemv_reduce);

/* ---- device memory and streams (the Kotlin side owns every buffer) ------------ */
int32_t kt_dev_alloc(size_t bytes, void** ptr);
int32_t kt_dev_free(void* ptr);
int32_t kt_memcpy_h2d(void* dst, const void* src, size_t bytes, void* stream);
int32_t kt_memcpy_d2h(void* dst, const void* src, size_t bytes, void* stream);
int32_t kt_memcpy_d2d(void* dst, const void* src, size_t bytes, void* stream);
int32_t kt_memset(void* dst, int32_t value, size_t bytes, void* stream);
int32_t kt_stream_create(void** stream);
int32_t kt_stream_destroy(void* stream);
/* kt_stream_sync and kt_memcpy_d2h (which synchronizes) also report a bounded wait
 * inside a kernel that gave up since the stream's last synchronization (the chained
 * stages of kt_qmatmul_chain, the split merge of kt_attention / kt_rope_attention: a
 * fault, never a schedule): KT_ERR_STATE, returned once, after the stream's internal
 * counters are cleared; the outputs of the calls since the last synchronization are
 * then not valid. No counterpart in the reference (its kernels do not wait on each
 * other). */
int32_t kt_stream_sync(void* stream);
/* Test hook for that report, no counterpart in the reference: spin_limit replaces the
 * polls a wait makes before it gives up (0 = the kernels' own limits) and withhold = 1
 * makes the producers of those waits (a chained stage's partition flags, an attention
 * split's tagged sums) withhold their signals, so that every wait gives up while every
 * kernel still exits normally. Process-wide; read when a call is enqueued (recorded
 * graphs keep the values they were recorded with). */
int32_t kt_debug_wait_limits(uint32_t spin_limit, int32_t withhold);
/* HIP graphs: kernels enqueued on `stream` between kt_graph_begin and kt_graph_end are
 * recorded (not run) and instantiated into *graph, which kt_graph_launch replays on a
 * stream. The replacement for a tracing compiler on the decode path: one decode step
 * is recorded once and replayed per token. No counterpart in the reference.
 * Workspace rules: a recorded call uses the workspace of the stream it was recorded
 * on, which must already be large enough (one eager call of the same shapes on that
 * stream sizes it); otherwise the call returns KT_ERR_STATE and nothing is allocated
 * or recorded for it. A workspace that a graph addresses is never freed before the
 * process ends, even when a later call grows it or the stream is destroyed. Replays
 * and eager calls that share a workspace must not run concurrently: replay a graph on
 * the stream it was recorded on, or keep that stream idle during the replay. */
int32_t kt_graph_begin(void* stream);
int32_t kt_graph_end(void* stream, void** graph);
int32_t kt_graph_launch(void* graph, void* stream);
int32_t kt_graph_destroy(void* graph);

/* ---- format helpers (pure host arithmetic, no device work) -------------------- */
/* groups, storedColumns, bytesPerRow and sizeInBytes of K/QuantizedTensor.kt:47-49,97-98. */
int32_t kt_qweight_layout(int32_t rows, int32_t columns, int32_t bits, int32_t group_size,
                          int32_t has_zeros, int64_t* out4);
/* Validates a weight the way the QuantizedTensor constructor does
 * (K/QuantizedTensor.kt:63-70). */
int32_t kt_qweight_check(const kt_qweight* w);

/* ---- the column-run copy (no counterpart in the reference) ---------------------
 * The reference's layout keeps a row of the weight contiguous, which makes a one-row
 * product at shapes like 4096 -> 14336 split its K range over workgroups and meet their
 * sums through memory. The column-run copy keeps each column's K values contiguous in
 * 16-column blocks (1 KB per 128 k for 4-bit, 2 KB for 8-bit), so the one-row kernel
 * reads whole columns with no cross-workgroup sums; the prefill GEMM (three or more
 * rows, group_size % 32 == 0) reads each lane's MFMA operand bytes from it as 16 or 8
 * contiguous bytes. After the weight blocks come the scales and zero points of every
 * 16-column set as rows [set][group][16] (fp32, then bytes), so that a wave reads the
 * groups of its K range as contiguous bytes. It is a device-side accelerator next to
 * qdata, scales and zeros, not a format: files, quantize and the accessors keep using
 * those. Write it once after they are final (and again if they change), then set
 * kt_qweight.packed. It ends in a 16-byte trailer: the weight's largest |scale| (fp32,
 * NaNs ignored), which the prefill GEMM takes as its dequantization range, then zeros.
 * Size: sets * ceil(rows / 128) * (bits == 4 ? 1024 : 2048) + sets * ceil(rows /
 * group_size) * 80 + 16 bytes with sets = ceil(columns / 16), 16-byte aligned. */
int32_t kt_qweight_packed_bytes(int32_t rows, int32_t columns, int32_t bits, int32_t group_size, int64_t* bytes);
/* Writes the copy of w's qdata, scales and zeros into `packed` (kt_qweight_packed_bytes
 * bytes of device memory, 16-byte aligned); w->packed is ignored. Asynchronous. */
int32_t kt_qweight_pack(const kt_qweight* w, void* packed, void* stream);

/* ---- quantize + pack ---------------------------------------------------------- */
/* QuantizedTensor.quantize(data, rows, columns, Quantization(bits, group_size)),
 * K/QuantizedTensor.kt:256-324. data fp32 [rows x columns] row-major on the device.
 * Writes qdata [rows x bytes_per_row], scales [groups x columns] and, for 4-bit,
 * zeros [groups x columns]; zeros must be NULL for 8-bit. Bit-exact with the
 * reference: scale = maxAbs/127 (8-bit) or (max-min)/15 with 0 inside [min,max]
 * (4-bit), q = Math.round(x * (1/scale)) (ties toward +inf), clamped.
 * SYNCHRONOUS: it waits for the stream, because a NaN in the rounding step makes
 * the reference throw; that case returns KT_ERR_NAN (output contents unspecified). */
int32_t kt_quantize(const float* data, int32_t rows, int32_t columns, int32_t bits,
                    int32_t group_size, void* qdata, float* scales, uint8_t* zeros,
                    void* stream);

/* ---- dequantizing matmul -------------------------------------------------------- */
/* MatMul.multiplyQuantized(a, weight, c, m, accumulate, alpha), K/MatMul.kt:460-486:
 *   c[m x N] = (accumulate ? c : 0) + alpha * (a[m x K] . deq(W)),
 * deq(W)[k][n] = scale[k/g][n] * (q[k][n] - zero[k/g][n]), applied per group after an
 * integer-valued accumulation (K/MatMul.kt:804-828,942-952). fp32 in and out.
 * m == 0 is a no-op (K/MatMul.kt:473). Asynchronous. */
int32_t kt_qmatmul(const float* a, int32_t m, const kt_qweight* w, float* c,
                   int32_t accumulate, float alpha, void* stream);

/* kt_qmatmul that allocates nothing. No counterpart in the reference: it is for callers
 * that cannot allocate device memory -- code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc. Same arguments, kernels and results (bit for
 * bit) as kt_qmatmul, but the kernels' scratch memory (split sums, counters, the
 * prepared x of the prefill GEMM) is a fixed 64 MiB device array of the library, one
 * per GPU, held until the process ends, instead of the per-stream workspace. A call
 * whose scratch would exceed it returns KT_ERR_SHAPE before launching anything (one-row
 * products need at most 8 bytes per output column, so N up to half a million fits; the
 * prefill GEMM needs about 2 * M * K bytes). The first call
 * on a device sets the array up and waits for that (KT_ERR_STATE if the stream is
 * capturing then); later calls may be recorded into graphs. Every call on a GPU shares
 * that GPU's array: calls that overlap in time on one GPU (two streams, two threads, or
 * a replay next to an eager call) race and must be serialized by the caller. */
int32_t kt_qmatmul_noalloc(const float* a, int32_t m, const kt_qweight* w, float* c,
                           int32_t accumulate, float alpha, void* stream);

/* QuantizedLinear.forwardInto(input, out), K/QuantizedLinear.kt:22-25 (with
 * Tensor.matmulDequantInto K/Tensor.kt:180-188 and addInPlace K/Tensor.kt:201-221):
 *   out[m x N] = a . deq(W) + bias (bias fp32 [N] broadcast over rows, or NULL). */
int32_t kt_qlinear_forward(const float* a, int32_t m, const kt_qweight* w, const float* bias,
                           float* out, void* stream);

/* Several projections of the same input in one call: for i < count,
 *   outputs[i] = (accumulate ? outputs[i] : 0) + alpha * a . deq(weights[i]) (+ biases[i]).
 * Replaces consecutive QuantizedLinear.forwardInto calls on one input -- wQ/wK/wV in
 * Attention.decodeInto (K/Attention.kt:220-222) and wGate/wUp in SwiGLU.forwardInto
 * (K/SwiGLU.kt:19-25) -- with one launch per four weights when m == 1. The weights
 * must share rows, bits and group size; columns may differ. biases may be NULL, or
 * an array whose entries may be NULL. Asynchronous. */
int32_t kt_qmatmul_group(const float* a, int32_t m, const kt_qweight* weights, int32_t count,
                         float* const* outputs, const float* const* biases, int32_t accumulate,
                         float alpha, void* stream);

/* MatMul.multiplyByQuantizedTransposed(dy, weight, dx, m, accumulate),
 * K/MatMul.kt:954-981:  dx[m x K] = (accumulate ? dx : 0) + dy[m x N] . deq(W)^T.
 * 8-bit rows are dequantized without zero points, as dequantizeRow does
 * (K/QuantizedTensor.kt:198-202). Asynchronous. */
int32_t kt_qmatmul_transposed(const float* dy, int32_t m, const kt_qweight* w, float* dx,
                              int32_t accumulate, void* stream);

/* fusedCrossEntropyLoss(hidden, head, targets, ignoreIndex) with a QuantizedLinear head,
 * K/Loss.kt:114-219: the loss and the gradients its backward closure adds for an upstream
 * gradient of 1. hidden [rows x K] device; head: K -> N with bias [N] (device, NULL =
 * zeros); targets [rows] HOST int32, each ignore_index or in [0, N) (read before the call
 * returns). *loss (device float) = mean over the other rows of max + ln(sum exp(l - max))
 * - l[target], l = hidden . deq(W) + bias. hidden_grad [rows x K] and bias_grad [N]
 * (device, each may be NULL) receive d loss / d hidden and d loss / d bias, added to
 * what they hold when accumulate != 0 (ignored rows get 0). Rows go through in chunks of
 * 2^22 / N logits as in the reference; scratch for one chunk is allocated on the stream
 * (hipMallocAsync) and freed after it. Asynchronous. KT_ERR_ARGUMENT for no rows or a
 * target out of range ("target t out of bounds N"). */
int32_t kt_fused_cross_entropy(const float* hidden, int32_t rows, const kt_qweight* head, const float* bias,
                               const int32_t* targets, int32_t ignore_index, float* loss, float* hidden_grad,
                               float* bias_grad, int32_t accumulate, void* stream);

/* ---- dequant accessors ---------------------------------------------------------- */
/* dequantizeRow for each index in rows[0..count) (device int32 array), writing
 * out[i x N]; the row gather of QuantizedEmbedding.lookupInto/forward
 * (K/Embedding.kt:73-113 -> K/QuantizedTensor.kt:188-213). Indices outside
 * [0, rows) yield rows of NaN (kotensor_amd checks indices on the host first). */
int32_t kt_dequantize_rows(const kt_qweight* w, const int32_t* rows, int32_t count, float* out,
                           void* stream);
/* dequantizeColumn for each index in columns[0..count), writing out[i x K]; the
 * tied-embedding gather of TiedQuantizedEmbedding (K/Embedding.kt:115-136 ->
 * K/QuantizedTensor.kt:235-241). An index outside [0, columns) produces NaN. */
int32_t kt_dequantize_columns(const kt_qweight* w, const int32_t* columns, int32_t count,
                              float* out, void* stream);

/* ---- the rest of the decode/prefill step (kt_decoder.hip) ------------------------
 * The pieces of Transformer.prefill/decode around the projections (K/Transformer.kt:
 * 99-154, K/TransformerBlock.kt:204-220), device-resident. `position` is a device
 * int32 holding the KV cache length (KVCache.length, K/KVCache.kt:12), read by the
 * kernels and advanced with kt_position_add, so a decode step can be recorded in a HIP
 * graph and replayed per token. The cache layout is KVCache's: keys and values of
 * [layers x kv_heads x max_seq x head_dim] fp32 (K/KVCache.kt:9-27). The host checks
 * capacity (the reference's "KV cache full" errors); the kernels never read or write
 * outside the cache. */

/* RoPE.invFreq with optional RoPEScaling (K/RoPE.kt:18-46), computed on the host into
 * out[head_dim / 2]; factor <= 0 means no scaling. */
int32_t kt_rope_inv_freq(int32_t head_dim, float base, float factor, float low, float high,
                         int32_t original_max, float* out);
/* RMSNorm.forwardInto (K/RMSNorm.kt:71-90): out[r] = x[r] * rsqrt(mean(x[r]^2) + eps) * weight,
 * rows x dim (out may alias nothing but itself). */
int32_t kt_rmsnorm(const float* x, int32_t rows, int32_t dim, const float* weight, float eps,
                   float* out, void* stream);
/* RoPE.applyRowsInPlace on q [tokens x num_heads*head_dim] and k [tokens x
 * num_kv_heads*head_dim] at positions *position + t (K/RoPE.kt:139-164), then the
 * cache writes of rotated k and of v for those positions (K/Attention.kt:254-270;
 * decodeInto :220-233 is tokens = 1). inv_freq: device [head_dim / 2]. */
int32_t kt_rope_kv(float* q, float* k, const float* v, int32_t tokens, int32_t num_heads,
                   int32_t num_kv_heads, int32_t head_dim, const float* inv_freq,
                   const int32_t* position, float* cache_k, float* cache_v, int32_t layer,
                   int32_t max_seq, void* stream);
/* Attention.attendCached (K/Attention.kt:277-349): for token t at position *position + t,
 * softmax(q . k_j / sqrt(head_dim)) over cached positions j <= that position, of the
 * kv head that serves its query head (GQA), times v, into context [tokens x
 * num_heads*head_dim]. key_bound >= *position + tokens bounds the keys (it sizes the
 * launch; a captured decode step passes max_seq). q and the caches are 16-byte aligned.
 * For fewer than 16 tokens the keys are split over workgroups whose partials meet in the
 * stream's workspace (its zeroed region, zero again when the launch ends); as for every
 * call that takes the workspace, a graph is recorded after one eager call of the same
 * shapes on the stream. */
int32_t kt_attention(const float* q, int32_t tokens, const int32_t* position, int32_t key_bound,
                     const float* cache_k, const float* cache_v, int32_t layer, int32_t max_seq,
                     int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float* context,
                     void* stream);
/* kt_rope_kv followed by kt_attention (Attention.decodeInto/prefillInto,
 * K/Attention.kt:207-275): RoPE on q and k at *position + t, k and v appended to the
 * cache, then the cached attention into context. For one token (a decode step) RoPE and
 * the append happen inside the attention launch: q and k are left as they were (the
 * rotated q lives in LDS) and the cache row is written by the workgroup that reads it.
 * For more tokens q and k are rotated in place, as kt_rope_kv does. Saves the RoPE
 * launch of a decode step. A one-token call for layer 0 also leaves cos and sin of its
 * position in the stream's workspace, and one-token calls for other layers use them when
 * position and frequencies match (otherwise they compute them: the same bits either way). */
int32_t kt_rope_attention(float* q, float* k, const float* v, const float* inv_freq, int32_t tokens,
                          const int32_t* position, int32_t key_bound, float* cache_k, float* cache_v,
                          int32_t layer, int32_t max_seq, int32_t num_heads, int32_t num_kv_heads,
                          int32_t head_dim, float* context, void* stream);
/* SwiGLU's gate (K/SwiGLU.kt:19-25; K/Tensor.kt:223-237): gate[i] = silu(gate[i]) * up[i]. */
int32_t kt_silu_mul(float* gate, const float* up, int64_t n, void* stream);
/* RMSNorm.forward (K/RMSNorm.kt) of x [m x K] with weight, then the grouped projections of
 * kt_qmatmul_group on the normalized rows: outputs[i] = (accumulate ? outputs[i] : 0)
 * + alpha * RMSNorm(x) . deq(W_i) (+ biases[i]) (Attention's q/k/v, SwiGLU's gate/up, all
 * weights with K rows). For one row and at most four weights the M = 1 kernel multiplies
 * x * weight and scales the sums by 1 / sqrt(mean(x^2) + eps), the sum of squares reduced
 * exactly as kt_rmsnorm reduces it (normed is not written); otherwise kt_rmsnorm writes
 * normed [m x K] and kt_qmatmul_group follows. Saves the RMSNorm launch of a decode step. */
int32_t kt_rmsnorm_qmatmul_group(const float* x, const float* norm_weight, float eps, float* normed, int32_t m,
                                 const kt_qweight* weights, int32_t count, float* const* outputs,
                                 const float* const* biases, int32_t accumulate, float alpha, void* stream);
/* SwiGLU's gate and up projections and its gate in one call (K/SwiGLU.kt:19-25; with
 * RMSNorm.forward of x first when norm_weight is not NULL, as the decoder block's norm2,
 * K/RMSNorm.kt): up = RMSNorm(x) . deq(w_up) (+ bias_up) and
 * gate = silu(RMSNorm(x) . deq(w_gate) (+ bias_gate)) * up, silu(g) = g / (1 + exp(-g))
 * exactly as kt_silu_mul computes it; gate and up are [m x N]. For one row on weights with
 * column-run copies one launch: each workgroup multiplies the same columns of both weights
 * and computes the gate in its epilogue (normed is not written); otherwise
 * kt_rmsnorm_qmatmul_group (or kt_qmatmul_group) then kt_silu_mul. The down projection is
 * then a plain product of gate. Saves a decode step's separate gate work. */
int32_t kt_rmsnorm_swiglu_gate(const float* x, const float* norm_weight, float eps, float* normed, int32_t m,
                               const kt_qweight* w_gate, const kt_qweight* w_up, const float* bias_gate,
                               const float* bias_up, float* gate, float* up, void* stream);
/* One step of kt_qmatmul_chain: a one-row kt_qmatmul_group over `count` weights sharing
 * K; with norm_weight, RMSNorm of x first (kt_rmsnorm_qmatmul_group; normed is its K
 * floats of scratch); with swiglu_gate, weights = {gate, up} and outputs = {gate, up} as
 * kt_rmsnorm_swiglu_gate gives them (accumulate 0, alpha 1). biases is NULL or `count`
 * pointers, each NULL or N floats. */
typedef struct kt_qmatmul_step {
    const float* x;
    const float* norm_weight;
    float eps;
    float* normed;
    const kt_qweight* weights;
    int32_t count;
    float* const* outputs;
    const float* const* biases;
    int32_t accumulate;
    float alpha;
    int32_t swiglu_gate;
} kt_qmatmul_step;

/* Dependent one-row products, in order, each free to read earlier steps' outputs and to
 * write what earlier steps read, with the effect of calling each step on its own: a
 * decoder layer's projections between two attention calls (K/TransformerBlock.kt:40-46:
 * wOut and its residual add into x, norm2 and the FFN, the down projection's residual add,
 * then the next layer's norm1 and q/k/v, K/Attention.kt:222-224). When every weight has
 * its column-run copy and all share one width and zero-point form, the steps run as one
 * launch in which a step's workgroups fetch their first weights while earlier steps
 * compute and wait on device counters (in the stream's workspace) only for their input
 * row; otherwise as the calls named, one after another. 1 to 6 steps. */
int32_t kt_qmatmul_chain(const kt_qmatmul_step* steps, int32_t count, void* stream);
/* SwiGLU.forwardInto's gate followed by the down projection (K/SwiGLU.kt:19-25 then
 * QuantizedLinear.forwardInto, K/QuantizedLinear.kt:16-25):
 * c = (accumulate ? c : 0) + alpha * (silu(gate) * up) . deq(W) (+ bias), gate and up
 * [m x K]. For one row the M = 1 kernel computes the gate while it loads its input and
 * gate is left unchanged; otherwise gate is overwritten with silu(gate) * up (exactly
 * kt_silu_mul) and the product follows. Saves the gate launch of a decode step. */
int32_t kt_swiglu_qmatmul(float* gate, const float* up, int32_t m, const kt_qweight* w, float* c,
                          int32_t accumulate, float alpha, const float* bias, void* stream);
/* Transformer.argmaxOfLastToken (K/Transformer.kt:253-266) of logits[0..n) into the
 * device int32 *index: the first index of the largest logit above -1e9, else 0. */
int32_t kt_argmax(const float* logits, int32_t n, int32_t* index, void* stream);
/* One greedy decode step's bookkeeping in one launch: kt_argmax(logits, n, token), then
 * *position += 1 (kt_position_add) and generated[*position] = *token when 0 <= *position <
 * capacity (kt_record_token; generated may be NULL). The effect of those three calls in
 * the order the reference's greedy loop makes them (K/Transformer.kt:224-231: take the
 * argmax, advance the cache, hand the token out); the argmax does not read the position. */
int32_t kt_argmax_advance(const float* logits, int32_t n, int32_t* token, int32_t* position,
                          int32_t* generated, int32_t capacity, void* stream);
/* KVCache.advance on the device copy of the length (K/KVCache.kt:29-35): *position += count. */
int32_t kt_position_add(int32_t* position, int32_t count, void* stream);
/* generated[*position] = *token when 0 <= *position < capacity: the device-side record of
 * the greedy tokens of generate (K/Transformer.kt:224-231 yields them one by one), read
 * by the host once at the end instead of after every step. */
int32_t kt_record_token(const int32_t* token, const int32_t* position, int32_t* generated,
                        int32_t capacity, void* stream);
/* Tensor.addInPlace (K/Tensor.kt:201-221): x[i] = x[i] + y[i]; the residual adds of
 * TransformerBlock.decodeInto/prefillInto (K/TransformerBlock.kt:207-219). */
int32_t kt_add_inplace(float* x, const float* y, int64_t n, void* stream);
/* Synthetic weights: out[i] = mean + stddev * N(0,1), element i a function of (seed, i)
 * only (SplitMix64 and Box-Muller). No counterpart in the reference, which draws its
 * initial weights from kotlin.random; used to build random-init models on the device. */
int32_t kt_fill_normal(float* out, int64_t n, uint64_t seed, float mean, float stddev, void* stream);

/* ---- saveQuantized files (safetensors) -------------------------------------------
 * The reference stores quantized models as safetensors (SafeTensors.kt:12-249): an
 * 8-byte little-endian header size, a JSON header (tensor name -> dtype, shape,
 * data_offsets; "__metadata__" -> string map), then the tensor bytes. saveQuantized
 * (Transformer.kt:402-430) writes each quantized weight NAME as NAME.qweight (I8 for
 * 8-bit, U8 for 4-bit) [rows x bytes_per_row], NAME.scales F32 [groups x columns] and,
 * with zero points, NAME.zeros U8 [groups x columns], plus kotensor.* metadata. These
 * entry points read such files into device buffers without repacking (the kernels
 * consume the file layout) and write them back byte for byte. Host-side; only
 * kt_st_load_qweight and kt_st_writer_save touch the device. */
typedef struct kt_st_file kt_st_file;      /* a read-only mapping of one file */
typedef struct kt_st_writer kt_st_writer;  /* entries and metadata of a file to write */

typedef struct kt_st_entry {
    char dtype[8];       /* "F32", "I8", "U8", ... (NUL-terminated) */
    int32_t rank;        /* number of dimensions, at most 8 */
    int64_t shape[8];
    int64_t offset;      /* byte offset of the data from the start of the file */
    int64_t nbytes;      /* data_offsets[1] - data_offsets[0] */
} kt_st_entry;

/* SafeTensorsFile(file) (SafeTensors.kt:37-67): maps the file read-only and parses the
 * header with the reference's checks (header size in 1 .. 100 MiB, every tensor with a
 * dtype and data_offsets inside the file). KT_ERR_ARGUMENT with the reference's
 * message on a malformed file. */
int32_t kt_st_open(const char* path, kt_st_file** file);
int32_t kt_st_close(kt_st_file* file);
/* names (:69-70): entry count and the index-th name in header order. */
int32_t kt_st_count(const kt_st_file* file, int32_t* count);
int32_t kt_st_name(const kt_st_file* file, int32_t index, char* buf, size_t len);
/* entry(name) (:74-75); KT_ERR_ARGUMENT "No tensor named ..." when absent. */
int32_t kt_st_find(const kt_st_file* file, const char* name, kt_st_entry* entry);
/* metadata[key] (:40, :51-55) as text; KT_ERR_ARGUMENT when the key is absent. */
int32_t kt_st_metadata(const kt_st_file* file, const char* key, char* buf, size_t len);
/* The index-th metadata key in header order; KT_ERR_RANGE past the last one. */
int32_t kt_st_metadata_key(const kt_st_file* file, int32_t index, char* buf, size_t len);
/* map(name) (:101-107): the entry's bytes inside the mapping (valid until kt_st_close). */
int32_t kt_st_data(const kt_st_file* file, const char* name, const void** data, int64_t* nbytes);
/* QuantizedTensor.mapFrom (QuantizedTensor.kt:109-125) onto the device: checks
 * NAME.qweight, NAME.scales (F32) and NAME.zeros against w's layout with the reference's
 * messages, then copies them into w's device buffers (w->zeros is written when NAME.zeros
 * is required, i.e. when w has zero points). Returns when the copies are done. */
int32_t kt_st_load_qweight(const kt_st_file* file, const char* name, const kt_qweight* w, void* stream);

/* SafeTensors.saveEntries (SafeTensors.kt:204-249): entries and metadata are written in
 * the order added, with the reference's header text, padding and data order, so a file
 * loaded and saved again is identical byte for byte (MappedModelTest.kt:108-119). */
int32_t kt_st_writer_create(kt_st_writer** writer);
int32_t kt_st_writer_destroy(kt_st_writer* writer);
int32_t kt_st_writer_metadata(kt_st_writer* writer, const char* key, const char* value);
/* One entry: nbytes of data at `data` (device memory when on_device != 0, else host
 * memory), kept by reference until kt_st_writer_save. */
int32_t kt_st_writer_add(kt_st_writer* writer, const char* name, const char* dtype, int32_t rank,
                         const int64_t* shape, const void* data, int64_t nbytes, int32_t on_device);
/* The entries saveQuantized writes for one quantized weight (Transformer.kt:425-428):
 * NAME.qweight, NAME.scales and (with zero points) NAME.zeros, from w's device buffers. */
int32_t kt_st_writer_add_qweight(kt_st_writer* writer, const char* name, const kt_qweight* w);
int32_t kt_st_writer_save(kt_st_writer* writer, const char* path, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* KOTENSOR_HIP_H */
