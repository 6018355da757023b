/*
 * higgs_qmm.h -- C ABI of the MI355X (gfx950) MLX-format affine
 * group-quantized linear path: quantized_matmul (qmv for decode, qmm for
 * prefill), gather_qmm (MoE experts) and dequantize.
 *
 * Conventions shared by every entry point
 *  - All data pointers are device pointers (HBM), caller-owned. Nothing in
 *    this library allocates device memory for these calls.
 *  - `stream` is a hipStream_t (NULL = the default stream). Work is enqueued
 *    on it and the call returns without synchronising.
 *  - Quantized matrices use MLX's layout: a logical [rows, cols] matrix of
 *    `bits`-bit unsigned integers is stored as uint32 [rows, cols*bits/32];
 *    element i of a row sits at bit i*bits of the row's little-endian
 *    bitstream, least significant bits first (3-, 5- and 6-bit values
 *    straddle word boundaries). scales and biases are [rows, cols/group_size]
 *    and dequantize as  w = scale * q + bias.
 *  - bits in {2, 3, 4, 5, 6, 8}; group_size in {32, 64, 128}.
 *  - x_dtype / s_dtype are hq_dtype codes for the activations and for the
 *    scales+biases. The output dtype follows MLX promotion:
 *    hq_result_dtype(x_dtype, s_dtype) (equal -> same, mixed -> float32).
 *  - Return value: HQ_OK (0) or an hq_status error; the message of the last
 *    error on the calling thread is returned by hq_last_error().
 *  - Calls on one stream are ordered. The library keeps no per-call state;
 *    its only shared state is one-time launcher setup per device (the CU
 *    count, opting kernels into more than 64 KB of LDS), held in atomics, so
 *    concurrent calls from several threads on different streams or devices
 *    are safe.
 */
#ifndef HIGGS_QMM_H
#define HIGGS_QMM_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HQ_ABI_VERSION 3

typedef enum hq_status {
  HQ_OK = 0,
  HQ_ERR_INVALID_ARGUMENT = 1, /* shape / dtype / bits / group_size rejected */
  HQ_ERR_UNSUPPORTED = 2,      /* valid for MLX but not implemented here */
  HQ_ERR_HIP = 3               /* a HIP runtime call or kernel launch failed */
} hq_status;

typedef enum hq_dtype {
  HQ_DTYPE_FLOAT32 = 0,
  HQ_DTYPE_FLOAT16 = 1,
  HQ_DTYPE_BFLOAT16 = 2
} hq_dtype;

/* Library version string, e.g. "higgs_qmm 0.1.0 (gfx950)". */
const char* hq_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* hq_last_error(void);

/* Output dtype of quantized_matmul / gather_qmm for these input dtypes, or
 * -1 if either code is not an hq_dtype. */
int hq_result_dtype(int x_dtype, int s_dtype);

/*
 * y = x . deq(W)^T  (transpose != 0) or  y = x . deq(W)  (transpose == 0).
 *
 * Replaces mlx-rs ops::quantized_matmul(x, w, scales, biases, transpose,
 * group_size, bits) as called by higgs' QLinear / quantized_forward
 * (crates/higgs-models/src/qwen3_next.rs:218-227, 255-264), QEmbedding::
 * as_linear (qwen3_next.rs:320-333), the fused dense FFN
 * (qwen3_next.rs:2539-2585) and every MaybeQuantized nn::Linear
 * (crates/higgs-models/src/transformer.rs:148-157, 257-259, 355-356, 843-847).
 *
 *   x: [M, K] of x_dtype (all leading batch dims of MLX's x flattened into M)
 *   transpose != 0: w [N, K*bits/32], scales/biases [N, K/group_size]
 *   transpose == 0: w [K, N*bits/32], scales/biases [K, N/group_size]
 *   y: [M, N] of hq_result_dtype(x_dtype, s_dtype)
 *
 * M == 0 or N == 0 is a valid empty call. K must be a positive multiple of
 * group_size when transpose != 0 (N likewise when transpose == 0).
 */
int hq_quantized_matmul(void* y, const void* x, const uint32_t* w,
                        const void* scales, const void* biases, int64_t M,
                        int64_t N, int64_t K, int transpose, int group_size,
                        int bits, int x_dtype, int s_dtype, void* stream);

/*
 * Quantized linear layer with an optional bias:  y = x . deq(W)^T + bias.
 *
 * Replaces mlx-rs QuantizedLinear::forward (quantized_matmul with
 * transpose=true, then add the bias when the layer has one), which
 * mlx_rs::nn::quantize makes of every MaybeQuantized nn::Linear at load
 * (crates/higgs-models/src/transformer.rs:954-965). Qwen2-style checkpoints
 * give q_proj, k_proj and v_proj a bias (qkv_bias, transformer.rs:180-191),
 * stored as <layer>.bias / .inner.bias (crates/higgs-models/src/lib.rs:
 * 1002-1005).
 *
 *   x: [M, K]; w: [N, K*bits/32]; scales/biases: [N, K/group_size];
 *   bias: [N] of bias_dtype, or NULL (then this is hq_quantized_matmul with
 *   transpose = 1); y: [M, N] of hq_result_dtype(x_dtype, s_dtype).
 *
 * Rounding: y = round(round(x . deq(W)^T) + bias) -- the product is rounded
 * to the output dtype as MLX materialises it, then the sum is rounded (one
 * rounding in all for float32 output). bias_dtype must equal the output
 * dtype (HQ_ERR_UNSUPPORTED otherwise; MLX would promote the sum).
 */
int hq_quantized_linear(void* y, const void* x, const uint32_t* w,
                        const void* scales, const void* biases, const void* bias,
                        int64_t M, int64_t N, int64_t K, int group_size, int bits,
                        int x_dtype, int s_dtype, int bias_dtype, void* stream);

/*
 * Batched quantized matmul with expert gather.
 *
 * Replaces mlx_sys::mlx_gather_qmm(res, x, w, scales, biases, lhs_indices,
 * rhs_indices, transpose, group_size, bits, "affine", sorted_indices, stream)
 * as wrapped by higgs' gather_qmm (crates/higgs-models/src/qwen3_next.rs:
 * 509-578) and called by SwitchMlpWeights::forward_gather /
 * forward_gather_global_sort (qwen3_next.rs:1660-1720, 1731-1809).
 *
 *   x: [x_batch, M, K]; w: [w_batch, N, K*bits/32] (transpose != 0) or
 *   [w_batch, K, N*bits/32] (transpose == 0); scales/biases: [w_batch, rows,
 *   cols/group_size]; lhs_indices, rhs_indices: uint32 [batch] (already
 *   broadcast against each other); y: [batch, M, N].
 *
 *   For i in [0, batch):
 *     xi = lhs_indices ? lhs_indices[i] : i / (batch / x_batch)
 *     wi = rhs_indices[i]
 *     y[i] = x[xi] . deq(W[wi])^T   (or . deq(W[wi]) when transpose == 0)
 *
 * lhs_indices == NULL is MLX's null-lhs sentinel for the broadcast higgs
 * uses: x's batch dims are a prefix of the output batch dims, each x batch
 * element repeated batch/x_batch times (batch % x_batch must be 0). Other
 * broadcasts pass explicit lhs_indices.
 * sorted_indices != 0 promises rhs_indices is non-decreasing (the global
 * expert sort, qwen3_next.rs:1748-1761); with transpose != 0 and same-type
 * 16-bit x and scales it selects the grouped kernel, which streams each
 * expert's weights once for all rows of that expert. As with MLX's sorted
 * path, the promise is relied on: unsorted indices with sorted_indices != 0
 * give unspecified results. sorted_indices == 0 accepts any order.
 * Indices out of range (xi >= x_batch or wi >= w_batch) never cause an
 * out-of-bounds read: their output rows are filled with NaN.
 */
int hq_gather_qmm(void* y, const void* x, const uint32_t* w, const void* scales,
                  const void* biases, const uint32_t* lhs_indices,
                  const uint32_t* rhs_indices, int64_t batch, int64_t x_batch,
                  int64_t w_batch, int64_t M, int64_t N, int64_t K,
                  int transpose, int group_size, int bits, int sorted_indices,
                  int x_dtype, int s_dtype, void* stream);

/*
 * out = scales * q + biases, in the scales' dtype (s_dtype).
 *
 * Replaces mlx-rs ops::dequantize(w, scales, biases, group_size, bits) as
 * called by higgs' QEmbedding::forward (crates/higgs-models/src/
 * qwen3_next.rs:308-318).
 *
 *   w: [rows, K*bits/32]; scales/biases: [rows, K/group_size]; out: [rows, K].
 *   rows * K < 2^34 (HQ_ERR_INVALID_ARGUMENT otherwise).
 *
 * Rounding: for 16-bit scales each element is round(round(q*s) + b) -- the
 * product and the sum each rounded to s_dtype (round-to-nearest-even), as
 * MLX's op-by-op dequantize computes it; for float32 scales the product and
 * the sum each round to float32 (no fused multiply-add).
 */
int hq_dequantize(void* out, const uint32_t* w, const void* scales,
                  const void* biases, int64_t rows, int64_t K, int group_size,
                  int bits, int s_dtype, void* stream);

/*
 * Affine group quantization: the inverse direction of hq_dequantize.
 *
 * Replaces mlx-rs ops::quantize(w, group_size, bits) -- used by higgs' tests
 * to make quantized operands (crates/higgs-models/src/qwen3_next.rs:
 * 4305-4307, 12942) and by mlx_rs::nn::quantize, which quantizes every
 * MaybeQuantized layer of a float checkpoint at load (crates/higgs-models/
 * src/transformer.rs:954-965).
 *
 *   w: [rows, K] of dtype; wq: uint32 [rows, K*bits/32] (MLX packing);
 *   scales, biases: [rows, K/group_size] of dtype. K % group_size == 0,
 *   rows * K < 2^40.
 *
 * Per group of group_size consecutive elements, every operation computed in
 * float32 and rounded to dtype (MLX's op-by-op form):
 *   mx = max, mn = min, n_bins = 2^bits - 1,
 *   scale = max((mx - mn) / n_bins, dtype(1e-7));
 *   if |mn| > |mx| the edge is mn, else the edge is mx and scale = -scale;
 *   q0 = rint(edge / scale); if q0 != 0: scale = edge / q0, bias = edge,
 *   else bias = 0;  q = clip(rint((w - bias) / scale), 0, n_bins).
 * The edge of larger magnitude is an exact multiple of the scale, so w = 0
 * maps to an integer code (zero is representable). rint rounds half to even;
 * divisions are IEEE. NaN inputs give unspecified codes.
 */
int hq_quantize(uint32_t* wq, void* scales, void* biases, const void* w,
                int64_t rows, int64_t K, int group_size, int bits, int dtype,
                void* stream);

/*
 * Row gather then dequantize: out[i] = deq(W[indices[i]]), i in [0, n).
 *
 * Replaces the take_axis(w/scales/biases) + ops::dequantize sequence of
 * higgs' QEmbedding::forward (crates/higgs-models/src/qwen3_next.rs:308-318),
 * fused so that only the selected rows are read.
 *
 *   w: [rows, K*bits/32]; scales/biases: [rows, K/group_size];
 *   indices: uint32 [n]; out: [n, K] of s_dtype. Rows whose index is
 *   >= rows are filled with NaN.
 */
int hq_embedding_dequantize(void* out, const uint32_t* w, const void* scales,
                            const void* biases, const uint32_t* indices,
                            int64_t n, int64_t rows, int64_t K, int group_size,
                            int bits, int s_dtype, void* stream);

/*
 * Fused gate/up projection and SwiGLU of a dense MLP:
 *   h = swiglu(x . deq(Wg)^T, x . deq(Wu)^T),  swiglu(g, u) = g * sigmoid(g) * u.
 *
 * Replaces higgs' FfnBlock::dense_hidden_fused (crates/higgs-models/src/
 * qwen3_next.rs:2539-2585): one quantized_matmul over gate and up
 * concatenated along N, split at N, then silu_mul (qwen3_next.rs:437-452;
 * swiglu at 340-342). Here both projections run in one launch and the
 * elementwise op is applied in the kernel's epilogue, so the [M, 2N]
 * intermediate never reaches HBM. The gate and up matrices may be two
 * halves of one concatenated buffer (w_up = w_gate + N*K*bits/32 words) or
 * separate buffers.
 *
 *   x: [M, K]; w_gate, w_up: [N, K*bits/32]; s_*, b_*: [N, K/group_size];
 *   h: [M, N] of x_dtype.
 *
 * Rounding: gate and up are each rounded to x_dtype (as the reference
 * materialises them), swiglu is evaluated in float32 and rounded once.
 * Supported: x_dtype == s_dtype in {float16, bfloat16}, and either
 * M <= 11 with K a multiple of 1024 (and M <= 4 when group_size == 32), or
 * M >= 12 with K a multiple of 64. Other shapes return HQ_ERR_UNSUPPORTED;
 * callers then use hq_quantized_matmul for both halves and hq_swiglu.
 */
int hq_quantized_matmul_swiglu(void* h, const void* x, const uint32_t* w_gate,
                               const void* s_gate, const void* b_gate,
                               const uint32_t* w_up, const void* s_up,
                               const void* b_up, int64_t M, int64_t N,
                               int64_t K, int group_size, int bits,
                               int x_dtype, int s_dtype, void* stream);

/*
 * Fused gate/up gather_qmm and SwiGLU of the MoE experts on the sorted path:
 *   h[i] = swiglu(x[xi] . deq(Wg[wi])^T, x[xi] . deq(Wu[wi])^T)
 * with xi, wi as in hq_gather_qmm.
 *
 * Replaces the gate_out / up_out gather_qmm pair and swiglu of
 * SwitchMlpWeights::forward_gather_global_sort (crates/higgs-models/src/
 * qwen3_next.rs:1764-1787). With lhs_indices = token_idx of hq_moe_sort the
 * x_sorted gather (qwen3_next.rs:1754-1757) is fused too.
 *
 *   x: [x_batch, M, K]; w_gate, w_up: [w_batch, N, K*bits/32];
 *   s_*, b_*: [w_batch, N, K/group_size]; h: [batch, M, N] of x_dtype.
 *
 * rhs_indices must be non-decreasing (sorted_indices semantics of
 * hq_gather_qmm). Supported: x_dtype == s_dtype in {float16, bfloat16}, K a
 * multiple of 64, w_batch < 65535; otherwise HQ_ERR_UNSUPPORTED. Rows with
 * out-of-range indices are NaN. Rounding as hq_quantized_matmul_swiglu.
 */
int hq_gather_qmm_swiglu(void* h, const void* x, const uint32_t* w_gate,
                         const void* s_gate, const void* b_gate,
                         const uint32_t* w_up, const void* s_up,
                         const void* b_up, const uint32_t* lhs_indices,
                         const uint32_t* rhs_indices, int64_t batch,
                         int64_t x_batch, int64_t w_batch, int64_t M,
                         int64_t N, int64_t K, int group_size, int bits,
                         int x_dtype, int s_dtype, void* stream);

/*
 * Elementwise out[i] = round(gate[i] * sigmoid(gate[i]) * up[i]), i < n,
 * evaluated in float32 (gate, up, out of `dtype`).
 *
 * Replaces higgs' swiglu / silu_mul (crates/higgs-models/src/qwen3_next.rs:
 * 340-342, 437-452) for the unfused paths.
 */
int hq_swiglu(void* out, const void* gate, const void* up, int64_t n,
              int dtype, void* stream);

/*
 * Global expert sort of the MoE global-sort path.
 *
 * Replaces the index work of SwitchMlpWeights::forward_gather_global_sort
 * (crates/higgs-models/src/qwen3_next.rs:1746-1761): with idx the flattened
 * [tokens, top_k] expert indices (n = tokens * top_k),
 *   order      = argsort(idx)   (stable: equal indices keep their order)
 *   inv_order  = argsort(order) (inv_order[order[p]] = p)
 *   idx_sorted = idx[order]     (non-decreasing)
 *   token_idx  = order / top_k
 * Any output may be NULL. Indices >= num_experts are placed after every
 * valid one, in their original order (their gather_qmm rows are NaN).
 * One workgroup does the sort; num_experts <= 2048, n < 2^31.
 */
int hq_moe_sort(uint32_t* order, uint32_t* inv_order, uint32_t* idx_sorted,
                uint32_t* token_idx, const uint32_t* idx, int64_t n,
                int64_t top_k, int64_t num_experts, void* stream);

/*
 * Unsort and score-weighted combine of the experts' outputs:
 *   out[t, d] = sum_{j < top_k} round(scores[t, j] * y[inv_order[t*top_k + j], d])
 * (summed in float32 in j order, rounded once to `dtype`).
 *
 * Replaces out_flat.take_axis(inv_order) and the reshape of
 * forward_gather_global_sort (crates/higgs-models/src/qwen3_next.rs:
 * 1802-1808) and the y * scores, sum over top_k of the MoE block
 * (crates/higgs-models/src/qwen3_moe.rs:355-357).
 *
 *   y: [tokens*top_k, D] of dtype (rows in sorted order); inv_order: uint32
 *   [tokens*top_k]; scores: [tokens, top_k] of score_dtype; out: [tokens, D].
 * A row whose inv_order is out of range makes its token's output NaN.
 */
int hq_moe_combine(void* out, const void* y, const uint32_t* inv_order,
                   const void* scores, int64_t tokens, int64_t top_k,
                   int64_t D, int dtype, int score_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* HIGGS_QMM_H */
