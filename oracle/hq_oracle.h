/*
 * hq_oracle.h -- CPU oracle for the MLX affine group-quantized linear path.
 *
 * TEST INFRASTRUCTURE ONLY. This is the checker, never the product: only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it. The shipped path (higgs_amd/libhiggs_qmm.so) never links or calls it.
 *
 * What it restates (reference = dusterbloom/higgs; the arithmetic itself lives
 * in MLX, pinned at mlx-rs rev af21d79 / MLX-C 0.4.0, Cargo.toml:94-95,
 * Cargo.lock:1932-1961, which is not present offline):
 *   - packing:      element i of a row sits at bit i*bits of the row's
 *                   little-endian u32 bitstream, LSB first
 *                   (crates/higgs-models/src/qwen3_next.rs:969-988 states it
 *                   for 4 bits; 3/5/6 bits straddle word boundaries).
 *   - dequantize:   out = s*q + b per group of group_size along the packed
 *                   axis, in the scales' dtype (qwen3_next.rs:308-318 calls
 *                   ops::dequantize). Default rounding convention: two
 *                   roundings, round(round(q*s) + b), i.e. MLX's op-by-op
 *                   CPU fallback (multiply, then add). fused=1 gives the
 *                   single-rounding alternative.
 *   - quantized_matmul: y = x . deq(W)^T for transpose=1
 *                   (qwen3_next.rs:218-227, always transpose=true in higgs),
 *                   y = x . deq(W) for transpose=0.
 *   - gather_qmm:   y[i] = x[lhs[i]] . deq(W[rhs[i]])^T
 *                   (qwen3_next.rs:509-578; lhs null sentinel = broadcast).
 *   - quantize:     MLX's affine quantize (ops::quantize, used at
 *                   qwen3_next.rs:4305-4307, 12942; nn::quantize at
 *                   transformer.rs:954-965), op by op in the weights' dtype.
 *   - gather sort:  order = stable argsort(idx), inv = argsort(order),
 *                   token = order / top_k (qwen3_next.rs:1748-1761,
 *                   benchmarks/bench_moe_sort.py:77-84).
 *
 * Dtype codes match include/higgs_qmm.h: 0 = float32, 1 = float16,
 * 2 = bfloat16.
 */
#ifndef HQ_ORACLE_H
#define HQ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HQO_F32 0
#define HQO_F16 1
#define HQO_BF16 2

/* Scalar conversions, round-to-nearest-even; NaN becomes the canonical quiet
 * NaN (0x7FC0 for bf16, 0x7E00 for fp16, sign kept for fp16). */
uint16_t hqo_f32_to_bf16(float f);
float hqo_bf16_to_f32(uint16_t h);
uint16_t hqo_f32_to_f16(float f);
float hqo_f16_to_f32(uint16_t h);
/* Round a double once to the given dtype, returned as float. */
float hqo_round_f64(double v, int dtype);

/* Elementwise array conversions (n elements). */
void hqo_to_f32(const void* src, int dtype, int64_t n, float* dst);
void hqo_from_f32(const float* src, int64_t n, int dtype, void* dst);

/* Bit packing of `rows` rows of `cols` unsigned values, bits in
 * {2,3,4,5,6,8}; cols*bits must be a multiple of 32. */
void hqo_pack(const uint32_t* q, int64_t rows, int64_t cols, int bits, uint32_t* w);
void hqo_unpack(const uint32_t* w, int64_t rows, int64_t cols, int bits, uint32_t* q);

/* dequantize: w [rows, K*bits/32], scales/biases [rows, K/group_size] of
 * `dtype`; out [rows, K] of `dtype`. Returns 0, or -1 on bad arguments. */
int hqo_dequantize(const uint32_t* w, const void* scales, const void* biases,
                   int64_t rows, int64_t K, int group_size, int bits, int dtype,
                   int fused, void* out);

/* Exact reference: fp64 accumulation of x . deq(W) with the dequantized
 * weights taken exactly (s*q+b in double). y is [M, N] double. */
int hqo_qmm_f64(const void* x, int x_dtype, const uint32_t* w,
                const void* scales, const void* biases, int s_dtype,
                int64_t M, int64_t N, int64_t K, int transpose, int group_size,
                int bits, double* y);

/* MLX-CPU-style restatement used as the timed CPU baseline (transpose=1):
 * x, scales and biases are first converted to the common result dtype T;
 * bits in {2,4,8}: weights dequantized in float (w*s, then +b), accumulated in
 * 8 float lanes, lanes summed, rounded once to T; bits in {3,5,6}: scalar loop
 * accumulating in T with every operation rounded to T. y is [M, N] of T.
 * Threads: number of OpenMP threads (<=0 keeps the current setting). */
int hqo_qmm_mlx(const void* x, int x_dtype, const uint32_t* w,
                const void* scales, const void* biases, int s_dtype,
                int64_t M, int64_t N, int64_t K, int group_size, int bits,
                int threads, void* y);

/* gather_qmm reference (fp64). For i in [0, batch):
 *   xi = lhs ? lhs[i] : i / (batch / x_batch),  wi = rhs[i]
 *   y[i] (M x N) = x[xi] (M x K) . deq(W[wi])^T      (transpose=1)
 * Rows whose xi >= x_batch or wi >= w_batch are filled with NaN. */
int hqo_gather_qmm_f64(const void* x, int x_dtype, const uint32_t* w,
                       const void* scales, const void* biases, int s_dtype,
                       const uint32_t* lhs, const uint32_t* rhs, int64_t batch,
                       int64_t x_batch, int64_t w_batch, int64_t M, int64_t N,
                       int64_t K, int transpose, int group_size, int bits,
                       double* y);

/* Global expert sort. idx has n = tokens*top_k entries. Outputs (any may be
 * NULL): order (stable argsort of idx), inv_order (argsort of order),
 * idx_sorted = idx[order], token_idx = order / top_k. */
void hqo_gather_sort(const uint32_t* idx, int64_t n, int64_t top_k,
                     uint32_t* order, uint32_t* inv_order, uint32_t* idx_sorted,
                     uint32_t* token_idx);

/* SwiGLU as higgs computes it: silu(gate) * up = gate * sigmoid(gate) * up,
 * in double, rounded once to `dtype` (qwen3_next.rs:340-346). */
void hqo_swiglu(const void* gate, const void* up, int dtype, int64_t n, void* out);

/* MoE unsort + score-weighted combine (qwen3_next.rs:1802-1808,
 * qwen3_moe.rs:355-357). y: [tokens*top_k, D] of dtype in sorted order;
 * out: [tokens, D] of dtype. */
void hqo_moe_combine(const void* y, int dtype, const uint32_t* inv, const void* scores,
                     int sdtype, int64_t tokens, int64_t top_k, int64_t D, void* out);

/* MLX affine quantize, op by op in dtype (each operation's result rounded to
 * dtype): w [rows, K] of dtype -> wq u32 [rows, K*bits/32] (LSB-first),
 * scales/biases [rows, K/group_size] of dtype. Per group: the min/max edge of
 * larger magnitude becomes the bias and an exact multiple of the scale, so 0
 * is representable (see hq_oracle.c). NaN inputs are outside the contract.
 * Returns 0, or -1 on bad arguments. */
int hqo_quantize(const void* w, int dtype, int64_t rows, int64_t K, int group_size, int bits,
                 uint32_t* wq, void* scales, void* biases);

int hqo_num_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* HQ_ORACLE_H */
