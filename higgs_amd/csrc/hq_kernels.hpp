// hq_kernels.hpp -- host-side launch interface between the C ABI
// (hq_capi.hip) and the kernel objects. Each kernel source is compiled once
// per bit width with -DHQ_BITS=<b>, so every object defines the launchers for
// one BITS value; hq_capi.hip switches on bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hq {

// One batched quantized product: for i in [0, batch)
//   y[i] (M x N) = x[xi] (M x K) . deq(W[wi])^T
// with xi = lhs ? lhs[i] : i / x_rep and wi = rhs ? rhs[i] : 0.
// Plain quantized_matmul is batch = 1 with no indices.
struct QArgs {
  void* y;
  const void* x;
  const uint32_t* w;
  const void* s;
  const void* b;
  const uint32_t* lhs;  // may be null
  const uint32_t* rhs;  // may be null (then every batch element uses W[0])
  int64_t batch;        // >= 1
  int64_t x_rep;        // batch / x_batch when lhs is null
  int64_t x_batch;      // bound for xi
  int64_t w_batch;      // bound for wi
  int64_t M, N, K;      // logical sizes of one product
  int group_size;
  int xdt, sdt;         // hq dtype codes
  int sorted;           // rhs is non-decreasing
  // SwiGLU fusion: when w2 is set, (w, s, b) is the gate projection and
  // (w2, s2, b2) the up projection, both N x K, and y = swiglu(x.Wg^T, x.Wu^T)
  // (N columns). Null for a plain product.
  const uint32_t* w2;
  const void* s2;
  const void* b2;
  // Bias of a quantized linear layer ([N] of the output dtype), added after
  // the product is rounded (linear_out); null for none. One product only
  // (batch == 1), never with the SwiGLU fusion.
  const void* lb;
  hipStream_t stream;
};

struct DeqArgs {
  void* out;
  const uint32_t* w;
  const void* s;
  const void* b;
  const uint32_t* rows_idx;  // may be null (identity)
  int64_t n_rows;            // rows produced
  int64_t src_rows;          // rows available in w (bound for rows_idx)
  int64_t K;
  int group_size;
  int sdt;
  hipStream_t stream;
};

// Affine group quantization (hq_quant.hip): w [rows, K] of dt -> wq u32
// [rows, K*bits/32], scales and biases [rows, K/group_size] of dt.
struct QuantArgs {
  uint32_t* wq;
  void* s;
  void* b;
  const void* w;
  int64_t rows, K;
  int group_size, bits, dt;
  hipStream_t stream;
};
hipError_t launch_quantize(const QuantArgs& a);

#define HQ_DECLARE_LAUNCHERS(B)                          \
  hipError_t launch_dequant_b##B(const DeqArgs& a);      \
  hipError_t launch_qmv_t_b##B(const QArgs& a);          \
  hipError_t launch_qmvx_t_b##B(const QArgs& a);         \
  hipError_t launch_gqmm_t_b##B(const QArgs& a);         \
  hipError_t launch_gqms_t_b##B(const QArgs& a);         \
  hipError_t launch_gqms_dense_t_b##B(const QArgs& a);   \
  hipError_t launch_qmm_t_b##B(const QArgs& a);          \
  hipError_t launch_qmv_n_b##B(const QArgs& a);

HQ_DECLARE_LAUNCHERS(2)
HQ_DECLARE_LAUNCHERS(3)
HQ_DECLARE_LAUNCHERS(4)
HQ_DECLARE_LAUNCHERS(5)
HQ_DECLARE_LAUNCHERS(6)
HQ_DECLARE_LAUNCHERS(8)

// Largest M handled by the GEMV kernels; larger M goes to the MFMA GEMM.
constexpr int kQmvMaxM = 8;
// Largest M of the GEMM path (grid.y = ceil(M / 128) <= 65535).
constexpr int64_t kQmmMaxM = (int64_t)65535 * 128;

}  // namespace hq
