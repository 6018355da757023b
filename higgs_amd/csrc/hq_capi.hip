// hq_capi.hip -- the extern "C" boundary (include/higgs_qmm.h): argument
// validation with MLX-style messages, the thread-local last error, and
// dispatch to the per-bit-width kernel launchers.
//
// Validation follows MLX's quantized_matmul / gather_qmm / dequantize checks
// as they surface through higgs' error path (crates/higgs-models/src/
// qwen3_next.rs:552-576 wraps the message with a shape dump): unsupported
// bits or group size, K not a multiple of the group size, non-float dtypes.
// Shape checks that need full MLX shapes (w.shape[-1]*32/bits vs
// scales.shape[-1]*group_size) live in the host facades, which own shapes.
#include <cstdarg>
#include <cstdio>
#include <string>

#include "../../include/higgs_qmm.h"
#include "hq_kernels.hpp"
#include "hq_moe.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

bool bits_ok(int b) { return b == 2 || b == 3 || b == 4 || b == 5 || b == 6 || b == 8; }
bool group_ok(int g) { return g == 32 || g == 64 || g == 128; }
bool dtype_ok(int d) { return d == HQ_DTYPE_FLOAT32 || d == HQ_DTYPE_FLOAT16 || d == HQ_DTYPE_BFLOAT16; }
bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_common(const char* tag, int group_size, int bits, int xdt, int sdt) {
  if (!bits_ok(bits))
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] The requested number of bits %d is not supported. The supported bits are 2, "
                "3, 4, 5, 6 and 8.",
                tag, bits);
  if (!group_ok(group_size))
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] The requested group size %d is not supported. The supported group sizes are "
                "32, 64, and 128.",
                tag, group_size);
  if (xdt >= 0 && !dtype_ok(xdt))
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] Only real floating types are supported but x has dtype code %d.", tag, xdt);
  if (!dtype_ok(sdt))
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] Only real floating types are supported but scales have dtype code %d.", tag,
                sdt);
  return HQ_OK;
}

constexpr int64_t kMaxDim = (int64_t)1 << 30;

hipError_t dispatch_q(int bits, const hq::QArgs& a, int which) {
#define HQ_Q_CASE(B)                                   \
  case B:                                              \
    if (which == 0) return hq::launch_qmv_t_b##B(a);   \
    if (which == 1) return hq::launch_qmm_t_b##B(a);   \
    if (which == 3) return hq::launch_qmvx_t_b##B(a);  \
    if (which == 4) return hq::launch_gqmm_t_b##B(a);  \
    if (which == 5) return hq::launch_gqms_dense_t_b##B(a); \
    return hq::launch_qmv_n_b##B(a);
  switch (bits) {
    HQ_Q_CASE(2)
    HQ_Q_CASE(3)
    HQ_Q_CASE(4)
    HQ_Q_CASE(5)
    HQ_Q_CASE(6)
    HQ_Q_CASE(8)
  }
#undef HQ_Q_CASE
  return hipErrorInvalidValue;
}

hipError_t dispatch_deq(int bits, const hq::DeqArgs& a) {
  switch (bits) {
    case 2: return hq::launch_dequant_b2(a);
    case 3: return hq::launch_dequant_b3(a);
    case 4: return hq::launch_dequant_b4(a);
    case 5: return hq::launch_dequant_b5(a);
    case 6: return hq::launch_dequant_b6(a);
    case 8: return hq::launch_dequant_b8(a);
  }
  return hipErrorInvalidValue;
}

int run_q(const char* tag, int bits, hq::QArgs& a, int transpose) {
  // 0: VALU GEMV (fp32 x), 3: matrix-core GEMV (16-bit x), 1: GEMM, 2: transpose=false.
  int which = !transpose ? 2 : (a.M <= hq::kQmvMaxM ? 0 : 1);
  if (which == 0 && a.xdt != HQ_DTYPE_FLOAT32) which = 3;
  // Sorted expert indices: the grouped kernel streams each expert's weights
  // once for all of its rows. It declines shapes it does not take.
  if (transpose && a.sorted && a.batch > 1) {
    hipError_t e = dispatch_q(bits, a, 4);
    if (e == hipSuccess) return HQ_OK;
    if (e != hipErrorNotSupported)
      return fail(HQ_ERR_HIP, "[%s] kernel launch failed: %s", tag, hipGetErrorString(e));
    (void)hipGetLastError();
  }
  if (which == 1 && a.M > hq::kQmmMaxM)
    return fail(HQ_ERR_UNSUPPORTED, "[%s] M=%lld exceeds the GEMM grid limit (%lld rows).", tag,
                (long long)a.M, (long long)hq::kQmmMaxM);
  if (which == 2 && (a.N / 32) * a.M > ((int64_t)1 << 31) * 255)
    return fail(HQ_ERR_UNSUPPORTED, "[%s] M*N too large for the transpose=false kernel.", tag);
  hipError_t e = dispatch_q(bits, a, which);
  if (e != hipSuccess)
    return fail(HQ_ERR_HIP, "[%s] kernel launch failed: %s", tag, hipGetErrorString(e));
  return HQ_OK;
}

}  // namespace

extern "C" {

const char* hq_version(void) { return "higgs_qmm 0.1.0 (gfx950)"; }

const char* hq_last_error(void) { return g_last_error.c_str(); }

int hq_result_dtype(int x_dtype, int s_dtype) {
  if (!dtype_ok(x_dtype) || !dtype_ok(s_dtype)) return -1;
  return x_dtype == s_dtype ? x_dtype : HQ_DTYPE_FLOAT32;
}

}  // extern "C"

namespace {

// quantized_matmul with an optional linear-layer bias (lb, [N] of the output
// dtype, transpose != 0 only).
int quantized_matmul_impl(const char* tag, void* y, const void* x, const uint32_t* w,
                          const void* scales, const void* biases, const void* lb, int64_t M,
                          int64_t N, int64_t K, int transpose, int group_size, int bits,
                          int x_dtype, int s_dtype, void* stream) {
  int rc = check_common(tag, group_size, bits, x_dtype, s_dtype);
  if (rc) return rc;
  if (M < 0 || N < 0 || K <= 0 || M > kMaxDim || N > kMaxDim || K > kMaxDim)
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] Invalid sizes M=%lld N=%lld K=%lld.", tag,
                (long long)M, (long long)N, (long long)K);
  const int64_t packed = transpose ? K : N;  // axis carrying packs and groups
  if (packed % group_size)
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] The last dimension of the quantized matrix (%lld) must be divisible by the "
                "group size %d (transpose=%d).",
                tag, (long long)packed, group_size, transpose ? 1 : 0);
  if (M == 0 || N == 0) return HQ_OK;
  if (!y || !x || !w || !scales || !biases)
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] NULL buffer pointer.", tag);
  if (!aligned16(x) || !aligned16(w) || !aligned16(y))
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] x, w and y must be 16-byte aligned.", tag);
  hq::QArgs a{};
  a.y = y; a.x = x; a.w = w; a.s = scales; a.b = biases;
  a.lhs = nullptr; a.rhs = nullptr;
  a.batch = 1; a.x_rep = 1; a.x_batch = 1; a.w_batch = 1;
  a.M = M; a.N = N; a.K = K;
  a.group_size = group_size; a.xdt = x_dtype; a.sdt = s_dtype; a.sorted = 0;
  a.lb = lb;
  a.stream = (hipStream_t)stream;
  return run_q(tag, bits, a, transpose);
}

}  // namespace

extern "C" {

int hq_quantized_matmul(void* y, const void* x, const uint32_t* w, const void* scales,
                        const void* biases, int64_t M, int64_t N, int64_t K, int transpose,
                        int group_size, int bits, int x_dtype, int s_dtype, void* stream) {
  return quantized_matmul_impl("quantized_matmul", y, x, w, scales, biases, nullptr, M, N, K,
                               transpose, group_size, bits, x_dtype, s_dtype, stream);
}

int hq_quantized_linear(void* y, const void* x, const uint32_t* w, const void* scales,
                        const void* biases, const void* bias, int64_t M, int64_t N, int64_t K,
                        int group_size, int bits, int x_dtype, int s_dtype, int bias_dtype,
                        void* stream) {
  const char* tag = "quantized_linear";
  if (bias != nullptr) {
    if (!dtype_ok(bias_dtype))
      return fail(HQ_ERR_INVALID_ARGUMENT,
                  "[%s] Only real floating types are supported but the bias has dtype code %d.",
                  tag, bias_dtype);
    if (dtype_ok(x_dtype) && dtype_ok(s_dtype) &&
        bias_dtype != (x_dtype == s_dtype ? x_dtype : HQ_DTYPE_FLOAT32))
      return fail(HQ_ERR_UNSUPPORTED,
                  "[%s] The bias dtype (%d) must be the output dtype of the product (%d).", tag,
                  bias_dtype, x_dtype == s_dtype ? x_dtype : HQ_DTYPE_FLOAT32);
  }
  return quantized_matmul_impl(tag, y, x, w, scales, biases, bias, M, N, K, 1, group_size, bits,
                               x_dtype, s_dtype, stream);
}

int hq_gather_qmm(void* y, const void* x, const uint32_t* w, const void* scales,
                  const void* biases, const uint32_t* lhs_indices, const uint32_t* rhs_indices,
                  int64_t batch, int64_t x_batch, int64_t w_batch, int64_t M, int64_t N, int64_t K,
                  int transpose, int group_size, int bits, int sorted_indices, int x_dtype,
                  int s_dtype, void* stream) {
  const char* tag = "gather_qmm";
  int rc = check_common(tag, group_size, bits, x_dtype, s_dtype);
  if (rc) return rc;
  if (batch < 0 || x_batch <= 0 || w_batch <= 0 || M < 0 || N < 0 || K <= 0 || M > kMaxDim ||
      N > kMaxDim || K > kMaxDim || batch > ((int64_t)1 << 40))
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] Invalid sizes batch=%lld x_batch=%lld w_batch=%lld M=%lld N=%lld K=%lld.",
                tag, (long long)batch, (long long)x_batch, (long long)w_batch, (long long)M,
                (long long)N, (long long)K);
  const int64_t packed = transpose ? K : N;
  if (packed % group_size)
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] The last dimension of the quantized matrix (%lld) must be divisible by the "
                "group size %d (transpose=%d).",
                tag, (long long)packed, group_size, transpose ? 1 : 0);
  if (!lhs_indices && batch % x_batch)
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] Without lhs_indices the batch (%lld) must be a multiple of x's batch (%lld).",
                tag, (long long)batch, (long long)x_batch);
  if (batch == 0 || M == 0 || N == 0) return HQ_OK;
  if (!rhs_indices)
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] rhs_indices must not be NULL.", tag);
  if (!y || !x || !w || !scales || !biases)
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] NULL buffer pointer.", tag);
  if (!aligned16(x) || !aligned16(w) || !aligned16(y))
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] x, w and y must be 16-byte aligned.", tag);
  hq::QArgs a{};
  a.y = y; a.x = x; a.w = w; a.s = scales; a.b = biases;
  a.lhs = lhs_indices; a.rhs = rhs_indices;
  a.batch = batch; a.x_rep = lhs_indices ? 1 : batch / x_batch;
  a.x_batch = x_batch; a.w_batch = w_batch;
  a.M = M; a.N = N; a.K = K;
  a.group_size = group_size; a.xdt = x_dtype; a.sdt = s_dtype; a.sorted = sorted_indices ? 1 : 0;
  a.stream = (hipStream_t)stream;
  return run_q(tag, bits, a, transpose);
}

static int deq_common(const char* tag, void* out, const uint32_t* w, const void* scales,
                      const void* biases, const uint32_t* idx, int64_t n, int64_t rows, int64_t K,
                      int group_size, int bits, int s_dtype, void* stream) {
  int rc = check_common(tag, group_size, bits, -1, s_dtype);
  if (rc) return rc;
  if (n < 0 || rows < 0 || K <= 0 || K % group_size)
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] Invalid sizes rows=%lld K=%lld: K must be a positive multiple of the group "
                "size %d.",
                tag, (long long)(idx ? n : rows), (long long)K, group_size);
  if ((n * (K / 32)) >= ((int64_t)1 << 29))  // 4 threads per 32-element pack, 32-bit indices
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] Too many elements (%lld x %lld).", tag,
                (long long)n, (long long)K);
  if (n == 0) return HQ_OK;
  if (!out || !w || !scales || !biases || (idx == nullptr && rows < n))
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] NULL buffer pointer.", tag);
  if (!aligned16(out) || !aligned16(w))
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] out and w must be 16-byte aligned.", tag);
  hq::DeqArgs a{};
  a.out = out; a.w = w; a.s = scales; a.b = biases; a.rows_idx = idx;
  a.n_rows = n; a.src_rows = rows; a.K = K; a.group_size = group_size; a.sdt = s_dtype;
  a.stream = (hipStream_t)stream;
  hipError_t e = dispatch_deq(bits, a);
  if (e != hipSuccess)
    return fail(HQ_ERR_HIP, "[%s] kernel launch failed: %s", tag, hipGetErrorString(e));
  return HQ_OK;
}

int hq_dequantize(void* out, const uint32_t* w, const void* scales, const void* biases,
                  int64_t rows, int64_t K, int group_size, int bits, int s_dtype, void* stream) {
  return deq_common("dequantize", out, w, scales, biases, nullptr, rows, rows, K, group_size, bits,
                    s_dtype, stream);
}

int hq_embedding_dequantize(void* out, const uint32_t* w, const void* scales, const void* biases,
                            const uint32_t* indices, int64_t n, int64_t rows, int64_t K,
                            int group_size, int bits, int s_dtype, void* stream) {
  if (n > 0 && !indices)
    return fail(HQ_ERR_INVALID_ARGUMENT, "[embedding_dequantize] indices must not be NULL.");
  return deq_common("embedding_dequantize", out, w, scales, biases, indices, n, rows, K, group_size,
                    bits, s_dtype, stream);
}

int hq_quantized_matmul_swiglu(void* h, const void* x, const uint32_t* w_gate,
                               const void* s_gate, const void* b_gate, const uint32_t* w_up,
                               const void* s_up, const void* b_up, int64_t M, int64_t N, int64_t K,
                               int group_size, int bits, int x_dtype, int s_dtype, void* stream) {
  const char* tag = "quantized_matmul_swiglu";
  int rc = check_common(tag, group_size, bits, x_dtype, s_dtype);
  if (rc) return rc;
  if (M < 0 || N < 0 || K <= 0 || M > kMaxDim || N > kMaxDim || K > kMaxDim)
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] Invalid sizes M=%lld N=%lld K=%lld.", tag,
                (long long)M, (long long)N, (long long)K);
  if (K % group_size)
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] The last dimension of the quantized matrix (%lld) must be divisible by the "
                "group size %d (transpose=1).",
                tag, (long long)K, group_size);
  if (M == 0 || N == 0) return HQ_OK;
  if (!h || !x || !w_gate || !s_gate || !b_gate || !w_up || !s_up || !b_up)
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] NULL buffer pointer.", tag);
  if (!aligned16(x) || !aligned16(w_gate) || !aligned16(w_up) || !aligned16(h))
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] x, w_gate, w_up and h must be 16-byte aligned.",
                tag);
  if (x_dtype != s_dtype || x_dtype == HQ_DTYPE_FLOAT32)
    return fail(HQ_ERR_UNSUPPORTED,
                "[%s] The fused kernel takes x and scales of one 16-bit dtype (got %d, %d).", tag,
                x_dtype, s_dtype);
  // 8-row GEMV chunks read the weights once per chunk; from 12 rows the
  // GEMM (weights once) is faster (14336 x 4096, gate and up: M = 9 45.9 vs
  // 53.6 us, M = 12 55.1 vs 53.4, M = 32 124.9 vs 54.8, M = 127 497 vs 57.6)
  const bool gemm = M >= 12;
  if (gemm ? (K % 64 != 0) : (K % 1024 != 0))
    return fail(HQ_ERR_UNSUPPORTED,
                "[%s] K=%lld: the fused kernel needs K %% %d == 0 at M=%lld.", tag, (long long)K,
                gemm ? 64 : 1024, (long long)M);
  hq::QArgs a{};
  a.y = h; a.x = x; a.w = w_gate; a.s = s_gate; a.b = b_gate;
  a.w2 = w_up; a.s2 = s_up; a.b2 = b_up;
  a.lhs = nullptr; a.rhs = nullptr;
  a.batch = 1; a.x_rep = 1; a.x_batch = 1; a.w_batch = 1;
  a.N = N; a.K = K;
  a.group_size = group_size; a.xdt = x_dtype; a.sdt = s_dtype; a.sorted = 0;
  a.stream = (hipStream_t)stream;
  hipError_t e = hipSuccess;
  bool dense = false;
  if (!gemm && M > hq::kQmvMaxM) {
    // 9-11 rows: the streaming kernel's dense form where it takes the shape
    // (4-bit, N >= 8192, K 2048 or 4096; the GEMM tries it first from 12
    // rows, the GEMV launcher at 8)
    a.M = M;
    e = dispatch_q(bits, a, 5);
    dense = e != hipErrorNotSupported;
    if (!dense) {
      (void)hipGetLastError();
      e = hipSuccess;
    }
  }
  if (dense) {
  } else if (gemm) {
    a.M = M;
    e = dispatch_q(bits, a, 1);
  } else {
    // GEMV kernel, up to kQmvMaxM rows of x per launch
    const size_t xb = x_dtype == HQ_DTYPE_FLOAT32 ? 4 : 2;
    for (int64_t m0 = 0; m0 < M && e == hipSuccess; m0 += hq::kQmvMaxM) {
      a.M = M - m0 < hq::kQmvMaxM ? M - m0 : hq::kQmvMaxM;
      a.x = static_cast<const char*>(x) + (size_t)(m0 * K) * xb;
      a.y = static_cast<char*>(h) + (size_t)(m0 * N) * xb;
      e = dispatch_q(bits, a, 3);
    }
  }
  if (e == hipErrorNotSupported) {
    (void)hipGetLastError();
    return fail(HQ_ERR_UNSUPPORTED, "[%s] shape M=%lld N=%lld K=%lld not taken by the fused kernel.",
                tag, (long long)M, (long long)N, (long long)K);
  }
  if (e != hipSuccess)
    return fail(HQ_ERR_HIP, "[%s] kernel launch failed: %s", tag, hipGetErrorString(e));
  return HQ_OK;
}

int hq_gather_qmm_swiglu(void* h, const void* x, const uint32_t* w_gate, const void* s_gate,
                         const void* b_gate, const uint32_t* w_up, const void* s_up,
                         const void* b_up, const uint32_t* lhs_indices,
                         const uint32_t* rhs_indices, int64_t batch, int64_t x_batch,
                         int64_t w_batch, int64_t M, int64_t N, int64_t K, int group_size,
                         int bits, int x_dtype, int s_dtype, void* stream) {
  const char* tag = "gather_qmm_swiglu";
  int rc = check_common(tag, group_size, bits, x_dtype, s_dtype);
  if (rc) return rc;
  if (batch < 0 || x_batch <= 0 || w_batch <= 0 || M < 0 || N < 0 || K <= 0 || M > kMaxDim ||
      N > kMaxDim || K > kMaxDim || batch > ((int64_t)1 << 40))
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] Invalid sizes batch=%lld x_batch=%lld w_batch=%lld M=%lld N=%lld K=%lld.",
                tag, (long long)batch, (long long)x_batch, (long long)w_batch, (long long)M,
                (long long)N, (long long)K);
  if (K % group_size)
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] The last dimension of the quantized matrix (%lld) must be divisible by the "
                "group size %d (transpose=1).",
                tag, (long long)K, group_size);
  if (!lhs_indices && batch % x_batch)
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] Without lhs_indices the batch (%lld) must be a multiple of x's batch (%lld).",
                tag, (long long)batch, (long long)x_batch);
  if (batch == 0 || M == 0 || N == 0) return HQ_OK;
  if (!rhs_indices)
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] rhs_indices must not be NULL.", tag);
  if (!h || !x || !w_gate || !s_gate || !b_gate || !w_up || !s_up || !b_up)
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] NULL buffer pointer.", tag);
  if (!aligned16(x) || !aligned16(w_gate) || !aligned16(w_up) || !aligned16(h))
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] x, w_gate, w_up and h must be 16-byte aligned.",
                tag);
  hq::QArgs a{};
  a.y = h; a.x = x; a.w = w_gate; a.s = s_gate; a.b = b_gate;
  a.w2 = w_up; a.s2 = s_up; a.b2 = b_up;
  a.lhs = lhs_indices; a.rhs = rhs_indices;
  a.batch = batch; a.x_rep = lhs_indices ? 1 : batch / x_batch;
  a.x_batch = x_batch; a.w_batch = w_batch;
  a.M = M; a.N = N; a.K = K;
  a.group_size = group_size; a.xdt = x_dtype; a.sdt = s_dtype; a.sorted = 1;
  a.stream = (hipStream_t)stream;
  hipError_t e = dispatch_q(bits, a, 4);
  if (e == hipErrorNotSupported) {
    (void)hipGetLastError();
    return fail(HQ_ERR_UNSUPPORTED,
                "[%s] the fused grouped kernel needs x and scales of one 16-bit dtype, K %% 64 "
                "== 0 and w_batch < 65535 (got dtypes %d, %d, K=%lld, w_batch=%lld).",
                tag, x_dtype, s_dtype, (long long)K, (long long)w_batch);
  }
  if (e != hipSuccess)
    return fail(HQ_ERR_HIP, "[%s] kernel launch failed: %s", tag, hipGetErrorString(e));
  return HQ_OK;
}

int hq_quantize(uint32_t* wq, void* scales, void* biases, const void* w, int64_t rows, int64_t K,
                int group_size, int bits, int dtype, void* stream) {
  const char* tag = "quantize";
  int rc = check_common(tag, group_size, bits, -1, dtype);
  if (rc) return rc;
  if (rows < 0 || K <= 0 || K % group_size || rows > kMaxDim || K > kMaxDim ||
      rows * K >= ((int64_t)1 << 40))
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] The last dimension of the matrix (%lld) must be divisible by the group size "
                "%d (rows=%lld).",
                tag, (long long)K, group_size, (long long)rows);
  if (rows == 0) return HQ_OK;
  if (!wq || !scales || !biases || !w)
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] NULL buffer pointer.", tag);
  if (!aligned16(w) || (reinterpret_cast<uintptr_t>(wq) & 3u) ||
      (reinterpret_cast<uintptr_t>(scales) & 1u) || (reinterpret_cast<uintptr_t>(biases) & 1u))
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] w must be 16-byte aligned, wq 4-byte aligned, scales and biases aligned to "
                "their dtype.", tag);
  if (dtype == HQ_DTYPE_FLOAT32 &&
      ((reinterpret_cast<uintptr_t>(scales) & 3u) || (reinterpret_cast<uintptr_t>(biases) & 3u)))
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] float32 scales and biases must be 4-byte aligned.",
                tag);
  hq::QuantArgs a{};
  a.wq = wq; a.s = scales; a.b = biases; a.w = w;
  a.rows = rows; a.K = K; a.group_size = group_size; a.bits = bits; a.dt = dtype;
  a.stream = (hipStream_t)stream;
  hipError_t e = hq::launch_quantize(a);
  if (e != hipSuccess)
    return fail(HQ_ERR_HIP, "[%s] kernel launch failed: %s", tag, hipGetErrorString(e));
  return HQ_OK;
}

int hq_swiglu(void* out, const void* gate, const void* up, int64_t n, int dtype, void* stream) {
  const char* tag = "swiglu";
  if (!dtype_ok(dtype))
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] Only real floating types are supported but the dtype code is %d.", tag, dtype);
  if (n < 0 || n > ((int64_t)1 << 40))
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] Invalid size n=%lld.", tag, (long long)n);
  if (n == 0) return HQ_OK;
  if (!out || !gate || !up) return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] NULL buffer pointer.", tag);
  hipError_t e = hq::launch_swiglu(gate, up, out, n, dtype, (hipStream_t)stream);
  if (e != hipSuccess)
    return fail(HQ_ERR_HIP, "[%s] kernel launch failed: %s", tag, hipGetErrorString(e));
  return HQ_OK;
}

int hq_moe_sort(uint32_t* order, uint32_t* inv_order, uint32_t* idx_sorted, uint32_t* token_idx,
                const uint32_t* idx, int64_t n, int64_t top_k, int64_t num_experts, void* stream) {
  const char* tag = "moe_sort";
  if (n < 0 || n >= ((int64_t)1 << 31) || top_k <= 0 || num_experts <= 0 ||
      num_experts > hq::kSortMaxExperts)
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] Invalid sizes n=%lld top_k=%lld num_experts=%lld (num_experts <= %lld, "
                "n < 2^31).",
                tag, (long long)n, (long long)top_k, (long long)num_experts,
                (long long)hq::kSortMaxExperts);
  if (n == 0) return HQ_OK;
  if (!idx) return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] idx must not be NULL.", tag);
  hq::SortArgs a{};
  a.idx = idx; a.n = n; a.top_k = top_k; a.E = num_experts;
  a.order = order; a.inv_order = inv_order; a.idx_sorted = idx_sorted; a.token_idx = token_idx;
  a.stream = (hipStream_t)stream;
  hipError_t e = hq::launch_moe_sort(a);
  if (e != hipSuccess)
    return fail(HQ_ERR_HIP, "[%s] kernel launch failed: %s", tag, hipGetErrorString(e));
  return HQ_OK;
}

int hq_moe_combine(void* out, const void* y, const uint32_t* inv_order, const void* scores,
                   int64_t tokens, int64_t top_k, int64_t D, int dtype, int score_dtype,
                   void* stream) {
  const char* tag = "moe_combine";
  if (!dtype_ok(dtype) || !dtype_ok(score_dtype))
    return fail(HQ_ERR_INVALID_ARGUMENT,
                "[%s] Only real floating types are supported but the dtype codes are %d, %d.", tag,
                dtype, score_dtype);
  if (tokens < 0 || top_k <= 0 || D <= 0 || tokens > kMaxDim || top_k > 4096 || D > kMaxDim ||
      tokens * top_k >= ((int64_t)1 << 32))
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] Invalid sizes tokens=%lld top_k=%lld D=%lld.", tag,
                (long long)tokens, (long long)top_k, (long long)D);
  if (tokens == 0) return HQ_OK;
  if (!out || !y || !inv_order || !scores)
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] NULL buffer pointer.", tag);
  if (!aligned16(y) || !aligned16(out))
    return fail(HQ_ERR_INVALID_ARGUMENT, "[%s] y and out must be 16-byte aligned.", tag);
  hq::CombineArgs a{};
  a.out = out; a.y = y; a.inv_order = inv_order; a.scores = scores;
  a.tokens = tokens; a.top_k = top_k; a.D = D; a.dt = dtype; a.sdt = score_dtype;
  a.stream = (hipStream_t)stream;
  hipError_t e = hq::launch_moe_combine(a);
  if (e != hipSuccess)
    return fail(HQ_ERR_HIP, "[%s] kernel launch failed: %s", tag, hipGetErrorString(e));
  return HQ_OK;
}

}  // extern "C"
