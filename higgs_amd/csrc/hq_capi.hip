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

int hq_quantized_matmul(void* y, const void* x, const uint32_t* w, const void* scales,
                        const void* biases, int64_t M, int64_t N, int64_t K, int transpose,
                        int group_size, int bits, int x_dtype, int s_dtype, void* stream) {
  const char* tag = "quantized_matmul";
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
  a.stream = (hipStream_t)stream;
  return run_q(tag, bits, a, transpose);
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
  if ((n * (K / 32)) >= ((int64_t)1 << 31))
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

}  // extern "C"
