// hq_qmv.hip -- quantized GEMV for decode (M <= 8 rows of x), one bit width
// (HQ_BITS), every dtype combination.
//
// y[m, n] = sum_k x[m, k] * (s[n, g] * q[n, k] + b[n, g]),  g = k / group_size
// (mlx-rs ops::quantized_matmul with transpose=true, as called from
// crates/higgs-models/src/qwen3_next.rs:218-227; the in-tree statement of the
// nibble order and group math is qwen3_next.rs:969-988).
//
// Generic VALU form: a wave owns ROWS weight rows; lanes stride over 32-element
// packs of K (one 128-bit load per pack for 4-bit), each pack is reduced per
// 8-element chunk as s*(q.x) + b*sum(x), accumulated in fp32, and the wave
// reduces at the end. Batched/gathered calls (gather_qmm) index x and W per
// batch element through blockIdx.y.
#include "hq_common.hpp"
#include "hq_kernels.hpp"

#ifndef HQ_BITS
#error "compile with -DHQ_BITS=<2|3|4|5|6|8>"
#endif

namespace hq {

struct QKern {
  void* y;
  const void* x;
  const uint32_t* w;
  const void* s;
  const void* b;
  const uint32_t* lhs;
  const uint32_t* rhs;
  int64_t batch, x_rep, x_batch, w_batch;
  int M, N, K;
  int gshift;
  const void* lb;  // linear bias [N] or null
};

static QKern to_kern(const QArgs& a) {
  QKern k;
  k.y = a.y; k.x = a.x; k.w = a.w; k.s = a.s; k.b = a.b;
  k.lhs = a.lhs; k.rhs = a.rhs;
  k.batch = a.batch; k.x_rep = a.x_rep; k.x_batch = a.x_batch; k.w_batch = a.w_batch;
  k.M = (int)a.M; k.N = (int)a.N; k.K = (int)a.K;
  k.gshift = __builtin_ctz((unsigned)a.group_size);
  k.lb = a.lb;
  return k;
}

template <int ODT>
__device__ __forceinline__ st_t<ODT> nan_of() {
  if constexpr (ODT == DT_F32) return __uint_as_float(0x7fc00000u);
  else if constexpr (ODT == DT_BF16) return (uint16_t)0x7fc0u;
  else return (uint16_t)0x7e00u;
}

// ---------------------------------------------------------------------------
// transpose = true
// ---------------------------------------------------------------------------

template <int BITS, int XDT, int SDT, int MB, int ROWS>
__global__ __launch_bounds__(256) void qmv_t_kernel(QKern a) {
  using XS = st_t<XDT>;
  using SS = st_t<SDT>;
  constexpr int ODT = result_dtype(XDT, SDT);
  using OS = st_t<ODT>;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int n0 = (blockIdx.x * 4 + wv) * ROWS;
  if (n0 >= a.N) return;
  const int M = a.M, N = a.N, K = a.K;
  const int64_t P = (int64_t)(K >> 5) * BITS;
  const int64_t G = K >> a.gshift;
  const int packs = K >> 5;
  const int gsp = a.gshift - 5;

  for (int64_t i = blockIdx.y; i < a.batch; i += gridDim.y) {
    const int64_t xi = a.lhs ? (int64_t)a.lhs[i] : i / a.x_rep;
    const int64_t wi = a.rhs ? (int64_t)a.rhs[i] : 0;
    OS* yi = (OS*)a.y + i * (int64_t)M * N;
    if (xi >= a.x_batch || wi >= a.w_batch) {
      if (lane < ROWS * MB) {
        const int r = lane / MB, m = lane % MB;
        if (n0 + r < N && m < M) yi[(int64_t)m * N + n0 + r] = nan_of<ODT>();
      }
      continue;
    }
    const XS* xb = (const XS*)a.x + xi * (int64_t)M * K;
    const uint32_t* wb = a.w + wi * (int64_t)N * P;
    const SS* sb = (const SS*)a.s + wi * (int64_t)N * G;
    const SS* bb = (const SS*)a.b + wi * (int64_t)N * G;

    float acc[ROWS][MB];
#pragma unroll
    for (int r = 0; r < ROWS; r++)
#pragma unroll
      for (int m = 0; m < MB; m++) acc[r][m] = 0.f;

    for (int p = lane; p < packs; p += 64) {
      const int g = p >> gsp;
      uint32_t wd[ROWS][BITS];
      float sc[ROWS], bi[ROWS];
#pragma unroll
      for (int r = 0; r < ROWS; r++) {
        const int64_t n = min(n0 + r, N - 1);
        load_pack<BITS>(wb + n * P + (int64_t)p * BITS, wd[r]);
        sc[r] = DT_<SDT>::load(sb, n * G + g);
        bi[r] = DT_<SDT>::load(bb, n * G + g);
      }
#pragma unroll
      for (int c = 0; c < 4; c++) {
        float xv[MB][8], xs[MB];
#pragma unroll
        for (int m = 0; m < MB; m++) {
          if (m < M) {
            load8_f32<XDT>(xb + (int64_t)m * K + p * 32 + c * 8, xv[m]);
          } else {
#pragma unroll
            for (int e = 0; e < 8; e++) xv[m][e] = 0.f;
          }
          xs[m] = ((xv[m][0] + xv[m][1]) + (xv[m][2] + xv[m][3])) +
                  ((xv[m][4] + xv[m][5]) + (xv[m][6] + xv[m][7]));
        }
#pragma unroll
        for (int r = 0; r < ROWS; r++) {
          float q[8];
#pragma unroll
          for (int e = 0; e < 8; e++) q[e] = (float)pack_elem<BITS>(wd[r], c * 8 + e);
#pragma unroll
          for (int m = 0; m < MB; m++) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < 8; e++) d = fmaf(q[e], xv[m][e], d);
            acc[r][m] = fmaf(sc[r], d, fmaf(bi[r], xs[m], acc[r][m]));
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < ROWS; r++)
#pragma unroll
      for (int m = 0; m < MB; m++) {
        const float v = wave_sum(acc[r][m]);
        if (lane == 0 && n0 + r < N && m < M) yi[(int64_t)m * N + n0 + r] = linear_out<ODT>(v, a.lb, n0 + r);
      }
  }
}

template <int XDT, int SDT, int MB>
static void run_qmv_t(const QArgs& a) {
  constexpr int ROWS = MB <= 2 ? 4 : 2;
  const int64_t rows_per_block = 4 * ROWS;
  dim3 grid((unsigned)((a.N + rows_per_block - 1) / rows_per_block),
            (unsigned)(a.batch < 65535 ? a.batch : 65535));
  qmv_t_kernel<HQ_BITS, XDT, SDT, MB, ROWS><<<grid, 256, 0, a.stream>>>(to_kern(a));
}

template <int XDT, int SDT>
static void run_qmv_t_m(const QArgs& a) {
  if (a.M <= 1) run_qmv_t<XDT, SDT, 1>(a);
  else if (a.M <= 2) run_qmv_t<XDT, SDT, 2>(a);
  else if (a.M <= 4) run_qmv_t<XDT, SDT, 4>(a);
  else run_qmv_t<XDT, SDT, 8>(a);
}

// ---------------------------------------------------------------------------
// transpose = false: y[m, n] = sum_k x[m, k] * deq(W)[k, n], W stored [K, N]
// with packs and groups along N. One thread per (m, 32-column pack).
// ---------------------------------------------------------------------------

template <int BITS, int XDT, int SDT>
__global__ __launch_bounds__(256) void qmv_n_kernel(QKern a) {
  using XS = st_t<XDT>;
  using SS = st_t<SDT>;
  constexpr int ODT = result_dtype(XDT, SDT);
  using OS = st_t<ODT>;
  const int M = a.M, N = a.N, K = a.K;
  const int packs = N >> 5;
  const int64_t P = (int64_t)packs * BITS;  // words per W row (row = one k)
  const int64_t G = N >> a.gshift;
  const int gsp = a.gshift - 5;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)packs * M) return;
  const int p = (int)(t % packs);
  const int m = (int)(t / packs);
  for (int64_t i = blockIdx.y; i < a.batch; i += gridDim.y) {
    const int64_t xi = a.lhs ? (int64_t)a.lhs[i] : i / a.x_rep;
    const int64_t wi = a.rhs ? (int64_t)a.rhs[i] : 0;
    OS* yo = (OS*)a.y + i * (int64_t)M * N + (int64_t)m * N + p * 32;
    if (xi >= a.x_batch || wi >= a.w_batch) {
      for (int e = 0; e < 32; e++) yo[e] = nan_of<ODT>();
      continue;
    }
    const XS* xr = (const XS*)a.x + xi * (int64_t)M * K + (int64_t)m * K;
    const uint32_t* wb = a.w + wi * (int64_t)K * P + (int64_t)p * BITS;
    const SS* sb = (const SS*)a.s + wi * (int64_t)K * G + (p >> gsp);
    const SS* bb = (const SS*)a.b + wi * (int64_t)K * G + (p >> gsp);
    float acc[32];
#pragma unroll
    for (int e = 0; e < 32; e++) acc[e] = 0.f;
    for (int k = 0; k < K; k++) {
      uint32_t wd[BITS];
      load_pack<BITS>(wb + (int64_t)k * P, wd);
      const float xv = DT_<XDT>::load(xr, k);
      const float sx = DT_<SDT>::load(sb, (int64_t)k * G) * xv;
      const float bx = DT_<SDT>::load(bb, (int64_t)k * G) * xv;
#pragma unroll
      for (int e = 0; e < 32; e++) acc[e] = fmaf((float)pack_elem<BITS>(wd, e), sx, acc[e] + bx);
    }
#pragma unroll
    for (int e = 0; e < 32; e++) yo[e] = DT_<ODT>::from_f32(acc[e]);
  }
}

template <int XDT, int SDT>
static void run_qmv_n(const QArgs& a) {
  const int64_t threads = (a.N / 32) * a.M;
  dim3 grid((unsigned)((threads + 255) / 256), (unsigned)(a.batch < 65535 ? a.batch : 65535));
  qmv_n_kernel<HQ_BITS, XDT, SDT><<<grid, 256, 0, a.stream>>>(to_kern(a));
}

// ---------------------------------------------------------------------------
// dtype dispatch
// ---------------------------------------------------------------------------

#define HQ_CAT_(a, b) a##b
#define HQ_CAT(a, b) HQ_CAT_(a, b)

#define HQ_DISPATCH_DT(FN, a)                                     \
  switch ((a).xdt * 3 + (a).sdt) {                                \
    case DT_F32 * 3 + DT_F32: FN<DT_F32, DT_F32>(a); break;       \
    case DT_F32 * 3 + DT_F16: FN<DT_F32, DT_F16>(a); break;       \
    case DT_F32 * 3 + DT_BF16: FN<DT_F32, DT_BF16>(a); break;     \
    case DT_F16 * 3 + DT_F32: FN<DT_F16, DT_F32>(a); break;       \
    case DT_F16 * 3 + DT_F16: FN<DT_F16, DT_F16>(a); break;       \
    case DT_F16 * 3 + DT_BF16: FN<DT_F16, DT_BF16>(a); break;     \
    case DT_BF16 * 3 + DT_F32: FN<DT_BF16, DT_F32>(a); break;     \
    case DT_BF16 * 3 + DT_F16: FN<DT_BF16, DT_F16>(a); break;     \
    default: FN<DT_BF16, DT_BF16>(a); break;                      \
  }

hipError_t HQ_CAT(launch_qmv_t_b, HQ_BITS)(const QArgs& a) {
  HQ_DISPATCH_DT(run_qmv_t_m, a);
  return hipGetLastError();
}

hipError_t HQ_CAT(launch_qmv_n_b, HQ_BITS)(const QArgs& a) {
  HQ_DISPATCH_DT(run_qmv_n, a);
  return hipGetLastError();
}

}  // namespace hq
