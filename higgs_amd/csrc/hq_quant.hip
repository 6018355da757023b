// hq_quant.hip -- affine group quantization (float -> packed u32 + scales +
// biases), every bit width, compiled once.
//
// mlx-rs ops::quantize(w, group_size, bits) as higgs' tests call it
// (crates/higgs-models/src/qwen3_next.rs:4305-4307, 12942) and as
// mlx_rs::nn::quantize applies it to every MaybeQuantized layer of a float
// checkpoint (crates/higgs-models/src/transformer.rs:954-965). Per group of
// group_size consecutive elements, each operation in float rounded to the
// weights' dtype T (MLX's op-by-op form):
//   mx = max(w), mn = min(w), n_bins = 2^bits - 1
//   scale = max((mx - mn) / n_bins, T(1e-7))
//   if |mn| > |mx|: edge = mn            else: edge = mx, scale = -scale
//   q0 = rint(edge / scale)
//   if q0 != 0: scale = edge / q0, bias = edge    else: bias = 0
//   q = clip(rint((w - bias) / scale), 0, n_bins)   (NaN -> 0)
//
// Layout: thread t takes elements [8t, 8t + 8) of the flattened [rows, K]
// input (groups and 32-element packs never straddle rows because K is a
// multiple of both), so its 8 codes are bytes [t*bits, t*bits + bits) of the
// flattened packed output. A group is GS/8 consecutive lanes, which reduce
// min and max with shuffles; the block's packed bytes meet in LDS and leave
// as whole, coalesced 32-bit words. HBM-bound: 2 (or 4) bytes read and
// bits/8 + 4/GS bytes written per element.
#include "hq_common.hpp"
#include "hq_kernels.hpp"

namespace hq {

namespace {

constexpr int kQThreads = 256;

struct QuantKern {
  uint32_t* wq;
  void* s;
  void* b;
  const void* w;
  int64_t n8;  // elements / 8 = threads of work
};

template <int DT, int BITS, int GS>
__global__ __launch_bounds__(kQThreads) void quantize_kernel(QuantKern a) {
  using S = st_t<DT>;
  constexpr int L = GS / 8;  // lanes per group
  __shared__ uint8_t packed[kQThreads * BITS];
  const int64_t t = (int64_t)blockIdx.x * kQThreads + threadIdx.x;
  const bool live = t < a.n8;
  const int64_t tc = live ? t : a.n8 - 1;  // idle lanes of the last block redo the last chunk

  float v[8];
  load8_f32<DT>((const S*)a.w + tc * 8, v);
  float mx = v[0], mn = v[0];
#pragma unroll
  for (int i = 1; i < 8; i++) {
    mx = fmaxf(mx, v[i]);
    mn = fminf(mn, v[i]);
  }
  // lanes of one group are L consecutive, L-aligned lanes of the wave (idle
  // lanes of the last block form whole groups of their own)
#pragma unroll
  for (int o = 1; o < L; o <<= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    mn = fminf(mn, __shfl_xor(mn, o, 64));
  }
  const float n_bins = (float)((1 << BITS) - 1);
  const float eps = DT_<DT>::round(1e-7f);
  float scale = DT_<DT>::round(DT_<DT>::round(mx - mn) / n_bins);
  if (!(scale > eps)) scale = eps;
  const bool side = fabsf(mn) > fabsf(mx);
  if (!side) scale = -scale;
  const float edge = side ? mn : mx;
  const float q0 = rintf(DT_<DT>::round(edge / scale));
  float bias = 0.f;
  if (q0 != 0.f) {
    scale = DT_<DT>::round(edge / q0);
    bias = edge;
  }
  if (live && (t % L) == 0) {
    const int64_t g = t / L;
    ((S*)a.s)[g] = DT_<DT>::from_f32(scale);
    ((S*)a.b)[g] = DT_<DT>::from_f32(bias);
  }
  uint64_t bitsv = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    float q = rintf(DT_<DT>::round(DT_<DT>::round(v[i] - bias) / scale));
    if (!(q >= 0.f)) q = 0.f;
    if (q > n_bins) q = n_bins;
    bitsv |= (uint64_t)(uint32_t)q << (i * BITS);
  }
#pragma unroll
  for (int j = 0; j < BITS; j++) packed[threadIdx.x * BITS + j] = (uint8_t)(bitsv >> (8 * j));
  __syncthreads();
  // active threads of this block are a multiple of 4 (n8 is: K % 32 == 0),
  // so the block's bytes are whole words
  const int64_t first = (int64_t)blockIdx.x * kQThreads;
  const int64_t active = a.n8 - first < kQThreads ? a.n8 - first : kQThreads;
  const int words = (int)(active * BITS / 4);
  uint32_t* out = a.wq + first * BITS / 4;
  for (int i = threadIdx.x; i < words; i += kQThreads)
    out[i] = *reinterpret_cast<const uint32_t*>(packed + 4 * i);
}

template <int DT, int BITS>
hipError_t run_quant_g(const QuantArgs& q, const QuantKern& k) {
  const unsigned grid = (unsigned)((k.n8 + kQThreads - 1) / kQThreads);
  switch (q.group_size) {
    case 32: hipLaunchKernelGGL((quantize_kernel<DT, BITS, 32>), dim3(grid), dim3(kQThreads), 0, q.stream, k); break;
    case 64: hipLaunchKernelGGL((quantize_kernel<DT, BITS, 64>), dim3(grid), dim3(kQThreads), 0, q.stream, k); break;
    default: hipLaunchKernelGGL((quantize_kernel<DT, BITS, 128>), dim3(grid), dim3(kQThreads), 0, q.stream, k); break;
  }
  return hipGetLastError();
}

template <int DT>
hipError_t run_quant_b(const QuantArgs& q, const QuantKern& k) {
  switch (q.bits) {
    case 2: return run_quant_g<DT, 2>(q, k);
    case 3: return run_quant_g<DT, 3>(q, k);
    case 4: return run_quant_g<DT, 4>(q, k);
    case 5: return run_quant_g<DT, 5>(q, k);
    case 6: return run_quant_g<DT, 6>(q, k);
    default: return run_quant_g<DT, 8>(q, k);
  }
}

}  // namespace

hipError_t launch_quantize(const QuantArgs& q) {
  QuantKern k;
  k.wq = q.wq; k.s = q.s; k.b = q.b; k.w = q.w;
  k.n8 = q.rows * q.K / 8;
  switch (q.dt) {
    case DT_F32: return run_quant_b<DT_F32>(q, k);
    case DT_F16: return run_quant_b<DT_F16>(q, k);
    default: return run_quant_b<DT_BF16>(q, k);
  }
}

}  // namespace hq
