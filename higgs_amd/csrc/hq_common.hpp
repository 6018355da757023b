// hq_common.hpp -- device helpers shared by the gfx950 kernels: dtype
// conversion, LSB-first bit unpacking of MLX-packed weights, wave reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hq {

enum Dtype : int { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

// Output dtype under MLX promotion for two floating dtypes.
__host__ __device__ constexpr int result_dtype(int a, int b) { return a == b ? a : DT_F32; }

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------------------
// scalar conversions
// ---------------------------------------------------------------------------

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// Round-to-nearest-even, NaN -> canonical 0x7FC0.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, (uint16_t)h);
  return (float)v;
}

// Hardware v_cvt_f16_f32: round-to-nearest-even, keeps fp16 denormals.
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  _Float16 v = (_Float16)f;
  uint32_t b = __builtin_bit_cast(uint16_t, v);
  if ((__float_as_uint(f) & 0x7fffffffu) > 0x7f800000u) b = (b & 0x8000u) | 0x7e00u;
  return b;
}

template <int DT> struct DT_;
template <> struct DT_<DT_F32> {
  using storage = float;
  static __device__ __forceinline__ float load(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ float to_f32(float v) { return v; }
  static __device__ __forceinline__ float from_f32(float v) { return v; }
  static __device__ __forceinline__ float round(float v) { return v; }
};
template <> struct DT_<DT_BF16> {
  using storage = uint16_t;
  static __device__ __forceinline__ float load(const uint16_t* p, int64_t i) { return bf16_bits_to_f32(p[i]); }
  static __device__ __forceinline__ float to_f32(uint16_t v) { return bf16_bits_to_f32(v); }
  static __device__ __forceinline__ uint16_t from_f32(float v) { return (uint16_t)f32_to_bf16_bits(v); }
  static __device__ __forceinline__ float round(float v) { return bf16_bits_to_f32(f32_to_bf16_bits(v)); }
};
template <> struct DT_<DT_F16> {
  using storage = uint16_t;
  static __device__ __forceinline__ float load(const uint16_t* p, int64_t i) { return f16_bits_to_f32(p[i]); }
  static __device__ __forceinline__ float to_f32(uint16_t v) { return f16_bits_to_f32(v); }
  static __device__ __forceinline__ uint16_t from_f32(float v) { return (uint16_t)f32_to_f16_bits(v); }
  static __device__ __forceinline__ float round(float v) { return f16_bits_to_f32(f32_to_f16_bits(v)); }
};

template <int DT> using st_t = typename DT_<DT>::storage;

// SwiGLU of one (gate, up) pair: gate * sigmoid(gate) * up
// (crates/higgs-models/src/qwen3_next.rs:340-342). Callers pass gate and up
// already rounded to the output dtype, as the reference materialises both
// projections before the elementwise op, and round the result once.
__device__ __forceinline__ float swiglu_f32(float g, float u) {
  return g / (1.f + __expf(-g)) * u;
}

// One output element of a quantized linear layer: the product rounded to the
// output dtype, then the layer's bias (`lbias`, [N] of the output dtype; null
// for none) added and rounded again -- mlx-rs QuantizedLinear::forward is
// quantized_matmul followed by an add (two roundings for 16-bit outputs).
template <int ODT>
__device__ __forceinline__ st_t<ODT> linear_out(float acc, const void* lbias, int64_t n) {
  if (lbias != nullptr)
    return DT_<ODT>::from_f32(DT_<ODT>::round(acc) + DT_<ODT>::load((const st_t<ODT>*)lbias, n));
  return DT_<ODT>::from_f32(acc);
}

// Load 8 consecutive elements (16 B for 16-bit types, 32 B for float32) and
// widen to float. `p` must be 16-B aligned for 16-bit types.
template <int DT>
__device__ __forceinline__ void load8_f32(const st_t<DT>* p, float (&v)[8]) {
  if constexpr (DT == DT_F32) {
    const float4* q = reinterpret_cast<const float4*>(p);
    float4 a = q[0], b = q[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    u32x4 d = *reinterpret_cast<const u32x4*>(p);
#pragma unroll
    for (int i = 0; i < 4; i++) {
      v[2 * i] = DT_<DT>::to_f32((uint16_t)(d[i] & 0xffffu));
      v[2 * i + 1] = DT_<DT>::to_f32((uint16_t)(d[i] >> 16));
    }
  }
}

// ---------------------------------------------------------------------------
// MLX packing: element i of a row is bits [i*BITS, i*BITS + BITS) of the
// row's little-endian u32 bitstream. A "pack" is 32 consecutive elements,
// i.e. exactly BITS words, so packs never share words for any BITS.
// ---------------------------------------------------------------------------

template <int BITS>
__device__ __forceinline__ void load_pack(const uint32_t* p, uint32_t (&wd)[BITS]) {
  if constexpr (BITS == 4) {
    u32x4 v = *reinterpret_cast<const u32x4*>(p);
    wd[0] = v[0]; wd[1] = v[1]; wd[2] = v[2]; wd[3] = v[3];
  } else if constexpr (BITS == 8) {
    u32x4 a = reinterpret_cast<const u32x4*>(p)[0];
    u32x4 b = reinterpret_cast<const u32x4*>(p)[1];
    wd[0] = a[0]; wd[1] = a[1]; wd[2] = a[2]; wd[3] = a[3];
    wd[4] = b[0]; wd[5] = b[1]; wd[6] = b[2]; wd[7] = b[3];
  } else if constexpr (BITS == 2) {
    u32x2 v = *reinterpret_cast<const u32x2*>(p);
    wd[0] = v[0]; wd[1] = v[1];
  } else {
#pragma unroll
    for (int i = 0; i < BITS; i++) wd[i] = p[i];
  }
}

// Element E (0..31, compile-time after unrolling) of a pack.
template <int BITS>
__device__ __forceinline__ uint32_t pack_elem(const uint32_t (&wd)[BITS], int e) {
  const int bit = e * BITS;
  const int w = bit >> 5, off = bit & 31;
  uint32_t v = wd[w] >> off;
  if (off + BITS > 32) v |= wd[w + 1] << (32 - off);
  return v & ((1u << BITS) - 1u);
}

// ---------------------------------------------------------------------------
// wave64 reductions
// ---------------------------------------------------------------------------

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ int ilog2(int v) { return 31 - __clz(v); }

// First index i in [0, n) with v[i] >= key (n if none), for non-decreasing v.
// Wave-uniform result; two or three rounds of 64 probes for n <= 2^18.
__device__ __forceinline__ int64_t wave_lower_bound(const uint32_t* v, int64_t n, uint32_t key) {
  const int lane = threadIdx.x & 63;
  int64_t lo = 0, hi = n;  // v[j] < key for j < lo; answer in [lo, hi]
  while (lo < hi) {
    const int64_t step = (hi - lo + 63) / 64;
    const int64_t p = lo + (int64_t)lane * step;
    const bool less = p < hi && v[p] < key;
    const int c = __popcll(__ballot(less));  // probes below key form a prefix
    if (c == 0) return lo;                  // v[lo] >= key
    const int64_t nlo = lo + (int64_t)(c - 1) * step + 1;
    const int64_t nhi = min(hi, lo + (int64_t)c * step);
    if (step == 1) return nhi;
    lo = nlo;
    hi = nhi;
  }
  return lo;
}

}  // namespace hq
