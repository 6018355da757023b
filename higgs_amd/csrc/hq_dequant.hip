// hq_dequant.hip -- dequantize and gathered-row dequantize (quantized
// embedding lookup) for one bit width (HQ_BITS).
//
// out[r, k] = round(round(q * s) + b) in the scales' dtype: the product and
// the sum each round separately (round-to-nearest-even), which is MLX's
// op-by-op dequantize (multiply, then add) as reached from
// crates/higgs-models/src/qwen3_next.rs:308-318. The kernel is HBM-bound:
// each thread turns one 32-element pack (HQ_BITS words, 128-bit loads where
// the width allows) into 32 outputs written with 128-bit stores.
#include "hq_common.hpp"
#include "hq_kernels.hpp"

#ifndef HQ_BITS
#error "compile with -DHQ_BITS=<2|3|4|5|6|8>"
#endif

namespace hq {

template <int SDT>
__device__ __forceinline__ float deq_round(uint32_t q, float s, float b) {
#pragma clang fp contract(off)
  float p = DT_<SDT>::round((float)q * s);
  return DT_<SDT>::round(p + b);
}

// Two adjacent 16-bit outputs round(round(q*s) + b), packed. The roundings
// are the hardware float -> bf16 / fp16 conversions (round to nearest even,
// v_cvt_pk_bf16_f32 / v_cvt_f16_f32), a third of the instructions of the
// integer rounding sequence; NaN results are rewritten to the canonical
// quiet NaN (bf16 0x7fc0; fp16 sign | 0x7e00) exactly as the integer
// sequence produces them. A NaN needs a non-finite scale or bias (q*s of
// finite values at most overflows to an infinity, and inf + finite is inf),
// so CANON = false skips the rewrite for groups whose scale and bias are
// finite.
template <int SDT, bool CANON>
__device__ __forceinline__ uint32_t deq_pair(uint32_t q0, uint32_t q1, float s, float b) {
#pragma clang fp contract(off)
  if constexpr (SDT == DT_BF16) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    bf2 p;
    p[0] = (__bf16)((float)q0 * s);
    p[1] = (__bf16)((float)q1 * s);
    const float r0 = (float)p[0] + b, r1 = (float)p[1] + b;
    bf2 o;
    o[0] = (__bf16)r0;
    o[1] = (__bf16)r1;
    uint32_t u = __builtin_bit_cast(uint32_t, o);
    if constexpr (CANON) {
      if (r0 != r0) u = (u & 0xffff0000u) | 0x7fc0u;
      if (r1 != r1) u = (u & 0x0000ffffu) | 0x7fc00000u;
    }
    return u;
  } else {
    // The product is exact in fp32 (at most 8 + 11 significant bits). The
    // empty asm keeps it a plain fp32 multiply: fused into v_fma_mixlo_f16
    // (q * s + 0) it would turn a -0 product into +0.
    float m0 = (float)q0 * s, m1 = (float)q1 * s;
    __asm__ volatile("" : "+v"(m0), "+v"(m1));
    const _Float16 p0 = (_Float16)m0, p1 = (_Float16)m1;
    const float r0 = (float)p0 + b, r1 = (float)p1 + b;
    uint32_t lo = __builtin_bit_cast(uint16_t, (_Float16)r0);
    uint32_t hi = __builtin_bit_cast(uint16_t, (_Float16)r1);
    if constexpr (CANON) {
      if (r0 != r0) lo = ((__float_as_uint(r0) >> 16) & 0x8000u) | 0x7e00u;
      if (r1 != r1) hi = ((__float_as_uint(r1) >> 16) & 0x8000u) | 0x7e00u;
    }
    return lo | (hi << 16);
  }
}

template <int BITS, int SDT>
__global__ __launch_bounds__(256) void dequant_kernel(st_t<SDT>* __restrict__ out,
                                                       const uint32_t* __restrict__ w,
                                                       const st_t<SDT>* __restrict__ s,
                                                       const st_t<SDT>* __restrict__ b,
                                                       const uint32_t* __restrict__ rows_idx,
                                                       uint32_t total_packs, uint32_t ppr,
                                                       int64_t src_rows, int gshift_packs) {
  const int64_t K = (int64_t)ppr * 32;
  const int64_t P = (int64_t)ppr * BITS;   // words per row
  const int64_t G = (int64_t)ppr >> gshift_packs;  // groups per row
  for (uint32_t t = blockIdx.x * 256u + threadIdx.x; t < total_packs; t += gridDim.x * 256u) {
    const uint32_t r = t / ppr;
    const uint32_t p = t - r * ppr;
    const int64_t src = rows_idx ? (int64_t)rows_idx[r] : (int64_t)r;
    st_t<SDT>* o = out + (int64_t)r * K + (int64_t)p * 32;
    if constexpr (SDT == DT_F32) {
      float v[32];
      if (src >= src_rows) {
#pragma unroll
        for (int e = 0; e < 32; e++) v[e] = __uint_as_float(0x7fc00000u);
      } else {
        uint32_t wd[BITS];
        load_pack<BITS>(w + src * P + (int64_t)p * BITS, wd);
        const int64_t gi = src * G + (p >> gshift_packs);
        const float sv = s[gi], bv = b[gi];
#pragma unroll
        for (int e = 0; e < 32; e++) v[e] = deq_round<SDT>(pack_elem<BITS>(wd, e), sv, bv);
      }
      float4* o4 = reinterpret_cast<float4*>(o);
#pragma unroll
      for (int i = 0; i < 8; i++) o4[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    } else {
      uint32_t h[16];
      if (src >= src_rows) {
        const uint32_t nan2 = SDT == DT_BF16 ? 0x7fc07fc0u : 0x7e007e00u;
#pragma unroll
        for (int i = 0; i < 16; i++) h[i] = nan2;
      } else {
        uint32_t wd[BITS];
        load_pack<BITS>(w + src * P + (int64_t)p * BITS, wd);
        const int64_t gi = src * G + (p >> gshift_packs);
        const float sv = DT_<SDT>::load(s, gi), bv = DT_<SDT>::load(b, gi);
        if (__builtin_isfinite(sv) && __builtin_isfinite(bv)) {
#pragma unroll
          for (int i = 0; i < 16; i++)
            h[i] = deq_pair<SDT, false>(pack_elem<BITS>(wd, 2 * i), pack_elem<BITS>(wd, 2 * i + 1), sv, bv);
        } else {
#pragma unroll
          for (int i = 0; i < 16; i++)
            h[i] = deq_pair<SDT, true>(pack_elem<BITS>(wd, 2 * i), pack_elem<BITS>(wd, 2 * i + 1), sv, bv);
        }
      }
      u32x4* o4 = reinterpret_cast<u32x4*>(o);
#pragma unroll
      for (int i = 0; i < 4; i++) o4[i] = u32x4{h[4 * i], h[4 * i + 1], h[4 * i + 2], h[4 * i + 3]};
    }
  }
}

// 16-bit outputs: one thread per 8 consecutive outputs (a quarter of a
// 32-element pack), so a wave's 16-byte stores cover 1 KB contiguously and
// its weight loads are contiguous too (BITS bytes per thread). The thread
// reads the 8*BITS bits of its quarter from at most two words of the pack.
// Each thread takes QPT quarters a grid stride apart and issues all their
// loads before the first use (addresses clamped, so no load sits under a
// branch): one 256-byte load per wave in flight is far too little to cover
// HBM latency (14336 x 4096: 39.2 us at one quarter per thread, 31.2 at 4).
// Small inputs get a grid of one block per 256 quarters instead (the other
// quarters of a thread then lie past the end: clamped loads, no store).
constexpr int kQPT = 4;

template <int BITS>
__device__ __forceinline__ void load_quarter(const uint32_t* pw, uint32_t qq, uint32_t (&v)[2]) {
  if constexpr (BITS == 4) {
    v[0] = pw[qq];
    v[1] = 0u;
  } else if constexpr (BITS == 2) {
    v[0] = pw[qq >> 1] >> (16u * (qq & 1u));
    v[1] = 0u;
  } else if constexpr (BITS == 8) {
    v[0] = pw[2 * qq];
    v[1] = pw[2 * qq + 1];
  } else {
    const uint32_t bit0 = qq * 8u * BITS, i0 = bit0 >> 5;
    const uint32_t i1 = i0 + 1 < (uint32_t)BITS ? i0 + 1 : i0;
    v[0] = pw[i0];
    v[1] = pw[i1];
  }
}

template <int BITS>
__device__ __forceinline__ void quarter_elems(const uint32_t (&v)[2], uint32_t qq, uint32_t (&e)[8]) {
  if constexpr (BITS == 4 || BITS == 2) {
#pragma unroll
    for (int j = 0; j < 8; j++) e[j] = (v[0] >> (BITS * j)) & ((1u << BITS) - 1u);
  } else if constexpr (BITS == 8) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      e[j] = (v[0] >> (8 * j)) & 0xffu;
      e[j + 4] = (v[1] >> (8 * j)) & 0xffu;
    }
  } else {
    const uint32_t off = (qq * 8u * BITS) & 31u;
    const uint64_t x = ((uint64_t)v[1] << 32 | v[0]) >> off;
#pragma unroll
    for (int j = 0; j < 8; j++) e[j] = (uint32_t)(x >> (BITS * j)) & ((1u << BITS) - 1u);
  }
}

template <int BITS, int SDT>
__global__ __launch_bounds__(256) void dequant8_kernel(uint16_t* __restrict__ out,
                                                        const uint32_t* __restrict__ w,
                                                        const uint16_t* __restrict__ s,
                                                        const uint16_t* __restrict__ b,
                                                        const uint32_t* __restrict__ rows_idx,
                                                        uint32_t total_q, uint32_t ppr,
                                                        int64_t src_rows, int gshift_packs) {
  const int64_t K = (int64_t)ppr * 32;
  const int64_t P = (int64_t)ppr * BITS;
  const int64_t G = (int64_t)ppr >> gshift_packs;
  const uint32_t stride = gridDim.x * 256u;
  for (uint32_t base = blockIdx.x * 256u + threadIdx.x; base < total_q; base += kQPT * stride) {
    uint32_t wv[kQPT][2], r[kQPT], p[kQPT], qq[kQPT];
    uint16_t sr[kQPT], br[kQPT];
    bool ok[kQPT];
#pragma unroll
    for (int k = 0; k < kQPT; k++) {
      const uint32_t t = min(base + (uint32_t)k * stride, total_q - 1u);
      const uint32_t pk = t >> 2;
      qq[k] = t & 3u;
      r[k] = pk / ppr;
      p[k] = pk - r[k] * ppr;
      const int64_t src = rows_idx ? (int64_t)rows_idx[r[k]] : (int64_t)r[k];
      ok[k] = src < src_rows;
      const int64_t sc = ok[k] ? src : 0;
      load_quarter<BITS>(w + sc * P + (int64_t)p[k] * BITS, qq[k], wv[k]);
      const int64_t gi = sc * G + (p[k] >> gshift_packs);
      sr[k] = s[gi];
      br[k] = b[gi];
    }
#pragma unroll
    for (int k = 0; k < kQPT; k++) {
      if (base + (uint32_t)k * stride >= total_q) continue;
      u32x4 h;
      if (!ok[k]) {
        const uint32_t nan2 = SDT == DT_BF16 ? 0x7fc07fc0u : 0x7e007e00u;
        h = u32x4{nan2, nan2, nan2, nan2};
      } else {
        uint32_t e[8];
        quarter_elems<BITS>(wv[k], qq[k], e);
        const float sv = DT_<SDT>::to_f32(sr[k]), bv = DT_<SDT>::to_f32(br[k]);
        if (__builtin_isfinite(sv) && __builtin_isfinite(bv)) {
#pragma unroll
          for (int i = 0; i < 4; i++) h[i] = deq_pair<SDT, false>(e[2 * i], e[2 * i + 1], sv, bv);
        } else {
#pragma unroll
          for (int i = 0; i < 4; i++) h[i] = deq_pair<SDT, true>(e[2 * i], e[2 * i + 1], sv, bv);
        }
      }
      *reinterpret_cast<u32x4*>(out + (int64_t)r[k] * K + (int64_t)p[k] * 32 + qq[k] * 8) = h;
    }
  }
}

// Internal linkage and BITS as a parameter: this file is compiled once per
// bit width, and one shared definition would launch one width's kernel for
// all of them.
namespace {
template <int BITS, int SDT>
void launch_deq8(const DeqArgs& a, uint64_t tq, uint32_t ppr, int gsp) {
  const uint64_t per_block = tq >= (1u << 20) ? 256 * kQPT : 256;
  uint32_t qb = (uint32_t)((tq + per_block - 1) / per_block);
  if (qb > 65536u * 8u) qb = 65536u * 8u;
  dequant8_kernel<BITS, SDT><<<qb, 256, 0, a.stream>>>(
      (uint16_t*)a.out, a.w, (const uint16_t*)a.s, (const uint16_t*)a.b, a.rows_idx, (uint32_t)tq,
      ppr, a.src_rows, gsp);
}
}  // namespace

#define HQ_CAT_(a, b) a##b
#define HQ_CAT(a, b) HQ_CAT_(a, b)

hipError_t HQ_CAT(launch_dequant_b, HQ_BITS)(const DeqArgs& a) {
  const uint32_t ppr = (uint32_t)(a.K / 32);
  const uint64_t total = (uint64_t)a.n_rows * ppr;
  const int gsp = __builtin_ctz((unsigned)(a.group_size / 32));
  uint32_t blocks = (uint32_t)((total + 255) / 256);
  if (blocks > 65536u * 8u) blocks = 65536u * 8u;
  if (blocks == 0) return hipSuccess;
  switch (a.sdt) {
    case DT_F32:
      dequant_kernel<HQ_BITS, DT_F32><<<blocks, 256, 0, a.stream>>>(
          (float*)a.out, a.w, (const float*)a.s, (const float*)a.b, a.rows_idx, (uint32_t)total, ppr,
          a.src_rows, gsp);
      break;
    case DT_F16:
    default: {
      // quarter packs: 4 threads per pack (total < 2^29, checked by the caller)
      const uint64_t tq = total * 4;
      if (a.sdt == DT_F16) launch_deq8<HQ_BITS, DT_F16>(a, tq, ppr, gsp);
      else launch_deq8<HQ_BITS, DT_BF16>(a, tq, ppr, gsp);
      break;
    }
  }
  return hipGetLastError();
}

}  // namespace hq
