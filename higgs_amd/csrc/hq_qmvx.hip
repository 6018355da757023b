// hq_qmvx.hip -- matrix-core GEMV for decode (M <= 8 rows of x, x in bf16 or
// fp16), one bit width (HQ_BITS).
//
// y[m, n] = sum_k x[m, k] * (s[n, g] * q[n, k] + b[n, g]),  g = k / group_size
// (mlx-rs ops::quantized_matmul, transpose=true, as called from
// crates/higgs-models/src/qwen3_next.rs:218-227; LSB-first packing and group
// math as stated in-tree at qwen3_next.rs:969-988).
//
// Why MFMA for a GEMV: at 8 TB/s a 4-bit weight stream is 16 G elements/s,
// and a scalar dequantize-multiply-add path needs ~3 VALU ops per element --
// more than the 39 T lane-ops/s the VALU has. Here the VALU only turns each
// u32 of nibbles into four (OFF + q) bf16 pairs with one AND-OR each
// (0.875 ops per element); the matrix cores do the multiply-add.
//
// Layout of one v_mfma_f32_16x16x32 step: B = 16 weight rows (n = lane % 16)
// x 32 k, A = x rows, D[m', n] in fp32. A wave walks 128-element "segments"
// of K: lane (n, q = lane / 16) loads pack q (32 elements, HQ_BITS words) of
// row n, and its four words feed four MFMA steps. Within a segment the packs
// of one lane group belong to group-half h = q * Z / 4 (Z = 128 / group_size
// groups per segment), and A row m' = 4h + m (8h + m when M > 4) carries x[m]
// only in the k-blocks of half h, zeros elsewhere. One MFMA therefore yields
// the per-group partial dot products for every (m, h) without mixing groups,
// and the epilogue applies  s * D + (b - OFF * s) * X  with X = sum of x over
// the group (the OFF term removes the exponent bias baked into OFF + q).
//
// x is staged once per block in LDS (row-major, each 8-element block stored in
// the MFMA pair order (0,4,1,5,2,6,3,7)), with a zero row that A lanes of other
// halves read; X sums are computed during staging. Waves of a block split K
// into contiguous segment ranges; partial sums are reduced through LDS in a
// fixed order (deterministic).
#include <type_traits>

#include "hq_common.hpp"
#include "hq_device.hpp"
#include "hq_kernels.hpp"

#ifndef HQ_BITS
#error "compile with -DHQ_BITS=<2|3|4|5|6|8>"
#endif

namespace hq {

namespace {

struct QXKern {
  void* y;
  const void* x;
  const uint32_t* w;
  const void* s;
  const void* b;
  const uint32_t* lhs;
  const uint32_t* rhs;
  int64_t batch, x_rep, x_batch, w_batch;
  int M, N, K;
  int KC;       // K elements staged per chunk (multiple of 128)
  int S;        // segments per wave per chunk
  const void* lb;  // linear bias [N] or null (batch == 1 only)
};

template <int XDT> struct XMma;
template <> struct XMma<DT_BF16> {
  using frag = bf16x8;
  static __device__ __forceinline__ floatx4 mma(frag a, frag b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  // bf16 128.0 in both halves: (0x4300 | q) == 128 + q exactly for q < 128.
  static constexpr uint32_t OFFB = 0x43004300u;
  static constexpr float OFF = 128.f;
};
template <> struct XMma<DT_F16> {
  using frag = f16x8;
  static __device__ __forceinline__ floatx4 mma(frag a, frag b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  // fp16 1024.0: (0x6400 | q) == 1024 + q exactly for q < 1024.
  static constexpr uint32_t OFFB = 0x64006400u;
  static constexpr float OFF = 1024.f;
};

// 8-bit weights with bf16 x: 128 + q does not fit bf16's 8-bit significand,
// so q is converted exactly (q <= 255 is a bf16 integer) and OFF is 0.
template <int BITS, int XDT>
constexpr bool kExact8 = (BITS == 8 && XDT == DT_BF16);

// Step i (0..3) of a 32-element pack: four u32, each two 16-bit MFMA operand
// values, element order (8i+j, 8i+j+4) for j = 0..3.
template <int BITS, int XDT>
__device__ __forceinline__ u32x4 unpack_step(const uint32_t (&wd)[BITS], int i) {
  u32x4 r;
  if constexpr (BITS == 4) {
    const uint32_t w = wd[i];
    r[0] = (w & 0x000F000Fu) | XMma<XDT>::OFFB;
    r[1] = ((w >> 4) & 0x000F000Fu) | XMma<XDT>::OFFB;
    r[2] = ((w >> 8) & 0x000F000Fu) | XMma<XDT>::OFFB;
    r[3] = ((w >> 12) & 0x000F000Fu) | XMma<XDT>::OFFB;
  } else if constexpr (kExact8<BITS, XDT>) {
    const uint32_t lo = wd[2 * i], hi = wd[2 * i + 1];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t fa = __float_as_uint((float)((lo >> (8 * j)) & 0xffu));
      const uint32_t fb = __float_as_uint((float)((hi >> (8 * j)) & 0xffu));
      r[j] = (fa >> 16) | (fb & 0xffff0000u);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint32_t qa = pack_elem<BITS>(wd, 8 * i + j);
      const uint32_t qb = pack_elem<BITS>(wd, 8 * i + j + 4);
      r[j] = (qa | (qb << 16)) | XMma<XDT>::OFFB;
    }
  }
  return r;
}

template <int ODT>
__device__ __forceinline__ st_t<ODT> nanv() {
  if constexpr (ODT == DT_F32) return __uint_as_float(0x7fc00000u);
  else if constexpr (ODT == DT_BF16) return (uint16_t)0x7fc0u;
  else return (uint16_t)0x7e00u;
}

constexpr int kU = 4;  // segments whose loads are issued together

// Bytes of one x row in LDS: 16 more than the row, so that the same column of
// consecutive rows falls in different LDS banks (rows of 128-element segments
// are whole multiples of the 256-byte bank cycle; several x rows read one
// column at a time measured 3.4 bank-conflict cycles per LDS cycle at 8 rows;
// the step time did not change, LDS is not what limits those kernels).
__host__ __device__ constexpr int xrow_bytes(int k) { return k * 2 + 16; }

// BITS, x dtype (bf16 | fp16), scale dtype, MB = M rounded up to 1/2/4/8,
// GS = group size.
template <int BITS, int XDT, int SDT, int MB, int GS>
__global__ __launch_bounds__(1024) void qmvx_kernel(QXKern a) {
  using XS = st_t<XDT>;
  using SS = st_t<SDT>;
  constexpr int ODT = result_dtype(XDT, SDT);
  using OS = st_t<ODT>;
  using T = XMma<XDT>;
  constexpr float OFF = kExact8<BITS, XDT> ? 0.f : T::OFF;
  constexpr int Z = 128 / GS;                    // groups per segment
  constexpr int RPH = MB <= 4 ? 4 : 8;           // A rows per group-half
  constexpr int NMF = (Z * RPH + 15) / 16;       // MFMAs per step
  constexpr int HPM = 16 / RPH;                  // halves per MFMA
  constexpr int VM = MB < 4 ? MB : 4;            // useful D values per lane

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int W = blockDim.x >> 6;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int M = a.M, N = a.N, K = a.K, KC = a.KC;
  const int n0 = blockIdx.x * 16;
  const int packs = K >> 5;
  const int64_t P = (int64_t)packs * BITS;  // words per weight row
  const int64_t G = K / GS;

  // LDS: x rows [M + 1][KC] (row M is zeros), X sums [KC/GS][RPH] floats,
  // reduction slots [W][Z][M][16] floats.
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem);
  float* Xs = reinterpret_cast<float*>(smem + (size_t)(M + 1) * xrow_bytes(KC));
  float* red = Xs + (KC / GS) * RPH;

  const int nl = lane & 15, q = lane >> 4;
  const int n_eff = min(n0 + nl, N - 1);

  // Per-lane A-operand base (bytes into xs) for each MFMA of a step.
  int abase[NMF];
#pragma unroll
  for (int mf = 0; mf < NMF; mf++) {
    const int mrow = nl;                            // A row m' of this lane
    const int h = mf * HPM + mrow / RPH;            // group-half of that row
    const int m = mrow % RPH;
    const int hq = q * Z / 4;                       // half of this lane's k-block
    const bool valid = (h == hq) && (m < M) && (h < Z);
    abase[mf] = (valid ? m : M) * xrow_bytes(KC) + q * 64;
  }
  // D-side: half and x-row of this lane's accumulator values, per MFMA.
  int dh[NMF];
#pragma unroll
  for (int mf = 0; mf < NMF; mf++) dh[mf] = mf * HPM + (MB <= 4 ? q : q / 2);
  const int dm0 = MB <= 4 ? 0 : 4 * (q & 1);  // x row of value v is dm0 + v

  for (int64_t bi = blockIdx.y; bi < a.batch; bi += gridDim.y) {
    const int64_t xi = a.lhs ? (int64_t)a.lhs[bi] : bi / a.x_rep;
    const int64_t wi = a.rhs ? (int64_t)a.rhs[bi] : 0;
    OS* yb = (OS*)a.y + bi * (int64_t)M * N;
    if (xi >= a.x_batch || wi >= a.w_batch) {
      for (int t = tid; t < M * 16; t += blockDim.x)
        if (n0 + (t & 15) < N) yb[(int64_t)(t >> 4) * N + n0 + (t & 15)] = nanv<ODT>();
      continue;
    }
    const XS* xb = (const XS*)a.x + xi * (int64_t)M * K;
    const uint32_t* wrow = a.w + wi * (int64_t)N * P + (int64_t)n_eff * P;
    const SS* srow = (const SS*)a.s + wi * (int64_t)N * G + (int64_t)n_eff * G;
    const SS* brow = (const SS*)a.b + wi * (int64_t)N * G + (int64_t)n_eff * G;

    float acc[NMF][4];
#pragma unroll
    for (int mf = 0; mf < NMF; mf++)
#pragma unroll
      for (int v = 0; v < 4; v++) acc[mf][v] = 0.f;

    for (int kc0 = 0; kc0 < K; kc0 += KC) {
      const int kcn = min(KC, K - kc0);          // elements in this chunk
      const int nseg = (kcn + 127) >> 7;
      const int seg_lo = min(wv * a.S, nseg);
      const int seg_hi = min(seg_lo + a.S, nseg);

      // ---- stage x chunk + group sums ----
      {
        const int cpr = KC >> 3;                  // 8-element blocks per row
        for (int t = tid; t < (M + 1) * cpr; t += blockDim.x) {
          const int m = t / cpr, c = t - m * cpr;
          const int k = kc0 + c * 8;
          u32x4 d = {0u, 0u, 0u, 0u};
          float sum = 0.f;
          if (m < M && k < K) {
            d = *reinterpret_cast<const u32x4*>(xb + (int64_t)m * K + k);
#pragma unroll
            for (int e = 0; e < 4; e++)
              sum += DT_<XDT>::to_f32((uint16_t)(d[e] & 0xffffu)) +
                     DT_<XDT>::to_f32((uint16_t)(d[e] >> 16));
          }
          u32x4 o;
          o[0] = (d[0] & 0xffffu) | (d[2] << 16);
          o[1] = (d[0] >> 16) | (d[2] & 0xffff0000u);
          o[2] = (d[1] & 0xffffu) | (d[3] << 16);
          o[3] = (d[1] >> 16) | (d[3] & 0xffff0000u);
          *reinterpret_cast<u32x4*>(smem + (size_t)m * xrow_bytes(KC) + c * 16) = o;
          // GS/8 consecutive threads hold one group: reduce in the wave.
#pragma unroll
          for (int o2 = 1; o2 < GS / 8; o2 <<= 1) sum += __shfl_xor(sum, o2, 64);
          if (m < M && (c & (GS / 8 - 1)) == 0) Xs[(c / (GS / 8)) * RPH + m] = sum;
        }
        for (int t = tid; t < (KC / GS) * RPH; t += blockDim.x)
          if ((t % RPH) >= M) Xs[t] = 0.f;
      }
      __syncthreads();

      // ---- stream this wave's segments ----
      for (int sb = seg_lo; sb < seg_hi; sb += kU) {
        uint32_t wd[kU][BITS];
        float sv[kU][NMF], bv[kU][NMF];
#pragma unroll
        for (int u = 0; u < kU; u++) {
          const int seg = sb + u;
          const int p = ((kc0 >> 7) + seg) * 4 + q;  // pack index in the row
          if (seg < seg_hi && p < packs) {
            load_pack<BITS>(wrow + (int64_t)p * BITS, wd[u]);
          } else {
#pragma unroll
            for (int i = 0; i < BITS; i++) wd[u][i] = 0u;
          }
#pragma unroll
          for (int mf = 0; mf < NMF; mf++) {
            const int hc = min(dh[mf], Z - 1);
            int64_t g = (int64_t)((kc0 >> 7) + seg) * Z + hc;
            g = min(g, G - 1);
            sv[u][mf] = DT_<SDT>::load(srow, g);
            bv[u][mf] = DT_<SDT>::load(brow, g);
          }
        }
#pragma unroll
        for (int u = 0; u < kU; u++) {
          // Segments past this wave's range (tail batch) are computed on a
          // clamped in-range address and contribute zero.
          const bool live = sb + u < seg_hi;
          const int seg = min(sb + u, nseg - 1);
          floatx4 d[NMF];
#pragma unroll
          for (int mf = 0; mf < NMF; mf++) d[mf] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const u32x4 bw = unpack_step<BITS, XDT>(wd[u], i);
#pragma unroll
            for (int mf = 0; mf < NMF; mf++) {
              const u32x4 av = *reinterpret_cast<const u32x4*>(
                  reinterpret_cast<const unsigned char*>(xs) + abase[mf] + seg * 256 + i * 16);
              d[mf] = T::mma(__builtin_bit_cast(typename T::frag, av),
                             __builtin_bit_cast(typename T::frag, bw), d[mf]);
            }
          }
#pragma unroll
          for (int mf = 0; mf < NMF; mf++) {
            const int hc = min(dh[mf], Z - 1);
            const float s = live ? sv[u][mf] : 0.f;
            const float bo = live ? fmaf(-OFF, sv[u][mf], bv[u][mf]) : 0.f;
            const floatx4 X = *reinterpret_cast<const floatx4*>(Xs + (seg * Z + hc) * RPH + dm0);
#pragma unroll
            for (int v = 0; v < VM; v++) acc[mf][v] = fmaf(s, d[mf][v], fmaf(bo, X[v], acc[mf][v]));
          }
        }
      }
      __syncthreads();  // xs / Xs are restaged by the next chunk
    }

    // ---- reduce over waves and halves, fixed order ----
#pragma unroll
    for (int mf = 0; mf < NMF; mf++) {
      const int h = dh[mf];
      if (h < Z) {
#pragma unroll
        for (int v = 0; v < VM; v++) {
          const int m = dm0 + v;
          if (m < M) red[((wv * Z + h) * M + m) * 16 + nl] = acc[mf][v];
        }
      }
    }
    __syncthreads();
    for (int t = tid; t < M * 16; t += blockDim.x) {
      const int m = t >> 4, n = t & 15;
      float r = 0.f;
      for (int w2 = 0; w2 < W; w2++)
#pragma unroll
        for (int h = 0; h < Z; h++) r += red[((w2 * Z + h) * M + m) * 16 + n];
      if (n0 + n < N) yb[(int64_t)m * N + n0 + n] = linear_out<ODT>(r, a.lb, n0 + n);
    }
    __syncthreads();  // red is rewritten by the next batch element
  }
}

// ---------------------------------------------------------------------------
// Persistent variant for one product (batch == 1) of exact shape
// (K % 1024 == 0): x is staged once per block, the block walks row tiles
// t = blockIdx.x + j * gridDim.x, and each tile is split into R rounds of W
// waves x S segments. A wave's S segments of a round share MFMA accumulators:
// segment u, group-half h, x row m goes to A row ((u % SU) * Z + h) * MB + m,
// so up to 16 / (Z * MB) segments fill one 16-row accumulator and the scale
// epilogue runs once per accumulator instead of once per segment. The loads
// of the next round (possibly of the next tile) are in flight while the
// current one is computed (register double buffer). Partials of a tile meet
// in LDS after one block barrier (double-buffered slots, fixed-order sum).
// ---------------------------------------------------------------------------

struct PKern {
  void* y;
  const void* x;
  const uint32_t* w;
  const void* s;
  const void* b;
  int M, N, K;
  int R;        // rounds per tile
  int ntiles;   // ceil(N / 16)
  // SwiGLU: up projection (gate is w/s/b); a tile's gate rounds run first,
  // then its up rounds, and the up finish combines both.
  const uint32_t* w2;
  const void* s2;
  const void* b2;
  // 0x000F000F and the operand offset pair, passed as kernel arguments so the
  // compiler keeps them in registers and emits one v_and_or_b32 per pair (gfx9
  // VOP3 cannot encode 32-bit literals).
  uint32_t nib_mask, off_pair;
  const void* lb;  // linear bias [N] or null (not with SwiGLU)
};

// NG consecutive scale values as floats (vector load).
template <int SDT, int NG>
__device__ __forceinline__ void load_groups(const st_t<SDT>* p, float (&o)[NG]) {
  if constexpr (SDT == DT_F32) {
    if constexpr (NG == 4) {
      const float4 v = *reinterpret_cast<const float4*>(p);
      o[0] = v.x; o[1] = v.y; o[2] = v.z; o[3] = v.w;
    } else if constexpr (NG == 2) {
      const float2 v = *reinterpret_cast<const float2*>(p);
      o[0] = v.x; o[1] = v.y;
    } else {
      o[0] = p[0];
    }
  } else {
    if constexpr (NG == 4) {
      const u32x2 v = *reinterpret_cast<const u32x2*>(p);
      o[0] = DT_<SDT>::to_f32((uint16_t)(v[0] & 0xffffu));
      o[1] = DT_<SDT>::to_f32((uint16_t)(v[0] >> 16));
      o[2] = DT_<SDT>::to_f32((uint16_t)(v[1] & 0xffffu));
      o[3] = DT_<SDT>::to_f32((uint16_t)(v[1] >> 16));
    } else if constexpr (NG == 2) {
      const uint32_t v = *reinterpret_cast<const uint32_t*>(p);
      o[0] = DT_<SDT>::to_f32((uint16_t)(v & 0xffffu));
      o[1] = DT_<SDT>::to_f32((uint16_t)(v >> 16));
    } else {
      o[0] = DT_<SDT>::to_f32(p[0]);
    }
  }
}

template <int BITS, int XDT, int SDT, int MB, int GS, int S>
struct PCfg {
  static constexpr int Z = 128 / GS;                 // groups per segment
  static constexpr int SU = (16 / (Z * MB)) < S ? (16 / (Z * MB)) : S;  // segs per acc
  static constexpr int NB = S / SU;                  // accumulators per round
  static constexpr int NSLOT = SU * Z;               // (segment, half) slots used
  static constexpr int NG = MB >= 4 ? 1 : 4 / MB;    // groups per lane per acc
  static_assert(Z * MB <= 16, "x rows x group-halves must fit 16 MFMA rows");
  static_assert(S % SU == 0, "segments per round must fill whole accumulators");
};

// DX (direct x): the A fragments come straight from global memory into the
// round's registers (each lane loads the 32 x values of its own slot, the
// rest of its A operand is zero), so there is no x staging in LDS and no
// block barrier before the first MFMA; the group sums X come from one extra
// MFMA per accumulator and k-step against an all-ones B operand.
template <int BITS, int XDT, int SDT, int MB, int GS, int S, bool DX>
struct RoundRegs {
  using C = PCfg<BITS, XDT, SDT, MB, GS, S>;
  uint32_t wd[S][BITS];
  float sv[C::NB][C::NG], bv[C::NB][C::NG];
  u32x4 xv[DX ? C::NB : 1][DX ? 4 : 1];
};

template <int BITS, int XDT, int SDT, int MB, int GS, int S, bool DX, bool SWI>
__global__ __launch_bounds__(512) void qmvp_kernel(PKern a) {
  using C = PCfg<BITS, XDT, SDT, MB, GS, S>;
  using XS = st_t<XDT>;
  using SS = st_t<SDT>;
  constexpr int ODT = result_dtype(XDT, SDT);
  using OS = st_t<ODT>;
  using T = XMma<XDT>;
  using Regs = RoundRegs<BITS, XDT, SDT, MB, GS, S, DX>;
  constexpr float OFF = kExact8<BITS, XDT> ? 0.f : T::OFF;
  constexpr int Z = C::Z, SU = C::SU, NB = C::NB, NSLOT = C::NSLOT, NG = C::NG;

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int W = blockDim.x >> 6;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int M = a.M, N = a.N, K = a.K, R = a.R;
  const int Kp = K;                       // exact: K % 1024 == 0
  const int64_t P = (int64_t)(K >> 5) * BITS;
  const int64_t G = K / GS;

  // LDS: x rows [M][K] | 64 B of zeros | X sums [G][MB] | red [2][W][MB][16]
  // (| gate sums [MB][16] with SWI); with DX no x rows, zeros or X sums.
  const int zoff = DX ? 0 : M * xrow_bytes(K);
  float* Xs = reinterpret_cast<float*>(smem + zoff + 64);
  float* red = DX ? reinterpret_cast<float*>(smem) : Xs + G * MB;

  const int nl = lane & 15, q = lane >> 4;
  // A side: this lane supplies x row mA of slot sigA for k-block q.
  const int sigA = nl / MB, mA = nl % MB;
  const int uA = sigA / Z, hA = sigA % Z;
  const bool validA = (hA == q * Z / 4) && (mA < M) && (sigA < NSLOT);
  const int xlane = mA * xrow_bytes(K) + q * 64;
  // D side: values v = 0..3 of this lane are rows 4q + v.
  const int sig0 = (4 * q) / MB;          // slot of value 0
  const int gsig = sig0 < NSLOT ? sig0 : 0;  // clamped for loads
  const int md0 = MB >= 8 ? 4 * (q & 1) : 0;

  // The offset goes through a VGPR (a plain v_mov, no hazards) so that the
  // mask is the AND-OR's only scalar operand (gfx9 VOP3 reads at most one).
  const uint32_t mask_s = a.nib_mask;
  uint32_t off_v;
  asm("v_mov_b32 %0, %1" : "=v"(off_v) : "s"(a.off_pair));

  auto unpack = [&](const uint32_t (&wd)[BITS], int i) -> u32x4 {
    if constexpr (BITS == 4) {
      const uint32_t w = wd[i];
      u32x4 r;
      r[0] = (w & mask_s) | off_v;
      r[1] = ((w >> 4) & mask_s) | off_v;
      r[2] = ((w >> 8) & mask_s) | off_v;
      r[3] = ((w >> 12) & mask_s) | off_v;
      return r;
    } else {
      return unpack_step<BITS, XDT>(wd, i);
    }
  };

  // Item rr of a tile: half hf = rr / R (1 = up projection, SWI only),
  // round rr % R.
  auto issue = [&](Regs& r, int t, int rr) {
    const int hf = SWI ? (rr >= R ? 1 : 0) : 0;
    const int rnd = rr - hf * R;
    const int n = min(t * 16 + nl, N - 1);
    const int seg_base = (rnd * W + wv) * S;
    const uint32_t* wp = (hf ? a.w2 : a.w) + (int64_t)n * P + (int64_t)(seg_base * 4 + q) * BITS;
#pragma unroll
    for (int u = 0; u < S; u++) load_pack<BITS>(wp + u * 4 * BITS, r.wd[u]);
    const SS* sp = (const SS*)(hf ? a.s2 : a.s) + (int64_t)n * G + seg_base * Z + gsig;
    const SS* bp = (const SS*)(hf ? a.b2 : a.b) + (int64_t)n * G + seg_base * Z + gsig;
#pragma unroll
    for (int j = 0; j < NB; j++) {
      load_groups<SDT, NG>(sp + j * NSLOT, r.sv[j]);
      load_groups<SDT, NG>(bp + j * NSLOT, r.bv[j]);
    }
    if constexpr (DX) {
      // x[mA, seg * 128 + q * 32 .. + 31] of this lane's slot; lanes without
      // a slot load row 0 of the round's first segment and zero it later.
      const int mx = validA ? mA : 0, ux = validA ? uA : 0;
      const XS* xp = (const XS*)a.x + (int64_t)mx * K + (seg_base + ux) * 128 + q * 32;
#pragma unroll
      for (int j = 0; j < NB; j++)
#pragma unroll
        for (int i = 0; i < 4; i++)
          r.xv[j][i] = *reinterpret_cast<const u32x4*>(xp + j * SU * 128 + i * 8);
    }
  };

  float acc[4] = {0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const Regs& r, int rr) {
    const int rnd = SWI ? (rr >= R ? rr - R : rr) : rr;
    const int seg_base = (rnd * W + wv) * S;
#pragma unroll
    for (int j = 0; j < NB; j++) {
      // the one segment of this accumulator whose A rows this lane fills
      const int real = xlane + (seg_base + j * SU + uA) * 256;
      floatx4 d = {0.f, 0.f, 0.f, 0.f};
      u32x4 xa[4];
      if constexpr (DX) {
        // this lane's x in MFMA pair order (0,4,1,5,2,6,3,7), or zeros
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const u32x4 dd = r.xv[j][i];
          xa[i][0] = validA ? ((dd[0] & 0xffffu) | (dd[2] << 16)) : 0u;
          xa[i][1] = validA ? ((dd[0] >> 16) | (dd[2] & 0xffff0000u)) : 0u;
          xa[i][2] = validA ? ((dd[1] & 0xffffu) | (dd[3] << 16)) : 0u;
          xa[i][3] = validA ? ((dd[1] >> 16) | (dd[3] & 0xffff0000u)) : 0u;
        }
      }
#pragma unroll
      for (int uu = 0; uu < SU; uu++) {
        const int addr = (validA && uA == uu) ? real : zoff;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const u32x4 bw = unpack(r.wd[j * SU + uu], i);
          u32x4 av;
          if constexpr (DX) {
            const bool on = (uA == uu);
            av[0] = on ? xa[i][0] : 0u;
            av[1] = on ? xa[i][1] : 0u;
            av[2] = on ? xa[i][2] : 0u;
            av[3] = on ? xa[i][3] : 0u;
          } else {
            av = *reinterpret_cast<const u32x4*>(smem + addr + i * 16);
          }
          d = T::mma(__builtin_bit_cast(typename T::frag, av),
                     __builtin_bit_cast(typename T::frag, bw), d);
        }
      }
      floatx4 X;
      if constexpr (DX) {
        // X[row] = sum of that row's x over its group: A (every segment of
        // the accumulator at once: a lane feeds exactly one) times ones.
        constexpr uint32_t ONE2 = XDT == DT_BF16 ? 0x3F803F80u : 0x3C003C00u;
        const u32x4 ones = {ONE2, ONE2, ONE2, ONE2};
        X = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int i = 0; i < 4; i++)
          X = T::mma(__builtin_bit_cast(typename T::frag, xa[i]),
                     __builtin_bit_cast(typename T::frag, ones), X);
      } else {
        const int g0 = seg_base * Z + j * NSLOT + gsig;
        X = *reinterpret_cast<const floatx4*>(Xs + g0 * MB + md0);
      }
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const int gi = NG == 4 ? v : (NG == 2 ? v / 2 : 0);
        const float s = r.sv[j][gi];
        const float bo = fmaf(-OFF, s, r.bv[j][gi]);
        acc[v] = fmaf(s, d[v], fmaf(bo, X[v], acc[v]));
      }
    }
  };

  // Per-lane value v is x row (4q+v) % MB of slot (4q+v) / MB; slots past
  // NSLOT hold no segment and are dropped.
  float keep[4];
#pragma unroll
  for (int v = 0; v < 4; v++) keep[v] = ((4 * q + v) / MB < NSLOT) ? 1.f : 0.f;
  constexpr int MV = MB < 4 ? MB : 4;  // distinct x rows per lane

  auto finish_tile = [&](int t, int hf, int buf) {
    // 1) fold this lane's values onto its x rows, 2) sum over the lane groups
    //    that hold other slots of the same rows, 3) one LDS slot per wave.
    float part[MV];
#pragma unroll
    for (int j = 0; j < MV; j++) part[j] = 0.f;
#pragma unroll
    for (int v = 0; v < 4; v++) part[v % MV] += keep[v] * acc[v];
#pragma unroll
    for (int v = 0; v < 4; v++) acc[v] = 0.f;
    if constexpr (MB < 8) {
#pragma unroll
      for (int j = 0; j < MV; j++) {
        part[j] += __shfl_xor(part[j], 16, 64);
        part[j] += __shfl_xor(part[j], 32, 64);
      }
    } else {
#pragma unroll
      for (int j = 0; j < MV; j++) part[j] += __shfl_xor(part[j], 32, 64);
    }
    float* rb = red + buf * (W * 16 * MB);
    // rows held by lane group q after the folds: q == 0 has rows 0..MV-1; for
    // MB == 8, q == 1 has rows 4..7.
    if (q == 0 || (MB == 8 && q == 1)) {
#pragma unroll
      for (int j = 0; j < MV; j++) {
        const int m = (MB == 8 ? 4 * q : 0) + j;
        rb[(wv * MB + m) * 16 + nl] = part[j];
      }
    }
    __syncthreads();
    for (int e = tid; e < M * 16; e += blockDim.x) {
      const int m = e >> 4, n = e & 15;
      float sum = 0.f;
      for (int w2 = 0; w2 < W; w2++) sum += rb[(w2 * MB + m) * 16 + n];
      if constexpr (SWI) {
        // the same thread handles element e in the gate and the up finish
        float* gsum = red + 2 * W * 16 * MB;
        if (hf == 0) {
          gsum[e] = sum;
          continue;
        }
        sum = swiglu_f32(DT_<ODT>::round(gsum[e]), DT_<ODT>::round(sum));
      }
      if (t * 16 + n < N) ((OS*)a.y)[(int64_t)m * N + t * 16 + n] = linear_out<ODT>(sum, a.lb, t * 16 + n);
    }
  };

  Regs r0, r1;
  const int step = gridDim.x;
  int t = blockIdx.x, rnd = 0;

  // ---- stage x + group sums (all threads) ----
  // The first two x loads of every thread go out before the first round's
  // weight loads, so waiting for x does not wait for the weights (loads
  // complete in issue order).
  const XS* xb = (const XS*)a.x;
  const int cpr = K >> 3;              // 8-element chunks per x row
  const int items = M * cpr;           // multiple of 128 (K % 1024 == 0)
  auto xload = [&](int e) -> u32x4 {
    const int m = e / cpr, c = e - m * cpr;
    return *reinterpret_cast<const u32x4*>(xb + (int64_t)m * K + c * 8);
  };
  auto stage = [&](int e, const u32x4 d) {
    const int m = e / cpr, c = e - m * cpr;
    float sum = 0.f;
#pragma unroll
    for (int j = 0; j < 4; j++)
      sum += DT_<XDT>::to_f32((uint16_t)(d[j] & 0xffffu)) + DT_<XDT>::to_f32((uint16_t)(d[j] >> 16));
    u32x4 o;
    o[0] = (d[0] & 0xffffu) | (d[2] << 16);
    o[1] = (d[0] >> 16) | (d[2] & 0xffff0000u);
    o[2] = (d[1] & 0xffffu) | (d[3] << 16);
    o[3] = (d[1] >> 16) | (d[3] & 0xffff0000u);
    *reinterpret_cast<u32x4*>(smem + (size_t)m * xrow_bytes(K) + c * 16) = o;
    // GS/8 consecutive lanes hold one group
#pragma unroll
    for (int o2 = 1; o2 < GS / 8; o2 <<= 1) sum += __shfl_xor(sum, o2, 64);
    if ((c & (GS / 8 - 1)) == 0) Xs[(c / (GS / 8)) * MB + m] = sum;
  };
  const int bd = blockDim.x;
  if constexpr (DX) {
    issue(r0, t, 0);
  } else {
    u32x4 xd0 = {0u, 0u, 0u, 0u}, xd1 = {0u, 0u, 0u, 0u};
    if (tid < items) xd0 = xload(tid);
    if (tid + bd < items) xd1 = xload(tid + bd);
    issue(r0, t, 0);
    if (tid < items) stage(tid, xd0);
    if (tid + bd < items) stage(tid + bd, xd1);
    for (int e = tid + 2 * bd; e < items; e += bd) stage(e, xload(e));
    for (int e = tid; e < G * MB; e += bd)
      if ((e % MB) >= M) Xs[e] = 0.f;
    if (tid < 4) reinterpret_cast<u32x4*>(smem + zoff)[tid] = u32x4{0u, 0u, 0u, 0u};
    __syncthreads();
  }

  // items (t, rr) in order; buffers alternate, the next item's loads are
  // issued before the current item is computed
  const int RH = SWI ? 2 * R : R;
  int buf = 0;
  while (true) {
    if (t >= a.ntiles) break;
    int t1 = t, r1n = rnd + 1;
    if (r1n == RH) { r1n = 0; t1 += step; }
    if (t1 < a.ntiles) issue(r1, t1, r1n);
    compute(r0, rnd);
    if (rnd == R - 1 || rnd == RH - 1) { finish_tile(t, rnd >= R, buf); buf ^= 1; }
    t = t1; rnd = r1n;
    if (t >= a.ntiles) break;
    t1 = t; r1n = rnd + 1;
    if (r1n == RH) { r1n = 0; t1 += step; }
    if (t1 < a.ntiles) issue(r0, t1, r1n);
    compute(r1, rnd);
    if (rnd == R - 1 || rnd == RH - 1) { finish_tile(t, rnd >= R, buf); buf ^= 1; }
    t = t1; rnd = r1n;
  }
}

// ---------------------------------------------------------------------------
// Streaming decode GEMV for MB <= 8 rows of x (M <= MB) with x and scales of
// one 16-bit type: the decode case.
//
// A row tile is 16 output columns; a block takes TPB consecutive tiles. Each
// of its W waves owns RW S-segment (S*128-element) K ranges of every tile, so
// K = W * RW * S * 128; an item is one (tile, half, range), where the half is the
// gate or the up projection of the fused SwiGLU (SWI) and there is one half
// otherwise. A wave loads its x ranges, issues the weight and scale loads of
// all its items, stages its x in LDS in the MFMA pair order (waves stage only
// what they read, so no block barrier precedes the first MFMA), then computes
// the items in order. The A rows of one accumulator are the slots
// (segment u, group h, x row m) of SU segments (row (u*Z + h)*MB + m), as in
// the persistent kernel below. The group sums X of x come from one MFMA per
// k-step against an all-ones operand, so staging does no arithmetic. With
// W > 1 the partial sums of a tile meet in LDS after one barrier
// (double-buffered slots, fixed order). Loads of a tile past the last one read
// the last tile again (never computed): the issue code stays straight, so
// waiting for one tile's loads does not wait for the next's.
// ---------------------------------------------------------------------------
// Whether the streaming kernel loads every x chunk before the weights, at
// addresses without a clamp: it then needs M == MB exactly.
template <int MB, int S>
constexpr bool kXPre = MB <= 2 || (S == 4 && (MB == 4 || MB == 8));

struct SKern {
  void* y;
  const void* x;
  const uint32_t* w;
  const void* s;
  const void* b;
  const uint32_t* w2;  // SWI: up projection (gate is w/s/b)
  const void* s2;
  const void* b2;
  int M, N, K;
  int ntiles;   // ceil(N / TR)
  uint32_t nib_mask, off_pair;
  const void* lb;  // linear bias [N] or null (not with SwiGLU)
};

// TR: W rows per tile, 16, or 8 to spread few W rows over more blocks (the
// MFMA's other 8 columns repeat them and are not stored).
template <int BITS, int XDT, int GS, int MB, int TPB, int RW, bool SWI, bool SPLIT, int S, bool XF,
          int TR = 16>
__global__ __launch_bounds__(512) void qmvs_kernel(SKern a) {
  static_assert(S == 4 || S == 8, "a K range is 512 or 1024 elements");  // S: segments per range
  constexpr int H = SWI ? 2 : 1;                     // halves (gate, up)
  constexpr int NI = TPB * H * RW;                   // items per wave
  constexpr int Z = 128 / GS;                        // groups per segment
  constexpr int SU = (16 / (Z * MB)) < S ? 16 / (Z * MB) : S;  // segments per accumulator
  constexpr int NB = S / SU;                         // accumulators per range
  constexpr int NSLOT = SU * Z;                      // (segment, group) slots used
  constexpr int NG = MB >= 4 ? 1 : 4 / MB;           // groups per lane per accumulator
  constexpr int MV = MB < 4 ? MB : 4;                // x rows per lane
  static_assert(Z * MB <= 16 && S % SU == 0, "slots must fit 16 MFMA rows");
  using T = XMma<XDT>;
  using XS = st_t<XDT>;
  using frag = typename T::frag;
  constexpr float OFF = kExact8<BITS, XDT> ? 0.f : T::OFF;

  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int W = blockDim.x >> 6;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int M = a.M, N = a.N, K = a.K;
  const int64_t P = (int64_t)(K >> 5) * BITS;  // words per weight row
  const int G = K / GS;                        // groups per row
  // LDS: x [M][K] in pair order | 64 B of zeros | red [2][W][MB][16] floats
  const int zoff = M * xrow_bytes(K);
  float* red = reinterpret_cast<float*>(smem + zoff + 64);

  const int nl = lane & 15, q = lane >> 4;
  // A side: A row nl is slot sigA = (segment uA, group hA) of x row mA; the
  // lane feeds k-block q of that segment when the block lies in group hA.
  const int sigA = nl / MB, mA = nl % MB;
  const int uA = sigA / Z, hA = sigA % Z;
  const bool validA = (hA == q * Z / 4) && (sigA < NSLOT) && (mA < M);
  // D side: value v of this lane is row 4q + v = slot (4q + v) / MB, x row
  // (4q + v) % MB; the lane's groups start at slot gsig.
  const int gsig = (4 * q) / MB < NSLOT ? (4 * q) / MB : 0;
  float keep[4];
#pragma unroll
  for (int v = 0; v < 4; v++) keep[v] = ((4 * q + v) / MB < NSLOT) ? 1.f : 0.f;

  const uint32_t mask_s = a.nib_mask;
  uint32_t off_v;
  asm("v_mov_b32 %0, %1" : "=v"(off_v) : "s"(a.off_pair));

  using SV = typename std::conditional<NG == 4, u32x2, typename std::conditional<NG == 2, uint32_t, uint16_t>::type>::type;
  struct Item {
    uint32_t wd[S][BITS];
    SV sv[NB], bv[NB];  // NG consecutive 16-bit scales / biases per accumulator
  };
  // item i: tile t0 + i / (H*RW), half (i / RW) % H, range wv*RW + i % RW
  auto issue = [&](Item& r, int t, int h, int seg_base) {
    const int n = min(t * TR + (nl & (TR - 1)), N - 1);
    const uint32_t* wp = (h ? a.w2 : a.w) + (int64_t)n * P + (int64_t)(seg_base * 4 + q) * BITS;
#pragma unroll
    for (int u = 0; u < S; u++) load_pack<BITS>(wp + u * 4 * BITS, r.wd[u]);
    const XS* sp = (const XS*)(h ? a.s2 : a.s) + (int64_t)n * G + seg_base * Z + gsig;
    const XS* bp = (const XS*)(h ? a.b2 : a.b) + (int64_t)n * G + seg_base * Z + gsig;
#pragma unroll
    for (int jb = 0; jb < NB; jb++) {
      r.sv[jb] = *reinterpret_cast<const SV*>(sp + jb * NSLOT);
      r.bv[jb] = *reinterpret_cast<const SV*>(bp + jb * NSLOT);
    }
  };

  // ---- x of this wave's K ranges, the weight loads of all items, then x
  // into LDS in pair order. With kXPre (the launcher then requires M == MB)
  // every x chunk of the wave (S / 4 per lane per range and row) is loaded
  // before the weights, at addresses that need no clamp, so the wait before
  // storing them covers only these loads; otherwise the rows are loaded after
  // the weights. ----
  const int seg0 = wv * RW * S;  // first segment of this wave's ranges
  constexpr int xch = RW * S * 16;  // 16-byte chunks per x row in the ranges
  constexpr int XPRE = kXPre<MB, S> ? (S / 4) * RW * MB : 0;
  auto xsrc = [&](int c) {  // chunk c = m * xch + j of the ranges
    const int m = c / xch, j = c - m * xch;
    return reinterpret_cast<const u32x4*>((const XS*)a.x + (int64_t)m * K + (int64_t)seg0 * 128 + j * 8);
  };
  auto xstore = [&](int c, const u32x4 d) {
    const int m = c / xch, j = c - m * xch;
    u32x4 o;
    o[0] = (d[0] & 0xffffu) | (d[2] << 16);
    o[1] = (d[0] >> 16) | (d[2] & 0xffff0000u);
    o[2] = (d[1] & 0xffffu) | (d[3] << 16);
    o[3] = (d[1] >> 16) | (d[3] & 0xffff0000u);
    *reinterpret_cast<u32x4*>(smem + (size_t)m * xrow_bytes(K) + seg0 * 256 + j * 16) = o;
  };
  u32x4 xr[XPRE > 0 ? XPRE : 1];
#pragma unroll
  for (int c = 0; c < XPRE; c++) xr[c] = *xsrc(lane + 64 * c);
  const int t0 = blockIdx.x * TPB;
  Item it[NI];
#pragma unroll
  for (int i = 0; i < NI; i++)
    issue(it[i], min(t0 + i / (H * RW), a.ntiles - 1), (i / RW) % H, seg0 + (i % RW) * S);
#pragma unroll
  for (int c = 0; c < XPRE; c++) xstore(lane + 64 * c, xr[c]);
  for (int c = lane + 64 * XPRE; c < M * xch; c += 64) xstore(c, *xsrc(c));
  if (lane < 4) reinterpret_cast<u32x4*>(smem + zoff)[lane] = u32x4{0u, 0u, 0u, 0u};

  constexpr uint32_t ONE2 = XDT == DT_BF16 ? 0x3F803F80u : 0x3C003C00u;
  const u32x4 ones = {ONE2, ONE2, ONE2, ONE2};
  const int xrowA = (validA ? mA : 0) * xrow_bytes(K);

  // Adds one item (K range starting at segment seg_base) to the 4 values per
  // lane.
  auto compute = [&](const Item& r, int seg_base, float (&acc)[4]) {
#pragma unroll
    for (int jb = 0; jb < NB; jb++) {
      const int real = validA ? xrowA + (seg_base + jb * SU + uA) * 256 + q * 64 : zoff;
      floatx4 d0 = {0.f, 0.f, 0.f, 0.f}, d1 = {0.f, 0.f, 0.f, 0.f};
      floatx4 X = {0.f, 0.f, 0.f, 0.f};
      // group sums: the lane's own x (or zeros) times ones. With XF they go
      // first, while the item's weights are still arriving (4096 x 4096,
      // 512-element ranges: 4.50 -> 4.22 us); for large N that order measured
      // slower (14336 x 4096: 8.86 -> 10.07 us at M = 1, 9.5 -> 10.5 us at
      // M = 2), so there they go last.
      auto group_sums = [&]() {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const u32x4 xa = *reinterpret_cast<const u32x4*>(smem + real + i * 16);
          X = T::mma(__builtin_bit_cast(frag, xa), __builtin_bit_cast(frag, ones), X);
        }
      };
      if constexpr (XF) group_sums();
      if constexpr (SU >= 2) {
        // two accumulator chains (even / odd segments) so consecutive MFMAs
        // do not wait for each other; segments are unpacked two at a time
#pragma unroll
        for (int uu = 0; uu < SU; uu += 2) {
          u32x4 av[2][4], bw[2][4];
#pragma unroll
          for (int e = 0; e < 2; e++) {
            const int addr = (uA == uu + e) ? real : zoff;
#pragma unroll
            for (int i = 0; i < 4; i++) av[e][i] = *reinterpret_cast<const u32x4*>(smem + addr + i * 16);
          }
#pragma unroll
          for (int e = 0; e < 2; e++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
              if constexpr (BITS == 4) {
                const uint32_t w = r.wd[jb * SU + uu + e][i];
                bw[e][i][0] = (w & mask_s) | off_v;
                bw[e][i][1] = ((w >> 4) & mask_s) | off_v;
                bw[e][i][2] = ((w >> 8) & mask_s) | off_v;
                bw[e][i][3] = ((w >> 12) & mask_s) | off_v;
              } else {
                bw[e][i] = unpack_step<BITS, XDT>(r.wd[jb * SU + uu + e], i);
              }
            }
#pragma unroll
          for (int i = 0; i < 4; i++) {
            d0 = T::mma(__builtin_bit_cast(frag, av[0][i]), __builtin_bit_cast(frag, bw[0][i]), d0);
            d1 = T::mma(__builtin_bit_cast(frag, av[1][i]), __builtin_bit_cast(frag, bw[1][i]), d1);
          }
        }
      } else {
        // one segment per accumulator: the two chains are its k-step halves
        u32x4 av[4], bw[4];
#pragma unroll
        for (int i = 0; i < 4; i++) av[i] = *reinterpret_cast<const u32x4*>(smem + real + i * 16);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          if constexpr (BITS == 4) {
            const uint32_t w = r.wd[jb][i];
            bw[i][0] = (w & mask_s) | off_v;
            bw[i][1] = ((w >> 4) & mask_s) | off_v;
            bw[i][2] = ((w >> 8) & mask_s) | off_v;
            bw[i][3] = ((w >> 12) & mask_s) | off_v;
          } else {
            bw[i] = unpack_step<BITS, XDT>(r.wd[jb], i);
          }
        }
#pragma unroll
        for (int i = 0; i < 4; i += 2) {
          d0 = T::mma(__builtin_bit_cast(frag, av[i]), __builtin_bit_cast(frag, bw[i]), d0);
          d1 = T::mma(__builtin_bit_cast(frag, av[i + 1]), __builtin_bit_cast(frag, bw[i + 1]), d1);
        }
      }
      if constexpr (!XF) group_sums();
      float sv[NG], bv[NG];
      if constexpr (NG == 4) {
        const u32x2 sp = r.sv[jb], bp = r.bv[jb];
        sv[0] = DT_<XDT>::to_f32((uint16_t)(sp[0] & 0xffffu));
        sv[1] = DT_<XDT>::to_f32((uint16_t)(sp[0] >> 16));
        sv[2] = DT_<XDT>::to_f32((uint16_t)(sp[1] & 0xffffu));
        sv[3] = DT_<XDT>::to_f32((uint16_t)(sp[1] >> 16));
        bv[0] = DT_<XDT>::to_f32((uint16_t)(bp[0] & 0xffffu));
        bv[1] = DT_<XDT>::to_f32((uint16_t)(bp[0] >> 16));
        bv[2] = DT_<XDT>::to_f32((uint16_t)(bp[1] & 0xffffu));
        bv[3] = DT_<XDT>::to_f32((uint16_t)(bp[1] >> 16));
      } else if constexpr (NG == 2) {
        sv[0] = DT_<XDT>::to_f32((uint16_t)(r.sv[jb] & 0xffffu));
        sv[1] = DT_<XDT>::to_f32((uint16_t)(r.sv[jb] >> 16));
        bv[0] = DT_<XDT>::to_f32((uint16_t)(r.bv[jb] & 0xffffu));
        bv[1] = DT_<XDT>::to_f32((uint16_t)(r.bv[jb] >> 16));
      } else {
        sv[0] = DT_<XDT>::to_f32(r.sv[jb]);
        bv[0] = DT_<XDT>::to_f32(r.bv[jb]);
      }
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const int gi = NG == 4 ? v : (NG == 2 ? v / 2 : 0);
        const float bo = fmaf(-OFF, sv[gi], bv[gi]);
        acc[v] = fmaf(sv[gi], d0[v] + d1[v], fmaf(bo, X[v], acc[v]));
      }
    }
  };

  // Column totals of one half of a tile for every x row: this wave's part,
  // summed over the block's waves in a fixed order (LDS slots, one barrier).
  // Thread e < M*16 of the block gets row e / 16, column e % 16.
  int buf = 0;
  auto reduce = [&](const float (&acc)[4]) -> float {
    float part[MV];
#pragma unroll
    for (int j = 0; j < MV; j++) part[j] = 0.f;
#pragma unroll
    for (int v = 0; v < 4; v++) part[v % MV] = fmaf(keep[v], acc[v], part[v % MV]);
#pragma unroll
    for (int j = 0; j < MV; j++) {
      if constexpr (MB < 8) part[j] += __shfl_xor(part[j], 16, 64);
      part[j] += __shfl_xor(part[j], 32, 64);
    }
    float* rb = red + buf * (W * MB * 16);
    if (q == 0 || (MB == 8 && q == 1)) {
#pragma unroll
      for (int j = 0; j < MV; j++) {
        const int m = (MB == 8 ? 4 * q : 0) + j;
        rb[(wv * MB + m) * 16 + nl] = part[j];
      }
    }
    if constexpr (SPLIT) __syncthreads();
    buf ^= 1;
    float sum = 0.f;
    if (tid < M * 16) {
      const int m = tid >> 4, n = tid & 15;
      for (int w2 = 0; w2 < W; w2++) sum += rb[(w2 * MB + m) * 16 + n];
    }
    return sum;
  };

#pragma unroll
  for (int tt = 0; tt < TPB; tt++) {
    const int t = t0 + tt;
    if (t < a.ntiles) {  // block-uniform
      float hs[H];
#pragma unroll
      for (int h = 0; h < H; h++) {
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int rr = 0; rr < RW; rr++) compute(it[(tt * H + h) * RW + rr], seg0 + rr * S, acc);
        hs[h] = reduce(acc);
      }
      float o = hs[0];
      if constexpr (SWI) o = swiglu_f32(DT_<XDT>::round(hs[0]), DT_<XDT>::round(hs[1]));
      if (tid < M * 16 && (tid & 15) < TR && t * TR + (tid & 15) < N) {
        const int n = t * TR + (tid & 15);
        ((st_t<XDT>*)a.y)[(int64_t)(tid >> 4) * N + n] =
            SWI ? DT_<XDT>::from_f32(o) : linear_out<XDT>(o, a.lb, n);
      }
    }
  }
}

// Launches the streaming kernel: K / (RW * 1024) waves per block, TPB tiles
// per block.
template <int XDT, int GS, int MB, int TPB, int RW, bool SWI, int S = 8, bool XF = false>
hipError_t run_qmvs(const QArgs& a) {
  const int W = (int)(a.K / (128 * S * RW));
  if (a.K % (128 * S * RW) != 0 || W < 2 || W > 8 || a.M > MB) return hipErrorNotSupported;
  if (kXPre<MB, S> && a.M != MB) return hipErrorNotSupported;
  const size_t lds = (size_t)a.M * xrow_bytes((int)a.K) + 64 + (size_t)2 * W * MB * 16 * 4;
  if (lds > 160 * 1024) return hipErrorNotSupported;
  SKern k;
  k.y = a.y; k.x = a.x; k.w = a.w; k.s = a.s; k.b = a.b;
  k.w2 = a.w2; k.s2 = a.s2; k.b2 = a.b2;
  k.M = (int)a.M; k.N = (int)a.N; k.K = (int)a.K;
  k.nib_mask = 0x000F000Fu;
  k.off_pair = XMma<XDT>::OFFB;
  k.lb = a.lb;
  // 8-row tiles at 4 and 8 x rows when 16-row tiles would occupy at most a
  // quarter of the CUs (k/v, 1024 x 4096: 128 blocks of 8 rows instead of 64
  // of 16: 4.61 -> 4.36 us at 4 rows, 5.93 -> 5.12 us at 8; at 1 row it was
  // slower, 3.76 -> 3.85 us)
  bool half = false;
  if constexpr (MB >= 4 && TPB == 1 && !SWI) half = (a.N + 15) / 16 <= device_cu_count() / 4;
  const int tr = half ? 8 : 16;
  k.ntiles = (int)((a.N + tr - 1) / tr);
  const int grid = (k.ntiles + TPB - 1) / TPB;
  auto fn = qmvs_kernel<HQ_BITS, XDT, GS, MB, TPB, RW, SWI, true, S, XF, 16>;
  if constexpr (MB >= 4 && TPB == 1 && !SWI) {
    if (half) fn = qmvs_kernel<HQ_BITS, XDT, GS, MB, TPB, RW, SWI, true, S, XF, 8>;
  }
  if (lds > 64 * 1024) {
    // one flag per kernel (the 8- and 16-row forms are separate functions)
    static std::atomic<uint64_t> raised16{0}, raised8{0};
    hipError_t e = raise_lds_limit(reinterpret_cast<const void*>(fn), 160 * 1024, half ? raised8 : raised16);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(fn, dim3(grid), dim3(64 * W), lds, a.stream, k);
  return hipGetLastError();
}

// Bytes of LDS one block of the persistent kernel uses.
inline size_t qmvp_lds(const QArgs& a, int W, int MB, int GS, bool dx, bool swi) {
  const size_t red = (size_t)2 * W * 16 * MB * 4 + (swi ? (size_t)MB * 16 * 4 : 0);
  if (dx) return red;
  return (size_t)a.M * xrow_bytes((int)a.K) + 64 + (size_t)(a.K / GS) * MB * 4 + red;
}

// Blocks per CU: as many as LDS and registers keep resident at once (up to
// 4), so every block's tiles stream concurrently. Returns the grid size.
inline int qmvp_grid(int ntiles, size_t lds, int vgprs, int W) {
  const int waves_per_simd = vgprs <= 128 ? 4 : (vgprs <= 168 ? 3 : (vgprs <= 256 ? 2 : 1));
  int per_cu = (int)((160 * 1024) / lds);
  if (per_cu > 4) per_cu = 4;
  if (per_cu > (4 * waves_per_simd) / W) per_cu = (4 * waves_per_simd) / W;
  if (per_cu < 1) per_cu = 1;
  const int maxb = per_cu * device_cu_count();
  const int per = (ntiles + maxb - 1) / maxb;
  return (ntiles + per - 1) / per;
}

template <int XDT, int SDT, int MB, int GS, int S, bool DX, bool SWI>
int qmvp_vgprs() {
  // a property of the code object (the same on every gfx950 device)
  static std::atomic<int> vg{0};
  int v = vg.load(std::memory_order_relaxed);
  if (v == 0) {
    hipFuncAttributes fa;
    auto fn = qmvp_kernel<HQ_BITS, XDT, SDT, MB, GS, S, DX, SWI>;
    v = (hipFuncGetAttributes(&fa, reinterpret_cast<const void*>(fn)) == hipSuccess && fa.numRegs > 0)
            ? fa.numRegs : 128;
    vg.store(v, std::memory_order_relaxed);
  }
  return v;
}

// Launches the persistent kernel with W waves per block and R rounds per
// tile, or returns hipErrorNotSupported when x does not fit LDS.
template <int XDT, int SDT, int MB, int GS, int S, bool DX, bool SWI>
hipError_t run_qmvp_s(const QArgs& a, int W, int R) {
  using C = PCfg<HQ_BITS, XDT, SDT, MB, GS, S>;
  const size_t lds = qmvp_lds(a, W, MB, GS, DX, SWI);
  if (lds > 160 * 1024) return hipErrorNotSupported;
  PKern k;
  k.y = a.y; k.x = a.x; k.w = a.w; k.s = a.s; k.b = a.b;
  k.M = (int)a.M; k.N = (int)a.N; k.K = (int)a.K; k.R = R;
  k.nib_mask = 0x000F000Fu;
  k.off_pair = XMma<XDT>::OFFB;
  k.w2 = a.w2; k.s2 = a.s2; k.b2 = a.b2;
  k.lb = a.lb;
  const int ntiles = (int)((a.N + 15) / 16);
  k.ntiles = ntiles;
  auto fn = qmvp_kernel<HQ_BITS, XDT, SDT, MB, GS, S, DX, SWI>;
  const int grid = qmvp_grid(ntiles, lds, qmvp_vgprs<XDT, SDT, MB, GS, S, DX, SWI>(), W);
  static std::atomic<uint64_t> raised{0};
  if (lds > 64 * 1024) {
    hipError_t e = raise_lds_limit(reinterpret_cast<const void*>(fn), 160 * 1024, raised);
    if (e != hipSuccess) return e;
  }
  (void)sizeof(C);
  hipLaunchKernelGGL(fn, dim3(grid), dim3(64 * W), lds, a.stream, k);
  return hipGetLastError();
}

// Direct x only where the round buffers stay within registers: per buffer a
// lane holds NB * 4 x fragments (16 VGPRs each accumulator), S * BITS weight
// words and 2 * NB * NG scale/bias values; two buffers and ~50 more VGPRs
// must fit 256.
template <int MB, int GS, int S>
constexpr bool kDirectOk = PCfg<HQ_BITS, DT_BF16, DT_BF16, MB, GS, S>::NB * 16 + S * HQ_BITS +
                               2 * PCfg<HQ_BITS, DT_BF16, DT_BF16, MB, GS, S>::NB *
                                   PCfg<HQ_BITS, DT_BF16, DT_BF16, MB, GS, S>::NG <= 100;

// Staged x is loaded once per block and reused by every tile the block
// walks; direct x is reloaded per tile but needs no LDS and no barrier
// before the first MFMA. Direct x is used when x does not fit LDS, or for
// M >= 2 when every block gets one tile both ways (direct x holds more
// registers, which can lower the blocks per CU). At M = 1 staging measured
// as fast or faster on every Llama-3-8B decode shape.
template <int XDT, int SDT, int MB, int GS, int S, bool SWI>
hipError_t run_qmvp_sd(const QArgs& a, int W, int R) {
  if constexpr (kDirectOk<MB, GS, S>) {
    const size_t lds = qmvp_lds(a, W, MB, GS, false, SWI);
    const int ntiles = (int)((a.N + 15) / 16);
    if (lds > 160 * 1024 ||
        (a.M >= 2 &&
         qmvp_grid(ntiles, lds, qmvp_vgprs<XDT, SDT, MB, GS, S, false, SWI>(), W) >= ntiles &&
         qmvp_grid(ntiles, qmvp_lds(a, W, MB, GS, true, SWI),
                   qmvp_vgprs<XDT, SDT, MB, GS, S, true, SWI>(), W) >= ntiles))
      return run_qmvp_s<XDT, SDT, MB, GS, S, true, SWI>(a, W, R);
  }
  return run_qmvp_s<XDT, SDT, MB, GS, S, false, SWI>(a, W, R);
}

template <int XDT, int SDT, int MB, int GS, bool SWI>
hipError_t run_qmvp(const QArgs& a) {
  constexpr int Z = 128 / GS;
  if constexpr (Z * MB > 16) {
    return hipErrorNotSupported;
  } else {
    if (a.K % 1024 != 0) return hipErrorNotSupported;
    const int nseg = (int)(a.K / 128);
    const int ntiles = (int)((a.N + 15) / 16);
    // S = 8 segments per round and W <= 8 waves with W * 8 dividing nseg.
    // Rounds of S = 4 instead (measured on the Llama-3-8B shapes at M = 1):
    // - when that leaves fewer than 8 waves per tile and tiles are few (small
    //   N): up to twice the waves per tile, or the same waves in twice the
    //   rounds (K = 14336: 11.0 against 11.35 us);
    // - when blocks walk many tiles (the vocabulary projection): 56.8 against
    //   59.5 us;
    // - for x that does not fit LDS when direct x at S = 8 would spill.
    auto pick = [&](int S) {
      for (int c = 8; c >= 1; c--)
        if ((nseg / S) % c == 0) return c;
      return 0;
    };
    const int W8 = pick(8), W4 = pick(4);
    if ((W8 < 8 && ntiles <= 512 && W4 >= W8) || (ntiles >= 16 * device_cu_count() && W4 == 8))
      return run_qmvp_sd<XDT, SDT, MB, GS, 4, SWI>(a, W4, nseg / (4 * W4));
    if (W8 == 0) return hipErrorNotSupported;
    if (!kDirectOk<MB, GS, 8> && qmvp_lds(a, W8, MB, GS, false, SWI) > 160 * 1024)
      return run_qmvp_sd<XDT, SDT, MB, GS, 4, SWI>(a, W4, nseg / (4 * W4));
    return run_qmvp_sd<XDT, SDT, MB, GS, 8, SWI>(a, W8, nseg / (8 * W8));
  }
}

template <int XDT, int SDT, int MB, int GS>
hipError_t run_qmvx(const QArgs& a) {
  QXKern k;
  k.y = a.y; k.x = a.x; k.w = a.w; k.s = a.s; k.b = a.b;
  k.lhs = a.lhs; k.rhs = a.rhs;
  k.batch = a.batch; k.x_rep = a.x_rep; k.x_batch = a.x_batch; k.w_batch = a.w_batch;
  k.M = (int)a.M; k.N = (int)a.N; k.K = (int)a.K;
  k.lb = a.lb;
  constexpr int RPH = MB <= 4 ? 4 : 8;
  constexpr int Z = 128 / GS;
  const int kpad = (int)((a.K + 127) / 128 * 128);
  // x chunk: at most ~40 KB of bf16 rows (+ zero row) so two blocks fit a CU.
  int kc = (40960 / ((int)a.M + 1)) / 128 * 128;
  if (kc < 128) kc = 128;
  if (kc > kpad) kc = kpad;
  k.KC = kc;
  const int nseg = kc / 128;
  int W = (nseg + kU - 1) / kU;
  if (W > 16) W = 16;
  if (W < 1) W = 1;
  k.S = (nseg + W - 1) / W;
  const size_t lds = (size_t)(a.M + 1) * xrow_bytes(kc) + (size_t)(kc / GS) * RPH * 4 +
                     (size_t)W * Z * a.M * 16 * 4;
  dim3 grid((unsigned)((a.N + 15) / 16), (unsigned)(a.batch < 65535 ? a.batch : 65535));
  auto fn = qmvx_kernel<HQ_BITS, XDT, SDT, MB, GS>;
  static std::atomic<uint64_t> raised{0};  // opt-in to > 64 KB once per device
  if (lds > 64 * 1024) {
    hipError_t e = raise_lds_limit(reinterpret_cast<const void*>(fn), 160 * 1024, raised);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(fn, grid, dim3(64 * W), lds, a.stream, k);
  return hipGetLastError();
}

// x and scales of one 16-bit type, K a multiple of 1024 above 2048, one or
// two rows of x (four or eight at K <= 4096): the streaming kernel, one K
// range per wave (two 1024-element ranges per wave above K = 8192), one tile
// per block (two for vocabulary-sized N at M = 1). Measured at M = 1 on the
// Llama-3-8B decode shapes (4-bit g64, graph of distinct weight copies)
// against the persistent kernel below, with 1024-element ranges: 4096 x 4096
// 4.66 vs 5.03 us, 14336 x 4096 8.77 vs 9.82 us, 128256 x 4096 54.8 vs
// 68.9 us; at K = 2048 the persistent kernel stays (8192 x 2048: 4.67 vs
// 4.90 us).
template <int XDT, int GS, int MB, bool SWI>
hipError_t run_qmvs_auto(const QArgs& a) {
  // Llama-3-8B step: B = 2 1.53 ms (1.63 with 1024-element ranges, 1.91 on
  // the persistent kernel); with 512-element ranges at K = 4096 (down stays
  // on the persistent kernel) B = 4 1.93 vs 2.34 ms and B = 8 2.69 vs
  // 3.20 ms. With 1024-element ranges the 4- and 8-row forms were slower
  // than the persistent kernel (2.80 vs 2.33, 3.63 vs 3.22 ms).
  if constexpr ((128 / GS) * MB > 16) {
    return hipErrorNotSupported;
  } else {
    if (a.K % 1024 != 0 || a.K <= 2048) return hipErrorNotSupported;
    const int64_t ntiles = (a.N + 15) / 16;
    const int kr = (int)(a.K / 1024);
    // 512-element K ranges (twice the waves, half the work left per wave
    // when its last weights land) at K <= 4096 for several x rows, and for one
    // row at N <= 4096; group sums first at N <= 4096. Several rows need
    // M == MB (the launcher checks it).
    const bool small_n = ntiles <= 256;
    if (kr <= 4 && (small_n || MB >= 2)) {
      // 8 rows at vocabulary-sized N measured slower here than on the
      // persistent kernel (128256 x 4096: 118.4 vs 111.0 us)
      if (MB == 8 && ntiles >= 2048) return hipErrorNotSupported;
      return small_n ? run_qmvs<XDT, GS, MB, 1, 1, SWI, 4, true>(a) : run_qmvs<XDT, GS, MB, 1, 1, SWI, 4>(a);
    }
    if constexpr (MB >= 4) {
      // K > 4096 at 4 and 8 rows stays on the persistent kernel (4 rows,
      // 14336: two 1024-element ranges per wave 18.9 vs 15.0 us)
      return hipErrorNotSupported;
    } else {
      if (kr <= 8) {
        if constexpr (!SWI && MB == 1) {
          if (ntiles >= 2048) return run_qmvs<XDT, GS, MB, 2, 1, false>(a);
        }
        return run_qmvs<XDT, GS, MB, 1, 1, SWI>(a);
      }
      if (kr % 2 == 0 && kr <= 16) return run_qmvs<XDT, GS, MB, 1, 2, SWI>(a);
      return hipErrorNotSupported;
    }
  }
}

template <int XDT, int SDT, int MB, int GS, bool SWI>
hipError_t run_qmvx_any(const QArgs& a) {
  const bool single = a.batch == 1 && !a.lhs && !a.rhs;
  if constexpr (XDT == SDT) {
    if (single) {
      hipError_t e = run_qmvs_auto<XDT, GS, MB, SWI>(a);
      if (e != hipErrorNotSupported) return e;
    }
  }
  if constexpr (SWI) {
    // fused SwiGLU: one product (batch 1, K % 1024 == 0)
    if (!single) return hipErrorNotSupported;
    return run_qmvp<XDT, SDT, MB, GS, true>(a);
  } else {
    if (single) {
      hipError_t e = run_qmvp<XDT, SDT, MB, GS, false>(a);
      if (e != hipErrorNotSupported) return e;
    }
    return run_qmvx<XDT, SDT, MB, GS>(a);
  }
}

template <int XDT, int SDT, int MB, bool SWI>
hipError_t run_qmvx_g(const QArgs& a) {
  switch (a.group_size) {
    case 32: return run_qmvx_any<XDT, SDT, MB, 32, SWI>(a);
    case 64: return run_qmvx_any<XDT, SDT, MB, 64, SWI>(a);
    default: return run_qmvx_any<XDT, SDT, MB, 128, SWI>(a);
  }
}

template <int XDT, int SDT, bool SWI = false>
hipError_t run_qmvx_m(const QArgs& a) {
  if (a.M <= 1) return run_qmvx_g<XDT, SDT, 1, SWI>(a);
  if (a.M <= 2) return run_qmvx_g<XDT, SDT, 2, SWI>(a);
  if (a.M <= 4) return run_qmvx_g<XDT, SDT, 4, SWI>(a);
  return run_qmvx_g<XDT, SDT, 8, SWI>(a);
}

}  // namespace

#define HQ_CAT_(a, b) a##b
#define HQ_CAT(a, b) HQ_CAT_(a, b)

hipError_t HQ_CAT(launch_qmvx_t_b, HQ_BITS)(const QArgs& a) {
  // 8 rows of 4-bit weights with many output tiles, plain or with the fused
  // SwiGLU: the streaming kernel's dense form (hq_gqms.hip)
  const hipError_t ed = HQ_CAT(launch_gqms_dense_t_b, HQ_BITS)(a);
  if (ed != hipErrorNotSupported) return ed;
  if (a.w2) {
    // fused SwiGLU: x and scales of one 16-bit dtype
    if (a.xdt == DT_BF16 && a.sdt == DT_BF16) return run_qmvx_m<DT_BF16, DT_BF16, true>(a);
    if (a.xdt == DT_F16 && a.sdt == DT_F16) return run_qmvx_m<DT_F16, DT_F16, true>(a);
    return hipErrorNotSupported;
  }
  switch (a.xdt * 3 + a.sdt) {
    case DT_BF16 * 3 + DT_BF16: return run_qmvx_m<DT_BF16, DT_BF16>(a);
    case DT_BF16 * 3 + DT_F16: return run_qmvx_m<DT_BF16, DT_F16>(a);
    case DT_BF16 * 3 + DT_F32: return run_qmvx_m<DT_BF16, DT_F32>(a);
    case DT_F16 * 3 + DT_F16: return run_qmvx_m<DT_F16, DT_F16>(a);
    case DT_F16 * 3 + DT_BF16: return run_qmvx_m<DT_F16, DT_BF16>(a);
    case DT_F16 * 3 + DT_F32: return run_qmvx_m<DT_F16, DT_F32>(a);
    default: return hipErrorInvalidValue;  // fp32 x uses the VALU kernel
  }
}

}  // namespace hq
