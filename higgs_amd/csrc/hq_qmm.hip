// hq_qmm.hip -- quantized GEMM for prefill (M > 8), one bit width (HQ_BITS).
//
// y = x . deq(W)^T (mlx-rs ops::quantized_matmul, transpose=true, as called
// from crates/higgs-models/src/qwen3_next.rs:218-227 and the Llama
// MaybeQuantized layers, crates/higgs-models/src/transformer.rs:257-259).
//
// Each 256-thread block computes a BM x BN tile of y. Per K step the block
// stages the x tile in LDS (converted to the compute type) and dequantizes the
// W tile straight into LDS as s*q+b rounded to the compute type, so the MFMA
// operands never leave the chip. Compute type: bf16 (16x16x32 bf16 MFMA) for
// bf16 x and scales, fp16 likewise, fp32 (16x16x4 fp32 MFMA) otherwise, all
// with fp32 accumulation. Gathered batches (gather_qmm with M > 8) use
// blockIdx.z.
#include <algorithm>
#include <type_traits>

#include "hq_common.hpp"
#include "hq_device.hpp"
#include "hq_kernels.hpp"

#ifndef HQ_BITS
#error "compile with -DHQ_BITS=<2|3|4|5|6|8>"
#endif

namespace hq {

struct QKernM {
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

template <int CT> struct Mma;
template <> struct Mma<DT_BF16> {
  static constexpr int KW = 32, E = 8, BK = 64, PAD = 8;
  using lds_t = uint16_t;
  using frag = bf16x8;
  static __device__ __forceinline__ floatx4 mma(frag a, frag b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t cvt(float v) { return f32_to_bf16_bits(v); }
};
template <> struct Mma<DT_F16> {
  static constexpr int KW = 32, E = 8, BK = 64, PAD = 8;
  using lds_t = uint16_t;
  using frag = f16x8;
  static __device__ __forceinline__ floatx4 mma(frag a, frag b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t cvt(float v) { return f32_to_f16_bits(v); }
};
template <> struct Mma<DT_F32> {
  static constexpr int KW = 4, E = 1, BK = 32, PAD = 4;
  using lds_t = float;
  using frag = float;
  static __device__ __forceinline__ floatx4 mma(frag a, frag b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

constexpr int BM = 128, BN = 128;

template <int BITS, int XDT, int SDT>
__global__ __launch_bounds__(256) void qmm_t_kernel(QKernM a) {
  constexpr int CT = (XDT == SDT && XDT != DT_F32) ? XDT : DT_F32;
  constexpr int ODT = result_dtype(XDT, SDT);
  using T = Mma<CT>;
  using L = typename T::lds_t;
  using XS = st_t<XDT>;
  using SS = st_t<SDT>;
  using OS = st_t<ODT>;
  constexpr int BK = T::BK;
  constexpr int LD = BK + T::PAD;  // LDS row stride in elements
  constexpr int A_CHUNKS = BM * BK / 8 / 256;    // 8-element chunks per thread
  constexpr int B_PACKS = BN * BK / 32;          // 32-element packs per stage
  __shared__ __attribute__((aligned(16))) L As[BM * LD];
  __shared__ __attribute__((aligned(16))) L Bs[BN * LD];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int wm = wv >> 1, wn = wv & 1;
  const int M = a.M, N = a.N, K = a.K;
  const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
  const int64_t P = (int64_t)(K >> 5) * BITS;
  const int64_t G = K >> a.gshift;
  const int gsp = a.gshift - 5;

  for (int64_t bi = blockIdx.z; bi < a.batch; bi += gridDim.z) {
    const int64_t xi = a.lhs ? (int64_t)a.lhs[bi] : bi / a.x_rep;
    const int64_t wi = a.rhs ? (int64_t)a.rhs[bi] : 0;
    OS* yb = (OS*)a.y + bi * (int64_t)M * N;
    const bool bad = xi >= a.x_batch || wi >= a.w_batch;
    const XS* xb = (const XS*)a.x + (bad ? 0 : xi) * (int64_t)M * K;
    const uint32_t* wb = a.w + (bad ? 0 : wi) * (int64_t)N * P;
    const SS* sb = (const SS*)a.s + (bad ? 0 : wi) * (int64_t)N * G;
    const SS* bb = (const SS*)a.b + (bad ? 0 : wi) * (int64_t)N * G;

    floatx4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    for (int k0 = 0; k0 < K && !bad; k0 += BK) {
      // ---- stage x tile (BM x BK) ----
#pragma unroll
      for (int c = 0; c < A_CHUNKS; c++) {
        const int chunk = tid + c * 256;
        const int row = chunk / (BK / 8), kc = chunk % (BK / 8);
        const int gm = m0 + row, gk = k0 + kc * 8;
        L* dst = &As[row * LD + kc * 8];
        if (gm < M && gk < K) {
          const XS* src = xb + (int64_t)gm * K + gk;
          if constexpr (CT == XDT && CT != DT_F32) {
            *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(src);
          } else {
            float v[8];
            load8_f32<XDT>(src, v);
            if constexpr (CT == DT_F32) {
#pragma unroll
              for (int e = 0; e < 8; e++) dst[e] = v[e];
            } else {
              u32x4 h;
#pragma unroll
              for (int e = 0; e < 4; e++) h[e] = T::cvt(v[2 * e]) | (T::cvt(v[2 * e + 1]) << 16);
              *reinterpret_cast<u32x4*>(dst) = h;
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; e++) dst[e] = (L)0;
        }
      }
      // ---- dequantize W tile (BN x BK) ----
      for (int pk = tid; pk < B_PACKS; pk += 256) {
        const int row = pk / (BK / 32), pc = pk % (BK / 32);
        const int gn = n0 + row, gk = k0 + pc * 32;
        L* dst = &Bs[row * LD + pc * 32];
        if (gn < N && gk < K) {
          uint32_t wd[BITS];
          load_pack<BITS>(wb + (int64_t)gn * P + (int64_t)(gk >> 5) * BITS, wd);
          const int64_t gi = (int64_t)gn * G + ((gk >> 5) >> gsp);
          const float sv = DT_<SDT>::load(sb, gi), bv = DT_<SDT>::load(bb, gi);
          if constexpr (CT == DT_F32) {
#pragma unroll
            for (int e = 0; e < 32; e++) dst[e] = fmaf(sv, (float)pack_elem<BITS>(wd, e), bv);
          } else {
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
              u32x4 h;
#pragma unroll
              for (int e = 0; e < 4; e++) {
                const int i0 = q4 * 8 + 2 * e;
                h[e] = T::cvt(fmaf(sv, (float)pack_elem<BITS>(wd, i0), bv)) |
                       (T::cvt(fmaf(sv, (float)pack_elem<BITS>(wd, i0 + 1), bv)) << 16);
              }
              *reinterpret_cast<u32x4*>(dst + q4 * 8) = h;
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < 32; e++) dst[e] = (L)0;
        }
      }
      __syncthreads();
      // ---- MFMA over the stage ----
#pragma unroll
      for (int ks = 0; ks < BK / T::KW; ks++) {
        typename T::frag fa[4], fb[4];
        const int kofs = ks * T::KW + (lane >> 4) * T::E;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const L* pa = &As[(wm * 64 + i * 16 + (lane & 15)) * LD + kofs];
          const L* pb = &Bs[(wn * 64 + i * 16 + (lane & 15)) * LD + kofs];
          if constexpr (CT == DT_F32) {
            fa[i] = *pa;
            fb[i] = *pb;
          } else {
            fa[i] = __builtin_bit_cast(typename T::frag, *reinterpret_cast<const u32x4*>(pa));
            fb[i] = __builtin_bit_cast(typename T::frag, *reinterpret_cast<const u32x4*>(pb));
          }
        }
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
          for (int j = 0; j < 4; j++) acc[i][j] = T::mma(fa[i], fb[j], acc[i][j]);
      }
      __syncthreads();
    }
    // ---- epilogue ----
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
          const int gm = m0 + wm * 64 + i * 16 + (lane >> 4) * 4 + v;
          const int gn = n0 + wn * 64 + j * 16 + (lane & 15);
          if (gm < M && gn < N) {
            const float o = bad ? __uint_as_float(0x7fc00000u) : acc[i][j][v];
            yb[(int64_t)gm * N + gn] = linear_out<ODT>(o, a.lb, gn);
          }
        }
  }
}

// ---------------------------------------------------------------------------
// Large-tile GEMM for one product with 16-bit x and scales of the same type
// (the prefill case): 256 x 256 output tile per 256-thread block, K-step 64.
// The W tile is dequantized once per K-step into LDS as CT = round(s*q + b),
// x is copied into LDS, both double-buffered: the global loads of step k+1
// are in flight while the MFMAs of step k run. Each wave owns a 128 x 128
// quarter of the tile as 8 x 8 fragments of v_mfma_f32_16x16x32 (fp32
// accumulators). The MFMA computes the transposed product D[n][m] (A = W rows,
// B = x rows) so every lane ends with 4 consecutive n of one m: 8-byte stores.
// With KS > 1 a block holds KS such wave groups, each with its own LDS buffers
// and one contiguous K / KS slice of the tile's K steps (split-K inside the
// block, for products with too few tiles to give every CU enough waves); the
// groups' accumulators meet in LDS and group 0 adds them in group order.
// ---------------------------------------------------------------------------
namespace {

constexpr int GBM = 256, GBN = 256, GBK = 64;

// Tile shapes of the large-tile GEMM: a block computes TN W rows x TM x rows
// with WAVES waves of WN x WM each (times KS wave groups with split-K). The
// id is the template key: 256 x 256 and 224 x 256 (8 waves, one block per
// CU; 224 leaves the last 32 threads without a W row), 256 x 128 (id 384, 8
// waves), 128 x 128 (4 waves), 96 x 128 (id 96), 64 x 128 (id 192) and
// 64 x 64; run_qgemm picks one by its cost model.
template <int SZ> struct GTile;
template <> struct GTile<256> {
  static constexpr int TN = 256, TM = 256, WAVES = 8, WN = 128, WM = 64;
};
template <> struct GTile<224> {
  static constexpr int TN = 224, TM = 256, WAVES = 8, WN = 112, WM = 64;
};
template <> struct GTile<384> {
  static constexpr int TN = 256, TM = 128, WAVES = 8, WN = 64, WM = 64;
};
template <> struct GTile<96> {
  static constexpr int TN = 96, TM = 128, WAVES = 4, WN = 48, WM = 64;
};
template <> struct GTile<192> {
  static constexpr int TN = 64, TM = 128, WAVES = 4, WN = 32, WM = 64;
};
template <> struct GTile<128> {
  static constexpr int TN = 128, TM = 128, WAVES = 4, WN = 64, WM = 64;
};
template <> struct GTile<64> {
  static constexpr int TN = 64, TM = 64, WAVES = 2, WN = 32, WM = 64;
};
constexpr int GLD = GBK + 16;  // LDS row stride (elements): 160 B (fewest bank conflicts measured)

// Least common multiple of two ring depths and 2 (the LDS buffer count): the
// unrolled group in which every ring slot and LDS buffer is a compile-time index.
constexpr int ring_group(int a, int b) {
  int x = a, y = b;
  while (y) { const int t = x % y; x = y; y = t; }
  const int l = a / x * b;
  return l % 2 ? 2 * l : l;
}

struct GKern {
  void* y;
  const void* x;
  const uint32_t* w;
  const void* s;
  const void* b;
  int M, N, K;
  const uint32_t* w2;  // SwiGLU up projection (gate is w/s/b), N rows
  const void* s2;
  const void* b2;
  const void* lb;      // linear bias [N] or null (not with SwiGLU)
};

template <int CT>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (CT == DT_BF16) {
    typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
    bf2 v;
    v[0] = (__bf16)lo;
    v[1] = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, v);
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    h2 v;
    v[0] = (_Float16)lo;
    v[1] = (_Float16)hi;
    return __builtin_bit_cast(uint32_t, v);
  }
}

// Eight consecutive elements (pack quarter qq) of a 32-element pack,
// dequantized to CT as round(s * q + b), as four packed pairs. For 4 bits the
// even and odd nibbles of the word are masked to bytes once, so each element
// costs one v_cvt_f32_ubyteN, one FMA and half a v_cvt_pk.
template <int BITS, int CT>
__device__ __forceinline__ u32x4 deq8(const uint32_t (&wd)[BITS], int qq, float s, float b) {
  u32x4 h;
  if constexpr (BITS == 4) {
    const uint32_t w = wd[qq];
    uint32_t ev = w & 0x0F0F0F0Fu, od = (w >> 4) & 0x0F0F0F0Fu;
    // Opaque to the optimizer: otherwise it folds the masks into per-element
    // bit-field extracts (v_bfe_u32 + v_cvt_f32_ubyte0, two instructions per
    // element instead of one v_cvt_f32_ubyteN; 15 % of the 4-bit GEMM loop).
    asm("" : "+v"(ev), "+v"(od));
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float q0 = (float)((ev >> (8 * e)) & 0xffu);  // element 2e
      const float q1 = (float)((od >> (8 * e)) & 0xffu);  // element 2e + 1
      h[e] = pack2<CT>(fmaf(s, q0, b), fmaf(s, q1, b));
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int i0 = qq * 8 + 2 * e;
      h[e] = pack2<CT>(fmaf(s, (float)pack_elem<BITS>(wd, i0), b),
                       fmaf(s, (float)pack_elem<BITS>(wd, i0 + 1), b));
    }
  }
  return h;
}

// SWI: the TN W rows of a tile are TN/2 output columns of the gate and the
// same columns of the up projection, arranged so that a wave's fragments
// i < NI/2 are gate rows and i + NI/2 the matching up rows; the epilogue
// writes swiglu(gate, up) for TN/2 columns from registers.
template <int BITS, int CT, int GS, bool SWI, int SZ, int KS>
__global__ __launch_bounds__(GTile<SZ>::WAVES * 64 * KS) void qgemm_kernel(GKern a) {
  using T = Mma<CT>;
  using ST = st_t<CT>;
  using TL = GTile<SZ>;
  constexpr int GBN = TL::TN, GBM = TL::TM, NT = TL::WAVES * 64;  // NT: threads per K group
  constexpr int NI = TL::WN / 16, NJ = TL::WM / 16;  // fragments per wave in n, m
  extern __shared__ __attribute__((aligned(16))) unsigned char gsm[];
  // K group kg: threads kg*NT.., LDS buffers [2][GBN][GLD] (W) then [2][GBM][GLD] (x)
  const int kg = KS > 1 ? (int)threadIdx.x / NT : 0;
  uint16_t* As = reinterpret_cast<uint16_t*>(gsm) + kg * (2 * (GBN + GBM) * GLD);
  uint16_t* Bs = As + 2 * GBN * GLD;

  const int tid = (int)threadIdx.x - kg * NT, lane = tid & 63, wv = tid >> 6;
  // wave owns n rows wn*WN.., m rows wm*WM..
  const int wn = wv / (GBM / TL::WM), wm = wv % (GBM / TL::WM);
  const int M = a.M, N = a.N, K = a.K;
  // XCD-aware tile order: consecutive block ids go to different XCDs (8 on
  // MI355X), so tile t is given to block id (t % per) * 8 + t / per; each XCD
  // then walks a contiguous, M-major range of tiles and keeps its x rows in
  // its own L2 while the W tiles stream past.
  constexpr int ONT = SWI ? GBN / 2 : GBN;  // output columns per tile
  const int ntn = (N + ONT - 1) / ONT;
  const int ntiles = ntn * ((M + GBM - 1) / GBM);
  int t = blockIdx.x;
  if ((ntiles & 7) == 0) {
    const int per = ntiles >> 3;
    t = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  }
  const int n0 = (t % ntn) * ONT, m0 = (t / ntn) * GBM;
  const int64_t P = (int64_t)(K >> 5) * BITS;
  const int64_t G = K / GS;
  const ST* xg = (const ST*)a.x;

  // x tile (GBM x 64): thread copies rows xr + (NT/8)j (j < XJ), 16-byte
  // chunk xc. Rows past M read row M-1 (never stored), so every load is
  // unconditional.
  constexpr int XJ = GBM / (NT / 8);
  const int xr = tid >> 3, xc = tid & 7;
  static_assert(GBM == XJ * (NT / 8) && GBN <= NT / 2, "thread maps cover the tiles");
  static_assert(!SWI || NI % 2 == 0, "SwiGLU pairs gate and up fragments");
  // W tile (GBN x 64): thread dequantizes pack wp of row wr. A tile of fewer
  // than NT / 2 rows (224) leaves the last threads without a row: they load
  // the tile's last row (a cache hit) and store nothing.
  const int wr = tid >> 1, wp = tid & 1;
  const bool w_row = GBN == NT / 2 || wr < GBN;
  uint32_t xoff[XJ];  // element offsets into x (the launcher checks M*K < 2^31)
#pragma unroll
  for (int j = 0; j < XJ; j++)
    xoff[j] = (uint32_t)min(m0 + xr + (NT / 8) * j, M - 1) * (uint32_t)K + xc * 8;
  // SWI: tile row wr is column n0 + (wr / WN) * WN/2 + wr % (WN/2) of the gate
  // (wr % WN < WN/2) or of the up projection.
  constexpr int HW = TL::WN / 2;
  const bool w_up = SWI && (wr % TL::WN) >= HW;
  const int wn_row = min(SWI ? n0 + (wr / TL::WN) * HW + (wr % HW) : n0 + min(wr, GBN - 1), N - 1);
  const uint32_t woff = (uint32_t)((int64_t)wn_row * P) + wp * BITS;
  const uint32_t goff = (uint32_t)((int64_t)wn_row * G);
  const uint32_t* wg = w_up ? a.w2 : a.w;
  const ST* sg = (const ST*)(w_up ? a.s2 : a.s);
  const ST* bg = (const ST*)(w_up ? a.b2 : a.b);

  // Register rings, indexed by compile-time slots inside an unrolled group of
  // kG steps: x of step kt + kRD and W of step kt + kWD are loaded at the end
  // of step kt. x reaches LDS at the end of step kt + kRD - 1, after kRD - 1
  // steps of MFMAs; W is dequantized into LDS from the start of step
  // kt + kWD - 1, so it has kWD - 2 steps of cover. (Rotating registers by
  // copies instead would make every copy wait for the loads just issued.)
  // x depth 2 with whole groups free of branches measured fastest (M = 2048
  // gate/up 300 -> 287 us, fused SwiGLU 561 -> 524 us, M = 256 and 512 2-6 %
  // faster); the 128 x 128 tile without split-K keeps depth 3 and per-step
  // tests, which hold it at two waves per SIMD (depth 2 unbranched took it
  // to one: down 337 -> 347 us). The 64 x 128 and 96 x 128 split-K tiles
  // give W a third slot (M = 512 4096 x 4096 38.8 -> 35.9 us, 4096 x 14336
  // 130 -> 119, M = 127 14336 x 4096 40.6 -> 38.1, M = 512 6144 x 2048
  // 27.3 -> 26.9); the 64 x 64 and 128 x 128 split-K tiles measured 2-5 %
  // slower with it (their steps are bound by the dequantization VALU and
  // the shared barrier, not by the W loads).
  constexpr int kRD = (SZ == 128 && KS == 1) ? 3 : 2;
  constexpr int kWD = (SZ == 192 || SZ == 96) && KS > 1 ? kRD + 1 : kRD;
  constexpr int kG = ring_group(kRD, kWD);
  using SV = std::conditional_t<(kWD > kRD), uint32_t, uint16_t>;

  // Scale and bias stay raw 16-bit values in the ring and are widened where
  // they are used: widening at the load makes the compiler wait for that load
  // at once. (With the deeper W ring they sit zero-extended in 32-bit slots,
  // so no zero-extension of its own gets placed ahead of their use.)
  struct WPre {
    uint32_t wd[BITS];
    SV sv, bv;
  };
  auto wload = [&](WPre& p, int k0) {
    load_pack<BITS>(wg + woff + (uint32_t)(k0 >> 5) * BITS, p.wd);
    const uint32_t gi = goff + (uint32_t)((k0 + wp * 32) / GS);
    p.sv = sg[gi];
    p.bv = bg[gi];
  };
  // Quarter qq (8 elements) of this thread's pack, one 16-byte LDS store.
  auto wchunk = [&](const WPre& p, float sf, float bf, int buf, int qq) {
    uint16_t* dst = As + buf * GBN * GLD + wr * GLD + wp * 32 + qq * 8;
    const u32x4 v = deq8<BITS, CT>(p.wd, qq, sf, bf);
    if (w_row) *reinterpret_cast<u32x4*>(dst) = v;
  };


  floatx4 acc[NI][NJ];
#pragma unroll
  for (int i = 0; i < NI; i++)
#pragma unroll
    for (int j = 0; j < NJ; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // MFMAs of one K-step on LDS buffer `buf`, with the dequantization of the
  // next step's W (registers `wn_`) threaded between them into `buf ^ 1`.
  auto step = [&](int buf, const WPre& wn_) {
    const uint16_t* as = As + buf * GBN * GLD;
    const uint16_t* bs = Bs + buf * GBM * GLD;
    // With the deeper W ring, scale and bias are widened here, where this
    // step first uses them: the empty volatile asm keeps the compiler from
    // widening them next to their loads (which makes it wait for those loads
    // there, kWD - 1 steps early).
    float sf = 0.f, bf = 0.f;
    if constexpr (kWD > kRD) {
      uint32_t sraw = wn_.sv, braw = wn_.bv;
      asm volatile("" : "+v"(sraw), "+v"(braw));
      sf = DT_<CT>::to_f32((uint16_t)sraw);
      bf = DT_<CT>::to_f32((uint16_t)braw);
    }
#pragma unroll
    for (int ks = 0; ks < GBK / 32; ks++) {
      const int kofs = ks * 32 + (lane >> 4) * 8;
      typename T::frag fb[NJ];
#pragma unroll
      for (int j = 0; j < NJ; j++)
        fb[j] = __builtin_bit_cast(typename T::frag, *reinterpret_cast<const u32x4*>(
                                                         bs + (wm * TL::WM + j * 16 + (lane & 15)) * GLD + kofs));
#pragma unroll
      for (int i = 0; i < NI; i++) {
        const typename T::frag fa = __builtin_bit_cast(
            typename T::frag,
            *reinterpret_cast<const u32x4*>(as + (wn * TL::WN + i * 16 + (lane & 15)) * GLD + kofs));
#pragma unroll
        for (int j = 0; j < NJ; j++) acc[i][j] = T::mma(fa, fb[j], acc[i][j]);
        if (i % ((NI + 1) / 2) == 0) {
          const int qq = ks * 2 + i / ((NI + 1) / 2);
          if constexpr (kWD > kRD) wchunk(wn_, sf, bf, buf ^ 1, qq);
          else wchunk(wn_, DT_<CT>::to_f32(wn_.sv), DT_<CT>::to_f32(wn_.bv), buf ^ 1, qq);
        }
      }
    }
  };

  const int nk = K / (GBK * KS);   // K steps of this group (the launcher checks KS | K / GBK)
  const int kb = kg * nk * GBK;    // first K element of this group's slice
  WPre wr_[kWD];
  u32x4 xr_[kRD][XJ];
  auto xload_to = [&](u32x4 (&d)[XJ], int k0) {
#pragma unroll
    for (int j = 0; j < XJ; j++) d[j] = *reinterpret_cast<const u32x4*>(xg + xoff[j] + k0);
  };
  auto xstore_from = [&](const u32x4 (&d)[XJ], int buf) {
    uint16_t* bs = Bs + buf * GBM * GLD;
#pragma unroll
    for (int j = 0; j < XJ; j++)
      *reinterpret_cast<u32x4*>(bs + (xr + (NT / 8) * j) * GLD + xc * 8) = d[j];
  };
  if constexpr (kWD > kRD) {
    // Prologue loads in the loop's own order (x of a step, then W of the
    // step kWD - kRD later), pinned against reordering: the loop header's
    // waits are merged over the prologue and the loop's back edge, so a
    // different order here would make every group's first step wait for
    // more loads.
    wload(wr_[0], kb);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int d = 0; d < kRD || d + 1 < kWD; d++) {
      if (d < kRD) xload_to(xr_[d], kb + min(d, nk - 1) * GBK);
      if (d + 1 < kWD) wload(wr_[d + 1], kb + min(d + 1, nk - 1) * GBK);
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
#pragma unroll
    for (int d = 0; d < kRD; d++) {
      xload_to(xr_[d], kb + min(d, nk - 1) * GBK);
      wload(wr_[d], kb + min(d, nk - 1) * GBK);
    }
  }
#pragma unroll
  for (int c = 0; c < 4; c++)
    wchunk(wr_[0], DT_<CT>::to_f32((uint16_t)wr_[0].sv), DT_<CT>::to_f32((uint16_t)wr_[0].bv), 0, c);
  xstore_from(xr_[0], 0);
  __syncthreads();
  // One K step at position dd of a group (ring slots dd % kRD and dd % kWD,
  // LDS buffer dd & 1).
  auto kstep = [&](int kt, int dd) {
    const int buf = dd & 1;
    step(buf, wr_[(dd + 1) % kWD]);
    xstore_from(xr_[(dd + 1) % kRD], buf ^ 1);
    // past the end: reload the last step (unused)
    xload_to(xr_[dd % kRD], kb + min(kt + kRD, nk - 1) * GBK);
    wload(wr_[dd % kWD], kb + min(kt + kWD, nk - 1) * GBK);
    __syncthreads();
  };
  if constexpr (kRD % 2 == 0) {
    // Whole groups of kG steps run with no branch between their steps (a
    // load issued under a branch makes the compiler drain every load in
    // flight at the join); the steps of a last partial group are tested one
    // by one.
    int kt0 = 0;
    for (; kt0 + kG <= nk; kt0 += kG) {
#pragma unroll
      for (int dd = 0; dd < kG; dd++) kstep(kt0 + dd, dd);
    }
#pragma unroll
    for (int dd = 0; dd < kG - 1; dd++)
      if (kt0 + dd < nk) kstep(kt0 + dd, dd);
  } else {
    for (int kt0 = 0; kt0 < nk; kt0 += kG) {
#pragma unroll
      for (int dd = 0; dd < kG; dd++)
        if (kt0 + dd < nk) kstep(kt0 + dd, dd);
    }
  }
  if constexpr (KS > 1) {
    // groups 1.. leave their accumulators in LDS (every group has passed the
    // last barrier of the K loop, so the staging buffers are free); group 0
    // adds them in group order and runs the epilogue
    floatx4* red = reinterpret_cast<floatx4*>(gsm);
    if (kg > 0) {
#pragma unroll
      for (int i = 0; i < NI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
          red[((((kg - 1) * TL::WAVES + wv) * NI + i) * NJ + j) * 64 + lane] = acc[i][j];
    }
    __syncthreads();
    if (kg > 0) return;
#pragma unroll
    for (int g = 1; g < KS; g++)
#pragma unroll
      for (int i = 0; i < NI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++) {
          const floatx4 o = red[((((g - 1) * TL::WAVES + wv) * NI + i) * NJ + j) * 64 + lane];
#pragma unroll
          for (int v = 0; v < 4; v++) acc[i][j][v] += o[v];
        }
  }

  // epilogue: acc[i][j][v] = y[m][n], n = n0 + wn*WN + i*16 + 4*(lane>>4) + v,
  // m = m0 + wm*WM + j*16 + (lane & 15)
  ST* yg = (ST*)a.y;
  if constexpr (SWI) {
    // acc[i] gate and acc[i + NI/2] up of column n0 + wn*WN/2 + i*16 + 4*(lane>>4) + v
#pragma unroll
    for (int i = 0; i < NI / 2; i++) {
      const int n = n0 + wn * HW + i * 16 + 4 * (lane >> 4);
#pragma unroll
      for (int j = 0; j < NJ; j++) {
        const int m = m0 + wm * TL::WM + j * 16 + (lane & 15);
        if (m >= M) continue;
        float h[4];
#pragma unroll
        for (int v = 0; v < 4; v++)
          h[v] = swiglu_f32(DT_<CT>::round(acc[i][j][v]), DT_<CT>::round(acc[i + NI / 2][j][v]));
        if (n + 3 < N) {
          u32x2 o;
          o[0] = pack2<CT>(h[0], h[1]);
          o[1] = pack2<CT>(h[2], h[3]);
          *reinterpret_cast<u32x2*>(yg + (int64_t)m * N + n) = o;
        } else {
#pragma unroll
          for (int v = 0; v < 4; v++)
            if (n + v < N) yg[(int64_t)m * N + n + v] = DT_<CT>::from_f32(h[v]);
        }
      }
    }
    return;
  }
  if (a.lb != nullptr) {
    // linear bias: round the product, add the bias, round again
    const ST* lb = (const ST*)a.lb;
#pragma unroll
    for (int i = 0; i < NI; i++) {
      const int n = n0 + wn * TL::WN + i * 16 + 4 * (lane >> 4);
      float bv[4];
#pragma unroll
      for (int v = 0; v < 4; v++) bv[v] = DT_<CT>::to_f32(lb[min(n + v, N - 1)]);
#pragma unroll
      for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int v = 0; v < 4; v++) acc[i][j][v] = DT_<CT>::round(acc[i][j][v]) + bv[v];
    }
  }
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int n = n0 + wn * TL::WN + i * 16 + 4 * (lane >> 4);
#pragma unroll
    for (int j = 0; j < NJ; j++) {
      const int m = m0 + wm * TL::WM + j * 16 + (lane & 15);
      if (m >= M) continue;
      if (n + 3 < N) {
        u32x2 o;
        o[0] = pack2<CT>(acc[i][j][0], acc[i][j][1]);
        o[1] = pack2<CT>(acc[i][j][2], acc[i][j][3]);
        *reinterpret_cast<u32x2*>(yg + (int64_t)m * N + n) = o;
      } else {
#pragma unroll
        for (int v = 0; v < 4; v++)
          if (n + v < N) yg[(int64_t)m * N + n + v] = DT_<CT>::from_f32(acc[i][j][v]);
      }
    }
  }
}

template <int CT, int GS, bool SWI, int SZ, int KS>
hipError_t run_qgemm_sz(const QArgs& a) {
  using TL = GTile<SZ>;
  static_assert((size_t)KS * 2 * (TL::TN + TL::TM) * GLD * 2 <= 160 * 1024, "LDS per block");
  static_assert((size_t)(KS - 1) * TL::TN * TL::TM * 4 <= (size_t)KS * 2 * (TL::TN + TL::TM) * GLD * 2,
                "split-K partial sums fit the staging buffers");
  if ((a.K / GBK) % KS != 0) return hipErrorNotSupported;
  GKern k;
  k.y = a.y; k.x = a.x; k.w = a.w; k.s = a.s; k.b = a.b;
  k.M = (int)a.M; k.N = (int)a.N; k.K = (int)a.K;
  k.w2 = a.w2; k.s2 = a.s2; k.b2 = a.b2;
  k.lb = a.lb;
  auto fn = qgemm_kernel<HQ_BITS, CT, GS, SWI, SZ, KS>;
  const size_t lds = (size_t)KS * 2 * (TL::TN + TL::TM) * GLD * 2;
  static std::atomic<uint64_t> raised{0};
  {
    hipError_t e = raise_lds_limit(reinterpret_cast<const void*>(fn), (int)lds, raised);
    if (e != hipSuccess) return e;
  }
  const int ont = SWI ? TL::TN / 2 : TL::TN;
  const unsigned ntiles = (unsigned)(((a.N + ont - 1) / ont) * ((a.M + TL::TM - 1) / TL::TM));
  hipLaunchKernelGGL(fn, dim3(ntiles), dim3(TL::WAVES * 64 * KS), lds, a.stream, k);
  return hipGetLastError();
}

// Tile choice by a cost model: the CU that runs the most tiles sets the
// time, so cost = ceil(tiles / CUs) x (MFMA work of a tile) / (throughput of
// that tile form relative to the 256 x 256 tile); the cheapest form runs.
// The relative throughputs were fitted to same-box measurements on random
// 4-bit g64 data, and the model picks the fastest measured form on every one
// of them (us, chosen form first): Llama-3-8B gate/up 14336 x 4096 at
// M = 2048 224x256 252-256 vs 256x256 265; M = 1024 224x256 127-134 vs
// 256x128 171; M = 256 128/2 54-56 vs 64x128/2 76, 96/2 89; down
// 4096 x 14336 at M = 1024 128/2 180 vs 128/1 235, 256x128 267; M = 512
// 64x128/2 126 vs 96/2 150, 128/2 164; q/o 4096 x 4096 at M = 1024 128/2
// 53 vs 128/1 71; M = 512 64x128/2 39 vs 96/2 47, 64/4 48; M = 127 at
// 14336 x 4096 64x128/2 39 vs 64/2 46; configs[3] gate/up 96/2 26.5 vs
// 128/2 28.7; configs[3] down 64/4 36 vs 64/2 49; the fused gate/up +
// SwiGLU (2 x 14336 x 4096) at M = 512 256x256 141 vs 256x128 176, M = 256
// 256x128 90 vs 128/1 100, M = 64 64/2 50 vs 128/2 56, M = 768 256x128 253
// vs 256x256 263. (x/y: K split over y wave groups inside the block;
// 256x128 is id 384, 64x128 id 192.) A 128 x 128 tile without split-K has
// 4 waves: it keeps up only with a second block on the CU. The SwiGLU form
// has no 224 x 256 or 96 x 128 tiles (its gate and up fragments pair up).
template <int CT, int GS, bool SWI>
hipError_t run_qgemm(const QArgs& a) {
  const int cus = device_cu_count();
  auto tiles2 = [&](int64_t tn, int64_t tm) {
    const int64_t ont = SWI ? tn / 2 : tn;
    return ((a.N + ont - 1) / ont) * ((a.M + tm - 1) / tm);
  };
  auto tiles = [&](int64_t t) { return tiles2(t, t); };
  const int64_t steps = a.K / GBK;
  enum { C256, C224, C384, C128x2, C128x1, C96x2, C192x2, C64x4, C64x2, C64x1 };
  double best = 0.0;
  int pick = -1;
  auto consider = [&](int c, int64_t t, double work, double eff, bool ok) {
    if (!ok) return;
    const double cost = (double)((t + cus - 1) / cus) * work / eff;
    if (pick < 0 || cost < best) {
      best = cost;
      pick = c;
    }
  };
  const int64_t t128 = tiles(128), t64 = tiles(64);
  consider(C256, tiles(256), 65536, 1.00, true);
  consider(C224, tiles2(224, 256), 57344, 0.91, !SWI);
  consider(C384, tiles2(256, 128), 32768, 0.78, true);
  consider(C128x2, t128, 16384, 0.58, steps % 2 == 0);
  consider(C128x1, t128, 16384, t128 > cus ? 0.69 : 0.44, true);
  consider(C96x2, tiles2(96, 128), 12288, 0.47, !SWI && steps % 2 == 0);
  consider(C192x2, tiles2(64, 128), 8192, 0.37, steps % 2 == 0);
  consider(C64x4, t64, 4096, 0.30, steps % 4 == 0);
  consider(C64x2, t64, 4096, t64 > cus ? 0.32 : 0.20, steps % 2 == 0);
  consider(C64x1, t64, 4096, 0.16, true);
  switch (pick) {
    case C256: return run_qgemm_sz<CT, GS, SWI, 256, 1>(a);
    case C224:
      if constexpr (!SWI) return run_qgemm_sz<CT, GS, SWI, 224, 1>(a);
      break;
    case C384: return run_qgemm_sz<CT, GS, SWI, 384, 1>(a);
    case C128x2: return run_qgemm_sz<CT, GS, SWI, 128, 2>(a);
    case C128x1: return run_qgemm_sz<CT, GS, SWI, 128, 1>(a);
    case C96x2:
      if constexpr (!SWI) return run_qgemm_sz<CT, GS, SWI, 96, 2>(a);
      break;
    case C192x2: return run_qgemm_sz<CT, GS, SWI, 192, 2>(a);
    case C64x4: return run_qgemm_sz<CT, GS, SWI, 64, 4>(a);
    case C64x2: return run_qgemm_sz<CT, GS, SWI, 64, 2>(a);
    default: break;
  }
  return run_qgemm_sz<CT, GS, SWI, 64, 1>(a);
}

template <int CT, bool SWI = false>
hipError_t run_qgemm_g(const QArgs& a) {
  switch (a.group_size) {
    case 32: return run_qgemm<CT, 32, SWI>(a);
    case 64: return run_qgemm<CT, 64, SWI>(a);
    default: return run_qgemm<CT, 128, SWI>(a);
  }
}

// ---------------------------------------------------------------------------
// Grouped GEMM for gather_qmm with sorted expert indices (the MoE global-sort
// path: SwitchMlpWeights::forward_gather_global_sort, crates/higgs-models/src/
// qwen3_next.rs:1731-1809, calls gather_qmm with sorted_indices = true).
// Block (nt, e) owns W rows nt*128.. of expert e. It finds the run of batch
// elements whose rhs index is e (two rounds of a 64-wide search over the
// sorted indices), then multiplies every row of that run, 64 rows at a time,
// by its W tile -- each expert's weights stream from HBM once per 64 rows.
// The extra block row e == w_batch fills the rows of out-of-range indices
// (sorted to the end) with NaN. Same LDS-dequant MFMA pipeline as the
// large-tile GEMM, at a 128 x 64 tile with 4 waves (2 blocks per CU), or
// 128 x 48 with 3 blocks per CU for K <= 1024.
// ---------------------------------------------------------------------------
constexpr int QBN = 128, QBM = 64;
constexpr int kGD = 4;  // register prefetch depth (K-steps) of the grouped kernel

struct GQKern {
  void* y;
  const void* x;
  const uint32_t* w;
  const void* s;
  const void* b;
  const uint32_t* lhs;
  const uint32_t* rhs;
  int64_t batch, x_rep, x_batch, w_batch;
  int M, N, K;
  const uint32_t* w2;  // SwiGLU up projection (gate is w/s/b), [w_batch, N, P]
  const void* s2;
  const void* b2;
};


// SWI: a tile's 128 W rows are 64 output columns of the gate and the same
// columns of the up projection; wave wn's fragment 0 holds gate columns
// n0 + wn*16 .. + 15 and fragment 1 the matching up columns, so the epilogue
// writes swiglu(gate, up) from registers.
template <int BITS, int CT, int GS, bool SWI, bool OCC>
__global__ __launch_bounds__(256) void gqmm_kernel(GQKern a) {
  // OCC (short K loops): 48 x rows, 144-byte LDS rows and a 2-deep ring,
  // 50.7 KB of LDS and under 168 VGPRs, so three blocks fit a CU (configs[4]
  // down, K = 768: 77 -> 73 us); with K = 2048 the shallow ring costs more
  // than the occupancy gains (gate 77 -> 89 us), so longer K keeps 64 x rows,
  // 160-byte rows and 4 steps of prefetch.
  constexpr int XM = OCC ? 48 : QBM;
  constexpr int LD = OCC ? GBK + 8 : GLD;
  constexpr int RD = OCC ? 2 : kGD;
  constexpr int NJX = XM / 16;
  using T = Mma<CT>;
  using ST = st_t<CT>;
  __shared__ __attribute__((aligned(16))) uint16_t As[2][QBN * LD];  // W (dequantized)
  __shared__ __attribute__((aligned(16))) uint16_t Bs[2][XM * LD];  // x rows
  __shared__ int64_t run[2];

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int M = a.M, N = a.N, K = a.K;
  constexpr int ONT = SWI ? QBN / 2 : QBN;  // output columns per tile
  const int n0 = blockIdx.x * ONT;
  const int64_t e = blockIdx.y;  // expert, or w_batch for the out-of-range tail
  if (wv == 0) {
    const int64_t s0 = wave_lower_bound(a.rhs, a.batch, (uint32_t)e);
    const int64_t s1 = e < a.w_batch ? wave_lower_bound(a.rhs, a.batch, (uint32_t)(e + 1)) : a.batch;
    if (lane == 0) { run[0] = s0; run[1] = s1; }
  }
  __syncthreads();
  const int64_t r_begin = run[0] * M, r_end = run[1] * M;  // flattened (element, m) rows
  if (r_begin >= r_end) return;
  ST* yg = (ST*)a.y;
  if (e >= a.w_batch) {
    const uint16_t nan16 = CT == DT_BF16 ? 0x7fc0u : 0x7e00u;
    for (int64_t r = r_begin; r < r_end; r++)
      for (int n = n0 + tid; n < min(n0 + ONT, N); n += 256) yg[r * N + n] = nan16;
    return;
  }

  const int64_t P = (int64_t)(K >> 5) * BITS;
  const int64_t G = K / GS;
  const ST* xg = (const ST*)a.x;
  const int wn = wv;  // wave owns W rows wn*32.. (2 fragments), all XM x rows

  // x tile (XM x 64): thread copies chunks xc and xc + 4 of row xr.
  // (with XM < 64, threads past row XM - 1 repeat that row's loads and
  // stores -- the same values -- so every thread runs the same code)
  const int xr = min(tid >> 2, XM - 1), xc = tid & 3;
  // W tile (128 x 64): thread dequantizes pack wp of row wr. SWI: row wr is
  // column n0 + (wr / 32) * 16 + wr % 16 of the gate (bit 4 of wr clear) or
  // of the up projection.
  const int wr = tid >> 1, wp = tid & 1;
  const bool w_up = SWI && (wr & 16);
  const ST* sg = (const ST*)(w_up ? a.s2 : a.s) + e * (int64_t)N * G;
  const ST* bg = (const ST*)(w_up ? a.b2 : a.b) + e * (int64_t)N * G;
  const uint32_t* wg = (w_up ? a.w2 : a.w) + e * (int64_t)N * P;
  const int n_w = min(SWI ? n0 + (wr >> 5) * 16 + (wr & 15) : n0 + wr, N - 1);
  const uint32_t* wrow = wg + (int64_t)n_w * P + wp * BITS;
  const ST* srow = sg + (int64_t)n_w * G;
  const ST* brow = bg + (int64_t)n_w * G;

  struct WPre {
    uint32_t wd[BITS];
    float sv, bv;
  };
  auto wload = [&](WPre& p, int k0) {
    load_pack<BITS>(wrow + (int64_t)(k0 >> 5) * BITS, p.wd);
    const int gi = (k0 + wp * 32) / GS;
    p.sv = DT_<CT>::load(srow, gi);
    p.bv = DT_<CT>::load(brow, gi);
  };
  auto wstore = [&](const WPre& p, int buf) {
    uint16_t* dst = As[buf] + wr * LD + wp * 32;
#pragma unroll
    for (int qq = 0; qq < 4; qq++) *reinterpret_cast<u32x4*>(dst + qq * 8) = deq8<BITS, CT>(p.wd, qq, p.sv, p.bv);
  };

  for (int64_t r0 = r_begin; r0 < r_end; r0 += XM) {
    // this thread's x row: flattened row r -> batch element r / M, row r % M
    const int64_t r = min(r0 + xr, r_end - 1);
    const int64_t bi = r / M;
    const int64_t xi = a.lhs ? (int64_t)a.lhs[bi] : bi / a.x_rep;
    const ST* xrow = xg + (min(xi, a.x_batch - 1) * M + (r - bi * M)) * (int64_t)K + xc * 8;

    floatx4 acc[2][NJX];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < NJX; j++) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // Register ring of RD steps: the loads of step kt + RD are issued at
    // step kt and land in LDS at step kt + RD - 1, so RD - 1 steps of
    // compute cover their latency. The ring index is a compile-time constant
    // inside the unrolled group, so no register copies force early waits.
    const int nk = K / GBK;
    WPre wr_[RD];
    u32x4 xr_[RD][2];
    auto xload_to = [&](u32x4 (&d)[2], int k0) {
      d[0] = *reinterpret_cast<const u32x4*>(xrow + k0);
      d[1] = *reinterpret_cast<const u32x4*>(xrow + k0 + 32);
    };
    auto xstore_from = [&](const u32x4 (&d)[2], int buf) {
      *reinterpret_cast<u32x4*>(Bs[buf] + xr * LD + xc * 8) = d[0];
      *reinterpret_cast<u32x4*>(Bs[buf] + xr * LD + xc * 8 + 32) = d[1];
    };
#pragma unroll
    for (int d = 0; d < RD; d++) {
      xload_to(xr_[d], min(d, nk - 1) * GBK);
      wload(wr_[d], min(d, nk - 1) * GBK);
    }
    wstore(wr_[0], 0);
    xstore_from(xr_[0], 0);
    __syncthreads();
    for (int kt0 = 0; kt0 < nk; kt0 += RD) {
#pragma unroll
      for (int d = 0; d < RD; d++) {
        const int kt = kt0 + d;
        if (kt < nk) {
          const int buf = d & 1;  // RD is even, so kt & 1 == d & 1
#pragma unroll
          for (int ks = 0; ks < GBK / 32; ks++) {
            const int kofs = ks * 32 + (lane >> 4) * 8;
            typename T::frag fb[NJX];
#pragma unroll
            for (int j = 0; j < NJX; j++)
              fb[j] = __builtin_bit_cast(typename T::frag, *reinterpret_cast<const u32x4*>(
                                                               Bs[buf] + (j * 16 + (lane & 15)) * LD + kofs));
#pragma unroll
            for (int i = 0; i < 2; i++) {
              const typename T::frag fa = __builtin_bit_cast(
                  typename T::frag,
                  *reinterpret_cast<const u32x4*>(As[buf] + (wn * 32 + i * 16 + (lane & 15)) * LD + kofs));
#pragma unroll
              for (int j = 0; j < NJX; j++) acc[i][j] = T::mma(fa, fb[j], acc[i][j]);
            }
          }
          // step kt + 1 (ring slot d + 1) into the other buffer; refill slot d
          // with step kt + RD (past the end: reload the last step, unused)
          wstore(wr_[(d + 1) % RD], buf ^ 1);
          xstore_from(xr_[(d + 1) % RD], buf ^ 1);
          xload_to(xr_[d], min(kt + RD, nk - 1) * GBK);
          wload(wr_[d], min(kt + RD, nk - 1) * GBK);
          __syncthreads();
        }
      }
    }

    // epilogue: acc[i][j][v] = y[row m][n], n = n0 + wn*32 + i*16 + 4*(lane>>4) + v
    // (SWI: acc[0] gate and acc[1] up of column n0 + wn*16 + 4*(lane>>4) + v)
    if constexpr (SWI) {
#pragma unroll
      for (int j = 0; j < NJX; j++)
#pragma unroll
        for (int v = 0; v < 4; v++)
          acc[0][j][v] = swiglu_f32(DT_<CT>::round(acc[0][j][v]), DT_<CT>::round(acc[1][j][v]));
    }
#pragma unroll
    for (int i = 0; i < (SWI ? 1 : 2); i++) {
      const int n = n0 + wn * (SWI ? 16 : 32) + i * 16 + 4 * (lane >> 4);
#pragma unroll
      for (int j = 0; j < NJX; j++) {
        const int64_t rr = r0 + j * 16 + (lane & 15);
        if (rr >= r_end) continue;
        const int64_t rb = rr / M;
        if ((a.lhs ? (int64_t)a.lhs[rb] : rb / a.x_rep) >= a.x_batch) {  // out-of-range x index
#pragma unroll
          for (int v = 0; v < 4; v++)
            if (n + v < N) yg[rr * N + n + v] = CT == DT_BF16 ? (uint16_t)0x7fc0u : (uint16_t)0x7e00u;
          continue;
        }
        if (n + 3 < N) {
          u32x2 o;
          o[0] = pack2<CT>(acc[i][j][0], acc[i][j][1]);
          o[1] = pack2<CT>(acc[i][j][2], acc[i][j][3]);
          *reinterpret_cast<u32x2*>(yg + rr * N + n) = o;
        } else {
#pragma unroll
          for (int v = 0; v < 4; v++)
            if (n + v < N) yg[rr * N + n + v] = DT_<CT>::from_f32(acc[i][j][v]);
        }
      }
    }
  }
}

template <int CT, int GS, bool SWI>
hipError_t run_gqmm(const QArgs& a) {
  GQKern k;
  k.y = a.y; k.x = a.x; k.w = a.w; k.s = a.s; k.b = a.b; k.lhs = a.lhs; k.rhs = a.rhs;
  k.batch = a.batch; k.x_rep = a.x_rep; k.x_batch = a.x_batch; k.w_batch = a.w_batch;
  k.M = (int)a.M; k.N = (int)a.N; k.K = (int)a.K;
  k.w2 = a.w2; k.s2 = a.s2; k.b2 = a.b2;
  const int ont = SWI ? QBN / 2 : QBN;
  dim3 grid((unsigned)((a.N + ont - 1) / ont), (unsigned)(a.w_batch + 1));
  if (a.K <= 1024)
    hipLaunchKernelGGL((gqmm_kernel<HQ_BITS, CT, GS, SWI, true>), grid, dim3(256), 0, a.stream, k);
  else
    hipLaunchKernelGGL((gqmm_kernel<HQ_BITS, CT, GS, SWI, false>), grid, dim3(256), 0, a.stream, k);
  return hipGetLastError();
}

template <bool SWI>
hipError_t run_gqmm_g(const QArgs& a) {
  const bool bf = a.xdt == DT_BF16;
  switch (a.group_size) {
    case 32: return bf ? run_gqmm<DT_BF16, 32, SWI>(a) : run_gqmm<DT_F16, 32, SWI>(a);
    case 64: return bf ? run_gqmm<DT_BF16, 64, SWI>(a) : run_gqmm<DT_F16, 64, SWI>(a);
    default: return bf ? run_gqmm<DT_BF16, 128, SWI>(a) : run_gqmm<DT_F16, 128, SWI>(a);
  }
}

}  // namespace

#define HQ_CAT_(a, b) a##b
#define HQ_CAT(a, b) HQ_CAT_(a, b)

// Sorted-index gather_qmm through the grouped kernel, or hipErrorNotSupported
// (dtype mix, K not a multiple of 64, too many experts for the grid).
hipError_t HQ_CAT(launch_gqmm_t_b, HQ_BITS)(const QArgs& a) {
  // few rows per expert: the streaming grouped kernel (hq_gqms.hip)
  const hipError_t es = HQ_CAT(launch_gqms_t_b, HQ_BITS)(a);
  if (es != hipErrorNotSupported) return es;
  if (a.xdt != a.sdt || a.xdt == DT_F32 || a.K % GBK != 0 || a.w_batch + 1 > 65535 || !a.rhs)
    return hipErrorNotSupported;
  return a.w2 ? run_gqmm_g<true>(a) : run_gqmm_g<false>(a);
}

template <int XDT, int SDT>
static void run_qmm_t(const QArgs& a) {
  QKernM k;
  k.y = a.y; k.x = a.x; k.w = a.w; k.s = a.s; k.b = a.b;
  k.lhs = a.lhs; k.rhs = a.rhs;
  k.batch = a.batch; k.x_rep = a.x_rep; k.x_batch = a.x_batch; k.w_batch = a.w_batch;
  k.M = (int)a.M; k.N = (int)a.N; k.K = (int)a.K;
  k.gshift = __builtin_ctz((unsigned)a.group_size);
  k.lb = a.lb;
  dim3 grid((unsigned)((a.N + BN - 1) / BN), (unsigned)((a.M + BM - 1) / BM),
            (unsigned)(a.batch < 65535 ? a.batch : 65535));
  qmm_t_kernel<HQ_BITS, XDT, SDT><<<grid, 256, 0, a.stream>>>(k);
}

hipError_t HQ_CAT(launch_qmm_t_b, HQ_BITS)(const QArgs& a) {
  // One product with same-type 16-bit x and scales, K a multiple of the step:
  // the large-tile GEMM, from 9 rows up (M = 9..127 at 14336 x 4096: 26-48 us
  // against 126-190 us on the general kernel, which re-reads W per 64 rows
  // of its 64 x 64 tiles). Everything else: the general batched kernel.
  // (the large-tile GEMM addresses x and W with 32-bit element offsets)
  const bool off32 = a.M * a.K < ((int64_t)1 << 31) &&
                     a.N * (a.K / 32) * HQ_BITS < ((int64_t)1 << 31);
  // 9-16 rows of 4-bit weights with many output tiles, plain or with the
  // fused SwiGLU: the streaming kernel's dense form (hq_gqms.hip, its own
  // conditions)
  if (a.M <= 16) {
    const hipError_t ed = HQ_CAT(launch_gqms_dense_t_b, HQ_BITS)(a);
    if (ed != hipErrorNotSupported) return ed;
  }
  const bool gemm_ok = a.batch == 1 && !a.lhs && !a.rhs && a.xdt == a.sdt && a.xdt != DT_F32 &&
                       a.K % GBK == 0 && a.M > kQmvMaxM && off32;
  // 9-32 rows on few output tiles: the GEMM's blocks then each stream a
  // 64-row W slice through a latency-bound K loop (~5.5 ns per K element,
  // 23 us at K = 4096 whatever N and M), while an 8-row GEMV launch streams
  // W at ~1.4 TB/s with a ~4.5 us floor. Run ceil(M / 8) GEMV launches
  // when that model says they are faster. Measured (4-bit g64, us, GEMM vs
  // GEMV launches): 1024 x 4096 M = 32 23.6 vs 19.0, M = 48 23.9 vs 28.3;
  // 4096 x 4096 M = 24 23.8 vs 17.3; 4096 x 14336 M = 16 74.3 vs 44.3,
  // M = 24 75.1 vs 65.8, M = 32 75.9 vs 87.4; 6144 x 4096 M = 16 23.8 vs
  // 18.0, M = 24 24.0 vs 26.5.
  if (gemm_ok && !a.w2 && a.M <= 4 * kQmvMaxM) {
    const int64_t launches = (a.M + kQmvMaxM - 1) / kQmvMaxM;
    const double w_mb = (double)a.N * (double)a.K * HQ_BITS / 8e6;
    const double t_gemv = std::max(4.5, w_mb / 1.4);
    const int64_t cus = device_cu_count();
    const int64_t rounds = ((a.N + 63) / 64 + cus - 1) / cus;
    const double t_gemm = (double)rounds * 0.0055 * (double)a.K;
    if ((double)launches * t_gemv < t_gemm) {
      const size_t xb = 2, yb = 2;  // same 16-bit dtype for x, scales and y
      QArgs c = a;
      hipError_t e = hipSuccess;
      for (int64_t m0 = 0; m0 < a.M && e == hipSuccess; m0 += kQmvMaxM) {
        c.M = std::min<int64_t>(a.M - m0, kQmvMaxM);
        c.x = static_cast<const char*>(a.x) + (size_t)(m0 * a.K) * xb;
        c.y = static_cast<char*>(a.y) + (size_t)(m0 * a.N) * yb;
        e = HQ_CAT(launch_qmvx_t_b, HQ_BITS)(c);
      }
      return e;
    }
  }
  if (gemm_ok) {
    if (a.w2) return a.xdt == DT_BF16 ? run_qgemm_g<DT_BF16, true>(a) : run_qgemm_g<DT_F16, true>(a);
    return a.xdt == DT_BF16 ? run_qgemm_g<DT_BF16>(a) : run_qgemm_g<DT_F16>(a);
  }
  if (a.w2) return hipErrorNotSupported;  // fused SwiGLU: large-tile GEMM only
  switch (a.xdt * 3 + a.sdt) {
    case DT_F32 * 3 + DT_F32: run_qmm_t<DT_F32, DT_F32>(a); break;
    case DT_F32 * 3 + DT_F16: run_qmm_t<DT_F32, DT_F16>(a); break;
    case DT_F32 * 3 + DT_BF16: run_qmm_t<DT_F32, DT_BF16>(a); break;
    case DT_F16 * 3 + DT_F32: run_qmm_t<DT_F16, DT_F32>(a); break;
    case DT_F16 * 3 + DT_F16: run_qmm_t<DT_F16, DT_F16>(a); break;
    case DT_F16 * 3 + DT_BF16: run_qmm_t<DT_F16, DT_BF16>(a); break;
    case DT_BF16 * 3 + DT_F32: run_qmm_t<DT_BF16, DT_F32>(a); break;
    case DT_BF16 * 3 + DT_F16: run_qmm_t<DT_BF16, DT_F16>(a); break;
    default: run_qmm_t<DT_BF16, DT_BF16>(a); break;
  }
  return hipGetLastError();
}

}  // namespace hq
