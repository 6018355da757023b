// hq_gqms.hip -- sorted-expert grouped quantized matmul, streaming form, for
// 4-bit weights: gather_qmm with sorted rhs indices (the MoE expert GEMM of
// crates/higgs-models/src/qwen3_next.rs:1764-1799, FFI at 509-578) and its
// fused gate/up + SwiGLU form (qwen3_next.rs:1764-1787), when each expert has
// few routed rows and K <= 2048, as in the MoE projections.
//
// y[r, n] = sum_k x[xi(r), k] * (s[e, n, g] * q[e, n, k] + b[e, n, g]),
// e = rhs[r / M] (non-decreasing), g = k / group_size.
//
// Why a second grouped kernel: with ~32 rows per expert (configs[4]: 4096
// routed rows over 128 experts) the LDS-dequantizing GEMM dequantizes every W
// tile for few rows. Here the matrix cores take the packed nibbles as
// (OFF + q) bf16/fp16 operands with no dequantization, and the per-group scale
// and bias are applied to the fp32 partial sums:
//   acc += s * D_g + (b - OFF * s) * X_g,   X_g = sum of x over the group.
//
// Layout of one v_mfma_f32_16x16x32 step: B = 16 W rows (lane n = lane % 16)
// x 32 k, A = 16 x rows, D[m, n]. Every MFMA step stays inside one scale
// group: at group size 128 lane group q = lane / 16 holds words [4q, 4q + 4)
// of the group, at 64 the words of a group pair are regrouped across the wave
// halves (see the compute step); x sits in LDS in the unpack's pair order
// (0,4,1,5,2,6,3,7) per 8-element block.
//
// Block (tile range, e, z): 8 waves. The block finds the run of rows routed
// to e by a wave-wide search over the sorted indices (unused experts cost no
// weight traffic), loads up to 64 (32) of those rows of x for the whole K
// straight into LDS (global_load_lds_dwordx4), computes the group sums (v_dot2
// against ones) and reorders x to the pair order in place, then each wave
// streams its 16-row W tiles through a register double buffer while it
// multiplies. The block row e == w_batch fills rows of out-of-range expert
// indices with NaN, and rows whose x index is out of range are NaN too.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "hq_common.hpp"
#include "hq_device.hpp"
#include "hq_kernels.hpp"

#ifndef HQ_BITS
#error "compile with -DHQ_BITS=<2|3|4|5|6|8>"
#endif

namespace hq {

namespace {

struct GSKern {
  void* y;
  const void* x;
  const uint32_t* w;
  const void* s;
  const void* b;
  const uint32_t* lhs;
  const uint32_t* rhs;
  int64_t batch, x_rep, x_batch, w_batch;
  int M, N, K;
  uint32_t nib_mask, off_pair;  // 0x000F000F and the (OFF, OFF) pair, kept out of literals
  int ntiles;                   // 16-column output tiles: ceil(N / 16)
  int ns;                       // blocks splitting the tiles (grid.x)
  const uint32_t* w2;           // fused SwiGLU: the up projection (w, s, b are the gate)
  const void* s2;
  const void* b2;
};

template <int XDT> struct SMma;
template <> struct SMma<DT_BF16> {
  using frag = bf16x8;
  static __device__ __forceinline__ floatx4 mma(frag a, frag b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static constexpr uint32_t OFFB = 0x43004300u;  // (128 + q) for q < 128
  static constexpr float OFF = 128.f;
  static constexpr uint32_t ONE2 = 0x3F803F80u;
};
template <> struct SMma<DT_F16> {
  using frag = f16x8;
  static __device__ __forceinline__ floatx4 mma(frag a, frag b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static constexpr uint32_t OFFB = 0x64006400u;  // (1024 + q) for q < 1024
  static constexpr float OFF = 1024.f;
  static constexpr uint32_t ONE2 = 0x3C003C00u;
};

// 16 (4) bytes per lane from global memory straight into LDS at
// lds_wave + 16 * lane (4 * lane); lds_wave is wave-uniform.
__device__ __forceinline__ void dma16(const void* g, void* lds_wave) {
  __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)g,
                                   (void __attribute__((address_space(3)))*)lds_wave, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* g, void* lds_wave) {
  __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)g,
                                   (void __attribute__((address_space(3)))*)lds_wave, 4, 0, 0);
}

// s_waitcnt immediate (gfx9 encoding): at most `vm` vector memory operations
// outstanding, every LDS operation complete.
constexpr int waitcnt_vm_lgkm0(int vm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4); }

constexpr int kMR = 64;  // x rows per block pass (four 16-row MFMA tiles)
// Row stride (floats) of the group sums in LDS for GQ groups per lane group:
// the fp32 MFMA's A read of lane group q starts q * GQ rows down, and a stride
// with GQ * stride = 16 (mod 64) puts the four lane groups on disjoint banks.
// At least `rows` floats per row (the rows a block pass stages).
constexpr int xsum_stride(int gq, int rows) {
  int s = rows;
  while ((gq * s) % 64 != 16) s++;
  return s;
}
// x rows in LDS. A ds_read_b128 is served in four cycles of 16 lanes: per
// half wave, the lanes l with an even, then an odd number of set bits in
// (l >> 2) & 7, i.e. {0-3, 12-15, 20-23, 24-27} and {4-7, 8-11, 16-19, 28-31}
// (+32 for the upper half); the 16 lanes of a cycle must hit distinct 16-byte
// bank slots (address bits 4-7) unless they read the same address (measured
// with SQ_LDS_BANK_CONFLICT on single-wave patterns). Row r starts at
// r * (2K + 256) bytes plus 16 * kRowSlot[r % 16]: rows 0-3 and 12-15 take
// slots {0,1,4,5,8,9,12,13}, rows 4-11 the rest, so the MFMA A reads (lane
// n reads row n + 16j; lane groups q = 0, 1 and q = 2, 3 read columns 64 bytes
// apart) and the row-per-lane group-sum pass are both conflict-free.
constexpr uint64_t kRowSlot = 0xDC98FEBA76325410ull;  // nibble r: slot of row r % 16
constexpr int xrow_elems(int k) { return k + 128; }
__device__ __forceinline__ int xrow_off(int r, int k) {
  return r * xrow_elems(k) + 8 * (int)((kRowSlot >> (4 * (r & 15))) & 15);
}
// Shape of one instantiation: KC chunks of 256 k; an item is one 16-row W
// tile over CP of them (a K part), so that two items of weights fit the
// registers; NS weight streams (2: gate and up of the fused SwiGLU); MR x
// rows per pass: 32 for K = 2048 (x then takes 139 KB of LDS) and for the
// SwiGLU form (two streams of four 16-row tiles would spill); with 32-row
// passes the passes of an expert alternate between ZS = 2 blocks.
//
// DENSE: one product of at most 16 x rows (batched decode) instead of a
// gather: no expert search, 16 x rows, and the K parts of a tile split over
// WPT = 2 waves whose partial sums meet in LDS, so that 4 tiles keep a
// block's 8 waves busy.
template <int KC, bool SWI, bool DENSE = false> struct GSShape {
  static constexpr int CP = SWI ? 2 : (KC % 4 == 0 ? 4 : KC);
  static constexpr int KP = KC / CP;
  static constexpr int NS = SWI ? 2 : 1;
  static constexpr int MR = DENSE ? 16 : (KC <= 4 && !SWI ? 64 : 32);
  static constexpr int ZS = DENSE ? 1 : 64 / MR;
  static constexpr int WPT = DENSE ? 2 : 1;   // waves per tile
  static constexpr int TPW = 8 / WPT;         // tiles in flight per block
  static constexpr int RED = DENSE ? 8 * 64 * 16 * NS : 0;  // LDS for the cross-wave sums
  // group-sum rows: the dense SwiGLU form strides them for its 16 rows (at
  // K = 4096 its LDS would not fit otherwise); every other form for 64
  static constexpr int XSR = SWI && DENSE ? MR : kMR;
};
// LDS of one block: group sums, the out-of-range flags, the x rows.
template <int GS, int KC, bool SWI, bool DENSE = false>
constexpr int gx_lds_bytes() {
  using SH = GSShape<KC, SWI, DENSE>;
  return (KC * 256 / GS) * xsum_stride(SH::CP * (256 / GS) / 4, SH::XSR) * 4 + SH::MR * 4 +
         SH::MR * xrow_elems(KC * 256) * 2 + SH::RED;
}

template <int XDT, int GS, int KC, bool SWI, bool DENSE>
__global__ __launch_bounds__(512, 2) void gqms_kernel(GSKern a) {
  using SH = GSShape<KC, SWI, DENSE>;
  constexpr int KK = KC * 256;
  constexpr int G = KK / GS;        // scale groups per W row
  constexpr int NGC = 256 / GS;     // groups per 256-element chunk
  constexpr int WPG = GS / 32;      // words per lane per group (2 or 4)
  constexpr int XLD = xrow_elems(KK);  // LDS row stride of x in elements
  constexpr int CP = SH::CP, KP = SH::KP, NS = SH::NS, MR = SH::MR, ZS = SH::ZS;
  constexpr int WPT = SH::WPT, TPW = SH::TPW, KPW = KP / WPT;  // K parts of a tile per wave
  constexpr int RPW = MR / 8;       // x rows each of the 8 waves stages
  constexpr int GPP = CP * NGC;     // scale groups per item part
  constexpr int GQ = GPP / 4;       // groups of a part each lane group owns
  constexpr int NWL = NS * CP * 2;  // weight load instructions per item (16 bytes per lane)
  static_assert(WPG == 2 || WPG == 4, "group size 64 or 128");
  static_assert(KC % CP == 0 && GPP % 4 == 0, "whole parts, whole fp32-MFMA steps of groups");
  constexpr int XSS = xsum_stride(GQ, SH::XSR);
  static_assert(gx_lds_bytes<GS, KC, SWI, DENSE>() <= 160 * 1024, "x rows fit the LDS");
  static_assert(KP % WPT == 0, "whole parts per wave");
  using T = SMma<XDT>;
  using frag = typename T::frag;
  using XS = st_t<XDT>;

  // the small arrays first, so every group-sum read folds its offset into
  // the instruction (LDS offsets stop at 64 KB)
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float* Xs = reinterpret_cast<float*>(smem);                                // [G][XSS] group sums
  int* xbad = reinterpret_cast<int*>(smem + G * XSS * 4);                    // [MR]
  uint16_t* xs = reinterpret_cast<uint16_t*>(smem + G * XSS * 4 + MR * 4);  // MR rows at xrow_off
  floatx4* red = reinterpret_cast<floatx4*>(smem + G * XSS * 4 + MR * 4 + MR * XLD * 2);  // DENSE: [NS][8][64]

  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int nl = lane & 15, q = lane >> 4;
  const int N = a.N, M = a.M;
  const int64_t e = DENSE ? 0 : blockIdx.y;
  const int z = (int)blockIdx.z;
  const int tpb = (a.ntiles + a.ns - 1) / a.ns;
  const int tb = blockIdx.x * tpb, te = min(a.ntiles, tb + tpb);
  if (tb >= te) return;
  const bool expert_ok = DENSE || e < a.w_batch;
  const int64_t s0 = DENSE ? 0 : wave_lower_bound(a.rhs, a.batch, (uint32_t)e);
  const int64_t s1 = DENSE ? 1 : (expert_ok ? wave_lower_bound(a.rhs, a.batch, (uint32_t)(e + 1)) : a.batch);
  const int64_t r_begin = s0 * M, r_end = s1 * M;  // flattened (element, m) rows
  if (r_begin + (int64_t)z * MR >= r_end) return;  // block-uniform
  XS* yg = (XS*)a.y;
  constexpr uint16_t kNaN = XDT == DT_BF16 ? 0x7fc0u : 0x7e00u;
  if (!expert_ok) {
    if (z != 0) return;
    const int c0 = tb * 16, c1 = min(te * 16, N);
    for (int64_t r = r_begin; r < r_end; r++)
      for (int n = c0 + tid; n < c1; n += 512) yg[r * N + n] = kNaN;
    return;
  }

  // this wave's tiles: tb + ts + TPW j, ts = wv % TPW; item i = part
  // kw + WPT (i % KPW) of tile j = i / KPW, kw = wv / TPW. DENSE: every wave
  // runs the same items (tiles past the range clamped, computed, not stored),
  // as the cross-wave sums take block barriers.
  const int ts = wv % TPW, kw = wv / TPW;
  const int NI = (DENSE ? (te - tb + TPW - 1) / TPW : max(0, (te - tb - ts + TPW - 1) / TPW)) * KPW;
  const int64_t P = KK / 8;  // words per W row

  // Lane group q owns the scales and biases of groups [q * GQ, q * GQ + GQ)
  // of a part: packed in words when GQ is even, one 16-bit value per register
  // otherwise.
  constexpr bool PK = GQ % 2 == 0;
  constexpr int SBW = PK ? GQ / 2 : GQ;
  struct Buf {
    uint32_t wd[NS][CP][8];
    uint32_t sv[NS][SBW], bv[NS][SBW];
  };
  // W row and part of item i (clamped to the last item: loads past the end
  // reload it and are never computed)
  auto item_at = [&](int i, int& part) __attribute__((always_inline)) -> int64_t {
    const int ii = min(i, max(NI - 1, 0));
    part = kw + WPT * (ii % KPW);
    const int t = min(tb + ts + TPW * (ii / KPW), te - 1);
    return e * N + min(t * 16 + nl, N - 1);
  };
  auto issue_sb = [&](Buf& b, int i) __attribute__((always_inline)) {
    int part;
    const int64_t row = item_at(i, part);
#pragma unroll
    for (int s = 0; s < NS; s++) {
      const XS* sp = (const XS*)(s ? a.s2 : a.s) + row * G + part * GPP + q * GQ;
      const XS* bp = (const XS*)(s ? a.b2 : a.b) + row * G + part * GPP + q * GQ;
      if constexpr (GQ == 4) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(sp), u = *reinterpret_cast<const u32x2*>(bp);
        b.sv[s][0] = v[0]; b.sv[s][1] = v[1]; b.bv[s][0] = u[0]; b.bv[s][1] = u[1];
      } else if constexpr (GQ == 2) {
        b.sv[s][0] = *reinterpret_cast<const uint32_t*>(sp);
        b.bv[s][0] = *reinterpret_cast<const uint32_t*>(bp);
      } else {
#pragma unroll
        for (int t = 0; t < GQ; t++) {
          b.sv[s][t] = sp[t];
          b.bv[s][t] = bp[t];
        }
      }
    }
  };
  // 16 bytes per lane: lane group q loads words [4q, 4q + 4) of each
  // 16-word span of the row (64 contiguous bytes per row per instruction).
  // At group size 128 a span is one group; at 64 it is two, and the compute
  // step regroups the words across the wave halves.
  auto issue_w = [&](Buf& b, int i) __attribute__((always_inline)) {
    int part;
    const int64_t row = item_at(i, part);
#pragma unroll
    for (int s = 0; s < NS; s++) {
      const uint32_t* wp = (s ? a.w2 : a.w) + row * P + part * (CP * 32) + q * 4;
#pragma unroll
      for (int c = 0; c < CP; c++)
#pragma unroll
        for (int h = 0; h < 2; h++) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(wp + c * 32 + h * 16);
#pragma unroll
          for (int t = 0; t < 4; t++) b.wd[s][c][4 * h + t] = v[t];
        }
    }
  };

  const uint32_t mask_s = a.nib_mask;
  uint32_t off_v;
  asm("v_mov_b32 %0, %1" : "=v"(off_v) : "s"(a.off_pair));

  Buf ba, bb;
  for (int64_t r0 = r_begin + (int64_t)z * MR; r0 < r_end; r0 += (int64_t)ZS * MR) {
    const int nrows = (int)min((int64_t)MR, r_end - r0);
    // x row offsets of this wave's rows (token gather through lhs)
    int64_t xoff[RPW];
#pragma unroll
    for (int k = 0; k < RPW; k++) {
      const int rr = wv + 8 * k;
      const int64_t r = r0 + min(rr, nrows - 1);
      const int64_t bi = M == 1 ? r : r / M;
      const int64_t xi = DENSE ? 0 : a.lhs ? (int64_t)a.lhs[bi] : (a.x_rep == 1 ? bi : bi / a.x_rep);
      xoff[k] = (min(xi, a.x_batch - 1) * M + (r - bi * M)) * (int64_t)KK;
      if (lane == 0 && rr < nrows) xbad[rr] = xi >= a.x_batch;
    }
    // The first item's scales, then x straight into LDS (every row slot of
    // the pass; slots past the last row repeat it), then the first item's
    // weights. The DMA code is branch-free, so the explicit wait below leaves
    // exactly those NWL weight loads in flight while it covers every DMA
    // (sched barriers keep the order; tests/test_capi.py checks the count in
    // the compiled code).
    issue_sb(ba, 0);
    __builtin_amdgcn_sched_barrier(0);
    // DENSE: slots k >= 1 past the last row are not staged (their MFMA rows
    // are never stored, and their sums are skipped), so 8 rows stage half of
    // the 16 slots. They go first, so the last DMA (slot 0, always staged)
    // is followed by straight-line code up to the wait. (The grouped form
    // keeps every slot: there the x row offsets come from loaded indices,
    // and a skipped DMA made the compiler wait for every load at the join.)
#pragma unroll
    for (int kk = 0; kk < RPW; kk++) {
      const int k = DENSE ? RPW - 1 - kk : kk;
      if (DENSE && k > 0 && wv + 8 * k >= nrows) continue;
      const XS* src = (const XS*)a.x + xoff[k] + lane * 8;
      uint16_t* dst = xs + xrow_off(wv + 8 * k, KK);
#pragma unroll
      for (int p = 0; p < KK / 512; p++) dma16(src + p * 512, dst + p * 512);
      if constexpr (KK % 512 != 0) {  // 256-element tail: two 4-byte pieces per lane
        const XS* ts = (const XS*)a.x + xoff[k] + (KK / 512) * 512 + lane * 2;
        dma4(ts, dst + (KK / 512) * 512);
        dma4(ts + 128, dst + (KK / 512) * 512 + 128);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    issue_w(ba, 0);
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(NWL));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // group sums of x (v_dot2 against ones) and the in-place reorder of every
    // 8-element block to the MFMA pair order (0,4,1,5,2,6,3,7); row-fastest
    // thread order keeps the 16-byte LDS accesses free of bank conflicts
    for (int idx = tid; idx < MR * G; idx += 512) {
      const int row = idx % MR, g = idx / MR;
      if (row < nrows) {
        uint16_t* p = xs + xrow_off(row, KK) + g * GS;
        float sum = 0.f;
#pragma unroll
        for (int pc = 0; pc < GS / 8; pc++) {
          const u32x4 d = *reinterpret_cast<const u32x4*>(p + pc * 8);
          // (the pairs are taken out by name: a bit_cast of d[j] inside a loop
          // compiled to four reads of d[0])
          const uint32_t d0 = d.x, d1 = d.y, d2 = d.z, d3 = d.w;
          if constexpr (XDT == DT_BF16) {
            typedef __bf16 b2 __attribute__((ext_vector_type(2)));
            const b2 one = __builtin_bit_cast(b2, 0x3F803F80u);
            sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, d0), one, sum, false);
            sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, d1), one, sum, false);
            sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, d2), one, sum, false);
            sum = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, d3), one, sum, false);
          } else {
            typedef _Float16 h2 __attribute__((ext_vector_type(2)));
            const h2 one = __builtin_bit_cast(h2, 0x3C003C00u);
            sum = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, d0), one, sum, false);
            sum = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, d1), one, sum, false);
            sum = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, d2), one, sum, false);
            sum = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, d3), one, sum, false);
          }
          u32x4 o;
          o[0] = (d[0] & 0xffffu) | (d[2] << 16);
          o[1] = (d[0] >> 16) | (d[2] & 0xffff0000u);
          o[2] = (d[1] & 0xffffu) | (d[3] << 16);
          o[3] = (d[1] >> 16) | (d[3] & 0xffff0000u);
          *reinterpret_cast<u32x4*>(p + pc * 8) = o;
        }
        Xs[g * XSS + row] = sum;
      }
    }
    // LDS writes done; the weight loads stay in flight
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    // items of MT active 16-row tiles, weights double-buffered in registers;
    // the accumulators carry over the KP parts of a tile
    auto run_items = [&](auto mt_c) __attribute__((always_inline)) {
      constexpr int MT = decltype(mt_c)::value;
      floatx4 acc[NS][MT];
      auto compute = [&](const Buf& b, int i) __attribute__((always_inline)) {
        // x and its sums do not change across items: without this the
        // compiler hoists every A-fragment read out of the item loop
        asm volatile("" ::: "memory");
        // lane coordinates opaque to the optimizer, so per-item addresses are
        // recomputed per item instead of living across the loop
        int qo = q, nlo = nl;
        asm volatile("" : "+v"(qo), "+v"(nlo));
        const int part = kw + WPT * (i % KPW);
        if (i % KPW == 0) {
#pragma unroll
          for (int s = 0; s < NS; s++)
#pragma unroll
            for (int j = 0; j < MT; j++) acc[s][j] = floatx4{0.f, 0.f, 0.f, 0.f};
        }
        // this lane's scales s and c = b - OFF * s, groups qo * GQ + t of the part
        float sf[NS][GQ], cf[NS][GQ];
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
          for (int t = 0; t < GQ; t++) {
            const uint32_t sh = PK ? (b.sv[s][t / 2] >> (16 * (t & 1))) & 0xffffu : b.sv[s][t];
            const uint32_t bh = PK ? (b.bv[s][t / 2] >> (16 * (t & 1))) & 0xffffu : b.bv[s][t];
            sf[s][t] = DT_<XDT>::to_f32((uint16_t)sh);
            cf[s][t] = fmaf(-T::OFF, sf[s][t], DT_<XDT>::to_f32((uint16_t)bh));
          }
        // the bias term sum_g X[m][g] * c[g][n] on the fp32 matrix cores:
        // k slot q of step t is group qo * GQ + t of the part, A = X of x row
        // m = nl, B = c of W row n = nl (the D layout is the bf16 MFMA's)
        const float* xsum = Xs + (part * GPP + qo * GQ) * XSS + nlo;
#pragma unroll
        for (int j = 0; j < MT; j++)
#pragma unroll
          for (int t = 0; t < GQ; t++) {
            const float xa = xsum[t * XSS + 16 * j];
#pragma unroll
            for (int s = 0; s < NS; s++)
              acc[s][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa, cf[s][t], acc[s][j], 0, 0, 0);
          }
        // byte addresses of lane nl of each lane group, for the scale broadcast
        int src[4];
#pragma unroll
        for (int o = 0; o < 4; o++) src[o] = (nlo + 16 * o) * 4;
        // A side: step t of a group takes x elements 8 * wq(t) .. + 7 of the
        // group, wq(t) the word the lane's B register holds at that step
        const uint16_t* xrow = xs + xrow_off(nlo, KK) + part * (CP * 256) +
                               (WPG == 4 ? qo * 32 : ((qo & 1) * 4 + (qo >> 1) * 2) * 8);
        // Software pipeline over the part's GPP groups: step gg issues the A
        // reads of group gg + 1 and the scale broadcast of group gg, runs the
        // MFMAs of group gg and the epilogue of group gg - 1, whose products
        // are complete by then (LDS and MFMA latency off the critical path).
        // Both weight streams use the same A fragments.
        u32x4 A[2][MT][WPG];
        auto load_a = [&](int gg) __attribute__((always_inline)) {
          const int c = gg / NGC, g = gg % NGC;
#pragma unroll
          for (int j = 0; j < MT; j++)
#pragma unroll
            for (int t = 0; t < WPG; t++)
              A[gg & 1][j][t] = *reinterpret_cast<const u32x4*>(xrow + 16 * j * XLD + c * 256 + g * GS + 8 * t);
        };
        uint32_t pair[NS][4];  // the regrouped span of the current group pair (group size 64)
        floatx4 Dp[NS][MT];
        float svp[NS];
        load_a(0);
#pragma unroll
        for (int gg = 0; gg < GPP; gg++) {
          __builtin_amdgcn_sched_barrier(0);  // one group at a time (bounded live registers)
          const int c = gg / NGC, g = gg % NGC;
          if (gg + 1 < GPP) load_a(gg + 1);
          float sv[NS];
#pragma unroll
          for (int s = 0; s < NS; s++)
            sv[s] = __int_as_float(__builtin_amdgcn_ds_bpermute(src[gg / GQ], __float_as_int(sf[s][gg % GQ])));
          floatx4 D[NS][MT];
#pragma unroll
          for (int s = 0; s < NS; s++) {
            uint32_t gw[WPG];
            if constexpr (WPG == 4) {
#pragma unroll
              for (int t = 0; t < 4; t++) gw[t] = b.wd[s][c][4 * g + t];
            } else {
              // span h = g / 2 holds words 4q..4q+3: lane groups 0, 1 have
              // group 2h, lane groups 2, 3 group 2h + 1. Swapping registers
              // 0 <-> 2 and 1 <-> 3 between the wave halves leaves group 2h
              // in registers 0, 1 of every lane (words (q&1)*4 + (q>>1)*2 + t)
              // and group 2h + 1 in registers 2, 3.
              if ((g & 1) == 0) {
                const auto s0 = __builtin_amdgcn_permlane32_swap(b.wd[s][c][2 * g], b.wd[s][c][2 * g + 2], false, false);
                const auto s1 = __builtin_amdgcn_permlane32_swap(b.wd[s][c][2 * g + 1], b.wd[s][c][2 * g + 3], false, false);
                pair[s][0] = s0[0]; pair[s][1] = s1[0]; pair[s][2] = s0[1]; pair[s][3] = s1[1];
              }
              gw[0] = pair[s][2 * (g & 1)];
              gw[1] = pair[s][2 * (g & 1) + 1];
            }
#pragma unroll
            for (int j = 0; j < MT; j++) D[s][j] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < WPG; t++) {
              const uint32_t w = gw[t];
              u32x4 bw;
              bw[0] = (w & mask_s) | off_v;
              bw[1] = ((w >> 4) & mask_s) | off_v;
              bw[2] = ((w >> 8) & mask_s) | off_v;
              bw[3] = ((w >> 12) & mask_s) | off_v;
#pragma unroll
              for (int j = 0; j < MT; j++)
                D[s][j] = T::mma(__builtin_bit_cast(frag, A[gg & 1][j][t]), __builtin_bit_cast(frag, bw), D[s][j]);
            }
          }
          if (gg > 0) {
#pragma unroll
            for (int s = 0; s < NS; s++)
#pragma unroll
              for (int j = 0; j < MT; j++) {
#pragma unroll
                for (int v = 0; v < 4; v++) acc[s][j][v] = fmaf(svp[s], Dp[s][j][v], acc[s][j][v]);
                // pin the epilogue to its step: left free, the compiler sinks
                // every group's FMAs to the end and keeps each group's partial
                // sums live (hundreds of registers)
                asm volatile("" : "+v"(acc[s][j]));
              }
          }
#pragma unroll
          for (int s = 0; s < NS; s++) {
#pragma unroll
            for (int j = 0; j < MT; j++) Dp[s][j] = D[s][j];
            svp[s] = sv[s];
          }
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
          for (int j = 0; j < MT; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) acc[s][j][v] = fmaf(svp[s], Dp[s][j][v], acc[s][j][v]);
        if (i % KPW != KPW - 1) return;
        if constexpr (DENSE) {
          // the WPT = 2 waves of a tile: the second hands its sums to the first
          // through LDS (fixed order, so results are deterministic)
          if (kw == 1) {
#pragma unroll
            for (int s = 0; s < NS; s++) red[(s * 8 + wv) * 64 + lane] = acc[s][0];
          }
          __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));
          __builtin_amdgcn_s_barrier();
          if (kw == 0) {
#pragma unroll
            for (int s = 0; s < NS; s++) {
              const floatx4 o = red[(s * 8 + wv + TPW) * 64 + lane];
#pragma unroll
              for (int v = 0; v < 4; v++) acc[s][0][v] += o[v];
            }
          }
          __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));
          __builtin_amdgcn_s_barrier();
          if (kw != 0) return;
        }
        // acc[s][j][v] = y[row 16j + 4q + v][column t*16 + nl]
        const int t = tb + ts + TPW * (i / KPW);
        if (t >= te) return;
        const int col = t * 16 + nlo;
        if (col >= N) return;
        XS* yp = yg + (r0 + 4 * qo) * N + col;  // row 4q of the pass
#pragma unroll
        for (int j = 0; j < MT; j++)
#pragma unroll
          for (int v = 0; v < 4; v++) {
            const int m = 16 * j + 4 * qo + v;
            if (m < nrows) {
              // SwiGLU of the two projections, each rounded to the output
              // type first, as the unfused form materialises them
              const float y = SWI ? swiglu_f32(DT_<XDT>::round(acc[0][j][v]), DT_<XDT>::round(acc[NS - 1][j][v]))
                                  : acc[0][j][v];
              yp[(int64_t)(16 * j + v) * N] = xbad[m] ? kNaN : DT_<XDT>::from_f32(y);
            }
          }
      };
      // loads stay out of branches (clamped item indices past the end reload
      // the last item, never computed), so each wait covers only older loads
#pragma nounroll
      for (int i = 0; i < NI; i += 2) {
        issue_sb(bb, i + 1);
        issue_w(bb, i + 1);
        compute(ba, i);
        issue_sb(ba, i + 2);
        issue_w(ba, i + 2);
        if (i + 1 < NI) compute(bb, i + 1);
      }
    };
    const int mt = (nrows + 15) / 16;
    if constexpr (MR == 16) {
      run_items(std::integral_constant<int, 1>{});
    } else if constexpr (MR == 32) {
      if (mt == 1) run_items(std::integral_constant<int, 1>{});
      else run_items(std::integral_constant<int, 2>{});
    } else {
      if (mt == 1) run_items(std::integral_constant<int, 1>{});
      else if (mt == 2) run_items(std::integral_constant<int, 2>{});
      else if (mt == 3) run_items(std::integral_constant<int, 3>{});
      else run_items(std::integral_constant<int, 4>{});
    }
    __syncthreads();  // x, its sums and xbad are rewritten by the next pass
  }
}

template <int XDT, int GS, int KC, bool SWI, bool DENSE = false>
hipError_t run_gqms(const QArgs& a) {
  using SH = GSShape<KC, SWI, DENSE>;
  constexpr int lds = gx_lds_bytes<GS, KC, SWI, DENSE>();
  GSKern k;
  k.y = a.y; k.x = a.x; k.w = a.w; k.s = a.s; k.b = a.b; k.lhs = a.lhs; k.rhs = a.rhs;
  k.w2 = a.w2; k.s2 = a.s2; k.b2 = a.b2;
  k.batch = a.batch; k.x_rep = a.x_rep; k.x_batch = a.x_batch; k.w_batch = a.w_batch;
  k.M = (int)a.M; k.N = (int)a.N; k.K = (int)a.K;
  k.nib_mask = 0x000F000Fu;
  k.off_pair = SMma<XDT>::OFFB;
  k.ntiles = (int)((a.N + 15) / 16);
  // up to 64 weight tiles (16 rows x K) per block; DENSE: groups of the 4
  // tiles its waves work on at once, at most one block per CU (the x rows
  // are staged once per block: lm_head at 8 rows, 2,004 blocks of 4 tiles,
  // staged them 2,004 times). The fused SwiGLU form takes every CU when
  // there are fewer than 4 tiles per CU (8192 x 2048 at 8 rows 13.5 -> 13.1
  // us, 8192 x 4096 21.7 -> 20.8); the plain form measured the same or 1 %
  // slower that way and keeps whole groups of 4.
  const int cus = device_cu_count();
  k.ns = DENSE ? (SWI ? std::min(k.ntiles, cus) : std::min((k.ntiles + SH::TPW - 1) / SH::TPW, cus))
               : (k.ntiles + 63) / 64;
  auto fn = gqms_kernel<XDT, GS, KC, SWI, DENSE>;
  static std::atomic<uint64_t> raised{0};
  hipError_t e = raise_lds_limit(reinterpret_cast<const void*>(fn), lds, raised);
  if (e != hipSuccess) return e;
  dim3 grid((unsigned)k.ns, DENSE ? 1u : (unsigned)(a.w_batch + 1), (unsigned)SH::ZS);
  hipLaunchKernelGGL(fn, grid, dim3(512), lds, a.stream, k);
  return hipGetLastError();
}

template <int XDT, int GS, bool SWI>
hipError_t run_gqms_k(const QArgs& a) {
  switch (a.K / 256) {
    case 2: return run_gqms<XDT, GS, 2, SWI>(a);
    case 3: if constexpr (GS == 64 && !SWI) return run_gqms<XDT, GS, 3, SWI>(a); else break;
    case 4: return run_gqms<XDT, GS, 4, SWI>(a);
    case 8: return run_gqms<XDT, GS, 8, SWI>(a);
    default: break;
  }
  return hipErrorNotSupported;
}

template <int XDT, bool SWI>
hipError_t run_gqms_g(const QArgs& a) {
  return a.group_size == 64 ? run_gqms_k<XDT, 64, SWI>(a) : run_gqms_k<XDT, 128, SWI>(a);
}

template <int XDT, int GS, bool SWI>
hipError_t run_gqms_dense_k(const QArgs& a) {
  switch (a.K / 256) {
    case 8: return run_gqms<XDT, GS, 8, SWI, true>(a);
    case 16: return run_gqms<XDT, GS, 16, SWI, true>(a);
    default: break;
  }
  return hipErrorNotSupported;
}

template <int XDT, int GS>
hipError_t run_gqms_dense_s(const QArgs& a) {
  return a.w2 ? run_gqms_dense_k<XDT, GS, true>(a) : run_gqms_dense_k<XDT, GS, false>(a);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

#define HQ_CAT_(a, b) a##b
#define HQ_CAT(a, b) HQ_CAT_(a, b)

// The streaming grouped kernel, or hipErrorNotSupported for what it does not
// take: other bit widths, group size 32, mixed or fp32 dtypes, K not one of
// 512/768/1024/2048 (768 only at group size 64 and unfused), scales or biases
// not 16-byte aligned, more than 64 rows per expert on average (the
// LDS-dequant GEMM amortises its dequantization there).
hipError_t HQ_CAT(launch_gqms_t_b, HQ_BITS)(const QArgs& a) {
  if constexpr (HQ_BITS != 4) {
    (void)a;
    return hipErrorNotSupported;
  } else {
    // Measured at configs[4] (4096 rows, 128 experts), same box, against the
    // LDS-dequant kernel: down (K = 768) 50-54 us vs 69-72, gate (K = 2048)
    // 50-57 vs 75, the fused gate/up + SwiGLU (K = 2048) 90-94 vs 125-128.
    if (a.xdt != a.sdt || a.xdt == DT_F32 || !a.rhs || a.w_batch + 1 > 65535) return hipErrorNotSupported;
    if (a.group_size != 64 && a.group_size != 128) return hipErrorNotSupported;
    if (a.K % 256 != 0 || a.K > 2048 || a.M > ((int64_t)1 << 30)) return hipErrorNotSupported;
    if (!aligned16(a.s) || !aligned16(a.b)) return hipErrorNotSupported;
    if (a.w2 && (!aligned16(a.s2) || !aligned16(a.b2))) return hipErrorNotSupported;
    if (a.batch * a.M > 64 * a.w_batch) return hipErrorNotSupported;  // few rows per expert
    if (a.w2) return a.xdt == DT_BF16 ? run_gqms_g<DT_BF16, true>(a) : run_gqms_g<DT_F16, true>(a);
    return a.xdt == DT_BF16 ? run_gqms_g<DT_BF16, false>(a) : run_gqms_g<DT_F16, false>(a);
  }
}

// Batched decode through the same kernel (DENSE): one product of 8-16 rows,
// plain or with the fused SwiGLU (both projections per tile), or
// hipErrorNotSupported: other bit widths and groups, mixed or fp32 dtypes,
// K other than 2048 or 4096, N below 8192 (fewer than 512 blocks of 4
// tiles), a linear bias, unaligned scales or biases.
// Measured against the GEMV kernels on the same data (8 rows): 14336 x 4096
// 15.0-15.5 vs 16.6-16.7 us, 14336 x 2048 11.5 vs 15.0, 128256 x 4096 105 vs
// 105; at 4 rows it was slower (15.3 vs 12.2 us), as its cost hardly depends
// on the row count (x staging and group sums for 16 row slots per block).
hipError_t HQ_CAT(launch_gqms_dense_t_b, HQ_BITS)(const QArgs& a) {
  if constexpr (HQ_BITS != 4) {
    (void)a;
    return hipErrorNotSupported;
  } else {
    if (a.lb || a.lhs || a.rhs || a.batch != 1 || a.xdt != a.sdt || a.xdt == DT_F32)
      return hipErrorNotSupported;
    // 4-7 rows only at vocabulary-sized N (its cost hardly depends on the
    // row count: below 8 rows the GEMV kernels win on smaller N)
    if (a.M < (a.N >= 65536 ? 4 : 8) || a.M > 16 || a.N < 8192 || a.N > ((int64_t)1 << 30))
      return hipErrorNotSupported;
    if (a.group_size != 64 && a.group_size != 128) return hipErrorNotSupported;
    if (!aligned16(a.s) || !aligned16(a.b)) return hipErrorNotSupported;
    if (a.w2 && (!aligned16(a.s2) || !aligned16(a.b2))) return hipErrorNotSupported;
    QArgs d = a;
    d.x_batch = 1;
    d.x_rep = 1;
    d.w_batch = 1;
    return a.xdt == DT_BF16 ? (a.group_size == 64 ? run_gqms_dense_s<DT_BF16, 64>(d) : run_gqms_dense_s<DT_BF16, 128>(d))
                            : (a.group_size == 64 ? run_gqms_dense_s<DT_F16, 64>(d) : run_gqms_dense_s<DT_F16, 128>(d));
  }
}

}  // namespace hq
