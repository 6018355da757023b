// hq_moe.hip -- the index and elementwise work around the MoE grouped GEMM:
// the global sort of expert indices, the score-weighted unsort-combine, and
// the elementwise SwiGLU. Compiled once (no bit width).
//
// The reference runs these as MLX ops (argsort, take, floor_divide, sigmoid,
// multiply, sum) around three gather_qmm calls:
//   crates/higgs-models/src/qwen3_next.rs:1746-1761  order / inv_order /
//       token_idx / idx_sorted (forward_gather_global_sort)
//   crates/higgs-models/src/qwen3_next.rs:1802-1808  out_flat.take(inv_order)
//   crates/higgs-models/src/qwen3_moe.rs:355-357     y * scores, sum over top_k
//   crates/higgs-models/src/qwen3_next.rs:340-342    swiglu(gate, up)
#include "hq_common.hpp"
#include "hq_device.hpp"
#include "hq_moe.hpp"

namespace hq {

namespace {

// ---------------------------------------------------------------------------
// Stable counting sort of n expert indices, one block of 1024 threads.
// Bucket of an index: the index itself, or E for every index >= E (those
// keep their original order after all valid ones). Keys are read in
// super-chunks of kSortKeys = 16 per thread (all loads of a super-chunk in
// flight at once; for n <= 16384 they stay in registers for both passes).
// Pass 1 counts buckets (LDS atomics) and scans them into start offsets.
// Pass 2 walks the keys in chunks of 1024, in order: a wave ranks each key
// among the equal-bucket lanes before it (ballots over the bucket bits), the
// waves' per-bucket counts give the offset of earlier waves, and the running
// per-bucket base gives the offset of earlier chunks. So the output position
// of element i is (start of its bucket) + (number of equal-bucket elements
// before i): the stable order, i.e. argsort with ties by position.
// ---------------------------------------------------------------------------
constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / 64;
constexpr int kSortKeys = 16;
constexpr int64_t kSortSuper = (int64_t)kSortThreads * kSortKeys;

__global__ __launch_bounds__(kSortThreads) void moe_sort_kernel(SortArgs a) {
  extern __shared__ int sm[];
  const int NB = a.E + 1;                  // buckets
  int* base = sm;                          // [NB] running start of each bucket
  int* cnt = sm + NB;                      // [kSortWaves][NB] per-wave counts of a chunk
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int64_t n = a.n;
  const uint32_t E = (uint32_t)a.E;

  // bucket keys of super-chunk sc0 (0xffffffff past n)
  uint32_t key[kSortKeys];
  auto load_keys = [&](int64_t sc0) {
#pragma unroll
    for (int j = 0; j < kSortKeys; j++) {
      const int64_t i = sc0 + (int64_t)j * kSortThreads + tid;
      const uint32_t k = i < n ? a.idx[i] : 0xffffffffu;
      key[j] = i < n ? (k < E ? k : E) : 0xffffffffu;
    }
  };

  for (int b = tid; b < NB; b += kSortThreads) base[b] = 0;
  for (int j = tid; j < kSortWaves * NB; j += kSortThreads) cnt[j] = 0;
  __syncthreads();
  for (int64_t sc0 = 0; sc0 < n; sc0 += kSortSuper) {
    load_keys(sc0);
#pragma unroll
    for (int j = 0; j < kSortKeys; j++)
      if (key[j] != 0xffffffffu) atomicAdd(&base[key[j]], 1);
  }
  __syncthreads();
  // exclusive scan of base[0..NB): each thread scans a contiguous run, the
  // run totals are scanned by wave 0 (in the first 1024 entries of cnt, which
  // holds at least that many and is cleared again below).
  {
    const int per = (NB + kSortThreads - 1) / kSortThreads;
    const int b0 = tid * per, b1 = min(b0 + per, NB);
    int run = 0;
    for (int b = b0; b < b1; b++) run += base[b];
    cnt[tid] = run;
    __syncthreads();
    if (wv == 0) {
      int v[16], s = 0;
#pragma unroll
      for (int j = 0; j < 16; j++) { v[j] = cnt[lane * 16 + j]; s += v[j]; }
      int inc = s;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(inc, o, 64);
        if (lane >= o) inc += t;
      }
      int ex = inc - s;
#pragma unroll
      for (int j = 0; j < 16; j++) { const int t = v[j]; cnt[lane * 16 + j] = ex; ex += t; }
    }
    __syncthreads();
    int off = cnt[tid];
    for (int b = b0; b < b1; b++) { const int t = base[b]; base[b] = off; off += t; }
    __syncthreads();
    cnt[tid] = 0;
    __syncthreads();
  }

  const int kbits = 32 - __clz(NB);  // bits of a bucket number
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int64_t sc0 = 0; sc0 < n; sc0 += kSortSuper) {
    if (n > kSortSuper) load_keys(sc0);
#pragma unroll
    for (int j = 0; j < kSortKeys; j++) {
      const int64_t c0 = sc0 + (int64_t)j * kSortThreads;
      if (c0 >= n) break;
      const int64_t i = c0 + tid;
      const bool valid = key[j] != 0xffffffffu;
      const uint32_t kb = valid ? key[j] : 0u;
      // lanes of this wave with the same bucket
      uint64_t peers = __ballot(valid);
      for (int bit = 0; bit < kbits; bit++) {
        const bool on = (kb >> bit) & 1u;
        const uint64_t m = __ballot(on);
        peers &= on ? m : ~m;
      }
      const int rank = __popcll(peers & lt);
      if (valid && rank == 0) cnt[wv * NB + kb] = __popcll(peers);
      __syncthreads();
      if (valid) {
        int pos = base[kb] + rank;
        for (int w = 0; w < wv; w++) pos += cnt[w * NB + kb];
        if (a.order) a.order[pos] = (uint32_t)i;
        if (a.inv_order) a.inv_order[i] = (uint32_t)pos;
        if (a.idx_sorted) a.idx_sorted[pos] = kb < E ? kb : a.idx[i];
        if (a.token_idx) a.token_idx[pos] = (uint32_t)(i / a.top_k);
      }
      __syncthreads();
      // advance each bucket's base by this chunk's count and clear the counts
      for (int b = tid; b < NB; b += kSortThreads) {
        int s = 0;
        for (int w = 0; w < kSortWaves; w++) {
          s += cnt[w * NB + b];
          cnt[w * NB + b] = 0;
        }
        base[b] += s;
      }
      __syncthreads();
    }
  }
}

// ---------------------------------------------------------------------------
// The same stable counting sort for n <= kSortSuper in three phases with
// three block barriers: wave w owns the contiguous elements [w L, (w+1) L)
// (L a multiple of 64, keys in registers) and counts them per bucket (LDS
// atomics); one thread per bucket turns the per-wave counts into per-wave
// offsets and bucket totals, which a block scan turns into bucket starts;
// then each wave places its elements in order, 64 at a time, with no further
// barrier (a wave ranks a key among the equal-bucket lanes before it, and the
// first lane of each bucket advances the wave's offset for that bucket).
// STAGE (when the LDS holds 8 n more bytes): the placement writes the sorted
// arrays into LDS, and one coalesced pass copies them out (scattered 4-byte
// stores from the one workgroup were most of its time).
// ---------------------------------------------------------------------------
template <bool STAGE>
__global__ __launch_bounds__(kSortThreads) void moe_sort_small_kernel(SortArgs a) {
  extern __shared__ int sm[];
  const int NB = a.E + 1;                  // buckets
  int* start = sm;                         // [NB] bucket totals, then starts
  int* cnt = sm + NB;                      // [kSortWaves][NB] per-wave counts, then offsets
  int* runs = cnt + kSortWaves * NB;       // [kSortThreads] scan of per-thread runs
  uint32_t* ord = reinterpret_cast<uint32_t*>(runs + kSortThreads);  // STAGE: [n] order
  uint32_t* kv = ord + a.n;                                          // STAGE: [n] sorted indices
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int n = (int)a.n;
  const uint32_t E = (uint32_t)a.E;
  const int L = (n + 64 * kSortWaves - 1) / (64 * kSortWaves) * 64;  // elements per wave
  const int SC = L / 64;                                              // <= kSortKeys

  for (int j = tid; j < kSortWaves * NB; j += kSortThreads) cnt[j] = 0;
  uint32_t key[kSortKeys];  // bucket of element wv L + 64 c + lane, 0xffffffff past n
#pragma unroll
  for (int c = 0; c < kSortKeys; c++) {
    const int i = wv * L + 64 * c + lane;
    const bool in = c < SC && i < n;
    const uint32_t k = in ? a.idx[i] : 0u;
    key[c] = in ? (k < E ? k : E) : 0xffffffffu;
  }
  __syncthreads();
#pragma unroll
  for (int c = 0; c < kSortKeys; c++)
    if (key[c] != 0xffffffffu) atomicAdd(&cnt[wv * NB + key[c]], 1);
  __syncthreads();
  // per bucket: exclusive prefix over the waves (in place) and the total
  for (int b = tid; b < NB; b += kSortThreads) {
    int s = 0;
#pragma unroll
    for (int w = 0; w < kSortWaves; w++) {
      const int t = cnt[w * NB + b];
      cnt[w * NB + b] = s;
      s += t;
    }
    start[b] = s;
  }
  __syncthreads();
  // exclusive scan of the totals: each thread a contiguous run, wave 0 scans
  // the run sums
  {
    const int per = (NB + kSortThreads - 1) / kSortThreads;
    const int b0 = min(tid * per, NB), b1 = min(b0 + per, NB);
    int run = 0;
    for (int b = b0; b < b1; b++) run += start[b];
    runs[tid] = run;
    __syncthreads();
    if (wv == 0) {
      int v[16], s = 0;
#pragma unroll
      for (int j = 0; j < 16; j++) { v[j] = runs[lane * 16 + j]; s += v[j]; }
      int inc = s;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(inc, o, 64);
        if (lane >= o) inc += t;
      }
      int ex = inc - s;
#pragma unroll
      for (int j = 0; j < 16; j++) { const int t = v[j]; runs[lane * 16 + j] = ex; ex += t; }
    }
    __syncthreads();
    int off = runs[tid];
    for (int b = b0; b < b1; b++) { const int t = start[b]; start[b] = off; off += t; }
  }
  __syncthreads();

  const int kbits = 32 - __clz(NB);  // bits of a bucket number
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int* woff = cnt + wv * NB;         // this wave's running offsets
#pragma unroll
  for (int c = 0; c < kSortKeys; c++) {
    if (c >= SC) break;              // wave-uniform
    const int i = wv * L + 64 * c + lane;
    const bool valid = key[c] != 0xffffffffu;
    const uint32_t kb = valid ? key[c] : 0u;
    uint64_t peers = __ballot(valid);
    for (int bit = 0; bit < kbits; bit++) {
      const bool on = (kb >> bit) & 1u;
      const uint64_t m = __ballot(on);
      peers &= on ? m : ~m;
    }
    const int rank = __popcll(peers & lt);
    const int pos = valid ? start[kb] + woff[kb] + rank : 0;
    if (valid) {
      if (a.inv_order) a.inv_order[i] = (uint32_t)pos;
      const uint32_t sv = kb < E ? kb : a.idx[i];
      if constexpr (STAGE) {
        ord[pos] = (uint32_t)i;
        kv[pos] = sv;
      } else {
        if (a.order) a.order[pos] = (uint32_t)i;
        if (a.idx_sorted) a.idx_sorted[pos] = sv;
        if (a.token_idx) a.token_idx[pos] = (uint32_t)i / (uint32_t)a.top_k;
      }
    }
    // every lane has read woff above (a wave's LDS accesses complete in
    // order); the first lane of each bucket advances it
    asm volatile("" ::: "memory");
    if (valid && rank == 0) woff[kb] += __popcll(peers);
    asm volatile("" ::: "memory");
  }
  if constexpr (STAGE) {
    __syncthreads();
    for (int p = tid; p < n; p += kSortThreads) {
      const uint32_t i = ord[p];
      if (a.order) a.order[p] = i;
      if (a.idx_sorted) a.idx_sorted[p] = kv[p];
      if (a.token_idx) a.token_idx[p] = i / (uint32_t)a.top_k;
    }
  }
}

// ---------------------------------------------------------------------------
// out[t, d] = sum_j round(scores[t, j] * y[inv[t*k + j], d]), j in order,
// fp32 sum, one rounding to the output dtype. Rows with inv out of range
// give NaN. VEC elements per thread (8 when D % 8 == 0).
// ---------------------------------------------------------------------------
template <int DT, int SDT, int VEC>
__global__ __launch_bounds__(256) void moe_combine_kernel(CombineArgs a) {
  using ST = st_t<DT>;
  const int64_t per_row = a.D / VEC;
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= a.tokens * per_row) return;
  const int64_t t = g / per_row, d0 = (g - t * per_row) * VEC;
  const int64_t rows = a.tokens * a.top_k;
  float acc[VEC];
#pragma unroll
  for (int v = 0; v < VEC; v++) acc[v] = 0.f;
  bool bad = false;
  // slots in batches of 8: the index and score loads of a batch, then its row
  // loads, are issued together (no load waits on the previous slot's)
  constexpr int JB = 8;
  for (int64_t j0 = 0; j0 < a.top_k; j0 += JB) {
    uint32_t r[JB];
    float sc[JB];
#pragma unroll
    for (int jj = 0; jj < JB; jj++) {
      const int64_t j = min(j0 + jj, a.top_k - 1);
      r[jj] = a.inv_order[t * a.top_k + j];
      sc[jj] = DT_<SDT>::load((const st_t<SDT>*)a.scores, t * a.top_k + j);
    }
    float yv[JB][VEC];
#pragma unroll
    for (int jj = 0; jj < JB; jj++) {
      const bool ok = (int64_t)r[jj] < rows;
      if (j0 + jj < a.top_k && !ok) bad = true;
      const ST* yp = (const ST*)a.y + (ok ? (int64_t)r[jj] : 0) * a.D + d0;
      if constexpr (VEC == 8) load8_f32<DT>(yp, yv[jj]);
      else yv[jj][0] = DT_<DT>::load(yp, 0);
    }
#pragma unroll
    for (int jj = 0; jj < JB; jj++) {
      if (j0 + jj >= a.top_k) break;
#pragma unroll
      for (int v = 0; v < VEC; v++) acc[v] += DT_<DT>::round(sc[jj] * yv[jj][v]);
    }
  }
  ST* op = (ST*)a.out + t * a.D + d0;
#pragma unroll
  for (int v = 0; v < VEC; v++)
    op[v] = DT_<DT>::from_f32(bad ? __uint_as_float(0x7fc00000u) : acc[v]);
}

// out[i] = round(swiglu(gate[i], up[i])), gate and up in the output dtype.
template <int DT>
__global__ __launch_bounds__(256) void swiglu_kernel(const void* gate, const void* up, void* out,
                                                     int64_t n) {
  using ST = st_t<DT>;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float g = DT_<DT>::load((const ST*)gate, i), u = DT_<DT>::load((const ST*)up, i);
  ((ST*)out)[i] = DT_<DT>::from_f32(swiglu_f32(g, u));
}

}  // namespace

// base [E + 1] and cnt [max(16 * (E + 1), 1024)] (the scan reuses cnt for
// the 1024 per-thread run totals).
size_t moe_sort_lds(int64_t E) {
  const int64_t nb = E + 1;
  const int64_t c = kSortWaves * nb > kSortThreads ? kSortWaves * nb : kSortThreads;
  return (size_t)(nb + c) * sizeof(int);
}

// [E + 1] bucket starts, [16 (E + 1)] per-wave offsets, [1024] scan runs
size_t moe_sort_small_lds(int64_t E) { return (size_t)((E + 1) * (1 + kSortWaves) + kSortThreads) * sizeof(int); }

namespace {
template <bool STAGE>
hipError_t launch_moe_sort_small(const SortArgs& a, size_t lds) {
  static std::atomic<uint64_t> raised{0};
  if (lds > 64 * 1024) {
    hipError_t e = raise_lds_limit(reinterpret_cast<const void*>(moe_sort_small_kernel<STAGE>), 160 * 1024, raised);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(moe_sort_small_kernel<STAGE>, dim3(1), dim3(kSortThreads), lds, a.stream, a);
  return hipGetLastError();
}
}  // namespace

hipError_t launch_moe_sort(const SortArgs& a) {
  if (a.n <= kSortSuper) {
    const size_t lds = moe_sort_small_lds(a.E), staged = lds + (size_t)a.n * 8;
    if (staged <= 160 * 1024) return launch_moe_sort_small<true>(a, staged);
    return launch_moe_sort_small<false>(a, lds);
  }
  const size_t lds = moe_sort_lds(a.E);
  static std::atomic<uint64_t> raised{0};
  if (lds > 64 * 1024) {
    hipError_t e = raise_lds_limit(reinterpret_cast<const void*>(moe_sort_kernel), 160 * 1024, raised);
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(moe_sort_kernel, dim3(1), dim3(kSortThreads), lds, a.stream, a);
  return hipGetLastError();
}

template <int DT, int SDT>
static hipError_t combine_dt(const CombineArgs& a) {
  const bool v8 = (a.D % 8) == 0;
  const int64_t work = a.tokens * (v8 ? a.D / 8 : a.D);
  const dim3 grid((unsigned)((work + 255) / 256));
  if (v8)
    hipLaunchKernelGGL((moe_combine_kernel<DT, SDT, 8>), grid, dim3(256), 0, a.stream, a);
  else
    hipLaunchKernelGGL((moe_combine_kernel<DT, SDT, 1>), grid, dim3(256), 0, a.stream, a);
  return hipGetLastError();
}

template <int DT>
static hipError_t combine_sdt(const CombineArgs& a) {
  switch (a.sdt) {
    case DT_F32: return combine_dt<DT, DT_F32>(a);
    case DT_F16: return combine_dt<DT, DT_F16>(a);
    default: return combine_dt<DT, DT_BF16>(a);
  }
}

hipError_t launch_moe_combine(const CombineArgs& a) {
  switch (a.dt) {
    case DT_F32: return combine_sdt<DT_F32>(a);
    case DT_F16: return combine_sdt<DT_F16>(a);
    default: return combine_sdt<DT_BF16>(a);
  }
}

hipError_t launch_swiglu(const void* gate, const void* up, void* out, int64_t n, int dt,
                         hipStream_t stream) {
  const dim3 grid((unsigned)((n + 255) / 256));
  switch (dt) {
    case DT_F32: hipLaunchKernelGGL(swiglu_kernel<DT_F32>, grid, dim3(256), 0, stream, gate, up, out, n); break;
    case DT_F16: hipLaunchKernelGGL(swiglu_kernel<DT_F16>, grid, dim3(256), 0, stream, gate, up, out, n); break;
    default: hipLaunchKernelGGL(swiglu_kernel<DT_BF16>, grid, dim3(256), 0, stream, gate, up, out, n); break;
  }
  return hipGetLastError();
}

}  // namespace hq
