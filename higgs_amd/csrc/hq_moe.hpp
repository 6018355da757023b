// hq_moe.hpp -- launch interface of hq_moe.hip (MoE index plumbing and the
// elementwise SwiGLU), used by the C ABI in hq_capi.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hq {

struct SortArgs {
  const uint32_t* idx;   // [n] expert index of each (token, slot), token-major
  int64_t n, top_k, E;
  uint32_t* order;       // [n] or null
  uint32_t* inv_order;   // [n] or null
  uint32_t* idx_sorted;  // [n] or null
  uint32_t* token_idx;   // [n] or null
  hipStream_t stream;
};

struct CombineArgs {
  void* out;                 // [tokens, D]
  const void* y;             // [tokens * top_k, D] rows in sorted order
  const uint32_t* inv_order; // [tokens * top_k]
  const void* scores;        // [tokens, top_k]
  int64_t tokens, top_k, D;
  int dt, sdt;               // dtype of y / out, dtype of scores
  hipStream_t stream;
};

// Largest expert count the one-block sort takes (its LDS holds 17 counters
// per bucket).
constexpr int64_t kSortMaxExperts = 2048;

size_t moe_sort_lds(int64_t E);
hipError_t launch_moe_sort(const SortArgs& a);
hipError_t launch_moe_combine(const CombineArgs& a);
hipError_t launch_swiglu(const void* gate, const void* up, void* out, int64_t n, int dt,
                         hipStream_t stream);

}  // namespace hq
