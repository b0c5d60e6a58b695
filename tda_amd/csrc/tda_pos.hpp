// tda_pos.hpp -- device helpers for query positions, causal tile ranges and the norm table
// layout of the gfx950 threshold-attention kernels (the conventions are stated in
// tda_params.hpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tda_params.hpp"

namespace tda {

// Element offset of row 0 of head bh in norm slot `slot` (see NormSlot).
template <class PP>
__device__ __forceinline__ int64_t norm_base(const PP& P, int slot, int bh) {
  const int64_t bhs = (int64_t)P.B * P.H, q = bhs * P.Nq, k = bhs * P.Nk;
  const int64_t s0 = slot == N_Q1 ? 0 : slot == N_K1 ? q : slot == N_Q2 ? q + k : 2 * q + k;
  return s0 + (int64_t)bh * ((slot & 1) ? P.Nk : P.Nq);
}
// Last key tile holding a key visible to some row of query tile qt (rows at positions
// qoff + 32 qt .. qoff + 32 qt + 31).
__device__ __forceinline__ int kt_last(int qt, int qoff, int nkt) {
  const int t = (qoff + 32 * qt + 31) >> 5;
  return t < nkt - 1 ? t : nkt - 1;
}
// First query tile one of whose rows sees some key of key tile kt; qt >= qt_first(kt) is
// exactly kt <= (qoff + 32 qt + 31) / 32.
__device__ __forceinline__ int qt_first(int kt, int qoff) {
  const int t = (32 * kt - qoff) >> 5;  // floor division
  return t > 0 ? t : 0;
}

}  // namespace tda
