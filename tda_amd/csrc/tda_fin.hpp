// tda_fin.hpp -- the fixed-order sum of the backward's dbeta / dlambda partials (bwd_finish,
// tda_bwd.hip).
#pragma once

#include "tda_common.hpp"
#include "tda_params.hpp"

namespace tda {

// ------------------------------------------------------------------ dbeta / dlambda sums
// The backward's partial pairs ws[2 k], ws[2 k + 1] (k < items, one per (branch, head, query
// tile)) are summed in one fixed order, whichever kernel does it: kFinSlices slices of
// per = ceil(items / kFinSlices) consecutive items, each summed in fp64 in item order; then one
// wave adds slices l, l + 64, .. on lane l in slice order and a butterfly over the 64 lanes (each
// step adds two values in either order, so every lane ends with the same bits).
__device__ __forceinline__ int64_t fin_per(int64_t items) { return (items + kFinSlices - 1) / kFinSlices; }
// slice s summed by one thread (the loads of eight items in flight at a time)
__device__ __forceinline__ double2 fin_slice_sum(const float* ws, int64_t items, int s) {
  const int64_t per = fin_per(items), i0 = (int64_t)s * per, i1 = min(items, i0 + per);
  const float2* w2 = reinterpret_cast<const float2*>(ws);
  double a = 0.0, c = 0.0;
  int64_t k = i0;
  for (; k + 8 <= i1; k += 8) {
    float2 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = w2[k + u];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      a += (double)v[u].x;
      c += (double)v[u].y;
    }
  }
  for (; k < i1; ++k) {
    a += (double)w2[k].x;
    c += (double)w2[k].y;
  }
  return double2{a, c};
}
// the total of the kFinSlices slice sums (sl: [kFinSlices][2]), by one wave
__device__ __forceinline__ double2 fin_total(const double* sl) {
  const int l = lane_id();
  double a = 0.0, c = 0.0;
  for (int r = 0; r < kFinSlices / 64; ++r) {
    const int k = l + 64 * r;
    a += sl[2 * k];
    c += sl[2 * k + 1];
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    a += __shfl_xor(a, o);
    c += __shfl_xor(c, o);
  }
  return double2{a, c};
}
// dbeta, and dlambda through torch.clamp's gate (gradient passed on [0, 1])
__device__ __forceinline__ void fin_store(double2 t, const float* lam, float* dbeta, float* dlam, int branches) {
  if (dbeta) dbeta[0] = (float)t.x;
  if (dlam && branches == 2) {
    const float lv = lam[0];
    dlam[0] = lv >= 0.f && lv <= 1.f ? (float)t.y : 0.f;
  }
}

}  // namespace tda
