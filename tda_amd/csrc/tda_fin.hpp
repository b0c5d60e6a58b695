// tda_fin.hpp -- the fixed-order sum of the backward's dbeta / dlambda partials (bwd_finish,
// tda_bwd.hip).
#pragma once

#include <type_traits>

#include "tda_common.hpp"
#include "tda_params.hpp"

namespace tda {

// ------------------------------------------------------------------ dbeta / dlambda sums
// The backward's partial pairs ws[2 k], ws[2 k + 1] (k < items, one per (branch, head, query
// tile)) are summed in one fixed order, whichever kernel does it: kFinSlices slices of
// per = ceil(items / kFinSlices) consecutive items, each summed in fp64 in item order; then one
// wave adds slices l, l + 64, .. on lane l in slice order, and pairwise lane sums (lane i with
// i ^ 1, i ^ 2 by quad permutes, with 7 - i and 15 - i within 16-lane rows, then i ^ 16, i ^ 32;
// each step adds two values in either order, so every lane ends with the same bits).
__device__ __forceinline__ int64_t fin_per(int64_t items) { return (items + kFinSlices - 1) / kFinSlices; }
// slice s summed by one thread: the partials of 16 items (8 16-byte loads) in flight at a time
__device__ __forceinline__ double2 fin_slice_sum(const float* ws, int64_t items, int s) {
  const int64_t per = fin_per(items), i0 = (int64_t)s * per, i1 = min(items, i0 + per);
  double a = 0.0, c = 0.0;
  int64_t k = i0;
  if ((k & 1) && k < i1) {  // to an even item: 16-byte aligned pairs of items from here
    a += (double)ws[2 * k];
    c += (double)ws[2 * k + 1];
    ++k;
  }
  const f32x4* w4 = reinterpret_cast<const f32x4*>(ws);
  for (; k + 16 <= i1; k += 16) {
    f32x4 v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = w4[k / 2 + u];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      a += (double)v[u][0];
      c += (double)v[u][1];
      a += (double)v[u][2];
      c += (double)v[u][3];
    }
  }
  for (; k < i1; ++k) {
    a += (double)ws[2 * k];
    c += (double)ws[2 * k + 1];
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
  // lane swaps: DPP moves of both 32-bit halves within 16-lane rows, then across rows
  auto dpp64 = [](double x, auto ctrl) {
    constexpr int C = decltype(ctrl)::value;
    const int2 h = __builtin_bit_cast(int2, x);
    return __builtin_bit_cast(double, int2{__builtin_amdgcn_mov_dpp(h.x, C, 0xF, 0xF, false),
                                           __builtin_amdgcn_mov_dpp(h.y, C, 0xF, 0xF, false)});
  };
  using q1 = std::integral_constant<int, 0xB1>;
  using q2 = std::integral_constant<int, 0x4E>;
  using hm = std::integral_constant<int, 0x141>;
  using rm = std::integral_constant<int, 0x140>;
  a += dpp64(a, q1{});
  c += dpp64(c, q1{});
  a += dpp64(a, q2{});
  c += dpp64(c, q2{});
  a += dpp64(a, hm{});
  c += dpp64(c, hm{});
  a += dpp64(a, rm{});
  c += dpp64(c, rm{});
  a += __shfl_xor(a, 16);
  c += __shfl_xor(c, 16);
  a += __shfl_xor(a, 32);
  c += __shfl_xor(c, 32);
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
