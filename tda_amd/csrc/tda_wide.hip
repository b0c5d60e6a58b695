// tda_wide.hip -- threshold attention at head_dim 256 (fp32 and bf16) for gfx950.
//
// Reference semantics (snap-research/TDA triton_threshold_attention.py, "TTA"): the forward
// kernel TTA:19-115 and the backward kernels TTA:118-324, whose BLOCK_D is the head_dim for any
// power of two (TTA:366-368, :431); the differential combine and normalisation TTA:489-519.
//
// At d = 256 a 32-row tile's output accumulators alone take 128 registers per lane, and its
// resident row fragments as many again per operand, so these kernels split the work by output
// column: every wave owns one half (128 columns) of the output rows of its tile, and computes
// the scores (contractions over all 256 elements) itself, streaming both operands' rows from
// memory in chunks instead of keeping either resident.  The two halves of a tile recompute the
// same scores bit for bit (the same operations on the same values), so they take the same
// decisions.  Launches:
//   wide_norms    inverse L2 norms of every q1, k1 (q2, k2) row into the norms table
//                 (normalise only); the other kernels read them from there.
//   wide_fwd      one wave per (query tile, half, head): every causal key tile's scores of both
//                 branches, the exact threshold test, and out_half += coef A V_half where the
//                 tile holds a non-zero weight; the half-0 wave writes the tile-occupancy
//                 bitmask and the counters.
//   wide_bwd_dq   one workgroup of two waves (the halves) per (query tile, head): the bitmask's
//                 tiles, dS = coef G (dO . v), dq^_half += dS rk k_half, the dbeta / dlambda
//                 partials (half 0), and the normalize backward, whose row dot q^ . dq^ the
//                 halves add through LDS.
//   wide_bwd_dkv  the same per (key tile, head): dv_half, dk^_half and the normalize backward.
// followed by the fixed-order dbeta / dlambda sum (bwd_finish, tda_bwd.hip).
#include "tda_common.hpp"
#include "tda_params.hpp"
#include "tda_pos.hpp"

namespace tda {
namespace {

constexpr int WD = 256;  // head_dim of this path
constexpr int WH = 128;  // output columns of one wave (one half of the row)

template <class Pol> struct WTile;
template <> struct WTile<PolBF16> { using type = TTileBF16<WH>; };
template <> struct WTile<PolF32> { using type = TTileF32<WH>; };

// acc += A B^T over the 256 elements of rows ra (A: lane (m, g) supplies row m) and rb (B: lane
// (n, g) supplies row n); a null row reads as zeros.  Both operands take their elements in the
// same order, streamed from memory four MFMA steps at a time (nothing resident).
template <class Pol>
__device__ __forceinline__ f32x16 dot256(const typename Pol::T* ra, const typename Pol::T* rb, int g, f32x16 acc) {
  if constexpr (sizeof(typename Pol::T) == 2) {
    // bf16: step t takes elements 16 t + 8 g .. + 7 (16 steps)
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      bf16x8 a[4], b[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = 16 * (4 * c + u) + 8 * g;
        a[u] = ra ? *reinterpret_cast<const bf16x8*>(ra + e) : bf16x8{};
        b[u] = rb ? *reinterpret_cast<const bf16x8*>(rb + e) : bf16x8{};
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) acc = Pol::mma(a[u], b[u], acc);
    }
  } else {
    // fp32: lane half g takes elements 128 g .. 128 g + 127, one per step (128 steps)
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      f32x4 a[4], b[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = 128 * g + 16 * c + 4 * u;
        a[u] = ra ? *reinterpret_cast<const f32x4*>(ra + e) : f32x4{0.f, 0.f, 0.f, 0.f};
        b[u] = rb ? *reinterpret_cast<const f32x4*>(rb + e) : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int x = 0; x < 4; ++x) acc = Pol::mma(a[u][x], b[u][x], acc);
    }
  }
  return acc;
}

// The same tensor view with its base moved to column WH * hh (the wave's half of each row).
template <class T>
__device__ __forceinline__ TRef<T> half_of(const TRef<T>& x, int hh) {
  return TRef<T>{x.p + WH * hh, x.sb, x.sh, x.st};
}

template <class Pol, class TT>
__device__ __forceinline__ void wide_stage(TT& tt, const TRef<const typename Pol::T>& x, int b, int h, int r0, int n) {
  if constexpr (sizeof(typename Pol::T) == 2) {
    tt.stage(x, b, h, r0, n);
    wave_lds_sync();
  } else {
    tt.set(x, b, h, r0, n);
  }
}
template <class Pol, class TT>
__device__ __forceinline__ void wide_release(TT&) {
  if constexpr (sizeof(typename Pol::T) == 2) wave_lds_sync();
}

// acc (this wave's 128 columns of a row, transposed C layout: lane = row, value r of column block
// c = column 32 c + crow(r, g) of the half) += tile^T e, e a 32 x 32 C tile packed as B operands.
template <class Pol, class TT>
__device__ __forceinline__ void acc_tile(f32x16 (&acc)[WH / 32], const TT& tt, const f32x16& e) {
  constexpr int NS = 32 / Pol::KS;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const typename Pol::frag bp = Pol::pack_c(e, s);
#pragma unroll
    for (int c = 0; c < WH / 32; ++c) acc[c] = Pol::mma(tt.frag(s, c), bp, acc[c]);
  }
}

// Partial dot x^ . acc over this wave's half of the row (x^ = x rinv), the same in both lanes of
// the row.
template <class T>
__device__ __forceinline__ float half_dot(const f32x16 (&acc)[WH / 32], const T* xrow, float rinv) {
  const int g = lane_id() >> 5;
  float dot = 0.f;
  if (xrow) {
#pragma unroll
    for (int c = 0; c < WH / 32; ++c)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const f32x4 x = load4(xrow + 32 * c + 8 * u + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) dot = __builtin_fmaf(x[e] * rinv, acc[c][4 * u + e], dot);
      }
  }
  return dot + __shfl_xor(dot, 32);
}

// Store this wave's half of a gradient row: with NORM the F.normalize backward
// (acc - x^ dot) rinv with dot the whole row's x^ . acc (acc rinv when |x| <= eps), else acc.
template <bool NORM, class T>
__device__ __forceinline__ void half_store(const f32x16 (&acc)[WH / 32], const T* xrow, T* grow, float rinv,
                                           float dot) {
  if (!grow) return;
  const int g = lane_id() >> 5;
  const bool clamped = rinv >= 1.0f / kNormEps;
#pragma unroll
  for (int c = 0; c < WH / 32; ++c)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float o[4];
      if constexpr (NORM) {
        const f32x4 x = load4(xrow + 32 * c + 8 * u + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a = acc[c][4 * u + e];
          o[e] = clamped ? a * rinv : (a - x[e] * rinv * dot) * rinv;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = acc[c][4 * u + e];
      }
      store4(grow + 32 * c + 8 * u + 4 * g, o[0], o[1], o[2], o[3]);
    }
}

// ------------------------------------------------------------------ wide_norms
// 1 / max(|x|, eps) of every row of q1, k1 (, q2, k2) into the norms table, flat index f:
// sixteen lanes per row, sixteen elements per lane, the sum of squares by DPP within the group.
template <class T, int BR>
__global__ void __launch_bounds__(256) wide_norms(FwdParams P) {
  const int l = lane_id(), sub = l & 15;
  const int64_t BH = (int64_t)P.B * P.H, q = BH * P.Nq, k = BH * P.Nk;
  const int64_t total = BR * (q + k);
  const int64_t f = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 4 + (l >> 4);
  const bool live = f < total;
  const int64_t ff = live ? f : 0;
  int slot;
  int64_t off;
  if (ff < q) slot = N_Q1, off = ff;
  else if (ff < q + k) slot = N_K1, off = ff - q;
  else if (ff < 2 * q + k) slot = N_Q2, off = ff - q - k;
  else slot = N_K2, off = ff - 2 * q - k;
  const int rows = (slot & 1) ? P.Nk : P.Nq;
  const int bh = (int)(off / rows), t = (int)(off % rows);
  const int fs = slot == N_Q1 ? F_Q1 : slot == N_K1 ? F_K1 : slot == N_Q2 ? F_Q2 : F_K2;
  const T* row = (const T*)P.in[fs] + (int64_t)(bh / P.H) * P.s[fs][0] + (int64_t)(bh % P.H) * P.s[fs][1] +
                 (int64_t)t * P.s[fs][2] + 16 * sub;
  float a = 0.f, c = 0.f;
  if constexpr (sizeof(T) == 2) {
    const bf16x8 v0 = *reinterpret_cast<const bf16x8*>(row), v1 = *reinterpret_cast<const bf16x8*>(row + 8);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a = __builtin_fmaf((float)v0[e], (float)v0[e], a);
      c = __builtin_fmaf((float)v1[e], (float)v1[e], c);
    }
  } else {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(row + 4 * u);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (u < 2) a = __builtin_fmaf(v[e], v[e], a);
        else c = __builtin_fmaf(v[e], v[e], c);
      }
    }
  }
  const float ss = group_sum<16>(a + c);
  if (live && sub == 0) P.norms[f] = inv_norm(ss);
}

// ------------------------------------------------------------------ wide_fwd
// One wave per (query tile, half, head), four independent waves per workgroup, longest query
// tiles first.  Score tiles S^T = K Q^T (lane = query, values = 16 keys of the tile), as in the
// d <= 128 kernels; the weights pack into the B operand of out_half^T += V_half^T A^T.
template <class Pol, int BR, int PK, bool NORM>
__global__ void __launch_bounds__(256) wide_fwd(FwdParams P) {
  using T = typename Pol::T;
  using TT = typename WTile<Pol>::type;
  constexpr int ND = WH / 32;
  const int l = lane_id(), n32 = l & 31, g = l >> 5, wv = threadIdx.x >> 6;
  const int BH = P.B * P.H;
  const int64_t item = (int64_t)blockIdx.x * 4 + wv;
  if (item >= (int64_t)BH * P.nqt * 2) return;  // whole wave leaves; no workgroup barriers below
  const int hh = (int)(item & 1);
  const int64_t pair = item >> 1;
  const int qt = P.nqt - 1 - (int)(pair / BH);
  const int bh = (int)(pair % BH);
  const int b = bh / P.H, h = bh % P.H;
  const int Nq = P.Nq, Nk = P.Nk, qoff = P.qoff;
  const int i = qt * 32 + n32;
  const bool qvalid = i < Nq;
  const int pq = qoff + i;
  const int ktl = kt_last(qt, qoff, P.nkt);

  const TRef<const T> q1{(const T*)P.in[0], P.s[F_Q1][0], P.s[F_Q1][1], P.s[F_Q1][2]};
  const TRef<const T> k1{(const T*)P.in[1], P.s[F_K1][0], P.s[F_K1][1], P.s[F_K1][2]};
  const TRef<const T> q2{(const T*)P.in[2], P.s[F_Q2][0], P.s[F_Q2][1], P.s[F_Q2][2]};
  const TRef<const T> k2{(const T*)P.in[3], P.s[F_K2][0], P.s[F_K2][1], P.s[F_K2][2]};
  const TRef<const T> vh = half_of(TRef<const T>{(const T*)P.in[4], P.s[F_V][0], P.s[F_V][1], P.s[F_V][2]}, hh);
  const TRef<T> out{(T*)P.out, P.s[F_OUT][0], P.s[F_OUT][1], P.s[F_OUT][2]};
  const T* qr1 = qvalid ? q1.row(b, h, i) : nullptr;
  const T* qr2 = (BR == 2 && qvalid) ? q2.row(b, h, i) : nullptr;

  float rq1 = 1.f, rq2 = 1.f;
  const float* nk1 = nullptr;
  const float* nk2 = nullptr;
  if constexpr (NORM) {
    if (qvalid) {
      rq1 = P.norms[norm_base(P, N_Q1, bh) + i];
      if constexpr (BR == 2) rq2 = P.norms[norm_base(P, N_Q2, bh) + i];
    }
    nk1 = P.norms + norm_base(P, N_K1, bh);
    if constexpr (BR == 2) nk2 = P.norms + norm_base(P, N_K2, bh);
  }
  const float pw = P.p;
  const float tau = (*P.beta) * tau_coeff(pq, P.inv_d);
  float lam = 0.f;
  if constexpr (BR == 2) lam = clamp01(*P.lam);

  __shared__ __attribute__((aligned(16))) bf16 lds_all[(sizeof(T) == 2) ? 4 * TTileBF16<WH>::ELEMS : 8];
  TT vt;
  if constexpr (sizeof(T) == 2) vt.lds = lds_all + wv * TTileBF16<WH>::ELEMS;

  f32x16 O[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) O[c] = f32x16{};
  uint32_t* occrow = (P.occ && hh == 0) ? P.occ + ((int64_t)bh * P.nqt + qt) * P.occ_w : nullptr;
  const int64_t occ_br = (int64_t)BH * P.nqt * P.occ_w;
  uint32_t word = 0, word2 = 0;
  unsigned visited = 0, computed = 0;

  for (int kt = 0; kt <= ktl; ++kt) {
    const int k0 = kt * 32;
    const int j = k0 + n32;  // key row this lane supplies to the A operand
    const bool jv = j < Nk;
    f32x16 S1 = dot256<Pol>(jv ? k1.row(b, h, j) : nullptr, qr1, g, f32x16{});
    f32x16 S2 = f32x16{};
    if constexpr (BR == 2) S2 = dot256<Pol>(jv ? k2.row(b, h, j) : nullptr, qr2, g, f32x16{});
    float rk1 = 1.f, rk2 = 1.f;
    if constexpr (NORM) {
      rk1 = jv ? nk1[j] : 0.f;
      if constexpr (BR == 2) rk2 = jv ? nk2[j] : 0.f;
    }
    // x = fma(s rk_j, rq_i, -tau_i) is monotone in s rk_j: the tile max decides "any x > 0"
    float m1 = -INFINITY, m2 = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = k0 + crow(r, g);
      const bool valid = qvalid && key <= pq && key < Nk;
      if constexpr (NORM) S1[r] *= __shfl(rk1, crow(r, g));
      m1 = fmaxf(m1, valid ? S1[r] : -INFINITY);
      if constexpr (BR == 2) {
        if constexpr (NORM) S2[r] *= __shfl(rk2, crow(r, g));
        m2 = fmaxf(m2, valid ? S2[r] : -INFINITY);
      }
    }
    const bool any1 = wave_ballot(__builtin_fmaf(m1, rq1, -tau) > 0.f) != 0ull;
    bool any2 = false;
    if constexpr (BR == 2) any2 = wave_ballot(__builtin_fmaf(m2, rq2, -tau) > 0.f) != 0ull;
    visited += BR;
    computed += (any1 ? 1 : 0) + (any2 ? 1 : 0);
    if (any1) word |= 1u << (kt & 31);
    if (any2) word2 |= 1u << (kt & 31);
    if (any1 || any2) {
      f32x16 C;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + crow(r, g);
        const bool valid = qvalid && key <= pq && key < Nk;
        const float x1 = __builtin_fmaf(S1[r], rq1, -tau);
        float a = (valid && x1 > 0.f) ? pow_p<PK>(x1, pw) : 0.f;
        if constexpr (BR == 2) {
          const float x2 = __builtin_fmaf(S2[r], rq2, -tau);
          const float a2 = (valid && x2 > 0.f) ? pow_p<PK>(x2, pw) : 0.f;
          a = __builtin_fmaf(-lam, a2, a);
        }
        C[r] = a;
      }
      wide_stage<Pol>(vt, vh, b, h, k0, Nk);
      acc_tile<Pol>(O, vt, C);
      wide_release<Pol>(vt);
    }
    if (occrow && (((kt & 31) == 31) || kt == ktl)) {
      if (l == 0) {
        occrow[kt >> 5] = word;
        if constexpr (BR == 2) occrow[occ_br + (kt >> 5)] = word2;
      }
      word = word2 = 0;
    }
  }
  if (occrow && l == 0) {
    for (int w = (ktl >> 5) + 1; w < P.occ_w; ++w) {
      occrow[w] = 0u;
      if constexpr (BR == 2) occrow[occ_br + w] = 0u;
    }
  }
  if (qvalid) {
    T* orow = out.row(b, h, i) + WH * hh;
#pragma unroll
    for (int c = 0; c < ND; ++c)
#pragma unroll
      for (int u = 0; u < 4; ++u)
        store4(orow + 32 * c + 8 * u + 4 * g, O[c][4 * u], O[c][4 * u + 1], O[c][4 * u + 2], O[c][4 * u + 3]);
  }
  if (P.stats && l == 0 && hh == 0) {
    atomicAdd(P.stats + 0, (unsigned long long)visited);
    atomicAdd(P.stats + 1, (unsigned long long)computed);
  }
}

// ------------------------------------------------------------------ wide_bwd_dq
// One workgroup of two waves per (query tile, head), longest first; wave hh owns columns
// 128 hh .. 128 hh + 127 of dq1 (dq2).  With x_ij = s_ij rk_j rq_i - tau_i, G = d(ReLU(x)^p)/dx,
// Dp_ij = dO_i . v_j: dS1 = G1 Dp, dS2 = -lam G2 Dp, dq^_i = sum_j dS_ij rk_j k_j, and
// dq = (dq^ - q^ (q^ . dq^)) rq; dbeta = -sum_i c_i sum_j (dS1 + dS2), dlambda = -sum A2 Dp.
// Without the bitmask every causal tile is tested.
template <class Pol, int BR, int PK, bool NORM>
__global__ void __launch_bounds__(128) wide_bwd_dq(BwdParams P) {
  using T = typename Pol::T;
  using TT = typename WTile<Pol>::type;
  constexpr int ND = WH / 32;
  const int l = lane_id(), n32 = l & 31, g = l >> 5, hh = threadIdx.x >> 6;
  const int BH = P.B * P.H;
  const int64_t item = blockIdx.x;
  if (item >= (int64_t)BH * P.nqt) return;  // uniform over the workgroup
  const int qt = P.nqt - 1 - (int)(item / BH);
  const int ktl = kt_last(qt, P.qoff, P.nkt);
  const int bh = (int)(item % BH);
  const int b = bh / P.H, h = bh % P.H;
  const int Nq = P.Nq, Nk = P.Nk, qoff = P.qoff;
  const int i = qt * 32 + n32;
  const bool qvalid = i < Nq;
  const int pq = qoff + i;

  const TRef<const T> q1{(const T*)P.in[0], P.s[B_Q1][0], P.s[B_Q1][1], P.s[B_Q1][2]};
  const TRef<const T> k1{(const T*)P.in[1], P.s[B_K1][0], P.s[B_K1][1], P.s[B_K1][2]};
  const TRef<const T> q2{(const T*)P.in[2], P.s[B_Q2][0], P.s[B_Q2][1], P.s[B_Q2][2]};
  const TRef<const T> k2{(const T*)P.in[3], P.s[B_K2][0], P.s[B_K2][1], P.s[B_K2][2]};
  const TRef<const T> vv{(const T*)P.in[4], P.s[B_V][0], P.s[B_V][1], P.s[B_V][2]};
  const TRef<const T> dO{(const T*)P.in[5], P.s[B_DO][0], P.s[B_DO][1], P.s[B_DO][2]};
  const TRef<T> dq1{(T*)P.grad[0], P.s[B_DQ1][0], P.s[B_DQ1][1], P.s[B_DQ1][2]};
  const TRef<T> dq2{(T*)P.grad[2], P.s[B_DQ2][0], P.s[B_DQ2][1], P.s[B_DQ2][2]};
  const T* qr1 = qvalid ? q1.row(b, h, i) : nullptr;
  const T* qr2 = (BR == 2 && qvalid) ? q2.row(b, h, i) : nullptr;
  const T* dor = qvalid ? dO.row(b, h, i) : nullptr;

  float rq1 = 1.f, rq2 = 1.f;
  if constexpr (NORM) {
    if (qvalid) {
      rq1 = P.norms[norm_base(P, N_Q1, bh) + i];
      if constexpr (BR == 2) rq2 = P.norms[norm_base(P, N_Q2, bh) + i];
    }
  }
  const float pw = P.p;
  const float ci = tau_coeff(pq, P.inv_d);
  const float tau = (*P.beta) * ci;
  float lam = 0.f;
  if constexpr (BR == 2) lam = clamp01(*P.lam);
  const float* nk1 = NORM ? P.norms + norm_base(P, N_K1, bh) : nullptr;
  const float* nk2 = NORM ? P.norms + norm_base(P, N_K2, bh) : nullptr;

  __shared__ __attribute__((aligned(16))) bf16 lds_all[(sizeof(T) == 2) ? 2 * TTileBF16<WH>::ELEMS : 8];
  __shared__ float red[2][2][32];  // [branch][half][row]: the halves' partial row dots
  TT tile;
  if constexpr (sizeof(T) == 2) tile.lds = lds_all + hh * TTileBF16<WH>::ELEMS;
  const TRef<const T> k1h = half_of(k1, hh), k2h = half_of(k2, hh);

  f32x16 A1[ND], A2[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) A1[c] = A2[c] = f32x16{};
  float bsum = 0.f, lsum = 0.f;
  unsigned visited = 0, computed = 0;
  const uint32_t* occrow = P.occ ? P.occ + ((int64_t)bh * P.nqt + qt) * P.occ_w : nullptr;
  const int64_t occ_br = (int64_t)BH * P.nqt * P.occ_w;

  for (int kt = 0; kt <= ktl; ++kt) {
    bool use1 = true, use2 = BR == 2;
    if (occrow) {
      use1 = (__builtin_amdgcn_readfirstlane((int)occrow[kt >> 5]) >> (kt & 31)) & 1;
      if constexpr (BR == 2) use2 = (__builtin_amdgcn_readfirstlane((int)occrow[occ_br + (kt >> 5)]) >> (kt & 31)) & 1;
      if (!use1 && !use2) continue;
    }
    ++visited;
    const int k0 = kt * 32;
    const int j = k0 + n32;
    const bool jv = j < Nk;
    f32x16 S1 = f32x16{}, S2 = f32x16{};
    if (use1) S1 = dot256<Pol>(jv ? k1.row(b, h, j) : nullptr, qr1, g, S1);
    if (BR == 2 && use2) S2 = dot256<Pol>(jv ? k2.row(b, h, j) : nullptr, qr2, g, S2);
    const f32x16 Dp = dot256<Pol>(jv ? vv.row(b, h, j) : nullptr, dor, g, f32x16{});
    f32x16 E1, E2;
    bool any = false;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = k0 + crow(r, g);
      const bool valid = qvalid && key <= pq && key < Nk;
      float rk1 = 1.f, rk2 = 1.f;
      if constexpr (NORM) {
        rk1 = valid ? nk1[key] : 0.f;
        if constexpr (BR == 2) rk2 = valid ? nk2[key] : 0.f;
      }
      const float x1 = __builtin_fmaf(NORM ? S1[r] * rk1 : S1[r], rq1, -tau);
      const bool p1 = use1 && valid && x1 > 0.f;
      const float ds1 = p1 ? dpow_p<PK>(x1, pw) * Dp[r] : 0.f;
      float ds2 = 0.f;
      bool p2 = false;
      if constexpr (BR == 2) {
        const float x2 = __builtin_fmaf(NORM ? S2[r] * rk2 : S2[r], rq2, -tau);
        p2 = use2 && valid && x2 > 0.f;
        ds2 = p2 ? -lam * dpow_p<PK>(x2, pw) * Dp[r] : 0.f;
        lsum = __builtin_fmaf(p2 ? pow_p<PK>(x2, pw) : 0.f, Dp[r], lsum);
      }
      bsum += ds1 + ds2;
      any = any || p1 || p2;
      E1[r] = NORM ? ds1 * rk1 : ds1;
      E2[r] = NORM ? ds2 * rk2 : ds2;
    }
    if (!occrow && wave_ballot(any) == 0ull) continue;  // the same decision in both halves
    ++computed;
    if (use1) {
      wide_stage<Pol>(tile, k1h, b, h, k0, Nk);
      acc_tile<Pol>(A1, tile, E1);
      wide_release<Pol>(tile);
    }
    if (BR == 2 && use2) {
      wide_stage<Pol>(tile, k2h, b, h, k0, Nk);
      acc_tile<Pol>(A2, tile, E2);
      wide_release<Pol>(tile);
    }
  }

  const T* xr1 = qr1 ? qr1 + WH * hh : nullptr;
  const T* xr2 = qr2 ? qr2 + WH * hh : nullptr;
  float dot1 = 0.f, dot2 = 0.f;
  if constexpr (NORM) {
    // the row dots q^ . dq^ of the whole rows: each half's part, added in half order
    const float p1 = half_dot(A1, xr1, rq1);
    const float p2 = BR == 2 ? half_dot(A2, xr2, rq2) : 0.f;
    if (g == 0) {
      red[0][hh][n32] = p1;
      red[1][hh][n32] = p2;
    }
    __syncthreads();
    dot1 = red[0][0][n32] + red[0][1][n32];
    dot2 = red[1][0][n32] + red[1][1][n32];
  }
  half_store<NORM>(A1, xr1, qvalid ? dq1.row(b, h, i) + WH * hh : nullptr, rq1, dot1);
  if constexpr (BR == 2) half_store<NORM>(A2, xr2, qvalid ? dq2.row(b, h, i) + WH * hh : nullptr, rq2, dot2);

  if (hh == 0) {
    const float pb = wave_sum(-ci * bsum);
    const float pl = wave_sum(-lsum);
    if (l == 0) {
      P.ws[2 * item + 0] = pb;
      P.ws[2 * item + 1] = pl;
      if (P.stats) {
        atomicAdd(P.stats + 0, (unsigned long long)visited);
        atomicAdd(P.stats + 1, (unsigned long long)computed);
      }
    }
  }
}

// ------------------------------------------------------------------ wide_bwd_dkv
// One workgroup of two waves per (key tile, head), the key tiles with the most query tiles
// first; wave hh owns columns 128 hh .. of dk1, dk2 and dv.  Scores S = Q K^T (lane = key,
// values = 16 queries of the tile): dv_j += sum_i (A1 - lam A2)_ij dO_i, dk^_j += sum_i dS_ij
// rq_i q_i, then the normalize backward.
template <class Pol, int BR, int PK, bool NORM>
__global__ void __launch_bounds__(128) wide_bwd_dkv(BwdParams P) {
  using T = typename Pol::T;
  using TT = typename WTile<Pol>::type;
  constexpr int ND = WH / 32;
  const int l = lane_id(), n32 = l & 31, g = l >> 5, hh = threadIdx.x >> 6;
  const int BH = P.B * P.H;
  const int64_t item = blockIdx.x;
  if (item >= (int64_t)BH * P.nkt) return;  // uniform over the workgroup
  const int kt = (int)(item / BH);
  const int bh = (int)(item % BH);
  const int b = bh / P.H, h = bh % P.H;
  const int Nq = P.Nq, Nk = P.Nk, qoff = P.qoff;
  const int j = kt * 32 + n32;
  const bool kvalid = j < Nk;

  const TRef<const T> q1{(const T*)P.in[0], P.s[B_Q1][0], P.s[B_Q1][1], P.s[B_Q1][2]};
  const TRef<const T> k1{(const T*)P.in[1], P.s[B_K1][0], P.s[B_K1][1], P.s[B_K1][2]};
  const TRef<const T> q2{(const T*)P.in[2], P.s[B_Q2][0], P.s[B_Q2][1], P.s[B_Q2][2]};
  const TRef<const T> k2{(const T*)P.in[3], P.s[B_K2][0], P.s[B_K2][1], P.s[B_K2][2]};
  const TRef<const T> vv{(const T*)P.in[4], P.s[B_V][0], P.s[B_V][1], P.s[B_V][2]};
  const TRef<const T> dO{(const T*)P.in[5], P.s[B_DO][0], P.s[B_DO][1], P.s[B_DO][2]};
  const TRef<T> dk1{(T*)P.grad[1], P.s[B_DK1][0], P.s[B_DK1][1], P.s[B_DK1][2]};
  const TRef<T> dk2{(T*)P.grad[3], P.s[B_DK2][0], P.s[B_DK2][1], P.s[B_DK2][2]};
  const TRef<T> dvv{(T*)P.grad[4], P.s[B_DV][0], P.s[B_DV][1], P.s[B_DV][2]};
  const T* kr1 = kvalid ? k1.row(b, h, j) : nullptr;
  const T* kr2 = (BR == 2 && kvalid) ? k2.row(b, h, j) : nullptr;
  const T* vr = kvalid ? vv.row(b, h, j) : nullptr;

  float rk1 = 1.f, rk2 = 1.f;
  if constexpr (NORM) {
    if (kvalid) {
      rk1 = P.norms[norm_base(P, N_K1, bh) + j];
      if constexpr (BR == 2) rk2 = P.norms[norm_base(P, N_K2, bh) + j];
    }
  }
  const float pw = P.p;
  const float beta = *P.beta;
  float lam = 0.f;
  if constexpr (BR == 2) lam = clamp01(*P.lam);
  const float* nq1 = NORM ? P.norms + norm_base(P, N_Q1, bh) : nullptr;
  const float* nq2 = NORM ? P.norms + norm_base(P, N_Q2, bh) : nullptr;

  __shared__ __attribute__((aligned(16))) bf16 lds_all[(sizeof(T) == 2) ? 2 * TTileBF16<WH>::ELEMS : 8];
  __shared__ float red[2][2][32];  // [branch][half][row]
  TT tile;
  if constexpr (sizeof(T) == 2) tile.lds = lds_all + hh * TTileBF16<WH>::ELEMS;
  const TRef<const T> q1h = half_of(q1, hh), q2h = half_of(q2, hh), doh = half_of(dO, hh);

  f32x16 AV[ND], AK1[ND], AK2[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) AV[c] = AK1[c] = AK2[c] = f32x16{};
  unsigned visited = 0, computed = 0;
  const uint32_t* occcol = P.occ ? P.occ + (int64_t)bh * P.nqt * P.occ_w + (kt >> 5) : nullptr;
  const int64_t occ_br = (int64_t)BH * P.nqt * P.occ_w;

  for (int qt = qt_first(kt, qoff); qt < P.nqt; ++qt) {
    bool use1 = true, use2 = BR == 2;
    if (occcol) {
      use1 = (__builtin_amdgcn_readfirstlane((int)occcol[(int64_t)qt * P.occ_w]) >> (kt & 31)) & 1;
      if constexpr (BR == 2)
        use2 = (__builtin_amdgcn_readfirstlane((int)occcol[occ_br + (int64_t)qt * P.occ_w]) >> (kt & 31)) & 1;
      if (!use1 && !use2) continue;
    }
    ++visited;
    const int q0 = qt * 32;
    const int ia = q0 + n32;  // query row this lane supplies to the A operand
    const bool iv = ia < Nq;
    f32x16 S1 = f32x16{}, S2 = f32x16{};
    if (use1) S1 = dot256<Pol>(iv ? q1.row(b, h, ia) : nullptr, kr1, g, S1);
    if (BR == 2 && use2) S2 = dot256<Pol>(iv ? q2.row(b, h, ia) : nullptr, kr2, g, S2);
    const f32x16 Dp = dot256<Pol>(iv ? dO.row(b, h, ia) : nullptr, vr, g, f32x16{});
    f32x16 EV, E1, E2;
    bool any = false;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int qi = q0 + crow(r, g);
      const bool valid = kvalid && qi < Nq && j <= qoff + qi;
      float rq1 = 1.f, rq2 = 1.f;
      if constexpr (NORM) {
        rq1 = valid ? nq1[qi] : 0.f;
        if constexpr (BR == 2) rq2 = valid ? nq2[qi] : 0.f;
      }
      const float tau = beta * tau_coeff(qoff + qi, P.inv_d);
      const float x1 = __builtin_fmaf(NORM ? S1[r] * rk1 : S1[r], rq1, -tau);
      const bool p1 = use1 && valid && x1 > 0.f;
      float a = p1 ? pow_p<PK>(x1, pw) : 0.f;
      const float ds1 = p1 ? dpow_p<PK>(x1, pw) * Dp[r] : 0.f;
      float ds2 = 0.f;
      bool p2 = false;
      if constexpr (BR == 2) {
        const float x2 = __builtin_fmaf(NORM ? S2[r] * rk2 : S2[r], rq2, -tau);
        p2 = use2 && valid && x2 > 0.f;
        a = __builtin_fmaf(-lam, p2 ? pow_p<PK>(x2, pw) : 0.f, a);
        ds2 = p2 ? -lam * dpow_p<PK>(x2, pw) * Dp[r] : 0.f;
      }
      any = any || p1 || p2;
      EV[r] = a;
      E1[r] = NORM ? ds1 * rq1 : ds1;
      E2[r] = NORM ? ds2 * rq2 : ds2;
    }
    if (!occcol && wave_ballot(any) == 0ull) continue;  // the same decision in both halves
    ++computed;
    wide_stage<Pol>(tile, doh, b, h, q0, Nq);
    acc_tile<Pol>(AV, tile, EV);
    wide_release<Pol>(tile);
    if (use1) {
      wide_stage<Pol>(tile, q1h, b, h, q0, Nq);
      acc_tile<Pol>(AK1, tile, E1);
      wide_release<Pol>(tile);
    }
    if (BR == 2 && use2) {
      wide_stage<Pol>(tile, q2h, b, h, q0, Nq);
      acc_tile<Pol>(AK2, tile, E2);
      wide_release<Pol>(tile);
    }
  }

  const T* xr1 = kr1 ? kr1 + WH * hh : nullptr;
  const T* xr2 = kr2 ? kr2 + WH * hh : nullptr;
  float dot1 = 0.f, dot2 = 0.f;
  if constexpr (NORM) {
    const float p1 = half_dot(AK1, xr1, rk1);
    const float p2 = BR == 2 ? half_dot(AK2, xr2, rk2) : 0.f;
    if (g == 0) {
      red[0][hh][n32] = p1;
      red[1][hh][n32] = p2;
    }
    __syncthreads();
    dot1 = red[0][0][n32] + red[0][1][n32];
    dot2 = red[1][0][n32] + red[1][1][n32];
  }
  half_store<false>(AV, (const T*)nullptr, kvalid ? dvv.row(b, h, j) + WH * hh : nullptr, 1.f, 0.f);
  half_store<NORM>(AK1, xr1, kvalid ? dk1.row(b, h, j) + WH * hh : nullptr, rk1, dot1);
  if constexpr (BR == 2) half_store<NORM>(AK2, xr2, kvalid ? dk2.row(b, h, j) + WH * hh : nullptr, rk2, dot2);
  if (P.stats && l == 0 && hh == 0) {
    atomicAdd(P.stats + 0, (unsigned long long)visited);
    atomicAdd(P.stats + 1, (unsigned long long)computed);
  }
}

// ------------------------------------------------------------------ dispatch
template <class Pol, int BR, int PK, bool NORM>
int wide_fwd_t(const FwdParams& p, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  if (NORM) {
    const int64_t rows = (int64_t)BR * p.B * p.H * ((int64_t)p.Nq + p.Nk);
    hipLaunchKernelGGL((wide_norms<typename Pol::T, BR>), dim3((unsigned)((rows + 15) / 16)), dim3(256), 0, s, p);
    launched(s, "wide_norms");
  }
  const int64_t items = (int64_t)p.B * p.H * p.nqt * 2;
  hipLaunchKernelGGL((wide_fwd<Pol, BR, PK, NORM>), dim3((unsigned)((items + 3) / 4)), dim3(256), 0, s, p);
  launched(s, "wide_fwd");
  return (int)hipGetLastError();
}

template <class Pol, int BR, int PK, bool NORM>
int wide_bwd_t(const BwdParams& p, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  const int64_t qitems = (int64_t)p.B * p.H * p.nqt, kitems = (int64_t)p.B * p.H * p.nkt;
  hipLaunchKernelGGL((wide_bwd_dq<Pol, BR, PK, NORM>), dim3((unsigned)qitems), dim3(128), 0, s, p);
  launched(s, "wide_bwd_dq");
  hipLaunchKernelGGL((wide_bwd_dkv<Pol, BR, PK, NORM>), dim3((unsigned)kitems), dim3(128), 0, s, p);
  launched(s, "wide_bwd_dkv");
  const int e = (int)hipGetLastError();
  return e ? e : launch_bwd_finish(p, BR, qitems, stream);
}

template <class Pol, int BR, int PK>
int wfsel_norm(const FwdParams& p, const KernelKey& k, void* s) {
  return k.normalize ? wide_fwd_t<Pol, BR, PK, true>(p, s) : wide_fwd_t<Pol, BR, PK, false>(p, s);
}
template <class Pol, int BR>
int wfsel_pk(const FwdParams& p, const KernelKey& k, void* s) {
  switch (k.pkind) {
    case 2: return wfsel_norm<Pol, BR, 2>(p, k, s);
    case 1: return wfsel_norm<Pol, BR, 1>(p, k, s);
    default: return wfsel_norm<Pol, BR, 0>(p, k, s);
  }
}
template <class Pol>
int wfsel_br(const FwdParams& p, const KernelKey& k, void* s) {
  return k.branches == 2 ? wfsel_pk<Pol, 2>(p, k, s) : wfsel_pk<Pol, 1>(p, k, s);
}

template <class Pol, int BR, int PK>
int wbsel_norm(const BwdParams& p, const KernelKey& k, void* s) {
  return k.normalize ? wide_bwd_t<Pol, BR, PK, true>(p, s) : wide_bwd_t<Pol, BR, PK, false>(p, s);
}
template <class Pol, int BR>
int wbsel_pk(const BwdParams& p, const KernelKey& k, void* s) {
  switch (k.pkind) {
    case 2: return wbsel_norm<Pol, BR, 2>(p, k, s);
    case 1: return wbsel_norm<Pol, BR, 1>(p, k, s);
    default: return wbsel_norm<Pol, BR, 0>(p, k, s);
  }
}
template <class Pol>
int wbsel_br(const BwdParams& p, const KernelKey& k, void* s) {
  return k.branches == 2 ? wbsel_pk<Pol, 2>(p, k, s) : wbsel_pk<Pol, 1>(p, k, s);
}

}  // namespace

int launch_fwd_wide(const FwdParams& p, const KernelKey& k, void* stream) {
  return k.dtype == 1 ? wfsel_br<PolBF16>(p, k, stream) : wfsel_br<PolF32>(p, k, stream);
}

int launch_bwd_wide(const BwdParams& p, const KernelKey& k, void* stream) {
  return k.dtype == 1 ? wbsel_br<PolBF16>(p, k, stream) : wbsel_br<PolF32>(p, k, stream);
}

}  // namespace tda
