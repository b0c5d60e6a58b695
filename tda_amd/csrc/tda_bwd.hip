// tda_bwd.hip -- backward pass of threshold attention (TRA / differential TDA) for gfx950.
//
// Reference semantics (snap-research/TDA triton_threshold_attention.py, "TTA"):
//   dQ kernel TTA:118-223, dK/dV kernel TTA:226-324, host backward TTA:406-469; the
//   normalize / clamp / combine gradients come from torch autograd of TTA:505-517; dbeta is
//   new (the reference returns None for beta, TTA:469).
//
// With x_ij = s_ij * rk_j * rq_i - tau_i (s = raw dot product, rq/rk = inverse row norms or 1),
// G = d(ReLU(x)^p)/dx, Dp_ij = dO_i . v_j:
//   dS1 = G1 * Dp,  dS2 = -lam * G2 * Dp               (lam = clamp(lambda, 0, 1))
//   dq^_i = sum_j dS_ij rk_j k_j,   dk^_j = sum_i dS_ij rq_i q_i
//   dv_j  = sum_i (A1_ij - lam A2_ij) dO_i
//   dq    = (dq^ - q^ (q^ . dq^)) rq          (F.normalize backward; dq = dq^ when not normalized)
//   dbeta = -sum_i c_i sum_j (dS1_ij + dS2_ij),  tau_i = beta c_i
//   dlam  = -[0 <= lambda <= 1] sum_ij A2_ij Dp_ij
// Two passes keep every output single-writer (no atomics, bitwise reproducible): a query-major
// pass (dq1, dq2 and the dbeta/dlambda partials) and a key-major pass (dk1, dk2, dv).  When the
// forward's tile-occupancy bitmask is given, both passes visit only tiles with a non-zero
// score: A = 0 on a tile implies G = 0 there, so nothing else contributes.
#include "tda_common.hpp"
#include "tda_fin.hpp"
#include "tda_params.hpp"
#include "tda_pos.hpp"

namespace tda {

template <class Pol, int D> struct TTileSelB;
template <int D> struct TTileSelB<PolBF16, D> { using type = TTileBF16<D>; };
template <int D> struct TTileSelB<PolF32, D> { using type = TTileF32<D>; };

template <class Pol, int D, class TT>
__device__ __forceinline__ void prepare_tile(TT& tt, const TRef<const typename Pol::T>& x, int b, int h,
                                             int r0, int n) {
  if constexpr (sizeof(typename Pol::T) == 2) {
    tt.stage(x, b, h, r0, n);
    wave_lds_sync();
  } else {
    tt.set(x, b, h, r0, n);
  }
}
template <class Pol, class TT>
__device__ __forceinline__ void release_tile(TT&) {
  if constexpr (sizeof(typename Pol::T) == 2) wave_lds_sync();
}

// acc += A B^T over d with both operands' row fragments streamed from memory (A: lane (m, g)
// supplies row ra of tile row m; B: lane (n, g) supplies row rb): the element order of
// load_rows / mma_row, so the sums are bitwise those of a resident operand.  A null row reads
// as zeros.  The fp32 passes keep no operand resident: three resident fragment sets of a 32-row
// tile (192 VGPRs at d = 128) next to the accumulators spilled to scratch.
template <class Pol, int NT>
__device__ __forceinline__ f32x16 mma_rows2(const typename Pol::T* ra, const typename Pol::T* rb, int g, f32x16 acc) {
  if constexpr (sizeof(typename Pol::T) == 4) {
    const f32x4* pa = reinterpret_cast<const f32x4*>(ra ? ra + g * NT : ra);
    const f32x4* pb = reinterpret_cast<const f32x4*>(rb ? rb + g * NT : rb);
#pragma unroll
    for (int m = 0; m < NT / 4; ++m) {
      const f32x4 a = ra ? pa[m] : f32x4{0.f, 0.f, 0.f, 0.f};
      const f32x4 b = rb ? pb[m] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = Pol::mma(a[e], b[e], acc);
    }
  } else {
#pragma unroll
    for (int t = 0; t < NT; ++t) acc = Pol::mma(Pol::load_row(ra, t, g), Pol::load_row(rb, t, g), acc);
  }
  return acc;
}

// Apply the F.normalize backward to a gradient tile held in the transposed C layout
// (lane = one row, value r of column block c = element 32c + crow(r, g)) and store it.
template <class Pol, int D, bool NORM>
__device__ __forceinline__ void finish_rows(const f32x16 (&acc)[D / 32], const typename Pol::T* xrow,
                                            typename Pol::T* grow, float rinv) {
  constexpr int ND = D / 32;
  const int g = lane_id() >> 5;
  if constexpr (NORM) {
    f32x4 xh[ND][4];
    float dot = 0.f;
#pragma unroll
    for (int c = 0; c < ND; ++c)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        f32x4 x = xrow ? load4(xrow + 32 * c + 8 * u + 4 * g) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xh[c][u][e] = x[e] * rinv;
          dot = __builtin_fmaf(xh[c][u][e], acc[c][4 * u + e], dot);
        }
      }
    dot += __shfl_xor(dot, 32);
    const bool clamped = rinv >= 1.0f / kNormEps;  // |x| <= eps: x^ = x / eps is linear in x
    if (grow) {
#pragma unroll
      for (int c = 0; c < ND; ++c)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          float o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float a = acc[c][4 * u + e];
            o[e] = clamped ? a * rinv : (a - xh[c][u][e] * dot) * rinv;
          }
          store4(grow + 32 * c + 8 * u + 4 * g, o[0], o[1], o[2], o[3]);
        }
    }
  } else {
    if (grow) {
#pragma unroll
      for (int c = 0; c < ND; ++c)
#pragma unroll
        for (int u = 0; u < 4; ++u)
          store4(grow + 32 * c + 8 * u + 4 * g, acc[c][4 * u], acc[c][4 * u + 1], acc[c][4 * u + 2],
                 acc[c][4 * u + 3]);
    }
  }
}

// ------------------------------------------------------------------ query-major pass
// One wave per 32-row query tile (rows i = 32 qt + lane%32), longest-first.  Score tiles are
// formed as in the forward (S^T = K Q^T: lane = query, values = keys); the gradient tile
// dS * rk packs into the B operand of dq^T += K^T (dS rk)^T, with K^T staged as a
// transposed tile.
//
// LISTS (fp32 with the forward's pair lists): one wave per (branch, query tile) list that did
// not fit (the pair pass bwd_dq_pairs took the others): only that branch's scores, dq rows and
// dbeta / dlambda partials (the list's workspace slot, as the pair pass's).
template <class Pol, int D, int BR, int PK, bool NORM, bool LISTS>
__device__ __forceinline__ void bwd_dq_item(const BwdParams& P, int qt, int bh, int lbr, int64_t slot, int wv);

template <class Pol, int D, int BR, int PK, bool NORM, bool LISTS = false>
__global__ void __launch_bounds__(256) bwd_dq(BwdParams P) {
  const int wv = threadIdx.x >> 6;
  const int BH = P.B * P.H;
  const int64_t item = (int64_t)blockIdx.x * 4 + wv;
  if constexpr (LISTS) {
    if (item >= (int64_t)BR * BH * P.nqt) return;
    const int br = BR == 2 ? (int)(item & 1) : 0;  // the item order of bwd_dq_pairs
    const int64_t rest = BR == 2 ? item >> 1 : item;
    const int qt = (int)(rest / BH), bh = (int)(rest % BH);
    const int64_t lidx = ((int64_t)br * BH + bh) * P.nqt + qt;
    if (P.pairs[pair_lists(BR, BH, P.nqt) * 4 * kPairCap + lidx] <= (uint32_t)kPairCap) return;
    bwd_dq_item<Pol, D, BR, PK, NORM, true>(P, qt, bh, br, lidx, wv);
  } else {
    if (item >= (int64_t)BH * P.nqt) return;
    bwd_dq_item<Pol, D, BR, PK, NORM, false>(P, P.nqt - 1 - (int)(item / BH), (int)(item % BH), 0, item, wv);
  }
}

template <class Pol, int D, int BR, int PK, bool NORM, bool LISTS>
__device__ __forceinline__ void bwd_dq_item(const BwdParams& P, int qt, int bh, int lbr, int64_t slot, int wv) {
  using T = typename Pol::T;
  using frag = typename Pol::frag;
  constexpr int NT = D / Pol::KS, NS = 32 / Pol::KS, ND = D / 32;
  using TT = typename TTileSelB<Pol, D>::type;

  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int BH = P.B * P.H;
  const int ktl = kt_last(qt, P.qoff, P.nkt);  // last key tile the query tile sees
  const int b = bh / P.H, h = bh % P.H;
  const int Nq = P.Nq, Nk = P.Nk, qoff = P.qoff;
  const int i = qt * 32 + n32;
  const bool qvalid = i < Nq;
  const int pq = qoff + i;  // the lane's query position

  const TRef<const T> q1{(const T*)P.in[0], P.s[B_Q1][0], P.s[B_Q1][1], P.s[B_Q1][2]};
  const TRef<const T> k1{(const T*)P.in[1], P.s[B_K1][0], P.s[B_K1][1], P.s[B_K1][2]};
  const TRef<const T> q2{(const T*)P.in[2], P.s[B_Q2][0], P.s[B_Q2][1], P.s[B_Q2][2]};
  const TRef<const T> k2{(const T*)P.in[3], P.s[B_K2][0], P.s[B_K2][1], P.s[B_K2][2]};
  const TRef<const T> vv{(const T*)P.in[4], P.s[B_V][0], P.s[B_V][1], P.s[B_V][2]};
  const TRef<const T> dO{(const T*)P.in[5], P.s[B_DO][0], P.s[B_DO][1], P.s[B_DO][2]};
  const TRef<T> dq1{(T*)P.grad[0], P.s[B_DQ1][0], P.s[B_DQ1][1], P.s[B_DQ1][2]};
  const TRef<T> dq2{(T*)P.grad[2], P.s[B_DQ2][0], P.s[B_DQ2][1], P.s[B_DQ2][2]};

  const T* qr1 = qvalid ? q1.row(b, h, i) : nullptr;  // this lane's rows (B operands, streamed)
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

  __shared__ __attribute__((aligned(16))) bf16 lds_all[(sizeof(T) == 2) ? 4 * TTileBF16<D>::ELEMS : 8];
  TT kt_tile;
  if constexpr (sizeof(T) == 2) kt_tile.lds = lds_all + wv * TTileBF16<D>::ELEMS;

  f32x16 A1[ND], A2[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) { A1[c] = f32x16{}; A2[c] = f32x16{}; }
  float bsum = 0.f, lsum = 0.f;
  unsigned visited = 0, computed = 0;
  const uint32_t* occrow = P.occ ? P.occ + ((int64_t)bh * P.nqt + qt) * P.occ_w : nullptr;
  const int64_t occ_br = (int64_t)BH * P.nqt * P.occ_w;  // branch-plane distance of the bitmask
  const float* nk1 = NORM ? P.norms + norm_base(P, N_K1, bh) : nullptr;
  const float* nk2 = NORM ? P.norms + norm_base(P, N_K2, bh) : nullptr;

  // With the bitmask the wave visits only the tiles with a bit set in either branch, one load
  // per bitmask word (not per key tile): the set bits of the current word, then the next word.
  int cw = -1;
  uint32_t w1 = 0u, w2 = 0u;  // the branches' bits of word cw
  auto next_kt = [&](int kt) {
    if (!occrow) return kt;
    while (kt <= ktl) {
      if ((kt >> 5) != cw) {
        cw = kt >> 5;
        w1 = (!LISTS || lbr == 0) ? (uint32_t)__builtin_amdgcn_readfirstlane((int)occrow[cw]) : 0u;
        if constexpr (BR == 2)
          w2 = (!LISTS || lbr == 1) ? (uint32_t)__builtin_amdgcn_readfirstlane((int)occrow[occ_br + cw]) : 0u;
      }
      const uint32_t m = (w1 | w2) >> (kt & 31);
      if (m) return kt + __builtin_ctz(m);
      kt = (kt | 31) + 1;
    }
    return kt;
  };
  for (int kt = next_kt(0); kt <= ktl; kt = next_kt(kt + 1)) {
    // with the bitmask: the branches holding a non-zero weight in the tile (a branch without
    // one adds nothing to any sum below, so its scores and products are skipped)
    bool use1 = true, use2 = BR == 2;
    if (occrow) {
      use1 = (w1 >> (kt & 31)) & 1u;
      if constexpr (BR == 2) use2 = (w2 >> (kt & 31)) & 1u;
    }
    ++visited;
    const int k0 = kt * 32;
    const int j = k0 + n32;
    f32x16 S1 = f32x16{}, S2 = f32x16{}, Dp = f32x16{};
    if (use1) {
      const T* r = (j < Nk) ? k1.row(b, h, j) : nullptr;
      S1 = mma_rows2<Pol, NT>(r, qr1, g, S1);
    }
    if (BR == 2 && use2) {
      const T* r = (j < Nk) ? k2.row(b, h, j) : nullptr;
      S2 = mma_rows2<Pol, NT>(r, qr2, g, S2);
    }
    {
      const T* r = (j < Nk) ? vv.row(b, h, j) : nullptr;
      Dp = mma_rows2<Pol, NT>(r, dor, g, Dp);
    }
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
    if (!occrow && wave_ballot(any) == 0ull) continue;
    ++computed;
    if (use1) {
      prepare_tile<Pol, D>(kt_tile, k1, b, h, k0, Nk);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const frag bp = Pol::pack_c(E1, s);
#pragma unroll
        for (int c = 0; c < ND; ++c) A1[c] = Pol::mma(kt_tile.frag(s, c), bp, A1[c]);
      }
      release_tile<Pol>(kt_tile);
    }
    if (BR == 2 && use2) {
      prepare_tile<Pol, D>(kt_tile, k2, b, h, k0, Nk);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const frag bp = Pol::pack_c(E2, s);
#pragma unroll
        for (int c = 0; c < ND; ++c) A2[c] = Pol::mma(kt_tile.frag(s, c), bp, A2[c]);
      }
      release_tile<Pol>(kt_tile);
    }
  }

  if (!LISTS || lbr == 0)
    finish_rows<Pol, D, NORM>(A1, qvalid ? q1.row(b, h, i) : nullptr, qvalid ? dq1.row(b, h, i) : nullptr, rq1);
  if (BR == 2 && (!LISTS || lbr == 1))
    finish_rows<Pol, D, NORM>(A2, qvalid ? q2.row(b, h, i) : nullptr, qvalid ? dq2.row(b, h, i) : nullptr, rq2);

  // per-wave dbeta / dlambda partials (lanes with g == 1 hold the same query as g == 0 but
  // other keys, so every lane contributes)
  const float pb = wave_sum(-ci * bsum);
  const float pl = wave_sum(-lsum);
  if (l == 0) {
    P.ws[2 * slot + 0] = pb;
    P.ws[2 * slot + 1] = pl;
    if (P.stats) {
      atomicAdd(P.stats + 0, (unsigned long long)visited);
      atomicAdd(P.stats + 1, (unsigned long long)computed);
    }
  }
}

// ------------------------------------------------------------------ key-major pass
// One wave per 32-row key tile (rows j = 32 kt + lane%32), longest-first (small kt has the
// most query tiles).  Scores are formed as S = Q K^T (lane = key, values = queries) so that the
// probability and gradient tiles pack into the B operand of dv^T += dO^T A and
// dk^T += Q^T (dS rq), with dO^T and Q^T staged as transposed tiles.
//
// QUEUE (fp32 with the forward's pair lists): only the key tiles the key-major pair pass
// (bwd_dkv_pairs) queued, whose columns hold a list that did not fit; the waves take them in turn.
template <class Pol, int D, int BR, int PK, bool NORM>
__device__ __forceinline__ void bwd_dkv_item(const BwdParams& P, int64_t item, int wv);

template <class Pol, int D, int BR, int PK, bool NORM, bool QUEUE = false>
__global__ void __launch_bounds__(256) bwd_dkv(BwdParams P) {
  const int wv = threadIdx.x >> 6;
  const int BH = P.B * P.H;
  if constexpr (QUEUE) {
    const uint32_t queued = P.dkvq[0];
    for (uint32_t k = blockIdx.x * 4u + (uint32_t)wv; k < queued; k += gridDim.x * 4u)
      bwd_dkv_item<Pol, D, BR, PK, NORM>(P, (int64_t)P.dkvq[1 + k], wv);
    return;
  }
  const int64_t item = (int64_t)blockIdx.x * 4 + wv;
  if (item >= (int64_t)BH * P.nkt) return;
  bwd_dkv_item<Pol, D, BR, PK, NORM>(P, item, wv);
}

template <class Pol, int D, int BR, int PK, bool NORM>
__device__ __forceinline__ void bwd_dkv_item(const BwdParams& P, int64_t item, int wv) {
  using T = typename Pol::T;
  using frag = typename Pol::frag;
  constexpr int NT = D / Pol::KS, NS = 32 / Pol::KS, ND = D / 32;
  using TT = typename TTileSelB<Pol, D>::type;

  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int BH = P.B * P.H;
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

  const T* kr1 = kvalid ? k1.row(b, h, j) : nullptr;  // this lane's rows (B operands, streamed)
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

  __shared__ __attribute__((aligned(16))) bf16 lds_all[(sizeof(T) == 2) ? 4 * TTileBF16<D>::ELEMS : 8];
  TT tile;
  if constexpr (sizeof(T) == 2) tile.lds = lds_all + wv * TTileBF16<D>::ELEMS;

  f32x16 AV[ND], AK1[ND], AK2[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) { AV[c] = f32x16{}; AK1[c] = f32x16{}; AK2[c] = f32x16{}; }
  unsigned visited = 0, computed = 0;
  const uint32_t* occcol = P.occ ? P.occ + (int64_t)bh * P.nqt * P.occ_w + (kt >> 5) : nullptr;
  const int64_t occ_br = (int64_t)BH * P.nqt * P.occ_w;  // branch-plane distance of the bitmask

  // With the bitmask the wave visits only the query tiles with the key tile's bit set in either
  // branch: the bits of 64 query tiles come in one lane-parallel load round and two ballots.
  int cb = -1;
  uint64_t m1 = 0ull, m2 = 0ull;  // the branches' bits of query tiles cb .. cb + 63
  auto next_qt = [&](int qt) {
    if (!occcol) return qt;
    while (qt < P.nqt) {
      if ((qt & ~63) != cb) {
        cb = qt & ~63;
        const int qq = cb + l;
        uint32_t a = 0u, c = 0u;
        if (qq < P.nqt) {
          a = occcol[(int64_t)qq * P.occ_w];
          if constexpr (BR == 2) c = occcol[occ_br + (int64_t)qq * P.occ_w];
        }
        m1 = wave_ballot((a >> (kt & 31)) & 1u);
        m2 = BR == 2 ? wave_ballot((c >> (kt & 31)) & 1u) : 0ull;
      }
      const uint64_t m = (m1 | m2) >> (qt & 63);
      if (m) return qt + (int)__builtin_ctzll(m);
      qt = (qt | 63) + 1;
    }
    return qt;
  };
  for (int qt = next_qt(qt_first(kt, qoff)); qt < P.nqt; qt = next_qt(qt + 1)) {
    // with the bitmask: the branches holding a non-zero weight in the tile (see bwd_dq)
    bool use1 = true, use2 = BR == 2;
    if (occcol) {
      use1 = (m1 >> (qt & 63)) & 1ull;
      if constexpr (BR == 2) use2 = (m2 >> (qt & 63)) & 1ull;
    }
    ++visited;
    const int q0 = qt * 32;
    const int ia = q0 + n32;  // query row this lane loads for the A operand
    f32x16 S1 = f32x16{}, S2 = f32x16{}, Dp = f32x16{};
    if (use1) {
      const T* r = (ia < Nq) ? q1.row(b, h, ia) : nullptr;
      S1 = mma_rows2<Pol, NT>(r, kr1, g, S1);
    }
    if (BR == 2 && use2) {
      const T* r = (ia < Nq) ? q2.row(b, h, ia) : nullptr;
      S2 = mma_rows2<Pol, NT>(r, kr2, g, S2);
    }
    {
      const T* r = (ia < Nq) ? dO.row(b, h, ia) : nullptr;
      Dp = mma_rows2<Pol, NT>(r, vr, g, Dp);
    }
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
    if (!occcol && wave_ballot(any) == 0ull) continue;
    ++computed;
    prepare_tile<Pol, D>(tile, dO, b, h, q0, Nq);
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const frag bp = Pol::pack_c(EV, s);
#pragma unroll
      for (int c = 0; c < ND; ++c) AV[c] = Pol::mma(tile.frag(s, c), bp, AV[c]);
    }
    release_tile<Pol>(tile);
    if (use1) {
      prepare_tile<Pol, D>(tile, q1, b, h, q0, Nq);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const frag bp = Pol::pack_c(E1, s);
#pragma unroll
        for (int c = 0; c < ND; ++c) AK1[c] = Pol::mma(tile.frag(s, c), bp, AK1[c]);
      }
      release_tile<Pol>(tile);
    }
    if (BR == 2 && use2) {
      prepare_tile<Pol, D>(tile, q2, b, h, q0, Nq);
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const frag bp = Pol::pack_c(E2, s);
#pragma unroll
        for (int c = 0; c < ND; ++c) AK2[c] = Pol::mma(tile.frag(s, c), bp, AK2[c]);
      }
      release_tile<Pol>(tile);
    }
  }

  finish_rows<Pol, D, false>(AV, nullptr, kvalid ? dvv.row(b, h, j) : nullptr, 1.f);
  finish_rows<Pol, D, NORM>(AK1, kvalid ? k1.row(b, h, j) : nullptr, kvalid ? dk1.row(b, h, j) : nullptr, rk1);
  if constexpr (BR == 2)
    finish_rows<Pol, D, NORM>(AK2, kvalid ? k2.row(b, h, j) : nullptr, kvalid ? dk2.row(b, h, j) : nullptr, rk2);
  if (P.stats && l == 0) {
    atomicAdd(P.stats + 0, (unsigned long long)visited);
    atomicAdd(P.stats + 1, (unsigned long long)computed);
  }
}

// ------------------------------------------------------------------ block tile passes (fp32)
// The fp32 backward without normalisation (the forward ran fwd_wave_blk: every query tile, the
// bitmask rows exact, no pair lists): four consecutive tiles of one head per workgroup, one
// wave each, walking the union of their bitmask tiles in step, as the bf16 block passes do.
// Each streamed tile's rows are loaded once per workgroup (each wave a quarter of the rows, one
// tile ahead into registers) into LDS, two barriers per tile.  The score and dp products take
// both operands in the load_rows element order (lane half g: elements g D/2 .., step t), so
// every score is bitwise the forward's; the contractions over a tile's 32 rows read the rows
// as A^T fragments (row crow(st, g), one column per lane), as fwd_wave_blk's A.V does.
constexpr int kF32Blk = 4;

// This wave's share of a 32-row fp32 tile: rows RPI (LPW wv + u) + l / CPR, 16-byte chunk
// l % CPR; rows past n read row n - 1 (their products are masked).
template <int D>
struct F32Rows {
  static constexpr int CPR = D / 4, RPI = 64 / CPR, LPW = 32 / RPI / kF32Blk;
  static_assert(LPW >= 1 && LPW * RPI * kF32Blk == 32, "tile rows split evenly over the waves");
  f32x4 v[LPW];
  __device__ __forceinline__ void load(const TRef<const float>& x, int b, int h, int r0, int n, int wv) {
    const int l = lane_id();
#pragma unroll
    for (int u = 0; u < LPW; ++u) {
      const int r = min(r0 + RPI * (LPW * wv + u) + l / CPR, n - 1);
      v[u] = *reinterpret_cast<const f32x4*>(x.row(b, h, r) + 4 * (l % CPR));
    }
  }
  template <int KS>
  __device__ __forceinline__ void store(float* tile, int wv) const {
    const int l = lane_id();
#pragma unroll
    for (int u = 0; u < LPW; ++u)
      *reinterpret_cast<f32x4*>(tile + (RPI * (LPW * wv + u) + l / CPR) * KS + 4 * (l % CPR)) = v[u];
  }
};

// S^T-layout product of a 32-row LDS tile (A operand: lane (m, g) row m, elements g D/2 + t)
// with a lane's register fragments (B operand, load_rows order): lane n, value r = row crow(r, g).
template <int D, int KS>
__device__ __forceinline__ f32x16 lds_rows_mma(const float* tile, const float (&bf)[D / 2], f32x16 acc) {
  constexpr int NT = D / 2;
  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const float* p = tile + n32 * KS + g * NT;
#pragma unroll
  for (int m = 0; m < NT / 4; ++m) {
    const f32x4 v = *reinterpret_cast<const f32x4*>(p + 4 * m);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc = PolF32::mma(v[e], bf[4 * m + e], acc);
  }
  return acc;
}
// acc[c] += tile^T E over the tile's 32 rows (lane n, value r of block c = column 32 c + crow(r, g)):
// step st takes rows crow(st, 0) and crow(st, 1), E's values st of lane n.
template <int D, int KS>
__device__ __forceinline__ void lds_tr_mma(const float* tile, const f32x16& E, f32x16 (&acc)[D / 32]) {
  const int l = lane_id(), n32 = l & 31, g = l >> 5;
#pragma unroll
  for (int st = 0; st < 16; ++st) {
    const float* p = tile + crow(st, g) * KS + n32;
#pragma unroll
    for (int c = 0; c < D / 32; ++c) acc[c] = PolF32::mma(p[32 * c], E[st], acc[c]);
  }
}

// Query-major: four query tiles of one (branch, head), streaming K and V.  dq rows, the
// (branch, head, query tile) dbeta / dlambda partials and the counters.
template <int D, int BR, int PK>
__global__ void __launch_bounds__(64 * kF32Blk) __attribute__((amdgpu_waves_per_eu(D <= 64 ? 2 : 1)))
bwd_dq_blk_f32(BwdParams P) {
  constexpr int W = kF32Blk, NT = D / 2, ND = D / 32;
  constexpr int KS = D + 4;  // row stride: the row-fragment reads (lane n32 at row n32) spread over the banks
  __shared__ __attribute__((aligned(16))) float klds[32 * KS];
  __shared__ __attribute__((aligned(16))) float vlds[32 * KS];
  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int BH = P.B * P.H, nqt = P.nqt, Nq = P.Nq, Nk = P.Nk, qoff = P.qoff;
  const int nqb = (nqt + W - 1) / W;
  // longest blocks (last query tiles) of every (head, branch) first, the branches adjacent
  const int bid = blockIdx.x, jb = nqb - 1 - bid / (BR * BH), rem = bid % (BR * BH);
  const int br = BR == 2 ? rem & 1 : 0, bh = BR == 2 ? rem >> 1 : rem;
  const int b = bh / P.H, h = bh % P.H;
  const int qt = W * jb + wv;
  const bool act = qt < nqt;  // wave-uniform: waves past the last query tile only load
  const int i = 32 * qt + n32;
  const bool qvalid = act && i < Nq;
  const int pq = qoff + i;
  const bool edge_rows = !act || 32 * qt + 31 >= Nq;
  const int64_t lrow0 = ((int64_t)br * BH + bh) * nqt + W * jb;  // bitmask row of the block's first tile
  const int qslot = br == 0 ? B_Q1 : B_Q2, kslot = br == 0 ? B_K1 : B_K2;
  const TRef<const float> qx{(const float*)P.in[br == 0 ? 0 : 2], P.s[qslot][0], P.s[qslot][1], P.s[qslot][2]};
  const TRef<const float> kx{(const float*)P.in[br == 0 ? 1 : 3], P.s[kslot][0], P.s[kslot][1], P.s[kslot][2]};
  const TRef<const float> vx{(const float*)P.in[4], P.s[B_V][0], P.s[B_V][1], P.s[B_V][2]};
  const TRef<const float> dox{(const float*)P.in[5], P.s[B_DO][0], P.s[B_DO][1], P.s[B_DO][2]};

  float Q[NT], DO[NT];
  PolF32::load_rows<NT>(qvalid ? qx.row(b, h, i) : nullptr, g, Q);
  PolF32::load_rows<NT>(qvalid ? dox.row(b, h, i) : nullptr, g, DO);
  const float ci = tau_coeff(pq, P.inv_d);
  const float tau = (*P.beta) * ci;
  const float pw = P.p;
  float coef = 1.f;
  if constexpr (BR == 2) coef = br == 0 ? 1.f : -clamp01(*P.lam);
  const bool want_l = BR == 2 && br == 1;  // dlambda comes from branch 2 alone
  float bsum = 0.f, lsum = 0.f;
  unsigned visited = 0, computed = 0;
  f32x16 A[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) A[c] = f32x16{};

  // word w of the block's row r, masked to the key tiles the row sees (uniform); every causal
  // tile without a bitmask
  const int klast_b = kt_last(min(W * jb + W - 1, nqt - 1), qoff, P.nkt);
  auto row_word = [&](int r, int w) -> uint32_t {
    if (W * jb + r >= nqt) return 0u;
    const int kl = kt_last(W * jb + r, qoff, P.nkt);
    if (w > (kl >> 5)) return 0u;
    uint32_t x = P.occ ? (uint32_t)__builtin_amdgcn_readfirstlane((int)P.occ[(lrow0 + r) * P.occ_w + w]) : 0xffffffffu;
    if (w == (kl >> 5) && (kl & 31) != 31) x &= (2u << (kl & 31)) - 1u;
    return x;
  };
  int sw = -1;
  uint32_t ub = 0u, sown = 0u;
  auto next_tile = [&](uint32_t& own_out) -> int {
    while (ub == 0u) {
      if (++sw > (klast_b >> 5)) return -1;
      uint32_t u = 0u, o = 0u;
#pragma unroll
      for (int r = 0; r < W; ++r) {
        const uint32_t x = row_word(r, sw);
        u |= x;
        o = r == wv ? x : o;
      }
      ub = u;
      sown = o;
    }
    const int kt = 32 * sw + __builtin_ctz(ub);
    ub &= ub - 1u;
    own_out = sown;
    return kt;
  };
  F32Rows<D> kr, vr;
  auto issue = [&](int kt) {
    kr.load(kx, b, h, 32 * kt, Nk, wv);
    vr.load(vx, b, h, 32 * kt, Nk, wv);
  };
  uint32_t cown = 0u;
  int kt = next_tile(cown);
  if (kt >= 0) issue(kt);
  while (kt >= 0) {
    lds_barrier();  // every wave is done with the previous tile
    kr.template store<KS>(klds, wv);
    vr.template store<KS>(vlds, wv);
    uint32_t nown = 0u;
    const int kt2 = next_tile(nown);
    if (kt2 >= 0) issue(kt2);  // in flight during this tile's products
    lds_barrier();             // tile kt in LDS
    if ((cown >> (kt & 31)) & 1u) {
      ++visited;
      const int k0 = 32 * kt;
      f32x16 S = lds_rows_mma<D, KS>(klds, Q, f32x16{});
      const f32x16 Dp = lds_rows_mma<D, KS>(vlds, DO, f32x16{});
      // exact x (the forward's expression), branch-free; keys after the query's position,
      // padding keys and rows past Nq set to -1 (only on the tiles that have any)
      f32x16 X;
#pragma unroll
      for (int r = 0; r < 16; ++r) X[r] = __builtin_fmaf(S[r], 1.f, -tau);
      if (k0 + 31 > min(qoff + 32 * qt, Nk - 1) || edge_rows) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + crow(r, g);
          X[r] = qvalid && key <= pq && key < Nk ? X[r] : -1.f;
        }
      }
      f32x16 E;
      float xm = X[0];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const bool pos = X[r] > 0.f;
        const float ds = pos ? coef * dpow_p<PK>(X[r], pw) * Dp[r] : 0.f;
        bsum += ds;
        if (want_l) lsum = __builtin_fmaf(pos ? pow_p<PK>(X[r], pw) : 0.f, Dp[r], lsum);
        E[r] = ds;
        xm = fmaxf(xm, X[r]);
      }
      computed += (P.occ || wave_ballot(xm > 0.f) != 0ull) ? 1u : 0u;
      lds_tr_mma<D, KS>(klds, E, A);
    }
    cown = nown;  // the own row's word of the next tile
    kt = kt2;
  }
  if (!act) return;
  const int gslot = br == 0 ? B_DQ1 : B_DQ2;
  const TRef<float> dqx{(float*)P.grad[br == 0 ? 0 : 2], P.s[gslot][0], P.s[gslot][1], P.s[gslot][2]};
  finish_rows<PolF32, D, false>(A, nullptr, qvalid ? dqx.row(b, h, i) : nullptr, 1.f);
  const float pb = wave_sum(-ci * bsum);
  const float pl = wave_sum(-lsum);
  if (l == 0) {
    const int64_t lidx = lrow0 + wv;
    P.ws[2 * lidx + 0] = pb;  // slot of (branch, head, query tile)
    P.ws[2 * lidx + 1] = pl;
    if (P.stats) {
      atomicAdd(P.stats + 0, (unsigned long long)visited);
      atomicAdd(P.stats + 1, (unsigned long long)computed);
    }
  }
}

// Key-major: four consecutive key tiles of one head (aligned: one bitmask word holds their
// bits), streaming per branch the query tiles' Q and dO rows and tau values; K (per branch) and
// V rows of the wave's key tile in registers.  dk rows per branch, dv rows at the end.
template <int D, int BR, int PK>
__global__ void __launch_bounds__(64 * kF32Blk) __attribute__((amdgpu_waves_per_eu(D <= 64 ? 2 : 1)))
bwd_dkv_blk_f32(BwdParams P) {
  constexpr int W = kF32Blk, NT = D / 2, ND = D / 32;
  constexpr int KS = D + 4;
  __shared__ __attribute__((aligned(16))) float qlds[32 * KS];
  __shared__ __attribute__((aligned(16))) float dlds[32 * KS];
  __shared__ __attribute__((aligned(16))) float tlds[32];  // tau of the tile's query rows
  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int BH = P.B * P.H, nqt = P.nqt, nkt = P.nkt, Nq = P.Nq, Nk = P.Nk, qoff = P.qoff;
  // longest blocks (first key tiles) of every head first
  const int bid = blockIdx.x, jb = bid / BH, bh = bid % BH;
  const int b = bh / P.H, h = bh % P.H;
  const int kt0 = W * jb, kt = kt0 + wv;
  const bool act = kt < nkt;
  const int j = 32 * kt + n32;
  const bool kvalid = act && j < Nk;
  const int qtf_b = qt_first(kt0, qoff);  // first query tile of the block
  const TRef<const float> vx{(const float*)P.in[4], P.s[B_V][0], P.s[B_V][1], P.s[B_V][2]};
  const TRef<const float> dox{(const float*)P.in[5], P.s[B_DO][0], P.s[B_DO][1], P.s[B_DO][2]};
  float Vf[NT];
  PolF32::load_rows<NT>(kvalid ? vx.row(b, h, j) : nullptr, g, Vf);
  const float beta = *P.beta;
  const float pw = P.p;
  float lam = 0.f;
  if constexpr (BR == 2) lam = clamp01(*P.lam);
  const bool edge_keys = !act || 32 * kt + 31 >= Nk;
  // the block's active key tiles (bits r: key tile kt0 + r)
  const uint32_t actm = nkt - kt0 >= W ? (1u << W) - 1u : (1u << (nkt - kt0)) - 1u;
  f32x16 AV[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) AV[c] = f32x16{};
  unsigned visited = 0, computed = 0;

#pragma unroll
  for (int br = 0; br < BR; ++br) {
    const int qslot = br == 0 ? B_Q1 : B_Q2, kslot = br == 0 ? B_K1 : B_K2;
    const TRef<const float> qx{(const float*)P.in[br == 0 ? 0 : 2], P.s[qslot][0], P.s[qslot][1], P.s[qslot][2]};
    const TRef<const float> kx{(const float*)P.in[br == 0 ? 1 : 3], P.s[kslot][0], P.s[kslot][1], P.s[kslot][2]};
    float Kf[NT];
    PolF32::load_rows<NT>(kvalid ? kx.row(b, h, j) : nullptr, g, Kf);
    const float coef = br == 0 ? 1.f : -lam;
    f32x16 AK[ND];
#pragma unroll
    for (int c = 0; c < ND; ++c) AK[c] = f32x16{};
    const int64_t row0 = ((int64_t)br * BH + bh) * nqt;  // bitmask row of query tile 0

    // union walk over query tiles qtf_b .. nqt - 1, 64 per round: lane q tests query tile q0c + q
    int q0c = qtf_b - 64;
    uint64_t um = 0ull, om = 0ull;
    auto next_tile = [&](bool& own_out) -> int {
      while (um == 0ull) {
        q0c += 64;
        if (q0c >= nqt) return -1;
        const int qtl = q0c + l;
        const bool in = qtl < nqt;
        const uint32_t w = !in ? 0u : P.occ ? P.occ[(row0 + qtl) * P.occ_w + (kt0 >> 5)] : 0xffffffffu;
        uint32_t bits = (w >> (kt0 & 31)) & actm;
        // causal: key tile kt0 + r is seen from query tile qt_first(kt0 + r) on
#pragma unroll
        for (int r = 0; r < W; ++r)
          if (qtl < qt_first(kt0 + r, qoff)) bits &= ~(1u << r);
        um = wave_ballot(bits != 0u);
        om = wave_ballot((bits >> wv) & 1u);
      }
      const int q = __builtin_ctzll(um);
      um &= um - 1ull;
      own_out = (om >> q) & 1ull;
      return q0c + q;
    };
    F32Rows<D> qr, dr;
    float vtq = 0.f;
    auto issue = [&](int qt) {
      qr.load(qx, b, h, 32 * qt, Nq, wv);
      dr.load(dox, b, h, 32 * qt, Nq, wv);
      if (wv == 0 && l < 32) vtq = beta * tau_coeff(qoff + 32 * qt + l, P.inv_d);
    };
    bool cown = false;
    int qt = next_tile(cown);
    if (qt >= 0) issue(qt);
    while (qt >= 0) {
      lds_barrier();  // every wave is done with the previous tile
      qr.template store<KS>(qlds, wv);
      dr.template store<KS>(dlds, wv);
      if (wv == 0 && l < 32) tlds[l] = vtq;
      bool nown = false;
      const int qt2 = next_tile(nown);
      if (qt2 >= 0) issue(qt2);  // in flight during this tile's products
      lds_barrier();             // tile qt in LDS
      if (cown) {
        ++visited;
        const int q0 = 32 * qt;
        // S = Q K^T: lane = key, values = query rows crow(r, g)
        const f32x16 S = lds_rows_mma<D, KS>(qlds, Kf, f32x16{});
        const f32x16 Dp = lds_rows_mma<D, KS>(dlds, Vf, f32x16{});
        f32x16 X;
#pragma unroll
        for (int r = 0; r < 16; ++r) X[r] = __builtin_fmaf(S[r], 1.f, -tlds[crow(r, g)]);
        // masks only on the tiles that need them: queries before the key (the diagonal), rows
        // past Nq, keys past Nk
        if (32 * kt + 31 > qoff + q0 || q0 + 31 >= Nq || edge_keys) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int qi = q0 + crow(r, g);
            X[r] = kvalid && qi < Nq && j <= qoff + qi ? X[r] : -1.f;
          }
        }
        f32x16 EV, EK;
        float xm = X[0];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const bool pos = X[r] > 0.f;
          EV[r] = pos ? coef * pow_p<PK>(X[r], pw) : 0.f;
          EK[r] = pos ? coef * dpow_p<PK>(X[r], pw) * Dp[r] : 0.f;
          xm = fmaxf(xm, X[r]);
        }
        computed += (P.occ || wave_ballot(xm > 0.f) != 0ull) ? 1u : 0u;
        lds_tr_mma<D, KS>(dlds, EV, AV);
        lds_tr_mma<D, KS>(qlds, EK, AK);
      }
      cown = nown;
      qt = qt2;
    }
    const int gslot = br == 0 ? B_DK1 : B_DK2;
    const TRef<float> dkx{(float*)P.grad[br == 0 ? 1 : 3], P.s[gslot][0], P.s[gslot][1], P.s[gslot][2]};
    if (act) finish_rows<PolF32, D, false>(AK, nullptr, kvalid ? dkx.row(b, h, j) : nullptr, 1.f);
  }
  if (!act) return;
  const TRef<float> dvx{(float*)P.grad[4], P.s[B_DV][0], P.s[B_DV][1], P.s[B_DV][2]};
  finish_rows<PolF32, D, false>(AV, nullptr, kvalid ? dvx.row(b, h, j) : nullptr, 1.f);
  if (P.stats && l == 0) {
    atomicAdd(P.stats + 0, (unsigned long long)visited);
    atomicAdd(P.stats + 1, (unsigned long long)computed);
  }
}

// Deterministic second stage: fixed-order fp64 sum of the per-wave partials.
constexpr int kFinThreads = kFinSlices;  // one thread per slice
// The partials in the fixed order of tda_fin.hpp: kFinSlices slice sums, then one wave's total.
__global__ void __launch_bounds__(kFinThreads) bwd_finish(const float* ws, int64_t items, const float* lam,
                                                          float* dbeta, float* dlam, int branches) {
  __shared__ double sl[2 * kFinSlices];
  const double2 v = fin_slice_sum(ws, items, (int)threadIdx.x);
  sl[2 * threadIdx.x] = v.x;
  sl[2 * threadIdx.x + 1] = v.y;
  __syncthreads();
  if (threadIdx.x < 64) {
    const double2 t = fin_total(sl);
    if (threadIdx.x == 0) fin_store(t, lam, dbeta, dlam, branches);
  }
}

// ------------------------------------------------------------------ dispatch
template <class Pol, int D, int BR, int PK, bool NORM>
static int launch_bwd_t(const BwdParams& p, void* stream) {
  const int64_t qitems = (int64_t)p.B * p.H * p.nqt, kitems = (int64_t)p.B * p.H * p.nkt;
  hipStream_t s = (hipStream_t)stream;
  if constexpr (!NORM && sizeof(typename Pol::T) == 4) {
    if (!p.pairs) {
      // the forward's block tile pass (every query tile, no lists): the block passes, then the
      // sum over the (branch, head, query tile) partials
      const int BH = p.B * p.H;
      hipLaunchKernelGGL((bwd_dq_blk_f32<D, BR, PK>), dim3((unsigned)(BR * BH * ((p.nqt + kF32Blk - 1) / kF32Blk))),
                         dim3(64 * kF32Blk), 0, s, p);
      launched(s, "bwd_dq");
      hipLaunchKernelGGL((bwd_dkv_blk_f32<D, BR, PK>), dim3((unsigned)(BH * ((p.nkt + kF32Blk - 1) / kF32Blk))),
                         dim3(64 * kF32Blk), 0, s, p);
      launched(s, "bwd_dkv");
      const int e = (int)hipGetLastError();
      return e ? e : launch_bwd_finish(p, BR, (int64_t)BR * qitems, stream);
    }
  }
  if (p.pairs && p.dkvq) {
    // the forward's pair lists (the fp32 candidate pass): the pair passes (tda_bwd_fast.hip),
    // then the tile passes over the lists and key tiles they left, then the sum over the lists'
    // partial slots
    int e = launch_bwd_pairs_f32(p, KernelKey{0, D, BR, PK, NORM ? 1 : 0}, stream);
    if (e) return e;
    const int64_t lists = (int64_t)BR * qitems;
    hipLaunchKernelGGL((bwd_dq<Pol, D, BR, PK, NORM, true>), dim3((unsigned)((lists + 3) / 4)), dim3(256), 0, s, p);
    launched(s, "bwd_dq");
    const unsigned qgrid = (unsigned)(((kitems < 2048 ? kitems : 2048) + 3) / 4);
    hipLaunchKernelGGL((bwd_dkv<Pol, D, BR, PK, NORM, true>), dim3(qgrid), dim3(256), 0, s, p);
    launched(s, "bwd_dkv");
    e = (int)hipGetLastError();
    return e ? e : launch_bwd_finish(p, BR, lists, stream);
  }
  hipLaunchKernelGGL((bwd_dq<Pol, D, BR, PK, NORM>), dim3((unsigned)((qitems + 3) / 4)), dim3(256), 0, s, p);
  launched(s, "bwd_dq");
  hipLaunchKernelGGL((bwd_dkv<Pol, D, BR, PK, NORM>), dim3((unsigned)((kitems + 3) / 4)), dim3(256), 0, s, p);
  launched(s, "bwd_dkv");
  const int e = (int)hipGetLastError();
  return e ? e : launch_bwd_finish(p, BR, (int64_t)p.B * p.H * p.nqt, stream);
}

template <class Pol, int D, int BR, int PK>
static int bsel_norm(const BwdParams& p, const KernelKey& k, void* s) {
  return k.normalize ? launch_bwd_t<Pol, D, BR, PK, true>(p, s) : launch_bwd_t<Pol, D, BR, PK, false>(p, s);
}
template <class Pol, int D, int BR>
static int bsel_pk(const BwdParams& p, const KernelKey& k, void* s) {
  switch (k.pkind) {
    case 2: return bsel_norm<Pol, D, BR, 2>(p, k, s);
    case 1: return bsel_norm<Pol, D, BR, 1>(p, k, s);
    default: return bsel_norm<Pol, D, BR, 0>(p, k, s);
  }
}
template <class Pol, int D>
static int bsel_br(const BwdParams& p, const KernelKey& k, void* s) {
  return k.branches == 2 ? bsel_pk<Pol, D, 2>(p, k, s) : bsel_pk<Pol, D, 1>(p, k, s);
}
template <class Pol>
static int bsel_d(const BwdParams& p, const KernelKey& k, void* s) {
  return k.d == 128 ? bsel_br<Pol, 128>(p, k, s) : bsel_br<Pol, 64>(p, k, s);
}

int launch_bwd_finish(const BwdParams& p, int branches, int64_t items, void* stream) {
  hipLaunchKernelGGL(bwd_finish, dim3(1), dim3(kFinThreads), 0, (hipStream_t)stream, (const float*)p.ws, items, p.lam,
                     p.dbeta, p.dlam, branches);
  launched(stream, "bwd_finish");
  return (int)hipGetLastError();
}

// head_dim 256 runs the column-split kernels of tda_wide.hip; otherwise bf16 runs the
// bitmask-driven kernels of tda_bwd_fast.hip and fp32 runs bwd_dq / bwd_dkv.
int launch_bwd(const BwdParams& p, const KernelKey& k, void* stream) {
  if (k.d == 256) return launch_bwd_wide(p, k, stream);
  return k.dtype == 1 ? launch_bwd_fast(p, k, stream) : bsel_d<PolF32>(p, k, stream);
}

}  // namespace tda
