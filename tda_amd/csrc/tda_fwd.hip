// tda_fwd.hip -- forward pass of threshold attention (TRA / differential TDA) for gfx950.
//
// Reference semantics (snap-research/TDA triton_threshold_attention.py, "TTA"):
//   forward kernel TTA:19-115, differential composition TTA:489-519.
// Every 32x32 (query tile, key tile) pair on or below the diagonal is visited; the scores of
// both branches are formed on the matrix cores, thresholded in registers, and the A.V
// product is issued only when a wave-wide ballot finds a non-zero entry (ReLU leaves almost
// every tile empty: TDA is ultra-sparse).  The two branches share one accumulator:
// out = sum_j (A1_ij - clamp(lambda) A2_ij) v_j, so the differential combine is free.
#include <type_traits>

#include "tda_common.hpp"
#include "tda_params.hpp"
#include "tda_pos.hpp"

namespace tda {

template <class Pol, int D> struct TTileSel;
template <int D> struct TTileSel<PolBF16, D> { using type = TTileBF16<D>; };
template <int D> struct TTileSel<PolF32, D> { using type = TTileF32<D>; };

// One wave per 32-row query tile, four independent waves per workgroup.  Work items are
// ordered longest-first (the last query tiles have the most causal key tiles).
//
// Layouts (see tda_common.hpp): the score tile is computed transposed, S^T = K Q^T, with the
// key rows as the A operand (row fragments loaded from HBM per key tile) and the wave's query
// rows as the resident B operand.  In the C layout each lane then owns one query and 16 keys,
// so the per-query threshold, inverse norm and the causal test are per-lane scalars, and the
// thresholded tile packs directly into the B operand of O^T += V^T A^T.
//
// SCR (fp32, normalised, after key_prep and fwd_screen_i8 ran on the same inputs): the screen's
// bitmask names every key tile holding a non-zero weight (a superset), so the wave visits only
// those tiles; the inverse norms come from the table the screen and key_prep wrote (the values
// the screen's bound is stated for), and the bitmask words are rewritten exactly.
//
// QUEUE (with SCR): only the query tiles the fp32 candidate pass (fwd_cand_f32) queued, whose
// candidate lists did not fit; the waves take them in turn.
template <class Pol, int D, int BR, int PK, bool NORM, bool SCR>
__device__ __forceinline__ void fwd_wave_tile(const FwdParams& P, int qt, int bh, int wv);

template <class Pol, int D, int BR, int PK, bool NORM, bool SCR = false, bool QUEUE = false>
__global__ void __launch_bounds__(256) fwd_wave(FwdParams P) {
  static_assert(!QUEUE || SCR, "the queue comes from the screened candidate pass");
  const int wv = threadIdx.x >> 6;
  const int BH = P.B * P.H;
  if constexpr (QUEUE) {
    const uint32_t queued = P.pvq[0];
    for (uint32_t k = blockIdx.x * 4u + (uint32_t)wv; k < queued; k += gridDim.x * 4u) {
      const int v = (int)P.pvq[1 + k];
      fwd_wave_tile<Pol, D, BR, PK, NORM, SCR>(P, v % P.nqt, v / P.nqt, wv);
    }
    return;
  }
  const int64_t item = (int64_t)blockIdx.x * 4 + wv;
  if (item >= (int64_t)BH * P.nqt) return;  // whole wave leaves; no workgroup barriers below
  fwd_wave_tile<Pol, D, BR, PK, NORM, SCR>(P, P.nqt - 1 - (int)(item / BH), (int)(item % BH), wv);
}

template <class Pol, int D, int BR, int PK, bool NORM, bool SCR>
__device__ __forceinline__ void fwd_wave_tile(const FwdParams& P, int qt, int bh, int wv) {
  static_assert(!SCR || NORM, "the screened pass is the normalised one");
  using T = typename Pol::T;
  using frag = typename Pol::frag;
  constexpr int NT = D / Pol::KS;  // MFMA steps over d
  constexpr int NS = 32 / Pol::KS; // MFMA steps over a 32-key tile
  constexpr int ND = D / 32;       // 32-wide column blocks of the output
  using TT = typename TTileSel<Pol, D>::type;

  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int BH = P.B * P.H;
  const int b = bh / P.H, h = bh % P.H;
  const int Nq = P.Nq, Nk = P.Nk, qoff = P.qoff;
  const int i = qt * 32 + n32;  // this lane's query row
  const bool qvalid = i < Nq;
  const int pq = qoff + i;                   // its position
  const int ktl = kt_last(qt, qoff, P.nkt);  // last key tile the query tile sees

  const TRef<const T> q1{(const T*)P.in[0], P.s[F_Q1][0], P.s[F_Q1][1], P.s[F_Q1][2]};
  const TRef<const T> k1{(const T*)P.in[1], P.s[F_K1][0], P.s[F_K1][1], P.s[F_K1][2]};
  const TRef<const T> q2{(const T*)P.in[2], P.s[F_Q2][0], P.s[F_Q2][1], P.s[F_Q2][2]};
  const TRef<const T> k2{(const T*)P.in[3], P.s[F_K2][0], P.s[F_K2][1], P.s[F_K2][2]};
  const TRef<const T> vv{(const T*)P.in[4], P.s[F_V][0], P.s[F_V][1], P.s[F_V][2]};
  const TRef<T> out{(T*)P.out, P.s[F_OUT][0], P.s[F_OUT][1], P.s[F_OUT][2]};

  frag Q1[NT], Q2[NT];
  {
    const T* r1 = qvalid ? q1.row(b, h, i) : nullptr;
    Pol::template load_rows<NT>(r1, g, Q1);
    if constexpr (BR == 2) {
      const T* r2 = qvalid ? q2.row(b, h, i) : nullptr;
      Pol::template load_rows<NT>(r2, g, Q2);
    }
  }
  float rq1 = 1.f, rq2 = 1.f;
  if constexpr (SCR) {
    if (qvalid) {
      rq1 = P.norms[norm_base(P, N_Q1, bh) + i];
      if constexpr (BR == 2) rq2 = P.norms[norm_base(P, N_Q2, bh) + i];
    }
  } else if constexpr (NORM) {
    rq1 = inv_norm(row_sumsq<Pol, NT>(Q1));
    if constexpr (BR == 2) rq2 = inv_norm(row_sumsq<Pol, NT>(Q2));
    if (P.norms && qvalid && g == 0) {
      P.norms[norm_base(P, N_Q1, bh) + i] = rq1;
      if constexpr (BR == 2) P.norms[norm_base(P, N_Q2, bh) + i] = rq2;
    }
  }
  const float pw = P.p;
  const float tau = (*P.beta) * tau_coeff(pq, P.inv_d);
  float lam = 0.f;
  if constexpr (BR == 2) lam = clamp01(*P.lam);

  __shared__ __attribute__((aligned(16))) bf16 lds_all[(sizeof(T) == 2) ? 4 * TTileBF16<D>::ELEMS : 8];
  TT vt;
  if constexpr (sizeof(T) == 2) vt.lds = lds_all + wv * TTileBF16<D>::ELEMS;

  f32x16 O[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) O[c] = f32x16{};

  // bitmask rows [branch][B*H][query tile][word] of this query tile
  uint32_t* occrow = P.occ ? P.occ + ((int64_t)bh * P.nqt + qt) * P.occ_w : nullptr;
  const int64_t occ_br = (int64_t)BH * P.nqt * P.occ_w;  // distance between the branch planes
  uint32_t word = 0, word2 = 0;
  unsigned visited = 0, computed = 0, checked = 0;

  for (int kt = 0; kt <= ktl; ++kt) {
    bool use1 = true, use2 = true;  // SCR: the branches the screen kept this tile in
    if constexpr (SCR) {
      // the screen's bits of this word (per branch), read before this wave rewrites the word
      const uint32_t s1 = (uint32_t)__builtin_amdgcn_readfirstlane((int)occrow[kt >> 5]);
      const uint32_t s2 = BR == 2 ? (uint32_t)__builtin_amdgcn_readfirstlane((int)occrow[occ_br + (kt >> 5)]) : 0u;
      const uint32_t keep = (s1 | s2) & (~0u << (kt & 31));  // kept tiles kt .. of the word
      const int next = keep ? (kt & ~31) + __builtin_ctz(keep) : (kt | 31) + 1;
      if (next > kt) {  // skipped tiles hold no weight: close the word if it ends among them
        const int wend = kt | 31;
        if (next > wend || next > ktl) {
          if (l == 0) {
            occrow[kt >> 5] = word;
            if constexpr (BR == 2) occrow[occ_br + (kt >> 5)] = word2;
          }
          word = word2 = 0;
          kt = wend;
          continue;
        }
        kt = next;
      }
      use1 = (s1 >> (kt & 31)) & 1u;
      use2 = (s2 >> (kt & 31)) & 1u;
      checked += (use1 ? 1u : 0u) + (use2 ? 1u : 0u);
    }
    const int k0 = kt * 32;
    const int j = k0 + n32;  // key row this lane loads for the A operand
    const bool kfirst = qt == qt_first(kt, qoff);  // the first query tile to see kt writes its norms
    f32x16 S1 = f32x16{}, S2 = f32x16{};
    float rk1r[16] = {}, rk2r[16] = {};
    // a branch the screen did not keep here holds no weight in the tile: no scores for it
    if (use1) {
      frag K1[NT];
      const T* r1 = (j < Nk) ? k1.row(b, h, j) : nullptr;
      Pol::template load_rows<NT>(r1, g, K1);
#pragma unroll
      for (int t = 0; t < NT; ++t) S1 = Pol::mma(K1[t], Q1[t], S1);
      if constexpr (NORM) {
        float rk;
        if constexpr (SCR) rk = j < Nk ? P.norms[norm_base(P, N_K1, bh) + j] : 0.f;
        else rk = inv_norm(row_sumsq<Pol, NT>(K1));
        if (!SCR && P.norms && kfirst && g == 0 && j < Nk) P.norms[norm_base(P, N_K1, bh) + j] = rk;
#pragma unroll
        for (int r = 0; r < 16; ++r) rk1r[r] = __shfl(rk, crow(r, g));
      }
    }
    if (BR == 2 && use2) {
      frag K2[NT];
      const T* r2 = (j < Nk) ? k2.row(b, h, j) : nullptr;
      Pol::template load_rows<NT>(r2, g, K2);
#pragma unroll
      for (int t = 0; t < NT; ++t) S2 = Pol::mma(K2[t], Q2[t], S2);
      if constexpr (NORM) {
        float rk;
        if constexpr (SCR) rk = j < Nk ? P.norms[norm_base(P, N_K2, bh) + j] : 0.f;
        else rk = inv_norm(row_sumsq<Pol, NT>(K2));
        if (!SCR && P.norms && kfirst && g == 0 && j < Nk) P.norms[norm_base(P, N_K2, bh) + j] = rk;
#pragma unroll
        for (int r = 0; r < 16; ++r) rk2r[r] = __shfl(rk, crow(r, g));
      }
    }

    // Threshold test.  x = fma(s * rk_j, rq_i, -tau_i) is monotone in s * rk_j, so the tile
    // max decides "any x > 0" exactly.
    float m1 = -INFINITY, m2 = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = k0 + crow(r, g);
      const bool valid = qvalid && key <= pq && key < Nk;
      if constexpr (NORM) S1[r] *= rk1r[r];
      m1 = fmaxf(m1, valid ? S1[r] : -INFINITY);
      if constexpr (BR == 2) {
        if constexpr (NORM) S2[r] *= rk2r[r];
        m2 = fmaxf(m2, valid ? S2[r] : -INFINITY);
      }
    }
    const bool any1 = use1 && wave_ballot(__builtin_fmaf(m1, rq1, -tau) > 0.f) != 0ull;
    bool any2 = false;
    if constexpr (BR == 2) any2 = use2 && wave_ballot(__builtin_fmaf(m2, rq2, -tau) > 0.f) != 0ull;
    visited += BR;
    computed += (any1 ? 1 : 0) + (any2 ? 1 : 0);
    if (any1) word |= 1u << (kt & 31);
    if (any2) word2 |= 1u << (kt & 31);
    // the query tile's pairs are in no list: the column bucket of the key tile is incomplete
    if (P.colcnt && (any1 || any2) && l == 0) atomicOr(P.colcnt + (int64_t)bh * P.nkt + kt, kColTaint);
    if (any1 || any2) {
      f32x16 C;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + crow(r, g);
        const bool valid = qvalid && key <= pq && key < Nk;
        const float x1 = __builtin_fmaf(S1[r], rq1, -tau);
        float a = (valid && any1 && x1 > 0.f) ? pow_p<PK>(x1, pw) : 0.f;
        if constexpr (BR == 2) {
          const float x2 = __builtin_fmaf(S2[r], rq2, -tau);
          const float a2 = (valid && any2 && x2 > 0.f) ? pow_p<PK>(x2, pw) : 0.f;
          a = __builtin_fmaf(-lam, a2, a);
        }
        C[r] = a;
      }
      if constexpr (sizeof(T) == 2) {
        vt.stage(vv, b, h, k0, Nk);
        wave_lds_sync();
      } else {
        vt.set(vv, b, h, k0, Nk);
      }
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        const frag bp = Pol::pack_c(C, s);
#pragma unroll
        for (int c = 0; c < ND; ++c) O[c] = Pol::mma(vt.frag(s, c), bp, O[c]);
      }
      if constexpr (sizeof(T) == 2) wave_lds_sync();
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
  if (P.pairs && l == 0) {  // this pass writes no pair list: the backward walks the tiles
#pragma unroll
    for (int br = 0; br < BR; ++br)
      P.pairs[pair_lists(BR, BH, P.nqt) * 4 * kPairCap + ((int64_t)br * BH + bh) * P.nqt + qt] = kPairOverflow;
  }

  // Key tiles no query tile sees (keys past the last query position): their inverse norms
  // still go to the table (the backward's normalize epilogue reads every key row's), written
  // by the last query tile's wave (with SCR key_prep wrote every key row's).
  if constexpr (NORM && !SCR) {
    if (P.norms && qt == P.nqt - 1) {
      for (int kt = ktl + 1; kt < P.nkt; ++kt) {
        const int j = 32 * kt + n32;
        frag K[NT];
        const T* r1 = (j < Nk) ? k1.row(b, h, j) : nullptr;
        Pol::template load_rows<NT>(r1, g, K);
        const float rka = inv_norm(row_sumsq<Pol, NT>(K));
        if (g == 0 && j < Nk) P.norms[norm_base(P, N_K1, bh) + j] = rka;
        if constexpr (BR == 2) {
          const T* r2 = (j < Nk) ? k2.row(b, h, j) : nullptr;
          Pol::template load_rows<NT>(r2, g, K);
          const float rkb = inv_norm(row_sumsq<Pol, NT>(K));
          if (g == 0 && j < Nk) P.norms[norm_base(P, N_K2, bh) + j] = rkb;
        }
      }
    }
  }

  if (qvalid) {
    T* orow = out.row(b, h, i);
#pragma unroll
    for (int c = 0; c < ND; ++c)
#pragma unroll
      for (int u = 0; u < 4; ++u)
        store4(orow + 32 * c + 8 * u + 4 * g, O[c][4 * u], O[c][4 * u + 1], O[c][4 * u + 2], O[c][4 * u + 3]);
  }
  if (P.stats && l == 0) {  // with SCR the screen counted the causal tiles; `checked`: its kept ones
    atomicAdd(P.stats + (SCR ? 2 : 0), (unsigned long long)(SCR ? checked : visited));
    atomicAdd(P.stats + 1, (unsigned long long)computed);
  }
}

// ------------------------------------------------------------------ fwd_wave_blk
// The fp32 pass without normalisation (every causal tile scored) over blocks of four
// consecutive query tiles of one head, one wave each, as fwd_pv_blk does for bf16: the waves walk
// the block's causal key tiles in step and share each tile's key rows (every branch) and V rows,
// which the workgroup loads once (each wave a quarter of the rows, one tile ahead into
// registers) into LDS; two barriers per tile (the tile is rewritten once every wave is done with
// it).  A wave scores only the tiles its own query tile sees, with fwd_wave's arithmetic: the
// key rows' fragments in the load_rows order (lane half g: elements g D/2 .. of row n), V^T one
// key per lane half and step, the same test, weights, bitmask, counters and output.
template <int D, int BR, int PK>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D <= 64 ? 2 : 1)))
fwd_wave_blk(FwdParams P) {
  using Pol = PolF32;
  constexpr int W = 4, NT = D / 2, NS = 16, ND = D / 32;
  constexpr int KS = D + 4;          // key tile row stride (floats)
  constexpr int VS = D + 8;          // V tile row stride: rows 4 apart 32 banks apart
  constexpr int CPR = D / 4;         // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;      // rows per load instruction
  constexpr int LPW = 32 / RPI / W;  // load instructions per wave and matrix
  static_assert(LPW >= 1 && LPW * RPI * W == 32, "tile rows split evenly over the waves");
  __shared__ __attribute__((aligned(16))) float klds[BR][32 * KS];
  __shared__ __attribute__((aligned(16))) float vlds[32 * VS];

  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int BH = P.B * P.H, Nq = P.Nq, Nk = P.Nk, nqt = P.nqt, qoff = P.qoff;
  const int nqb = (nqt + W - 1) / W;
  // longest blocks (last query tiles) of every head first
  const int bid = blockIdx.x, jb = nqb - 1 - bid / BH, bh = bid % BH;
  const int b = bh / P.H, h = bh % P.H;
  const int qt = W * jb + wv;
  const bool act = qt < nqt;  // wave-uniform: waves past the last query tile only load
  const int i = 32 * qt + n32;
  const bool qvalid = act && i < Nq;
  const int pq = qoff + i;
  const int ktl = act ? kt_last(qt, qoff, P.nkt) : -1;                       // this wave's last key tile
  const int ktl_b = kt_last(min(W * jb + W - 1, nqt - 1), qoff, P.nkt);  // the block's

  const TRef<const float> qr[2] = {{(const float*)P.in[F_Q1], P.s[F_Q1][0], P.s[F_Q1][1], P.s[F_Q1][2]},
                                   {(const float*)P.in[F_Q2], P.s[F_Q2][0], P.s[F_Q2][1], P.s[F_Q2][2]}};
  const TRef<const float> kr[2] = {{(const float*)P.in[F_K1], P.s[F_K1][0], P.s[F_K1][1], P.s[F_K1][2]},
                                   {(const float*)P.in[F_K2], P.s[F_K2][0], P.s[F_K2][1], P.s[F_K2][2]}};
  const TRef<const float> vv{(const float*)P.in[F_V], P.s[F_V][0], P.s[F_V][1], P.s[F_V][2]};
  const TRef<float> out{(float*)P.out, P.s[F_OUT][0], P.s[F_OUT][1], P.s[F_OUT][2]};

  float Q[BR][NT];
#pragma unroll
  for (int br = 0; br < BR; ++br) Pol::template load_rows<NT>(qvalid ? qr[br].row(b, h, i) : nullptr, g, Q[br]);
  const float pw = P.p;
  const float tau = (*P.beta) * tau_coeff(pq, P.inv_d);
  float lam = 0.f;
  if constexpr (BR == 2) lam = clamp01(*P.lam);

  // this wave's rows of a tile: RPI (LPW wv + u) + l / CPR, chunk l % CPR (rows past Nk: Nk - 1)
  f32x4 kreg[BR][LPW], vreg[LPW];
  auto issue = [&](int kt) {
#pragma unroll
    for (int u = 0; u < LPW; ++u) {
      const int r = min(32 * kt + RPI * (LPW * wv + u) + l / CPR, Nk - 1);
#pragma unroll
      for (int br = 0; br < BR; ++br) kreg[br][u] = *reinterpret_cast<const f32x4*>(kr[br].row(b, h, r) + 4 * (l % CPR));
      vreg[u] = *reinterpret_cast<const f32x4*>(vv.row(b, h, r) + 4 * (l % CPR));
    }
  };

  f32x16 O[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) O[c] = f32x16{};
  uint32_t* occrow = P.occ && act ? P.occ + ((int64_t)bh * nqt + qt) * P.occ_w : nullptr;
  const int64_t occ_br = (int64_t)BH * nqt * P.occ_w;  // distance between the branch planes
  uint32_t word = 0, word2 = 0;
  unsigned visited = 0, computed = 0;

  issue(0);
  for (int kt = 0; kt <= ktl_b; ++kt) {
    lds_barrier();  // every wave is done with the previous tile
#pragma unroll
    for (int u = 0; u < LPW; ++u) {
      const int r = RPI * (LPW * wv + u) + l / CPR;
#pragma unroll
      for (int br = 0; br < BR; ++br) *reinterpret_cast<f32x4*>(klds[br] + r * KS + 4 * (l % CPR)) = kreg[br][u];
      *reinterpret_cast<f32x4*>(vlds + r * VS + 4 * (l % CPR)) = vreg[u];
    }
    if (kt < ktl_b) issue(kt + 1);  // in flight during this tile's products
    lds_barrier();                  // tile kt in LDS
    if (kt > ktl) continue;         // (uniform) not seen by this wave's query tile
    const int k0 = 32 * kt;
    f32x16 S[BR];
#pragma unroll
    for (int br = 0; br < BR; ++br) {
      S[br] = f32x16{};
      const float* kp = klds[br] + n32 * KS + g * NT;
#pragma unroll
      for (int m = 0; m < NT / 4; ++m) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(kp + 4 * m);
#pragma unroll
        for (int e = 0; e < 4; ++e) S[br] = Pol::mma(v[e], Q[br][4 * m + e], S[br]);
      }
    }
    // threshold test: the tile max of the valid scores decides "any x > 0" exactly
    bool any[2] = {false, false};
#pragma unroll
    for (int br = 0; br < BR; ++br) {
      float m = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + crow(r, g);
        const bool valid = qvalid && key <= pq && key < Nk;
        m = fmaxf(m, valid ? S[br][r] : -INFINITY);
      }
      any[br] = wave_ballot(m - tau > 0.f) != 0ull;
    }
    visited += BR;
    computed += (any[0] ? 1 : 0) + (any[1] ? 1 : 0);
    if (any[0]) word |= 1u << (kt & 31);
    if (any[1]) word2 |= 1u << (kt & 31);
    // the query tile's pairs are in no list: the column bucket of the key tile is incomplete
    if (P.colcnt && (any[0] || any[1]) && l == 0) atomicOr(P.colcnt + (int64_t)bh * P.nkt + kt, kColTaint);
    if (any[0] || any[1]) {
      f32x16 C;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + crow(r, g);
        const bool valid = qvalid && key <= pq && key < Nk;
        const float x1 = __builtin_fmaf(S[0][r], 1.f, -tau);
        float a = (valid && any[0] && x1 > 0.f) ? pow_p<PK>(x1, pw) : 0.f;
        if constexpr (BR == 2) {
          const float x2 = __builtin_fmaf(S[1][r], 1.f, -tau);
          const float a2 = (valid && any[1] && x2 > 0.f) ? pow_p<PK>(x2, pw) : 0.f;
          a = __builtin_fmaf(-lam, a2, a);
        }
        C[r] = a;
      }
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        const float* vp = vlds + crow(st, g) * VS + n32;
#pragma unroll
        for (int c = 0; c < ND; ++c) O[c] = Pol::mma(vp[32 * c], C[st], O[c]);
      }
    }
    if (occrow && (((kt & 31) == 31) || kt == ktl)) {
      if (l == 0) {
        occrow[kt >> 5] = word;
        if constexpr (BR == 2) occrow[occ_br + (kt >> 5)] = word2;
      }
      word = word2 = 0;
    }
  }
  if (!act) return;
  if (occrow && l == 0) {
    for (int w = (ktl >> 5) + 1; w < P.occ_w; ++w) {
      occrow[w] = 0u;
      if constexpr (BR == 2) occrow[occ_br + w] = 0u;
    }
  }
  if (P.pairs && l == 0) {  // this pass writes no pair list: the backward walks the tiles
#pragma unroll
    for (int br = 0; br < BR; ++br)
      P.pairs[pair_lists(BR, BH, nqt) * 4 * kPairCap + ((int64_t)br * BH + bh) * nqt + qt] = kPairOverflow;
  }
  if (qvalid) {
    float* orow = out.row(b, h, i);
#pragma unroll
    for (int c = 0; c < ND; ++c)
#pragma unroll
      for (int u = 0; u < 4; ++u)
        store4(orow + 32 * c + 8 * u + 4 * g, O[c][4 * u], O[c][4 * u + 1], O[c][4 * u + 2], O[c][4 * u + 3]);
  }
  if (P.stats && l == 0) {
    atomicAdd(P.stats + 0, (unsigned long long)visited);
    atomicAdd(P.stats + 1, (unsigned long long)computed);
  }
}

// ------------------------------------------------------------------ fwd_cand_f32
// The fp32 exact pass over the screen's candidate keys (normalised, more than one query tile):
// one workgroup per query tile whose candidate lists (every branch) fit, one wave per branch.
// The score tile of the query rows against the candidate keys (row c = candidate c; rows past
// the count zero) takes the operands straight from the rows, in the element order of fwd_wave's
// row fragments (lane half g: elements g d/2 + t, step t), so each score is bitwise the one
// fwd_wave and the backward compute for that pair; the weights ReLU(x)^p with x = fma(s rk, rq,
// -tau) and the causal mask accumulate coef A V over the candidates with a non-zero weight, one
// fused multiply-add per output element and candidate in key order (the sums do not depend on the
// list's other keys).  The bitmask row is rewritten from the key tiles holding a
// non-zero weight.  A query tile whose list overflowed goes to the queue of fwd_wave<QUEUE>.  With
// two branches the second wave's sum is added to the first's through LDS.
template <int D, int BR, int PK>
__global__ void __launch_bounds__(64 * BR) fwd_cand_f32(FwdParams P) {
  constexpr int NT = D / 2, ND = D / 32;
  __shared__ int ckeys[BR][32];     // candidate keys (-1: none)
  __shared__ float crks[BR][32];    // their inverse norms
  __shared__ float xch[BR == 2 ? 16 * ND * 64 : 1];
  __shared__ __attribute__((aligned(16))) u32x4 plists[BR][kPairCap];  // the branch's pair list

  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int wv = BR == 2 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) : 0;  // = its branch
  const int BH = P.B * P.H, Nq = P.Nq, Nk = P.Nk, nqt = P.nqt, qoff = P.qoff;
  int bh, qt;
  {
    const int bid = blockIdx.x;  // one head's query tiles consecutive on one XCD
    if (BH % 8 == 0) {
      const int x = bid & 7, j = bid >> 3;
      bh = x + 8 * (j / nqt);
      qt = j % nqt;
    } else {
      bh = bid / nqt;
      qt = bid % nqt;
    }
  }
  if (bh >= BH) return;  // the same for both waves
  const uint32_t* counts = P.cand + pair_lists(BR, BH, nqt) * kCandCap;
  uint32_t nc[BR];
#pragma unroll
  for (int br = 0; br < BR; ++br) nc[br] = counts[((int64_t)br * BH + bh) * nqt + qt];
  bool fit = true;
#pragma unroll
  for (int br = 0; br < BR; ++br) fit = fit && nc[br] <= (uint32_t)kCandCap;
  if (!fit) {  // fwd_wave<QUEUE> walks the bitmask tiles (both waves leave: the test is the same)
    if (l == 0 && wv == 0) P.pvq[1 + atomicAdd(P.pvq, 1u)] = (uint32_t)(bh * nqt + qt);
    return;
  }
  const int br = wv;
  const uint32_t n = nc[br];
  const int64_t lidx = ((int64_t)br * BH + bh) * nqt + qt;
  int kraw = (int)P.cand[lidx * kCandCap + (l & 31)];
  if (P.screen_items > (Nq + 255) / 256) {
    // the screen split some key ranges over several items, which append in any order: sort the
    // list (its keys are distinct) by rank, so the sums run in key order
    int rank = l & 31;
    if ((uint32_t)(l & 31) < n) {
      rank = 0;
      for (int f = 0; f < 32; ++f) {
        const int a = __builtin_amdgcn_readlane(kraw, f);
        rank += ((uint32_t)f < n && a < kraw) ? 1 : 0;
      }
    }
    kraw = __builtin_amdgcn_ds_permute(4 * rank, kraw);
  }

  const int b = bh / P.H, h = bh % P.H;
  const int iq = 32 * qt + n32;
  const bool valid = iq < Nq;
  const int pq = qoff + iq;
  const int klast = kt_last(qt, qoff, P.nkt);
  const int nw = (klast >> 5) + 1;  // bitmask words of the row
  const float tau = *P.beta * tau_coeff(pq, P.inv_d);
  const float pw = P.p;
  float lam = 0.f;
  if constexpr (BR == 2) lam = clamp01(*P.lam);
  int* ckey = ckeys[br];
  float* crk = crks[br];
  uint32_t* orow = P.occ + lidx * P.occ_w;
  unsigned computed = 0, checked = 0;
  uint32_t npairs = 0;

  f32x16 O[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) O[c] = f32x16{};
  if (n > 0) {
    const int qslot = br ? F_Q2 : F_Q1, kslot = br ? F_K2 : F_K1;
    const float* qhead = (const float*)P.in[qslot] + (int64_t)b * P.s[qslot][0] + (int64_t)h * P.s[qslot][1];
    const float* khead = (const float*)P.in[kslot] + (int64_t)b * P.s[kslot][0] + (int64_t)h * P.s[kslot][1];
    const float* vhead = (const float*)P.in[F_V] + (int64_t)b * P.s[F_V][0] + (int64_t)h * P.s[F_V][1];
    const int64_t sq = P.s[qslot][2], sk = P.s[kslot][2], sv = P.s[F_V][2];
    const float coef = br == 0 ? 1.f : -lam;
    const int key_l = l < (int)n && kraw >= 0 && kraw < Nk ? kraw : -1;  // lanes 0..31: candidate l
    const float rk_l = key_l >= 0 ? P.norms[norm_base(P, br ? N_K2 : N_K1, bh) + key_l] : 0.f;
    const float rq = P.norms[norm_base(P, br ? N_Q2 : N_Q1, bh) + min(iq, Nq - 1)];
    if (l < 32) {
      ckey[l] = key_l;
      crk[l] = rk_l;
    }
    const int key_m = __shfl(key_l, n32);  // the candidate this lane supplies to the A operand
    const float* krow = key_m >= 0 ? khead + (int64_t)key_m * sk + g * NT : nullptr;
    const float* qrow = qhead + (int64_t)min(iq, Nq - 1) * sq + g * NT;
    f32x16 S = {};
#pragma unroll
    for (int m = 0; m < NT / 4; ++m) {
      const f32x4 a = krow ? *reinterpret_cast<const f32x4*>(krow + 4 * m) : f32x4{0.f, 0.f, 0.f, 0.f};
      const f32x4 q = *reinterpret_cast<const f32x4*>(qrow + 4 * m);
#pragma unroll
      for (int e = 0; e < 4; ++e) S = PolF32::mma(a[e], q[e], S);
    }
    wave_lds_sync();
    uint32_t cnz = 0u;  // candidates with a non-zero weight
    f32x16 C;           // value r: the weight of candidate crow(r, g) for the lane's query
    u32x4* plist = plists[br];
    uint32_t* pent = P.pairs ? P.pairs + lidx * (4 * kPairCap) : nullptr;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int c = crow(r, g);
      const int key = ckey[c];
      const float x = __builtin_fmaf(S[r] * crk[c], rq, -tau);
      const bool pos = key >= 0 && key <= pq && key < Nk && x > 0.f;
      C[r] = pos ? coef * pow_p<PK>(x, pw) : 0.f;
      const bool hit = valid && pos;
      const uint64_t bal = wave_ballot(hit);
      cnz |= ((uint32_t)bal ? 1u << crow(r, 0) : 0u) | ((uint32_t)(bal >> 32) ? 1u << crow(r, 1) : 0u);
      if (pent) {  // the pair list: the non-zero weights in the order (value r, lane)
        const uint32_t slot = npairs + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
        if (hit && slot < (uint32_t)kPairCap)
          plist[slot] = u32x4{(uint32_t)key, (uint32_t)n32, __builtin_bit_cast(uint32_t, x), kNoSlot};
        npairs += (uint32_t)__builtin_popcountll(bal);
      }
    }
    // The list's entries, lane e for entry e: with column buckets each takes a slot in the bucket
    // of its key tile and the entry records it; a list past the cap taints the columns of every
    // candidate with a non-zero weight instead (its pairs past the cap are in no list).
    const uint32_t ne = min(npairs, (uint32_t)kPairCap);
    u32x4 pe = u32x4{0u, 0u, 0u, kNoSlot};
    uint32_t* ccol = P.colcnt ? P.colcnt + (int64_t)bh * P.nkt : nullptr;
    if (pent) {
      wave_lds_sync();
      if ((uint32_t)l < ne) {
        pe = plist[l];
        if (ccol) pe[3] = atomicAdd(ccol + ((int)pe[0] >> 5), 1u) & ~kColTaint;  // the slot
      }
      if (ccol && npairs > (uint32_t)kPairCap && l < 32 && ((cnz >> l) & 1u)) atomicOr(ccol + (ckey[l] >> 5), kColTaint);
      if ((uint32_t)l < ne) {
        *reinterpret_cast<u32x4*>(pent + 4 * l) = pe;
        if (ccol && pe[3] < (uint32_t)kColCap)
          *reinterpret_cast<u32x4*>(P.colbuf + (((int64_t)bh * P.nkt + ((int)pe[0] >> 5)) * kColCap + pe[3]) * 4) =
              u32x4{((uint32_t)(32 * qt) + pe[1]) | (br ? 0x80000000u : 0u), pe[0] & 31u, pe[2], 0u};
      }
    }
    // out_i += w_ic v_c over the candidates with a non-zero weight, one fused multiply-add per
    // element in increasing key order: each row's sum takes exactly its own non-zero terms in key
    // order (the other candidates add w = 0), so it does not depend on which other keys the
    // tile's list holds (another tiling, keys past the last position).  Lane (n, g) holds the
    // elements 32 c + 8 u + 4 g .. + 3 of row n.
#pragma unroll
    for (int c = 0; c < 32; ++c) {
      if (!((cnz >> c) & 1u)) continue;
      const int r = (c & 3) | ((c >> 3) << 2), gc = (c >> 2) & 1;  // crow(r, gc) = c
      const float w = __shfl(C[r], n32 + 32 * gc);
      const float* vrow = vhead + (int64_t)__builtin_amdgcn_readfirstlane(ckey[c]) * sv + 4 * g;
#pragma unroll
      for (int cb = 0; cb < ND; ++cb)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const f32x4 vv4 = *reinterpret_cast<const f32x4*>(vrow + 32 * cb + 8 * u);
#pragma unroll
          for (int e = 0; e < 4; ++e) O[cb][4 * u + e] = __builtin_fmaf(w, vv4[e], O[cb][4 * u + e]);
        }
    }
    // the bitmask row: lane w rewrites word w from the key tiles of the candidates with a
    // non-zero weight (the screen's words cover the key tiles of all candidates, nothing else)
    for (int w0 = 0; w0 < nw; w0 += 64) {
      uint32_t word = 0u;
      for (uint32_t m = cnz; m; m &= m - 1u) {
        const int kt = __builtin_amdgcn_readfirstlane(ckey[__builtin_ctz(m)]) >> 5;
        word |= (kt >> 5) == w0 + l ? 1u << (kt & 31) : 0u;
      }
      if (w0 + l < nw) {
        if (P.stats) checked += (unsigned)__builtin_popcount(orow[w0 + l]);
        orow[w0 + l] = word;
      }
      computed += (unsigned)__builtin_popcount(word);
    }
  }
  if (P.pairs && l == 0) P.pairs[pair_lists(P.nbr, BH, nqt) * 4 * kPairCap + lidx] = npairs;
  if (P.stats) {
    const float cs = wave_sum((float)computed), ks = wave_sum((float)checked);
    if (l == 0 && ks > 0.f) {
      atomicAdd(P.stats + 1, (unsigned long long)cs);
      atomicAdd(P.stats + 2, (unsigned long long)ks);
    }
  }
  if constexpr (BR == 2) {
    // out = O (branch 0's wave) + O (branch 1's wave, -lambda A2 V), added through LDS
    __syncthreads();
    if (wv == 1) {
#pragma unroll
      for (int c = 0; c < ND; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) xch[(16 * c + r) * 64 + l] = O[c][r];
    }
    __syncthreads();
    if (wv == 1) return;
#pragma unroll
    for (int c = 0; c < ND; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) O[c][r] += xch[(16 * c + r) * 64 + l];
  }
  if (valid) {
    float* orow_out = (float*)P.out + (int64_t)b * P.s[F_OUT][0] + (int64_t)h * P.s[F_OUT][1] + (int64_t)iq * P.s[F_OUT][2];
#pragma unroll
    for (int c = 0; c < ND; ++c)
#pragma unroll
      for (int u = 0; u < 4; ++u)
        store4(orow_out + 32 * c + 8 * u + 4 * g, O[c][4 * u], O[c][4 * u + 1], O[c][4 * u + 2], O[c][4 * u + 3]);
  }
}

// ------------------------------------------------------------------ dispatch
// Normalised fp32 calls with more than one query tile and the int8 keys' workspace run the int8
// screen first (key_prep and fwd_screen_i8 on the fp32 rows, tda_fwd_sparse.hip), then the
// screened fwd_wave.
template <class Pol, int D, int BR, int PK, bool NORM>
static int launch_fwd_t(const FwdParams& p, const KernelKey& k, void* stream) {
  static_assert(std::is_same<Pol, PolF32>::value, "the fp32 dispatch (bf16 runs tda_fwd_sparse.hip)");
  const int64_t items = (int64_t)p.B * p.H * p.nqt;
  const unsigned grid = (unsigned)((items + 3) / 4);
  if (NORM && p.k8 && p.nqt > 1 && p.cand) {
    // the int8 screen with candidate lists, the candidate pass, then the tile pass over the query
    // tiles whose lists overflowed
    const int e = launch_fwd_screen_f32(p, k, stream);
    if (e) return e;
    hipLaunchKernelGGL((fwd_cand_f32<D, BR, PK>), dim3((unsigned)items), dim3(64 * BR), 0, (hipStream_t)stream, p);
    launched(stream, "fwd_cand_f32");
    const unsigned qgrid = (unsigned)(((items < 2048 ? items : 2048) + 3) / 4);
    hipLaunchKernelGGL((fwd_wave<Pol, D, BR, PK, NORM, NORM, NORM>), dim3(qgrid), dim3(256), 0, (hipStream_t)stream, p);
  } else if (!NORM && p.nqt > 1) {  // blocks of query tiles sharing their key and V tiles
    const unsigned blocks = (unsigned)(p.B * p.H * ((p.nqt + 3) / 4));
    hipLaunchKernelGGL((fwd_wave_blk<D, BR, PK>), dim3(blocks), dim3(256), 0, (hipStream_t)stream, p);
  } else {
    hipLaunchKernelGGL((fwd_wave<Pol, D, BR, PK, NORM>), dim3(grid), dim3(256), 0, (hipStream_t)stream, p);
  }
  launched(stream, "fwd_wave");
  return (int)hipGetLastError();
}

template <class Pol, int D, int BR, int PK>
static int sel_norm(const FwdParams& p, const KernelKey& k, void* s) {
  return k.normalize ? launch_fwd_t<Pol, D, BR, PK, true>(p, k, s) : launch_fwd_t<Pol, D, BR, PK, false>(p, k, s);
}
template <class Pol, int D, int BR>
static int sel_pk(const FwdParams& p, const KernelKey& k, void* s) {
  switch (k.pkind) {
    case 2: return sel_norm<Pol, D, BR, 2>(p, k, s);
    case 1: return sel_norm<Pol, D, BR, 1>(p, k, s);
    default: return sel_norm<Pol, D, BR, 0>(p, k, s);
  }
}
template <class Pol, int D>
static int sel_br(const FwdParams& p, const KernelKey& k, void* s) {
  return k.branches == 2 ? sel_pk<Pol, D, 2>(p, k, s) : sel_pk<Pol, D, 1>(p, k, s);
}
template <class Pol>
static int sel_d(const FwdParams& p, const KernelKey& k, void* s) {
  return k.d == 128 ? sel_br<Pol, 128>(p, k, s) : sel_br<Pol, 64>(p, k, s);
}

// The zero range of a call whose path has no screen (which clears it otherwise): 16 bytes per
// lane, streaming stores.
__global__ void __launch_bounds__(256) zero_range(void* z, int64_t units) {
  for (int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x; u < units; u += (int64_t)gridDim.x * 256)
    __builtin_nontemporal_store(u32x4{0u, 0u, 0u, 0u}, reinterpret_cast<u32x4*>(z) + u);
}
int launch_zero(const FwdParams& p, void* stream) {
  if (!p.zero || p.zero_units <= 0) return 0;
  const int64_t blocks = (p.zero_units + 255) / 256;
  hipLaunchKernelGGL(zero_range, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, (hipStream_t)stream,
                     p.zero, p.zero_units);
  launched(stream, "zero_range");
  return (int)hipGetLastError();
}

// head_dim 256 runs tda_wide.hip; otherwise bf16 runs the screen + sparse A.V kernels (tda_fwd_sparse.hip), or with a single query tile
// the split-key decode kernels (tda_fwd_decode.hip); fp32 runs fwd_wave, after the int8 screen
// when normalised with more than one query tile.  The screens, and the bf16 block tile pass
// without normalisation, clear the call's zero range; the other paths launch zero_range.
int launch_fwd(const FwdParams& p, const KernelKey& k, void* stream) {
  if (p.zero && p.zero_per_it == 0) {
    // a zero range too large for the screen's per-item slices: cleared whole first
    const int ez = launch_zero(p, stream);
    if (ez) return ez;
    FwdParams q = p;
    q.zero = nullptr;
    q.zero_units = 0;
    return launch_fwd(q, k, stream);
  }
  int e;
  if (k.d == 256) {  // both dtypes: the column-split kernels of tda_wide.hip (no screen)
    e = launch_fwd_wide(p, k, stream);
    return e ? e : launch_zero(p, stream);
  }
  if (k.dtype == 1 && !(p.nqt == 1 && p.part)) return launch_fwd_sparse(p, k, stream);
  if (k.dtype == 1) e = launch_fwd_decode(p, k, p.part, stream);
  else e = sel_d<PolF32>(p, k, stream);
  const bool screened = k.dtype == 0 && k.normalize && p.k8 && p.nqt > 1;  // the screen cleared it
  return e ? e : screened ? 0 : launch_zero(p, stream);
}

}  // namespace tda
