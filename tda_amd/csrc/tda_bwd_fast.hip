// tda_bwd_fast.hip -- bf16 backward of threshold attention for gfx950, driven by the forward's
// tile-occupancy bitmask.
//
// Reference semantics: snap-research/TDA triton_threshold_attention.py backward kernels
// (TTA:118-324) and host backward (TTA:406-469); the normalize / clamp / combine gradients
// follow torch autograd of TTA:505-517; dbeta is new (the reference returns None, TTA:469).
// The formulas are listed at the top of tda_bwd.hip.
//
// Layout of the work.  With the forward's pair lists (the non-zero weights of each (branch,
// query tile), see tda_params.hpp) the backward touches only the rows those weights name:
//   * bwd_dq_pairs: one wave per (branch, query tile) whose list fit; whole-row vector work per
//     pair, the tile's other gradient rows stored as zeros.
//   * bwd_dkv_pairs: one wave per key tile whose bitmask column has only lists that fit; whole-
//     row vector work per key row its pairs name, with the dk weight of each pair stored by
//     bwd_dq_pairs (no V, no matrix cores), the tile's other gradient rows stored as zeros.
// Gradient rows are streaming (non-temporal) stores: nothing reads them back soon.
// The tile passes take the rest (lists past the cap, or no lists at all), driven by the bitmask:
//   * bwd_dq_fast: per (branch, query tile), several to a wave when lists exist (their counts
//     tested in one round); walks the set bits of the bitmask row, so only key tiles with a
//     non-zero score are touched; dq_br is finished (F.normalize backward) at the end.
//   * bwd_dkv_fast: per key tile, from the queue bwd_dkv_pairs fills when lists exist; walks
//     the set bits of the bitmask column of each branch; dv accumulates over both branches
//     (A1 - lam A2), dk_br is finished per branch.
// The tile passes fetch each visited tile with direct global->LDS loads into a wave-private,
// chunk-swizzled row-major tile that serves both as row fragments (ds_read_b128) and, through
// the LDS transpose read, as transposed fragments.  dbeta / dlambda partials: one pair per
// (branch, query tile), summed in a fixed order by bwd_finish.
#include "tda_common.hpp"
#include "tda_params.hpp"
#include "tda_pos.hpp"

namespace tda {


// Direct global->LDS load of rows r0..r0+31 of a (N, D) row set (row stride st elements;
// rows >= n clamped to n-1, their values only meet zero weights) into a swizzled tile.
// One instruction moves 1 KiB: 64 lanes x 16 bytes.
template <int D>
__device__ __forceinline__ void dma_tile(const bf16* rows, int64_t st, int r0, int n, bf16* tile) {
  constexpr int CH = D / 8, RPI = 64 / CH;
  const int l = lane_id();
#pragma unroll
  for (int u = 0; u < 32 / RPI; ++u) {
    const int r = u * RPI + l / CH;
    const int c = (l % CH) ^ bswz<D>(r);
    const bf16* src = rows + (int64_t)min(r0 + r, n - 1) * st + 8 * c;
    __builtin_amdgcn_global_load_lds((const void*)src, LDS_PTR(void, tile + u * RPI * D), 16, 0, 0);
  }
}
// 32 floats (one per tile row) by direct load; rows >= n clamped.
__device__ __forceinline__ void dma_row_vals(const float* vals, int r0, int n, float* dst) {
  const int l = lane_id();
  if (l < 32) __builtin_amdgcn_global_load_lds((const void*)(vals + min(r0 + l, n - 1)), LDS_PTR(void, dst), 4, 0, 0);
}
__device__ __forceinline__ void wait_all_loads() { __builtin_amdgcn_s_waitcnt(0); }

// The same loads through a buffer descriptor per tile: the tile sets the descriptor's base and
// size, the lanes add 32-bit offsets within the tile; rows past n read as zeros (the
// descriptor's range check).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
template <int D>
__device__ __forceinline__ void dma_tile_b(const bf16* rows, int64_t st, int r0, int n, bf16* tile) {
  constexpr int CH = D / 8, RPI = 64 / CH;
  const int l = lane_id();
  const int nr = min(32, n - r0);
  const __amdgpu_buffer_rsrc_t rs = rows_rsrc(rows + (int64_t)r0 * st, (uint32_t)(((int64_t)(nr - 1) * st + D) * 2));
  const uint32_t st2 = (uint32_t)(2 * st);  // row stride in bytes (at most 2^26)
#pragma unroll
  for (int u = 0; u < 32 / RPI; ++u) {
    const int r = u * RPI + l / CH;
    const uint32_t off = (uint32_t)r * st2 + 16u * (uint32_t)((l % CH) ^ bswz<D>(r));
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, LDS_PTR(void, tile + u * RPI * D), 16, off, 0, 0, 0);
  }
}
// Lane-distributed pair list: lane e < n holds entry e (key, query row in the tile, x).
struct PairLanes {
  int key, row;
  float x;
  uint32_t slot;  // the pair's column-bucket slot (kNoSlot: none)
};
__device__ __forceinline__ PairLanes load_pairs(const uint32_t* ent, uint32_t n) {
  const int l = lane_id();
  u32x4 e = u32x4{0u, 0u, 0u, 0u};
  if ((uint32_t)l < n) e = *reinterpret_cast<const u32x4*>(ent + 4 * l);
  // x through a bit cast of the whole vector: hipcc compiled __builtin_bit_cast(float, e[2])
  // to element 0 (the key index)
  const f32x4 ef = __builtin_bit_cast(f32x4, e);
  return PairLanes{(int)e[0], (int)e[1], ef[2], e[3]};
}

__device__ __forceinline__ void dma_row_vals_b(const float* vals, int r0, int n, float* dst) {
  const __amdgpu_buffer_rsrc_t rs = rows_rsrc(vals + r0, (uint32_t)(min(32, n - r0) * 4));
  if (lane_id() < 32) __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, LDS_PTR(void, dst), 4, 4 * lane_id(), 0, 0, 0);
}

// Row fragment t of a swizzled tile: lane (m, g) gets elements 16t + 8g .. +7 of row m.
template <int D>
__device__ __forceinline__ bf16x8 tile_row_frag(const bf16* tile, int t) {
  const int l = lane_id(), m = l & 31, g = l >> 5;
  return *reinterpret_cast<const bf16x8*>(tile + m * D + 8 * ((2 * t + g) ^ bswz<D>(m)));
}
// Load this lane's 16 values of a 32-float row table at C rows crow(r, g).
__device__ __forceinline__ void crow_vals(const float* tab, float (&v)[16]) {
  const int g = lane_id() >> 5;
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const f32x4 x = *reinterpret_cast<const f32x4*>(tab + 8 * u + 4 * g);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[4 * u + e] = x[e];
  }
}

// This lane's elements of an input row in the transposed C layout of a gradient tile
// (elements 32c + 8u + 4g .. +3), for the F.normalize backward.
template <int D>
struct GradRow {
  bf16x4 x[D / 32][4];
};
template <int D>
__device__ __forceinline__ void load_grad_row(const bf16* xrow, GradRow<D>& r) {
  const int g = lane_id() >> 5;
#pragma unroll
  for (int c = 0; c < D / 32; ++c)
#pragma unroll
    for (int u = 0; u < 4; ++u) r.x[c][u] = *reinterpret_cast<const bf16x4*>(xrow + 32 * c + 8 * u + 4 * g);
}

// Apply the F.normalize backward to a gradient tile in the transposed C layout (lane = row,
// value r of column block c = element 32c + crow(r, g)) and store it (see finish_rows in
// tda_bwd.hip; same arithmetic).  xr: the input row (NORM only).
template <int D, bool NORM>
__device__ __forceinline__ void store_grad_rows(const f32x16 (&acc)[D / 32], const GradRow<D>& xr, bf16* grow,
                                                float rinv) {
  constexpr int ND = D / 32;
  const int g = lane_id() >> 5;
  float dot = 0.f;
  f32x4 xh[ND][4];
  if constexpr (NORM) {
#pragma unroll
    for (int c = 0; c < ND; ++c)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          xh[c][u][e] = (float)xr.x[c][u][e] * rinv;
          dot = __builtin_fmaf(xh[c][u][e], acc[c][4 * u + e], dot);
        }
      }
    dot += __shfl_xor(dot, 32);
  }
  const bool clamped = NORM && rinv >= 1.0f / kNormEps;
#pragma unroll
  for (int c = 0; c < ND; ++c)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      float o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = acc[c][4 * u + e];
        if constexpr (NORM) o[e] = clamped ? a * rinv : (a - xh[c][u][e] * dot) * rinv;
        else o[e] = a;
      }
      store4(grow + 32 * c + 8 * u + 4 * g, o[0], o[1], o[2], o[3]);
    }
}

template <int D>
struct BwdWaveLds {
  bf16 a[32 * D];  // K (dq pass) or Q (dkv pass) tile
  bf16 b[32 * D];  // V (dq pass) or dO (dkv pass) tile
  float rows[32];  // key inverse norms (dq) or query inverse norms (dkv)
  float taus[32];  // tau coefficients of the query rows (dkv)
};

// Waves per workgroup of both passes.  The work per item varies with its number of non-zero
// tiles; single-wave workgroups retire independently.
constexpr int kBwdWaves = 1;

// ------------------------------------------------------------------ query-major pass, tiles
// One wave per (branch, query tile) whose pair list did not fit (or with no lists at all): it
// walks the set bits of the branch's bitmask row.  A branch's resident operands (its query
// fragments, dO, one dq accumulator) are half of both branches', which lets two waves share a
// SIMD.
// (branch, head, query tile) of query-major tile-pass item `item`: longest first (query tiles
// from the last); the two branches of a (head, query tile) adjacent.
template <int BR>
__device__ __forceinline__ void dq_item(int64_t item, int BH, int nqt, int& br, int& qt, int& bh) {
  br = BR == 2 ? (int)(item & 1) : 0;
  const int64_t rest = BR == 2 ? item >> 1 : item;
  qt = nqt - 1 - (int)(rest / BH);
  bh = (int)(rest % BH);
}

// The tile pass over one (branch, query tile) item: one wave, W its LDS.
template <int D, int BR, int PK, bool NORM>
__device__ __forceinline__ void bwd_dq_tile(const BwdParams& P, BwdWaveLds<D>& W, int64_t item) {
  constexpr int NT = D / 16, ND = D / 32;
  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int BH = P.B * P.H;
  int br, qt, bh;
  dq_item<BR>(item, BH, P.nqt, br, qt, bh);
  const int b = bh / P.H, h = bh % P.H;
  const int Nq = P.Nq, Nk = P.Nk, qoff = P.qoff;
  const int i = qt * 32 + n32;
  const bool qvalid = i < Nq;
  const int ic = min(i, Nq - 1);
  const int pq = qoff + i;                   // the lane's query position
  const int ktl = kt_last(qt, qoff, P.nkt);  // last key tile the query tile sees
  auto base = [&](int slot) {
    return (const bf16*)P.in[slot] + (int64_t)b * P.s[slot][0] + (int64_t)h * P.s[slot][1];
  };
  const int qslot = br == 0 ? B_Q1 : B_Q2, kslot = br == 0 ? B_K1 : B_K2;

  // row operands, all issued before the first wait: dO and query fragments, the inverse query
  // norm, bitmask words 0..63 of the branch's row (lane w holds word w)
  const int nw = (ktl >> 5) + 1;  // bitmask words covering key tiles 0..ktl
  // the forward's pair list of (branch, head, query tile), when it fit (else the tile path)
  const int64_t lidx = ((int64_t)br * BH + bh) * P.nqt + qt;
  const uint32_t npairs = P.pairs ? P.pairs[pair_lists(BR, BH, P.nqt) * 4 * kPairCap + lidx] : kPairOverflow;
  if (npairs <= (uint32_t)kPairCap) return;  // bwd_dq_pairs handles the lists that fit
  bf16x8 DO[NT], Q[NT];
  {
    const bf16* r = base(B_DO) + (int64_t)ic * P.s[B_DO][2];
    const bf16* rq_ = base(qslot) + (int64_t)ic * P.s[qslot][2];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      DO[t] = *reinterpret_cast<const bf16x8*>(r + 16 * t + 8 * g);
      Q[t] = *reinterpret_cast<const bf16x8*>(rq_ + 16 * t + 8 * g);
    }
  }
  const float rq = NORM ? P.norms[norm_base(P, br == 0 ? N_Q1 : N_Q2, bh) + ic] : 1.f;
  const uint32_t* occrow = P.occ ? P.occ + (((int64_t)br * BH + bh) * P.nqt + qt) * P.occ_w : nullptr;
  const uint32_t lw0 = l < nw ? (occrow ? occrow[l] : 0xffffffffu) : 0u;
  const float ci = tau_coeff(pq, P.inv_d);
  const float tau = (*P.beta) * ci;
  const float pw = P.p;
  float coef = 1.f;
  if constexpr (BR == 2) coef = br == 0 ? 1.f : -clamp01(*P.lam);
  const bool want_l = BR == 2 && br == 1;  // dlambda comes from branch 2 alone
  const bf16* vb = base(B_V);
  const int64_t sv = P.s[B_V][2];
  const bf16* kb = base(kslot);
  const int64_t sk = P.s[kslot][2];
  const float* nk = nullptr;
  if constexpr (NORM) nk = P.norms + norm_base(P, br == 0 ? N_K1 : N_K2, bh);
  float bsum = 0.f, lsum = 0.f;
  unsigned visited = 0, computed = 0;

  f32x16 A[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) A[c] = f32x16{};

  for (int w0 = 0; w0 < nw; w0 += 64) {
    const uint32_t lw = w0 == 0 ? lw0 : (w0 + l < nw) ? (occrow ? occrow[w0 + l] : 0xffffffffu) : 0u;
    for (int w = w0; w < min(nw, w0 + 64); ++w) {
      uint32_t bits = __builtin_amdgcn_readlane(lw, w - w0);
      if (w == (ktl >> 5)) bits &= (ktl & 31) == 31 ? 0xffffffffu : ((2u << (ktl & 31)) - 1u);
      while (bits) {
        const int kt = 32 * w + __builtin_ctz(bits);
        bits &= bits - 1u;
        ++visited;
        const int k0 = 32 * kt;
        dma_tile_b<D>(kb, sk, k0, Nk, W.a);
        dma_tile_b<D>(vb, sv, k0, Nk, W.b);
        if constexpr (NORM) dma_row_vals_b(nk, k0, Nk, W.rows);
        wait_all_loads();
        f32x16 S = f32x16{}, Dp = f32x16{};
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          S = PolBF16::mma(tile_row_frag<D>(W.a, t), Q[t], S);
          Dp = PolBF16::mma(tile_row_frag<D>(W.b, t), DO[t], Dp);
        }
        float rk[16];
        if constexpr (NORM) crow_vals(W.rows, rk);
        f32x16 E;
        bool any = false;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int key = k0 + crow(r, g);
          const bool valid = qvalid && key <= pq && key < Nk;  // rows past Nk read as zeros
          const float sr = NORM ? S[r] * rk[r] : S[r];
          const float x = __builtin_fmaf(sr, rq, -tau);
          const bool pos = valid && x > 0.f;
          const float ds = pos ? coef * dpow_p<PK>(x, pw) * Dp[r] : 0.f;
          bsum += ds;
          lsum = __builtin_fmaf(pos && want_l ? pow_p<PK>(x, pw) : 0.f, Dp[r], lsum);
          any = any || pos;
          E[r] = NORM ? ds * rk[r] : ds;
        }
        if (!occrow && wave_ballot(any) == 0ull) continue;
        ++computed;
        const bf16x8 E0 = PolBF16::pack_c(E, 0), E1 = PolBF16::pack_c(E, 1);
#pragma unroll
        for (int c = 0; c < ND; ++c) {
          A[c] = PolBF16::mma(tile_tr_frag<D>(W.a, 0, c), E0, A[c]);
          A[c] = PolBF16::mma(tile_tr_frag<D>(W.a, 1, c), E1, A[c]);
        }
      }
    }
  }
  if (qvalid) {
    // the query row for the normalize backward, loaded after the tiles (held during them, it
    // would push the wave past the register budget of two waves per SIMD)
    GradRow<D> XR;
    if constexpr (NORM) load_grad_row<D>(base(qslot) + (int64_t)ic * P.s[qslot][2], XR);
    const int gslot = br == 0 ? B_DQ1 : B_DQ2;
    bf16* grow = (bf16*)P.grad[br == 0 ? 0 : 2] + (int64_t)b * P.s[gslot][0] + (int64_t)h * P.s[gslot][1] +
                 (int64_t)i * P.s[gslot][2];
    store_grad_rows<D, NORM>(A, XR, grow, rq);
  }

  const float pb = wave_sum(-ci * bsum);
  const float pl = wave_sum(-lsum);
  if (l == 0) {
    P.ws[2 * lidx + 0] = pb;  // slot of (branch, head, query tile), whichever pass takes it
    P.ws[2 * lidx + 1] = pl;
    if (P.stats) {
      atomicAdd(P.stats + 0, (unsigned long long)visited);
      atomicAdd(P.stats + 1, (unsigned long long)computed);
    }
  }
}

// One wave per workgroup and `per_wave` consecutive items per wave.  With pair lists, the items
// whose list fit belong to bwd_dq_pairs: the wave tests its items' counts in one lane-parallel
// round and runs only the others (per_wave 8: a launch where every list fits costs two waves per
// SIMD); without lists every item runs (per_wave 1).
template <int D, int BR, int PK, bool NORM>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) bwd_dq_fast(BwdParams P, int per_wave) {
  __shared__ __attribute__((aligned(16))) BwdWaveLds<D> W;
  const int l = lane_id();
  const int BH = P.B * P.H;
  const int64_t n = (int64_t)BR * BH * P.nqt, first = (int64_t)blockIdx.x * per_wave;
  bool need = false;
  if (l < per_wave && first + l < n) {
    need = true;
    if (P.pairs) {
      int br, qt, bh;
      dq_item<BR>(first + l, BH, P.nqt, br, qt, bh);
      need = P.pairs[pair_lists(BR, BH, P.nqt) * 4 * kPairCap + ((int64_t)br * BH + bh) * P.nqt + qt] > (uint32_t)kPairCap;
    }
  }
  for (uint64_t m = wave_ballot(need); m; m &= m - 1ull) bwd_dq_tile<D, BR, PK, NORM>(P, W, first + __builtin_ctzll(m));
}

// ------------------------------------------------------------------ query-major pass, pairs
// One wave per (branch, query tile) whose pair list fit.  A list holds a few non-zero weights,
// so the wave works on whole rows, D / 64 elements per lane: the tile's gradient rows that no
// pair names are stored as zeros (16-byte stores), and for each named row i, in increasing
// order, dq_i = sum over its pairs, in list order, of dS k_j (times the key's inverse norm with
// normalisation), dS = coef p x^(p-1) (do_i . v_j) with x the forward's exact value; then the
// normalize backward of the row.  Each pair's dk weight, dS (times rq_i with normalisation),
// goes to the workspace slot of its list entry and to its column-bucket entry for
// bwd_dkv_pairs.  No LDS, no matrix cores: per pair two row loads and one wave-wide dot product.
template <int D>
struct RowVec {
  static constexpr int E = D / 64;  // elements per lane
  float v[E];
};
template <int D>
__device__ __forceinline__ RowVec<D> load_rowvec(const bf16* row) {
  RowVec<D> r;
  const int l = lane_id();
  if constexpr (D == 128) {
    const bf16x2 x = *reinterpret_cast<const bf16x2*>(row + 2 * l);
    r.v[0] = (float)x[0];
    r.v[1] = (float)x[1];
  } else {
    r.v[0] = (float)row[l];
  }
  return r;
}
template <int D>
__device__ __forceinline__ RowVec<D> load_rowvec(const float* row) {
  RowVec<D> r;
  const int l = lane_id();
  if constexpr (D == 128) {
    const float2 x = *reinterpret_cast<const float2*>(row + 2 * l);
    r.v[0] = x.x;
    r.v[1] = x.y;
  } else {
    r.v[0] = row[l];
  }
  return r;
}
// The lane's D/64 elements of a row as loaded (bf16: the bits, element 2l in the low half for
// D = 128, one register per row while loads are in flight; fp32: the values).
template <int D, class T>
struct RowRaw;
template <int D>
struct RowRaw<D, bf16> {
  uint32_t u;
};
template <int D>
struct RowRaw<D, float> {
  float v[D / 64];
};
template <int D>
__device__ __forceinline__ RowRaw<D, bf16> load_rowraw(const bf16* row) {
  const int l = lane_id();
  if constexpr (D == 128) return RowRaw<D, bf16>{*reinterpret_cast<const uint32_t*>(row + 2 * l)};
  else return RowRaw<D, bf16>{(uint32_t)*reinterpret_cast<const uint16_t*>(row + l)};
}
template <int D>
__device__ __forceinline__ RowRaw<D, float> load_rowraw(const float* row) {
  RowRaw<D, float> r;
  const RowVec<D> v = load_rowvec<D>(row);
#pragma unroll
  for (int e = 0; e < D / 64; ++e) r.v[e] = v.v[e];
  return r;
}
template <int D>
__device__ __forceinline__ RowVec<D> unpack(RowRaw<D, bf16> r) {
  RowVec<D> v;
  v.v[0] = __uint_as_float(r.u << 16);
  if constexpr (D == 128) v.v[1] = __uint_as_float(r.u & 0xffff0000u);
  return v;
}
template <int D>
__device__ __forceinline__ RowVec<D> unpack(RowRaw<D, float> r) {
  RowVec<D> v;
#pragma unroll
  for (int e = 0; e < D / 64; ++e) v.v[e] = r.v[e];
  return v;
}
template <int D>
__device__ __forceinline__ void store_rowvec(bf16* row, const RowVec<D>& r) {
  const int l = lane_id();
  if constexpr (D == 128)
    __builtin_nontemporal_store(__builtin_bit_cast(uint32_t, bf16x2{(bf16)r.v[0], (bf16)r.v[1]}),
                                reinterpret_cast<uint32_t*>(row + 2 * l));
  else row[l] = (bf16)r.v[0];
}
template <int D>
__device__ __forceinline__ void store_rowvec(float* row, const RowVec<D>& r) {
  const int l = lane_id();
  if constexpr (D == 128)
    __builtin_nontemporal_store(__builtin_bit_cast(uint64_t, float2{r.v[0], r.v[1]}),
                                reinterpret_cast<uint64_t*>(row + 2 * l));
  else __builtin_nontemporal_store(r.v[0], row + l);
}
template <int D>
__device__ __forceinline__ float row_dot(const RowVec<D>& a, const RowVec<D>& b) {
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < RowVec<D>::E; ++e) s = __builtin_fmaf(a.v[e], b.v[e], s);
  return wave_sum(s);
}
// The F.normalize backward of one row (see store_grad_rows): x the input row, rinv its inverse norm.
template <int D, bool NORM>
__device__ __forceinline__ RowVec<D> normalize_back(const RowVec<D>& g, const RowVec<D>& x, float rinv) {
  if constexpr (!NORM) return g;
  RowVec<D> xh, o;
#pragma unroll
  for (int e = 0; e < RowVec<D>::E; ++e) xh.v[e] = x.v[e] * rinv;
  const float dot = row_dot<D>(xh, g);
  const bool clamped = rinv >= 1.0f / kNormEps;
#pragma unroll
  for (int e = 0; e < RowVec<D>::E; ++e) o.v[e] = clamped ? g.v[e] * rinv : (g.v[e] - xh.v[e] * dot) * rinv;
  return o;
}
// Zero rows 0..nrows-1 of a 32-row tile except those in `keep` (16 bytes per lane and store).
template <int D, class T>
__device__ __forceinline__ void zero_rows(T* tile0, int64_t st, int nrows, uint32_t keep) {
  constexpr int EPC = 16 / sizeof(T), CH = D / EPC, RPI = 64 / CH;  // elements per chunk, chunks per row
  const int l = lane_id();
#pragma unroll
  for (int u = 0; u < 32 / RPI; ++u) {
    const int r = u * RPI + l / CH;
    if (r < nrows && !((keep >> r) & 1u))  // streaming stores: nothing reads them soon
      __builtin_nontemporal_store(u32x4{0u, 0u, 0u, 0u},
                                  reinterpret_cast<u32x4*>(tile0 + (int64_t)r * st + EPC * (l % CH)));
  }
}

// Pairs whose row loads the pair passes keep in flight together: the query-major pass 4 (64
// VGPRs, eight waves per SIMD: 23.6 us against 24.8 with 8 at B4 H16 N4096 d128), the
// key-major pass 8.
constexpr int kRowBatch = 4;
constexpr int kColBatch = 8;

// A pair list sorted by query row, then list order: lane s < n holds the entry of rank s, and
// e = its index in the list; lanes past n hold their own slot (a permutation of the lanes, so
// the forward permutes below write every lane once).
struct SortedPairs {
  int key, row, e;
  float x;
};
__device__ __forceinline__ SortedPairs sort_pairs(const PairLanes& PL, uint32_t n) {
  const int l = lane_id();
  int rank = l;
  if ((uint32_t)l < n) {
    rank = 0;
    for (uint32_t f = 0; f < n; ++f) {
      const int rf = __builtin_amdgcn_readlane(PL.row, (int)f);
      rank += rf < PL.row || (rf == PL.row && (int)f < l) ? 1 : 0;
    }
  }
  SortedPairs S;
  S.key = __builtin_amdgcn_ds_permute(4 * rank, PL.key);
  S.row = __builtin_amdgcn_ds_permute(4 * rank, PL.row);
  S.e = __builtin_amdgcn_ds_permute(4 * rank, l);
  S.x = __builtin_bit_cast(float, __builtin_amdgcn_ds_permute(4 * rank, __builtin_bit_cast(int, PL.x)));
  return S;
}

template <int D, int BR, int PK, bool NORM, class T = bf16>
__global__ void __launch_bounds__(64) bwd_dq_pairs(BwdParams P) {
  const int l = lane_id();
  const int BH = P.B * P.H;
  // (query tile, head, branch), query tiles ascending: the early rows' thresholds are the
  // lowest, their lists the longest
  const int64_t item = blockIdx.x;
  if (item >= (int64_t)BR * BH * P.nqt) return;
  const int br = BR == 2 ? (int)(item & 1) : 0;
  const int64_t rest = BR == 2 ? item >> 1 : item;
  const int qt = (int)(rest / BH);
  const int bh = (int)(rest % BH);
  const int b = bh / P.H, h = bh % P.H;
  const int64_t lidx = ((int64_t)br * BH + bh) * P.nqt + qt;
  // the count and every entry slot at once (slots past the count are never used)
  const PairLanes PL = load_pairs(P.pairs + lidx * (4 * kPairCap), (uint32_t)kPairCap);
  const uint32_t npairs = P.pairs[pair_lists(BR, BH, P.nqt) * 4 * kPairCap + lidx];
  if (P.dkvq && item == 0 && l == 0) P.dkvq[0] = 0u;  // the key-major pair pass fills it later
  if (npairs > (uint32_t)kPairCap) return;  // bwd_dq_fast walks the tiles

  auto base = [&](int slot) {
    return (const T*)P.in[slot] + (int64_t)b * P.s[slot][0] + (int64_t)h * P.s[slot][1];
  };
  const int qslot = br == 0 ? B_Q1 : B_Q2, kslot = br == 0 ? B_K1 : B_K2, gslot = br == 0 ? B_DQ1 : B_DQ2;
  const int64_t sq = P.s[qslot][2], sk = P.s[kslot][2], sv = P.s[B_V][2], sdo = P.s[B_DO][2], sg = P.s[gslot][2];
  const T* qb = base(qslot);
  const T* kb = base(kslot);
  const T* vb = base(B_V);
  const T* dob = base(B_DO);
  T* gb = (T*)P.grad[br == 0 ? 0 : 2] + (int64_t)b * P.s[gslot][0] + (int64_t)h * P.s[gslot][1];
  const float* nq = NORM ? P.norms + norm_base(P, br == 0 ? N_Q1 : N_Q2, bh) : nullptr;
  const float* nk = NORM ? P.norms + norm_base(P, br == 0 ? N_K1 : N_K2, bh) : nullptr;
  const float pw = P.p;
  float coef = 1.f;
  if constexpr (BR == 2) coef = br == 0 ? 1.f : -clamp01(*P.lam);
  const bool want_l = BR == 2 && br == 1;  // dlambda comes from branch 2 alone

  uint32_t used = 0u;  // rows (within the tile) some pair names
  unsigned tiles = 0;
  int last_kt = -1;
  for (uint32_t e = 0; e < npairs; ++e) {
    used |= 1u << __builtin_amdgcn_readlane(PL.row, (int)e);
    const int kt = __builtin_amdgcn_readlane(PL.key, (int)e) >> 5;
    tiles += kt != last_kt ? 1u : 0u;  // pairs of one key tile are consecutive
    last_kt = kt;
  }
  const int q0 = 32 * qt;
  if (!P.grads_zeroed) zero_rows<D>(gb + (int64_t)q0 * sg, sg, min(32, P.Nq - q0), used);

  // The pairs sorted by query row, then list order: lane s gets the pair of rank s (lanes past
  // the count keep their own slot, so the ranks form a permutation of the lanes).
  const SortedPairs SP = sort_pairs(PL, npairs);

  // Rows in increasing order, each row's pairs in list order; the loads of kRowBatch pairs at a
  // time are in flight together, a row is finished when the next pair names another.
  float pb = 0.f, pl = 0.f;  // dbeta, dlambda partials (the same in every lane)
  float wks = 0.f;           // lane s: the dk weight of sorted pair s
  int cur = -1;              // row being accumulated
  RowVec<D> acc = {}, cur_x = {};
  float cur_r = 1.f;
  auto finish = [&]() {
    if (cur >= 0) store_rowvec<D>(gb + (int64_t)(q0 + cur) * sg, normalize_back<D, NORM>(acc, cur_x, cur_r));
  };
  for (uint32_t s0 = 0; s0 < npairs; s0 += kRowBatch) {
    int il[kRowBatch], jj[kRowBatch];
    float rq[kRowBatch], rk[kRowBatch];
    RowRaw<D, T> dor[kRowBatch], qr[kRowBatch], kr[kRowBatch], vr[kRowBatch];
#pragma unroll
    for (int u = 0; u < kRowBatch; ++u) {
      const int s = (int)s0 + u;
      if ((uint32_t)s >= npairs) continue;
      il[u] = __builtin_amdgcn_readlane(SP.row, s);
      jj[u] = __builtin_amdgcn_readlane(SP.key, s);
      const int i = q0 + il[u];
      dor[u] = load_rowraw<D>(dob + (int64_t)i * sdo);
      kr[u] = load_rowraw<D>(kb + (int64_t)jj[u] * sk);
      vr[u] = load_rowraw<D>(vb + (int64_t)jj[u] * sv);
      qr[u] = RowRaw<D, T>{};
      rq[u] = rk[u] = 1.f;
      if constexpr (NORM) {
        qr[u] = load_rowraw<D>(qb + (int64_t)i * sq);
        rq[u] = nq[i];
        rk[u] = nk[jj[u]];
      }
    }
#pragma unroll
    for (int u = 0; u < kRowBatch; ++u) {
      const int s = (int)s0 + u;
      if ((uint32_t)s >= npairs) continue;
      if (il[u] != cur) {
        finish();
        acc = RowVec<D>{};
        cur = il[u];
        cur_x = unpack<D>(qr[u]);
        cur_r = rq[u];
      }
      const float xx = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, SP.x), s));
      const float ci = tau_coeff(P.qoff + q0 + il[u], P.inv_d);
      const float dp = row_dot<D>(unpack<D>(dor[u]), unpack<D>(vr[u]));
      const float ds = coef * dpow_p<PK>(xx, pw) * dp;
      pb = __builtin_fmaf(-ci, ds, pb);
      if (want_l) pl = __builtin_fmaf(-pow_p<PK>(xx, pw), dp, pl);
      const float w = NORM ? ds * rk[u] : ds;
      wks = l == s ? (NORM ? ds * rq[u] : ds) : wks;
      const RowVec<D> kv = unpack<D>(kr[u]);
#pragma unroll
      for (int c = 0; c < RowVec<D>::E; ++c) acc.v[c] = __builtin_fmaf(w, kv.v[c], acc.v[c]);
    }
  }
  finish();
  // back to list order: lane s sends its weight to the lane of its list entry
  const float wkl = __builtin_bit_cast(float, __builtin_amdgcn_ds_permute(4 * SP.e, __builtin_bit_cast(int, wks)));
  if ((uint32_t)l < npairs) {
    P.pws[lidx * kPairCap + l] = wkl;
    if (P.colbuf && PL.slot < (uint32_t)kColCap)  // the dk weight of the pair's column-bucket entry
      P.colbuf[(((int64_t)bh * P.nkt + (PL.key >> 5)) * kColCap + PL.slot) * 4 + 3] = __builtin_bit_cast(uint32_t, wkl);
  }
  if (l == 0) {
    P.ws[2 * lidx + 0] = pb;  // slot of (branch, head, query tile), whichever pass takes it
    P.ws[2 * lidx + 1] = pl;
    if (P.stats) {
      atomicAdd(P.stats + 0, (unsigned long long)tiles);
      atomicAdd(P.stats + 1, (unsigned long long)tiles);
    }
  }
}

// ------------------------------------------------------------------ key-major pass, pairs
// Whether the bitmask column of key tile kt (query tiles qtf.., every branch) has a query tile
// whose pair list did not fit: the key tile then goes to the tile pass, else to the pair pass.
// Both key-major passes decide with this test.
template <int BR>
__device__ __forceinline__ bool column_overflows(const BwdParams& P, int bh, int kt, int qtf) {
  const int BH = P.B * P.H, l = lane_id();
  const uint32_t* counts = P.pairs + pair_lists(BR, BH, P.nqt) * 4 * kPairCap;
  bool ovf = false;
  for (int q0c = qtf; q0c < P.nqt; q0c += 64) {
    const int qt = q0c + l;
    const bool in = qt < P.nqt;
    uint32_t w[BR], c[BR];
#pragma unroll
    for (int br = 0; br < BR; ++br) {  // every load of the chunk before the first use
      const int64_t row = ((int64_t)br * BH + bh) * P.nqt + (in ? qt : P.nqt - 1);
      w[br] = P.occ[row * P.occ_w + (kt >> 5)];
      c[br] = counts[row];
    }
#pragma unroll
    for (int br = 0; br < BR; ++br) ovf = ovf || (in && ((w[br] >> (kt & 31)) & 1u) && c[br] > (uint32_t)kPairCap);
  }
  return wave_ballot(ovf) != 0ull;
}

// LDS slots of the key-major pair pass: pairs of one column gathered at once.
constexpr int kColPairs = 64;
static_assert(kColCap == kColPairs && kColCap == 64, "a column bucket: one entry per lane, as many as the slots");
// List-load rounds of one walk step of the key-major pair pass (two lists per round).
constexpr int kWalkRounds = 4;

// One entry of a column's pair list as seen by one lane of the key-major pair pass.
struct ColEntry {
  bool valid;  // the lane holds an entry
  int br;      // branch of the lane's list
  int key;     // key index j
  int i;       // query row
  float x;     // exact forward value
  float wk;    // dk weight from the query-major pair pass
};

// One wave per key tile whose column has only lists that fit.  Its pairs come from the column's
// bucket when the forward filled one with all of them (every entry with its dk weight: one round
// of loads), else it walks the column's lists (both branches, query-tile chunks of 64, two lists
// per step: lanes 0-31 and 32-63) and keeps the pairs with a key in this tile.  For each key row j that some pair names, in increasing
// order, whole-row vector work over its pairs:
//   dv_j  += coef A_ij do_i          A_ij = x^p (x the forward's exact value)
//   dk_j  += w_ij q_i                w_ij = coef p x^(p-1) (do_i . v_j) (times rq_i with
//                                    normalisation), stored by the query-major pair pass
// then the normalize backward of dk_j; the tile's other gradient rows are stored as zeros.
// Pairs of a row meet its accumulators in walk order (chunk, branch, query tile, list entry),
// or, from a bucket, in the order (branch, query row).
// Up to kColPairs pairs are gathered into LDS slots in one walk; a column with more walks its
// lists once per named row.  No matrix cores and no V: per pair two row loads.
template <int D, int BR, int PK, bool NORM, class T = bf16>
__global__ void __launch_bounds__(64) bwd_dkv_pairs(BwdParams P) {
  __shared__ int ps_i[kColPairs];    // query row, branch in bit 31
  __shared__ int ps_jl[kColPairs];   // key row within the tile
  __shared__ float ps_x[kColPairs];  // exact forward value x
  __shared__ float ps_w[kColPairs];  // dk weight

  const int l = lane_id();
  const int BH = P.B * P.H;
  const int64_t item = blockIdx.x;  // (key tile, head), in the order of bwd_dkv_fast
  if (item >= (int64_t)BH * P.nkt) return;
  const int kt = (int)(item / BH), bh = (int)(item % BH);
  const int b = bh / P.H, h = bh % P.H;
  const int qtf = qt_first(kt, P.qoff);

  auto base = [&](int slot) {
    return (const T*)P.in[slot] + (int64_t)b * P.s[slot][0] + (int64_t)h * P.s[slot][1];
  };
  auto gbase = [&](int slot, int gi) {
    return (T*)P.grad[gi] + (int64_t)b * P.s[slot][0] + (int64_t)h * P.s[slot][1];
  };
  const uint32_t* counts = P.pairs + pair_lists(BR, BH, P.nqt) * 4 * kPairCap;
  const float pw = P.p;
  float lam = 0.f;
  if constexpr (BR == 2) lam = clamp01(*P.lam);

  // Walk the column's lists in the order (query-tile chunk of 64, branch, query tile): the
  // bitmask bits and counts of 128 query tiles per load round, then 2 kWalkRounds lists per
  // step, all loaded before the first is used (lanes 0-31 and 32-63 take one list each per
  // round); body(entry) once per round.  Returns false, before any body call of that chunk pair, when a
  // list of the column did not fit (the same test as column_overflows: the tile pass takes the
  // key tile); the caller has then written nothing.
  auto walk = [&](auto&& body) -> bool {
    for (int q0c = qtf; q0c < P.nqt; q0c += 128) {
      uint64_t mask[2 * BR];  // [chunk * BR + branch]
      uint32_t cnt_l[2 * BR];
      bool ovf = false;
#pragma unroll
      for (int k = 0; k < 2 * BR; ++k) {
        const int c = k / BR, br = k % BR;
        const int qtl = q0c + 64 * c + l;
        const bool in = qtl < P.nqt;
        const int64_t row = ((int64_t)br * BH + bh) * P.nqt + (in ? qtl : P.nqt - 1);
        const uint32_t w = P.occ[row * P.occ_w + (kt >> 5)];
        cnt_l[k] = counts[row];
        const bool has = in && ((w >> (kt & 31)) & 1u);
        ovf = ovf || (has && cnt_l[k] > (uint32_t)kPairCap);
        mask[k] = wave_ballot(has);
      }
      if (wave_ballot(ovf) != 0ull) return false;
      while (true) {
        int ix[2 * kWalkRounds], sx[2 * kWalkRounds];
        uint32_t cx[2 * kWalkRounds];
#pragma unroll
        for (int u = 0; u < 2 * kWalkRounds; ++u) {  // next lists
          ix[u] = -1;
          sx[u] = 0;
          cx[u] = 0u;
          bool found = false;
#pragma unroll
          for (int k = 0; k < 2 * BR; ++k)
            if (!found && mask[k]) {
              found = true;
              ix[u] = k;
              sx[u] = __builtin_ctzll(mask[k]);
              mask[k] &= mask[k] - 1ull;
              cx[u] = (uint32_t)__builtin_amdgcn_readlane((int)cnt_l[k], sx[u]);
            }
        }
        if (ix[0] < 0) break;
        u32x4 ent[kWalkRounds];
        float wk[kWalkRounds];
        int brl[kWalkRounds], qtl[kWalkRounds];
        bool valid[kWalkRounds];
#pragma unroll
        for (int r = 0; r < kWalkRounds; ++r) {
          const int idx = l < 32 ? ix[2 * r] : ix[2 * r + 1];
          const int sel = l < 32 ? sx[2 * r] : sx[2 * r + 1];
          const uint32_t cnt = l < 32 ? cx[2 * r] : cx[2 * r + 1];
          const int e = l & 31;
          brl[r] = idx >= 0 ? idx % BR : 0;
          qtl[r] = q0c + 64 * (idx >= 0 ? idx / BR : 0) + sel;
          valid[r] = idx >= 0 && (uint32_t)e < cnt;
          const int64_t lidx = ((int64_t)brl[r] * BH + bh) * P.nqt + qtl[r];
          ent[r] = u32x4{0u, 0u, 0u, 0u};
          wk[r] = 0.f;
          if (valid[r]) {
            ent[r] = *reinterpret_cast<const u32x4*>(P.pairs + lidx * (4 * kPairCap) + 4 * e);
            wk[r] = P.pws[lidx * kPairCap + e];
          }
        }
#pragma unroll
        for (int r = 0; r < kWalkRounds; ++r) {
          if (ix[2 * r] < 0) break;
          // x through a bit cast of the whole vector (see load_pairs)
          const f32x4 ef = __builtin_bit_cast(f32x4, ent[r]);
          ColEntry c;
          c.valid = valid[r];
          c.br = brl[r];
          c.key = (int)ent[r][0];
          c.i = 32 * qtl[r] + (int)ent[r][1];
          c.x = ef[2];
          c.wk = wk[r];
          body(c);
        }
      }
    }
    return true;
  };

  uint32_t np = 0;
  unsigned visited = 0;
  uint32_t used[BR];  // key rows named by a pair, per branch
#pragma unroll
  for (int br = 0; br < BR; ++br) used[br] = 0u;
  // lane s < np: pair s {query row | branch << 31, key row in the tile, x, dk weight}, and the
  // second key of the order the pairs are taken in (after the key row)
  int pi_l = 0, pjl_l = 0;
  float px_l = 0.f, pw_l = 0.f;
  uint32_t k2_l = (uint32_t)l;

  // ---- the column's bucket, when the forward filled it with every pair of the column (one
  // round of loads; the pairs are then taken in the order (key row, branch, query row))
  bool from_bucket = false;
  if (P.colcnt) {
    const int64_t col = (int64_t)bh * P.nkt + kt;
    const uint32_t cc = (uint32_t)__builtin_amdgcn_readfirstlane((int)P.colcnt[col]);
    const u32x4 be = *reinterpret_cast<const u32x4*>(P.colbuf + (col * kColCap + l) * 4);
    if (!(cc & kColTaint) && cc <= (uint32_t)kColCap) {
      from_bucket = true;
      np = cc;
      const bool in = (uint32_t)l < np;
      const f32x4 bf = __builtin_bit_cast(f32x4, be);  // x, w: a bit cast of the whole vector (see load_pairs)
      pi_l = in ? (int)be[0] : 0;
      pjl_l = in ? (int)be[1] : 0;
      px_l = in ? bf[2] : 0.f;
      pw_l = in ? bf[3] : 0.f;
      k2_l = (uint32_t)pi_l;
#pragma unroll
      for (int br = 0; br < BR; ++br)
        used[br] = wave_or(in && (int)(((uint32_t)pi_l >> 31) & 1u) == br ? 1u << pjl_l : 0u);
      if (P.stats) {  // the counters as the walk counts them: (branch, query tile) lists in the column
        const int lk = (int)(((uint32_t)pi_l >> 31) << 30) | ((pi_l & 0x7fffffff) >> 5);
        bool dup = false;
        for (int f = 0; f < (int)np; ++f) dup = dup || (f < l && __builtin_amdgcn_readlane(lk, f) == lk);
        visited = (unsigned)__builtin_popcountll(wave_ballot(in && !dup));
      }
    }
  }

  // ---- else the first walk: rows named, pairs into the slots while they fit
  const bool fits = from_bucket || walk([&](const ColEntry& c) {
    const bool match = c.valid && (c.key >> 5) == kt;
    const uint64_t mm = wave_ballot(match);
    visited += ((mm & 0xffffffffull) ? 1u : 0u) + ((mm >> 32) ? 1u : 0u);
    const uint32_t slot = np + __builtin_amdgcn_mbcnt_hi((uint32_t)(mm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mm, 0u));
    if (match && slot < (uint32_t)kColPairs) {
      ps_i[slot] = c.i | (c.br ? (int)0x80000000u : 0);
      ps_jl[slot] = c.key & 31;
      ps_x[slot] = c.x;
      ps_w[slot] = c.wk;
    }
#pragma unroll
    for (int br = 0; br < BR; ++br) {
      uint32_t ub = match && c.br == br ? 1u << (c.key & 31) : 0u;
      ub = wave_or(ub);
      used[br] |= ub;
    }
    np += (uint32_t)__builtin_popcountll(mm);
  });
  if (!fits) {  // bwd_dkv_fast takes the key tile
    if (P.dkvq && l == 0) P.dkvq[1 + atomicAdd(P.dkvq, 1u)] = (uint32_t)item;
    return;
  }
  wave_lds_sync();  // slots written by other lanes
  const bool slotted = np <= (uint32_t)kColPairs;

  // ---- rows: zeros for the rows no pair names, then each named key row
  const int nrows = min(32, P.Nk - 32 * kt);
  const uint32_t uall = BR == 2 ? used[0] | used[BR - 1] : used[0];
  T* dvb = gbase(B_DV, 4);
  const int64_t sdv = P.s[B_DV][2];
  if (!P.grads_zeroed) {
    zero_rows<D>(dvb + (int64_t)(32 * kt) * sdv, sdv, nrows, uall);
#pragma unroll
    for (int br = 0; br < BR; ++br) {
      const int gslot = br == 0 ? B_DK1 : B_DK2;
      zero_rows<D>(gbase(gslot, br == 0 ? 1 : 3) + (int64_t)(32 * kt) * P.s[gslot][2], P.s[gslot][2], nrows, used[br]);
    }
  }
  const T* dob = base(B_DO);
  const int64_t sdo = P.s[B_DO][2];
  // key row jl's finished rows: dv, and dk of each branch whose pairs name it (the others were
  // stored as zeros above)
  auto store_key_row = [&](int jl, const RowVec<D>& av, const RowVec<D>(&ak)[BR], const RowVec<D>(&kx)[BR],
                           const float(&rk)[BR]) {
    const int j = 32 * kt + jl;
    store_rowvec<D>(dvb + (int64_t)j * sdv, av);
#pragma unroll
    for (int br = 0; br < BR; ++br) {
      if (!((used[br] >> jl) & 1u)) continue;
      const int gslot = br == 0 ? B_DK1 : B_DK2;
      store_rowvec<D>(gbase(gslot, br == 0 ? 1 : 3) + (int64_t)j * P.s[gslot][2],
                      normalize_back<D, NORM>(ak[br], kx[br], rk[br]));
    }
  };
  // the same, packed (rows zero, norms 1 where not needed)
  auto load_key_raw = [&](int jl, RowRaw<D, T>(&kx)[BR], float(&rk)[BR]) {
    const int j = 32 * kt + jl;
#pragma unroll
    for (int br = 0; br < BR; ++br) {
      kx[br] = RowRaw<D, T>{};
      rk[br] = 1.f;
      if constexpr (NORM)
        if ((used[br] >> jl) & 1u) {
          const int kslot = br == 0 ? B_K1 : B_K2;
          kx[br] = load_rowraw<D>(base(kslot) + (int64_t)j * P.s[kslot][2]);
          rk[br] = P.norms[norm_base(P, br == 0 ? N_K1 : N_K2, bh) + j];
        }
    }
  };
  // the key rows and inverse norms of key row jl for the normalize backward
  auto load_key_rows = [&](int jl, RowVec<D>(&kx)[BR], float(&rk)[BR]) {
    const int j = 32 * kt + jl;
#pragma unroll
    for (int br = 0; br < BR; ++br) {
      kx[br] = RowVec<D>{};
      rk[br] = 1.f;
      if constexpr (NORM)
        if ((used[br] >> jl) & 1u) {
          const int kslot = br == 0 ? B_K1 : B_K2;
          kx[br] = load_rowvec<D>(base(kslot) + (int64_t)j * P.s[kslot][2]);
          rk[br] = P.norms[norm_base(P, br == 0 ? N_K1 : N_K2, bh) + j];
        }
    }
  };

  if (slotted) {
    // The pairs sorted by key row, then the second key (walk: slot order; bucket: branch and
    // query row): lane s gets the pair of rank s (lanes past np keep their own slot).  Then the
    // pairs in that order, the loads of kColBatch at a time in flight together; a key row is
    // finished when the next pair names another.
    if (!from_bucket) {
      const int sl = (uint32_t)l < np ? l : 0;
      pi_l = ps_i[sl];
      pjl_l = ps_jl[sl];
      px_l = ps_x[sl];
      pw_l = ps_w[sl];
    }
    int rank = l;
    if ((uint32_t)l < np) {
      rank = 0;
      for (uint32_t f = 0; f < np; ++f) {
        const int jf = __builtin_amdgcn_readlane(pjl_l, (int)f);
        const uint32_t kf = (uint32_t)__builtin_amdgcn_readlane((int)k2_l, (int)f);
        rank += jf < pjl_l || (jf == pjl_l && kf < k2_l) ? 1 : 0;
      }
    }
    const int s_i = __builtin_amdgcn_ds_permute(4 * rank, pi_l);
    const int s_jl = __builtin_amdgcn_ds_permute(4 * rank, pjl_l);
    const int s_x = __builtin_amdgcn_ds_permute(4 * rank, __builtin_bit_cast(int, px_l));
    const int s_w = __builtin_amdgcn_ds_permute(4 * rank, __builtin_bit_cast(int, pw_l));
    int cur = -1;
    RowVec<D> av = {}, ak[BR], kx[BR];
    float rk[BR];
#pragma unroll
    for (int br = 0; br < BR; ++br) {
      ak[br] = kx[br] = RowVec<D>{};
      rk[br] = 1.f;
    }
    for (uint32_t s0 = 0; s0 < np; s0 += kColBatch) {
      int jl[kColBatch], ibr[kColBatch];
      RowRaw<D, T> dor[kColBatch], qr[kColBatch], kxu[kColBatch][BR];
      float rku[kColBatch][BR];
#pragma unroll
      for (int u = 0; u < kColBatch; ++u) {
        const int s = (int)s0 + u;
        ibr[u] = 0;
        if ((uint32_t)s >= np) continue;
        jl[u] = __builtin_amdgcn_readlane(s_jl, s);
        const int pi = __builtin_amdgcn_readlane(s_i, s);
        const int i = pi & 0x7fffffff;
        ibr[u] = (pi >> 31) & 1;
        const int qslot = ibr[u] ? B_Q2 : B_Q1;
        dor[u] = load_rowraw<D>(dob + (int64_t)i * sdo);
        qr[u] = load_rowraw<D>(base(qslot) + (int64_t)i * P.s[qslot][2]);
        load_key_raw(jl[u], kxu[u], rku[u]);
      }
#pragma unroll
      for (int u = 0; u < kColBatch; ++u) {
        const int s = (int)s0 + u;
        if ((uint32_t)s >= np) continue;
        if (jl[u] != cur) {
          if (cur >= 0) store_key_row(cur, av, ak, kx, rk);
          cur = jl[u];
          av = RowVec<D>{};
#pragma unroll
          for (int br = 0; br < BR; ++br) {
            ak[br] = RowVec<D>{};
            kx[br] = unpack<D>(kxu[u][br]);
            rk[br] = rku[u][br];
          }
        }
        const float x = __builtin_bit_cast(float, __builtin_amdgcn_readlane(s_x, s));
        const float wk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(s_w, s));
        const float wa = (ibr[u] ? -lam : 1.f) * pow_p<PK>(x, pw);
        const RowVec<D> dv_ = unpack<D>(dor[u]), qv = unpack<D>(qr[u]);
#pragma unroll
        for (int c = 0; c < RowVec<D>::E; ++c) av.v[c] = __builtin_fmaf(wa, dv_.v[c], av.v[c]);
#pragma unroll
        for (int br = 0; br < BR; ++br)
          if (ibr[u] == br)
#pragma unroll
            for (int c = 0; c < RowVec<D>::E; ++c) ak[br].v[c] = __builtin_fmaf(wk, qv.v[c], ak[br].v[c]);
      }
    }
    if (cur >= 0) store_key_row(cur, av, ak, kx, rk);
  } else {
    // more pairs than slots: each named key row walks the lists for its own pairs (lane order
    // within a step), up to four row pairs in flight
    for (uint32_t um = uall; um; um &= um - 1u) {
      const int jl = __builtin_ctz(um), j = 32 * kt + jl;
      RowVec<D> kx[BR];
      float rk[BR];
      load_key_rows(jl, kx, rk);
      RowVec<D> av = {}, ak[BR];
#pragma unroll
      for (int br = 0; br < BR; ++br) ak[br] = RowVec<D>{};
      walk([&](const ColEntry& c) {
        uint64_t pm = wave_ballot(c.valid && c.key == j);
        while (pm) {
          int e[4], ibr[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            e[u] = pm ? __builtin_ctzll(pm) : -1;
            if (pm) pm &= pm - 1ull;
          }
          RowVec<D> dor[4], qr[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            ibr[u] = 0;
            if (e[u] < 0) continue;
            const int i = __builtin_amdgcn_readlane(c.i, e[u]);
            ibr[u] = __builtin_amdgcn_readlane(c.br, e[u]);
            const int qslot = ibr[u] ? B_Q2 : B_Q1;
            dor[u] = load_rowvec<D>(dob + (int64_t)i * sdo);
            qr[u] = load_rowvec<D>(base(qslot) + (int64_t)i * P.s[qslot][2]);
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            if (e[u] < 0) continue;
            const float x = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, c.x), e[u]));
            const float wk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, c.wk), e[u]));
            const float wa = (ibr[u] ? -lam : 1.f) * pow_p<PK>(x, pw);
#pragma unroll
            for (int cc = 0; cc < RowVec<D>::E; ++cc) av.v[cc] = __builtin_fmaf(wa, dor[u].v[cc], av.v[cc]);
#pragma unroll
            for (int br = 0; br < BR; ++br)
              if (ibr[u] == br)
#pragma unroll
                for (int cc = 0; cc < RowVec<D>::E; ++cc) ak[br].v[cc] = __builtin_fmaf(wk, qr[u].v[cc], ak[br].v[cc]);
          }
        }
      });
      store_key_row(jl, av, ak, kx, rk);
    }
  }
  if (P.stats && l == 0) {
    atomicAdd(P.stats + 0, (unsigned long long)visited);
    atomicAdd(P.stats + 1, (unsigned long long)visited);
  }
}

// ------------------------------------------------------------------ key-major pass
// The tile pass over one key tile (item = (key tile, head)): one wave, W its LDS.
template <int D, int BR, int PK, bool NORM>
__device__ __forceinline__ void bwd_dkv_tile(const BwdParams& P, BwdWaveLds<D>& W, int64_t item) {
  constexpr int NT = D / 16, ND = D / 32;
  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int BH = P.B * P.H;
  const int kt = (int)(item / BH);
  const int bh = (int)(item % BH);
  const int b = bh / P.H, h = bh % P.H;
  const int Nq = P.Nq, Nk = P.Nk, qoff = P.qoff;
  const int j = kt * 32 + n32;
  const bool kvalid = j < Nk;
  const int jc = min(j, Nk - 1);
  const int qtf = qt_first(kt, qoff);  // first query tile that sees the key tile
  auto base = [&](int slot) {
    return (const bf16*)P.in[slot] + (int64_t)b * P.s[slot][0] + (int64_t)h * P.s[slot][1];
  };

  bf16x8 V[NT];
  {
    const bf16* r = base(B_V) + (int64_t)jc * P.s[B_V][2];
#pragma unroll
    for (int t = 0; t < NT; ++t) V[t] = *reinterpret_cast<const bf16x8*>(r + 16 * t + 8 * g);
  }
  const float beta = *P.beta;
  const float pw = P.p;
  float lam = 0.f;
  if constexpr (BR == 2) lam = clamp01(*P.lam);
  const bf16* dob = base(B_DO);
  const int64_t sdo = P.s[B_DO][2];
  f32x16 AV[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) AV[c] = f32x16{};
  unsigned visited = 0, computed = 0;

  // Both branches' row operands, issued with V so that one memory round trip covers them:
  // inverse key norms, and the bitmask column bits of query tiles qtf .. qtf+63 (lane q holds
  // tile qtf + q).  The key fragments are loaded by the tile path, which alone needs them.
  float RK[BR];
  bool HAS[BR];
#pragma unroll
  for (int br = 0; br < BR; ++br) {
    RK[br] = NORM ? P.norms[norm_base(P, br == 0 ? N_K1 : N_K2, bh) + jc] : 1.f;
    const uint32_t* occcol = P.occ ? P.occ + ((int64_t)br * BH + bh) * P.nqt * P.occ_w + (kt >> 5) : nullptr;
    const int qtl = qtf + l;
    HAS[br] = qtl < P.nqt && (!occcol || ((occcol[(int64_t)qtl * P.occ_w] >> (kt & 31)) & 1u));
  }

#pragma unroll
  for (int br = 0; br < BR; ++br) {
    const int qslot = br == 0 ? B_Q1 : B_Q2, kslot = br == 0 ? B_K1 : B_K2;
    const bf16* qb = base(qslot);
    const int64_t sq = P.s[qslot][2];
    const bf16* krow = base(kslot) + (int64_t)jc * P.s[kslot][2];
    const float rk = RK[br];
    const float* nq = nullptr;
    if constexpr (NORM) nq = P.norms + norm_base(P, br == 0 ? N_Q1 : N_Q2, bh);
    const float coef = br == 0 ? 1.f : -lam;
    f32x16 AK[ND];
#pragma unroll
    for (int c = 0; c < ND; ++c) AK[c] = f32x16{};
    // bitmask column: bit kt % 32 of word (br, bh, qt, kt / 32) for qt = qtf .. nqt-1
    const uint32_t* occcol = P.occ ? P.occ + ((int64_t)br * BH + bh) * P.nqt * P.occ_w + (kt >> 5) : nullptr;

    for (int q0c = qtf; q0c < P.nqt; q0c += 64) {
      const int qtl = q0c + l;
      const bool has = q0c == qtf ? HAS[br] : qtl < P.nqt && (!occcol || ((occcol[(int64_t)qtl * P.occ_w] >> (kt & 31)) & 1u));
      uint64_t mask = wave_ballot(has);
      while (mask) {
        const int qt = q0c + __builtin_ctzll(mask);
        mask &= mask - 1ull;
        ++visited;
        const int q0 = 32 * qt;
        bf16x8 K[NT];  // the key fragments, for the score recompute
#pragma unroll
        for (int t = 0; t < NT; ++t) K[t] = *reinterpret_cast<const bf16x8*>(krow + 16 * t + 8 * g);
        dma_tile<D>(qb, sq, q0, Nq, W.a);
        dma_tile<D>(dob, sdo, q0, Nq, W.b);
        if constexpr (NORM) dma_row_vals(nq, q0, Nq, W.rows);
        if (l < 32) W.taus[l] = beta * tau_coeff(qoff + q0 + l, P.inv_d);
        wait_all_loads();
        f32x16 S = f32x16{}, Dp = f32x16{};
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          S = PolBF16::mma(tile_row_frag<D>(W.a, t), K[t], S);
          Dp = PolBF16::mma(tile_row_frag<D>(W.b, t), V[t], Dp);
        }
        float rq[16], tq[16];
        if constexpr (NORM) crow_vals(W.rows, rq);
        crow_vals(W.taus, tq);
        f32x16 EV, EK;
        bool any = false;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int qi = q0 + crow(r, g);
          const bool valid = kvalid && qi < Nq && j <= qoff + qi;
          const float sr = NORM ? S[r] * rk : S[r];
          const float x = __builtin_fmaf(sr, NORM ? rq[r] : 1.f, -tq[r]);
          const bool pos = valid && x > 0.f;
          EV[r] = pos ? coef * pow_p<PK>(x, pw) : 0.f;
          const float ds = pos ? coef * dpow_p<PK>(x, pw) * Dp[r] : 0.f;
          EK[r] = NORM ? ds * rq[r] : ds;
          any = any || pos;
        }
        if (!occcol && wave_ballot(any) == 0ull) continue;
        ++computed;
        const bf16x8 V0 = PolBF16::pack_c(EV, 0), V1 = PolBF16::pack_c(EV, 1);
        const bf16x8 K0 = PolBF16::pack_c(EK, 0), K1 = PolBF16::pack_c(EK, 1);
#pragma unroll
        for (int c = 0; c < ND; ++c) {
          AV[c] = PolBF16::mma(tile_tr_frag<D>(W.b, 0, c), V0, AV[c]);
          AV[c] = PolBF16::mma(tile_tr_frag<D>(W.b, 1, c), V1, AV[c]);
          AK[c] = PolBF16::mma(tile_tr_frag<D>(W.a, 0, c), K0, AK[c]);
          AK[c] = PolBF16::mma(tile_tr_frag<D>(W.a, 1, c), K1, AK[c]);
        }
      }
    }
    if (kvalid) {
      GradRow<D> XR;  // the key row for the normalize backward
      if constexpr (NORM) load_grad_row<D>(krow, XR);
      const int gslot = br == 0 ? B_DK1 : B_DK2;
      bf16* grow = (bf16*)P.grad[br == 0 ? 1 : 3] + (int64_t)b * P.s[gslot][0] + (int64_t)h * P.s[gslot][1] +
                   (int64_t)j * P.s[gslot][2];
      store_grad_rows<D, NORM>(AK, XR, grow, rk);
    }
  }
  if (kvalid) {
    bf16* vrow = (bf16*)P.grad[4] + (int64_t)b * P.s[B_DV][0] + (int64_t)h * P.s[B_DV][1] + (int64_t)j * P.s[B_DV][2];
    store_grad_rows<D, false>(AV, GradRow<D>{}, vrow, 1.f);
  }
  if (P.stats && l == 0) {
    atomicAdd(P.stats + 0, (unsigned long long)visited);
    atomicAdd(P.stats + 1, (unsigned long long)computed);
  }
}

// Bit k set when the column of key-major item first + k (k < count <= 4) has a list that did
// not fit (the test of column_overflows): the bitmask bits and counts of the first 128 query
// tiles of every column in one round, longer columns' rest column by column.
template <int BR>
__device__ __forceinline__ uint32_t columns_overflow(const BwdParams& P, int64_t first, int count) {
  const int BH = P.B * P.H, l = lane_id();
  const uint32_t* counts = P.pairs + pair_lists(BR, BH, P.nqt) * 4 * kPairCap;
  int kt[4], bh[4], qtf[4];
  bool ovf[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int64_t item = first + (k < count ? k : 0);
    kt[k] = (int)(item / BH);
    bh[k] = (int)(item % BH);
    qtf[k] = qt_first(kt[k], P.qoff);
    ovf[k] = false;
  }
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int br = 0; br < BR; ++br) {
        const int qt = qtf[k] + 64 * c + l;
        const bool in = k < count && qt < P.nqt;
        const int64_t row = ((int64_t)br * BH + bh[k]) * P.nqt + (in ? qt : P.nqt - 1);
        const uint32_t w = P.occ[row * P.occ_w + (kt[k] >> 5)];
        const uint32_t n = counts[row];
        ovf[k] = ovf[k] || (in && ((w >> (kt[k] & 31)) & 1u) && n > (uint32_t)kPairCap);
      }
  uint32_t out = 0u;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    if (k >= count) continue;
    bool o = wave_ballot(ovf[k]) != 0ull;
    if (!o && qtf[k] + 128 < P.nqt) o = column_overflows<BR>(P, bh[k], kt[k], qtf[k] + 128);
    out |= o ? 1u << k : 0u;
  }
  return out;
}

// One wave per workgroup and `per_wave` consecutive items per wave.  With pair lists, the key
// tiles whose columns have only lists that fit belong to bwd_dkv_pairs: the wave tests its
// items' columns in one round and runs only the others (per_wave 4); without lists every item
// runs (per_wave 1).
// With the key-tile queue (per_wave 0), the waves take the queued key tiles in turn instead.
template <int D, int BR, int PK, bool NORM>
__global__ void __launch_bounds__(64) bwd_dkv_fast(BwdParams P, int per_wave) {
  __shared__ __attribute__((aligned(16))) BwdWaveLds<D> W;
  if (per_wave == 0) {
    const uint32_t queued = P.dkvq[0];
    for (uint32_t k = blockIdx.x; k < queued; k += gridDim.x) bwd_dkv_tile<D, BR, PK, NORM>(P, W, P.dkvq[1 + k]);
    return;
  }
  const int64_t n = (int64_t)P.B * P.H * P.nkt, first = (int64_t)blockIdx.x * per_wave;
  const int count = (int)min((int64_t)per_wave, n - first);
  if (count <= 0) return;
  uint32_t run = count >= 32 ? 0xffffffffu : (1u << count) - 1u;
  if (P.pairs) run = columns_overflow<BR>(P, first, count);
  for (; run; run &= run - 1u) bwd_dkv_tile<D, BR, PK, NORM>(P, W, first + __builtin_ctz(run));
}

// ------------------------------------------------------------------ both tile passes, one launch
// With pair lists and the key-tile queue: single-wave workgroups that first run the
// query-major tile pass for the lists that did not fit (64 list counts tested per round, the
// lists in order) and then take the key tiles the key-major pair pass queued.  The query-major
// items do not depend on the key-major pass, so they run after it here, which saves the launch
// of a separate query-major tile pass.  (Adding the dbeta / dlambda sum here, by the last
// workgroup to finish, cost more than the launch it saved: every workgroup's release fence
// wrote back its XCD's L2.)
template <int D, int BR, int PK, bool NORM>
__global__ void __launch_bounds__(64) bwd_tiles(BwdParams P) {
  __shared__ __attribute__((aligned(16))) BwdWaveLds<D> W;
  const int l = lane_id();
  const int BH = P.B * P.H;
  const int64_t lists = (int64_t)BR * BH * P.nqt, lists_h = (int64_t)BH * P.nqt;
  const uint32_t* counts = P.pairs + pair_lists(BR, BH, P.nqt) * 4 * kPairCap;
  for (int64_t f = (int64_t)blockIdx.x * 64; f < lists; f += (int64_t)gridDim.x * 64) {
    const bool need = f + l < lists && counts[f + l] > (uint32_t)kPairCap;
    for (uint64_t m = wave_ballot(need); m; m &= m - 1ull) {
      const int64_t lx = f + __builtin_ctzll(m);  // list (branch, head, query tile) -> tile-pass item
      const int br = (int)(lx / lists_h);
      const int64_t rem = lx % lists_h;
      const int bh = (int)(rem / P.nqt), qt = (int)(rem % P.nqt);
      const int64_t rest = (int64_t)(P.nqt - 1 - qt) * BH + bh;
      bwd_dq_tile<D, BR, PK, NORM>(P, W, BR == 2 ? 2 * rest + br : rest);
    }
  }
  const uint32_t queued = P.dkvq[0];
  for (uint32_t k = blockIdx.x; k < queued; k += gridDim.x) bwd_dkv_tile<D, BR, PK, NORM>(P, W, P.dkvq[1 + k]);
}

// ------------------------------------------------------------------ block tile passes
// For the backwards whose forward ran the block tile pass (no candidate lists, every query tile
// runs): kBwdBlk consecutive tiles of one head per workgroup, one wave each, walking the union of
// their bitmask tiles in step; each streamed tile's rows are loaded once per workgroup (each wave
// a quarter, one tile ahead into registers) into a two-stage LDS ring of swizzled tiles (the
// layout of dma_tile_b: tile_row_frag / tile_tr_frag read it), one fence-free barrier per tile.
// A wave computes only its own tiles, with the arithmetic of bwd_dq_tile / bwd_dkv_tile, the
// masks branch-free and only on the tiles that need them.
constexpr int kBwdBlk = 4;

// max(x, 0) of 16 values on their bits: a float is > 0 iff its bits as an int32 are.
__device__ __forceinline__ f32x16 relu_bits(const f32x16& x) {
  typedef int i32x16_ __attribute__((ext_vector_type(16)));
  i32x16_ b = __builtin_bit_cast(i32x16_, x);
#pragma unroll
  for (int r = 0; r < 16; ++r) b[r] = max(b[r], 0);
  return __builtin_bit_cast(f32x16, b);
}

// This wave's share of a 32-row tile of D columns: rows RPI (LPW wv + i) + l / CH, chunk l % CH.
template <int D>
struct BlkRows {
  static constexpr int CH = D / 8, RPI = 64 / CH, LPW = 32 / RPI / kBwdBlk;
  static_assert(LPW >= 1 && LPW * RPI * kBwdBlk == 32, "tile rows split evenly over the waves");
  u32x4 v[LPW];
  __device__ __forceinline__ void load(const bf16* rows, int64_t st, int r0, int n, int wv) {
    const int l = lane_id();
    const int nr = min(32, n - r0);
    const __amdgpu_buffer_rsrc_t rs = rows_rsrc(rows + (int64_t)r0 * st, (uint32_t)(((int64_t)(nr - 1) * st + D) * 2));
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int r = RPI * (LPW * wv + i) + l / CH;
      v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, (uint32_t)(((int64_t)r * st + 8 * (l % CH)) * 2), 0, 0);
    }
  }
  __device__ __forceinline__ void store(bf16* tile, int wv) const {
    const int l = lane_id();
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int r = RPI * (LPW * wv + i) + l / CH;
      *reinterpret_cast<u32x4*>(tile + r * D + 8 * ((l % CH) ^ bswz<D>(r))) = v[i];
    }
  }
};

// Query-major: kBwdBlk query tiles of one (branch, head), streaming K, V and the key norms.
template <int D, int BR, int PK, bool NORM>
__global__ void __launch_bounds__(64 * kBwdBlk) __attribute__((amdgpu_waves_per_eu(2))) bwd_dq_blk(BwdParams P) {
  constexpr int W = kBwdBlk, NT = D / 16, ND = D / 32;
  constexpr int STAGE = 2 * 32 * D;  // K tile, V tile
  __shared__ __attribute__((aligned(16))) bf16 ring[2 * STAGE];
  __shared__ __attribute__((aligned(16))) float nring[2][32];
  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int BH = P.B * P.H, nqt = P.nqt, Nq = P.Nq, Nk = P.Nk, qoff = P.qoff;
  const int nqb = (nqt + W - 1) / W;
  // longest blocks (last query tiles) of every (head, branch) first, the branches adjacent
  const int bid = blockIdx.x, jb = nqb - 1 - bid / (BR * BH), rem = bid % (BR * BH);
  const int br = BR == 2 ? rem & 1 : 0, bh = BR == 2 ? rem >> 1 : rem;
  const int b = bh / P.H, h = bh % P.H;
  const uint32_t* counts = P.pairs ? P.pairs + pair_lists(BR, BH, nqt) * 4 * kPairCap : nullptr;
  const int64_t lrow0 = ((int64_t)br * BH + bh) * nqt + W * jb;  // list / bitmask row of the block's first tile
  // the tiles whose lists did not fit (or all, without lists): the same for every wave
  uint32_t needm = 0u;
#pragma unroll
  for (int r = 0; r < W; ++r) {
    const int q = W * jb + r;
    const bool nd = q < nqt && (!counts || (uint32_t)__builtin_amdgcn_readfirstlane((int)counts[lrow0 + r]) > (uint32_t)kPairCap);
    needm |= nd ? 1u << r : 0u;
  }
  if (!needm) return;
  const int qt = W * jb + wv;
  const bool need = (needm >> wv) & 1u;
  const int qtc = min(qt, nqt - 1);
  const int i = 32 * qt + n32;
  const bool qvalid = need && i < Nq;
  const int ic = min(32 * qtc + n32, Nq - 1);
  const int pq = qoff + i;
  const bool rowpad = 32 * qt + 31 >= Nq;
  auto base = [&](int slot) {
    return (const bf16*)P.in[slot] + (int64_t)b * P.s[slot][0] + (int64_t)h * P.s[slot][1];
  };
  const int qslot = br == 0 ? B_Q1 : B_Q2, kslot = br == 0 ? B_K1 : B_K2;
  bf16x8 DO[NT], Q[NT];
  {
    const bf16* r = base(B_DO) + (int64_t)ic * P.s[B_DO][2];
    const bf16* rq_ = base(qslot) + (int64_t)ic * P.s[qslot][2];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      DO[t] = *reinterpret_cast<const bf16x8*>(r + 16 * t + 8 * g);
      Q[t] = *reinterpret_cast<const bf16x8*>(rq_ + 16 * t + 8 * g);
    }
  }
  const float rq = NORM ? P.norms[norm_base(P, br == 0 ? N_Q1 : N_Q2, bh) + ic] : 1.f;
  const float ci = tau_coeff(pq, P.inv_d);
  const float tau = (*P.beta) * ci;
  const float pw = P.p;
  float coef = 1.f;
  if constexpr (BR == 2) coef = br == 0 ? 1.f : -clamp01(*P.lam);
  const bool want_l = BR == 2 && br == 1;  // dlambda comes from branch 2 alone
  const bf16* vb = base(B_V);
  const int64_t sv = P.s[B_V][2];
  const bf16* kb = base(kslot);
  const int64_t sk = P.s[kslot][2];
  const float* nk = nullptr;
  if constexpr (NORM) nk = P.norms + norm_base(P, br == 0 ? N_K1 : N_K2, bh);
  float bsum = 0.f, lsum = 0.f;
  unsigned visited = 0, computed = 0;

  f32x16 A[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) A[c] = f32x16{};

  // word w of the block's row r, masked to the key tiles the row sees (uniform); every causal
  // tile without a bitmask
  const int klast_b = kt_last(min(W * jb + W - 1, nqt - 1), qoff, P.nkt);
  auto row_word = [&](int r, int w) -> uint32_t {
    if (!((needm >> r) & 1u)) return 0u;
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
  BlkRows<D> kr, vr;
  f32x4 nr = {};
  auto issue = [&](int kt) {
    kr.load(kb, sk, 32 * kt, Nk, wv);
    vr.load(vb, sv, 32 * kt, Nk, wv);
    if (NORM && wv == 0 && l < 8)
      nr = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                          rows_rsrc(nk + 32 * kt, (uint32_t)(min(32, Nk - 32 * kt) * 4)), 16u * (uint32_t)l, 0, 0));
  };
  uint32_t cown = 0u;
  int kt = next_tile(cown);
  if (kt >= 0) issue(kt);
  int it = 0;
  while (kt >= 0) {
    bf16* kst = ring + (it & 1) * STAGE;
    bf16* vst = kst + 32 * D;
    float* nst = nring[it & 1];
    kr.store(kst, wv);
    vr.store(vst, wv);
    if (NORM && wv == 0 && l < 8) *reinterpret_cast<f32x4*>(nst + 4 * l) = nr;
    uint32_t nown = 0u;
    const int kt2 = next_tile(nown);
    if (kt2 >= 0) issue(kt2);  // in flight during this tile's work
    lds_barrier();
    ++it;
    if ((cown >> (kt & 31)) & 1u) {
      ++visited;
      const int k0 = 32 * kt;
      bool anyw = true;  // without a bitmask the counters count the tiles with a weight
      f32x16 S = f32x16{}, Dp = f32x16{};
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        S = PolBF16::mma(tile_row_frag<D>(kst, t), Q[t], S);
        Dp = PolBF16::mma(tile_row_frag<D>(vst, t), DO[t], Dp);
      }
      float rk[16];
      if constexpr (NORM) crow_vals(nst, rk);
      // exact x, branch-free; keys after the query's position, padding keys and rows past Nq
      // set to -1 (only on the tiles that have any)
      f32x16 X;
#pragma unroll
      for (int r = 0; r < 16; ++r) X[r] = __builtin_fmaf(NORM ? S[r] * rk[r] : S[r], rq, -tau);
      if (k0 + 31 > min(qoff + 32 * qt, Nk - 1) || rowpad) {
        // key crow(r, g) = c_r + 4 g (c_r = 8 (r / 4) + r % 4) is visible iff c_r <= lim: one
        // comparison per value
        const int lim = (qvalid ? min(pq, Nk - 1) - k0 : -1) - 4 * g;
#pragma unroll
        for (int r = 0; r < 16; ++r) X[r] = 8 * (r >> 2) + (r & 3) <= lim ? X[r] : -1.f;
      }
      f32x16 E;
      if constexpr (PK == 2) {
        // relu on the bits (a float is > 0 iff its bits as an int32 are): t = max(x, 0) with no
        // comparison per value; 2 t and t^2 vanish with t.  (Whole-vector bit casts: hipcc
        // compiled a bit cast of one element of an ext_vector to element 0.)
        const f32x16 T = relu_bits(X);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float ds = coef * (T[r] + T[r]) * Dp[r];
          bsum += ds;
          if (want_l) lsum = __builtin_fmaf(T[r] * T[r], Dp[r], lsum);
          E[r] = NORM ? ds * rk[r] : ds;
        }
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const bool pos = X[r] > 0.f;
          const float ds = pos ? coef * dpow_p<PK>(X[r], pw) * Dp[r] : 0.f;
          bsum += ds;
          if (want_l) lsum = __builtin_fmaf(pos ? pow_p<PK>(X[r], pw) : 0.f, Dp[r], lsum);
          E[r] = NORM ? ds * rk[r] : ds;
        }
      }
      if (!P.occ) {
        float xm = X[0];
#pragma unroll
        for (int r = 1; r < 16; ++r) xm = fmaxf(xm, X[r]);
        anyw = wave_ballot(xm > 0.f) != 0ull;
      }
      computed += anyw ? 1u : 0u;
      const bf16x8 E0 = PolBF16::pack_c(E, 0), E1 = PolBF16::pack_c(E, 1);
#pragma unroll
      for (int c = 0; c < ND; ++c) {
        A[c] = PolBF16::mma(tile_tr_frag<D>(kst, 0, c), E0, A[c]);
        A[c] = PolBF16::mma(tile_tr_frag<D>(kst, 1, c), E1, A[c]);
      }
    }
    cown = nown;  // the own row's word of the next tile
    kt = kt2;
  }
  if (!need) return;
  if (qvalid) {
    GradRow<D> XR;  // the query row for the normalize backward
    if constexpr (NORM) load_grad_row<D>(base(qslot) + (int64_t)ic * P.s[qslot][2], XR);
    const int gslot = br == 0 ? B_DQ1 : B_DQ2;
    bf16* grow = (bf16*)P.grad[br == 0 ? 0 : 2] + (int64_t)b * P.s[gslot][0] + (int64_t)h * P.s[gslot][1] +
                 (int64_t)i * P.s[gslot][2];
    store_grad_rows<D, NORM>(A, XR, grow, rq);
  }
  const float pb = wave_sum(-ci * bsum);
  const float pl = wave_sum(-lsum);
  if (l == 0) {
    const int64_t lidx = lrow0 + wv;
    P.ws[2 * lidx + 0] = pb;  // slot of (branch, head, query tile), whichever pass takes it
    P.ws[2 * lidx + 1] = pl;
    if (P.stats) {
      atomicAdd(P.stats + 0, (unsigned long long)visited);
      atomicAdd(P.stats + 1, (unsigned long long)computed);
    }
  }
}

// Key-major: kBwdBlk consecutive key tiles of one head (aligned: one bitmask word holds their
// bits), streaming per branch the query tiles' Q and dO rows, query norms and tau values.  A key
// tile takes this pass when a list of its column did not fit (the test bwd_dkv_pairs queues
// by; it writes nothing for such a key tile), or always without lists.
template <int D, int BR, int PK, bool NORM>
__global__ void __launch_bounds__(64 * kBwdBlk) __attribute__((amdgpu_waves_per_eu(BR == 2 ? (D <= 64 ? 2 : 1) : (D <= 64 ? 3 : 2)))) bwd_dkv_blk(BwdParams P) {
  constexpr int W = kBwdBlk, NT = D / 16, ND = D / 32;
  constexpr int STAGE = 2 * 32 * D;  // Q tile, dO tile
  __shared__ __attribute__((aligned(16))) bf16 ring[2 * STAGE];
  __shared__ __attribute__((aligned(16))) float vring[2][2][32];  // [stage][query norms, tau values]
  __shared__ __attribute__((aligned(16))) bf16 ktiles[W][32 * D];  // each wave's key rows (swizzled)
  __shared__ uint32_t needs[W];
  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int BH = P.B * P.H, nqt = P.nqt, nkt = P.nkt, Nq = P.Nq, Nk = P.Nk, qoff = P.qoff;
  const int nkb = (nkt + W - 1) / W;
  // longest blocks (first key tiles) of every head first
  const int bid = blockIdx.x, jb = bid / BH, bh = bid % BH;
  const int b = bh / P.H, h = bh % P.H;
  const int kt0 = W * jb, kt = kt0 + wv;
  const int qtf_b = qt_first(kt0, qoff);  // first query tile of the block
  const uint32_t* counts = P.pairs ? P.pairs + pair_lists(BR, BH, nqt) * 4 * kPairCap : nullptr;
  // this wave's key tile: does a list of its column not fit (every branch, query tiles from
  // the first that sees it)?
  {
    bool nd = kt < nkt;
    if (nd && counts) {
      const int qtf = qt_first(kt, qoff);
      bool ovf = false;
      for (int q0c = qtf; q0c < nqt && !ovf; q0c += 64) {
        bool o = false;
#pragma unroll
        for (int br = 0; br < BR; ++br) {
          const int qtl = q0c + l;
          const bool in = qtl < nqt;
          const int64_t row = ((int64_t)br * BH + bh) * nqt + (in ? qtl : nqt - 1);
          const uint32_t w = P.occ ? P.occ[row * P.occ_w + (kt >> 5)] : 0xffffffffu;
          o = o || (in && ((w >> (kt & 31)) & 1u) && counts[row] > (uint32_t)kPairCap);
        }
        ovf = wave_ballot(o) != 0ull;
      }
      nd = ovf;
    }
    if (l == 0) needs[wv] = nd ? 1u : 0u;
  }
  __syncthreads();
  uint32_t needm = 0u;
#pragma unroll
  for (int r = 0; r < W; ++r) needm |= needs[r] ? 1u << r : 0u;
  needm = (uint32_t)__builtin_amdgcn_readfirstlane((int)needm);
  if (!needm) return;
  const bool need = (needm >> wv) & 1u;
  const int j = 32 * kt + n32;
  const bool kvalid = need && j < Nk;
  const int jc = min(j, Nk - 1);
  const int qtf_w = qt_first(kt, qoff);  // first query tile that sees this wave's key tile
  auto base = [&](int slot) {
    return (const bf16*)P.in[slot] + (int64_t)b * P.s[slot][0] + (int64_t)h * P.s[slot][1];
  };

  bf16x8 V[NT];
  {
    const bf16* r = base(B_V) + (int64_t)jc * P.s[B_V][2];
#pragma unroll
    for (int t = 0; t < NT; ++t) V[t] = *reinterpret_cast<const bf16x8*>(r + 16 * t + 8 * g);
  }
  const float beta = *P.beta;
  const float pw = P.p;
  float lam = 0.f;
  if constexpr (BR == 2) lam = clamp01(*P.lam);
  const bf16* dob = base(B_DO);
  const int64_t sdo = P.s[B_DO][2];
  f32x16 AV[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) AV[c] = f32x16{};
  unsigned visited = 0, computed = 0;
  int it = 0;  // ring position, continued across the branches
  bf16* kti = ktiles[wv];

#pragma unroll
  for (int br = 0; br < BR; ++br) {
    const int qslot = br == 0 ? B_Q1 : B_Q2, kslot = br == 0 ? B_K1 : B_K2;
    const bf16* qb = base(qslot);
    const int64_t sq = P.s[qslot][2];
    const float rk = NORM ? P.norms[norm_base(P, br == 0 ? N_K1 : N_K2, bh) + jc] : 1.f;
    const float* nq = nullptr;
    if constexpr (NORM) nq = P.norms + norm_base(P, br == 0 ? N_Q1 : N_Q2, bh);
    const float coef = br == 0 ? 1.f : -lam;
    // the wave's key rows (swizzled tile; rows past Nk read as zeros), read as score operands
    {
      BlkRows<D> kr4[kBwdBlk];
#pragma unroll
      for (int s4 = 0; s4 < kBwdBlk; ++s4) kr4[s4].load(base(kslot), P.s[kslot][2], 32 * min(kt, nkt - 1), Nk, s4);
#pragma unroll
      for (int s4 = 0; s4 < kBwdBlk; ++s4) kr4[s4].store(kti, s4);
    }
    f32x16 AK[ND];
#pragma unroll
    for (int c = 0; c < ND; ++c) AK[c] = f32x16{};
    const int64_t row0 = ((int64_t)br * BH + bh) * nqt;  // bitmask / list row of query tile 0

    // union walk over query tiles qtf_b .. nqt-1, 64 per round: lane q tests query tile q0c + q
    int q0c = qtf_b - 64;
    uint64_t um = 0ull, om = 0ull;
    auto next_tile = [&](bool& own_out) -> int {
      while (um == 0ull) {
        q0c += 64;
        if (q0c >= nqt) return -1;
        const int qtl = q0c + l;
        const bool in = qtl < nqt;
        const uint32_t w = !in ? 0u : P.occ ? P.occ[(row0 + qtl) * P.occ_w + (kt0 >> 5)] : 0xffffffffu;
        uint32_t bits = (w >> (kt0 & 31)) & 0xfu & needm;
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
    BlkRows<D> qr, dr;
    float vrq = 1.f, vtq = 0.f;
    auto issue = [&](int qt) {
      qr.load(qb, sq, 32 * qt, Nq, wv);
      dr.load(dob, sdo, 32 * qt, Nq, wv);
      if (wv == 0 && l < 32) {
        const int qi = min(32 * qt + l, Nq - 1);
        vrq = NORM ? nq[qi] : 1.f;
        vtq = beta * tau_coeff(qoff + 32 * qt + l, P.inv_d);
      }
    };
    bool cown = false;
    int qt = next_tile(cown);
    if (qt >= 0) issue(qt);
    while (qt >= 0) {
      bf16* qst = ring + (it & 1) * STAGE;
      bf16* dst = qst + 32 * D;
      float* rqs = vring[it & 1][0];
      float* tqs = vring[it & 1][1];
      qr.store(qst, wv);
      dr.store(dst, wv);
      if (wv == 0 && l < 32) {
        rqs[l] = vrq;
        tqs[l] = vtq;
      }
      bool nown = false;
      const int qt2 = next_tile(nown);
      if (qt2 >= 0) issue(qt2);  // in flight during this tile's work
      lds_barrier();
      ++it;
      if (cown) {
        ++visited;
        const int q0 = 32 * qt;
        f32x16 S = f32x16{}, Dp = f32x16{};
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          S = PolBF16::mma(tile_row_frag<D>(qst, t), tile_row_frag<D>(kti, t), S);
          Dp = PolBF16::mma(tile_row_frag<D>(dst, t), V[t], Dp);
        }
        float rq[16], tq[16];
        if constexpr (NORM) crow_vals(rqs, rq);
        crow_vals(tqs, tq);
        f32x16 X;
#pragma unroll
        for (int r = 0; r < 16; ++r) X[r] = __builtin_fmaf(NORM ? S[r] * rk : S[r], NORM ? rq[r] : 1.f, -tq[r]);
        // masks only on the tiles that need them: queries before the key (the diagonal), rows
        // past Nq, keys past Nk
        if (32 * kt + 31 > qoff + q0 || q0 + 31 >= Nq || 32 * kt + 31 >= Nk) {
          // query row crow(r, g) = c_r + 4 g (c_r = 8 (r / 4) + r % 4) sees the key iff
          // lo <= c_r <= lo + span: one unsigned comparison per value (an empty range: lo past
          // every c_r)
          const int lo0 = j - qoff - q0 - 4 * g, hi0 = Nq - 1 - q0 - 4 * g;
          const bool some = kvalid && hi0 >= lo0;
          const int lo = some ? lo0 : 64;
          const uint32_t span = some ? (uint32_t)(hi0 - lo0) : 0u;
#pragma unroll
          for (int r = 0; r < 16; ++r) X[r] = (uint32_t)(8 * (r >> 2) + (r & 3) - lo) <= span ? X[r] : -1.f;
        }
        f32x16 EV, EK;
        if constexpr (PK == 2) {  // relu on the bits, as in bwd_dq_blk
          const f32x16 T = relu_bits(X);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            EV[r] = coef * (T[r] * T[r]);
            const float ds = coef * (T[r] + T[r]) * Dp[r];
            EK[r] = NORM ? ds * rq[r] : ds;
          }
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const bool pos = X[r] > 0.f;
            EV[r] = pos ? coef * pow_p<PK>(X[r], pw) : 0.f;
            const float ds = pos ? coef * dpow_p<PK>(X[r], pw) * Dp[r] : 0.f;
            EK[r] = NORM ? ds * rq[r] : ds;
          }
        }
        bool anyw = true;  // without a bitmask the counters count the tiles with a weight
        if (!P.occ) {
          float xm = X[0];
#pragma unroll
          for (int r = 1; r < 16; ++r) xm = fmaxf(xm, X[r]);
          anyw = wave_ballot(xm > 0.f) != 0ull;
        }
        computed += anyw ? 1u : 0u;
        const bf16x8 V0 = PolBF16::pack_c(EV, 0), V1 = PolBF16::pack_c(EV, 1);
        const bf16x8 K0 = PolBF16::pack_c(EK, 0), K1 = PolBF16::pack_c(EK, 1);
#pragma unroll
        for (int c = 0; c < ND; ++c) {
          AV[c] = PolBF16::mma(tile_tr_frag<D>(dst, 0, c), V0, AV[c]);
          AV[c] = PolBF16::mma(tile_tr_frag<D>(dst, 1, c), V1, AV[c]);
          AK[c] = PolBF16::mma(tile_tr_frag<D>(qst, 0, c), K0, AK[c]);
          AK[c] = PolBF16::mma(tile_tr_frag<D>(qst, 1, c), K1, AK[c]);
        }
      }
      cown = nown;
      qt = qt2;
    }
    if (kvalid) {
      GradRow<D> XR;  // the key row for the normalize backward
      if constexpr (NORM) load_grad_row<D>(base(kslot) + (int64_t)jc * P.s[kslot][2], XR);
      const int gslot = br == 0 ? B_DK1 : B_DK2;
      bf16* grow = (bf16*)P.grad[br == 0 ? 1 : 3] + (int64_t)b * P.s[gslot][0] + (int64_t)h * P.s[gslot][1] +
                   (int64_t)j * P.s[gslot][2];
      store_grad_rows<D, NORM>(AK, XR, grow, rk);
    }
    lds_barrier();  // every wave is done with its key tile before the next branch's rows
  }
  if (kvalid) {
    bf16* vrow = (bf16*)P.grad[4] + (int64_t)b * P.s[B_DV][0] + (int64_t)h * P.s[B_DV][1] + (int64_t)j * P.s[B_DV][2];
    store_grad_rows<D, false>(AV, GradRow<D>{}, vrow, 1.f);
  }
  if (P.stats && l == 0 && need) {
    atomicAdd(P.stats + 0, (unsigned long long)visited);
    atomicAdd(P.stats + 1, (unsigned long long)computed);
  }
}

// ------------------------------------------------------------------ dispatch
template <int D, int BR, int PK, bool NORM>
static int launch_t(const BwdParams& p, void* stream) {
  const int64_t qitems = (int64_t)BR * p.B * p.H * p.nqt, kitems = (int64_t)p.B * p.H * p.nkt;
  hipStream_t s = (hipStream_t)stream;
  if constexpr (!NORM) {
    // The forward ran its block tile pass (every query tile): the pair passes take the lists
    // that fit, then the block tile passes everything else (no key-tile queue), the sum.
    BwdParams q = p;
    q.dkvq = nullptr;
    if (q.pairs) {
      hipLaunchKernelGGL((bwd_dq_pairs<D, BR, PK, NORM>), dim3((unsigned)qitems), dim3(64), 0, s, q);
      launched(s, "bwd_dq_pairs");
      hipLaunchKernelGGL((bwd_dkv_pairs<D, BR, PK, NORM>), dim3((unsigned)kitems), dim3(64), 0, s, q);
      launched(s, "bwd_dkv_pairs");
    }
    const int BH = q.B * q.H;
    hipLaunchKernelGGL((bwd_dq_blk<D, BR, PK, NORM>), dim3((unsigned)(BR * BH * ((q.nqt + kBwdBlk - 1) / kBwdBlk))),
                       dim3(64 * kBwdBlk), 0, s, q);
    launched(s, "bwd_dq_blk");
    hipLaunchKernelGGL((bwd_dkv_blk<D, BR, PK, NORM>), dim3((unsigned)(BH * ((q.nkt + kBwdBlk - 1) / kBwdBlk))),
                       dim3(64 * kBwdBlk), 0, s, q);
    launched(s, "bwd_dkv_blk");
    const int e = (int)hipGetLastError();
    return e ? e : launch_bwd_finish(q, BR, qitems, stream);
  }
  if (p.pairs && p.dkvq) {  // the pair passes, both tile passes in one launch, the sum
    hipLaunchKernelGGL((bwd_dq_pairs<D, BR, PK, NORM>), dim3((unsigned)qitems), dim3(64), 0, s, p);
    launched(s, "bwd_dq_pairs");
    hipLaunchKernelGGL((bwd_dkv_pairs<D, BR, PK, NORM>), dim3((unsigned)kitems), dim3(64), 0, s, p);
    launched(s, "bwd_dkv_pairs");
    // one wave per SIMD (the key-major tile body's registers)
    hipLaunchKernelGGL((bwd_tiles<D, BR, PK, NORM>), dim3(1024u), dim3(64), 0, s, p);
    launched(s, "bwd_tiles");
    const int e = (int)hipGetLastError();
    return e ? e : launch_bwd_finish(p, BR, qitems, stream);
  }
  if (p.pairs) {
    hipLaunchKernelGGL((bwd_dq_pairs<D, BR, PK, NORM>), dim3((unsigned)qitems), dim3(64), 0, s, p);
    launched(s, "bwd_dq_pairs");
  }
  const int dq_per_wave = p.pairs ? 8 : 1;  // with pair lists most items exit at once
  hipLaunchKernelGGL((bwd_dq_fast<D, BR, PK, NORM>), dim3((unsigned)((qitems + dq_per_wave - 1) / dq_per_wave)),
                     dim3(64), 0, s, p, dq_per_wave);
  launched(s, "bwd_dq_fast");
  if (p.pairs) {
    hipLaunchKernelGGL((bwd_dkv_pairs<D, BR, PK, NORM>), dim3((unsigned)kitems), dim3(64), 0, s, p);
    launched(s, "bwd_dkv_pairs");
  }
  if (p.dkvq) {  // the key tiles the pair pass could not take, from its queue: one wave per SIMD
    hipLaunchKernelGGL((bwd_dkv_fast<D, BR, PK, NORM>), dim3((unsigned)(kitems < 1024 ? kitems : 1024)), dim3(64), 0, s,
                       p, 0);
  } else {
    const int dkv_per_wave = p.pairs ? 4 : 1;  // with pair lists most key tiles exit at once
    hipLaunchKernelGGL((bwd_dkv_fast<D, BR, PK, NORM>), dim3((unsigned)((kitems + dkv_per_wave - 1) / dkv_per_wave)),
                       dim3(64), 0, s, p, dkv_per_wave);
  }
  launched(s, "bwd_dkv_fast");
  const int e = (int)hipGetLastError();
  return e ? e : launch_bwd_finish(p, BR, qitems, stream);
}
template <int D, int BR, int PK>
static int sel_norm(const BwdParams& p, const KernelKey& k, void* s) {
  return k.normalize ? launch_t<D, BR, PK, true>(p, s) : launch_t<D, BR, PK, false>(p, s);
}
template <int D, int BR>
static int sel_pk(const BwdParams& p, const KernelKey& k, void* s) {
  switch (k.pkind) {
    case 2: return sel_norm<D, BR, 2>(p, k, s);
    case 1: return sel_norm<D, BR, 1>(p, k, s);
    default: return sel_norm<D, BR, 0>(p, k, s);
  }
}
template <int D>
static int sel_br(const BwdParams& p, const KernelKey& k, void* s) {
  return k.branches == 2 ? sel_pk<D, 2>(p, k, s) : sel_pk<D, 1>(p, k, s);
}

int launch_bwd_fast(const BwdParams& p, const KernelKey& k, void* stream) {
  return k.d == 128 ? sel_br<128>(p, k, stream) : sel_br<64>(p, k, stream);
}

// The pair passes on fp32 rows (the fp32 backward's launcher in tda_bwd.hip runs the tile passes
// for what they leave).
template <int D, int BR, int PK, bool NORM>
static int pairs_f32_t(const BwdParams& p, hipStream_t s) {
  const int64_t qitems = (int64_t)BR * p.B * p.H * p.nqt, kitems = (int64_t)p.B * p.H * p.nkt;
  hipLaunchKernelGGL((bwd_dq_pairs<D, BR, PK, NORM, float>), dim3((unsigned)qitems), dim3(64), 0, s, p);
  launched(s, "bwd_dq_pairs");
  hipLaunchKernelGGL((bwd_dkv_pairs<D, BR, PK, NORM, float>), dim3((unsigned)kitems), dim3(64), 0, s, p);
  launched(s, "bwd_dkv_pairs");
  return (int)hipGetLastError();
}
template <int D, int BR, int PK>
static int pairs_f32_norm(const BwdParams& p, const KernelKey& k, hipStream_t s) {
  return k.normalize ? pairs_f32_t<D, BR, PK, true>(p, s) : pairs_f32_t<D, BR, PK, false>(p, s);
}
template <int D, int BR>
static int pairs_f32_pk(const BwdParams& p, const KernelKey& k, hipStream_t s) {
  switch (k.pkind) {
    case 2: return pairs_f32_norm<D, BR, 2>(p, k, s);
    case 1: return pairs_f32_norm<D, BR, 1>(p, k, s);
    default: return pairs_f32_norm<D, BR, 0>(p, k, s);
  }
}
template <int D>
static int pairs_f32_br(const BwdParams& p, const KernelKey& k, hipStream_t s) {
  return k.branches == 2 ? pairs_f32_pk<D, 2>(p, k, s) : pairs_f32_pk<D, 1>(p, k, s);
}
int launch_bwd_pairs_f32(const BwdParams& p, const KernelKey& k, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  return k.d == 128 ? pairs_f32_br<128>(p, k, s) : pairs_f32_br<64>(p, k, s);
}

}  // namespace tda
