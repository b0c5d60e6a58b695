// tda_fwd_decode.hip -- bf16 forward of threshold attention for a single query tile
// (Nq <= 32 rows: KV-cache decode), gfx950.
//
// Reference semantics: snap-research/TDA triton_threshold_attention.py forward kernel
// (TTA:19-115) and the differential composition (TTA:489-519), with query row i at position
// qoff + i seeing the keys j <= qoff + i (the reference's case is qoff = 0, Nq = Nk).
//
// With one query tile the work is one pass over the key rows, HBM-bound: the keys of both
// branches are read once (their inverse norms computed on the fly, no separate pass) and V only
// for the key tiles holding a non-zero weight.  The key range is split for parallelism:
//   fwd_decode      one workgroup per (head, chunk of 32 key tiles); wave w takes the chunk's
//                   key tiles w, w + 4, ...  Pass 1, per (key tile, branch), with the next two
//                   items' key rows in flight: the key fragments, their inverse norms (written
//                   to the norms table), the transposed score tile S^T = K Q^T on the matrix
//                   cores and the exact test, a wave ballot into the tile's bitmask bit.  Pass 2,
//                   per tile with a non-zero weight: the same scores and weights again and
//                   O^T += V^T A^T with V staged through the wave's LDS.  The four waves'
//                   partial outputs are summed through LDS into one fp32 partial per chunk; the
//                   chunk's 32 tile bits form bitmask word `chunk` of the query tile's row,
//                   written whole.
//   fwd_decode_sum  out = sum of the chunk partials, chunk by chunk in order (deterministic).
#include "tda_common.hpp"
#include "tda_params.hpp"
#include "tda_pos.hpp"

namespace tda {
namespace {

constexpr int kDecWaves = 4;  // waves per workgroup; key tiles per chunk = 32

// Sum of squares of a row held as NT bf16x8 fragments per lane half (the row's two halves in
// lanes n and n + 32): bf16 pairs by dot2 (each product exact in fp32), two chains over the
// even and odd fragments, then the other half's sum.  A quarter of the instructions of
// converting and multiplying each element; the decode kernel computes every norm it uses (and
// writes to the norms table) with it.
template <int NT>
__device__ __forceinline__ float dec_sumsq(const bf16x8 (&f)[NT]) {
  float a[2] = {0.f, 0.f};
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const bf16x8 w = f[t];
    const bf16x2 p0 = __builtin_shufflevector(w, w, 0, 1), p1 = __builtin_shufflevector(w, w, 2, 3);
    const bf16x2 p2 = __builtin_shufflevector(w, w, 4, 5), p3 = __builtin_shufflevector(w, w, 6, 7);
    float& x = a[t & 1];
    x = __builtin_amdgcn_fdot2_f32_bf16(p0, p0, x, false);
    x = __builtin_amdgcn_fdot2_f32_bf16(p1, p1, x, false);
    x = __builtin_amdgcn_fdot2_f32_bf16(p2, p2, x, false);
    x = __builtin_amdgcn_fdot2_f32_bf16(p3, p3, x, false);
  }
  const float v = a[0] + a[1];
  return v + __shfl_xor(v, 32);
}

template <int D, int BR, int PK, bool NORM>
__global__ void __launch_bounds__(64 * kDecWaves, 2) fwd_decode(FwdParams P, float* part) {
  using Pol = PolBF16;
  constexpr int NT = D / 16, ND = D / 32;
  __shared__ __attribute__((aligned(16))) bf16 vlds[kDecWaves][TTileBF16<D>::ELEMS];
  __shared__ __attribute__((aligned(16))) float red[D][33];  // partial O^T (d, query), padded
  __shared__ uint32_t wbits[BR][kDecWaves];
  __shared__ __attribute__((aligned(16))) float rkl[kDecWaves][32];  // a tile's key norms, per wave

  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int BH = P.B * P.H, Nq = P.Nq, Nk = P.Nk, qoff = P.qoff;
  const int nch = (P.nkt + 31) / 32;
  const int bh = blockIdx.x / nch, chunk = blockIdx.x % nch;
  const int b = bh / P.H, h = bh % P.H;
  const int klast = kt_last(0, qoff, P.nkt);  // last key tile the query tile sees

  const TRef<const bf16> qr[2] = {{(const bf16*)P.in[F_Q1], P.s[F_Q1][0], P.s[F_Q1][1], P.s[F_Q1][2]},
                                  {(const bf16*)P.in[F_Q2], P.s[F_Q2][0], P.s[F_Q2][1], P.s[F_Q2][2]}};
  const TRef<const bf16> kr[2] = {{(const bf16*)P.in[F_K1], P.s[F_K1][0], P.s[F_K1][1], P.s[F_K1][2]},
                                  {(const bf16*)P.in[F_K2], P.s[F_K2][0], P.s[F_K2][1], P.s[F_K2][2]}};
  const TRef<const bf16> vv{(const bf16*)P.in[F_V], P.s[F_V][0], P.s[F_V][1], P.s[F_V][2]};

  // this lane's query row (B operand): rows past Nq are zeros and never hold a weight
  const int i = n32;
  const bool qvalid = i < Nq;
  const int pq = qoff + i;
  bf16x8 Q[BR][NT];
  float rq[BR];
#pragma unroll
  for (int br = 0; br < BR; ++br) {
    const bf16* row = qvalid ? qr[br].row(b, h, i) : nullptr;
#pragma unroll
    for (int t = 0; t < NT; ++t) Q[br][t] = Pol::load_row(row, t, g);
    rq[br] = 1.f;
    if constexpr (NORM) {
      rq[br] = inv_norm(dec_sumsq<NT>(Q[br]));
      if (chunk == 0 && wv == 0 && g == 0 && qvalid) P.norms[norm_base(P, br ? N_Q2 : N_Q1, bh) + i] = rq[br];
    }
  }
  const float tau = (*P.beta) * tau_coeff(pq, P.inv_d);
  const float pw = P.p;
  float lam = 0.f;
  if constexpr (BR == 2) lam = clamp01(*P.lam);

  // Pass 1, every key tile of the wave (kt = 32 chunk + wv + 4 m) and branch: the key rows
  // (those of the next two (tile, branch) items in flight while one is tested), their inverse
  // norms into the norms table, the score tile and the exact test, which sets the tile's bitmask
  // bit.  No V and no output accumulators: the registers hold three items' key rows instead.
  // Pass 2 recomputes the few tiles with a non-zero weight (the same operations on the same
  // values: the same scores and weights) and accumulates O^T += V^T A^T.
  // A lane past Nk loads row Nk - 1, and an item past the last key tile loads that tile (no
  // branch around the loads): such scores are masked by key < Nk, such norms are not stored.
  auto load_rows_br = [&](int kt, int br, bf16x8 (&K)[NT]) {
    const int j = min(32 * kt + n32, Nk - 1);
    const bf16* row = kr[br].row(b, h, j);
#pragma unroll
    for (int t = 0; t < NT; ++t) K[t] = *reinterpret_cast<const bf16x8*>(row + 16 * t + 8 * g);
  };
  auto load_k = [&](int kt, bf16x8 (&K)[BR][NT]) {
#pragma unroll
    for (int br = 0; br < BR; ++br) load_rows_br(kt, br, K[br]);
  };
  float* rkw = rkl[wv];
  // the inverse norms of a tile's keys in branch br (written to the norms table when `store`)
  // and the values r of this lane (keys crow(r, g)) from the wave's LDS slots
  auto key_norms = [&](int kt, int br, const bf16x8 (&K)[NT], f32x4 (&rk4)[4], bool store) {
    const int j = 32 * kt + n32;
    float rk = 1.f;
    if constexpr (NORM) {
      rk = inv_norm(dec_sumsq<NT>(K));
      if (store && g == 0 && j < Nk) P.norms[norm_base(P, br ? N_K2 : N_K1, bh) + j] = rk;
    }
    if (g == 0) rkw[n32] = rk;
    wave_lds_sync();
#pragma unroll
    for (int u = 0; u < 4; ++u) rk4[u] = *reinterpret_cast<const f32x4*>(rkw + 8 * u + 4 * g);
    wave_lds_sync();  // the slots are rewritten by the next item
  };
  // the score tile of branch br: this lane's 16 values (query n32, keys crow(r, g))
  auto scores = [&](const bf16x8 (&K)[NT], int br) {
    f32x16 S = {};
#pragma unroll
    for (int t = 0; t < NT; ++t) S = Pol::mma(K[t], Q[br][t], S);
    return S;
  };
  auto weight_pos = [&](int key, float s, float rkr, float rqb, float& x) {
    x = __builtin_fmaf(s * rkr, rqb, -tau);
    return qvalid && key <= pq && key < Nk && x > 0.f;
  };

  uint32_t word[BR];
#pragma unroll
  for (int br = 0; br < BR; ++br) word[br] = 0u;
  unsigned visited = 0, computed = 0;
  {
    constexpr int NI = (32 / kDecWaves) * BR;  // (tile, branch) items of the wave
    constexpr int NB = 3;                      // key-row buffers: two items in flight
    auto item_kt = [&](int it) { return 32 * chunk + wv + kDecWaves * (it / BR); };
    bf16x8 Kr[NB][NT];
#pragma unroll
    for (int it = 0; it < NB - 1; ++it) load_rows_br(min(item_kt(it), P.nkt - 1), it % BR, Kr[it]);
#pragma unroll
    for (int it = 0; it < NI; ++it) {
      if (it + NB - 1 < NI)
        load_rows_br(min(item_kt(it + NB - 1), P.nkt - 1), (it + NB - 1) % BR, Kr[(it + NB - 1) % NB]);
      const int kt = item_kt(it), br = it % BR;
      if (kt >= P.nkt) continue;
      f32x4 rk4[4];
      key_norms(kt, br, Kr[it % NB], rk4, true);
      if (kt > klast) continue;  // keys after the last query position: norms only
      if (br == 0) visited += BR;
      const f32x16 S = scores(Kr[it % NB], br);
      const int k0 = 32 * kt;
      bool pos_any = false;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x;
        pos_any |= weight_pos(k0 + crow(r, g), S[r], rk4[r >> 2][r & 3], rq[br], x);
      }
      const bool any = wave_ballot(pos_any) != 0ull;
      word[br] |= (uint32_t)any << (kt & 31);
      computed += any ? 1u : 0u;
    }
  }

  // Pass 2: the tiles of this wave with a non-zero weight in either branch.
  TTileBF16<D> vt;
  vt.lds = vlds[wv];
  f32x16 O[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) O[c] = f32x16{};
  uint32_t hits = word[0];
  if constexpr (BR == 2) hits |= word[1];
  for (; hits; hits &= hits - 1u) {
    const int kt = 32 * chunk + __builtin_ctz(hits), k0 = 32 * kt;
    bf16x8 K[BR][NT];
    load_k(kt, K);
    f32x16 C = {};
#pragma unroll
    for (int br = 0; br < BR; ++br) {
      f32x4 rk4[4];
      key_norms(kt, br, K[br], rk4, false);
      const f32x16 S = scores(K[br], br);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float x;
        const bool pos = weight_pos(k0 + crow(r, g), S[r], rk4[r >> 2][r & 3], rq[br], x);
        const float a = pos ? pow_p<PK>(x, pw) : 0.f;
        C[r] = br == 0 ? a : __builtin_fmaf(-lam, a, C[r]);
      }
    }
    vt.stage(vv, b, h, k0, Nk);
    wave_lds_sync();
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const bf16x8 bp = Pol::pack_c(C, s);
#pragma unroll
      for (int c = 0; c < ND; ++c) O[c] = Pol::mma(vt.frag(s, c), bp, O[c]);
    }
    wave_lds_sync();
  }

  // sum the waves' partial outputs (O^T: lane (n, g) holds d = 32c + crow(r, g) of query n)
  if (l == 0) {
#pragma unroll
    for (int br = 0; br < BR; ++br) wbits[br][wv] = word[br];
  }
  for (int w = 0; w < kDecWaves; ++w) {
    if (wv == w) {
#pragma unroll
      for (int c = 0; c < ND; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float& cell = red[32 * c + crow(r, g)][n32];
          cell = w == 0 ? O[c][r] : cell + O[c][r];
        }
    }
    __syncthreads();
  }
  // the chunk's partial rows (valid queries only) and its bitmask words
  float* dst = part + ((int64_t)bh * nch + chunk) * Nq * D;
  for (int e = threadIdx.x; e < Nq * D; e += 64 * kDecWaves) {
    const int n = e / D, d = e % D;
    dst[e] = red[d][n];
  }
  if (P.pairs && chunk == 0 && threadIdx.x < BR)  // no pair lists here: the backward uses the bitmask
    P.pairs[pair_lists(BR, BH, 1) * 4 * kPairCap + (int64_t)threadIdx.x * BH + bh] = kPairOverflow;
  if (threadIdx.x < BR && P.occ) {
    const int br = threadIdx.x;
    uint32_t w = 0u;
#pragma unroll
    for (int x = 0; x < kDecWaves; ++x) w |= wbits[br][x];
    P.occ[((int64_t)br * BH + bh) * P.occ_w + chunk] = w;  // one query tile: row (br, bh, 0)
  }
  if (P.stats && l == 0 && visited) {
    atomicAdd(P.stats + 0, (unsigned long long)visited);
    atomicAdd(P.stats + 1, (unsigned long long)computed);
    atomicAdd(P.stats + 2, (unsigned long long)computed);  // every visited tile is tested exactly
  }
}

// out[bh][n][d] = sum over chunks of part[bh][chunk][n][d], in chunk order.
template <int D>
__global__ void __launch_bounds__(256) fwd_decode_sum(FwdParams P, const float* part) {
  const int BH = P.B * P.H, Nq = P.Nq;
  const int nch = (P.nkt + 31) / 32;
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= (int64_t)BH * Nq * D) return;
  const int bh = (int)(e / (Nq * D)), r = (int)(e % (Nq * D));
  const int n = r / D, d = r % D;
  const float* src = part + (int64_t)bh * nch * Nq * D + r;
  const int64_t cs = (int64_t)Nq * D;  // distance between two chunks' partials
  // eight chunks' loads in flight at a time, added in chunk order
  float acc = 0.f;
  int c = 0;
  for (; c + 8 <= nch; c += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = src[(int64_t)(c + u) * cs];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += v[u];
  }
  for (; c < nch; ++c) acc += src[(int64_t)c * cs];
  const int b = bh / P.H, h = bh % P.H;
  bf16* o = (bf16*)P.out + (int64_t)b * P.s[F_OUT][0] + (int64_t)h * P.s[F_OUT][1] + (int64_t)n * P.s[F_OUT][2];
  o[d] = (bf16)acc;
}

template <int D, int BR, int PK, bool NORM>
int launch_decode_t(const FwdParams& p, float* part, hipStream_t s) {
  const int BH = p.B * p.H;
  const int nch = (p.nkt + 31) / 32;
  hipLaunchKernelGGL((fwd_decode<D, BR, PK, NORM>), dim3((unsigned)(BH * nch)), dim3(64 * kDecWaves), 0, s, p, part);
  launched(s, "fwd_decode");
  const int64_t n = (int64_t)BH * p.Nq * D;
  hipLaunchKernelGGL((fwd_decode_sum<D>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, (const float*)part);
  launched(s, "fwd_decode_sum");
  return (int)hipGetLastError();
}
template <int D, int BR, int PK>
int dsel_norm(const FwdParams& p, const KernelKey& k, float* part, hipStream_t s) {
  return k.normalize ? launch_decode_t<D, BR, PK, true>(p, part, s) : launch_decode_t<D, BR, PK, false>(p, part, s);
}
template <int D, int BR>
int dsel_pk(const FwdParams& p, const KernelKey& k, float* part, hipStream_t s) {
  switch (k.pkind) {
    case 2: return dsel_norm<D, BR, 2>(p, k, part, s);
    case 1: return dsel_norm<D, BR, 1>(p, k, part, s);
    default: return dsel_norm<D, BR, 0>(p, k, part, s);
  }
}
template <int D>
int dsel_br(const FwdParams& p, const KernelKey& k, float* part, hipStream_t s) {
  return k.branches == 2 ? dsel_pk<D, 2>(p, k, part, s) : dsel_pk<D, 1>(p, k, part, s);
}

}  // namespace

int launch_fwd_decode(const FwdParams& p, const KernelKey& k, float* part, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  return k.d == 128 ? dsel_br<128>(p, k, part, s) : dsel_br<64>(p, k, part, s);
}

}  // namespace tda
