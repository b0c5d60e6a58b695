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
//                   key tiles w, w + 4, ...  Per key tile: the key fragments of both branches,
//                   their inverse norms (written to the norms table), the transposed score tiles
//                   S^T = K Q^T on the matrix cores, the exact weights, and, when a wave ballot
//                   finds a non-zero one, O^T += V^T A^T with V staged through the wave's LDS.
//                   The four waves' partial outputs are summed through LDS into one fp32 partial
//                   per chunk; the chunk's 32 tile bits form bitmask word `chunk` of the query
//                   tile's row, written whole.
//   fwd_decode_sum  out = sum of the chunk partials, chunk by chunk in order (deterministic).
#include "tda_common.hpp"
#include "tda_params.hpp"
#include "tda_pos.hpp"

namespace tda {
namespace {

constexpr int kDecWaves = 4;  // waves per workgroup; key tiles per chunk = 32

template <int D, int BR, int PK, bool NORM>
__global__ void __launch_bounds__(64 * kDecWaves, 2) fwd_decode(FwdParams P, float* part) {
  using Pol = PolBF16;
  constexpr int NT = D / 16, ND = D / 32;
  __shared__ __attribute__((aligned(16))) bf16 vlds[kDecWaves][TTileBF16<D>::ELEMS];
  __shared__ __attribute__((aligned(16))) float red[D][33];  // partial O^T (d, query), padded
  __shared__ uint32_t wbits[BR][kDecWaves];

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
      rq[br] = inv_norm(row_sumsq<Pol, NT>(Q[br]));
      if (chunk == 0 && wv == 0 && g == 0 && qvalid) P.norms[norm_base(P, br ? N_Q2 : N_Q1, bh) + i] = rq[br];
    }
  }
  const float tau = (*P.beta) * tau_coeff(pq, P.inv_d);
  const float pw = P.p;
  float lam = 0.f;
  if constexpr (BR == 2) lam = clamp01(*P.lam);

  TTileBF16<D> vt;
  vt.lds = vlds[wv];
  f32x16 O[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) O[c] = f32x16{};
  uint32_t word[BR];
#pragma unroll
  for (int br = 0; br < BR; ++br) word[br] = 0u;
  unsigned visited = 0, computed = 0;

  for (int u = wv; u < 32; u += kDecWaves) {
    const int kt = 32 * chunk + u;
    if (kt >= P.nkt) break;
    const int k0 = 32 * kt, j = k0 + n32;  // key row this lane loads (A operand row)
    bf16x8 K[BR][NT];
#pragma unroll
    for (int br = 0; br < BR; ++br) {
      const bf16* row = j < Nk ? kr[br].row(b, h, j) : nullptr;
#pragma unroll
      for (int t = 0; t < NT; ++t) K[br][t] = Pol::load_row(row, t, g);
    }
    float rk[BR];
#pragma unroll
    for (int br = 0; br < BR; ++br) {
      rk[br] = 1.f;
      if constexpr (NORM) {
        rk[br] = inv_norm(row_sumsq<Pol, NT>(K[br]));
        if (g == 0 && j < Nk) P.norms[norm_base(P, br ? N_K2 : N_K1, bh) + j] = rk[br];
      }
    }
    if (kt > klast) continue;  // keys after the last query position: norms only
    visited += BR;
    f32x16 C = {};
    bool any[BR];
#pragma unroll
    for (int br = 0; br < BR; ++br) {
      f32x16 S = {};
#pragma unroll
      for (int t = 0; t < NT; ++t) S = Pol::mma(K[br][t], Q[br][t], S);
      bool pos_any = false;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int key = k0 + crow(r, g);
        const float rkr = NORM ? __shfl(rk[br], crow(r, g)) : 1.f;
        const float x = __builtin_fmaf(S[r] * rkr, rq[br], -tau);
        const bool pos = qvalid && key <= pq && key < Nk && x > 0.f;
        const float a = pos ? pow_p<PK>(x, pw) : 0.f;
        C[r] = br == 0 ? a : __builtin_fmaf(-lam, a, C[r]);
        pos_any |= pos;
      }
      any[br] = wave_ballot(pos_any) != 0ull;
      word[br] |= (uint32_t)any[br] << (kt & 31);
      computed += any[br] ? 1u : 0u;
    }
    bool need = any[0];
    if constexpr (BR == 2) need = need || any[1];
    if (!need) continue;
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
  float acc = 0.f;
  for (int c = 0; c < nch; ++c) acc += src[(int64_t)c * Nq * D];
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
