// tda_fwd_sparse.hip -- bf16 forward of threshold attention for gfx950, built around the
// sparsity of the weights: with cosine scores and tau_i = beta sqrt(2 ln(i+1)/d), only a few
// percent of the 32x32 (query tile, key tile) weight blocks hold a non-zero entry.
//
// Reference semantics: snap-research/TDA triton_threshold_attention.py forward kernel
// (TTA:19-115: scores, threshold, ReLU^p, causal mask, A.V) and the differential composition
// out = A1 V - clamp(lambda, 0, 1) A2 V (TTA:489-519).
//
// Launches, in stream order:
//   key_norms   inverse L2 norms rk_j of the key rows, into the norms table (normalize only).
//   fwd_screen  for every causal (query tile, key tile) pair of a branch, a score tile on the
//               matrix cores and a test that keeps every tile holding a non-zero weight
//               (x_ij = fma(s_ij rk_j, rq_i, -tau_i) > 0 for some pair).  Without normalisation
//               the test is exact; with it, the queries enter pre-scaled by their inverse norms
//               and the test carries a margin bounded per query tile from the bf16 rounding
//               residuals of its rows (screen_tlo), so it may keep a few tiles whose weights
//               are all zero.  No V and no output accumulators: the kernel
//               holds only Q fragments and two score tiles per wave, so MFMA results stay in
//               ordinary VGPRs and several waves share a SIMD.  With normalisation it also
//               lists each query tile's candidate keys (the keys of its passing lanes).
//   fwd_pv_cand (normalize) one wave per query tile whose candidate lists fit: the score tile
//               of its rows against the candidate keys (the same MFMA sequence and operand
//               values as fwd_pv, so the same scores), the exact weights and out += coef A V
//               over the candidates' V rows; the bitmask row is rewritten exactly.  Query
//               tiles whose lists overflow go to a queue for fwd_pv.
//   fwd_pv      the tile pass, one wave per query tile (every tile without normalisation, the
//               queued ones with it): walks the set bits of both branches, recomputes the
//               score tile, forms the exact weights ReLU(x)^p with the causal mask, and
//               accumulates out += coef A V.  Tiles whose exact weights are all zero lose their
//               bit, so the bitmask ends exact.
// The screen tests every key of the tile, including keys after the query on the diagonal tile
// (and, without normalisation, padding keys past Nk): it may keep a tile the mask empties, never
// drop a non-zero one.  With normalisation padding keys are cleared from the hit bits, so no
// candidate list names a key row past Nk.
#include "tda_common.hpp"
#include "tda_params.hpp"
#include "tda_pos.hpp"

namespace tda {
namespace {


// Raw buffer descriptor over [base, base + bytes): loads past the end return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// Descriptor over the 32-row tile kt of a (N, D) head whose rows are `stride` elements apart:
// rows past N read as zeros.
template <int D>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_rsrc(const bf16* head, int64_t stride, int kt, int N) {
  const int rows = min(32, N - 32 * kt);
  return make_rsrc(head + (int64_t)(32 * kt) * stride, (uint32_t)(((int64_t)(rows - 1) * stride + D) * 2));
}

__device__ __forceinline__ float max16(const f32x16& v) {
  const float a = fmaxf(fmaxf(v[0], v[1]), fmaxf(v[2], v[3]));
  const float b = fmaxf(fmaxf(v[4], v[5]), fmaxf(v[6], v[7]));
  const float c = fmaxf(fmaxf(v[8], v[9]), fmaxf(v[10], v[11]));
  const float d = fmaxf(fmaxf(v[12], v[13]), fmaxf(v[14], v[15]));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Largest of 16 values, NaN if any is NaN (v_maximum3_f32: no NaN canonicalisation of the
// inputs, which the NaN-ignoring fmaxf needs in IEEE mode).
__device__ __forceinline__ float maximum16(const f32x16& v) {
  auto m3 = [](float a, float b, float c) {
    return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
  };
  const float a = m3(v[0], v[1], v[2]), b = m3(v[3], v[4], v[5]), c = m3(v[6], v[7], v[8]);
  const float d = m3(v[9], v[10], v[11]), e = m3(v[12], v[13], v[14]);
  return m3(m3(a, b, c), m3(d, e, v[15]), v[15]);
}

// Threshold of the normalised screen for one query tile, in cosine units.
//
// The exact pass keeps weight (i, j) iff x_ij = fma(fl(S_ij rk_j), rq_i, -tau_i) > 0, with S_ij
// the fp32 MFMA sum of q_i . k_j; the screen tests fl(sh_ij rk_j) > tlo with sh_ij the fp32 MFMA
// sum of qh_i . k_j and qh_i = bf16(fl(q_i rq_i)) (rq_i, rk_j: the same fp32 inverse norms on
// both sides).  Write qh_i = rq_i q_i + r_i + f_i, r_i = qh_i - fl(q_i rq_i) the bf16 rounding
// residual (exact in fp32) and |f_i| <= 2^-24 rq_i |q_i| the fp32 product's.  Then
//   |sh_ij - rq_i S_ij| <= (|r_i| + 2^-24 + 2^-17 |qh_i| + 2^-17 rq_i |q_i|) |k_j|
// (each 128-term fp32 accumulation errs by at most 128 * 2^-24 = 2^-17 of |a||b|, Cauchy-
// Schwarz), and with rq_i |q_i|, rk_j |k_j| <= 1 + 2^-16 and |qh_i| <= 1.01 the difference
// after the factor rk_j stays below |r_i| (1 + 2^-16) + 2^-15.  The two fp32 products of the
// tests add a relative 2^-24 each on values of magnitude <= 1.02.  So with
//   tlo = min_i tau_i - |min_i tau_i| 2^-19 - (max_i |r_i| (1 + 2^-14) + 2^-14)
// every kept weight passes the screen: max_i |r_i| is computed per query tile where qh is
// formed (fp32 sum of squares and square root: relative error below 2^-16, covered by the
// 2^-14 factor), and 2^-14 covers the 2^-15 of the accumulations plus the products' 2^-22.
// tau_i, evaluated in fp32 with a few ulps of error, is monotone in i up to a relative 2^-20;
// the 2^-19 term covers that and the products' relative error on tau.  A bf16 residual is
// at most 2^-8 of each element (unit roundoff of an 8-bit significand), so |r_i| <= 2^-8 |qh_i|;
// on N(0,1) rows it is about 0.0016.
__device__ __forceinline__ float screen_tlo(float tmin, float rmax) {
  return tmin - fabsf(tmin) * 0x1p-19f - (rmax * (1.f + 0x1p-14f) + 0x1p-14f);
}

// XCD-aware order of the (stream, block) work items of a grid: consecutive workgroup ids go to
// the 8 XCDs in turn, so all blocks of a stream (one head of one branch) run on one XCD and
// share its L2.  Blocks are handed out from the last (the longest causal row range) down.
struct WorkItem {
  int stream, block;
};
__device__ __forceinline__ WorkItem xcd_order(int bid, int nstreams, int nblocks) {
  WorkItem w;
  if (nstreams % 8 == 0) {
    const int x = bid & 7, j = bid >> 3, sp = nstreams >> 3;
    w.block = nblocks - 1 - j / sp;
    w.stream = x + 8 * (j % sp);
  } else {
    w.block = nblocks - 1 - bid / nstreams;
    w.stream = bid % nstreams;
  }
  return w;
}

// ------------------------------------------------------------------ key_norms
// Inverse L2 norms of the key rows of every branch.  A group of D/8 lanes reads one row (16
// bytes per lane, whole rows per load instruction); each wave covers KN_ROWS consecutive rows
// of one (branch, head) with all its loads issued before the first reduction.
constexpr int KN_GROUPS = 4;  // row groups per wave
template <int D>
__global__ void __launch_bounds__(256) key_norms(FwdParams P, int BR) {
  constexpr int LPR = D / 8;        // lanes per row
  constexpr int RPG = 64 / LPR;     // rows per load instruction
  constexpr int ROWS = RPG * KN_GROUPS;
  const int l = lane_id(), sub = l % LPR;
  const int BH = P.B * P.H, N = P.Nk;     // key rows
  const int wpr = (N + ROWS - 1) / ROWS;  // waves per (branch, head)
  const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wid >= (int64_t)BR * BH * wpr) return;  // whole wave, no barriers
  const int sidx = (int)(wid / wpr), br = sidx / BH, bh = sidx % BH;
  const int t0 = (int)(wid % wpr) * ROWS + l / LPR;
  const int slot = br ? F_K2 : F_K1;
  const int64_t st = P.s[slot][2];
  const bf16* head = (const bf16*)P.in[slot] + (int64_t)(bh / P.H) * P.s[slot][0] + (int64_t)(bh % P.H) * P.s[slot][1];
  bf16x8 x[KN_GROUPS];
#pragma unroll
  for (int u = 0; u < KN_GROUPS; ++u) {
    const int t = min(t0 + RPG * u, N - 1);
    x[u] = *reinterpret_cast<const bf16x8*>(head + (int64_t)t * st + 8 * sub);
  }
  float* out = P.norms + norm_base(P, br ? N_K2 : N_K1, bh);
#pragma unroll
  for (int u = 0; u < KN_GROUPS; ++u) {
    float ss = PolBF16::sumsq(x[u]);
#pragma unroll
    for (int o = LPR / 2; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
    const int t = t0 + RPG * u;
    if (sub == 0 && t < N) out[t] = inv_norm(ss);
  }
}

// ------------------------------------------------------------------ fwd_screen
// Workgroup = 256 query rows of one branch of one head, QPW 32-row query tiles per wave
// (8 / QPW waves); grid = branches x heads x ceil(N / 256).  Key tiles stream through LDS in
// groups of TPB tiles ("super-stages", two of them in a ring): buffer loads into VGPRs one
// iteration ahead, LDS writes of the next group while the current one is read, one barrier per
// group.
// Without normalisation, score tiles are computed transposed, S^T = K Q^T: each lane holds one
// query i and 16 of its keys, so "max_j s_ij > tau_i" is the exact test with one compare per
// lane.  With normalisation the weight test is s_ij rk_j rq_i > tau_i; the queries enter
// pre-scaled, qh_i = bf16(q_i rq_i), and the tile is computed as S = Qh K^T, so each lane holds
// one key j (and 16 queries): the per-lane test "max_i sh_ij * rk_j > tlo" needs one multiply
// per lane instead of one per score, with tlo = the tile's smallest tau minus screen_margin.
// Dispatch uses QPW = 2 (three waves per SIMD) and TPB = 1: one query tile per wave (twice the
// LDS fragment reads per MFMA) and larger groups (fewer waves) both measured slower at the
// headline shape.
template <int D, bool NORM, int QPW, int TPB>
__global__ void __launch_bounds__(512 / QPW, 2) fwd_screen(FwdParams P, int BR) {
  constexpr int NT = D / 16;                // MFMA steps over d
  constexpr int KS = D + 8;                 // LDS row stride (elements): conflict-free fragment reads
  constexpr int NTHR = 512 / QPW;           // threads per workgroup
  constexpr int CPR = D / 8;                // 16-byte chunks per key row
  constexpr int TPR = CPR < NTHR / 32 ? CPR : NTHR / 32;  // staging threads per row
  constexpr int CPT = CPR / TPR;            // chunks per staging thread
  __shared__ __attribute__((aligned(16))) bf16 kst[2 * TPB][32 * KS];
  __shared__ __attribute__((aligned(16))) float krk[2 * TPB][32];  // inverse key norms of each tile

  const int l = lane_id(), n32 = l & 31, g = l >> 5, tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int BH = P.B * P.H, Nq = P.Nq, Nk = P.Nk, nqt = P.nqt, qoff = P.qoff;
  if (NORM && P.pvq && blockIdx.x == 0 && tid == 0) P.pvq[0] = 0u;  // the candidate pass fills it
  const WorkItem wi = xcd_order(blockIdx.x, BR * BH, (Nq + 255) / 256);
  const int sidx = wi.stream, qb = wi.block;
  const int br = sidx / BH, bh = sidx % BH;
  const int b = bh / P.H, h = bh % P.H;
  const int qslot = br ? F_Q2 : F_Q1, kslot = br ? F_K2 : F_K1;
  const int q0w = qb * 256 + 32 * QPW * wv;  // first row of this wave
  const int qt0 = q0w >> 5;                  // this wave's query tiles: qt0 .. qt0 + QPW - 1
  const int nkt = kt_last(min(8 * qb + 7, nqt - 1), qoff, P.nkt) + 1;  // key tiles of the workgroup
  const int nit = (nkt + TPB - 1) / TPB;
  bool live[QPW];
  int ktl[QPW];  // last key tile each query tile sees
#pragma unroll
  for (int s = 0; s < QPW; ++s) {
    live[s] = qt0 + s < nqt;
    ktl[s] = kt_last(qt0 + s, qoff, P.nkt);
  }

  // ---- staging
  const bf16* khead = (const bf16*)P.in[kslot] + (int64_t)b * P.s[kslot][0] + (int64_t)h * P.s[kslot][1];
  const int64_t sk = P.s[kslot][2];
  const int srow = tid / TPR, sch = tid % TPR;
  const bool stager = tid < 32 * TPR;
  const uint32_t soff = (uint32_t)((srow * sk + 8 * sch) * 2);
  // key norms: threads 0..7 stage four rows each (rows past N read as 0, never used)
  const __amdgpu_buffer_rsrc_t rnorm =
      make_rsrc(NORM ? P.norms + norm_base(P, br ? N_K2 : N_K1, bh) : nullptr, NORM ? (uint32_t)Nk * 4 : 0u);
  u32x4 R[TPB][CPT], RN[TPB];
  auto fetch = [&](int it) {  // tiles of group it into registers
#pragma unroll
    for (int j = 0; j < TPB; ++j) {
      const int kt = TPB * it + j;
      if (kt >= nkt) break;
      if (stager) {
        const __amdgpu_buffer_rsrc_t rs = tile_rsrc<D>(khead, sk, kt, Nk);
#pragma unroll
        for (int c = 0; c < CPT; ++c) R[j][c] = buf_load16(rs, soff + 16 * TPR * c);
      }
      if constexpr (NORM)
        if (tid < 8) RN[j] = buf_load16(rnorm, (uint32_t)(32 * kt + 4 * tid) * 4);
    }
  };
  auto commit = [&](int it) {  // group it into its super-stage
#pragma unroll
    for (int j = 0; j < TPB; ++j) {
      const int kt = TPB * it + j;
      if (kt >= nkt) break;
      const int st = TPB * (it & 1) + j;
      if (stager) {
        bf16* k = &kst[st][srow * KS + 8 * sch];
#pragma unroll
        for (int c = 0; c < CPT; ++c) *reinterpret_cast<u32x4*>(k + 8 * TPR * c) = R[j][c];
      }
      if constexpr (NORM)
        if (tid < 8) *reinterpret_cast<u32x4*>(&krk[st][4 * tid]) = RN[j];
    }
  };

  // ---- resident query fragments, inverse norms, thresholds
  const bf16* qhead = (const bf16*)P.in[qslot] + (int64_t)b * P.s[qslot][0] + (int64_t)h * P.s[qslot][1];
  const float beta = *P.beta;
  bf16x8 Q[QPW][NT];
  float tau[QPW];  // without normalisation tau_i of the lane's query; with it the tile's tlo
  bool valid[QPW];
#pragma unroll
  for (int s = 0; s < QPW; ++s) {
    const int iq = q0w + 32 * s + n32;
    valid[s] = iq < Nq;
    const bf16* row = qhead + (int64_t)min(iq, Nq - 1) * P.s[qslot][2];  // rows >= Nq: never vote
#pragma unroll
    for (int t = 0; t < NT; ++t) Q[s][t] = *reinterpret_cast<const bf16x8*>(row + 16 * t + 8 * g);
    if constexpr (NORM) {
      const float rq = inv_norm(row_sumsq<PolBF16, NT>(Q[s]));
      if (g == 0 && valid[s]) P.norms[norm_base(P, br ? N_Q2 : N_Q1, bh) + iq] = rq;
      // rows past Nq score 0; so do non-finite elements (NaN/Inf inputs), whose exact weights
      // are 0 (x > 0 fails on NaN), so a NaN score can only come from a non-finite key row:
      // it poisons the maximum of that key's lane alone, whose weights are 0 as well
      const float sc = valid[s] ? rq : 0.f;
      float r2 = 0.f;  // squared norm of the row's bf16 rounding residual (this lane's half)
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float x0 = (float)Q[s][t][j] * sc;
          const float x = __builtin_isfinite(x0) ? x0 : 0.f;
          const bf16 xb = (bf16)x;
          const float r = (float)xb - x;  // exact: xb and x are within a factor of two
          r2 = __builtin_fmaf(r, r, r2);
          Q[s][t][j] = xb;
        }
      r2 += __shfl_xor(r2, 32);
#pragma unroll
      for (int o = 16; o >= 1; o >>= 1) r2 = fmaxf(r2, __shfl_xor(r2, o));  // largest of the tile
      // tau is monotone in the position: its smallest value over the tile's rows is at one of
      // the ends
      const int i0 = q0w + 32 * s, i1 = max(i0, min(i0 + 31, Nq - 1));
      tau[s] = screen_tlo(fminf(beta * tau_coeff(qoff + i0, P.inv_d), beta * tau_coeff(qoff + i1, P.inv_d)),
                          sqrtf(r2));
    } else {
      tau[s] = beta * tau_coeff(qoff + iq, P.inv_d);
    }
  }

  // ---- the call's zero range (the backward's gradients in training), spread over the steps of
  // every workgroup: workgroup (stream, block) clears zero_per_it units per key tile it walks,
  // from the sum of the steps of the workgroups before it in (stream, block) order
  int64_t z0 = 0, zend = 0;
  if (P.zero) {
    int64_t before = 0, per_stream = 0;
    for (int q = 0; q < (Nq + 255) / 256; ++q) {
      const int n = kt_last(min(8 * q + 7, nqt - 1), qoff, P.nkt) + 1;
      before += q < qb ? n : 0;
      per_stream += n;
    }
    z0 = ((int64_t)sidx * per_stream + before) * P.zero_per_it;
    zend = min(z0 + (int64_t)nkt * P.zero_per_it, P.zero_units);
  }
  // buffer stores over the workgroup's slice: the hardware drops those past its end (a slice
  // is below 1 MiB, so 32-bit offsets); streaming (nt): the backward reads them much later
  const __amdgpu_buffer_rsrc_t rzero =
      make_rsrc(P.zero ? reinterpret_cast<u32x4*>(P.zero) + z0 : nullptr, (uint32_t)(zend > z0 ? (zend - z0) * 16 : 0));
  auto clear = [&](int kt) {
    const uint32_t step = (uint32_t)kt * (uint32_t)P.zero_per_it * 16u;
    for (int u = tid; u < P.zero_per_it; u += NTHR)
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, rzero, (uint32_t)u * 16u, step, 2);
  };

  uint32_t* occ0 = P.occ + ((int64_t)sidx * nqt + qt0) * P.occ_w;  // bitmask row of qt0 (then qt0 + 1)
  // Per lane and query tile: bit kt % 32 set when the lane's test passed for key tile kt.  The
  // wave ORs them when a 32-tile word is complete (cheaper than a ballot per tile).
  uint32_t hb[QPW];
  uint32_t cn[QPW];  // candidate keys met per query tile (may pass the cap)
#pragma unroll
  for (int s = 0; s < QPW; ++s) hb[s] = cn[s] = 0u;
  const int koff = n32 * KS + 8 * g;

  // Threshold test of key tile kt (in stage st) against this wave's query tiles.
  auto process = [&](int kt, int st) {
    if (!(live[0] && kt <= ktl[QPW - 1])) return;
    const bf16* kp = &kst[st][koff];
    bf16x8 fk[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {  // in MFMA order: LDS returns in order, the chain waits per step
      fk[t] = *reinterpret_cast<const bf16x8*>(kp + 16 * t);
      __builtin_amdgcn_sched_barrier(0);
    }
    float rk = 1.f;
    if constexpr (NORM) rk = krk[st][n32];  // the lane's key (0 past N)
    __builtin_amdgcn_sched_barrier(0);  // all fragment reads in flight before the first MFMA
    f32x16 S[QPW];
#pragma unroll
    for (int s = 0; s < QPW; ++s) S[s] = f32x16{};
    // One query tile's chain at a time: dependent MFMAs back to back on the same accumulator
    // take the accumulate fast path; alternating two VGPR accumulators measured ~20 % slower.
#pragma unroll
    for (int s = 0; s < QPW; ++s) {
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if constexpr (NORM) S[s] = PolBF16::mma(Q[s][t], fk[t], S[s]);  // S = Qh K^T
        else S[s] = PolBF16::mma(fk[t], Q[s][t], S[s]);                 // S^T = K Q^T
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the chains apart
    }
    const uint32_t bit = 1u << (kt & 31);
    // Both tests run on every path, masked by selects: the MFMA results are read only in
    // straight-line code after the chains, where the compiler counts the wait states the
    // hardware needs between an MFMA writing a register and a VALU reading it.  (With a branch
    // skipping the first test, the compiler placed the second test's reads too early on the
    // branch path: 7 wait states where 12 are needed, so the test could read scores that were
    // not yet written.)
#pragma unroll
    for (int s = 0; s < QPW; ++s) {
      bool hit;
      if constexpr (NORM) hit = maximum16(S[s]) * rk > tau[s];  // largest score of the lane's key
      else hit = valid[s] && max16(S[s]) > tau[s];          // largest score of the lane's query
      // key tiles after the query tile's last position hold no causal pair; a query tile past
      // the last row (the wave's second, at the end of the sequence) has no list
      const bool lh = live[s] && hit && kt <= ktl[s];
      hb[s] |= lh ? bit : 0u;
    }
  };
  // bitmask words of this wave's rows: word kt/32 is complete after key tile kt
  const int kpad = P.nkt - 1;  // the key tile that may hold padding keys
  auto flush = [&](int kt) {
    if (live[0] && ((kt & 31) == 31 || kt == nkt - 1)) {
#pragma unroll
      for (int s = 0; s < QPW; ++s) {
        uint32_t w = hb[s];
        if constexpr (NORM) {
          // a padding key (past Nk, in the last key tile) scores 0 and passes a threshold below 0
          // (the query tile at position 0, beta <= 0): it holds no weight and must not be listed
          if ((kt >> 5) == (kpad >> 5) && n32 >= Nk - 32 * kpad) w &= ~(1u << (kpad & 31));
        }
        const uint32_t hm = w | (uint32_t)__shfl_xor((int)w, 32);  // lane n32: tiles its key passed
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) w |= (uint32_t)__shfl_xor((int)w, o);
        hb[s] = 0u;
        if constexpr (NORM) {
          // candidate keys of the word's tiles: per tile with a passing lane (a few per cent),
          // the keys of its passing lanes in increasing order, appended to the query tile's list
          if (P.cand) {
            uint32_t* clist = P.cand + ((int64_t)sidx * nqt + qt0 + s) * kCandCap;
            for (uint32_t m = (uint32_t)__builtin_amdgcn_readfirstlane((int)w); m; m &= m - 1u) {
              const int b = __builtin_ctz(m);
              const uint32_t keys = (uint32_t)wave_ballot(l < 32 && ((hm >> b) & 1u));
              const uint32_t slot = cn[s] + (uint32_t)__builtin_popcount(keys & ((1u << n32) - 1u));
              if (l < 32 && ((keys >> l) & 1u) && slot < (uint32_t)kCandCap)
                clist[slot] = (uint32_t)(32 * (32 * (kt >> 5) + b) + l);
              cn[s] += (uint32_t)__builtin_popcount(keys);
            }
          }
        }
        if (l == 0 && live[s]) {
          uint32_t* row = occ0 + s * P.occ_w;
          row[kt >> 5] = w;
          if (kt == nkt - 1)  // words of key tiles this workgroup never reaches
            for (int x = (kt >> 5) + 1; x < P.occ_w; ++x) row[x] = 0u;
        }
      }
    }
  };

  fetch(0);
  commit(0);
  if (nit > 1) fetch(1);
  __syncthreads();
  for (int it = 0; it < nit; ++it) {
#pragma unroll
    for (int j = 0; j < TPB; ++j) {
      const int kt = TPB * it + j;
      if (kt >= nkt) break;
      if (P.zero) clear(kt);
      process(kt, TPB * (it & 1) + j);
      flush(kt);
    }
    // the other super-stage was last read before the previous barrier
    if (it + 1 < nit) commit(it + 1);
    if (it + 2 < nit) fetch(it + 2);
    __syncthreads();
  }
  if (NORM && P.cand && l == 0) {
#pragma unroll
    for (int s = 0; s < QPW; ++s)
      if (live[s]) P.cand[pair_lists(BR, BH, nqt) * kCandCap + (int64_t)sidx * nqt + qt0 + s] = cn[s];
  }
  if (P.stats && l == 0) {
    // causal (query tile, key tile) pairs of this wave: key tiles 0 .. qt of each live query tile
    unsigned visited = 0;
#pragma unroll
    for (int s = 0; s < QPW; ++s) visited += live[s] ? (unsigned)(ktl[s] + 1) : 0u;
    if (visited) atomicAdd(P.stats + 0, (unsigned long long)visited);
  }
}

// ------------------------------------------------------------------ fwd_pv
// Transposed A fragment of one 32-column block and one 16-row step from a row-major tile
// with row stride VS: lane (n, g) gets column n of the block at tile rows crow(8*st + j, g),
// j = 0..7, by two LDS transpose reads.  `p` already includes this lane's base offset.
template <int VS>
__device__ __forceinline__ bf16x8 tr_frag(const bf16* p) {
  const bf16x4 a = __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(s16x4, p)));
  const bf16x4 c = __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(s16x4, p + 8 * VS)));
  return bf16x8{a[0], a[1], a[2], a[3], c[0], c[1], c[2], c[3]};
}

// The tile pass over one query tile (bh, qt): one wave; vt / ktl its LDS tiles.
template <int D, int BR, int PK, bool NORM>
__device__ __forceinline__ void fwd_pv_tile(const FwdParams& P, bf16* vt_, bf16* kt_, int bh, int qt) {
  constexpr int NT = D / 16, ND = D / 32;
  constexpr int VS = D + 32;     // LDS row stride of a V tile: conflict-free transpose reads
  constexpr int CPR = D / 8;     // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;  // rows per V load instruction
  constexpr int VL = 32 / RPI;   // V load instructions per tile
  constexpr int KS = D + 8;      // LDS row stride of a K tile: conflict-free row-fragment reads
  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int BH = P.B * P.H, Nq = P.Nq, Nk = P.Nk, nqt = P.nqt, qoff = P.qoff;
  const int b = bh / P.H, h = bh % P.H;
  const int iq = 32 * qt + n32;
  const bool valid = iq < Nq;
  const int pq = qoff + iq;                  // the lane's query position
  const int klast = kt_last(qt, qoff, P.nkt);  // last key tile the query tile sees
  const float tau = *P.beta * tau_coeff(pq, P.inv_d);
  const float pw = P.p;
  float lam = 0.f;
  if constexpr (BR == 2) lam = clamp01(*P.lam);

  bf16* vt = vt_;
  bf16* ktl = kt_;
  const int vrow = l / CPR, vch = l % CPR;
  const int bk = l >> 4, jj = l & 15;
  const int voff = (4 * (bk >> 1) + (jj >> 2)) * VS + 16 * (bk & 1) + 4 * (jj & 3);

  f32x16 O[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) O[c] = f32x16{};
  unsigned computed = 0, checked = 0;

#pragma unroll
  for (int br = 0; br < BR; ++br) {
    const int qslot = br ? F_Q2 : F_Q1, kslot = br ? F_K2 : F_K1;
    uint32_t* orow = P.occ + ((int64_t)(br * BH + bh) * nqt + qt) * P.occ_w;
    const bf16* khead = (const bf16*)P.in[kslot] + (int64_t)b * P.s[kslot][0] + (int64_t)h * P.s[kslot][1];
    const bf16* vhead = (const bf16*)P.in[F_V] + (int64_t)b * P.s[F_V][0] + (int64_t)h * P.s[F_V][1];
    const int64_t sk = P.s[kslot][2], sv = P.s[F_V][2];
    const __amdgpu_buffer_rsrc_t rn =
        make_rsrc(NORM ? P.norms + norm_base(P, br ? N_K2 : N_K1, bh) : nullptr, NORM ? (uint32_t)Nk * 4 : 0u);
    const float coef = br == 0 ? 1.f : -lam;
    bool have_q = false;
    bf16x8 Q[NT];
    float rq = 1.f;
    // pair list of (branch, head, query tile): npairs entries written so far (may pass the cap)
    const int64_t lidx = ((int64_t)br * BH + bh) * nqt + qt;
    uint32_t* pent = P.pairs ? P.pairs + lidx * (4 * kPairCap) : nullptr;
    uint32_t npairs = 0;
    for (int w = 0; w <= (klast >> 5); ++w) {
      const uint32_t bits0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)orow[w]);
      uint32_t bits = bits0, keep = bits0;
      while (bits) {
        const int kt = 32 * w + __builtin_ctz(bits);
        bits &= bits - 1u;
        ++checked;
        if (!have_q) {
          // query tile rows with whole-row loads, through the (still free) K tile buffer
          const bf16* qhead = (const bf16*)P.in[qslot] + (int64_t)b * P.s[qslot][0] + (int64_t)h * P.s[qslot][1];
          const __amdgpu_buffer_rsrc_t rq_ = tile_rsrc<D>(qhead, P.s[qslot][2], qt, Nq);
          u32x4 qr[VL];
#pragma unroll
          for (int i = 0; i < VL; ++i)
            qr[i] = buf_load16(rq_, (uint32_t)(((vrow + RPI * i) * P.s[qslot][2] + 8 * vch) * 2));
#pragma unroll
          for (int i = 0; i < VL; ++i) *reinterpret_cast<u32x4*>(ktl + (vrow + RPI * i) * KS + 8 * vch) = qr[i];
          wave_lds_sync();
          const bf16* qp = ktl + n32 * KS + 8 * g;
#pragma unroll
          for (int t = 0; t < NT; ++t) Q[t] = *reinterpret_cast<const bf16x8*>(qp + 16 * t);
          wave_lds_sync();
          if constexpr (NORM) rq = P.norms[norm_base(P, br ? N_Q2 : N_Q1, bh) + min(iq, Nq - 1)];
          have_q = true;
        }
        // loads of the key tile (A operand rows), the V tile and the key norms
        const __amdgpu_buffer_rsrc_t rk = tile_rsrc<D>(khead, sk, kt, Nk);
        const __amdgpu_buffer_rsrc_t rv = tile_rsrc<D>(vhead, sv, kt, Nk);
        // whole rows per load instruction (coalesced), staged through LDS like V
        u32x4 kr[VL];
#pragma unroll
        for (int i = 0; i < VL; ++i) kr[i] = buf_load16(rk, (uint32_t)(((vrow + RPI * i) * sk + 8 * vch) * 2));
        u32x4 vr[VL];
#pragma unroll
        for (int i = 0; i < VL; ++i) vr[i] = buf_load16(rv, (uint32_t)(((vrow + RPI * i) * sv + 8 * vch) * 2));
        f32x4 rk4[4] = {{1.f, 1.f, 1.f, 1.f}, {1.f, 1.f, 1.f, 1.f}, {1.f, 1.f, 1.f, 1.f}, {1.f, 1.f, 1.f, 1.f}};
        if constexpr (NORM) {
#pragma unroll
          for (int u = 0; u < 4; ++u)
            rk4[u] = __builtin_bit_cast(f32x4, buf_load16(rn, (uint32_t)(32 * kt + 8 * u + 4 * g) * 4));
        }
#pragma unroll
        for (int i = 0; i < VL; ++i) *reinterpret_cast<u32x4*>(ktl + (vrow + RPI * i) * KS + 8 * vch) = kr[i];
        wave_lds_sync();
        f32x16 S = {};
        const bf16* kp = ktl + n32 * KS + 8 * g;
#pragma unroll
        for (int t = 0; t < NT; ++t) S = PolBF16::mma(*reinterpret_cast<const bf16x8*>(kp + 16 * t), Q[t], S);
#pragma unroll
        for (int i = 0; i < VL; ++i) *reinterpret_cast<u32x4*>(vt + (vrow + RPI * i) * VS + 8 * vch) = vr[i];

        // exact weights: keys after the query's position and padding keys past Nk are masked
        // (only tiles reaching past the position of the tile's first row, or past Nk, have any)
        const bool edge = 32 * kt + 31 > min(qoff + 32 * qt, Nk - 1);
        f32x16 C;
        bool pos_any = false;
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * u + e;
            const float x = __builtin_fmaf(NORM ? S[r] * rk4[u][e] : S[r], rq, -tau);
            const int key = 32 * kt + crow(r, g);
            const bool pos = (!edge || (key <= pq && key < Nk)) && x > 0.f;
            C[r] = pos ? coef * pow_p<PK>(x, pw) : 0.f;
            pos_any |= pos;
            if (pent) {
              // list entry of each non-zero weight, in the order (value r, lane)
              const bool hit = valid && pos;
              const uint64_t bal = wave_ballot(hit);
              const uint32_t slot = npairs + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
              if (hit && slot < (uint32_t)kPairCap)
                *reinterpret_cast<u32x4*>(pent + 4 * slot) = u32x4{(uint32_t)key, (uint32_t)n32, __builtin_bit_cast(uint32_t, x), 0u};
              npairs += (uint32_t)__builtin_popcountll(bal);
            }
          }
        if (wave_ballot(valid && pos_any) == 0ull) {
          keep &= ~(1u << (kt & 31));
          continue;
        }
        ++computed;
        const bf16x8 PF0 = PolBF16::pack_c(C, 0), PF1 = PolBF16::pack_c(C, 1);
        wave_lds_sync();
        const bf16* vp = vt + voff;
#pragma unroll
        for (int c = 0; c < ND; ++c) {
          O[c] = PolBF16::mma(tr_frag<VS>(vp + 32 * c), PF0, O[c]);
          O[c] = PolBF16::mma(tr_frag<VS>(vp + 32 * c + 16 * VS), PF1, O[c]);
        }
        wave_lds_sync();
      }
      if (keep != bits0 && l == 0) orow[w] = keep;
    }
    if (pent && l == 0) P.pairs[pair_lists(P.nbr, BH, nqt) * 4 * kPairCap + lidx] = npairs;
  }

  // Output rows through LDS (the K tile buffer): lane (n, g) holds elements 32c + crow(r, g) of
  // row n; stores then cover whole rows, 16 bytes per lane.
  wave_lds_sync();
#pragma unroll
  for (int c = 0; c < ND; ++c)
#pragma unroll
    for (int u = 0; u < 4; ++u)
      store4(ktl + n32 * KS + 32 * c + 8 * u + 4 * g, O[c][4 * u], O[c][4 * u + 1], O[c][4 * u + 2], O[c][4 * u + 3]);
  wave_lds_sync();
  {
    bf16* ohead = (bf16*)P.out + (int64_t)b * P.s[F_OUT][0] + (int64_t)h * P.s[F_OUT][1];
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      const int r = vrow + RPI * i, row = 32 * qt + r;
      if (row < Nq)
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(ktl + r * KS + 8 * vch),
                                    reinterpret_cast<u32x4*>(ohead + (int64_t)row * P.s[F_OUT][2] + 8 * vch));
    }
  }
  if (P.stats && l == 0 && checked) {
    atomicAdd(P.stats + 1, (unsigned long long)computed);
    atomicAdd(P.stats + 2, (unsigned long long)checked);
  }
}

// Query tile of tile-pass item `item`: one head's query tiles consecutive on one XCD (when the
// heads fill the eight XCDs), longest (last query tile) first.
__device__ __forceinline__ void pv_item(int item, int BH, int nqt, int& bh, int& qt) {
  if (BH % 8 == 0) {
    const int x = item & 7, j = item >> 3;
    bh = x + 8 * (j / nqt);
    qt = nqt - 1 - j % nqt;
  } else {
    bh = item / nqt;
    qt = nqt - 1 - item % nqt;
  }
}

// One wave per workgroup and `per_wave` consecutive items per wave: the work per query tile
// varies with its number of non-zero tiles, and single-wave workgroups retire independently.
// With candidate lists (normalised bf16) the items whose lists all fit belong to fwd_pv_cand:
// the wave tests its items' counts in one lane-parallel round and runs only the others, so a
// launch where every list fits costs a few waves per SIMD (per_wave 4) instead of one per
// query tile; without lists every item runs (per_wave 1).
// With the candidate pass's queue (per_wave 0), the waves take the queued query tiles in turn.
template <int D, int BR, int PK, bool NORM>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(2))) fwd_pv(FwdParams P, int per_wave) {
  constexpr int VS = D + 32, KS = D + 8;
  __shared__ __attribute__((aligned(16))) bf16 vst[32 * VS];
  __shared__ __attribute__((aligned(16))) bf16 kst[32 * KS];
  const int l = lane_id();
  const int BH = P.B * P.H, nqt = P.nqt, n = BH * nqt;
  if (per_wave == 0) {
    const uint32_t queued = P.pvq[0];
    for (uint32_t k = blockIdx.x; k < queued; k += gridDim.x) {
      const int v = (int)P.pvq[1 + k];
      fwd_pv_tile<D, BR, PK, NORM>(P, vst, kst, v / nqt, v % nqt);
    }
    return;
  }
  const int first = (int)blockIdx.x * per_wave;
  bool need = false;
  if (l < per_wave && first + l < n) {
    int bh, qt;
    pv_item(first + l, BH, nqt, bh, qt);
    need = true;
    if (NORM && P.cand) {
      const uint32_t* counts = P.cand + pair_lists(BR, BH, nqt) * kCandCap;
      bool fit = true;
#pragma unroll
      for (int br = 0; br < BR; ++br) fit = fit && counts[((int64_t)br * BH + bh) * nqt + qt] <= (uint32_t)kCandCap;
      need = !fit;
    }
  }
  for (uint64_t m = wave_ballot(need); m; m &= m - 1ull) {
    int bh, qt;
    pv_item(first + __builtin_ctzll(m), BH, nqt, bh, qt);
    fwd_pv_tile<D, BR, PK, NORM>(P, vst, kst, bh, qt);
  }
}

// ------------------------------------------------------------------ fwd_pv_cand
// The exact pass of the query tiles whose candidate-key lists (every branch, normalised scores)
// fit: per branch the score tile of the query rows against the candidate keys' rows (row c =
// candidate c, rows past the count zero) is computed with the MFMA sequence of fwd_pv, its
// operands loaded straight from the rows (the same values in the same operands: bitwise the same
// scores); the candidates' V rows go to a swizzled LDS tile by direct loads, and the exact
// weights with the causal mask accumulate out += coef A V as in fwd_pv.  One gather round
// per branch replaces one per kept key tile.  The bitmask row is rewritten from the key tiles
// holding a non-zero weight; the pair list takes the non-zero weights in the order (value r,
// lane).
template <int D, int BR, int PK>
__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(3))) fwd_pv_cand(FwdParams P) {
  constexpr int NT = D / 16, ND = D / 32;
  constexpr int CPR = D / 8;     // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;  // rows per load instruction
  constexpr int VL = 32 / RPI;   // load instructions per tile
  __shared__ __attribute__((aligned(16))) bf16 vt[32 * D];  // V rows, chunk-swizzled (bswz)
  __shared__ __attribute__((aligned(16))) int ckey[32];     // candidate keys (padding: -1)
  __shared__ __attribute__((aligned(16))) float crk[32];   // their inverse norms

  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int BH = P.B * P.H, Nq = P.Nq, Nk = P.Nk, nqt = P.nqt, qoff = P.qoff;
  int bh, qt;
  {
    const int bid = blockIdx.x;
    // one head's query tiles consecutive on one XCD, early tiles (lowest thresholds, the most
    // candidates) first
    if (BH % 8 == 0) {
      const int x = bid & 7, j = bid >> 3;
      bh = x + 8 * (j / nqt);
      qt = j % nqt;
    } else {
      bh = bid / nqt;
      qt = bid % nqt;
    }
  }
  if (bh >= BH) return;
  // the counts of every branch and, in the same round, every list slot (lanes 0-31: branch 0,
  // lanes 32-63: branch 1; slots past a count are never used)
  const uint32_t* counts = P.cand + pair_lists(BR, BH, nqt) * kCandCap;
  uint32_t nc[BR];
#pragma unroll
  for (int br = 0; br < BR; ++br) nc[br] = counts[((int64_t)br * BH + bh) * nqt + qt];
  const int kraw = (int)P.cand[(((int64_t)(BR == 2 ? (l >> 5) : 0) * BH + bh) * nqt + qt) * kCandCap + (l & 31)];
  bool fit = true;
#pragma unroll
  for (int br = 0; br < BR; ++br) fit = fit && nc[br] <= (uint32_t)kCandCap;
  if (!fit) {  // fwd_pv walks the bitmask tiles
    if (l == 0) P.pvq[1 + atomicAdd(P.pvq, 1u)] = (uint32_t)(bh * nqt + qt);
    return;
  }

  const int b = bh / P.H, h = bh % P.H;
  const int iq = 32 * qt + n32;
  const bool valid = iq < Nq;
  const int pq = qoff + iq;                    // the lane's query position
  const int klast = kt_last(qt, qoff, P.nkt);  // last key tile the query tile sees
  const int nw = (klast >> 5) + 1;             // bitmask words of the row
  const float tau = *P.beta * tau_coeff(pq, P.inv_d);
  const float pw = P.p;
  float lam = 0.f;
  if constexpr (BR == 2) lam = clamp01(*P.lam);
  const int vrow = l / CPR, vch = l % CPR;

  f32x16 O[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) O[c] = f32x16{};
  unsigned computed = 0, checked = 0;

#pragma unroll
  for (int br = 0; br < BR; ++br) {
    const uint32_t n = nc[br];
    const int64_t lidx = ((int64_t)br * BH + bh) * nqt + qt;
    uint32_t* orow = P.occ + lidx * P.occ_w;
    uint32_t npairs = 0;
    if (n > 0) {
      const int qslot = br ? F_Q2 : F_Q1, kslot = br ? F_K2 : F_K1;
      const bf16* qhead = (const bf16*)P.in[qslot] + (int64_t)b * P.s[qslot][0] + (int64_t)h * P.s[qslot][1];
      const bf16* khead = (const bf16*)P.in[kslot] + (int64_t)b * P.s[kslot][0] + (int64_t)h * P.s[kslot][1];
      const bf16* vhead = (const bf16*)P.in[F_V] + (int64_t)b * P.s[F_V][0] + (int64_t)h * P.s[F_V][1];
      const int64_t sq = P.s[qslot][2], sk = P.s[kslot][2], sv = P.s[F_V][2];
      const float coef = br == 0 ? 1.f : -lam;
      const int kb = __shfl(kraw, (32 * br + (l & 31)) & 63);  // this branch's slots: lanes 32 br ..
      const int key_l = l < (int)n && kb >= 0 && kb < Nk ? kb : -1;  // the screen lists keys < Nk only
      const float rk_l = key_l >= 0 ? P.norms[norm_base(P, br ? N_K2 : N_K1, bh) + key_l] : 0.f;
      const float rq = P.norms[norm_base(P, br ? N_Q2 : N_Q1, bh) + min(iq, Nq - 1)];
      // Every load of the branch in one round.  The operands of the score MFMAs straight from
      // the rows (lane (m, g): elements 16 t + 8 g .. of query row m, and of candidate m's key
      // row): no LDS staging.  V rows by direct global->LDS loads into the swizzled tile (rows
      // past the count take candidate 0's row, zeroed below).
      const int key_m = __shfl(key_l, n32);
      const int key0 = max(__builtin_amdgcn_readfirstlane(key_l), 0);  // a row every lane may load
      const bf16* qrow = qhead + (int64_t)min(iq, Nq - 1) * sq;
      const bf16* krow = khead + (int64_t)(key_m >= 0 ? key_m : key0) * sk;
      bf16x8 Q[NT], K[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        Q[t] = *reinterpret_cast<const bf16x8*>(qrow + 16 * t + 8 * g);
        K[t] = *reinterpret_cast<const bf16x8*>(krow + 16 * t + 8 * g);
      }
      wave_lds_sync();  // the previous branch's reads of the tile are done
#pragma unroll
      for (int u = 0; u < VL; ++u) {
        const int r = u * RPI + l / CPR;
        const int key = __shfl(key_l, r);
        const int c = (l % CPR) ^ bswz<D>(r);
        __builtin_amdgcn_global_load_lds((const void*)(vhead + (int64_t)(key >= 0 ? key : key0) * sv + 8 * c),
                                         LDS_PTR(void, vt + u * RPI * D), 16, 0, 0);
      }
      if (l < 32) {
        ckey[l] = key_l;
        crk[l] = rk_l;
      }
      __builtin_amdgcn_s_waitcnt(0);
      if (n < 32u) {  // rows past the count: zeros (their weights are zero; keep them finite)
#pragma unroll
        for (int u = 0; u < VL; ++u) {
          const int r = u * RPI + l / CPR;
          if (r >= (int)n) *reinterpret_cast<u32x4*>(vt + r * D + 8 * (l % CPR)) = u32x4{0u, 0u, 0u, 0u};
        }
      }
      wave_lds_sync();
      f32x16 S = {};
#pragma unroll
      for (int t = 0; t < NT; ++t) S = PolBF16::mma(key_m >= 0 ? K[t] : bf16x8{}, Q[t], S);
      // value r of the lane: candidate crow(r, g)
      f32x4 rk4[4];
      u32x4 key4[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        rk4[u] = *reinterpret_cast<const f32x4*>(crk + 8 * u + 4 * g);
        key4[u] = *reinterpret_cast<const u32x4*>(ckey + 8 * u + 4 * g);
      }
      uint32_t* pent = P.pairs ? P.pairs + lidx * (4 * kPairCap) : nullptr;
      uint32_t cnz = 0u;  // candidates with a non-zero weight
      f32x16 C;
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * u + e;
          const int key = (int)key4[u][e];
          const float x = __builtin_fmaf(S[r] * rk4[u][e], rq, -tau);
          const bool pos = key >= 0 && key <= pq && key < Nk && x > 0.f;
          C[r] = pos ? coef * pow_p<PK>(x, pw) : 0.f;
          const bool hit = valid && pos;
          const uint64_t bal = wave_ballot(hit);
          cnz |= ((uint32_t)bal ? 1u << crow(r, 0) : 0u) | ((uint32_t)(bal >> 32) ? 1u << crow(r, 1) : 0u);
          if (pent) {
            const uint32_t slot = npairs + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                                     __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
            if (hit && slot < (uint32_t)kPairCap)
              *reinterpret_cast<u32x4*>(pent + 4 * slot) = u32x4{(uint32_t)key, (uint32_t)n32, __builtin_bit_cast(uint32_t, x), 0u};
            npairs += (uint32_t)__builtin_popcountll(bal);
          }
        }
      if (cnz) {
        const bf16x8 PF0 = PolBF16::pack_c(C, 0), PF1 = PolBF16::pack_c(C, 1);
#pragma unroll
        for (int c = 0; c < ND; ++c) {
          O[c] = PolBF16::mma(tile_tr_frag<D>(vt, 0, c), PF0, O[c]);
          O[c] = PolBF16::mma(tile_tr_frag<D>(vt, 1, c), PF1, O[c]);
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
      wave_lds_sync();  // the tiles are reused by the next branch and the output
    }
    if (P.pairs && l == 0) P.pairs[pair_lists(P.nbr, BH, nqt) * 4 * kPairCap + lidx] = npairs;
  }

  // Output rows through LDS (the swizzled V tile): lane (n, g) holds elements 32c + crow(r, g) of
  // row n, i.e. half g of chunk 4c + u for values 4u .. 4u + 3; stores then cover whole rows
  // (streaming stores, as in fwd_pv: nothing here reads the output again).
  wave_lds_sync();
#pragma unroll
  for (int c = 0; c < ND; ++c)
#pragma unroll
    for (int u = 0; u < 4; ++u)
      store4(vt + n32 * D + 8 * ((4 * c + u) ^ bswz<D>(n32)) + 4 * g, O[c][4 * u], O[c][4 * u + 1], O[c][4 * u + 2],
             O[c][4 * u + 3]);
  wave_lds_sync();
  {
    bf16* ohead = (bf16*)P.out + (int64_t)b * P.s[F_OUT][0] + (int64_t)h * P.s[F_OUT][1];
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      const int r = vrow + RPI * i, row = 32 * qt + r;
      if (row < Nq)
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(vt + r * D + 8 * (vch ^ bswz<D>(r))),
                                    reinterpret_cast<u32x4*>(ohead + (int64_t)row * P.s[F_OUT][2] + 8 * vch));
    }
  }
  if (P.stats) {
    const float cs = wave_sum((float)computed), ks = wave_sum((float)checked);
    if (l == 0 && ks > 0.f) {
      atomicAdd(P.stats + 1, (unsigned long long)cs);
      atomicAdd(P.stats + 2, (unsigned long long)ks);
    }
  }
}

// ------------------------------------------------------------------ dispatch
template <int D, int BR, int PK, bool NORM>
int launch_sparse_t(const FwdParams& p, hipStream_t s) {
  const int BH = p.B * p.H;
  if constexpr (NORM) {
    constexpr int rows = (64 / (D / 8)) * KN_GROUPS;  // rows per wave
    const int64_t waves = (int64_t)BR * BH * ((p.Nk + rows - 1) / rows);
    hipLaunchKernelGGL(key_norms<D>, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, p, BR);
    launched(s, "key_norms");
  }
  const unsigned nqb = (unsigned)((p.Nq + 255) / 256);
  constexpr int QPW = 2, TPB = 1;
  hipLaunchKernelGGL((fwd_screen<D, NORM, QPW, TPB>), dim3((unsigned)(BR * BH) * nqb), dim3(512 / QPW), 0, s, p, BR);
  launched(s, "fwd_screen");
  if (NORM && p.cand) {
    hipLaunchKernelGGL((fwd_pv_cand<D, BR, PK>), dim3((unsigned)(BH * p.nqt)), dim3(64), 0, s, p);
    launched(s, "fwd_pv_cand");
  }
  if (NORM && p.cand) {  // the query tiles the candidate pass could not take, from its queue
    const int items = BH * p.nqt;
    hipLaunchKernelGGL((fwd_pv<D, BR, PK, NORM>), dim3((unsigned)(items < 2048 ? items : 2048)), dim3(64), 0, s, p, 0);
  } else {
    hipLaunchKernelGGL((fwd_pv<D, BR, PK, NORM>), dim3((unsigned)(BH * p.nqt)), dim3(64), 0, s, p, 1);
  }
  launched(s, "fwd_pv");
  return (int)hipGetLastError();
}

template <int D, int BR, int PK>
int sel_norm(const FwdParams& p, const KernelKey& k, hipStream_t s) {
  return k.normalize ? launch_sparse_t<D, BR, PK, true>(p, s) : launch_sparse_t<D, BR, PK, false>(p, s);
}
template <int D, int BR>
int sel_pk(const FwdParams& p, const KernelKey& k, hipStream_t s) {
  switch (k.pkind) {
    case 2: return sel_norm<D, BR, 2>(p, k, s);
    case 1: return sel_norm<D, BR, 1>(p, k, s);
    default: return sel_norm<D, BR, 0>(p, k, s);
  }
}
template <int D>
int sel_br(const FwdParams& p, const KernelKey& k, hipStream_t s) {
  return k.branches == 2 ? sel_pk<D, 2>(p, k, s) : sel_pk<D, 1>(p, k, s);
}

}  // namespace

int launch_fwd_sparse(const FwdParams& p, const KernelKey& k, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  return k.d == 128 ? sel_br<128>(p, k, s) : sel_br<64>(p, k, s);
}

}  // namespace tda
