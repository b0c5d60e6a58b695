// tda_fwd_fast.hip -- LDS-staged bf16 forward of threshold attention for gfx950.
//
// Reference semantics: snap-research/TDA triton_threshold_attention.py forward kernel
// (TTA:19-115) and the differential composition (TTA:489-519).
//
// Workgroup = 4 waves x 64 query rows (two 32-row query tiles per wave), 256 rows in all.
// The key loop runs once per branch (K1, then K2); both passes accumulate into the same
// output registers, O += A1 V and then O += (-lam A2) V, so only one branch's query fragments
// are resident at a time.  Key tiles of 32 rows go through a 2-stage LDS ring: each thread
// fetches its share of the next K/V tile into VGPRs while the current tile is consumed, then
// writes it to the other stage.  Per key tile and wave:
//   S^T(query tile) = K Q^T on the matrix cores (K row fragments from LDS, Q resident in
//   registers); the tile max of S^T * rk is thresholded per lane and a ballot decides whether
//   any score of the tile is non-zero; only then is the weight tile packed to bf16 and
//   O^T += V^T A^T issued, with V^T read straight from the row-major tile by the LDS
//   transpose read.  O never leaves the accumulators until the epilogue.
// The key inverse norms come from a small prologue kernel (row_inv_norms).
//
// LDS rows are padded (K: 2D+16 bytes, V: 2D+64 bytes) so that every fragment address is one
// per-lane base plus an immediate offset and both the 16-byte row-fragment reads and the
// transpose reads avoid bank conflicts (64 banks).
#include "tda_common.hpp"
#include "tda_params.hpp"

#include <type_traits>

namespace tda {

#define LDS_PTR(T, p) ((__attribute__((address_space(3))) T*)(p))

template <int D>
struct FastLayout {
  static constexpr int KS = D + 8;    // K row stride (elements)
  static constexpr int VS = D + 32;   // V row stride (elements)
  static constexpr int TPR = D / 16;  // staging threads per row (2 chunks of 8 each)
};

template <int D>
struct FastStage {
  bf16 k[32 * FastLayout<D>::KS];
  bf16 v[32 * FastLayout<D>::VS];
  float rk[32];
};

// Staging registers: thread t owns tile row t / TPR and 16 consecutive elements starting at
// 16 * (t % TPR); D = 128 uses all 256 threads, D = 64 threads 0..127.
struct Chunk2 {
  bf16x8 v[2];
};

// Transposed A fragments of one 32-column block for both 16-row steps, from a row-major
// tile with row stride VS: lane (n, g) gets column n of the block at tile rows
// crow(8*st + j, g), j = 0..7 -- two transpose reads per step.  Inline assembly with its own
// lgkmcnt wait, so that the compiler does not treat it as aliasing the staging traffic.
template <int D>
__device__ __forceinline__ void lds_tr_frags(uint32_t base, bf16x8& f0, bf16x8& f1) {
  constexpr int VS = FastLayout<D>::VS;
  typedef int i2 __attribute__((ext_vector_type(2)));
  typedef int i4 __attribute__((ext_vector_type(4)));
  i2 r0, r1, r2, r3;
  asm volatile(
      "ds_read_b64_tr_b16 %0, %4\n\t"
      "ds_read_b64_tr_b16 %1, %4 offset:%5\n\t"
      "ds_read_b64_tr_b16 %2, %4 offset:%6\n\t"
      "ds_read_b64_tr_b16 %3, %4 offset:%7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(r0), "=&v"(r1), "=&v"(r2), "=&v"(r3)
      : "v"(base), "i"(2 * 8 * VS), "i"(2 * 16 * VS), "i"(2 * 24 * VS));
  f0 = __builtin_bit_cast(bf16x8, i4{r0[0], r0[1], r1[0], r1[1]});
  f1 = __builtin_bit_cast(bf16x8, i4{r2[0], r2[1], r3[0], r3[1]});
}

template <int D, int BR, int PK, bool NORM>
__global__ void __launch_bounds__(256, 1) fwd_fast(FwdParams P) {
  constexpr int NT = D / 16;  // MFMA steps over d
  constexpr int ND = D / 32;  // 32-column output blocks
  constexpr int KS = FastLayout<D>::KS, VS = FastLayout<D>::VS, TPR = FastLayout<D>::TPR;
  using Stage = FastStage<D>;
  __shared__ __attribute__((aligned(16))) Stage stage[2];

  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR) by construction
  const int BH = P.B * P.H;
  const int N = P.N;
  const int nqb = (N + 255) / 256;
  int bh, qb;
  {
    const int bid = blockIdx.x;
    if (BH % 8 == 0) {  // XCD-aware: all query blocks of a head on one XCD (one L2), longest first
      const int x = bid & 7, j = bid >> 3, hp = BH >> 3;
      qb = nqb - 1 - j / hp;
      bh = x + 8 * (j % hp);
    } else {
      qb = nqb - 1 - bid / BH;
      bh = bid % BH;
    }
  }
  const int b = bh / P.H, h = bh % P.H;
  const int q0w = qb * 256 + 64 * wv;                     // first row of this wave
  const int qt0 = q0w >> 5;                               // this wave's query tiles: qt0, qt0 + 1
  const int nkt = min(P.nqt, (qb * 256 + 255) / 32 + 1);  // key tiles per pass
  const int nit = BR * nkt;                               // loop length over both passes

  auto base = [&](int slot) {
    return (const bf16*)P.in[slot] + (int64_t)b * P.s[slot][0] + (int64_t)h * P.s[slot][1];
  };

  // staging: this thread's row and chunk pair within a key tile
  const int srow = tid / TPR, scol = 16 * (tid % TPR);
  const bool stager = tid < 32 * TPR;
  const bf16* ks0 = base(F_K1) + scol;
  const bf16* ks1 = base(F_K2) + scol;
  const bf16* vs = base(F_V) + scol;
  const int64_t sk0 = P.s[F_K1][2], sk1 = P.s[F_K2][2], sv = P.s[F_V][2];
  const float* nk0 = NORM ? P.norms + ((int64_t)N_K1 * BH + bh) * N : nullptr;
  const float* nk1 = NORM ? P.norms + ((int64_t)N_K2 * BH + bh) * N : nullptr;

  Chunk2 rK, rV;
  float rRk = 0.f;
  auto fetch = [&](int it) {
    const bool second = it >= nkt;
    const int kt = second ? it - nkt : it;
    const int row = min(kt * 32 + srow, N - 1);  // rows >= N only ever meet zero scores
    if (stager) {
      const bf16* a = second ? ks1 + row * sk1 : ks0 + row * sk0;
      rK.v[0] = *reinterpret_cast<const bf16x8*>(a);
      rK.v[1] = *reinterpret_cast<const bf16x8*>(a + 8);
      const bf16* e = vs + row * sv;
      rV.v[0] = *reinterpret_cast<const bf16x8*>(e);
      rV.v[1] = *reinterpret_cast<const bf16x8*>(e + 8);
    }
    if constexpr (NORM) {
      if (tid < 32) rRk = (second ? nk1 : nk0)[min(kt * 32 + tid, N - 1)];
    }
  };
  auto commit = [&](Stage& s) {
    if (stager) {
      bf16* k = s.k + srow * KS + scol;
      *reinterpret_cast<bf16x8*>(k) = rK.v[0];
      *reinterpret_cast<bf16x8*>(k + 8) = rK.v[1];
      bf16* v = s.v + srow * VS + scol;
      *reinterpret_cast<bf16x8*>(v) = rV.v[0];
      *reinterpret_cast<bf16x8*>(v + 8) = rV.v[1];
    }
    if constexpr (NORM) {
      if (tid < 32) s.rk[tid] = rRk;
    }
  };

  fetch(0);

  const float beta = *P.beta;
  const float pw = P.p;
  float lam = 0.f;
  if constexpr (BR == 2) lam = clamp01(*P.lam);
  float tau[2];
#pragma unroll
  for (int s = 0; s < 2; ++s) tau[s] = beta * tau_coeff(q0w + 32 * s + n32, P.inv_d);

  // Query fragments of the current branch (resident B operands) and their inverse norms.
  bf16x8 Q[2][NT];
  float rq[2] = {1.f, 1.f};
  auto load_q = [&](int br) {
    const int slot = br == 0 ? F_Q1 : F_Q2;
    const bf16* qb_ = base(slot);
    const int64_t sq = P.s[slot][2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int iq = q0w + 32 * s + n32;
      const bf16* r = qb_ + min(iq, N - 1) * sq;  // rows >= N: any valid row, never stored
#pragma unroll
      for (int t = 0; t < NT; ++t) Q[s][t] = *reinterpret_cast<const bf16x8*>(r + 16 * t + 8 * g);
      if constexpr (NORM) {
        rq[s] = inv_norm(row_sumsq<PolBF16, NT>(Q[s]));
        if (g == 0 && iq < N) P.norms[((int64_t)(br == 0 ? N_Q1 : N_Q2) * BH + bh) * N + iq] = rq[s];
      }
    }
  };
  load_q(0);

  commit(stage[0]);
  __syncthreads();

  f32x16 O[2][ND];
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int c = 0; c < ND; ++c) O[s][c] = f32x16{};
  uint32_t word[2] = {0u, 0u};
  unsigned visited = 0, computed = 0;
  uint32_t* occ = P.occ;

  // per-lane LDS offsets (elements) inside a stage
  const int koff = n32 * KS + 8 * g;  // row fragment: row n32, elements 8g..
  const int rkoff = 4 * g;            // key norms of this lane's C rows
  const int bk = l >> 4, jj = l & 15;
  const int voff = (4 * (bk >> 1) + (jj >> 2)) * VS + 16 * (bk & 1) + 4 * (jj & 3);  // transpose read

  for (int it = 0; it < nit; ++it) {
    const int br = it >= nkt ? 1 : 0;
    const int kt = it - br * nkt;
    Stage& cur = stage[it & 1];
    if (BR == 2 && it == nkt) load_q(1);  // second pass: swap in the q2 fragments
    if (it + 1 < nit) fetch(it + 1);

    if (kt <= qt0 + 1) {  // some query tile of this wave sees key tile kt
      f32x16 S[2] = {f32x16{}, f32x16{}};
      const bf16* kp = cur.k + koff;
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        const bf16x8 fk = *reinterpret_cast<const bf16x8*>(kp + 16 * t);
        S[0] = PolBF16::mma(fk, Q[0][t], S[0]);
        S[1] = PolBF16::mma(fk, Q[1][t], S[1]);
      }
      // Tile max of s * rk per lane (query).  x = fma(s * rk, rq, -tau) is monotone in
      // s * rk, so "max > threshold" is exactly "some x > 0".
      const int kq = 32 * kt;
      float m[2] = {-INFINITY, -INFINITY};
      auto tile_max = [&](auto masked) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          f32x4 rk4 = {1.f, 1.f, 1.f, 1.f};
          if constexpr (NORM) rk4 = *reinterpret_cast<const f32x4*>(&cur.rk[8 * u] + rkoff);
#pragma unroll
          for (int s = 0; s < 2; ++s)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int r = 4 * u + e;
              float v = NORM ? S[s][r] * rk4[e] : S[s][r];
              if constexpr (decltype(masked)::value)
                if (kq + crow(r, g) > q0w + 32 * s + n32) v = -INFINITY;
              m[s] = fmaxf(m[s], v);
            }
        }
      };
      if (kt < qt0) tile_max(std::false_type{});  // every key precedes every query
      else tile_max(std::true_type{});            // diagonal tiles: mask keys after the query
      bool any[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        any[s] = wave_ballot(__builtin_fmaf(m[s], rq[s], -tau[s]) > 0.f) != 0ull;
        if (kt <= qt0 + s && qt0 + s < P.nqt) ++visited;
        if (any[s]) {
          word[s] |= 1u << (kt & 31);
          ++computed;
        }
      }
      if (any[0] || any[1]) {
        const float coef = br == 0 ? 1.f : -lam;
        bf16x8 PF[2][2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          f32x16 C;
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            f32x4 rk4 = {1.f, 1.f, 1.f, 1.f};
            if constexpr (NORM) rk4 = *reinterpret_cast<const f32x4*>(&cur.rk[8 * u] + rkoff);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int r = 4 * u + e;
              const bool keep = kq + crow(r, g) <= q0w + 32 * s + n32;
              const float x = __builtin_fmaf(NORM ? S[s][r] * rk4[e] : S[s][r], rq[s], -tau[s]);
              C[r] = (keep && x > 0.f) ? coef * pow_p<PK>(x, pw) : 0.f;
            }
          }
          PF[s][0] = PolBF16::pack_c(C, 0);
          PF[s][1] = PolBF16::pack_c(C, 1);
        }
        const uint32_t vbase = (uint32_t)(size_t)LDS_PTR(const bf16, cur.v + voff);
#pragma unroll
        for (int c = 0; c < ND; ++c) {
          bf16x8 va0, va1;
          lds_tr_frags<D>(vbase + 64 * c, va0, va1);
          if (any[0]) {
            O[0][c] = PolBF16::mma(va0, PF[0][0], O[0][c]);
            O[0][c] = PolBF16::mma(va1, PF[0][1], O[0][c]);
          }
          if (any[1]) {
            O[1][c] = PolBF16::mma(va0, PF[1][0], O[1][c]);
            O[1][c] = PolBF16::mma(va1, PF[1][1], O[1][c]);
          }
        }
      }
    }
    // bitmask words of this wave's query tiles for branch br: word kt/32 is complete after
    // key tile kt; layout [branch][B*H][query tile][word]
    if (occ && (((kt & 31) == 31) || kt == nkt - 1)) {
      if (l == 0) {
        const int64_t row0 = (((int64_t)br * BH + bh) * P.nqt + qt0) * P.occ_w;
        if (qt0 < P.nqt) occ[row0 + (kt >> 5)] = word[0];
        if (qt0 + 1 < P.nqt) occ[row0 + P.occ_w + (kt >> 5)] = word[1];
        if (kt == nkt - 1) {  // words of key tiles the workgroup never visits
          for (int w = (kt >> 5) + 1; w < P.occ_w; ++w) {
            if (qt0 < P.nqt) occ[row0 + w] = 0u;
            if (qt0 + 1 < P.nqt) occ[row0 + P.occ_w + w] = 0u;
          }
        }
      }
      word[0] = word[1] = 0u;
    }
    if (it + 1 < nit) commit(stage[(it + 1) & 1]);
    __syncthreads();
  }

  bf16* ob = (bf16*)P.out + (int64_t)b * P.s[F_OUT][0] + (int64_t)h * P.s[F_OUT][1];
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int i = q0w + 32 * s + n32;
    if (i < N) {
      bf16* orow = ob + i * P.s[F_OUT][2];
#pragma unroll
      for (int c = 0; c < ND; ++c)
#pragma unroll
        for (int u = 0; u < 4; ++u)
          store4(orow + 32 * c + 8 * u + 4 * g, O[s][c][4 * u], O[s][c][4 * u + 1], O[s][c][4 * u + 2],
                 O[s][c][4 * u + 3]);
    }
  }
  if (P.stats && l == 0) {
    atomicAdd(P.stats + 0, (unsigned long long)visited);
    atomicAdd(P.stats + 1, (unsigned long long)computed);
  }
}

// Inverse L2 norms 1/max(|x|, eps) of the rows of k1 (and k2) into the norms table.
// One 16-lane group per row (8 bf16 per lane), rows in order.
template <int D>
__global__ void __launch_bounds__(256) row_inv_norms(FwdParams P, int branches) {
  const int BH = P.B * P.H, N = P.N;
  const int64_t rows = (int64_t)BH * N;
  const int lane16 = threadIdx.x & 15;
  const int64_t gid = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 4;  // row id over branches
  const int br = (int)(gid / rows);
  const int64_t rid = gid - (int64_t)br * rows;
  float ss = 0.f;
  const bool ok = br < branches;
  if (ok) {
    const int slot = br == 0 ? F_K1 : F_K2;
    const int bh = (int)(rid / N), t = (int)(rid % N);
    const TRef<const bf16> x{(const bf16*)P.in[slot], P.s[slot][0], P.s[slot][1], P.s[slot][2]};
    const bf16* row = x.row(bh / P.H, bh % P.H, t);
    for (int c = lane16; c < D / 8; c += 16) {
      const bf16x8 v = *reinterpret_cast<const bf16x8*>(row + 8 * c);
#pragma unroll
      for (int e = 0; e < 8; ++e) { const float f = (float)v[e]; ss = __builtin_fmaf(f, f, ss); }
    }
  }
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) ss += __shfl_xor(ss, o);
  if (ok && lane16 == 0) P.norms[(int64_t)(br == 0 ? N_K1 : N_K2) * rows + rid] = inv_norm(ss);
}

// ------------------------------------------------------------------ dispatch
template <int D, int BR, int PK, bool NORM>
static int launch_fast_t(const FwdParams& p, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  const int BH = p.B * p.H;
  if constexpr (NORM) {
    const int64_t rows = (int64_t)BH * p.N * BR;
    hipLaunchKernelGGL(row_inv_norms<D>, dim3((unsigned)((rows * 16 + 255) / 256)), dim3(256), 0, s, p, BR);
  }
  const unsigned grid = (unsigned)BH * (unsigned)((p.N + 255) / 256);
  hipLaunchKernelGGL((fwd_fast<D, BR, PK, NORM>), dim3(grid), dim3(256), 0, s, p);
  return (int)hipGetLastError();
}

template <int D, int BR, int PK>
static int fsel_norm(const FwdParams& p, const KernelKey& k, void* s) {
  return k.normalize ? launch_fast_t<D, BR, PK, true>(p, s) : launch_fast_t<D, BR, PK, false>(p, s);
}
template <int D, int BR>
static int fsel_pk(const FwdParams& p, const KernelKey& k, void* s) {
  switch (k.pkind) {
    case 2: return fsel_norm<D, BR, 2>(p, k, s);
    case 1: return fsel_norm<D, BR, 1>(p, k, s);
    default: return fsel_norm<D, BR, 0>(p, k, s);
  }
}
template <int D>
static int fsel_br(const FwdParams& p, const KernelKey& k, void* s) {
  return k.branches == 2 ? fsel_pk<D, 2>(p, k, s) : fsel_pk<D, 1>(p, k, s);
}

int launch_fwd_fast(const FwdParams& p, const KernelKey& k, void* stream) {
  return k.d == 128 ? fsel_br<128>(p, k, stream) : fsel_br<64>(p, k, stream);
}

}  // namespace tda
