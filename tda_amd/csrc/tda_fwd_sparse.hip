// tda_fwd_sparse.hip -- bf16 forward of threshold attention for gfx950, built around the
// sparsity of the weights: with cosine scores and tau_i = beta sqrt(2 ln(i+1)/d), only a few
// percent of the 32x32 (query tile, key tile) weight blocks hold a non-zero entry.
//
// Reference semantics: snap-research/TDA triton_threshold_attention.py forward kernel
// (TTA:19-115: scores, threshold, ReLU^p, causal mask, A.V) and the differential composition
// out = A1 V - clamp(lambda, 0, 1) A2 V (TTA:489-519).
//
// Launches, in stream order, with normalisation:
//   key_prep    inverse L2 norms rk_j of the key rows into the norms table, and the normalised
//               key rows quantised to int8 with a per-row scale and residual bound.
//   fwd_screen  (fwd_screen_i8) for every causal (query tile, key tile) pair of a branch, an int8
//               score tile of the quantised normalised rows on the matrix cores and a test that
//               carries a bound on the quantisation residuals: it keeps every tile holding a
//               non-zero weight (x_ij = fma(s_ij rk_j, rq_i, -tau_i) > 0 for some pair) and may
//               keep tiles and keys whose weights are all zero.  No V and no output
//               accumulators, so several waves share a SIMD.  It also lists each query tile's
//               candidate keys (the keys of its passing lanes).
//   fwd_pv_cand one wave per branch of a query tile whose candidate lists fit: the score tile
//               of its rows against the candidate keys (the same MFMA sequence and operand
//               values as fwd_pv, so the same scores), the exact weights and coef A V over the
//               candidates' V rows, the branches' sums added through LDS; the bitmask row is
//               rewritten exactly.  Query tiles whose lists overflow go to a queue for fwd_pv.
//   fwd_pv      the tile pass for the queued query tiles, one wave per query tile: walks the set
//               bits of both branches, recomputes the score tile, forms the exact weights
//               ReLU(x)^p with the causal mask, and accumulates out += coef A V.  Tiles whose
//               exact weights are all zero lose their bit, so the bitmask ends exact.
// Without normalisation one launch, fwd_pv_blk: every query tile, four per workgroup sharing
// each key tile's rows, scores every causal key tile and forms the weights, A V and the exact
// bitmask itself (a screen would compute the same bf16 scores once more); its workgroups also
// clear the call's zero range, a share each after their own tiles.
// The screen tests every key of the tile, including keys after the query on the diagonal tile:
// it may keep a tile the mask empties, never drop a non-zero one.  Padding keys are cleared from
// the hit bits, so no candidate list names a key row past Nk.
#include <type_traits>

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

// Descriptor over the whole (N, D) head, for tile loads at a per-tile offset added to the lane's
// offset (the range check covers the vector offset only): rows past N read as zeros.  Usable
// when the byte offsets of 32 ceil(N / 32) rows stay below 2^31 (head_fits).
template <int D>
__device__ __forceinline__ __amdgpu_buffer_rsrc_t head_rsrc(const bf16* head, int64_t stride, int N) {
  return make_rsrc(head, (uint32_t)(((int64_t)(N - 1) * stride + D) * 2));
}
__device__ __forceinline__ bool head_fits(int64_t stride, int N) {
  return (int64_t)(32 * ((N + 31) / 32)) * stride * 2 < ((int64_t)1 << 31);
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

// Work item of the screens: key tiles [k0, k1) of one 256-row block of one stream (branch,
// head).  A block's causal key range (key tiles 0 .. nkt - 1) is cut into chunks of screen_kc
// tiles (whole bitmask words), so that small problems have enough items and no item is much
// longer than the others; items are numbered per stream in (block, chunk) order and handed out
// from the last (the longest block's).  tiles_before / per_stream: key-tile steps of the stream's
// earlier items / of all of them (they place the item's slice of the zero range).
struct ScreenItem {
  int sidx, qb, chunk, nkt, k0, k1;
  int64_t tiles_before, per_stream;
};
__device__ __forceinline__ ScreenItem screen_item(const FwdParams& P, int BR) {
  const int nqt = P.nqt, qoff = P.qoff;
  const WorkItem wi = xcd_order(blockIdx.x, BR * P.B * P.H, P.screen_items);
  const int KC = P.screen_kc;
  ScreenItem it{wi.stream, 0, 0, 1, 0, 1, 0, 0};
  int t = wi.block;
  bool found = false;
  for (int q = 0; q < (P.Nq + 255) / 256; ++q) {
    const int n = kt_last(min(8 * q + 7, nqt - 1), qoff, P.nkt) + 1;
    const int c = (n + KC - 1) / KC;
    if (!found && t < c) {
      it.qb = q;
      it.chunk = t;
      it.nkt = n;
      it.tiles_before += (int64_t)t * KC;
      found = true;
    } else if (!found) {
      t -= c;
      it.tiles_before += n;
    }
    it.per_stream += n;
  }
  it.k0 = it.chunk * KC;
  it.k1 = min(it.k0 + KC, it.nkt);
  return it;
}

// The item's slice of the call's zero range (the backward's gradients in training): an item
// clears zero_per_it 16-byte units per key tile it walks, from the steps of the items before it
// in (stream, block, chunk) order.  Buffer stores over the slice: the hardware drops those past
// its end (the host hands the screen slices below 2^31 bytes, so 32-bit offsets; a larger range
// is cleared whole by zero_range before the screen); streaming (nt): the backward reads them
// much later.
struct ZeroSlice {
  __amdgpu_buffer_rsrc_t r;
  __device__ __forceinline__ void init(const FwdParams& P, const ScreenItem& it) {
    int64_t z0 = 0, zend = 0;
    if (P.zero) {
      z0 = ((int64_t)it.sidx * it.per_stream + it.tiles_before) * P.zero_per_it;
      zend = min(z0 + (int64_t)(it.k1 - it.k0) * P.zero_per_it, P.zero_units);
    }
    r = make_rsrc(P.zero ? reinterpret_cast<u32x4*>(P.zero) + z0 : nullptr,
                  (uint32_t)(zend > z0 ? (zend - z0) * 16 : 0));
  }
  // The slices of key-tile steps step .. step + n - 1.  The whole offset is the per-lane one:
  // the descriptor's range check (which drops the stores past the slice) does not cover the
  // scalar offset.
  template <int NTHR>
  __device__ __forceinline__ void clear(const FwdParams& P, int step, int tid, int n = 1) const {
    const uint32_t base = (uint32_t)step * (uint32_t)P.zero_per_it * 16u;
    const int units = n * P.zero_per_it;
    for (int u = tid; u < units; u += NTHR)
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{0u, 0u, 0u, 0u}, r, base + (uint32_t)u * 16u, 0, 2);
  }
};

// Bitmask words (and, with candidate lists, the candidate keys) of one wave's query tiles after
// key tile kt, when a 32-tile word is complete or the item ends.  hb[s]: per lane, bit kt % 32
// set when the lane's test passed for key tile kt (lane n32 of either half: key n32 of the tile
// when CAND, the lane's query row otherwise).  The item owns whole words of each row.
// Candidate slots: an item that covers its block's whole key range is the lists' only producer
// and counts in cn[s] (stored at the end, screen_counts); the items of a split block take their
// slots with one atomic add per word on the count (zeroed by key_prep).
template <int QPW, bool CAND>
__device__ __forceinline__ void screen_flush(const FwdParams& P, int BR, const ScreenItem& it, int qt0,
                                             const bool (&live)[QPW], uint32_t (&hb)[QPW], uint32_t (&cn)[QPW],
                                             int kt) {
  const int l = lane_id(), n32 = l & 31;
  const int BH = P.B * P.H, nqt = P.nqt, Nk = P.Nk;
  if (!(live[0] && ((kt & 31) == 31 || kt == it.k1 - 1))) return;
  uint32_t* occ0 = P.occ + ((int64_t)it.sidx * nqt + qt0) * P.occ_w;
  const int kpad = P.nkt - 1;  // the key tile that may hold padding keys
#pragma unroll
  for (int s = 0; s < QPW; ++s) {
    uint32_t w = hb[s];
    if constexpr (CAND) {
      // a padding key (past Nk, in the last key tile) scores 0 and passes a threshold below 0
      // (the query tile at position 0, beta <= 0): it holds no weight and must not be listed
      if ((kt >> 5) == (kpad >> 5) && n32 >= Nk - 32 * kpad) w &= ~(1u << (kpad & 31));
      // nor is a key after the query tile's last position (its diagonal key tile): no row of the
      // tile sees it, so the lists hold the same keys whatever follows the tile's rows
      const int lastk = P.qoff + min(32 * (qt0 + s) + 31, P.Nq - 1), kdiag = lastk >> 5;
      if ((kt >> 5) == (kdiag >> 5) && 32 * kdiag + n32 > lastk) w &= ~(1u << (kdiag & 31));
    }
    const uint32_t hm = w | (uint32_t)__shfl_xor((int)w, 32);  // lane n32: tiles its key passed
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) w |= (uint32_t)__shfl_xor((int)w, o);
    hb[s] = 0u;
    if constexpr (CAND) {
      // candidate keys of the word's tiles: per tile with a passing lane (a few per cent), the
      // keys of its passing lanes in increasing order, appended to the query tile's list
      const uint32_t m0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)w);
      if (P.cand && m0) {
        const int64_t list = (int64_t)it.sidx * nqt + qt0 + s;
        uint32_t* clist = P.cand + list * kCandCap;
        uint32_t run = cn[s];
        if (!(it.k0 == 0 && it.k1 == it.nkt)) {  // a split block: slots by atomic add
          uint32_t total = 0u;
          for (uint32_t m = m0; m; m &= m - 1u)
            total += (uint32_t)__builtin_popcountll(wave_ballot(l < 32 && ((hm >> __builtin_ctz(m)) & 1u)));
          uint32_t base = 0u;
          if (l == 0) base = atomicAdd(P.cand + pair_lists(BR, BH, nqt) * kCandCap + list, total);
          run = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
        }
        for (uint32_t m = m0; m; m &= m - 1u) {
          const int b = __builtin_ctz(m);
          const uint32_t keys = (uint32_t)wave_ballot(l < 32 && ((hm >> b) & 1u));
          const uint32_t slot = run + (uint32_t)__builtin_popcount(keys & ((1u << n32) - 1u));
          if (l < 32 && ((keys >> l) & 1u) && slot < (uint32_t)kCandCap)
            clist[slot] = (uint32_t)(32 * (32 * (kt >> 5) + b) + l);
          run += (uint32_t)__builtin_popcount(keys);
        }
        cn[s] = run;
      }
    }
    if (l == 0 && live[s]) {
      uint32_t* row = occ0 + s * P.occ_w;
      row[kt >> 5] = w;
      if (kt == it.nkt - 1)  // words of key tiles no item of the block reaches
        for (int x = (kt >> 5) + 1; x < P.occ_w; ++x) row[x] = 0u;
    }
  }
}

// The candidate counts of an item that is its lists' only producer (see screen_flush).
template <int QPW>
__device__ __forceinline__ void screen_counts(const FwdParams& P, int BR, const ScreenItem& it, int qt0,
                                              const bool (&live)[QPW], const uint32_t (&cn)[QPW]) {
  if (!P.cand || lane_id() != 0 || !(it.k0 == 0 && it.k1 == it.nkt)) return;
  const int64_t base = pair_lists(BR, P.B * P.H, P.nqt) * kCandCap + (int64_t)it.sidx * P.nqt + qt0;
#pragma unroll
  for (int s = 0; s < QPW; ++s)
    if (live[s]) P.cand[base + s] = cn[s];
}

// Causal (query tile, key tile) pairs of one wave's query tiles in the item, for the counters.
template <int QPW>
__device__ __forceinline__ void screen_count(const FwdParams& P, const ScreenItem& it, const bool (&live)[QPW],
                                             const int (&ktl)[QPW]) {
  if (!P.stats || lane_id() != 0) return;
  unsigned visited = 0;
#pragma unroll
  for (int s = 0; s < QPW; ++s) visited += live[s] ? (unsigned)max(0, min(it.k1 - 1, ktl[s]) - it.k0 + 1) : 0u;
  if (visited) atomicAdd(P.stats + 0, (unsigned long long)visited);
}

// ------------------------------------------------------------------ int8 screening bound
// The normalised screen (fwd_screen_i8) tests int8 scores.  The exact pass keeps weight (i, j)
// iff x_ij = fma(fl(S_ij rk_j), rq_i, -tau_i) > 0, S_ij the fp32 MFMA sum of the bf16 products
// q_i . k_j (rq, rk: fp32 inverse row norms, the same values on both sides).  With qt = rq q_i
// and kt = rk k_j (real), x > 0 implies
//   qt . kt > tau_i (1 - 2^-24) - 2^-17 (1 + 2^-20)
// (the fp32 product and fma roundings, and 128 * 2^-24 = 2^-17 of |q||k| for the accumulation).
// The screen forms qh = fl(q rq) and kh = fl(k rk) (each within 2^-24 of qt, kt per element) and
// quantises them: qh = sq a + rq_res with one scale sq per 32-row query tile (sq = max |qh| /
// 127 over the tile, a = rint(qh / sq) in [-127, 127]) and kh = s_j b + rk_res per key row (s_j
// = max |kh_j| / 127); the residuals are computed exactly (fma) and eq >= |rq_res|, ek_j >=
// |rk_res| bound their norms (fp32 sums of squares and square roots, times 1 + 2^-12).  With
// A_ij = a . b_j (exact int32) and |qh|, |kh| <= 1 + 2^-20:
//   qt . kt <= sq s_j A_ij + (eq + ek_j)(1 + 2^-20) + 3 eq ek_j + 2^-22.
// So with tmin the tile's smallest tau (tau is monotone in the position up to a relative
// 2^-20) every kept weight passes
//   fl(fl(float(max_i A_ij) * fl(sq s_j))) > thr_j = tmin - |tmin| 2^-19 - 2^-14
//                                                   - eq (1 + 2^-10) - ek_j (1 + 2^-10 + 4 eq):
// 2^-14 covers 2^-17 + 2^-22 and the fp32 roundings of the test (relative 2^-23 on values below
// 1.02), |tmin| 2^-19 the threshold's, and the (1 + 2^-10) factors and 4 eq ek_j the rest.  On
// N(0, 1) rows eq is about 0.009 and ek_j about 0.006 (against a bf16-residual margin of 0.002),
// so the screen keeps about twice the candidate keys of an exact test; the exact pass drops them.
__device__ __forceinline__ float i8_tmin(float tmin, float eq) {
  return tmin - fabsf(tmin) * 0x1p-19f - 0x1p-14f - eq * (1.f + 0x1p-10f);
}
__device__ __forceinline__ float i8_ekcoef(float eq) { return 1.f + 0x1p-10f + 4.f * eq; }
__device__ __forceinline__ float res_bound(float sumsq) { return sqrtf(sumsq) * (1.f + 0x1p-12f); }

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

// rint(x y) of the exact product, |x y| < 2^22, by one fma: x y + 1.5 * 2^23 rounds to an integer
// (ties to even) whose low bits are that integer's two's complement; returns the sum.  The
// integer as a float is the sum minus the constant (exact).
constexpr float kRintMagic = 12582912.0f;
__device__ __forceinline__ float rint_fma(float x, float y) { return __builtin_fmaf(x, y, kRintMagic); }
// The low bytes of four rint_fma sums (int8 values in [-127, 127]) packed into one int, byte e
// from argument e, by three byte permutes.
__device__ __forceinline__ int pack4_rint(float a, float b, float c, float d) {
  const uint32_t ab = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, b), __builtin_bit_cast(uint32_t, a), 0x0c0c0400u);
  const uint32_t cd = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, d), __builtin_bit_cast(uint32_t, c), 0x0c0c0400u);
  return (int)__builtin_amdgcn_perm(cd, ab, 0x05040100u);
}

__device__ __forceinline__ int max16i(const i32x16& v) {
  // five three-input maxima, two more, one max: 8 instructions
  const int a = max(max(v[0], v[1]), v[2]), b = max(max(v[3], v[4]), v[5]), c = max(max(v[6], v[7]), v[8]);
  const int d = max(max(v[9], v[10]), v[11]), e = max(max(v[12], v[13]), v[14]);
  return max(max(max(a, b), c), max(max(d, e), v[15]));
}

// ------------------------------------------------------------------ key_prep
// Per key row of every branch: the inverse L2 norm rk_j into the norms table and, for the int8
// screen (P.k8 set), the row kh_j = fl(k_j rk_j) quantised to int8 (P.k8, [stream][Nk][D] bytes)
// with its scale s_j and residual bound ek_j (P.ksc, [stream][Nk] {s_j, ek_j}).  Non-finite
// elements quantise as 0 (such a key's exact weights are 0); a row whose sum of squares is finite
// has none.  A group of D/16 lanes reads one row (two 16-byte loads and one 16-byte int8 store per
// lane), the row sums and maxima are DPP reductions within the group; each wave covers
// KN_GROUPS row groups of one (branch, head) with all its loads issued before the first
// reduction and its stores after the last.  It also zeroes the screen's candidate counts, the
// tile-pass queue count and the column buckets' counts.  (Eight elements per lane, half-size
// stores, measured 56 us against 46 at B4 H16 N4096 d128, two branches.)
// Row groups per wave: 4 at d = 128 (64 rows), 2 at d = 64 (32 rows; measured 11.2 us against
// 12.1 with 4 at B4 H16 N2048 d64, one branch, where the grid is small).
template <int D>
constexpr int kn_groups() {
  return D == 64 ? 2 : 4;
}
// Row elements of a key_prep or screen lane: 16 consecutive bf16 (two 16-byte vectors) or fp32
// (four) values; element j as a float.
template <class T>
struct Row16 {
  static constexpr int E = 16 / sizeof(T);  // elements per 16-byte vector
  using V = std::conditional_t<sizeof(T) == 2, bf16x8, f32x4>;
  V v[16 / E];
  __device__ __forceinline__ void load(const T* r) {
#pragma unroll
    for (int u = 0; u < 16 / E; ++u) v[u] = *reinterpret_cast<const V*>(r + E * u);
  }
  __device__ __forceinline__ float operator[](int j) const { return (float)v[j / E][j % E]; }
  // the sum of squares: two fma chains over elements 0-7 and 8-15, added
  __device__ __forceinline__ float sumsq() const {
    float a = 0.f, b = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      a = __builtin_fmaf((*this)[j], (*this)[j], a);
      b = __builtin_fmaf((*this)[8 + j], (*this)[8 + j], b);
    }
    return a + b;
  }
};

template <int D, class T>
__global__ void __launch_bounds__(256) key_prep(FwdParams P, int BR) {
  constexpr int KN_GROUPS = kn_groups<D>();
  constexpr int LPR = D / 16, RPG = 64 / LPR, ROWS = RPG * KN_GROUPS;
  const int l = lane_id(), sub = l % LPR;
  const int BH = P.B * P.H, N = P.Nk;
  const uint32_t wpr = (uint32_t)(N + ROWS - 1) / ROWS;
  const uint32_t wid = blockIdx.x * 4u + (threadIdx.x >> 6);
  if (P.cand) {
    const int64_t lists = pair_lists(BR, BH, P.nqt), nthr = (int64_t)gridDim.x * 256;
    uint32_t* counts = P.cand + lists * kCandCap;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < lists; i += nthr) counts[i] = 0u;
    if (blockIdx.x == 0 && threadIdx.x == 0) P.pvq[0] = 0u;
    if (P.colcnt)  // the column buckets' counts (the candidate pass appends)
      for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < (int64_t)BH * P.nkt; i += nthr) P.colcnt[i] = 0u;
  }
  if ((int64_t)wid >= (int64_t)BR * BH * wpr) return;
  const int sidx = (int)(wid / wpr), br = sidx / BH, bh = sidx % BH;
  const int t0 = (int)(wid % wpr) * ROWS + l / LPR;
  const T* kin = (const T*)(br ? P.in[F_K2] : P.in[F_K1]);
  const int64_t sb = br ? P.s[F_K2][0] : P.s[F_K1][0], sh = br ? P.s[F_K2][1] : P.s[F_K1][1];
  const int64_t st = br ? P.s[F_K2][2] : P.s[F_K1][2];
  const T* head = kin + (int64_t)(bh / P.H) * sb + (int64_t)(bh % P.H) * sh;
  Row16<T> x[KN_GROUPS];
#pragma unroll
  for (int u = 0; u < KN_GROUPS; ++u) {
    const int t = min(t0 + RPG * u, N - 1);
    x[u].load(head + (int64_t)t * st + 16 * sub);
  }
  float ss[KN_GROUPS], rk[KN_GROUPS];
#pragma unroll
  for (int u = 0; u < KN_GROUPS; ++u) {
    ss[u] = group_sum<LPR>(x[u].sumsq());
    rk[u] = inv_norm(ss[u]);
  }
  float* out = P.norms + norm_base(P, br ? N_K2 : N_K1, bh);
  if (!P.k8) {  // norms only
#pragma unroll
    for (int u = 0; u < KN_GROUPS; ++u) {
      const int t = t0 + RPG * u;
      if (sub == 0 && t < N) out[t] = rk[u];
    }
    return;
  }
  i32x4 packed[KN_GROUPS];
  float2 se[KN_GROUPS];
#pragma unroll
  for (int u = 0; u < KN_GROUPS; ++u) {
    float kh[16], m = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) kh[j] = x[u][j] * rk[u];
    if (wave_ballot(!__builtin_isfinite(ss[u])) != 0ull) {  // a branch only where a row has any
#pragma unroll
      for (int j = 0; j < 16; ++j) kh[j] = __builtin_isfinite(kh[j]) ? kh[j] : 0.f;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) m = fmaxf(m, fabsf(kh[j]));
    m = group_max<LPR>(m);
    // every |kh| <= m, so b = rint(kh 127 / m) of the exact product lies in [-127, 127]
    const float sc = m * (1.f / 127.f), inv = m > 0.f ? 127.f / m : 0.f;
    float rs[16], e2 = 0.f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      rs[j] = rint_fma(kh[j], inv);
      const float r = __builtin_fmaf(-sc, rs[j] - kRintMagic, kh[j]);
      e2 = __builtin_fmaf(r, r, e2);
    }
    packed[u] = i32x4{pack4_rint(rs[0], rs[1], rs[2], rs[3]), pack4_rint(rs[4], rs[5], rs[6], rs[7]),
                      pack4_rint(rs[8], rs[9], rs[10], rs[11]), pack4_rint(rs[12], rs[13], rs[14], rs[15])};
    se[u] = float2{sc, res_bound(group_sum<LPR>(e2))};
  }
#pragma unroll
  for (int u = 0; u < KN_GROUPS; ++u) {
    const int t = t0 + RPG * u;
    if (t < N) {
      *reinterpret_cast<i32x4*>(P.k8 + ((int64_t)sidx * N + t) * D + 16 * sub) = packed[u];
      if (sub == 0) {
        out[t] = rk[u];
        *reinterpret_cast<float2*>(P.ksc + 2 * ((int64_t)sidx * N + t)) = se[u];
      }
    }
  }
}

// ------------------------------------------------------------------ fwd_screen_i8 (normalised)
// The normalised screen on int8 matrix cores (v_mfma_i32_32x32x32_i8, twice the bf16 rate, half
// the operand bytes).  Workgroup = one work item (ScreenItem), four waves of two 32-row query
// tiles.  Per wave the query rows are normalised (their inverse norms rq go to the norms table),
// quantised to int8 with one scale per query tile and held as A fragments.  The int8 key tiles
// of key_prep (32 x D bytes, contiguous) and their {s_j, ek_j} stream through a ring of
// I8_STAGES LDS stages of I8_TPI tiles by direct buffer->LDS loads issued I8_STAGES - 1 stages
// ahead (rows past Nk read 0; one wait on the wave's own loads and one barrier per stage).  The
// tile is S = A B^T: each lane holds one key j and 16 query rows, and the test (the int8 bound
// above) is "float(max_i A_ij) * (sq s_j) > thr_j", a few operations per lane and query tile.
// Hit bits give the bitmask words and the candidate keys (screen_flush).
constexpr int I8_STAGES = 4;
constexpr int I8_TPI = 2;                // key tiles per stage (a divisor of 32)
constexpr int I8_AHEAD = I8_STAGES - 1;  // stages in flight past the one being tested
static_assert(32 % I8_TPI == 0 && I8_TPI <= 4, "stages of whole parts of a bitmask word");
// Chunk swizzle of an int8 key tile row (16-byte chunks): conflict-free fragment reads, where
// lane (m, g) reads chunk 2 t + g of row m.
template <int D>
__device__ __forceinline__ int i8swz(int r) {
  if constexpr (D == 128) return (r ^ (r >> 3)) & 7;
  else return ((r >> 1) ^ (r >> 3)) & 3;
}
// 32-bit LDS address of a __shared__ object (for inline-asm LDS instructions).
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
template <int N>
__device__ __forceinline__ void wait_vm() {  // vmcnt(N) with the other counters left alone
  static_assert(N >= 0 && N < 64, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
template <int D, class T>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) fwd_screen_i8(FwdParams P, int BR) {
  constexpr int QPW = 2, NTHR = 256, TPI = I8_TPI;
  constexpr int NK = D / 32;                     // int8 MFMA steps over d
  constexpr int CPR = D / 16;                    // 16-byte chunks per int8 key row
  constexpr int RPI = 64 / CPR;                  // key rows per load instruction
  constexpr int KI = TPI * 32 / RPI;             // key load instructions per stage
  constexpr int TB = 32 * D;                     // bytes of one int8 key tile
  __shared__ __attribute__((aligned(16))) int8_t kst[I8_STAGES][TPI * TB];
  __shared__ __attribute__((aligned(16))) float2 ksc[I8_STAGES][TPI * 32];  // {s_j, ek_j} per key

  const int l = lane_id(), n32 = l & 31, g = l >> 5, tid = threadIdx.x;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int BH = P.B * P.H, Nq = P.Nq, Nk = P.Nk, nqt = P.nqt, qoff = P.qoff;
  const ScreenItem it = screen_item(P, BR);
  const int k0 = it.k0, k1 = it.k1, nit = k1 - k0, nst = (nit + TPI - 1) / TPI;
  const int br = it.sidx / BH, bh = it.sidx % BH;
  const int b = bh / P.H, h = bh % P.H;
  const int q0w = it.qb * 256 + 32 * QPW * wv;  // first row of this wave
  const int qt0 = q0w >> 5;                     // this wave's query tiles: qt0, qt0 + 1
  bool live[QPW];
  int ktl[QPW];  // last key tile each query tile sees
#pragma unroll
  for (int s = 0; s < QPW; ++s) {
    live[s] = qt0 + s < nqt;
    ktl[s] = kt_last(qt0 + s, qoff, P.nkt);
  }

  // ---- staging: stage j holds tiles k0 + TPI j .. + TPI - 1 (the stream's int8 key rows,
  // contiguous, D bytes each) and their {s_j, ek_j}.  The buffer descriptors start at the item's
  // first key row (host: an item spans under 2^30 bytes); rows past Nk read 0.  Every wave issues
  // the same loads per stage: key load instructions wv, wv + 4, .. (1 KiB: RPI rows each; lane L
  // moves stage row R = RPI k + L / CPR, chunk (L % CPR) ^ swz(R % 32)) and a quarter of the
  // stage's {s_j, ek_j} (4 TPI lanes of 16 bytes).
  static_assert(KI % 4 == 0, "key load instructions spread evenly over the four waves");
  constexpr int LK = KI / 4;      // key load instructions per wave and stage
  constexpr int LW = LK + 1;      // loads per wave and stage
  const int64_t rows_left = (int64_t)Nk - 32 * (int64_t)k0;
  const int8_t* k8base = P.k8 + ((int64_t)it.sidx * Nk + 32 * (int64_t)k0) * D;
  const float* scbase = P.ksc + 2 * ((int64_t)it.sidx * Nk + 32 * (int64_t)k0);
  const uint32_t k8bytes = (uint32_t)(rows_left * D < 0xffffff00ll ? rows_left * D : 0xffffff00ll);
  const uint32_t scbytes = (uint32_t)(rows_left * 8 < 0xffffff00ll ? rows_left * 8 : 0xffffff00ll);
  uint32_t loff[LK];
#pragma unroll
  for (int u = 0; u < LK; ++u) {
    const int R = RPI * (4 * u + wv) + l / CPR;
    loff[u] = (uint32_t)(R * D + 16 * ((l % CPR) ^ i8swz<D>(R & 31)));
  }
  const uint32_t soff = (uint32_t)(16 * (4 * TPI * wv + l));  // this lane's {s_j, ek_j} chunk
  // The stage offset goes into the per-lane offset, which the descriptor's range check covers
  // (rows past Nk must read 0), not into the scalar offset.
  auto issue = [&](int j) {  // stage j into ring slot j % I8_STAGES
    const int st = j % I8_STAGES;
    const uint32_t so = (uint32_t)j * (uint32_t)(TPI * TB);
#pragma unroll
    for (int u = 0; u < LK; ++u)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(k8base, k8bytes), LDS_PTR(void, &kst[st][1024 * (4 * u + wv)]), 16,
                                               (uint32_t)(loff[u] + so), 0, 0, 0);
    if (l < 4 * TPI)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(make_rsrc(scbase, scbytes), LDS_PTR(void, &ksc[st][8 * TPI * wv]), 16,
                                               (uint32_t)(soff + (uint32_t)j * (uint32_t)(TPI * 256)), 0, 0, 0);
  };
  // Wait for this wave's loads of stage j: the loads of later stages may stay in flight (loads
  // complete in order; stores or atomics issued since only lengthen the wait).
  auto wait_stage = [&](int j) {
    if (j + I8_AHEAD <= nst) wait_vm<LW * (I8_AHEAD - 1)>();  // stages j + 1 .. j + I8_AHEAD - 1 issued
    else wait_vm<0>();
  };
  // issued before the query setup, whose loads and latency they overlap
#pragma unroll
  for (int j = 0; j < I8_AHEAD; ++j)
    if (j < nst) issue(j);

  // ---- resident int8 query fragments and the per-tile constants of the test
  const int qslot = br ? F_Q2 : F_Q1;
  const T* qin = (const T*)(br ? P.in[F_Q2] : P.in[F_Q1]);
  const int64_t qsb = br ? P.s[F_Q2][0] : P.s[F_Q1][0], qsh = br ? P.s[F_Q2][1] : P.s[F_Q1][1];
  const int64_t qst = br ? P.s[F_Q2][2] : P.s[F_Q1][2];
  (void)qslot;
  const T* qhead = qin + (int64_t)b * qsb + (int64_t)h * qsh;
  const float beta = *P.beta;
  i32x4 A8[QPW][NK];
  float sq[QPW], tq[QPW], cq[QPW];  // scale, thr part of the tile, coefficient of ek_j
#pragma unroll
  for (int s = 0; s < QPW; ++s) {
    const int iq = q0w + 32 * s + n32;
    const bool valid = iq < Nq;
    const T* row = qhead + (int64_t)min(iq, Nq - 1) * qst;  // rows >= Nq: never vote
    Row16<T> qv[NK];  // lane (m, g): elements 32 t + 16 g .. + 16 of row m
#pragma unroll
    for (int t = 0; t < NK; ++t) qv[t].load(row + 32 * t + 16 * g);
    // the row's sum of squares and largest |q|; a row with a finite sum of squares has only
    // finite elements, and every element of it then scales to |x| <= m below
    float ss = 0.f, mq = 0.f;
#pragma unroll
    for (int t = 0; t < NK; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float x = qv[t][j];
        ss = __builtin_fmaf(x, x, ss);
        mq = fmaxf(mq, fabsf(x));
      }
    ss += __shfl_xor(ss, 32);
    const bool finite_row = __builtin_isfinite(ss);
    if (!finite_row) {  // the largest finite |q| (non-finite elements quantise as 0)
      if constexpr (sizeof(T) == 2) {
        uint32_t mb = 0u;
#pragma unroll
        for (int t = 0; t < NK; ++t)
#pragma unroll
          for (int c = 0; c < 2; ++c) {
            const u32x4 w = __builtin_bit_cast(u32x4, qv[t].v[c]);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              const uint32_t lo = w[k] & 0x7fffu, hi = (w[k] >> 16) & 0x7fffu;
              mb = max(mb, (lo & 0x7f80u) != 0x7f80u ? lo : 0u);
              mb = max(mb, (hi & 0x7f80u) != 0x7f80u ? hi : 0u);
            }
          }
        mq = __builtin_bit_cast(float, mb << 16);
      } else {
        mq = 0.f;
#pragma unroll
        for (int t = 0; t < NK; ++t)
#pragma unroll
          for (int j = 0; j < 16; ++j) mq = fmaxf(mq, __builtin_isfinite(qv[t][j]) ? fabsf(qv[t][j]) : 0.f);
      }
    }
    if constexpr (sizeof(T) == 2) {
      // the row values are converted again below, not kept as fp32 (register pressure)
#pragma unroll
      for (int t = 0; t < NK; ++t)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
          u32x4 w = __builtin_bit_cast(u32x4, qv[t].v[c]);
          asm volatile("" : "+v"(w));
          qv[t].v[c] = __builtin_bit_cast(bf16x8, w);
        }
    }
    const float rq = inv_norm(ss);
    if (g == 0 && valid && it.chunk == 0) P.norms[norm_base(P, br ? N_Q2 : N_Q1, bh) + iq] = rq;
    const float sc = valid ? rq : 0.f;
    // the scale, one per query tile: sq = m / 127 with m the tile's largest |qh| = max over its
    // rows of rq_i max |q_i|; every |x| <= m, so x 127 / m rounds into [-127, 127]
    mq = fmaxf(mq, __shfl_xor(mq, 32));  // the row's largest |q|
    float m = mq * sc;
    m = __builtin_isfinite(m) ? m : 0.f;
    m = group_max<16>(m);
    m = fmaxf(m, __shfl_xor(m, 16));  // over the tile's rows
    sq[s] = m * (1.f / 127.f);
    const float inv = m > 0.f ? 127.f / m : 0.f;
    const bool any_nonfinite = wave_ballot(!finite_row) != 0ull;
    float r2 = 0.f;  // squared norm of the row's quantisation residual (this lane's half)
#pragma unroll
    for (int t = 0; t < NK; ++t) {
      int w[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float rs[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = 4 * u + e;
          float x = qv[t][j] * sc;
          if (any_nonfinite) x = __builtin_isfinite(x) ? x : 0.f;
          rs[e] = rint_fma(x, inv);  // rint(x inv) of the exact product, |x inv| <= 127 (1 + 2^-22)
          const float r = __builtin_fmaf(-sq[s], rs[e] - kRintMagic, x);
          r2 = __builtin_fmaf(r, r, r2);
        }
        w[u] = pack4_rint(rs[0], rs[1], rs[2], rs[3]);
      }
      A8[s][t] = i32x4{w[0], w[1], w[2], w[3]};
      __builtin_amdgcn_sched_barrier(0);  // one step's values live at a time
    }
    r2 += __shfl_xor(r2, 32);
    r2 = group_max<16>(r2);
    r2 = fmaxf(r2, __shfl_xor(r2, 16));  // largest row of the tile
    const float eq = res_bound(r2);
    // tau is monotone in the position: its smallest value over the tile's rows is at one end
    const int i0 = q0w + 32 * s, i1 = max(i0, min(i0 + 31, Nq - 1));
    tq[s] = i8_tmin(fminf(beta * tau_coeff(qoff + i0, P.inv_d), beta * tau_coeff(qoff + i1, P.inv_d)), eq);
    cq[s] = i8_ekcoef(eq);
    __builtin_amdgcn_sched_barrier(0);  // one query tile's rows live at a time
  }
  ZeroSlice zs;
  zs.init(P, it);

  uint32_t hb[QPW], cn[QPW];  // hit bits; candidate keys met per query tile (may pass the cap)
#pragma unroll
  for (int s = 0; s < QPW; ++s) hb[s] = cn[s] = 0u;
  // LDS addresses of this lane's fragment chunks in ring slot 0, tile 0 (row n32, chunk 2 t + g)
  // and of its key's {s_j, ek_j}; the slot and tile go into the instructions' offset fields
  uint32_t kaddr[NK];
#pragma unroll
  for (int t = 0; t < NK; ++t) kaddr[t] = lds_addr(&kst[0][0]) + (uint32_t)(n32 * D + 16 * ((2 * t + g) ^ i8swz<D>(n32)));
  const uint32_t saddr = lds_addr(&ksc[0][0]) + 8u * (uint32_t)n32;

  // One tile: the fragment reads are inline asm (the compiler orders every LDS read after all
  // outstanding direct-to-LDS loads, vmcnt(0), which would drain the ring each tile, while
  // wait_stage and the barrier already order this stage's loads before them); the wait that ends
  // them takes the fragments as operands, so no use of them is scheduled before it.
  auto process = [&](int kt, auto TOFF, auto SOFF) {
    constexpr uint32_t toff = decltype(TOFF)::value, soff_ = decltype(SOFF)::value;
    i32x4 fk[NK];
#pragma unroll
    for (int t = 0; t < NK; ++t)
      asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(fk[t]) : "v"(kaddr[t]), "i"(toff) : "memory");
    float2 kq;  // the lane's key: {s_j, ek_j} (0 past Nk)
    asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(kq) : "v"(saddr), "i"(soff_) : "memory");
    if constexpr (NK == 4)
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(fk[0]), "+v"(fk[1]), "+v"(fk[2]), "+v"(fk[3]), "+v"(kq) : : "memory");
    else
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(fk[0]), "+v"(fk[1]), "+v"(kq) : : "memory");
    __builtin_amdgcn_sched_barrier(0);
    i32x16 S[QPW];
#pragma unroll
    for (int s = 0; s < QPW; ++s) {
#pragma unroll
      for (int t = 0; t < NK; ++t)
        S[s] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A8[s][t], fk[t], t ? S[s] : i32x16{}, 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);  // keep the chains apart
    }
    const uint32_t bit = 1u << (kt & 31);
    // straight-line tests on every path: the compiler counts the wait states after an MFMA on
    // the fall-through path only, so a branch here could read scores not yet written
#pragma unroll
    for (int s = 0; s < QPW; ++s) {
      const float thr = __builtin_fmaf(-kq.y, cq[s], tq[s]);
      const bool hit = (float)max16i(S[s]) * (sq[s] * kq.x) > thr;
      hb[s] |= live[s] && hit && kt <= ktl[s] ? bit : 0u;
    }
  };

  // the last stage with a tile some query tile of the wave sees (later tiles of a stage are
  // masked in the test)
  const int jl = live[0] ? (ktl[QPW - 1] - k0) / TPI : -1;
  // stage j sits in ring slot j % I8_STAGES: the loop is unrolled over the slots so that every
  // slot's LDS offsets are constants
  static_assert(I8_STAGES == 4 && TPI == 2, "unrolled for a 4-slot ring of 2-tile stages");
  auto stage = [&](int j, auto SLOT) {
    constexpr int st = decltype(SLOT)::value;
    wait_stage(j);
    lds_barrier();  // stage j is in LDS; every wave is past stage j - 1, whose slot is reloaded
    if (j + I8_AHEAD < nst) issue(j + I8_AHEAD);
    if (P.zero) zs.clear<NTHR>(P, TPI * j, tid, min(TPI, nit - TPI * j));
    if (j <= jl) {
      process(k0 + TPI * j, std::integral_constant<uint32_t, st * TPI * TB>{},
              std::integral_constant<uint32_t, st * TPI * 256>{});
      process(k0 + TPI * j + 1, std::integral_constant<uint32_t, st * TPI * TB + TB>{},
              std::integral_constant<uint32_t, st * TPI * 256 + 256>{});
    }
    // the stage's last tile of the item (stages never straddle a bitmask word)
    screen_flush<QPW, true>(P, BR, it, qt0, live, hb, cn, min(k0 + TPI * j + TPI - 1, k1 - 1));
  };
  for (int j = 0; j < nst; j += I8_STAGES) {
    stage(j, std::integral_constant<int, 0>{});
    if (j + 1 < nst) stage(j + 1, std::integral_constant<int, 1>{});
    if (j + 2 < nst) stage(j + 2, std::integral_constant<int, 2>{});
    if (j + 3 < nst) stage(j + 3, std::integral_constant<int, 3>{});
  }
  screen_counts<QPW>(P, BR, it, qt0, live, cn);
  screen_count<QPW>(P, it, live, ktl);
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
                *reinterpret_cast<u32x4*>(pent + 4 * slot) = u32x4{(uint32_t)key, (uint32_t)n32, __builtin_bit_cast(uint32_t, x), kNoSlot};
              npairs += (uint32_t)__builtin_popcountll(bal);
            }
          }
        if (wave_ballot(valid && pos_any) == 0ull) {
          keep &= ~(1u << (kt & 31));
          continue;
        }
        // pairs of the tile pass are in no column bucket: the key-major backward walks the lists
        if (P.colcnt && l == 0) atomicOr(P.colcnt + (int64_t)bh * P.nkt + kt, kColTaint);
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

// ------------------------------------------------------------------ fwd_pv_blk
// The tile pass of the forwards without candidate lists (every query tile runs), over kBlkTiles
// consecutive query tiles of one head, one wave each.  The waves walk the union of their bitmask
// rows' kept key tiles in step and share each key tile's K and V rows (and key norms): the
// workgroup loads them once, each wave a quarter of the rows, one tile ahead into registers,
// then into a two-stage LDS ring (one barrier per tile: a stage is rewritten two tiles after it
// was read, and every wave has passed the barrier between).  A wave computes only the tiles its
// own row keeps, exactly as fwd_pv_tile does (the same MFMA sequence on the same operands: the
// same rows, bitmask rewrite, pair lists and counters).  Once a pair list has passed its cap
// the wave only counts its non-zero weights (one wave sum at the end) instead of placing them.
// WALK (no screen ran before it): every causal key tile of a row counts as kept, the row's
// bitmask words are all written (the words past its last key tile as zeros) and the causal
// tiles are counted into stats[0].  ZR (with WALK): the workgroup then clears its even share of
// the call's zero range.  K and V tiles load through one descriptor per head at a per-tile
// offset when the head's offsets fit 31 bits, else through one descriptor per tile.
constexpr int kBlkTiles = 4;

template <int D, int BR, int PK, bool NORM, bool WALK = false, bool ZR = false>
__global__ void __launch_bounds__(64 * kBlkTiles) __attribute__((amdgpu_waves_per_eu(D <= 64 ? 3 : 2))) fwd_pv_blk(FwdParams P) {
  static_assert(!ZR || WALK, "the zero range is cleared by the walk");
  constexpr int W = kBlkTiles;
  constexpr int NT = D / 16, ND = D / 32;
  constexpr int VS = D + 32;     // LDS row stride of a V tile: conflict-free transpose reads
  constexpr int KS = D + 8;      // LDS row stride of a K tile: conflict-free row-fragment reads
  constexpr int CPR = D / 8;     // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;  // rows per load instruction
  constexpr int LPW = 32 / RPI / W;  // load instructions per wave, K and V each
  static_assert(LPW >= 1 && LPW * RPI * W == 32, "K/V tile rows split evenly over the waves");
  constexpr int STAGE = 32 * KS + 32 * VS;
  static_assert(2 * STAGE >= W * 32 * KS, "the ring holds the waves' output rows");
  __shared__ __attribute__((aligned(16))) bf16 ring[2 * STAGE];
  __shared__ __attribute__((aligned(16))) float nring[2][32];

  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int BH = P.B * P.H, Nq = P.Nq, Nk = P.Nk, nqt = P.nqt, qoff = P.qoff;
  const int nqb = (nqt + W - 1) / W;
  int bh, jb;
  {
    // longest blocks (last query tiles) of every head first; one head's blocks on one XCD when
    // the heads fill the eight XCDs
    const int bid = blockIdx.x;
    if (BH % 8 == 0) {
      const int x = bid & 7, j = bid >> 3, hg = BH / 8;
      bh = x + 8 * (j % hg);
      jb = nqb - 1 - j / hg;
    } else {
      bh = bid % BH;
      jb = nqb - 1 - bid / BH;
    }
  }
  const int b = bh / P.H, h = bh % P.H;
  const int qt = W * jb + wv;
  const bool act = qt < nqt;  // wave-uniform: waves past the last query tile only load
  const int qtc = act ? qt : nqt - 1;
  const int iq = 32 * qt + n32;
  const bool valid = act && iq < Nq;
  const bool rowpad = 32 * qt + 31 >= Nq;  // the query tile has rows past Nq (uniform)
  const int pq = qoff + iq;  // the lane's query position
  const int klast_b = kt_last(min(W * jb + W - 1, nqt - 1), qoff, P.nkt);  // the block's last key tile
  const float tau = *P.beta * tau_coeff(pq, P.inv_d);
  const float pw = P.p;
  float lam = 0.f;
  if constexpr (BR == 2) lam = clamp01(*P.lam);

  const int vrow0 = RPI * LPW * wv + l / CPR, vch = l % CPR;  // this wave's rows of the K/V tiles
  const int bk = l >> 4, jj = l & 15;
  const int voff = (4 * (bk >> 1) + (jj >> 2)) * VS + 16 * (bk & 1) + 4 * (jj & 3);

  f32x16 O[ND];
#pragma unroll
  for (int c = 0; c < ND; ++c) O[c] = f32x16{};
  unsigned computed = 0, checked = 0;
  int it = 0;  // ring position, continued across the branches

#pragma unroll
  for (int br = 0; br < BR; ++br) {
    const int qslot = br ? F_Q2 : F_Q1, kslot = br ? F_K2 : F_K1;
    uint32_t* orow0 = P.occ + ((int64_t)(br * BH + bh) * nqt + W * jb) * P.occ_w;  // the block's first row
    const bf16* khead = (const bf16*)P.in[kslot] + (int64_t)b * P.s[kslot][0] + (int64_t)h * P.s[kslot][1];
    const bf16* vhead = (const bf16*)P.in[F_V] + (int64_t)b * P.s[F_V][0] + (int64_t)h * P.s[F_V][1];
    const int64_t sk = P.s[kslot][2], sv = P.s[F_V][2];
    const __amdgpu_buffer_rsrc_t rn =
        make_rsrc(NORM ? P.norms + norm_base(P, br ? N_K2 : N_K1, bh) : nullptr, NORM ? (uint32_t)Nk * 4 : 0u);
    const float coef = br == 0 ? 1.f : -lam;
    // query fragments straight from the rows (rows past Nq read as zeros), the inverse norm
    bf16x8 Q[NT];
    {
      const bf16* qhead = (const bf16*)P.in[qslot] + (int64_t)b * P.s[qslot][0] + (int64_t)h * P.s[qslot][1];
      const int64_t sq = P.s[qslot][2];
      const __amdgpu_buffer_rsrc_t rq_ = tile_rsrc<D>(qhead, sq, qtc, Nq);
#pragma unroll
      for (int t = 0; t < NT; ++t)
        Q[t] = __builtin_bit_cast(bf16x8, buf_load16(rq_, (uint32_t)((n32 * sq + 16 * t + 8 * g) * 2)));
    }
    float rq = 1.f;
    if constexpr (NORM) rq = P.norms[norm_base(P, br ? N_Q2 : N_Q1, bh) + min(32 * qtc + n32, Nq - 1)];
    const int64_t lidx = ((int64_t)br * BH + bh) * nqt + qtc;
    uint32_t* pent = P.pairs && act ? P.pairs + lidx * (4 * kPairCap) : nullptr;
    uint32_t npairs = 0, extra = 0;

    // word w of row r of the block, masked to the key tiles the row sees (uniform)
    auto row_word = [&](int r, int w) -> uint32_t {
      const int q = W * jb + r;
      if (q >= nqt) return 0u;
      const int kl = kt_last(q, qoff, P.nkt);
      if (w > (kl >> 5)) return 0u;
      uint32_t x = WALK ? 0xffffffffu : (uint32_t)__builtin_amdgcn_readfirstlane((int)orow0[(int64_t)r * P.occ_w + w]);
      if (w == (kl >> 5) && (kl & 31) != 31) x &= (2u << (kl & 31)) - 1u;
      return x;
    };
    // the union walk: next key tile any row keeps, its word, and the own row's word
    int sw = -1;
    uint32_t ub = 0u, sown = 0u;
    auto next_tile = [&](int& w_out, uint32_t& own_out) -> int {
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
      w_out = sw;
      own_out = sown;
      return kt;
    };
    u32x4 kr[LPW], vr[LPW];
    f32x4 nr = {};
    // one descriptor per head and a per-tile offset when the heads' offsets fit 31 bits (uniform),
    // else one descriptor per tile
    const bool whole = head_fits(sk, Nk) && head_fits(sv, Nk);
    const __amdgpu_buffer_rsrc_t rkh = head_rsrc<D>(khead, sk, Nk), rvh = head_rsrc<D>(vhead, sv, Nk);
    auto issue = [&](int kt) {
      if (whole) {
        const uint32_t tk = (uint32_t)(32 * kt) * (uint32_t)(2 * sk), tv = (uint32_t)(32 * kt) * (uint32_t)(2 * sv);
#pragma unroll
        for (int i = 0; i < LPW; ++i) kr[i] = buf_load16(rkh, tk + (uint32_t)(((vrow0 + RPI * i) * sk + 8 * vch) * 2));
#pragma unroll
        for (int i = 0; i < LPW; ++i) vr[i] = buf_load16(rvh, tv + (uint32_t)(((vrow0 + RPI * i) * sv + 8 * vch) * 2));
      } else {
        const __amdgpu_buffer_rsrc_t rk = tile_rsrc<D>(khead, sk, kt, Nk);
        const __amdgpu_buffer_rsrc_t rv = tile_rsrc<D>(vhead, sv, kt, Nk);
#pragma unroll
        for (int i = 0; i < LPW; ++i) kr[i] = buf_load16(rk, (uint32_t)(((vrow0 + RPI * i) * sk + 8 * vch) * 2));
#pragma unroll
        for (int i = 0; i < LPW; ++i) vr[i] = buf_load16(rv, (uint32_t)(((vrow0 + RPI * i) * sv + 8 * vch) * 2));
      }
      if (NORM && wv == 0 && l < 8) nr = __builtin_bit_cast(f32x4, buf_load16(rn, (uint32_t)(32 * kt + 4 * l) * 4));
    };

    int cw = 0;
    uint32_t cown = 0u;
    int kt = next_tile(cw, cown);
    if (kt >= 0) issue(kt);
    uint32_t keep = cown;  // own word cw with the tiles of no non-zero weight cleared
    while (kt >= 0) {
      bf16* kst = ring + (it & 1) * STAGE;
      bf16* vst = kst + 32 * KS;
      float* nst = nring[it & 1];
#pragma unroll
      for (int i = 0; i < LPW; ++i) {
        *reinterpret_cast<u32x4*>(kst + (vrow0 + RPI * i) * KS + 8 * vch) = kr[i];
        *reinterpret_cast<u32x4*>(vst + (vrow0 + RPI * i) * VS + 8 * vch) = vr[i];
      }
      if (NORM && wv == 0 && l < 8) *reinterpret_cast<f32x4*>(nst + 4 * l) = nr;
      int nw = 0;
      uint32_t nown = 0u;
      const int kt2 = next_tile(nw, nown);
      if (kt2 >= 0) issue(kt2);  // in flight during this tile's work
      lds_barrier();
      ++it;
      if ((cown >> (kt & 31)) & 1u) {
        ++checked;
        f32x16 S = {};
        const bf16* kp = kst + n32 * KS + 8 * g;
#pragma unroll
        for (int t = 0; t < NT; ++t) S = PolBF16::mma(*reinterpret_cast<const bf16x8*>(kp + 16 * t), Q[t], S);
        f32x4 rk4[4] = {{1.f, 1.f, 1.f, 1.f}, {1.f, 1.f, 1.f, 1.f}, {1.f, 1.f, 1.f, 1.f}, {1.f, 1.f, 1.f, 1.f}};
        if constexpr (NORM) {
#pragma unroll
          for (int u = 0; u < 4; ++u) rk4[u] = *reinterpret_cast<const f32x4*>(nst + 8 * u + 4 * g);
        }
        // exact values x, branch-free: keys after the query's position, padding keys past Nk
        // and query rows past Nq are set to -1 (no weight).  Only tiles reaching past the
        // position of the tile's first row or past Nk, and the last query tile when Nq is not a
        // multiple of 32, have any.
        f32x16 X;
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
          for (int e = 0; e < 4; ++e) X[4 * u + e] = __builtin_fmaf(NORM ? S[4 * u + e] * rk4[u][e] : S[4 * u + e], rq, -tau);
        if (32 * kt + 31 > min(qoff + 32 * qt, Nk - 1) || rowpad) {
          // key crow(r, g) = c_r + 4 g (c_r = 8 (r / 4) + r % 4) is visible iff c_r <= lim: one
          // comparison per value
          const int lim = (valid ? min(pq, Nk - 1) - 32 * kt : -1) - 4 * g;
#pragma unroll
          for (int r = 0; r < 16; ++r) X[r] = 8 * (r >> 2) + (r & 3) <= lim ? X[r] : -1.f;
        }
        // weights coef relu(x)^p and the lane's largest x (some weight of the tile is non-zero
        // iff a lane's is > 0), on the bits: a float is > 0 iff its bits as an int32 are, so the
        // integer max(bits, 0) is relu(x) (no NaN handling to pay for in float max); p other than
        // 1, 2 select on x > 0.  (Whole-vector bit casts: hipcc compiled a bit cast of one
        // element of an ext_vector to element 0.)
        typedef int i32x16 __attribute__((ext_vector_type(16)));
        const i32x16 XB = __builtin_bit_cast(i32x16, X);
        i32x16 TB;
        int xmb = XB[0];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          TB[r] = max(XB[r], 0);
          if (r) xmb = max(xmb, XB[r]);
        }
        const f32x16 T = __builtin_bit_cast(f32x16, TB);
        f32x16 C;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          if constexpr (PK == 2) C[r] = T[r] * (coef * T[r]);
          else if constexpr (PK == 1) C[r] = coef * T[r];
          else C[r] = X[r] > 0.f ? coef * pow_p<PK>(X[r], pw) : 0.f;
        }
        const bool pos_any = xmb > 0;
        if (pent) {
          if (npairs < (uint32_t)kPairCap) {
            // list entries of the non-zero weights, in the order (value r, lane); x's bits through
            // a bit cast of the whole vector (hipcc compiled a bit cast of one element of an
            // ext_vector to element 0)
            typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));
            const u32x16 XU = __builtin_bit_cast(u32x16, X);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const bool hit = X[r] > 0.f;
              const uint64_t bal = wave_ballot(hit);
              const uint32_t slot = npairs + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32),
                                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
              if (hit && slot < (uint32_t)kPairCap)
                *reinterpret_cast<u32x4*>(pent + 4 * slot) =
                    u32x4{(uint32_t)(32 * kt + crow(r, g)), (uint32_t)n32, XU[r], kNoSlot};
              npairs += (uint32_t)__builtin_popcountll(bal);
            }
          } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) extra += X[r] > 0.f ? 1u : 0u;
          }
        }
        if (wave_ballot(pos_any) == 0ull) {
          keep &= ~(1u << (kt & 31));
        } else {
          // pairs of the tile pass are in no column bucket: the key-major backward walks the lists
          if (P.colcnt && l == 0) atomicOr(P.colcnt + (int64_t)bh * P.nkt + kt, kColTaint);
          ++computed;
        }
        // A V on every tile the row keeps (a tile of zero weights adds zero products: the same
        // sums bit for bit, and no branch around the accumulators)
        const bf16x8 PF0 = PolBF16::pack_c(C, 0), PF1 = PolBF16::pack_c(C, 1);
        const bf16* vp = vst + voff;
#pragma unroll
        for (int c = 0; c < ND; ++c) {
          O[c] = PolBF16::mma(tr_frag<VS>(vp + 32 * c), PF0, O[c]);
          O[c] = PolBF16::mma(tr_frag<VS>(vp + 32 * c + 16 * VS), PF1, O[c]);
        }
      }
      if (kt2 < 0 || nw != cw) {  // the own row's word cw is done
        if (act && (WALK || keep != cown) && l == 0) orow0[(int64_t)wv * P.occ_w + cw] = keep;
        cw = nw;
        cown = keep = nown;
      }
      kt = kt2;
    }
    if (WALK && act && l == 0) {  // the own row's words past its last key tile (no screen wrote them)
      for (int w = (kt_last(qt, qoff, P.nkt) >> 5) + 1; w < P.occ_w; ++w) orow0[(int64_t)wv * P.occ_w + w] = 0u;
    }
    if (pent) {
      npairs += wave_sum_u32(extra);
      if (l == 0) P.pairs[pair_lists(P.nbr, BH, nqt) * 4 * kPairCap + lidx] = npairs;
    }
  }

  if (ZR) {
    // the call's zero range (the backward's gradients in training): the workgroup's even share of
    // the 16-byte units, streaming stores that drain while other workgroups still compute (the
    // host picks ZR only for shares of at most 65536 units)
    // (units / nwg each, the first units % nwg one more; no product that could pass 64 bits)
    const int64_t nwg = gridDim.x, per = P.zero_units / nwg, extra = P.zero_units % nwg, bid = blockIdx.x;
    u32x4* zbase = reinterpret_cast<u32x4*>(P.zero) + (bid * per + min(bid, extra));
    const uint32_t zn = (uint32_t)(per + (bid < extra ? 1 : 0));
    for (uint32_t u = threadIdx.x; u < zn; u += 64 * W) __builtin_nontemporal_store(u32x4{0u, 0u, 0u, 0u}, zbase + u);
  }

  // Output rows through LDS (the wave's slice of the ring, free once every wave has passed the
  // barrier below): lane (n, g) holds elements 32c + crow(r, g) of row n; stores then cover whole
  // rows, 16 bytes per lane.
  __syncthreads();
  if (!act) return;
  bf16* ost = ring + wv * 32 * KS;
#pragma unroll
  for (int c = 0; c < ND; ++c)
#pragma unroll
    for (int u = 0; u < 4; ++u)
      store4(ost + n32 * KS + 32 * c + 8 * u + 4 * g, O[c][4 * u], O[c][4 * u + 1], O[c][4 * u + 2], O[c][4 * u + 3]);
  wave_lds_sync();
  {
    bf16* ohead = (bf16*)P.out + (int64_t)b * P.s[F_OUT][0] + (int64_t)h * P.s[F_OUT][1];
    constexpr int OL = 32 / RPI;
#pragma unroll
    for (int i = 0; i < OL; ++i) {
      const int r = l / CPR + RPI * i, row = 32 * qt + r;
      if (row < Nq)
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4*>(ost + r * KS + 8 * vch),
                                    reinterpret_cast<u32x4*>(ohead + (int64_t)row * P.s[F_OUT][2] + 8 * vch));
    }
  }
  if (P.stats && l == 0 && checked) {
    if (WALK) atomicAdd(P.stats + 0, (unsigned long long)checked);  // every causal tile is tested
    atomicAdd(P.stats + 1, (unsigned long long)computed);
    atomicAdd(P.stats + 2, (unsigned long long)checked);
  }
}

// ------------------------------------------------------------------ fwd_pv_cand
// The exact pass of the query tiles whose candidate-key lists (every branch, normalised scores)
// fit: per branch the score tile of the query rows against the candidate keys' rows (row c =
// candidate c, rows past the count zero) is computed with the MFMA sequence of fwd_pv, its
// operands loaded straight from the rows (the same values in the same operands: bitwise the same
// scores); the candidates' V rows go to a swizzled LDS tile by direct loads, and the exact
// weights with the causal mask accumulate coef A V as in fwd_pv.  One gather round per branch
// replaces one per kept key tile.  With two branches each runs on its own wave of the workgroup
// (half the dependent loads per wave; LDS per wave as with one) and the second wave's sum is
// added to the first's through LDS before the first stores the rows.  The bitmask row is rewritten from the key tiles
// holding a non-zero weight; the pair list takes the non-zero weights in the order (value r,
// lane).
template <int D, int BR, int PK>
__global__ void __launch_bounds__(64 * BR) __attribute__((amdgpu_waves_per_eu(3))) fwd_pv_cand(FwdParams P) {
  constexpr int NT = D / 16, ND = D / 32;
  constexpr int CPR = D / 8;     // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;  // rows per load instruction
  constexpr int VL = 32 / RPI;   // load instructions per tile
  // one wave per branch, each with its own tiles
  __shared__ __attribute__((aligned(16))) bf16 vts[BR][32 * D];  // V rows, chunk-swizzled (bswz)
  __shared__ __attribute__((aligned(16))) int ckeys[BR][32];     // candidate keys (padding: -1)
  __shared__ __attribute__((aligned(16))) float crks[BR][32];   // their inverse norms
  __shared__ __attribute__((aligned(16))) u32x4 plists[BR][kPairCap];  // the branch's pair list

  const int l = lane_id(), n32 = l & 31, g = l >> 5;
  const int wv = BR == 2 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) : 0;  // = its branch
  bf16* vt = vts[wv];
  int* ckey = ckeys[wv];
  float* crk = crks[wv];
  u32x4* plist = plists[wv];
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
  int kraw = (int)P.cand[(((int64_t)(BR == 2 ? (l >> 5) : 0) * BH + bh) * nqt + qt) * kCandCap + (l & 31)];
  bool fit = true;
#pragma unroll
  for (int br = 0; br < BR; ++br) fit = fit && nc[br] <= (uint32_t)kCandCap;
  if (!fit) {  // fwd_pv walks the bitmask tiles (both waves leave: the test is the same)
    if (l == 0 && wv == 0) P.pvq[1 + atomicAdd(P.pvq, 1u)] = (uint32_t)(bh * nqt + qt);
    return;
  }
  if (P.screen_items > (Nq + 255) / 256) {
    // the screen split some key ranges over several items, which append in any order: sort each
    // list (lanes 0-31: branch 0, lanes 32-63: branch 1; its keys are distinct) by rank
    const int half = BR == 2 ? (l >> 5) : 0;
    const uint32_t nh = nc[BR == 2 ? half : 0];
    int rank = l & 31;
    if ((uint32_t)(l & 31) < nh) {
      rank = 0;
      for (int f = 0; f < 32; ++f) {
        const int a = __builtin_amdgcn_readlane(kraw, f), c = __builtin_amdgcn_readlane(kraw, 32 + f);
        rank += ((uint32_t)f < nh && (half ? c : a) < kraw) ? 1 : 0;
      }
    }
    kraw = __builtin_amdgcn_ds_permute(4 * ((l & 32) + rank), kraw);
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

  {
    const int br = wv;
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
      wave_lds_sync();
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
              plist[slot] = u32x4{(uint32_t)key, (uint32_t)n32, __builtin_bit_cast(uint32_t, x), kNoSlot};
            npairs += (uint32_t)__builtin_popcountll(bal);
          }
        }
      // The list's entries, lane e for entry e: with column buckets each takes a slot in the
      // bucket of its key tile (the adds are in flight during the products below) and the entry
      // records it; a list past the cap taints the columns of every candidate with a non-zero
      // weight instead (its pairs past the cap are in no list).
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
      }
      if (cnz) {
        const bf16x8 PF0 = PolBF16::pack_c(C, 0), PF1 = PolBF16::pack_c(C, 1);
#pragma unroll
        for (int c = 0; c < ND; ++c) {
          O[c] = PolBF16::mma(tile_tr_frag<D>(vt, 0, c), PF0, O[c]);
          O[c] = PolBF16::mma(tile_tr_frag<D>(vt, 1, c), PF1, O[c]);
        }
      }
      if (pent && (uint32_t)l < ne) {
        *reinterpret_cast<u32x4*>(pent + 4 * l) = pe;
        if (ccol && pe[3] < (uint32_t)kColCap)
          *reinterpret_cast<u32x4*>(P.colbuf + (((int64_t)bh * P.nkt + ((int)pe[0] >> 5)) * kColCap + pe[3]) * 4) =
              u32x4{((uint32_t)(32 * qt) + pe[1]) | (br ? 0x80000000u : 0u), pe[0] & 31u, pe[2], 0u};
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
      wave_lds_sync();  // the tile is reused by the output
    }
    if (P.pairs && l == 0) P.pairs[pair_lists(P.nbr, BH, nqt) * 4 * kPairCap + lidx] = npairs;
  }
  if (P.stats) {
    const float cs = wave_sum((float)computed), ks = wave_sum((float)checked);
    if (l == 0 && ks > 0.f) {
      atomicAdd(P.stats + 1, (unsigned long long)cs);
      atomicAdd(P.stats + 2, (unsigned long long)ks);
    }
  }
  if constexpr (BR == 2) {
    // out = O (branch 1's wave, -lambda A2 V) + O (branch 0's wave, A1 V): the second through
    // the (now unused) V tiles of both waves, then the first wave stores the rows
    static_assert(BR * 32 * D * 2 >= 64 * 16 * ND * 4, "accumulators fit the tiles");
    float* xch = reinterpret_cast<float*>(&vts[0][0]);
    __syncthreads();  // both waves are done with their tiles
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

  // Output rows through LDS (the V tile's space): lane (n, g) holds elements 32c + crow(r, g) of
  // row n, i.e. half g of chunk k = 4c + u for values 4u .. 4u + 3.  Its 8 bytes go to half-chunk
  // 2 (k ^ osig(n)) + (g ^ otau(n)) of the row: the two halves of chunk k share a 16-byte slot
  // (swapped when otau(n) = 1) and the 32 rows of a half-wave's store fall on distinct banks (with
  // the tile's 16-byte swizzle they met in pairs, two extra cycles per store); the row reads then
  // take 16-byte slots, and the stores cover whole rows (streaming stores, as in fwd_pv: nothing
  // here reads the output again).
  auto osig = [](int r) { return (r >> 1) & (CPR - 1); };
  auto otau = [](int r) { return D == 128 ? (r & 1) : ((r >> 4) & 1); };
  wave_lds_sync();
#pragma unroll
  for (int c = 0; c < ND; ++c)
#pragma unroll
    for (int u = 0; u < 4; ++u)
      store4(vt + n32 * D + 4 * (2 * ((4 * c + u) ^ osig(n32)) + (g ^ otau(n32))), O[c][4 * u], O[c][4 * u + 1],
             O[c][4 * u + 2], O[c][4 * u + 3]);
  wave_lds_sync();
  {
    bf16* ohead = (bf16*)P.out + (int64_t)b * P.s[F_OUT][0] + (int64_t)h * P.s[F_OUT][1];
#pragma unroll
    for (int i = 0; i < VL; ++i) {
      const int r = vrow + RPI * i, row = 32 * qt + r;
      u32x4 w = *reinterpret_cast<const u32x4*>(vt + r * D + 8 * (vch ^ osig(r)));
      if (otau(r)) w = u32x4{w[2], w[3], w[0], w[1]};
      if (row < Nq)
        __builtin_nontemporal_store(w, reinterpret_cast<u32x4*>(ohead + (int64_t)row * P.s[F_OUT][2] + 8 * vch));
    }
  }
}

// ------------------------------------------------------------------ dispatch
template <int D, int BR, int PK, bool NORM>
int launch_sparse_t(const FwdParams& p, hipStream_t s) {
  const int BH = p.B * p.H;
  if constexpr (NORM) {
    constexpr int rows = (64 / (D / 16)) * kn_groups<D>();  // rows per wave
    const int64_t waves = (int64_t)BR * BH * ((p.Nk + rows - 1) / rows);
    hipLaunchKernelGGL((key_prep<D, bf16>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, p, BR);
    launched(s, "key_prep");
  }
  if constexpr (!NORM) {
    // without normalisation every query tile runs the block tile pass over all its causal key
    // tiles (its scores decide the weights and write the bitmask; a screen would compute the
    // same scores once more); it also clears the call's zero range when each workgroup's share
    // is at most 1 MiB (a training step's gradients: 48 d units of 16 bytes per workgroup), else
    // zero_range clears it across the whole GPU afterwards
    const unsigned blocks = (unsigned)(BH * ((p.nqt + kBlkTiles - 1) / kBlkTiles));
    const bool zr = p.zero && p.zero_units > 0 && p.zero_units <= (int64_t)blocks * 65536;
    if (zr)
      hipLaunchKernelGGL((fwd_pv_blk<D, BR, PK, NORM, true, true>), dim3(blocks), dim3(64 * kBlkTiles), 0, s, p);
    else
      hipLaunchKernelGGL((fwd_pv_blk<D, BR, PK, NORM, true>), dim3(blocks), dim3(64 * kBlkTiles), 0, s, p);
    launched(s, "fwd_pv");
    const int e = (int)hipGetLastError();
    return e || zr ? e : launch_zero(p, s);
  } else {
    const dim3 grid((unsigned)(BR * BH) * (unsigned)p.screen_items);
    hipLaunchKernelGGL((fwd_screen_i8<D, bf16>), grid, dim3(256), 0, s, p, BR);
    launched(s, "fwd_screen");
    if (p.cand) {
      hipLaunchKernelGGL((fwd_pv_cand<D, BR, PK>), dim3((unsigned)(BH * p.nqt)), dim3(64 * BR), 0, s, p);
      launched(s, "fwd_pv_cand");
      // the query tiles the candidate pass could not take, from its queue
      const int items = BH * p.nqt;
      hipLaunchKernelGGL((fwd_pv<D, BR, PK, NORM>), dim3((unsigned)(items < 2048 ? items : 2048)), dim3(64), 0, s, p, 0);
    } else {  // every query tile runs: blocks of query tiles sharing their key tiles
      const unsigned blocks = (unsigned)(BH * ((p.nqt + kBlkTiles - 1) / kBlkTiles));
      hipLaunchKernelGGL((fwd_pv_blk<D, BR, PK, NORM>), dim3(blocks), dim3(64 * kBlkTiles), 0, s, p);
    }
    launched(s, "fwd_pv");
    return (int)hipGetLastError();
  }
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

// The int8 screen over fp32 rows, for the normalised fp32 pass (fwd_wave in its screened form,
// tda_fwd.hip): key_prep and fwd_screen_i8 read the fp32 inputs and write the norms table and a
// bitmask that keeps every tile holding a non-zero weight.  No candidate lists: the fp32 pass
// walks the bitmask.
int launch_fwd_screen_f32(const FwdParams& p0, const KernelKey& k, void* stream) {
  hipStream_t s = (hipStream_t)stream;
  FwdParams p = p0;  // with candidate lists: the fp32 candidate pass reads them
  const int BR = k.branches, BH = p.B * p.H;
  const dim3 grid((unsigned)(BR * BH) * (unsigned)p.screen_items);
  auto run = [&](auto dc) {
    constexpr int D = decltype(dc)::value;
    constexpr int rows = (64 / (D / 16)) * kn_groups<D>();  // rows per wave
    const int64_t waves = (int64_t)BR * BH * ((p.Nk + rows - 1) / rows);
    hipLaunchKernelGGL((key_prep<D, float>), dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, s, p, BR);
    launched(s, "key_prep");
    hipLaunchKernelGGL((fwd_screen_i8<D, float>), grid, dim3(256), 0, s, p, BR);
    launched(s, "fwd_screen");
  };
  if (k.d == 128) run(std::integral_constant<int, 128>{});
  else run(std::integral_constant<int, 64>{});
  return (int)hipGetLastError();
}

}  // namespace tda
