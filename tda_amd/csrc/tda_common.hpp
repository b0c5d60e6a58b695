// tda_common.hpp -- device building blocks shared by the gfx950 threshold-attention kernels.
//
// Matrix-core conventions (CDNA3/CDNA4 32x32 MFMA family, wave64):
//   C/D (32x32 fp32, 16 values per lane): lane l holds column n = l % 32 and,
//       in value r (0..15), row  crow(r, g) = 8*(r/4) + 4*g + (r%4),  g = l / 32.
//   A (M x K): lane l holds row m = l % 32 and E consecutive K indices starting at E*g.
//   B (K x N): lane l holds column n = l % 32 and E consecutive K indices starting at E*g.
// bf16 uses v_mfma_f32_32x32x16_bf16 (K = 16 per instruction, E = 8 elements per lane);
// fp32 uses v_mfma_f32_32x32x2f32 (K = 2, E = 1; over d its row fragments take the elements in
// another order, see PolF32::load_rows).
//
// Two operand shapes appear in every kernel:
//   * "row fragments": a 32-row tile of a (N, d) tensor contracted over d.  Lane (m, g) holds
//     row m, elements d = KS*t + E*g + [0, E) for step t.  Rows load straight from HBM.
//   * "transposed fragments": the same kind of tile contracted over its rows (the sequence
//     axis), with lane (n, g) holding column d = n.  For step s, element j sits at tile row
//     crow(s*E + j, g): that matches the C layout of a score tile, so a score tile in
//     registers feeds the next MFMA as the B operand with no data movement (pack_c below).
//     bf16 stages such a tile through LDS in a transposed, row-permuted layout; fp32 reads
//     its single element per step straight from memory.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tda {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float kNormEps = 1e-12f;  // torch.nn.functional.normalize default eps

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

// Row of C value r for lane group g (see header comment).
__device__ __forceinline__ constexpr int crow(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

// ------------------------------------------------------------------ MFMA policies
struct PolBF16 {
  using T = bf16;
  using frag = bf16x8;
  static constexpr int KS = 16;  // contraction length of one instruction
  static constexpr int E = 8;    // operand elements per lane
  __device__ __forceinline__ static f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static frag zero() { return frag{}; }
  // Row-fragment step t of a row whose first element is `row` (null -> zeros).
  __device__ __forceinline__ static frag load_row(const T* row, int t, int g) {
    if (!row) return zero();
    return *reinterpret_cast<const frag*>(row + KS * t + E * g);
  }
  // All NT = D / KS steps of a row.
  template <int NT>
  __device__ __forceinline__ static void load_rows(const T* row, int g, frag (&out)[NT]) {
#pragma unroll
    for (int t = 0; t < NT; ++t) out[t] = load_row(row, t, g);
  }
  // acc += (row fragments, streamed from `row`) x (resident fragments b), over the NT steps.
  template <int NT>
  __device__ __forceinline__ static f32x16 mma_row(const T* row, int g, const frag (&b)[NT], f32x16 acc) {
#pragma unroll
    for (int t = 0; t < NT; ++t) acc = mma(load_row(row, t, g), b[t], acc);
    return acc;
  }
  // Pack values [s*E, s*E+E) of a C tile into a B operand (round to nearest even).
  __device__ __forceinline__ static frag pack_c(const f32x16& c, int s) {
    frag f;
#pragma unroll
    for (int j = 0; j < E; ++j) f[j] = (bf16)c[s * E + j];
    return f;
  }
  __device__ __forceinline__ static float sumsq(frag f) {
    float a = 0.f;
#pragma unroll
    for (int j = 0; j < E; ++j) { float x = (float)f[j]; a = __builtin_fmaf(x, x, a); }
    return a;
  }
};

struct PolF32 {
  using T = float;
  using frag = float;
  static constexpr int KS = 2;
  static constexpr int E = 1;
  __device__ __forceinline__ static f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  __device__ __forceinline__ static frag zero() { return 0.f; }
  // All NT = D / 2 steps of a row: lane half g takes elements g NT .. g NT + NT - 1, one per
  // step (a contraction over d may assign the elements to steps in any order, the same for both
  // operands; every fp32 contraction over d takes both from load_rows).  16-byte loads.
  template <int NT>
  __device__ __forceinline__ static void load_rows(const T* row, int g, frag (&out)[NT]) {
    static_assert(NT % 4 == 0, "whole 16-byte vectors");
    if (!row) {
#pragma unroll
      for (int t = 0; t < NT; ++t) out[t] = 0.f;
      return;
    }
    const f32x4* p = reinterpret_cast<const f32x4*>(row + g * NT);
#pragma unroll
    for (int m = 0; m < NT / 4; ++m) {
      const f32x4 v = p[m];
#pragma unroll
      for (int e = 0; e < 4; ++e) out[4 * m + e] = v[e];
    }
  }
  // acc += (row fragments, streamed from `row` four steps per 16-byte load) x b, over NT steps.
  template <int NT>
  __device__ __forceinline__ static f32x16 mma_row(const T* row, int g, const frag (&b)[NT], f32x16 acc) {
    const f32x4* p = reinterpret_cast<const f32x4*>(row ? row + g * NT : row);
#pragma unroll
    for (int m = 0; m < NT / 4; ++m) {
      const f32x4 v = row ? p[m] : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = mma(v[e], b[4 * m + e], acc);
    }
    return acc;
  }
  __device__ __forceinline__ static frag pack_c(const f32x16& c, int s) { return c[s]; }
  __device__ __forceinline__ static float sumsq(frag f) { return f * f; }
};

// ------------------------------------------------------------------ tensors
template <class T>
struct TRef {
  T* p;
  int64_t sb, sh, st;  // element strides of the batch, head and sequence axes (d stride == 1)
  __device__ __forceinline__ T* row(int b, int h, int t) const {
    return p + (int64_t)b * sb + (int64_t)h * sh + (int64_t)t * st;
  }
};

// ------------------------------------------------------------------ threshold and power
// c_i = sqrt(2 ln(i+1) / d); tau_i = beta * c_i  (reference: TTA:59-63)
__device__ __forceinline__ float tau_coeff(int i, float inv_d) {
  return sqrtf(2.0f * logf((float)i + 1.0f) * inv_d);
}

// x^p and d(x^p)/dx for x > 0.  PK: 2 -> p == 2, 1 -> p == 1, 0 -> general p via
// 2^(p log2 x) on the hardware exp2/log2 units.
template <int PK>
__device__ __forceinline__ float pow_p(float x, float p) {
  if constexpr (PK == 2) return x * x;
  else if constexpr (PK == 1) return x;
  else return __builtin_amdgcn_exp2f(p * __builtin_amdgcn_logf(x));
}
template <int PK>
__device__ __forceinline__ float dpow_p(float x, float p) {
  if constexpr (PK == 2) return 2.0f * x;
  else if constexpr (PK == 1) return 1.0f;
  else return p * __builtin_amdgcn_exp2f((p - 1.0f) * __builtin_amdgcn_logf(x));
}

__device__ __forceinline__ float clamp01(float x) { return fminf(fmaxf(x, 0.0f), 1.0f); }

// inverse row norm 1/max(|x|, eps) from a sum of squares
__device__ __forceinline__ float inv_norm(float ss) { return 1.0f / fmaxf(sqrtf(ss), kNormEps); }

// Sum over the lane's row fragments plus the partner lane (l ^ 32), which holds the rest of
// the row: every lane ends with the full sum of squares of its row.
template <class Pol, int NT>
__device__ __forceinline__ float row_sumsq(const typename Pol::frag (&f)[NT]) {
  float a = 0.f;
#pragma unroll
  for (int t = 0; t < NT; ++t) a += Pol::sumsq(f[t]);
  return a + __shfl_xor(a, 32);
}

__device__ __forceinline__ unsigned long long wave_ballot(bool b) { return __ballot(b); }


// Sum / maximum over aligned groups of W lanes (W = 2, 4, 8 or 16) by DPP moves within a 16-lane
// row (no LDS round trip): quad_perm [1,0,3,2] and [2,3,0,1] pair lanes within quads, then
// row_half_mirror (lane i <- 7 - i) and row_mirror (i <- 15 - i) pair quads and half-rows.  Each
// step adds two values in either order, so every lane of a group ends with the same bits.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
template <int W>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(W == 2 || W == 4 || W == 8 || W == 16, "group of 2..16 lanes");
  x += dpp_mov<0xB1>(x);
  if constexpr (W >= 4) x += dpp_mov<0x4E>(x);
  if constexpr (W >= 8) x += dpp_mov<0x141>(x);
  if constexpr (W >= 16) x += dpp_mov<0x140>(x);
  return x;
}
// Wave-wide sum, deterministic: DPP within each 16-lane row, then two lane swaps (every lane
// ends with the same bits).  Call with every lane active.
__device__ __forceinline__ float wave_sum(float v) {
  v = group_sum<16>(v);
  v += __shfl_xor(v, 16);
  return v + __shfl_xor(v, 32);
}
// Workgroup barrier for hand-offs through LDS only: the wave's LDS operations complete
// (lgkmcnt(0)), then s_barrier; the wavefront-scope fences keep the compiler from moving memory
// operations across it.  __syncthreads()'s workgroup release fence also waits for every
// outstanding global load and store (vmcnt(0)), which would drain loads issued ahead (into
// registers, or into LDS by direct loads whose own completion the caller waits for); here they
// stay in flight.  Not for data handed over through global memory.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt at their maxima (no wait)
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
// Wave-wide integer sum (every lane ends with the total).  Call with every lane active.
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) v += (uint32_t)__shfl_xor((int)v, m);
  return v;
}
// Wave-wide OR, the same way.
__device__ __forceinline__ uint32_t wave_or(uint32_t v) {
  v |= (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
  v |= (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
  v |= (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false);
  v |= (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false);
  v |= (uint32_t)__shfl_xor((int)v, 16);
  return v | (uint32_t)__shfl_xor((int)v, 32);
}
template <int W>
__device__ __forceinline__ float group_max(float x) {
  static_assert(W == 2 || W == 4 || W == 8 || W == 16, "group of 2..16 lanes");
  x = fmaxf(x, dpp_mov<0xB1>(x));
  if constexpr (W >= 4) x = fmaxf(x, dpp_mov<0x4E>(x));
  if constexpr (W >= 8) x = fmaxf(x, dpp_mov<0x141>(x));
  if constexpr (W >= 16) x = fmaxf(x, dpp_mov<0x140>(x));
  return x;
}

// ------------------------------------------------------------------ transposed tiles
// A 32-row x D tile used as the A operand of a contraction over its rows.
// bf16: staged in (wave-private) LDS as T[d][pos(row)], pos() swapping bits 2 and 3 of the
// row index, row stride TS elements.  Then the E = 8 elements of step s for lane group g
// (tile rows crow(8s + j, g), j = 0..7) are the 8 contiguous positions 16s + 8g + j.
template <int D>
struct TTileBF16 {
  static constexpr int TS = 40;  // 32 positions + 8 padding: 80-byte rows, conflict-free b128 reads
  static constexpr int ELEMS = D * TS;
  bf16* lds;

  __device__ __forceinline__ static int pos4(int a) {  // position of row 4a (a = 0..7)
    return 4 * ((a & 4) | ((a & 1) << 1) | ((a >> 1) & 1));
  }
  // Stage rows r0..r0+31 of the tensor `base` (rows >= n read as zeros) into LDS.
  __device__ __forceinline__ void stage(const TRef<const bf16>& x, int b, int h, int r0, int n) const {
    const int l = lane_id();
#pragma unroll
    for (int it = 0; it < D / 64; ++it) {
      const int mt = l + 64 * it;      // micro-tile: 4 rows x 8 columns
      const int a = mt / (D / 8);      // row group (rows 4a..4a+3)
      const int d0 = (mt % (D / 8)) * 8;
      bf16x8 v[4];
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int r = r0 + 4 * a + c;
        v[c] = (r < n) ? *reinterpret_cast<const bf16x8*>(x.row(b, h, r) + d0) : bf16x8{};
      }
      const int p = pos4(a);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        bf16x4 w = {v[0][j], v[1][j], v[2][j], v[3][j]};
        *reinterpret_cast<bf16x4*>(lds + (d0 + j) * TS + p) = w;
      }
    }
  }
  __device__ __forceinline__ bf16x8 frag(int s, int dsub) const {
    const int l = lane_id();
    return *reinterpret_cast<const bf16x8*>(lds + (32 * dsub + (l & 31)) * TS + 16 * s + 8 * (l >> 5));
  }
};

// fp32: the single element of step s for lane (n, g) is X[r0 + crow(s, g)][32 dsub + n],
// read straight from memory (coalesced over n).
template <int D>
struct TTileF32 {
  TRef<const float> x;
  int b, h, r0, n;
  __device__ __forceinline__ void set(const TRef<const float>& x_, int b_, int h_, int r0_, int n_) {
    x = x_; b = b_; h = h_; r0 = r0_; n = n_;
  }
  __device__ __forceinline__ float frag(int s, int dsub) const {
    const int l = lane_id();
    const int r = r0 + crow(s, l >> 5);
    return (r < n) ? x.row(b, h, r)[32 * dsub + (l & 31)] : 0.f;
  }
};

// Make LDS writes of this wave visible to its own later LDS reads (and order reads before
// later overwrites).  LDS instructions of one wave execute in order; the fences keep the
// compiler from reordering across the hand-off and wait for outstanding LDS traffic.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Store 4 consecutive output elements (fp32 accumulators -> T).
__device__ __forceinline__ void store4(bf16* p, float a, float b, float c, float d) {
  bf16x4 w = {(bf16)a, (bf16)b, (bf16)c, (bf16)d};
  *reinterpret_cast<bf16x4*>(p) = w;
}
__device__ __forceinline__ void store4(float* p, float a, float b, float c, float d) {
  *reinterpret_cast<f32x4*>(p) = f32x4{a, b, c, d};
}
__device__ __forceinline__ f32x4 load4(const bf16* p) {
  bf16x4 w = *reinterpret_cast<const bf16x4*>(p);
  return f32x4{(float)w[0], (float)w[1], (float)w[2], (float)w[3]};
}
__device__ __forceinline__ f32x4 load4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }


// ------------------------------------------------------------------ swizzled LDS tiles
#define LDS_PTR(T, p) ((__attribute__((address_space(3))) T*)(p))
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

// 16-byte chunk swizzle of a row-major 32-row tile (D/8 chunks per row).  Conflict-free for the
// row-fragment reads (32 rows, one chunk each) and for the transpose reads (4 rows x 2 chunks
// per 16 lanes), with 32 or 64 banks.
template <int D>
__device__ __forceinline__ int bswz(int r) {
  if constexpr (D == 128) return (r ^ (4 * (r & 3))) & 15;
  else return ((r ^ (r >> 1)) ^ (2 * (r & 1)) ^ (4 * ((r >> 1) & 1))) & 7;
}

// Transposed fragment (step st over the 32 rows, column block dsub): lane (n, g) gets column
// 32*dsub + n at tile rows crow(8*st + j, g), j = 0..7.
template <int D>
__device__ __forceinline__ bf16x8 tile_tr_frag(const bf16* tile, int st, int dsub) {
  const int l = lane_id(), bk = l >> 4, j = l & 15;
  const int d = 32 * dsub + 16 * (bk & 1) + 4 * (j & 3);
  bf16x8 out;
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int r = 16 * st + 8 * hh + 4 * (bk >> 1) + (j >> 2);
    const bf16* p = tile + r * D + 8 * ((d >> 3) ^ bswz<D>(r)) + (d & 7);
    const bf16x4 w = __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_PTR(s16x4, p)));
#pragma unroll
    for (int e = 0; e < 4; ++e) out[4 * hh + e] = w[e];
  }
  return out;
}

}  // namespace tda
