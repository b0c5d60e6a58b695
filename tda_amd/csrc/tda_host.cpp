// tda_host.cpp -- C ABI of libtda_hip.so: argument validation, buffer sizing and dispatch.
//
// Replaces the host side of the reference (snap-research/TDA triton_threshold_attention.py):
// ThresholdRelaFunction.forward/backward (TTA:336-469) and their Triton launches
// (TTA:374-389, TTA:433-460).  Unlike the reference, beta and lambda stay on the device (no
// .item() synchronisation, TTA:352), nothing is up-cast or copied (TTA:356-360), and every
// argument is checked before any GPU work (the reference only asserts equal shapes, TTA:348).
#include <cmath>
#include <cstdint>
#include <cstring>

#include "../../include/tda.h"
#include "tda_params.hpp"

namespace {

thread_local int32_t g_last_hip_error = 0;

constexpr int64_t kMaxSeqStride = int64_t(1) << 25;

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

int32_t check_tensor(const tda_tensor& t, int64_t elem_bytes) {
  if (!t.data) return TDA_ERR_NULL_POINTER;
  if (t.stride[3] != 1) return TDA_ERR_LAYOUT;
  if (reinterpret_cast<uintptr_t>(t.data) % 16 != 0) return TDA_ERR_LAYOUT;
  for (int k = 0; k < 3; ++k) {
    if (t.stride[k] < 0) return TDA_ERR_LAYOUT;
    if ((t.stride[k] * elem_bytes) % 16 != 0) return TDA_ERR_LAYOUT;
  }
  // 32 rows of a tile span less than 2^31 bytes: the kernels address a tile with 32-bit offsets
  if (t.stride[2] > kMaxSeqStride) return TDA_ERR_LAYOUT;
  return TDA_OK;
}

struct Common {
  int32_t abi_version, dtype, branches, normalize, causal;
  float relu_power;
  int64_t batch, heads, seq_len, head_dim;
  const float* beta;
  const float* lambda_param;
  int64_t seq_len_kv, q_offset;  // seq_len_kv resolved (0 -> seq_len)
};

constexpr int64_t kMaxPos = (int64_t(1) << 30) - 64;  // positions and row counts stay in int32

int32_t check_common(const Common& c) {
  if (c.abi_version != TDA_ABI_VERSION) return TDA_ERR_ABI;
  if (c.dtype != TDA_DTYPE_F32 && c.dtype != TDA_DTYPE_BF16) return TDA_ERR_DTYPE;
  if (c.branches != 1 && c.branches != 2) return TDA_ERR_BRANCHES;
  if (c.causal != 1) return TDA_ERR_CAUSAL;
  if (c.head_dim != 64 && c.head_dim != 128 && c.head_dim != 256) return TDA_ERR_HEAD_DIM;
  if (c.batch < 1 || c.heads < 1 || c.seq_len < 1) return TDA_ERR_SHAPE;
  if (c.seq_len > (int64_t(1) << 30)) return TDA_ERR_SHAPE;
  if (c.batch * c.heads > (int64_t(1) << 24)) return TDA_ERR_SHAPE;
  if (c.batch * c.heads * ceil_div(c.seq_len, 32) > (int64_t(1) << 31) - 4) return TDA_ERR_SHAPE;
  if (c.q_offset < 0 || c.seq_len_kv < 1 || c.seq_len_kv > kMaxPos || c.q_offset + c.seq_len > kMaxPos)
    return TDA_ERR_OFFSET;
  if (c.batch * c.heads * ceil_div(c.seq_len_kv, 32) > (int64_t(1) << 31) - 4) return TDA_ERR_SHAPE;
  if (!std::isfinite(c.relu_power) || c.relu_power < 0.f) return TDA_ERR_POWER;
  if (!c.beta) return TDA_ERR_NULL_POINTER;
  if (c.branches == 2 && !c.lambda_param) return TDA_ERR_NULL_POINTER;
  return TDA_OK;
}

int64_t round256(int64_t x) { return (x + 255) / 256 * 256; }

// Forward workspace: the bitmask scratch used when the caller asks for no occupancy output
// (the bf16 forward always builds the bitmask: its second pass reads it).
int64_t occ_words(int64_t bh, int64_t seq_len, int64_t seq_len_kv, int64_t branches) {
  return branches * bh * ceil_div(seq_len, 32) * ceil_div(ceil_div(seq_len_kv, 32), 32);
}
// Forward workspace: the bitmask scratch (used when the caller asks for no occupancy output;
// the bf16 forward always builds the bitmask), then, when there is a single query tile
// (seq_len <= 32), the per-chunk partial outputs of the bf16 decode kernels:
// [B*H][ceil(key tiles / 32)][seq_len][128] floats (head_dim <= 128) ...
int64_t fwd_occ_bytes(int64_t bh, int64_t seq_len, int64_t seq_len_kv, int64_t branches) {
  return round256(occ_words(bh, seq_len, seq_len_kv, branches) * (int64_t)sizeof(uint32_t));
}
int64_t fwd_part_bytes(int64_t bh, int64_t seq_len, int64_t seq_len_kv) {
  if (seq_len > 32) return 0;
  return round256(bh * ceil_div(ceil_div(seq_len_kv, 32), 32) * seq_len * 128 * (int64_t)sizeof(float));
}
// ... or, with more than one query tile, the candidate lists of the bf16 screen.
// ... and a queue of query tiles for the tile pass (a count block, one item per (head, tile)).
int64_t fwd_cand_list_bytes(int64_t bh, int64_t seq_len, int64_t branches) {
  return round256(tda::cand_words(branches * bh * ceil_div(seq_len, 32)) * (int64_t)sizeof(uint32_t));
}
int64_t fwd_cand_bytes(int64_t bh, int64_t seq_len, int64_t branches) {
  if (seq_len <= 32) return 0;
  return fwd_cand_list_bytes(bh, seq_len, branches) +
         round256((64 + bh * ceil_div(seq_len, 32)) * (int64_t)sizeof(uint32_t));
}
// ... and, for the int8 screen (bf16 with normalisation, more than one query tile), the
// quantised key rows (kd bytes each, kd = head_dim) and their {scale, residual bound}.
int64_t fwd_k8_bytes(int64_t bh, int64_t seq_len, int64_t seq_len_kv, int64_t branches, int64_t kd) {
  if (seq_len <= 32 || kd == 0) return 0;
  return round256(branches * bh * seq_len_kv * kd) + round256(branches * bh * seq_len_kv * 8);
}
int64_t fwd_ws_bytes(int64_t bh, int64_t seq_len, int64_t seq_len_kv, int64_t branches, int64_t kd) {
  return fwd_occ_bytes(bh, seq_len, seq_len_kv, branches) + fwd_part_bytes(bh, seq_len, seq_len_kv) +
         fwd_cand_bytes(bh, seq_len, branches) + fwd_k8_bytes(bh, seq_len, seq_len_kv, branches, kd);
}
// Row bytes of the int8 keys a call needs (0: it uses none): the normalised calls, whose int8
// screen runs on bf16 and on fp32 rows, up to head_dim 128 (head_dim 256 has no screen).
int64_t k8_row_bytes(const tda_fwd_args& a) {
  return a.normalize && a.head_dim <= 128 ? a.head_dim : 0;
}
constexpr int64_t kMaxHeadDim = 128;  // the size functions without head_dim assume the largest
bool size_args_ok(int64_t batch, int64_t heads, int64_t seq_len, int64_t seq_len_kv, int32_t branches) {
  return batch >= 1 && heads >= 1 && seq_len >= 1 && seq_len_kv >= 1 && (branches == 1 || branches == 2);
}

int pkind_of(float p) { return p == 2.0f ? 2 : (p == 1.0f ? 1 : 0); }

template <class A>
Common common_of(const A& a) {
  return Common{a.abi_version, a.dtype, a.branches, a.normalize, a.causal, a.relu_power,
                a.batch, a.heads, a.seq_len, a.head_dim, a.beta, a.lambda_param,
                a.seq_len_kv ? a.seq_len_kv : a.seq_len, a.q_offset};
}

void copy_strides(int64_t dst[3], const tda_tensor& t) {
  dst[0] = t.stride[0];
  dst[1] = t.stride[1];
  dst[2] = t.stride[2];
}

}  // namespace

namespace tda {
void record_hip_error(int e) { g_last_hip_error = e; }
}  // namespace tda

// The column buckets of the pair buffer (tda_params.hpp), on both sides of a training step under
// the same condition: normalisation, head_dim up to 128 and more than one query tile (the bf16
// and fp32 candidate passes write them) and no more key tiles than query tiles (the buffer is
// sized for nqt columns).
template <class Params>
static void set_columns(Params& p, int64_t bh, int32_t branches, int32_t normalize, int64_t head_dim,
                        int64_t seq_len) {
  if (!p.pairs || !normalize || head_dim > 128 || seq_len <= 32 || p.nkt > p.nqt) return;
  uint32_t* cc = const_cast<uint32_t*>(p.pairs) + tda::pair_list_words(branches, bh, p.nqt);
  p.colcnt = cc;
  p.colbuf = cc + tda::col_count_words(bh, p.nqt);
}

extern "C" {

int32_t tda_abi_version(void) { return TDA_ABI_VERSION; }

int32_t tda_last_hip_error(void) { return g_last_hip_error; }

const char* tda_error_string(int32_t code) {
  switch (code) {
    case TDA_OK: return "ok";
    case TDA_ERR_NULL_POINTER: return "a required pointer is NULL";
    case TDA_ERR_SHAPE: return "batch, heads or seq_len out of range";
    case TDA_ERR_HEAD_DIM: return "head_dim must be 64, 128 or 256";
    case TDA_ERR_DTYPE: return "dtype must be float32 or bfloat16";
    case TDA_ERR_LAYOUT:
      return "tensor layout unsupported: last-dim stride must be 1, strides/pointers 16-byte aligned, "
             "sequence stride at most 2^25 elements";
    case TDA_ERR_POWER: return "relu_power must be finite and >= 0";
    case TDA_ERR_BRANCHES: return "branches must be 1 or 2";
    case TDA_ERR_WORKSPACE: return "workspace missing, too small or not 16-byte aligned";
    case TDA_ERR_ABI: return "abi_version mismatch";
    case TDA_ERR_CAUSAL: return "only the causal form is implemented (causal must be 1)";
    case TDA_ERR_NORMS: return "normalize requires the norms buffer (forward: output, backward: the forward's output)";
    case TDA_ERR_OFFSET: return "q_offset must be >= 0, and seq_len_kv and q_offset + seq_len at most 2^30 - 64";
    case TDA_ERR_SCRATCH:
      return "tda_fwd_noalloc: the call needs more workspace than the library's device array "
             "(TDA_NOALLOC_SCRATCH_BYTES, 16 MiB); use tda_fwd with a caller workspace";
    case TDA_ERR_HIP: return "HIP kernel launch failed";
    default: return "unknown error";
  }
}

size_t tda_occupancy_words_kv(int64_t batch, int64_t heads, int64_t seq_len, int64_t seq_len_kv,
                              int32_t branches) {
  if (!size_args_ok(batch, heads, seq_len, seq_len_kv, branches)) return 0;
  return (size_t)occ_words(batch * heads, seq_len, seq_len_kv, branches);
}

size_t tda_norms_floats_kv(int64_t batch, int64_t heads, int64_t seq_len, int64_t seq_len_kv,
                           int32_t branches) {
  if (!size_args_ok(batch, heads, seq_len, seq_len_kv, branches)) return 0;
  return (size_t)(branches * batch * heads * (seq_len + seq_len_kv));
}

size_t tda_fwd_workspace_bytes_kv(int64_t batch, int64_t heads, int64_t seq_len, int64_t seq_len_kv,
                                  int32_t branches) {
  if (!size_args_ok(batch, heads, seq_len, seq_len_kv, branches)) return 0;
  return (size_t)fwd_ws_bytes(batch * heads, seq_len, seq_len_kv, branches, kMaxHeadDim);
}

size_t tda_fwd_workspace_bytes_for(const tda_fwd_args* a) {
  if (!a) return 0;
  // the shape fields decide the size; the device pointers (beta, lambda) are not needed yet
  Common c = common_of(*a);
  c.beta = c.lambda_param = reinterpret_cast<const float*>(a);
  if (check_common(c) != TDA_OK) return 0;
  return (size_t)fwd_ws_bytes(a->batch * a->heads, a->seq_len, c.seq_len_kv, a->branches, k8_row_bytes(*a));
}

size_t tda_pair_words(int64_t batch, int64_t heads, int64_t seq_len, int32_t branches) {
  if (!size_args_ok(batch, heads, seq_len, seq_len, branches)) return 0;
  return (size_t)tda::pair_words(branches, batch * heads, ceil_div(seq_len, 32));
}

size_t tda_occupancy_words(int64_t batch, int64_t heads, int64_t seq_len, int32_t branches) {
  return tda_occupancy_words_kv(batch, heads, seq_len, seq_len, branches);
}

size_t tda_norms_floats(int64_t batch, int64_t heads, int64_t seq_len, int32_t branches) {
  return tda_norms_floats_kv(batch, heads, seq_len, seq_len, branches);
}

size_t tda_fwd_workspace_bytes(int64_t batch, int64_t heads, int64_t seq_len, int32_t branches) {
  return tda_fwd_workspace_bytes_kv(batch, heads, seq_len, seq_len, branches);
}

size_t tda_bwd_workspace_bytes(int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim) {
  (void)head_dim;
  if (batch < 1 || heads < 1 || seq_len < 1) return 0;
  // per (branch, head, query tile), for two branches: one (dbeta, dlambda) partial pair, then
  // the dk weight of each pair-list slot; then a queue of key tiles (a count and as many items
  // as dk weights; used when every key tile fits, i.e. Nk <= 64 Nq)
  const int64_t lists = 2 * batch * heads * ceil_div(seq_len, 32);
  return (size_t)(lists * (2 + tda::kPairCap) + 64 + lists * tda::kPairCap) * sizeof(float);
}

int32_t tda_validate_fwd(const tda_fwd_args* a) {
  if (!a) return TDA_ERR_NULL_POINTER;
  int32_t rc = check_common(common_of(*a));
  if (rc) return rc;
  const int64_t eb = a->dtype == TDA_DTYPE_BF16 ? 2 : 4;
  const tda_tensor* ts[] = {&a->q1, &a->k1, &a->v, &a->out, &a->q2, &a->k2};
  const int n = a->branches == 2 ? 6 : 4;
  for (int k = 0; k < n; ++k)
    if ((rc = check_tensor(*ts[k], eb))) return rc;
  if (a->normalize && !a->norms) return TDA_ERR_NORMS;
  if (!a->workspace || a->workspace_bytes < tda_fwd_workspace_bytes_for(a)) return TDA_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(a->workspace) % 16 != 0) return TDA_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(a->pairs) % 16 != 0) return TDA_ERR_LAYOUT;
  if (a->zero_bytes % 16 != 0 || reinterpret_cast<uintptr_t>(a->zero) % 16 != 0) return TDA_ERR_LAYOUT;
  if (a->zero_bytes && !a->zero) return TDA_ERR_NULL_POINTER;
  return TDA_OK;
}

int32_t tda_validate_bwd(const tda_bwd_args* a) {
  if (!a) return TDA_ERR_NULL_POINTER;
  int32_t rc = check_common(common_of(*a));
  if (rc) return rc;
  const int64_t eb = a->dtype == TDA_DTYPE_BF16 ? 2 : 4;
  const tda_tensor* ts[] = {&a->q1, &a->k1, &a->v, &a->dout, &a->dq1, &a->dk1, &a->dv, &a->q2, &a->k2, &a->dq2,
                            &a->dk2};
  const int n = a->branches == 2 ? 11 : 7;
  for (int k = 0; k < n; ++k)
    if ((rc = check_tensor(*ts[k], eb))) return rc;
  if (a->normalize && !a->norms) return TDA_ERR_NORMS;
  if (!a->workspace ||
      a->workspace_bytes < tda_bwd_workspace_bytes(a->batch, a->heads, a->seq_len, a->head_dim))
    return TDA_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(a->workspace) % 16 != 0) return TDA_ERR_WORKSPACE;
  if (reinterpret_cast<uintptr_t>(a->pairs) % 16 != 0) return TDA_ERR_LAYOUT;
  return TDA_OK;
}

int32_t tda_fwd(const tda_fwd_args* a, void* stream) {
  int32_t rc = tda_validate_fwd(a);
  if (rc) return rc;
  tda::FwdParams p;
  std::memset(&p, 0, sizeof(p));
  const tda_tensor* in[5] = {&a->q1, &a->k1, &a->q2, &a->k2, &a->v};
  const bool two = a->branches == 2;
  for (int k = 0; k < 5; ++k) {
    const tda_tensor& t = (!two && (k == 2 || k == 3)) ? *in[k - 2] : *in[k];
    p.in[k] = t.data;
    copy_strides(p.s[k], t);
  }
  p.out = a->out.data;
  copy_strides(p.s[tda::F_OUT], a->out);
  const Common c = common_of(*a);
  p.B = (int)a->batch;
  p.H = (int)a->heads;
  p.Nq = (int)a->seq_len;
  p.Nk = (int)c.seq_len_kv;
  p.qoff = (int)c.q_offset;
  p.nqt = (int)ceil_div(a->seq_len, 32);
  p.nkt = (int)ceil_div(c.seq_len_kv, 32);
  p.occ_w = (int)ceil_div(p.nkt, 32);
  p.p = a->relu_power;
  p.inv_d = 1.0f / (float)a->head_dim;
  p.beta = a->beta;
  p.lam = a->lambda_param;
  p.norms = a->normalize ? a->norms : nullptr;
  p.occ = a->occupancy ? a->occupancy : static_cast<uint32_t*>(a->workspace);
  char* after_occ = static_cast<char*>(a->workspace) +
                   fwd_occ_bytes(a->batch * a->heads, a->seq_len, c.seq_len_kv, a->branches);
  if (a->seq_len <= 32) p.part = reinterpret_cast<float*>(after_occ);
  else {
    const int64_t bh = a->batch * a->heads;
    p.cand = reinterpret_cast<uint32_t*>(after_occ);
    p.pvq = reinterpret_cast<uint32_t*>(after_occ + fwd_cand_list_bytes(bh, a->seq_len, a->branches));
    const int64_t kd = k8_row_bytes(*a);
    if (kd) {
      char* k8 = after_occ + fwd_cand_bytes(bh, a->seq_len, a->branches);
      p.k8 = reinterpret_cast<int8_t*>(k8);
      p.ksc = reinterpret_cast<float*>(k8 + round256(a->branches * bh * c.seq_len_kv * kd));
    }
  }
  p.stats = a->stats;
  p.pairs = a->pairs;
  p.nbr = a->branches;
  set_columns(p, a->batch * a->heads, a->branches, a->normalize, a->head_dim, a->seq_len);
  {
    // screen work items: a 256-row block's key tiles 0 .. n - 1 (n grows with the block) cut
    // into chunks of kc tiles; kc is the largest multiple of 32 (whole bitmask words) that still
    // gives at least kMinItems items, so that small problems spread over the whole GPU and no
    // item's chain of key tiles is much longer than the rest
    constexpr int64_t kMinItems = 1536;
    const int nqb = (p.Nq + 255) / 256;
    auto blk_tiles = [&](int qb) {
      const int qt = qb * 8 + 7 < p.nqt - 1 ? qb * 8 + 7 : p.nqt - 1;
      const int64_t t = ((int64_t)p.qoff + 32 * qt + 31) / 32;
      return (int)(t < p.nkt - 1 ? t : p.nkt - 1) + 1;
    };
    auto items = [&](int kc) {
      int64_t t = 0;
      for (int qb = 0; qb < nqb; ++qb) t += (blk_tiles(qb) + kc - 1) / kc;
      return t;
    };
    // at most 2^18 key tiles per item: an item's int8 key rows (32 x 128 bytes per tile) then
    // span under 2^30 bytes, within the screen's 32-bit buffer offsets
    constexpr int kMaxKc = 1 << 18;
    const int64_t streams = (int64_t)a->branches * a->batch * a->heads;
    int kc = (blk_tiles(nqb - 1) + 31) / 32 * 32;
    if (kc > kMaxKc) kc = kMaxKc;
    while (kc > 32 && streams * items(kc) < kMinItems) kc -= 32;
    p.screen_kc = kc;
    p.screen_items = (int)items(kc);
  }
  if (a->zero_bytes) {
    p.zero = a->zero;
    p.zero_units = (int64_t)(a->zero_bytes / 16);
    // the screen's workgroups walk sum over (branch, head, 256-row block) of its key tiles:
    // spread the units evenly over those steps
    int64_t steps = 0;
    for (int qb = 0; qb < (p.Nq + 255) / 256; ++qb) {
      const int qt = qb * 8 + 7 < p.nqt - 1 ? qb * 8 + 7 : p.nqt - 1;
      const int64_t last = (int64_t)p.qoff + 32 * qt + 31;  // last position of the block
      const int64_t klast = last / 32 < p.nkt - 1 ? last / 32 : p.nkt - 1;
      steps += klast + 1;
    }
    steps *= (int64_t)a->branches * a->batch * a->heads;
    // an item's slice (zero_per_it units per key tile, at most screen_kc tiles) is addressed
    // with 32-bit byte offsets: a range whose slices could reach 2^31 bytes (a large range
    // against a small problem) is cleared whole by zero_range instead (zero_per_it 0)
    const int64_t per_it = (p.zero_units + steps - 1) / steps;
    p.zero_per_it = per_it * 16 * p.screen_kc < (int64_t(1) << 31) ? (int)per_it : 0;
  }
  const tda::KernelKey key{a->dtype, (int)a->head_dim, a->branches, pkind_of(a->relu_power), a->normalize ? 1 : 0};
  tda::timing_begin(stream);
  int e = tda::launch_fwd(p, key, stream);
  const int te = tda::timing_end();
  if (e == 0) e = te;
  if (e != 0) {
    g_last_hip_error = e;
    return TDA_ERR_HIP;
  }
  return TDA_OK;
}

int32_t tda_bwd(const tda_bwd_args* a, void* stream) {
  int32_t rc = tda_validate_bwd(a);
  if (rc) return rc;
  tda::BwdParams p;
  std::memset(&p, 0, sizeof(p));
  const bool two = a->branches == 2;
  const tda_tensor* in[6] = {&a->q1, &a->k1, &a->q2, &a->k2, &a->v, &a->dout};
  for (int k = 0; k < 6; ++k) {
    const tda_tensor& t = (!two && (k == 2 || k == 3)) ? *in[k - 2] : *in[k];
    p.in[k] = t.data;
    copy_strides(p.s[k], t);
  }
  // Single-branch calls alias the second-branch gradient slots to the first: the kernels
  // never write them when branches == 1.
  const tda_tensor* gr[5] = {&a->dq1, &a->dk1, &a->dq2, &a->dk2, &a->dv};
  for (int k = 0; k < 5; ++k) {
    const tda_tensor& t = (!two && (k == 2 || k == 3)) ? *gr[k - 2] : *gr[k];
    p.grad[k] = t.data;
    copy_strides(p.s[tda::B_DQ1 + k], t);
  }
  const Common c = common_of(*a);
  p.B = (int)a->batch;
  p.H = (int)a->heads;
  p.Nq = (int)a->seq_len;
  p.Nk = (int)c.seq_len_kv;
  p.qoff = (int)c.q_offset;
  p.nqt = (int)ceil_div(a->seq_len, 32);
  p.nkt = (int)ceil_div(c.seq_len_kv, 32);
  p.occ_w = (int)ceil_div(p.nkt, 32);
  p.p = a->relu_power;
  p.inv_d = 1.0f / (float)a->head_dim;
  p.beta = a->beta;
  p.lam = a->lambda_param;
  p.dbeta = a->dbeta;
  p.dlam = a->dlambda;
  p.norms = a->normalize ? a->norms : nullptr;
  p.occ = a->occupancy;
  p.ws = static_cast<float*>(a->workspace);
  const int64_t lists = 2 * (int64_t)a->batch * a->heads * p.nqt;
  p.pws = p.ws + 2 * lists;  // after the partial pairs
  p.stats = a->stats;
  p.pairs = a->occupancy ? a->pairs : nullptr;  // the key-major pass finds the lists through the bitmask
  p.grads_zeroed = a->grads_zeroed ? 1 : 0;
  set_columns(p, (int64_t)a->batch * a->heads, a->branches, a->normalize, a->head_dim, a->seq_len);
  // the key-tile queue, when it holds every key tile
  if (p.pairs && (int64_t)a->batch * a->heads * p.nkt <= lists * tda::kPairCap)
    p.dkvq = reinterpret_cast<uint32_t*>(p.pws + lists * tda::kPairCap);
  const tda::KernelKey key{a->dtype, (int)a->head_dim, a->branches, pkind_of(a->relu_power), a->normalize ? 1 : 0};
  tda::timing_begin(stream);
  int e = tda::launch_bwd(p, key, stream);
  const int te = tda::timing_end();
  if (e == 0) e = te;
  if (e != 0) {
    g_last_hip_error = e;
    return TDA_ERR_HIP;
  }
  return TDA_OK;
}

}  // extern "C"
