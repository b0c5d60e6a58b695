// abi_driver.cpp -- runs the C ABI's host code (tda_host.cpp) under AddressSanitizer and
// UndefinedBehaviorSanitizer: argument validation (every rejection path), buffer sizes, the
// error strings, and the parameter blocks tda_fwd / tda_bwd hand to the (stub) launchers.
// Exit status 0 when every check holds; a sanitizer report aborts the run.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <initializer_list>

#include "../../include/tda.h"
#include "stub_launch.hpp"

static int failures = 0;
#define CHECK(cond)                                                   \
  do {                                                                \
    if (!(cond)) {                                                    \
      std::fprintf(stderr, "%s:%d: check failed: %s\n", __FILE__, __LINE__, #cond); \
      ++failures;                                                     \
    }                                                                 \
  } while (0)

// Addresses are never dereferenced by the host code: any 256-aligned value stands in.
static void* const FAKE = reinterpret_cast<void*>(uintptr_t(1) << 20);
static float kScalar = 1.f;

static tda_tensor tensor(int64_t b, int64_t h, int64_t n, int64_t d) {
  tda_tensor t;
  std::memset(&t, 0, sizeof(t));
  t.data = FAKE;
  t.stride[0] = h * n * d;
  t.stride[1] = n * d;
  t.stride[2] = d;
  t.stride[3] = 1;
  (void)b;
  return t;
}

static tda_fwd_args fwd_args(int64_t B = 2, int64_t H = 3, int64_t N = 100, int64_t D = 128, int32_t br = 2) {
  tda_fwd_args a;
  std::memset(&a, 0, sizeof(a));
  a.abi_version = TDA_ABI_VERSION;
  a.dtype = TDA_DTYPE_BF16;
  a.branches = br;
  a.normalize = 1;
  a.causal = 1;
  a.relu_power = 2.f;
  a.batch = B, a.heads = H, a.seq_len = N, a.head_dim = D;
  a.q1 = a.k1 = a.q2 = a.k2 = a.v = a.out = tensor(B, H, N, D);
  a.beta = &kScalar;
  a.lambda_param = &kScalar;
  a.norms = static_cast<float*>(FAKE);
  a.workspace = FAKE;
  a.workspace_bytes = tda_fwd_workspace_bytes(B, H, N, br);
  return a;
}

static tda_bwd_args bwd_args(int64_t B = 2, int64_t H = 3, int64_t N = 100, int64_t D = 128, int32_t br = 2) {
  tda_bwd_args a;
  std::memset(&a, 0, sizeof(a));
  a.abi_version = TDA_ABI_VERSION;
  a.dtype = TDA_DTYPE_BF16;
  a.branches = br;
  a.normalize = 1;
  a.causal = 1;
  a.relu_power = 2.f;
  a.batch = B, a.heads = H, a.seq_len = N, a.head_dim = D;
  a.q1 = a.k1 = a.q2 = a.k2 = a.v = a.dout = tensor(B, H, N, D);
  a.dq1 = a.dk1 = a.dq2 = a.dk2 = a.dv = tensor(B, H, N, D);
  a.beta = &kScalar;
  a.lambda_param = &kScalar;
  a.norms = static_cast<const float*>(FAKE);
  a.workspace = FAKE;
  a.workspace_bytes = tda_bwd_workspace_bytes(B, H, N, D);
  return a;
}

template <class F>
static void fwd_rejects(F mutate, int32_t code) {
  tda_fwd_args a = fwd_args();
  mutate(a);
  const int calls = stub::fwd_calls;
  CHECK(tda_validate_fwd(&a) == code);
  CHECK(tda_fwd(&a, nullptr) == code);
  CHECK(stub::fwd_calls == calls);  // rejected before any launch
}
template <class F>
static void bwd_rejects(F mutate, int32_t code) {
  tda_bwd_args a = bwd_args();
  mutate(a);
  const int calls = stub::bwd_calls;
  CHECK(tda_validate_bwd(&a) == code);
  CHECK(tda_bwd(&a, nullptr) == code);
  CHECK(stub::bwd_calls == calls);
}

int main() {
  CHECK(tda_abi_version() == TDA_ABI_VERSION);
  CHECK(tda_validate_fwd(nullptr) == TDA_ERR_NULL_POINTER);
  CHECK(tda_validate_bwd(nullptr) == TDA_ERR_NULL_POINTER);

  // ---- valid calls reach the launchers with the parameter blocks they describe
  {
    tda_fwd_args a = fwd_args(4, 16, 4096, 128, 2);
    a.zero = FAKE;
    a.zero_bytes = (uint64_t)5 * 4 * 16 * 4096 * 128 * 2;
    CHECK(tda_fwd(&a, nullptr) == TDA_OK);
    const tda::FwdParams& p = stub::last_fwd;
    CHECK(p.B == 4 && p.H == 16 && p.Nq == 4096 && p.Nk == 4096 && p.qoff == 0);
    CHECK(p.nqt == 128 && p.nkt == 128 && p.occ_w == 4);
    CHECK(p.norms != nullptr && p.cand != nullptr && p.part == nullptr);
    CHECK(p.k8 != nullptr && p.ksc != nullptr);  // the int8 screen's keys, after the candidate lists
    CHECK((char*)p.k8 - (char*)p.cand >= (int64_t)2 * 64 * 128 * 33 * 4);
    CHECK((char*)p.ksc - (char*)p.k8 == (int64_t)2 * 64 * 4096 * 128);
    CHECK(tda_fwd_workspace_bytes_for(&a) <= a.workspace_bytes);
    CHECK(stub::last_key.d == 128 && stub::last_key.branches == 2 && stub::last_key.pkind == 2);
    // the screen's steps: per (branch, head) sum over the 16 blocks of 8 (qb + 1) key tiles
    const int64_t steps = (int64_t)2 * 64 * 8 * (16 * 17 / 2);
    CHECK(p.zero_units == (int64_t)a.zero_bytes / 16);
    CHECK((int64_t)p.zero_per_it == (p.zero_units + steps - 1) / steps);
    CHECK((int64_t)p.zero_per_it * steps >= p.zero_units);
    CHECK((int64_t)p.zero_per_it * 16 * p.screen_kc < (int64_t(1) << 31));
  }
  {
    // a zero range far larger than the problem (two key-tile steps): the screen's 32-bit slice
    // offsets would wrap, so the host leaves the whole range to zero_range (zero_per_it 0)
    tda_fwd_args a = fwd_args(1, 1, 64, 128, 1);
    a.workspace_bytes = tda_fwd_workspace_bytes(1, 1, 64, 1);
    a.zero = FAKE;
    a.zero_bytes = (uint64_t)1 << 33;
    CHECK(tda_fwd(&a, nullptr) == TDA_OK);
    CHECK(stub::last_fwd.zero == FAKE && stub::last_fwd.zero_units == (int64_t)1 << 29);
    CHECK(stub::last_fwd.zero_per_it == 0);
    a.zero_bytes = (uint64_t)1 << 20;  // a small range keeps the per-item slices
    CHECK(tda_fwd(&a, nullptr) == TDA_OK);
    CHECK(stub::last_fwd.zero_per_it > 0 && (int64_t)stub::last_fwd.zero_per_it * 16 * stub::last_fwd.screen_kc < (int64_t(1) << 31));
  }
  {
    tda_fwd_args a = fwd_args(1, 2, 5, 64, 1);  // one query tile: the decode partials
    a.seq_len_kv = 900;
    a.q_offset = 895;
    a.workspace_bytes = tda_fwd_workspace_bytes_kv(1, 2, 5, 900, 1);
    a.relu_power = 1.5f;
    CHECK(tda_fwd(&a, nullptr) == TDA_OK);
    CHECK(stub::last_fwd.part != nullptr && stub::last_fwd.cand == nullptr);
    CHECK(stub::last_fwd.Nk == 900 && stub::last_fwd.nkt == 29 && stub::last_key.pkind == 0);
    CHECK(stub::last_fwd.zero == nullptr && stub::last_fwd.k8 == nullptr);
    a.normalize = 0;  // one query tile and no normalisation: no int8 keys either way
    CHECK(tda_fwd_workspace_bytes_for(&a) == tda_fwd_workspace_bytes_kv(1, 2, 5, 900, 1));
  }
  {
    tda_fwd_args a = fwd_args(1, 2, 100, 64, 2);
    a.dtype = TDA_DTYPE_F32;
    a.workspace_bytes = tda_fwd_workspace_bytes_for(&a);
    CHECK(tda_fwd(&a, nullptr) == TDA_OK);
    // normalised fp32 with more than one query tile: the int8 screen runs on the fp32 rows
    CHECK(stub::last_fwd.k8 != nullptr && stub::last_fwd.ksc != nullptr);
    CHECK(stub::last_fwd.screen_items >= 1 && stub::last_fwd.screen_kc % 32 == 0);
    a.normalize = 0;
    a.workspace_bytes = tda_fwd_workspace_bytes_for(&a);
    CHECK(tda_fwd(&a, nullptr) == TDA_OK);
    CHECK(stub::last_fwd.k8 == nullptr);
  }
  {
    tda_bwd_args a = bwd_args();
    a.grads_zeroed = 1;
    a.occupancy = static_cast<const uint32_t*>(FAKE);
    a.pairs = static_cast<uint32_t*>(FAKE);
    CHECK(tda_bwd(&a, nullptr) == TDA_OK);
    CHECK(stub::last_bwd.grads_zeroed == 1 && stub::last_bwd.pairs != nullptr && stub::last_bwd.dkvq != nullptr);
    // column buckets after the 2 * 6 * 4 lists (129 words each), counts of 6 * 4 columns
    CHECK(stub::last_bwd.colcnt == static_cast<const uint32_t*>(FAKE) + 48 * 129 &&
          stub::last_bwd.colbuf == static_cast<uint32_t*>(FAKE) + 48 * 129 + 24);
    a.occupancy = nullptr;  // without the bitmask the pair lists are not used
    CHECK(tda_bwd(&a, nullptr) == TDA_OK);
    CHECK(stub::last_bwd.pairs == nullptr && stub::last_bwd.colcnt == nullptr);
  }
  {  // a failed launch maps to TDA_ERR_HIP and is kept for tda_last_hip_error
    tda_fwd_args a = fwd_args();
    stub::fail_with = 98;
    CHECK(tda_fwd(&a, nullptr) == TDA_ERR_HIP);
    CHECK(tda_last_hip_error() == 98);
  }

  // ---- every rejection path of the forward validator
  fwd_rejects([](tda_fwd_args& a) { a.abi_version = 99; }, TDA_ERR_ABI);
  fwd_rejects([](tda_fwd_args& a) { a.dtype = 7; }, TDA_ERR_DTYPE);
  fwd_rejects([](tda_fwd_args& a) { a.branches = 3; }, TDA_ERR_BRANCHES);
  fwd_rejects([](tda_fwd_args& a) { a.causal = 0; }, TDA_ERR_CAUSAL);
  fwd_rejects([](tda_fwd_args& a) { a.head_dim = 96; }, TDA_ERR_HEAD_DIM);
  fwd_rejects([](tda_fwd_args& a) { a.seq_len = 0; }, TDA_ERR_SHAPE);
  fwd_rejects([](tda_fwd_args& a) { a.batch = 0; }, TDA_ERR_SHAPE);
  fwd_rejects([](tda_fwd_args& a) { a.heads = (int64_t)1 << 40; }, TDA_ERR_SHAPE);
  fwd_rejects([](tda_fwd_args& a) { a.relu_power = -1.f; }, TDA_ERR_POWER);
  fwd_rejects([](tda_fwd_args& a) { a.relu_power = __builtin_nanf(""); }, TDA_ERR_POWER);
  fwd_rejects([](tda_fwd_args& a) { a.relu_power = __builtin_inff(); }, TDA_ERR_POWER);
  fwd_rejects([](tda_fwd_args& a) { a.beta = nullptr; }, TDA_ERR_NULL_POINTER);
  fwd_rejects([](tda_fwd_args& a) { a.lambda_param = nullptr; }, TDA_ERR_NULL_POINTER);
  fwd_rejects([](tda_fwd_args& a) { a.q2.data = nullptr; }, TDA_ERR_NULL_POINTER);
  fwd_rejects([](tda_fwd_args& a) { a.v.stride[3] = 2; }, TDA_ERR_LAYOUT);
  fwd_rejects([](tda_fwd_args& a) { a.k1.stride[2] = 129; }, TDA_ERR_LAYOUT);
  fwd_rejects([](tda_fwd_args& a) { a.q1.stride[0] = -128; }, TDA_ERR_LAYOUT);
  fwd_rejects([](tda_fwd_args& a) { a.k1.stride[2] = ((int64_t)1 << 25) + 8; }, TDA_ERR_LAYOUT);
  fwd_rejects([](tda_fwd_args& a) { a.q1.data = static_cast<char*>(FAKE) + 2; }, TDA_ERR_LAYOUT);
  fwd_rejects([](tda_fwd_args& a) { a.norms = nullptr; }, TDA_ERR_NORMS);
  fwd_rejects([](tda_fwd_args& a) { a.workspace = nullptr; }, TDA_ERR_WORKSPACE);
  fwd_rejects([](tda_fwd_args& a) { a.workspace_bytes -= 4; }, TDA_ERR_WORKSPACE);
  fwd_rejects([](tda_fwd_args& a) { a.workspace = static_cast<char*>(FAKE) + 8; }, TDA_ERR_WORKSPACE);
  fwd_rejects([](tda_fwd_args& a) { a.q_offset = -1; }, TDA_ERR_OFFSET);
  fwd_rejects([](tda_fwd_args& a) { a.q_offset = ((int64_t)1 << 30) - 64; }, TDA_ERR_OFFSET);
  fwd_rejects([](tda_fwd_args& a) { a.seq_len_kv = (int64_t)1 << 30; }, TDA_ERR_OFFSET);
  fwd_rejects([](tda_fwd_args& a) { a.seq_len_kv = -5; }, TDA_ERR_OFFSET);
  fwd_rejects([](tda_fwd_args& a) { a.seq_len_kv = 5000; }, TDA_ERR_WORKSPACE);
  fwd_rejects([](tda_fwd_args& a) { a.pairs = reinterpret_cast<uint32_t*>(static_cast<char*>(FAKE) + 4); },
              TDA_ERR_LAYOUT);
  fwd_rejects([](tda_fwd_args& a) { a.zero = FAKE; a.zero_bytes = 40; }, TDA_ERR_LAYOUT);
  fwd_rejects([](tda_fwd_args& a) { a.zero = static_cast<char*>(FAKE) + 8; a.zero_bytes = 64; }, TDA_ERR_LAYOUT);
  fwd_rejects([](tda_fwd_args& a) { a.zero = nullptr; a.zero_bytes = 64; }, TDA_ERR_NULL_POINTER);

  // ---- the backward validator
  bwd_rejects([](tda_bwd_args& a) { a.norms = nullptr; }, TDA_ERR_NORMS);
  bwd_rejects([](tda_bwd_args& a) { a.workspace = nullptr; }, TDA_ERR_WORKSPACE);
  bwd_rejects([](tda_bwd_args& a) { a.workspace_bytes = 8; }, TDA_ERR_WORKSPACE);
  bwd_rejects([](tda_bwd_args& a) { a.dk2.data = nullptr; }, TDA_ERR_NULL_POINTER);
  bwd_rejects([](tda_bwd_args& a) { a.dout.data = nullptr; }, TDA_ERR_NULL_POINTER);
  bwd_rejects([](tda_bwd_args& a) { a.head_dim = 32; }, TDA_ERR_HEAD_DIM);
  bwd_rejects([](tda_bwd_args& a) { a.q_offset = -3; }, TDA_ERR_OFFSET);
  {
    tda_bwd_args a = bwd_args();
    for (int k = 0; k < 3; ++k) a.dout.stride[k] = 0;  // a broadcast upstream gradient
    CHECK(tda_validate_bwd(&a) == TDA_OK);
    a.normalize = 0;
    a.norms = nullptr;
    CHECK(tda_validate_bwd(&a) == TDA_OK);
  }

  // ---- buffer sizes (0 for invalid arguments) and error strings
  CHECK(tda_occupancy_words(4, 16, 4096, 2) == (size_t)2 * 64 * 128 * 4);
  CHECK(tda_occupancy_words_kv(1, 1, 1, 5000, 1) == (size_t)((5000 + 31) / 32 + 31) / 32);
  CHECK(tda_occupancy_words(0, 1, 1, 1) == 0 && tda_occupancy_words(1, 1, 33, 3) == 0);
  CHECK(tda_norms_floats_kv(2, 3, 10, 20, 2) == (size_t)2 * 6 * 30);
  CHECK(tda_fwd_workspace_bytes_kv(1, 1, 1, 5000, 1) == (size_t)256 + 5 * 1 * 128 * 4);
  CHECK(tda_fwd_workspace_bytes(1, 1, 33, 3) == 0);
  // the lists (entries and counts), the column counts, kColCap = 64 entries of 4 words per column
  CHECK(tda_pair_words(4, 16, 4096, 2) == (size_t)2 * 64 * 128 * (1 + 4 * 32) + 64 * 128 + (size_t)64 * 128 * 64 * 4);
  CHECK(tda_pair_words(1, 1, 33, 1) == (size_t)(2 * (1 + 4 * 32) + 2) + 4 + (size_t)2 * 64 * 4);
  CHECK(tda_bwd_workspace_bytes(0, 1, 1, 128) == 0);
  for (int32_t code : {0, -1, -2, -3, -4, -5, -6, -7, -8, -9, -10, -11, -12, -13, -100}) {
    const char* s = tda_error_string(code);
    CHECK(s && std::strcmp(s, "unknown error") != 0);
  }
  CHECK(std::strcmp(tda_error_string(-55), "unknown error") == 0);

  if (failures) std::fprintf(stderr, "%d check(s) failed\n", failures);
  else std::printf("abi_driver: all checks passed\n");
  return failures ? 1 : 0;
}
