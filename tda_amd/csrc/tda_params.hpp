// tda_params.hpp -- kernel argument blocks passed by value from the host launcher to the
// gfx950 kernels, plus the launcher entry points each kernel file exports.
#pragma once

#include <stdint.h>

namespace tda {

// Tensor slots in the stride table.
enum FwdSlot { F_Q1 = 0, F_K1, F_Q2, F_K2, F_V, F_OUT, F_NSLOT };
enum BwdSlot { B_Q1 = 0, B_K1, B_Q2, B_K2, B_V, B_DO, B_DQ1, B_DK1, B_DQ2, B_DK2, B_DV, B_NSLOT };

// Row-norm table: slots q1, k1, q2, k2 back to back, each [B*H][rows] with rows = Nq for the
// query slots and Nk for the key slots (norm_base).
enum NormSlot { N_Q1 = 0, N_K1 = 1, N_Q2 = 2, N_K2 = 3 };

// Pair lists (bf16): for each (branch, head, query tile) the non-zero weights of the tile's
// rows, written by the forward's exact pass and read by the backward, which then touches only
// the rows they name.  Layout: the entries, kPairCap per list (list = (branch * B*H + bh) * nqt
// + qt), each 4 u32 {key index j, query row within the tile, bits of x_ij = fma(s rk, rq, -tau),
// 0}, in the order the exact pass met them (key tiles ascending); then the counts, u32 per list.
// A count above kPairCap marks a list that did not fit: the backward then runs its tile path
// for that query tile.
constexpr int kPairCap = 32;
constexpr int64_t pair_lists(int64_t branches, int64_t bh, int64_t nqt) { return branches * bh * nqt; }
constexpr uint32_t kPairOverflow = 0xffffffffu;  // count of a list the forward did not write

// Column buckets (after the lists, same buffer): for each (head, key tile) the pairs of every
// branch whose key lies in the tile, so that the backward's key-major pass reads its pairs in one
// round instead of walking every query tile's list.  Layout (u32 words from the buffer start,
// each part 16-byte aligned): the counts, one per column (col = bh * nkt + kt), zeroed by
// key_prep and raised by the exact pass's atomic adds, kColTaint set when the bucket does not
// hold every pair of the column with its dk weight (a pair list past kPairCap, pairs from the
// tile pass); then kColCap entries per column, each 4 u32 {query row i | branch << 31, key row
// within the tile, bits of x_ij, bits of the dk weight (written by the backward's query-major
// pass)}, in no fixed order (appended by atomics: the reader sorts them).  The pair entry's
// fourth word holds its bucket slot.  Sized for nkt <= nqt; used only then (bf16, normalised,
// more than one query tile).
constexpr int kColCap = 64;
constexpr uint32_t kColTaint = 0x80000000u;
constexpr uint32_t kNoSlot = 0xffffffffu;
constexpr int64_t round4(int64_t w) { return (w + 3) / 4 * 4; }
constexpr int64_t pair_list_words(int64_t branches, int64_t bh, int64_t nqt) {
  return round4(pair_lists(branches, bh, nqt) * (1 + 4 * kPairCap));
}
constexpr int64_t col_count_words(int64_t bh, int64_t nkt) { return round4(bh * nkt); }
constexpr int64_t pair_words(int64_t branches, int64_t bh, int64_t nqt) {
  return pair_list_words(branches, bh, nqt) + col_count_words(bh, nqt) + bh * nqt * kColCap * 4;
}

// Candidate keys (bf16 with normalisation, forward workspace): for each (branch, head, query
// tile) the keys j whose screen lane passed (max over its query rows of the screen score above
// the tile's threshold minus the screen's rounding margin), a superset of the keys with a non-zero
// weight in the query tile; the exact pass gathers only these rows.  Layout: the keys,
// kCandCap u32 per list, each distinct (increasing when the list has one producer; a query tile
// whose key range the screen splits over several work items gets its keys in any order, which the
// exact pass sorts); then the counts, u32 per list (zeroed by key_prep, raised by the screen's
// atomic adds).  A count above kCandCap marks a list that did not fit: the exact pass then walks
// the bitmask tiles of that query tile.
constexpr int kCandCap = 32;
// Slices of the fixed-order dbeta / dlambda sum (tda_fin.hpp, bwd_finish).
constexpr int kFinSlices = 1024;
constexpr int64_t cand_words(int64_t lists) { return lists * (1 + kCandCap); }

// Positions: query row i of a head sits at absolute position qoff + i and sees the keys
// j <= qoff + i of the Nk key rows (qoff = 0 and Nq = Nk is the plain causal case).  Tiles are
// 32 rows: nqt = ceil(Nq / 32) query tiles, nkt = ceil(Nk / 32) key tiles.

struct FwdParams {
  const void* in[5];         // q1, k1, q2, k2, v
  void* out;
  int64_t s[F_NSLOT][3];     // batch, head, sequence strides in elements
  int B, H, Nq, Nk, qoff;
  int nqt, nkt;              // query tiles, key tiles
  int occ_w;                 // bitmask words per query tile: ceil(nkt / 32)
  float p;                   // relu_power
  float inv_d;               // 1 / head_dim
  const float* beta;
  const float* lam;
  float* norms;              // may be null
  uint32_t* occ;             // may be null (bf16: never, the host points it at workspace)
  unsigned long long* stats; // may be null
  float* part;               // bf16 with one query tile: per-chunk partial outputs (workspace)
  uint32_t* pairs;           // may be null: pair lists (bf16)
  uint32_t* colcnt;          // may be null: column bucket counts and entries (in pairs)
  uint32_t* colbuf;
  int nbr;                   // branches
  uint32_t* cand;            // candidate keys (workspace; null for a single query tile)
  uint32_t* pvq;             // with cand: query tiles for the tile pass ([0] count, then bh nqt + qt),
                             // zeroed by the screen, filled by the candidate pass (workspace)
  void* zero;                // may be null: 16-byte units [0, zero_units) the call sets to zero
  int64_t zero_units;
  int zero_per_it;           // units each screen workgroup clears per key tile it walks
  int screen_kc;             // key tiles per screen work item (a multiple of 32): a 256-row block
                             // whose causal key range is longer is split into several items
  int screen_items;          // screen work items per (branch, head)
  int8_t* k8;                // int8 screen (bf16, normalised): key rows quantised by key_prep,
                             // [branch * B*H + bh][Nk][D] (workspace)
  float* ksc;                // their {scale s_j, residual bound ek_j}, [branch * B*H + bh][Nk][2]
};

struct BwdParams {
  const void* in[6];         // q1, k1, q2, k2, v, dout
  void* grad[5];             // dq1, dk1, dq2, dk2, dv
  int64_t s[B_NSLOT][3];
  int B, H, Nq, Nk, qoff;
  int nqt, nkt, occ_w;
  float p, inv_d;
  const float* beta;
  const float* lam;
  float* dbeta;
  float* dlam;
  const float* norms;
  const uint32_t* occ;       // may be null: every causal tile is tested
  float* ws;                 // [branches * BH * nqt][2] dbeta / dlambda partials of the dQ pass
  unsigned long long* stats;
  const uint32_t* pairs;     // may be null: the forward's pair lists (used with occ)
  float* pws;                // [pair lists][kPairCap] dk weight of each pair (workspace), written by
                             // the query-major pair pass, read by the key-major one
  const uint32_t* colcnt;    // may be null: the forward's column buckets (counts, entries; the
  uint32_t* colbuf;          // query-major pair pass writes each entry's dk weight)
  uint32_t* dkvq;            // may be null: key tiles for the key-major tile pass ([0] count, then
                             // items), zeroed by the query-major pair pass, filled by the key-major
                             // pair pass (workspace)
  int grads_zeroed;          // the gradient rows hold zeros: the pair passes store named rows only
};

// Kernel-family launchers (return a hipError_t value).  Template selection happens inside.
struct KernelKey {
  int dtype;      // 0 f32, 1 bf16
  int d;          // 64, 128 or 256
  int branches;   // 1 or 2
  int pkind;      // 2: p == 2, 1: p == 1, 0: general
  int normalize;  // 0 or 1
};

int launch_fwd(const FwdParams& p, const KernelKey& k, void* stream);
int launch_fwd_sparse(const FwdParams& p, const KernelKey& k, void* stream);
int launch_fwd_screen_f32(const FwdParams& p, const KernelKey& k, void* stream);
int launch_fwd_decode(const FwdParams& p, const KernelKey& k, float* part, void* stream);
int launch_bwd(const BwdParams& p, const KernelKey& k, void* stream);
int launch_bwd_fast(const BwdParams& p, const KernelKey& k, void* stream);
// fp32 with the forward's pair lists: the query-major and key-major pair passes (tda_bwd_fast.hip)
int launch_bwd_pairs_f32(const BwdParams& p, const KernelKey& k, void* stream);
// head_dim 256 (tda_wide.hip): the column-split forward and backward
int launch_fwd_wide(const FwdParams& p, const KernelKey& k, void* stream);
int launch_bwd_wide(const BwdParams& p, const KernelKey& k, void* stream);
// Set the forward's zero range to zero (paths without the screen, which clears it otherwise).
int launch_zero(const FwdParams& p, void* stream);
// Sum the (dbeta, dlambda) partial pairs ws[2 * item], item < items, in a fixed order.
int launch_bwd_finish(const BwdParams& p, int branches, int64_t items, void* stream);
// Record a hipError_t for tda_last_hip_error() (this thread).
void record_hip_error(int e);
// Per-launch timing of one call (tda_time_next_call; tda_timing.cpp): the C-ABI entry points
// bracket their launches with timing_begin / timing_end (which returns the first failed event
// record, 0 if none) and every launcher reports each kernel launch, in stream order.
void timing_begin(void* stream);
void launched(void* stream, const char* name);
int timing_end();

}  // namespace tda
