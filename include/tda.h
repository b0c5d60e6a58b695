/*
 * tda.h -- C ABI of the MI355X (gfx950) threshold-attention library libtda_hip.so.
 *
 * The library computes Threshold Rectified Attention (TRA, one branch) and
 * Threshold Differential Attention (TDA, two branches), causal, on queries of
 * shape (B, H, Nq, d) and keys/values of shape (B, H, Nk, d):
 *
 *   P_i    = q_offset + i                               absolute position of query row i
 *   tau_i  = beta * sqrt(2 ln(P_i+1) / d)
 *   A_ij   = ReLU(s(q_i, k_j) - tau_i)^p  for j <= P_i  s = dot, or cosine when normalize
 *   out    = A(q1,k1) V                                 branches == 1
 *   out    = (A(q1,k1) - clamp(lambda,0,1) A(q2,k2)) V  branches == 2
 *
 * Reference interface replaced (reference = snap-research/TDA,
 * triton_threshold_attention.py, cited as TTA:<line>):
 *   tda_fwd  <- ThresholdRelaFunction.forward host code and the
 *               _threshold_rela_fwd_kernel launch (TTA:336-403, TTA:374-389);
 *               branches == 2 also replaces the two-call composition, the
 *               F.normalize calls and the lambda combine of
 *               differential_threshold_rela_triton (TTA:505-517).
 *   tda_bwd  <- ThresholdRelaFunction.backward and the
 *               _threshold_rela_bwd_kernel_dq / _dkv launches (TTA:406-469,
 *               TTA:433-460), plus the torch-autograd backward of the
 *               normalize/clamp/combine ops (TTA:505-517) and dbeta, which the
 *               reference does not compute (it returns None, TTA:469).
 *   tda_validate_fwd / tda_validate_bwd <- the shape assert (TTA:348), extended
 *               to every argument; host-only, never touches a GPU.
 *   seq_len_kv / q_offset: no counterpart (the reference's query index is always the
 *               absolute position, TTA:62, with Nq = Nk); they serve KV-cache decode and
 *               chunked prefill.  Zero for both is the reference's case.
 *
 * Conventions
 *   - Every pointer in the argument structs is a device pointer, except the
 *     struct itself.  The caller allocates everything (outputs and the
 *     workspace of each pass); the library never allocates or frees device
 *     memory and keeps no per-call state.  The one exception is tda_fwd_noalloc,
 *     whose workspace is a fixed device array of the library (see there).
 *   - Strides are in elements, for the (B, H, N, d) axes.  stride[3] must be 1;
 *     the other strides and every base pointer must keep 16-byte alignment;
 *     the sequence stride is at most 2^25 elements.
 *     stride[0] is honoured (the reference ignores it, TTA:49).
 *   - beta and lambda are read on the device (no host synchronisation);
 *     lambda is clamped to [0, 1] on the device.
 *   - All work is enqueued on `stream` (a hipStream_t; NULL = default stream);
 *     there is no device-wide synchronisation.  Calls are thread-safe.
 *   - Return value: 0 on success, a negative TDA_ERR_* code otherwise;
 *     tda_error_string() gives a static description.
 */
#ifndef TDA_H_
#define TDA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TDA_ABI_VERSION 7

/* element types of q, k, v, out and gradients */
#define TDA_DTYPE_F32  0
#define TDA_DTYPE_BF16 1

/* error codes */
#define TDA_OK                 0
#define TDA_ERR_NULL_POINTER  -1   /* a required pointer is NULL */
#define TDA_ERR_SHAPE         -2   /* batch/heads/seq_len out of range */
#define TDA_ERR_HEAD_DIM      -3   /* head_dim not in {64, 128, 256} */
#define TDA_ERR_DTYPE         -4   /* dtype not TDA_DTYPE_F32 / TDA_DTYPE_BF16 */
#define TDA_ERR_LAYOUT        -5   /* stride[3] != 1, 16-byte alignment broken, or a
                                      sequence stride above 2^25 elements */
#define TDA_ERR_POWER         -6   /* relu_power negative or not finite */
#define TDA_ERR_BRANCHES      -7   /* branches not 1 or 2 */
#define TDA_ERR_WORKSPACE     -8   /* workspace missing, too small or misaligned */
#define TDA_ERR_ABI           -9   /* abi_version != TDA_ABI_VERSION */
#define TDA_ERR_CAUSAL       -10   /* causal != 1 (only the causal form exists) */
#define TDA_ERR_NORMS        -11   /* normalize set but the norms buffer is missing */
#define TDA_ERR_OFFSET       -12   /* q_offset negative, or seq_len_kv / q_offset + seq_len
                                      beyond 2^30 - 64 */
#define TDA_ERR_SCRATCH      -13   /* tda_fwd_noalloc: the call needs more workspace than
                                      TDA_NOALLOC_SCRATCH_BYTES */
#define TDA_ERR_HIP         -100   /* a HIP launch failed; see tda_last_hip_error() */

/* Size of the device array that tda_fwd_noalloc uses as its workspace (per GPU). */
#define TDA_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)

/* One (B, H, N, d) tensor: data pointer plus strides in elements. */
typedef struct tda_tensor {
  void*   data;
  int64_t stride[4];
} tda_tensor;

typedef struct tda_fwd_args {
  int32_t abi_version;      /* TDA_ABI_VERSION */
  int32_t dtype;            /* TDA_DTYPE_* of every tensor */
  int32_t branches;         /* 1 = TRA (q1, k1, v), 2 = TDA (q1, k1, q2, k2, v) */
  int32_t normalize;        /* 1 = cosine scores (F.normalize of q and k rows) */
  int32_t causal;           /* must be 1 */
  float   relu_power;       /* p >= 0; p == 1 and p == 2 take integer fast paths */
  int64_t batch, heads, seq_len, head_dim;  /* seq_len = Nq, the query rows */
  tda_tensor q1, k1, q2, k2, v;   /* inputs (q2, k2 ignored when branches == 1): q rows Nq,
                                     k and v rows Nk */
  tda_tensor out;                 /* output (Nq rows), same dtype as the inputs */
  const float* beta;        /* device scalar */
  const float* lambda_param;/* device scalar, raw (clamped on device); branches == 2 */
  float*    norms;          /* tda_norms_floats_kv() floats: inverse row norms
                               1/max(|x|,1e-12) of q1 [B*H][Nq], k1 [B*H][Nk] (, q2
                               [B*H][Nq], k2 [B*H][Nk]), back to back; required and written
                               when normalize == 1 (the backward reads them), else unused */
  /* optional outputs (may be NULL): */
  uint32_t* occupancy;      /* tile-occupancy bitmask, tda_occupancy_words_kv() words laid
                               out [branch][B*H][query tile][ceil(key tiles/32)]: bit kt of
                               row (branch, bh, qt) is set when some A_ij of that branch is
                               non-zero in the 32x32 tile (query tile qt, key tile kt) */
  unsigned long long* stats;/* 3 counters: [0] += (query tile, key tile, branch) triples
                               on or below the diagonal, [1] += those with a non-zero
                               weight tile (A.V issued), [2] += those whose exact weights
                               were evaluated (bf16: the tiles the screen kept, or every
                               causal tile without normalisation; a superset of [1]; f32
                               leaves [2] alone); tiles are 32x32 */
  void*  workspace;         /* device scratch of tda_fwd_workspace_bytes_for(args) bytes (or
                               the larger tda_fwd_workspace_bytes_kv()), 16-byte aligned: holds
                               the tile bitmask when occupancy is NULL and, when seq_len <= 32,
                               the fp32 per-chunk partial outputs of the single-query-tile
                               (decode) kernels, else the screen's candidate keys per (branch,
                               head, query tile) and, for normalised calls of either dtype at
                               head_dim 64 or 128 with more than 32 query rows, the key rows
                               quantised to int8 for the screen (head_dim + 8 bytes per key row
                               and branch) */
  size_t workspace_bytes;
  int64_t seq_len_kv;       /* Nk, the key/value rows; 0 means Nk = seq_len */
  int64_t q_offset;         /* position of query row 0 (>= 0); 0 with Nk = Nq is the
                               reference's causal case, Nk - Nq the KV-cache alignment */
  uint32_t* pairs;          /* optional output (may be NULL), tda_pair_words() words, 16-byte
                               aligned: for each (branch, head, query tile) the list of its
                               non-zero weights (key index, row, exact threshold margin), which
                               lets the backward read only the rows they name, and (normalised,
                               more than 32 query rows, Nk <= Nq rounded up to 32) the same pairs
                               bucketed by key tile.  Written by the bf16 forward and by the f32
                               forward when normalised with more than 32 query rows; the other
                               f32 forwards mark every list "not written" (the backward then walks
                               the tiles); head_dim 256 leaves it alone and its backward ignores
                               it */
  void*    zero;            /* optional (may be NULL with zero_bytes == 0): a device range the
                               call sets to zero, 16-byte aligned, zero_bytes a multiple of 16.
                               For training: the buffer of the backward's gradients, zeroed while
                               the forward's matrix-core pass runs (its HBM is mostly idle), so
                               the backward (grads_zeroed = 1) writes only the non-zero rows.  It
                               must not overlap any other buffer of the call.  No counterpart in
                               the reference. */
  uint64_t zero_bytes;
} tda_fwd_args;

typedef struct tda_bwd_args {
  int32_t abi_version;
  int32_t dtype;
  int32_t branches;
  int32_t normalize;
  int32_t causal;
  float   relu_power;
  int64_t batch, heads, seq_len, head_dim;
  tda_tensor q1, k1, q2, k2, v;   /* forward inputs */
  tda_tensor dout;                /* upstream gradient of out */
  tda_tensor dq1, dk1, dq2, dk2, dv;  /* outputs (dq2, dk2 ignored when branches == 1) */
  const float* beta;
  const float* lambda_param;
  float* dbeta;             /* device scalar out, may be NULL */
  float* dlambda;           /* device scalar out (branches == 2), may be NULL */
  const float*    norms;    /* the forward's norms output; required when normalize == 1 */
  const uint32_t* occupancy;/* the forward's bitmask, or NULL to test every causal tile */
  void*  workspace;         /* device scratch of tda_bwd_workspace_bytes() bytes, 16-byte
                               aligned: dbeta / dlambda partials and the dk weight of each
                               pair-list entry */
  size_t workspace_bytes;
  unsigned long long* stats;/* optional: [0] += tiles visited, [1] += tiles computed */
  int64_t seq_len_kv;       /* as in tda_fwd_args (dq, dout: Nq rows; dk, dv: Nk rows) */
  int64_t q_offset;
  uint32_t* pairs;          /* the forward's pair buffer, or NULL; used only with occupancy
                               (bf16): lists that did not fit fall back to the bitmask tiles.
                               The call writes each bucketed pair's dk weight into it, so two
                               backward calls on one pair buffer must not overlap. */
  int32_t grads_zeroed;     /* 1: dq1, dk1, (dq2, dk2,) dv hold zeros already (e.g. the forward's
                               zero range); the call then stores only the gradient rows that a
                               non-zero weight reaches.  0: every row is stored.  No counterpart
                               in the reference. */
} tda_bwd_args;

int32_t     tda_abi_version(void);
const char* tda_error_string(int32_t code);
/* hipError_t of the last failed launch on this thread (0 if none) */
int32_t     tda_last_hip_error(void);

/* Host-only argument checks (no GPU access). */
int32_t tda_validate_fwd(const tda_fwd_args* args);
int32_t tda_validate_bwd(const tda_bwd_args* args);

/* Buffer sizes for the optional forward outputs and the backward workspace (0 for invalid
   arguments).  The _kv forms take the key rows Nk; the others are the Nk = Nq case.  The forward
   workspace functions without a tda_fwd_args return the largest any call of that shape needs
   (bf16 with normalize, head_dim 128); tda_fwd_workspace_bytes_for gives the exact need of one
   call (from its shape fields, dtype, normalize and head_dim; the pointers are not read). */
size_t tda_occupancy_words(int64_t batch, int64_t heads, int64_t seq_len, int32_t branches);
size_t tda_norms_floats(int64_t batch, int64_t heads, int64_t seq_len, int32_t branches);
size_t tda_fwd_workspace_bytes(int64_t batch, int64_t heads, int64_t seq_len, int32_t branches);
size_t tda_occupancy_words_kv(int64_t batch, int64_t heads, int64_t seq_len, int64_t seq_len_kv,
                              int32_t branches);
size_t tda_norms_floats_kv(int64_t batch, int64_t heads, int64_t seq_len, int64_t seq_len_kv,
                           int32_t branches);
size_t tda_fwd_workspace_bytes_kv(int64_t batch, int64_t heads, int64_t seq_len, int64_t seq_len_kv,
                                  int32_t branches);
size_t tda_fwd_workspace_bytes_for(const tda_fwd_args* args);
size_t tda_bwd_workspace_bytes(int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim);
/* Words of the pair buffer: the lists and the column buckets (queries seq_len; no dependence
   on the key rows: the buckets are used only when the key tiles are no more than the query
   tiles). */
size_t tda_pair_words(int64_t batch, int64_t heads, int64_t seq_len, int32_t branches);

/* Enqueue the forward / backward pass on `stream` (a hipStream_t). */
int32_t tda_fwd(const tda_fwd_args* args, void* stream);
int32_t tda_bwd(const tda_bwd_args* args, void* stream);

/* tda_fwd without a caller workspace, and without any allocation: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  Same arguments, results and errors
 * as tda_fwd, except that args->workspace and args->workspace_bytes are ignored: the workspace
 * is a device array of the library, TDA_NOALLOC_SCRATCH_BYTES (16 MiB) per GPU, held from the
 * first call on that GPU until the process ends.  A call whose workspace
 * (tda_fwd_workspace_bytes_for) exceeds it returns TDA_ERR_SCRATCH before touching the GPU.
 * A normalised forward (bf16 or fp32, head_dim 64 or 128, more than 32 query rows) holds int8
 * copies of the key rows in its workspace (head_dim + 8 bytes per key row and branch): TRA at
 * B*H = 64, seq_len 2048, head_dim 64 needs 9.6 MiB and fits (in either dtype); fp32 TRA at
 * B*H = 16, seq_len 4096, head_dim 128 needs 8.8 MiB and fits; differential TDA at B*H = 64,
 * seq_len 4096, head_dim 128 needs 70.3 MiB and does not; without normalize the same call needs
 * 2.3 MiB, and one query against B*H = 64 heads of 16384 keys 0.5 MiB.  Every call on one GPU shares that GPU's array, which keeps the last call's
 * contents: calls that overlap on one GPU (other streams, unordered host threads) race and
 * must be serialised by the caller.  The outputs (out, norms, occupancy, pairs, stats) are
 * the caller's as for tda_fwd. */
int32_t tda_fwd_noalloc(const tda_fwd_args* args, void* stream);

/* Per-launch timing of one call: no counterpart in the reference (whose Triton launches are
 * timed from outside); for benchmarks that need each kernel's duration without a tracer.
 * Arms the calling thread: its next tda_fwd, tda_fwd_noalloc or tda_bwd call that passes
 * validation records events[0] (hipEvent_t, created by the caller) on its stream before its
 * first kernel launch and events[k] right after its k-th launch, k = 1 .. n - 1 (later launches
 * are not bracketed), then disarms.  n = 0 (or events == NULL) disarms.  Returns TDA_OK, or
 * TDA_ERR_NULL_POINTER for events == NULL with n > 0.  A failed event record fails the call
 * with TDA_ERR_HIP. */
int32_t tda_time_next_call(void* const* events, int32_t n);
/* Kernel launches of the last timed call on this thread, and the name of launch k (0-based;
 * NULL past the end).  Names are the kernel families: "key_prep", "fwd_screen", ... */
int32_t     tda_timed_launches(void);
const char* tda_timed_launch_name(int32_t k);

#ifdef __cplusplus
}
#endif

#endif /* TDA_H_ */
