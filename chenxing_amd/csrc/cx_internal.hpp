// cx_internal.hpp -- layouts shared by the host entry points and the kernels.
#pragma once
#include <stdint.h>
#include <stddef.h>
#include "cx_sampler.h"

namespace cx {

constexpr int CAPW = 256;                 // per-wave candidate buffer (entries)
constexpr int KW_MAX = 128;               // entries a wave keeps when it compacts
constexpr int FIN_CAP = 4096;             // region finisher capacity (4 entries per thread)
constexpr int WIN_MAX = 4095;             // longest penalty window held in LDS
constexpr int CAPS = 16 * CAPW + 4096;    // candidates per (row, slice) in the workspace
constexpr int LEAN_CAP = 256;             // region size the one-wave finisher sorts
constexpr uint32_t HEMPTY = 0xFFFFFFFFu;  // empty hash slot
constexpr double TOL_S = 4e-6;            // relative error bound of the fp32-term normaliser
constexpr double TOL_T = 2e-6;            // relative error bound of one fp32 stream term
constexpr double TOL_MAX = 1e-4;          // rows whose bound exceeds this are recomputed exactly

// SplitStats.flags
constexpr int SF_OVERFLOW = 1;            // a wave buffer flooded with ties
constexpr int SF_UNSUPPORTED = 2;         // window longer than WIN_MAX
constexpr int SF_INEXACT = 4;             // the slice's normaliser has no usable error bound
constexpr int SF_EXACT = 8;               // sx holds the slice's fp64 normaliser (bound sxtol)


// Internal row_status values, never returned to the caller, for slow_kernel:
// the fused path could not decide the row and the exact multi-pass path must
// finish it (PENDING); the row's region is complete and only a top-p cut
// within the streamed normaliser's error bound is open, so the normaliser is
// recomputed in fp64 and the region finished again (REFINE); the row's
// region and statistics are written for the region finisher (FINISH; rows
// computed in several slices are always finished there and carry no mark).
constexpr int ROW_PENDING = 0x40000000;
constexpr int ROW_REFINE = 0x40000001;
constexpr int ROW_FINISH = 0x40000002;
// In a single-slice row's hand-off mark (SampleArgs::counters), beside its
// ROW_* value: the row may take the counted deep-nucleus path
// (deep_candidate, top-k allowed), and it has a top-k bound.
constexpr int MARK_DEEP = 0x00010000;
constexpr int MARK_TOPK = 0x00020000;

struct SplitStats {       // one per (row, slice), 64 bytes
  double m;               // max of the slice's penalised values (stochastic rows)
  double s;               // sum of exp((x - m) / T) over the slice
  double best_v;          // first maximum (greedy rows)
  double tol;             // relative error bound of s (stochastic rows)
  int32_t best_i;         // its index (INT_MAX if none)
  int32_t nan_i;          // first NaN index (INT_MAX if none)
  uint32_t tau;           // region threshold key; <= 1 means the region is the whole slice
  int32_t ncand;          // region entries written to the workspace
  int32_t flags;
  float sxtol;            // with SF_EXACT: relative error bound of sx (0: every term
                          // within 1 ulp; else the split sum's)
  double sx;              // with SF_EXACT: sum of exp((x - m) / T) over the slice in fp64
                          // (sliced top-p rows)
};
static_assert(sizeof(SplitStats) == 64, "SplitStats layout");

struct Cand {             // 16 bytes
  uint64_t key;           // orderable key of the fp64 (penalised) value
  int32_t idx;
  int32_t pad;
};

struct SampleArgs {
  const void* logits;
  int64_t ld;
  int32_t B, V;
  const int32_t* hist;
  const int32_t* hist_len;
  int64_t ldh;
  const cx_row_params* prm;
  const double* u;
  int32_t* out_id;
  int32_t* row_status;
  float* out_probs;
  // [B + 1], each written by the fused kernel before the later kernels read
  // it: [row] of a sliced row, 0; [row] of a single-slice row, its hand-off
  // mark (ROW_FINISH, ROW_REFINE,
  // ROW_PENDING, or 0 if decided, with MARK_DEEP and MARK_TOPK), which,
  // unlike row_status, the finishing kernels leave as it is; [B],
  // finish16_kernel's work-item counter (zeroed)
  int32_t* counters;
  SplitStats* stats;      // [B * nsplit]
  Cand* cands;            // [B * nsplit * CAPS]
  int32_t nsplit, split_len;
  int32_t ns, ns_log2;    // penalty hash slots (power of two, >= 2 x window) and log2
  int32_t vec_ok;         // rows are 16-byte aligned
  int32_t off_bitmap, off_hword, off_hval, off_dense, off_wkey, off_widx, off_gather;
  int32_t lds_bytes;      // fused kernel dynamic LDS
  int32_t bf16;           // logits are bf16 bit patterns
  int32_t f64;            // logits are fp64 (exact multi-pass path only)
  int32_t all_slow;       // every row takes the exact multi-pass path
  double logV;            // log(V)
  double* out64;          // [B, ldo] fp64 output of the penalty and truncation kernels
  int64_t ldo;
  int32_t slow_nbw;       // multi-pass kernel: full-row bitmap words (power of two)
  int32_t slow_off_hkey, slow_off_work, slow_off_tsum, slow_lds_bytes;
  // slow_kernel takes only rows marked ROW_PENDING (after finish16_kernel)
  int32_t pending_only;
};

// ---------------------------------------------------------------- verify
constexpr int VCHUNK = 2048;           // elements per verify stats partial: one wave, 32 per lane
constexpr int GAMMA_MAX = 256;         // longest draft the verify kernels accept

struct ChunkStats {                    // 32 bytes per (row, chunk)
  float m;                             // chunk max of x (stochastic rows)
  float bv;                            // first max (greedy rows)
  int32_t bi;
  int32_t nan_i;
  double s;                            // sum exp2((x - m) * c)
  float xt;                            // the row's logit at the drafted token, if in this chunk
  int32_t has_xt;
};

struct SeqState {                      // 64 bytes per sequence
  int32_t accepted, next_tok, used, status;
  int32_t rej1;                        // rejected position + 1; 0 if none
  int32_t exact;                       // normalisers below are exact fp64
  float Mt, Mq;                        // row maxima of x at position rej
  double St, Sq;                       // normalisers at position rej
  double R, pad;
};

static_assert(sizeof(ChunkStats) == 32, "ChunkStats layout");
static_assert(sizeof(SeqState) == 64, "SeqState layout");

constexpr int SUB = 512;               // elements per normaliser partial: one wave, 8 per lane
constexpr int NORM_WGS = 8;             // verify_norm workgroups per sequence
constexpr int AMB_CAP = 8;             // undecided residual signs kept per partial

// Exact normaliser partials of the rejected position's row pair over one
// 512-element sub-chunk, with e = exp(z_t - max z_t), f = exp(z_q - max z_q)
// and lam0 the normalisers' ratio known before the pass: the residual
// max(e / St - f / Sq, 0) is St^-1 max(e - lam f, 0) with lam = St / Sq,
// positive for sure where e > lam0 (1 + eps) f, zero where
// e < lam0 (1 - eps) f, and undecided (listed) in between.
struct NormPart {                      // 64 bytes per (sequence, sub-chunk)
  double se, sf;                       // sum e, sum f
  double dp;                           // sum over sure-positive elements of e - lam0 f
  double fp;                           // sum over sure-positive elements of f
  int32_t namb;                        // undecided elements (> AMB_CAP: list overflowed)
  int32_t pad[7];
};
struct AmbEntry {                      // 16 bytes
  double e, f;
};
static_assert(sizeof(NormPart) == 64, "NormPart layout");

struct VerifyArgs {
  const float* target;
  const float* draft;
  const int32_t* draft_ids;
  const double* u;
  const float* temperature;
  int32_t B, gamma, V, nchunk, nsub;
  int32_t draft_rows;                  // the stats grid includes the draft rows
  int32_t* accepted;
  int32_t* next_tok;
  int32_t* used;
  int32_t* row_status;
  ChunkStats* cstats;                  // [(B*(gamma+1) + B*gamma) * nchunk]
  SeqState* seq;                       // [B]
  NormPart* npart;                     // [B * nsub]
  AmbEntry* amb;                       // [B * nsub * AMB_CAP]
};

// Workspace layout (bytes), identical on host and device.
struct SampleWorkspace {
  size_t off_counters, off_stats, off_cands, total;
};

inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

constexpr int SLICE_MAX = 1 << 18;        // elements per slice (bitmap index limit)
constexpr int SLICE_CAP = 8;              // slices per row (V < 2^20 needs at most 4)

// Slices per row: one when the batch alone fills the 256 CUs (no cross-
// workgroup merge at all); otherwise enough slices for about one workgroup
// per CU, each at least 16384 elements long.  (A second round of
// workgroups on a CU pays the start-up and the tail again: at B=64,
// V=128256 seven slices took 41 us for top-p rows and 14 us for greedy rows,
// four take 33 us and 10 us.)
inline int choose_nsplit(int B, int V) {
  int n = B >= 256 ? 1 : (256 + B - 1) / (B > 0 ? B : 1);
  int by_len = V / 16384 > 0 ? V / 16384 : 1;
  if (n > by_len) n = by_len;
  if (n > SLICE_CAP) n = SLICE_CAP;
  int need = (V + SLICE_MAX - 1) / SLICE_MAX;
  if (n < need) n = need;
  return n < 1 ? 1 : n;
}

struct VerifyWorkspace {
  size_t off_cstats, off_seq, off_npart, off_amb, total;
};

inline VerifyWorkspace verify_workspace_layout(int B, int gamma, int V) {
  VerifyWorkspace w;
  int nchunk = (V + VCHUNK - 1) / VCHUNK;
  int nsub = (V + SUB - 1) / SUB;
  size_t rows = (size_t)B * (gamma + 1) + (size_t)B * gamma;
  w.off_cstats = 0;
  w.off_seq = align_up(rows * nchunk * sizeof(ChunkStats), 256);
  w.off_npart = align_up(w.off_seq + (size_t)B * sizeof(SeqState), 256);
  w.off_amb = align_up(w.off_npart + (size_t)B * nsub * sizeof(NormPart), 256);
  w.total = align_up(w.off_amb + (size_t)B * nsub * AMB_CAP * sizeof(AmbEntry), 256);
  return w;
}

inline SampleWorkspace sample_workspace_layout(int B, int ns) {
  SampleWorkspace w;
  w.off_counters = 0;
  w.off_stats = align_up((size_t)(B + 1) * 4, 256);
  w.off_cands = align_up(w.off_stats + (size_t)B * ns * sizeof(SplitStats), 256);
  w.total = align_up(w.off_cands + (size_t)B * ns * CAPS * sizeof(Cand), 256);
  return w;
}

// Record a failure in the thread-local message cx_last_error() returns and
// return `code` (cx_api.hip); for entry points outside cx_api.hip.
int api_fail(int code, const char* fmt, ...);

}  // namespace cx
