// cx_verify.hip -- speculative-decoding verify step for gfx950
// (reference chenxing/engine/speculative.py:67-69 and :145-171).
//
// The reference walks the gamma draft positions serially and stops at the
// first rejection.  Every position's accept test depends only on its own
// target/draft row pair and its own uniform, so the device evaluates all
// positions in parallel and then takes the first rejection.  Stream-ordered
// launches, each reading what the previous one wrote: 1, 3 and 4 when any
// sequence is stochastic (the decision, 2, is taken inside each verify_norm
// workgroup), 1 and 2 when every sequence is greedy:
//
//   1. verify_stats   one wave per 2048-element chunk of every target and
//                     draft row (one HBM read): the chunk max,
//                     sum exp((x - m) / T) (fp32 exp2 terms, fp64 sums) and
//                     the logit at the drafted token, or for greedy rows the
//                     first argmax / first NaN.
//   2. verify_decide  grid B: one wave per row merges its chunks, one lane
//                     per position runs the accept test with Python's
//                     min/max semantics; a test whose ratio lies within the
//                     normalisers' error bound of its uniform is re-decided
//                     with exact fp64 normalisers.
//   3. verify_norm    NORM_WGS workgroups per sequence, each wave looping over
//                     512-element sub-chunks of the row pair at the rejected
//                     position r (the next one's loads in flight): exact fp64 normaliser
//                     partials of p and q, and the residual max(p - q, 0)
//                     split into elements whose sign is sure (summed) and the
//                     few that are not (listed).
//   4. verify_draw    grid B: wave 0 alone sums the exact normalisers, scans
//                     the residual mass of every sub-chunk from the partials,
//                     finds the sub-chunk holding u * R and scans its 512
//                     elements with wave-level prefix sums, with no block
//                     barrier; a draw within 1e-12 (relative) of a step is
//                     redone by the whole workgroup over the whole row pair.
//
// fp64 terms use exp64 (table-driven, within 1 ulp) of fl32(x / T), the
// reference's fp32 quotient (div32).
#include "cx_device.hpp"
#include "cx_sampler.h"
#include "cx_internal.hpp"
#include "cx_timing.hpp"

namespace cx {

// verify_stats workgroups: four waves, each one chunk (no barrier, no LDS).
// Smaller workgroups start as soon as a quarter of a CU's wave slots free up:
// 0.6 us off the 44 us pass at B=32, gamma=7, V=128256 against 16 waves.
// (Waves that loop over chunks with the next chunk's loads in flight were
// slower, 47-52 us.)
constexpr int VS_WG = 256;
constexpr int VS_NW = VS_WG / 64;

// Relative error bound of a chunked normaliser: fp32 exp2 terms (~2 ulp),
// fp32 arguments, and the reference's rounding of x / T to fp32, which
// perturbs each exponent by up to one ulp of |z| (so the bound grows with
// the row maximum zm).
__device__ __forceinline__ double tol_norm(float zm) {
  return 6e-6 + 2.4e-7 * fabs((double)zm);
}

__device__ __forceinline__ const float* trow(const VerifyArgs& A, int b, int i) {
  return A.target + ((size_t)b * (A.gamma + 1) + i) * (size_t)A.V;
}
__device__ __forceinline__ const float* drow(const VerifyArgs& A, int b, int i) {
  return A.draft + ((size_t)b * A.gamma + i) * (size_t)A.V;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Exact normaliser of softmax64(row / T): sum exp(fl32(x / T) - fl32(max x / T)).
__device__ inline double exact_row_sum(const float* row, int V, double invT, double zm,
                                       const double* tab, double* red_d) {
  double s = 0.0;
  for (int e = threadIdx.x; e < V; e += WG) s += exp64(div32(row[e], invT) - zm, tab);
  return block_sum(s, red_d);
}

// Python's min(1.0, p / max(q, 1e-12)) (speculative.py:158).
__device__ __forceinline__ double accept_threshold(double p, double q) {
  double qq = 1e-12 > q ? 1e-12 : q;
  double r = p / qq;
  return r < 1.0 ? r : 1.0;
}

// The rejected position's row pair as the residual sees it.
struct ResidCtx {
  double invT;            // 1 / T
  double zmt, zmq;        // fl32(max x / T) of the target and draft rows
  double invSt, invSq;    // 1 / normalisers
  const double* tab;      // EXP64_TAB in LDS
};

// Residual weight max(p - q, 0) of one element, fp64 (speculative.py:161).
__device__ __forceinline__ double resid(float xt, float xq, const ResidCtx& C) {
  double p = exp64(div32(xt, C.invT) - C.zmt, C.tab) * C.invSt;
  double q = exp64(div32(xq, C.invT) - C.zmq, C.tab) * C.invSq;
  double d = p - q;
  return d > 0.0 ? d : 0.0;
}

// Exact residual draw over the whole row pair (single workgroup, fp64):
// numpy's choice(V, p=r/R) with r = max(p - q, 0) (speculative.py:161-166).
// Returns -1 when R <= 0 (the caller falls back to argmax(row)).
__device__ inline int exact_residual_draw(const float* tr, const float* dr, int V,
                                          const ResidCtx& C, double u, double* red_d,
                                          int* red_i, double* tsum) {
  const int t = threadIdx.x;
  const int per = (V + WG - 1) / WG;
  const int e0 = min(V, t * per), e1 = min(V, e0 + per);
  double s = 0.0;
  for (int e = e0; e < e1; ++e) s += resid(tr[e], dr[e], C);
  tsum[t] = s;
  const double R = block_sum(s, red_d);
  if (!(R > 0.0)) return -1;
  block_scan(tsum, WG, red_d);            // inclusive prefix of the per-thread sums
  const double prev = t > 0 ? tsum[t - 1] : 0.0;
  int found = INT_MAX;
  if ((prev / R) / (tsum[WG - 1] / R) <= u && (tsum[t] / R) / (tsum[WG - 1] / R) > u) {
    double run = prev;
    for (int e = e0; e < e1; ++e) {
      run += resid(tr[e], dr[e], C);
      if ((run / R) / (tsum[WG - 1] / R) > u) { found = e; break; }
    }
  }
  found = block_min(found, red_i, INT_MAX);
  if (found == INT_MAX) found = V - 1;
  return found;
}

__device__ inline int row_argmax(const float* row, int V, double* red_d, int* red_i) {
  double bv = -__builtin_inf();
  int bi = INT_MAX, ni = INT_MAX;
  for (int e = threadIdx.x; e < V; e += WG) {
    float x = row[e];
    if (x != x) ni = min(ni, e);
    else argmax_merge(bv, bi, (double)x, e);
  }
  block_argmax(bv, bi, red_d, red_i);
  ni = block_min(ni, red_i, INT_MAX);
  return ni != INT_MAX ? ni : (bi == INT_MAX ? 0 : bi);
}

// ------------------------------------------------------------ 1. stats
static_assert(VCHUNK == 64 * 32, "a stats partial is one wave of 8 float4 per lane");

// One wave per 2048-element chunk of a row: every load in flight at once,
// wave-level reductions only (no barriers), one ChunkStats per wave.
__global__ __launch_bounds__(VS_WG) void verify_stats(VerifyArgs A) {
  const int g = A.gamma;
  const int nt = A.B * (g + 1);
  const int per_row = (A.nchunk + VS_NW - 1) / VS_NW;
  const int r = blockIdx.x / per_row;
  const int ch = (blockIdx.x % per_row) * VS_NW + wave_id();
  if (ch >= A.nchunk) return;
  int b, i;
  const float* row;
  bool target;
  if (r < nt) { b = r / (g + 1); i = r % (g + 1); row = trow(A, b, i); target = true; }
  else { b = (r - nt) / g; i = (r - nt) % g; row = drow(A, b, i); target = false; }
  const float T = A.temperature[b];
  const bool greedy = T == 0.0f;
  if (greedy && !target) return;                     // greedy never reads q rows
  const int l = lane_id();
  const int lo = ch * VCHUNK, hi = min(A.V, lo + VCHUNK);
  float x[32];
  if (hi - lo == VCHUNK && (((uintptr_t)(row + lo)) & 15) == 0) {
    const f32x4* vp = (const f32x4*)(row + lo);
    f32x4 q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = __builtin_nontemporal_load(&vp[j * 64 + l]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      x[4 * j] = q[j].x; x[4 * j + 1] = q[j].y; x[4 * j + 2] = q[j].z; x[4 * j + 3] = q[j].w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int e = lo + (j * 64 + l) * 4 + c;
        x[4 * j + c] = e < hi ? row[e] : -__builtin_inff();
      }
  }
  // element index of x[4 j + c]: lo + (j * 64 + l) * 4 + c
  ChunkStats cs;
  cs.m = 0.0f; cs.bv = 0.0f; cs.bi = INT_MAX; cs.nan_i = INT_MAX; cs.s = 0.0;
  if (greedy) {
    // first maximum: the largest (orderable value, ~index) key; NaN apart
    uint64_t key = 0;
    int ni = INT_MAX;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float v = x[4 * j + c];
        const int e = lo + (j * 64 + l) * 4 + c;
        if (v != v) { ni = min(ni, e); continue; }
        if (e >= hi) continue;
        const uint64_t k = ((uint64_t)f2key(v) << 32) | (uint32_t)~(uint32_t)e;
        key = k > key ? k : key;
      }
    key = wave_reduce(key, OpMax());
    ni = wave_reduce(ni, OpMin());
    if (key != 0) { cs.bv = key2f((uint32_t)(key >> 32)); cs.bi = (int)~(uint32_t)key; }
    cs.nan_i = ni;
  } else {
    float m = -__builtin_inff();
#pragma unroll
    for (int k = 0; k < 32; ++k) m = fmaxf(m, x[k]);
    const float M = wave_reduce(m, OpMax());
    const float mm = fmaxf(M, -3.402823466e38f);
    const float c = (float)(1.4426950408889634 / (double)T);
    double sd = 0.0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {                     // four fp32 terms, then fp64
      float ts = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) ts += __builtin_amdgcn_exp2f((x[4 * j + k] - mm) * c);
      sd += (double)ts;
    }
    cs.m = M;
    cs.s = wave_reduce(sd, OpAdd());
  }
  const int tok = i < g ? A.draft_ids[(size_t)b * g + i] : -1;
  const bool here = tok >= lo && tok < hi;
  cs.has_xt = here ? 1 : 0;
  cs.xt = 0.0f;
  if (l == 0) {
    if (here) cs.xt = row[tok];
    A.cstats[(size_t)r * A.nchunk + ch] = cs;
  }
}

// ------------------------------------------------------------ 2. decide
// Merge the chunk statistics of stochastic row r (one wave): max of x, sum
// exp((x - max) / T) and the logit at the drafted token.
__device__ inline void merge_row(const VerifyArgs& A, int r, float T, float& M, double& S,
                                 float& xt) {
  const ChunkStats* cs = A.cstats + (size_t)r * A.nchunk;
  const double c = (double)(float)(1.4426950408889634 / (double)T);
  const int l = lane_id();
  constexpr int PL = 8;                               // partials per lane (nchunk <= 512)
  float m[PL];
  double s[PL];
  float xv = 0.0f;
  int has = 0;
#pragma unroll
  for (int j = 0; j < PL; ++j) {
    const int k = j * 64 + l;
    const bool in = k < A.nchunk;
    m[j] = in ? cs[k].m : -__builtin_inff();
    s[j] = in ? cs[k].s : 0.0;
    if (in && cs[k].has_xt) { has = 1; xv = cs[k].xt; }
  }
  float lm = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < PL; ++j) lm = fmaxf(lm, m[j]);
  M = wave_reduce(lm, OpMax());
  double ls = 0.0;
  int nan = 0;
#pragma unroll
  for (int j = 0; j < PL; ++j) {
    nan |= s[j] != s[j];
    if (s[j] != 0.0) ls += s[j] * exp2((double)(m[j] - M) * c);
  }
  S = wave_reduce(ls, OpAdd());
  if (wave_reduce(nan, OpMax())) S = __builtin_nan("");
  const uint64_t hb = __ballot(has);
  xt = hb ? lane_read(xv, __builtin_ctzll(hb)) : 0.0f;
}

// First maximum / first NaN of greedy row r from its chunk statistics (one
// wave).
__device__ inline int merge_greedy(const VerifyArgs& A, int r) {
  const ChunkStats* cs = A.cstats + (size_t)r * A.nchunk;
  const int l = lane_id();
  uint64_t key = 0;
  int ni = INT_MAX;
  for (int k = l; k < A.nchunk; k += 64) {
    const ChunkStats c = cs[k];
    if (c.bi != INT_MAX) {
      const uint64_t kk = ((uint64_t)f2key(c.bv) << 32) | (uint32_t)~(uint32_t)c.bi;
      key = kk > key ? kk : key;
    }
    ni = min(ni, c.nan_i);
  }
  key = wave_reduce(key, OpMax());
  ni = wave_reduce(ni, OpMin());
  return ni != INT_MAX ? ni : (key == 0 ? 0 : (int)~(uint32_t)key);
}

// The decision of sequence b (all threads of the workgroup; the same state
// on every thread): the accept tests, the first rejection, and its row
// pair's statistics.  `write`: also store the sequence's outputs and its
// SeqState.  tab: EXP64_TAB in LDS.
__device__ inline SeqState decide_seq(const VerifyArgs& A, int b, bool write, const double* tab) {
  __shared__ double red_d[2 * NWAVE + 4];
  __shared__ int red_i[2 * NWAVE + 4];
  __shared__ float s_M[2 * GAMMA_MAX + 1];
  __shared__ double s_S[2 * GAMMA_MAX + 1];
  __shared__ float s_x[2 * GAMMA_MAX + 1];
  __shared__ int s_best[GAMMA_MAX + 1];
  __shared__ int s_f, s_kind;
  __shared__ SeqState s_out;
  const int g = A.gamma;
  const int t = threadIdx.x;
  const float T = A.temperature[b];
  const int nt = A.B * (g + 1);
  const int32_t* ids = A.draft_ids + (size_t)b * g;
  SeqState out;
  out.accepted = 0; out.next_tok = -1; out.used = 0; out.status = 0;
  out.rej1 = 0; out.exact = 0; out.Mt = 0.f; out.Mq = 0.f;
  out.St = 0.0; out.Sq = 0.0; out.R = 0.0; out.pad = 0.0;
  if (T == 0.0f) {                                    // speculative.py:150-155
    for (int i = wave_id(); i <= g; i += NWAVE) {
      const int best = merge_greedy(A, b * (g + 1) + i);
      if (lane_id() == 0) s_best[i] = best;
    }
    __syncthreads();
    if (t == 0) {
      int acc = 0;
      while (acc < g && ids[acc] == s_best[acc]) ++acc;
      if (write) {
        A.accepted[b] = acc;
        A.next_tok[b] = s_best[acc];                  // row gamma: the bonus token
        A.used[b] = 0;
        A.row_status[b] = CX_ROW_GREEDY;
        A.seq[b] = out;
      }
      s_out = out;
    }
    __syncthreads();
    return s_out;
  }
  // ids outside [0, V) or missing draft rows cannot be verified: report the
  // sequence as unsupported
  int bad = (A.draft == nullptr || !A.draft_rows) ? 1 : 0;
  for (int k = t; k < g; k += WG) bad |= (ids[k] < 0 || ids[k] >= A.V) ? 1 : 0;
  bad = block_max(bad, red_i, 0);
  if (bad) {
    if (t == 0) {
      if (write) {
        A.accepted[b] = 0; A.next_tok[b] = -1; A.used[b] = 0;
        A.row_status[b] = CX_ROW_UNSUPPORTED;
        A.seq[b] = out;
      }
      s_out = out;
    }
    __syncthreads();
    return s_out;
  }
  // one wave per row: target rows 0..g-1 at [0, g), draft rows at [g, 2g)
  for (int j = wave_id(); j < 2 * g; j += NWAVE) {
    const int r = j < g ? b * (g + 1) + j : nt + b * g + (j - g);
    float M, xt;
    double S;
    merge_row(A, r, T, M, S, xt);
    if (lane_id() == 0) { s_M[j] = M; s_S[j] = S; s_x[j] = xt; }
  }
  __syncthreads();
  const double* ub = A.u + (size_t)b * (g + 1);
  const double invT = 1.0 / (double)T;
  int start = 0, rej = -1;
  bool exact = false;
  double St = 0.0, Sq = 0.0;
  for (;;) {
    // first position at or after `start` that rejects, or whose test lies
    // within the error bound of its uniform (speculative.py:156-160)
    if (t < 64) {
      int f = -1;
      for (int base = start; base < g && f < 0; base += 64) {
        const int i = base + t;
        bool rj = false, nr = false;
        if (i < g) {
          const float zmt = s_M[i] / T, zmq = s_M[g + i] / T;
          const double st = s_S[i], sqq = s_S[g + i];
          const double et = exp64(div32(s_x[i], invT) - (double)zmt, tab);
          const double eq = exp64(div32(s_x[g + i], invT) - (double)zmq, tab);
          const double thr = accept_threshold(et / st, eq / sqq);
          const double ui = ub[i];
          const double rel = 2.0 * (tol_norm(zmt) + tol_norm(zmq));
          const double tol = rel * (thr == thr ? thr : 1.0) + 1e-300;
          const bool q_floor_near = fabs(eq / sqq - 1e-12) <= rel * 1e-12;
          nr = st == st && sqq == sqq && (fabs(ui - thr) <= tol || q_floor_near);
          rj = !(ui < thr);
        }
        const uint64_t m = __ballot(rj || nr);
        if (m) {
          const int fl = __builtin_ctzll(m);
          f = base + fl;
          if (t == fl) { s_f = f; s_kind = nr ? 2 : 1; }
        }
      }
      if (t == 0 && f < 0) { s_f = g; s_kind = 0; }
    }
    __syncthreads();
    const int f = s_f, kind = s_kind;
    __syncthreads();
    if (kind == 0) break;                              // every test accepts
    St = s_S[f];
    Sq = s_S[g + f];
    if (kind == 1) { rej = f; break; }
    // near the decision: recompute both normalisers exactly (fp64 over the rows)
    const float zmt = s_M[f] / T, zmq = s_M[g + f] / T;
    St = exact_row_sum(trow(A, b, f), A.V, invT, (double)zmt, tab, red_d);
    Sq = exact_row_sum(drow(A, b, f), A.V, invT, (double)zmq, tab, red_d);
    const double et = exp64(div32(s_x[f], invT) - (double)zmt, tab);
    const double eq = exp64(div32(s_x[g + f], invT) - (double)zmq, tab);
    if (!(ub[f] < accept_threshold(et / St, eq / Sq))) { rej = f; exact = true; break; }
    start = f + 1;
  }
  if (t == 0) {
    if (rej >= 0) {
      out.rej1 = rej + 1;
      out.Mt = s_M[rej];
      out.Mq = s_M[g + rej];
      out.St = St;
      out.Sq = Sq;
      out.exact = exact;
    }
    if (write) {
      if (rej < 0) {                                  // speculative.py:168-171
        A.accepted[b] = g;
        A.next_tok[b] = -1;
        A.used[b] = g;
        A.row_status[b] = CX_ROW_OK;
      } else {
        A.accepted[b] = rej;
        A.used[b] = rej + 2;                          // tests 0..rej, then the residual draw
      }
      A.seq[b] = out;
    }
    s_out = out;
  }
  __syncthreads();
  return s_out;
}

// Batches whose sequences are all greedy: the decision alone, one workgroup
// per sequence.
__global__ __launch_bounds__(WG) void verify_decide(VerifyArgs A) {
  __shared__ double tab[64];
  load_exp64_tab(tab);
  decide_seq(A, blockIdx.x, true, tab);
}

// ------------------------------------------------------------ 3. normaliser partials
// The margin around lam0 inside which a residual sign is not yet known:
// well above the error of the fp32-term normalisers behind lam0, or tiny
// when lam0 came from exact ones.
__device__ __forceinline__ double sign_margin(const SeqState& q, float T) {
  if (q.exact) return 1e-9;
  const double m = 20.0 * (tol_norm(q.Mt / T) + tol_norm(q.Mq / T));
  return m > 1e-3 ? m : 1e-3;
}

// Eight consecutive logits [e0, e0 + 8) of a row (zeros past hi), with two
// 16-byte loads when they are whole and aligned.  Plain loads: the draw reads
// one sub-chunk of the same row pair again, from the L2 (1 us off the verify
// step against non-temporal ones; the stats pass keeps them: 4 us slower
// without).
__device__ __forceinline__ void load8(const float* row, int e0, int hi, float (&x)[8]) {
  if (e0 + 8 <= hi && (((uintptr_t)(row + e0)) & 15) == 0) {
    const f32x4 a = *((const f32x4*)(row + e0));
    const f32x4 c = *((const f32x4*)(row + e0) + 1);
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = c.x; x[5] = c.y; x[6] = c.z; x[7] = c.w;
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = e0 + j < hi ? row[e0 + j] : 0.0f;
  }
}

static_assert(SUB == 64 * 8, "a normaliser partial is one wave of 8 elements per lane");

// e = exp(fl32(xt / T) - zmt) and f = exp(fl32(xq / T) - zmq) for eight
// elements (zero past hi); UNIT: T == 1, so fl32(x / T) = x.
template <bool UNIT>
__device__ __forceinline__ void pair_terms(const float (&xt)[8], const float (&xq)[8], int e0,
                                           int hi, double invT, double zmt, double zmq,
                                           const double* tab, double (&ev)[8],
                                           double (&fv)[8]) {
#pragma unroll
  for (int j = 0; j < 8; ++j) {                       // branch-free: the exps interleave
    const bool in = e0 + j < hi;
    const double zt = UNIT ? (double)xt[j] : div32(xt[j], invT);
    const double zq = UNIT ? (double)xq[j] : div32(xq[j], invT);
    ev[j] = in ? exp64_neg(zt - zmt, tab) : 0.0;
    fv[j] = in ? exp64_neg(zq - zmq, tab) : 0.0;
  }
}

// One wave per 512-element sub-chunk of the rejected row pair.
__global__ __launch_bounds__(WG) void verify_norm(VerifyArgs A) {
  __shared__ double tab[64];
  const int b = blockIdx.x / NORM_WGS;
  load_exp64_tab(tab);
  // every workgroup of the sequence takes the decision itself (a launch
  // less than a separate decide kernel); the first one stores it
  const SeqState q = decide_seq(A, b, blockIdx.x % NORM_WGS == 0, tab);
  const float T = A.temperature[b];
  if (T == 0.0f || q.rej1 == 0) return;
  const int r = q.rej1 - 1;
  const float* tr = trow(A, b, r);
  const float* dr = drow(A, b, r);
  const double zmt = q.Mt / T, zmq = q.Mq / T;
  const double invT = 1.0 / (double)T;
  const double lam0 = q.St / q.Sq;
  const double eps = sign_margin(q, T);
  const int l = lane_id();
  // this wave's sub-chunks: sub0, sub0 + stride, ...; the next one's loads
  // are issued before the current one is reduced
  const int stride = NORM_WGS * NWAVE;
  int sub = (blockIdx.x % NORM_WGS) * NWAVE + wave_id();
  float xt[8], xq[8];
  if (sub < A.nsub) {
    load8(tr, sub * SUB + l * 8, A.V, xt);
    load8(dr, sub * SUB + l * 8, A.V, xq);
  }
  for (; sub < A.nsub; sub += stride) {
    const int e0 = sub * SUB + l * 8;
    double ev[8], fv[8];
    if (T == 1.0f) pair_terms<true>(xt, xq, e0, A.V, invT, zmt, zmq, tab, ev, fv);
    else pair_terms<false>(xt, xq, e0, A.V, invT, zmt, zmq, tab, ev, fv);
    if (sub + stride < A.nsub) {
      load8(tr, (sub + stride) * SUB + l * 8, A.V, xt);
      load8(dr, (sub + stride) * SUB + l * 8, A.V, xq);
    }
    double se = 0.0, sf = 0.0, dp = 0.0, fp = 0.0;
    unsigned amb = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const double e = ev[j], f = fv[j];
      se += e;
      sf += f;
      const double lf = lam0 * f;
      const bool pos = e > lf * (1.0 + eps);
      dp += pos ? e - lf : 0.0;
      fp += pos ? f : 0.0;
      amb |= (!pos && e >= lf * (1.0 - eps) && (e != 0.0 || f != 0.0)) ? 1u << j : 0u;
    }
    se = wave_reduce(se, OpAdd());
    sf = wave_reduce(sf, OpAdd());
    dp = wave_reduce(dp, OpAdd());
    fp = wave_reduce(fp, OpAdd());
    const size_t part = (size_t)b * A.nsub + sub;
    int namb = 0;
    if (__ballot(amb != 0)) {                         // rare: list the undecided signs
      AmbEntry* out = A.amb + part * AMB_CAP;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const bool a = (amb >> j) & 1u;
        const uint64_t m = __ballot(a);
        const int idx = namb + lanes_below(m);
        if (a && idx < AMB_CAP) { out[idx].e = ev[j]; out[idx].f = fv[j]; }
        namb += __builtin_popcountll(m);
      }
    }
    if (l == 0) {
      NormPart P;
      P.se = se; P.sf = sf; P.dp = dp; P.fp = fp;
      P.namb = namb;
      for (int k = 0; k < 7; ++k) P.pad[k] = 0;
      A.npart[part] = P;
    }
  }
}

// ------------------------------------------------------------ 4. draw
// Partials s0, s0 + 64, s0 + 128, s0 + 192 of a sequence (indices past ns
// read the last one, unused), loaded together.
__device__ __forceinline__ void load_parts(const NormPart* np, int ns, int s0, double (&se)[4],
                                           double (&sf)[4], double (&dp)[4], double (&fp)[4],
                                           int (&na)[4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const NormPart& P = np[min(s0 + 64 * j, ns - 1)];
    se[j] = P.se;
    sf[j] = P.sf;
    dp[j] = P.dp;
    fp[j] = P.fp;
    na[j] = P.namb;
  }
}

// numpy's choice(V, p=r/R) with r = max(p - q, 0) (speculative.py:161-166).
// With e, f the exp terms of the rejected row pair, St, Sq their exact sums
// and lam = St / Sq, r = St^-1 w with w = max(e - lam f, 0): the draw runs on
// w and W = sum w.
__global__ __launch_bounds__(WG) void verify_draw(VerifyArgs A) {
  __shared__ double red_d[2 * NWAVE + 4];
  __shared__ int red_i[2 * NWAVE + 4];
  __shared__ double tab[64];
  __shared__ double tsum[2 * WG];
  __shared__ double s_fp[2 * WG];                     // the partials' fp, then ...
  __shared__ int s_na[2 * WG];                        // ... namb, kept from the first pass
  __shared__ double s_lam[3];
  __shared__ int s_state[2];                          // {0 undecided, 1 token, 2 NaN}, token
  const int b = blockIdx.x;
  const int t = threadIdx.x;
  const float T = A.temperature[b];
  const SeqState q = A.seq[b];
  const int ns = A.nsub;                              // <= 2 * WG
  const NormPart* np = A.npart + (size_t)b * ns;
  // wave 0's first four partials per lane, in flight with the state and the
  // table (the workspace holds them whether or not the row draws)
  double pse[4], psf[4], pdp[4], pfp[4];
  int pna[4];
  if (wave_id() == 0) load_parts(np, ns, lane_id(), pse, psf, pdp, pfp, pna);
  load_exp64_tab(tab);
  if (T == 0.0f || q.rej1 == 0) return;
  const int r = q.rej1 - 1;
  const int g = A.gamma;
  const float* tr = trow(A, b, r);
  const float* dr = drow(A, b, r);
  const double u = A.u[(size_t)b * (g + 1) + r + 1];
  ResidCtx C;
  C.invT = 1.0 / (double)T;
  C.zmt = q.Mt / T;
  C.zmq = q.Mq / T;
  C.tab = tab;
  const double err = 1e-12;                           // relative rounding of the sums
  // Wave 0 decides from the partials (lane-strided sums and wave scans, no
  // block barriers): the exact normalisers, every sub-chunk's residual mass,
  // the sub-chunk holding u * W and, scanned in id order, the element in it.
  // A draw within err of a step, a list that overflowed, W too small or NaN
  // leave the row to the block-wide exact redo below.
  if (wave_id() == 0) {
    const int l = lane_id();
    // one pass over the partials, four per lane loaded together: the sums,
    // and each lane keeps its sub-chunks' dp, fp and namb in LDS for the
    // residual masses
    double st = 0.0, sq = 0.0;
    for (int s0 = l; s0 < ns; s0 += 4 * 64) {
      if (s0 != l) load_parts(np, ns, s0, pse, psf, pdp, pfp, pna);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int s = s0 + 64 * j;
        if (s < ns) {
          st += pse[j];
          sq += psf[j];
          tsum[s] = pdp[j];
          s_fp[s] = pfp[j];
          s_na[s] = pna[j];
        }
      }
    }
    const double St = wave_reduce(st, OpAdd()), Sq = wave_reduce(sq, OpAdd());
    const double lam = St / Sq, lam0 = q.St / q.Sq;
    // residual mass of each sub-chunk: the sure-positive part and the list
    // (a list's entries are loaded together)
    bool over = false;
    for (int s = l; s < ns; s += 64) {
      const int na = s_na[s];
      double w = 0.0;
      if (na > AMB_CAP) {
        over = true;
      } else {
        w = tsum[s] - (lam - lam0) * s_fp[s];
        if (na > 0) {
          const AmbEntry* am = A.amb + ((size_t)b * ns + s) * AMB_CAP;
          AmbEntry a[AMB_CAP];
#pragma unroll
          for (int j = 0; j < AMB_CAP; ++j)
            if (j < na) a[j] = am[j];
#pragma unroll
          for (int j = 0; j < AMB_CAP; ++j)
            if (j < na) {
              const double d = a[j].e - lam * a[j].f;
              w += d > 0.0 ? d : 0.0;
            }
        }
      }
      tsum[s] = w;
    }
    const bool ok0 = !wave_reduce((int)over, OpOr());
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // prefix sums over the sub-chunks in place (tsum[s] = mass through s),
    // 64 at a time with a carry; each lane rewrites only its own entries
    double carry = 0.0;
    for (int s0 = 0; s0 < ns; s0 += 64) {
      const double w = s0 + l < ns ? tsum[s0 + l] : 0.0;
      const double incl = carry + wave_scan_dpp(w);
      if (s0 + l < ns) tsum[s0 + l] = incl;
      carry = lane_read(incl, 63);
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    const double W = carry;
    int state = 0, tok = -1;
    if (W != W || St != St || Sq != Sq) {
      state = 2;                                      // NaN probabilities: numpy raises
    } else if (ok0 && W > err * St) {
      // the sub-chunk holding u * W, and u's distance to its edges
      int found = INT_MAX;
      double gap = 1.0;
      for (int s = l; s < ns; s += 64) {
        const double lo = s > 0 ? tsum[s - 1] / W : 0.0, hi = tsum[s] / W;
        if (lo <= u && u < hi) {
          found = s;
          gap = fmin(s > 0 ? u - lo : 1.0, s < ns - 1 ? hi - u : 1.0);
        }
      }
      found = wave_reduce(found, OpMin());
      gap = wave_reduce(gap, OpMin());
      if (found != INT_MAX && gap > err) {
        // the sub-chunk's elements in id order, eight consecutive per lane
        const double before = found > 0 ? tsum[found - 1] : 0.0;
        const int e0 = found * SUB + l * 8;
        double w8[8];
        double run = 0.0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int e = e0 + j;
          double d = 0.0;
          if (e < A.V)
            d = exp64_neg(div32(tr[e], C.invT) - C.zmt, tab) -
                lam * exp64_neg(div32(dr[e], C.invT) - C.zmq, tab);
          run += d > 0.0 ? d : 0.0;
          w8[j] = run;                                // inclusive prefix within the lane
        }
        const double incl = wave_scan_dpp(run);
        const double lane0 = before + (incl - run);   // prefix before this lane
        int hit = INT_MAX;
        double margin = 1.0;
#pragma unroll
        for (int j = 7; j >= 0; --j) {
          const int e = e0 + j;
          if (e >= A.V) continue;
          const double lo = (lane0 + (j > 0 ? w8[j - 1] : 0.0)) / W;
          const double hi = (lane0 + w8[j]) / W;
          if (lo <= u && u < hi) { hit = e; margin = fmin(u - lo, hi - u); }
        }
        hit = wave_reduce(hit, OpMin());
        margin = wave_reduce(margin, OpMin());
        if (hit != INT_MAX && margin > err) { state = 1; tok = hit; }
      }
    }
    if (l == 0) {
      s_state[0] = state;
      s_state[1] = tok;
      s_lam[0] = St; s_lam[1] = Sq;
    }
  }
  __syncthreads();
  const int state = s_state[0];
  int tok = s_state[1], flag = 0;
  if (state == 2) {
    if (t == 0) {
      A.next_tok[b] = -1;
      A.used[b] = r + 1;
      A.row_status[b] = CX_ROW_ERROR;
    }
    return;
  }
  if (state == 0) {                                   // exact fp64 redo over the row pair
    C.invSt = 1.0 / s_lam[0];
    C.invSq = 1.0 / s_lam[1];
    tok = exact_residual_draw(tr, dr, A.V, C, u, red_d, red_i, tsum);
    flag = CX_ROW_FLAG_EXACT;
    if (tok < 0) {                                    // R <= 0: argmax(row), no draw
      tok = row_argmax(tr, A.V, red_d, red_i);
      if (t == 0) A.used[b] = r + 1;
    }
  }
  if (t == 0) {
    A.next_tok[b] = tok;
    A.row_status[b] = CX_ROW_OK | flag;
  }
}

int launch_verify(const VerifyArgs& A, bool any_stochastic, hipStream_t s) {
  const int nt = A.B * (A.gamma + 1);
  const int nrows = nt + (any_stochastic ? A.B * A.gamma : 0);
  const int per_row = (A.nchunk + VS_NW - 1) / VS_NW;
  timed_launch(CX_KERNEL_VERIFY_STATS, verify_stats, dim3(nrows * per_row), dim3(VS_WG), 0, s, A);
  if (any_stochastic) {
    // verify_norm takes the decision in each of its workgroups
    timed_launch(CX_KERNEL_VERIFY_REST, verify_norm, dim3(A.B * NORM_WGS), dim3(WG), 0, s, A);
    timed_launch(CX_KERNEL_VERIFY_REST, verify_draw, dim3(A.B), dim3(WG), 0, s, A);
  } else {
    timed_launch(CX_KERNEL_VERIFY_REST, verify_decide, dim3(A.B), dim3(WG), 0, s, A);
  }
  return (int)hipGetLastError();
}

}  // namespace cx
