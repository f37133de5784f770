// cx_verify.hip -- speculative-decoding verify step for gfx950
// (reference chenxing/engine/speculative.py:67-69 and :145-171).
//
// The reference walks the gamma draft positions serially and stops at the
// first rejection.  Every position's accept test depends only on its own
// target/draft row pair and its own uniform, so the device evaluates all
// positions in parallel and then takes the first rejection:
//
//   1. verify_stats    grid (rows x chunks): one HBM read of every target
//                      and draft row; per chunk the row max and
//                      sum exp((x - m) / T) (fp32 exp2 terms, fp64 sums), or
//                      for greedy rows the first argmax / first NaN.
//   2. verify_decide   grid B: merges the chunks and runs the accept tests in
//                      order with Python's min/max semantics.  A test whose
//                      ratio lies within the normalisers' error bound of its
//                      uniform is re-decided with exact fp64 normalisers.
//   3. verify_residual grid (B x chunks): for a rejected position r, the
//                      chunk masses of max(p - q, 0) (fp64).
//   4. verify_draw     grid B: locates u * R among the chunk masses and scans
//                      the chunk; a draw within the error bound of a step,
//                      or R <= 0, is redone exactly in fp64.
#include "cx_device.hpp"
#include "cx_sampler.h"
#include "cx_internal.hpp"
#include "cx_timing.hpp"

namespace cx {

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

// ------------------------------------------------------------ 1. stats
__global__ __launch_bounds__(WG) void verify_stats(VerifyArgs A) {
  __shared__ double red_d[2 * NWAVE + 4];
  __shared__ int red_i[2 * NWAVE + 4];
  const int nt = A.B * (A.gamma + 1);
  const int r = blockIdx.x / A.nchunk;
  const int ch = blockIdx.x % A.nchunk;
  int b, i;
  const float* row;
  if (r < nt) { b = r / (A.gamma + 1); i = r % (A.gamma + 1); row = trow(A, b, i); }
  else { b = (r - nt) / A.gamma; i = (r - nt) % A.gamma; row = drow(A, b, i); }
  const float T = A.temperature[b];
  const bool greedy = T == 0.0f;
  if (greedy && r >= nt) return;                       // greedy never reads q rows
  const int lo = ch * VCHUNK, hi = min(A.V, lo + VCHUNK);
  const int t = threadIdx.x;
  ChunkStats* out = A.cstats + (size_t)r * A.nchunk + ch;
  const bool vec = (((uintptr_t)row) & 15) == 0;
  const int64_t v0 = vec ? lo / 4 : 0, v1 = vec ? hi / 4 : 0;
  const f32x4* vp = (const f32x4*)row;
  if (greedy) {
    float bv = -__builtin_inff();
    int bi = INT_MAX, ni = INT_MAX;
    for (int64_t vi = v0 + t; vi < v1; vi += WG) {
      f32x4 q = __builtin_nontemporal_load(&vp[vi]);
      float x[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (x[j] > bv) { bv = x[j]; bi = (int)(vi * 4 + j); }
        if (x[j] != x[j] && ni == INT_MAX) ni = (int)(vi * 4 + j);
      }
    }
    for (int64_t e = (vec ? (v1 * 4 > lo ? v1 * 4 : lo) : lo) + t; e < hi; e += WG) {
      float x = row[e];
      if (x > bv) { bv = x; bi = (int)e; }
      if (x != x && ni == INT_MAX) ni = (int)e;
    }
    double dv = bi == INT_MAX ? -__builtin_inf() : (double)bv;
    block_argmax(dv, bi, red_d, red_i);
    ni = block_min(ni, red_i, INT_MAX);
    if (t == 0) { out->bv = (float)dv; out->bi = bi; out->nan_i = ni; out->m = 0; out->s = 0; }
    return;
  }
  const float c = (float)(1.4426950408889634 / (double)T);
  float m = -__builtin_inff();
  double s = 0.0;
  constexpr int U = 4;
  for (int64_t base = v0 + t; base < v1; base += (int64_t)U * WG) {
    f32x4 q[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (base + u * WG < v1) q[u] = __builtin_nontemporal_load(&vp[base + u * WG]);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (base + u * WG >= v1) break;
      float x[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
      float vm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
      if (vm > m) {
        if (s != 0.0) s *= exp2((double)(m - vm) * (double)c);
        m = vm;
      }
      const float mm = fmaxf(m, -3.402823466e38f);
      float ts = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) ts += __builtin_amdgcn_exp2f((x[j] - mm) * c);
      s += (double)ts;
    }
  }
  for (int64_t e = (vec ? (v1 * 4 > lo ? v1 * 4 : lo) : lo) + t; e < hi; e += WG) {
    float x = row[e];
    if (x > m) {
      if (s != 0.0) s *= exp2((double)(m - x) * (double)c);
      m = x;
    }
    s += (double)__builtin_amdgcn_exp2f((x - fmaxf(m, -3.402823466e38f)) * c);
  }
  float M = block_max(m, (float*)red_d, -__builtin_inff());
  double sc = s != 0.0 ? s * exp2((double)(m - M) * (double)c) : 0.0;
  double S = block_sum(sc, red_d);
  if (t == 0) { out->m = M; out->s = S; out->bi = INT_MAX; out->nan_i = INT_MAX; out->bv = 0; }
}

// Merge a row's chunk statistics: max of x and sum exp((x - max) / T).
__device__ inline void merge_row(const VerifyArgs& A, int r, float T, float& M, double& S) {
  const ChunkStats* cs = A.cstats + (size_t)r * A.nchunk;
  const double c = (double)(float)(1.4426950408889634 / (double)T);
  M = -__builtin_inff();
  for (int k = 0; k < A.nchunk; ++k) M = fmaxf(M, cs[k].m);
  S = 0.0;
  bool nan = false;
  for (int k = 0; k < A.nchunk; ++k) {
    nan |= cs[k].s != cs[k].s;
    if (cs[k].s != 0.0) S += cs[k].s * exp2((double)(cs[k].m - M) * c);
  }
  if (nan) S = __builtin_nan("");
}

// Exact normaliser of softmax64(row / T): sum exp(f64(x / T) - f64(max(x) / T)).
__device__ inline double exact_row_sum(const float* row, int V, float T, float zm,
                                       double* red_d) {
  double s = 0.0;
  for (int e = threadIdx.x; e < V; e += WG) s += exp((double)(row[e] / T) - (double)zm);
  return block_sum(s, red_d);
}

// Python's min(1.0, p / max(q, 1e-12)) (speculative.py:158).
__device__ __forceinline__ double accept_threshold(double p, double q) {
  double qq = 1e-12 > q ? 1e-12 : q;
  double r = p / qq;
  return r < 1.0 ? r : 1.0;
}

// ------------------------------------------------------------ 2. decide
__global__ __launch_bounds__(WG) void verify_decide(VerifyArgs A) {
  __shared__ double red_d[2 * NWAVE + 4];
  __shared__ int s_verdict;
  const int b = blockIdx.x;
  const int t = threadIdx.x;
  const int g = A.gamma;
  const float T = A.temperature[b];
  SeqState* sq = A.seq + b;
  const int nt = A.B * (g + 1);
  if (T == 0.0f) {                                    // speculative.py:150-155
    if (t == 0) {
      int acc = 0, nxt = -1;
      for (int i = 0; i <= g; ++i) {
        const ChunkStats* cs = A.cstats + ((size_t)b * (g + 1) + i) * A.nchunk;
        double bv = -__builtin_inf();
        int bi = INT_MAX, ni = INT_MAX;
        for (int k = 0; k < A.nchunk; ++k) {
          if (cs[k].bi != INT_MAX) argmax_merge(bv, bi, (double)cs[k].bv, cs[k].bi);
          ni = min(ni, cs[k].nan_i);
        }
        int best = ni != INT_MAX ? ni : (bi == INT_MAX ? 0 : bi);
        if (i == g || A.draft_ids[(size_t)b * g + i] != best) { nxt = best; break; }
        ++acc;
      }
      A.accepted[b] = acc;
      A.next_tok[b] = nxt;
      A.used[b] = 0;
      A.row_status[b] = CX_ROW_GREEDY;
      sq->rej = -1;
    }
    return;
  }
  // ids outside [0, V) or a missing draft tensor cannot be verified: report
  // the sequence as unsupported without touching any row.
  bool bad = A.draft == nullptr;
  for (int k = 0; k < g; ++k) {
    const int id = A.draft_ids[(size_t)b * g + k];
    bad |= id < 0 || id >= A.V;
  }
  if (bad) {
    if (t == 0) {
      sq->rej = -1;
      A.accepted[b] = 0; A.next_tok[b] = -1; A.used[b] = 0;
      A.row_status[b] = CX_ROW_UNSUPPORTED;
    }
    return;
  }
  const double* ub = A.u + (size_t)b * (g + 1);
  int i = 0;
  for (; i < g; ++i) {
    const int tok = A.draft_ids[(size_t)b * g + i];
    const float* tr = trow(A, b, i);
    const float* dr = drow(A, b, i);
    float Mt, Mq;
    double St, Sq;
    merge_row(A, b * (g + 1) + i, T, Mt, St);
    merge_row(A, nt + b * g + i, T, Mq, Sq);
    const float zmt = Mt / T, zmq = Mq / T;
    const double et = exp((double)(tr[tok] / T) - (double)zmt);
    const double eq = exp((double)(dr[tok] / T) - (double)zmq);
    double thr = accept_threshold(et / St, eq / Sq);
    const double ui = ub[i];
    bool exact = false;
    // near the decision: recompute both normalisers exactly (fp64 over the rows)
    const double rel = 2.0 * (tol_norm(zmt) + tol_norm(zmq));
    const double tol = rel * (thr == thr ? thr : 1.0) + 1e-300;
    const bool q_floor_near = fabs(eq / Sq - 1e-12) <= rel * 1e-12;
    if (St == St && Sq == Sq && (fabs(ui - thr) <= tol || q_floor_near)) {
      St = exact_row_sum(tr, A.V, T, zmt, red_d);
      Sq = exact_row_sum(dr, A.V, T, zmq, red_d);
      thr = accept_threshold(et / St, eq / Sq);
      exact = true;
    }
    if (ui < thr) continue;
    if (t == 0) {
      sq->rej = i; sq->Mt = Mt; sq->Mq = Mq; sq->St = St; sq->Sq = Sq; sq->exact = exact;
    }
    break;
  }
  if (t == 0) {
    A.accepted[b] = i;
    if (i == g) {                                     // speculative.py:168-171
      sq->rej = -1;
      A.next_tok[b] = -1;
      A.used[b] = g;
      A.row_status[b] = CX_ROW_OK;
    } else {
      A.used[b] = i + 2;                              // tests 0..i, then the residual draw
    }
  }
}

// Residual weight of element e at position (b, rej): max(p - q, 0) in fp64.
__device__ __forceinline__ double resid(float xt, float xq, float T, float zmt, float zmq,
                                        double invSt, double invSq) {
  double p = exp((double)(xt / T) - (double)zmt) * invSt;
  double q = exp((double)(xq / T) - (double)zmq) * invSq;
  double d = p - q;
  return d > 0.0 ? d : 0.0;
}

// ------------------------------------------------------------ 3. residual chunk masses
__global__ __launch_bounds__(WG) void verify_residual(VerifyArgs A) {
  __shared__ double red_d[2 * NWAVE + 4];
  const int b = blockIdx.x / A.nchunk, ch = blockIdx.x % A.nchunk;
  const float T = A.temperature[b];
  const SeqState* sq = A.seq + b;
  if (T == 0.0f || sq->rej < 0) return;
  const int r = sq->rej;
  const float* tr = trow(A, b, r);
  const float* dr = drow(A, b, r);
  const float zmt = sq->Mt / T, zmq = sq->Mq / T;
  const double it = 1.0 / sq->St, iq = 1.0 / sq->Sq;
  const int lo = ch * VCHUNK, hi = min(A.V, lo + VCHUNK);
  double s = 0.0;
  for (int e = lo + threadIdx.x; e < hi; e += WG) s += resid(tr[e], dr[e], T, zmt, zmq, it, iq);
  s = block_sum(s, red_d);
  if (threadIdx.x == 0) A.rmass[(size_t)b * A.nchunk + ch] = s;
}

// Exact residual draw over the whole row pair (single workgroup, fp64):
// numpy's choice(V, p=r/R) with r = max(p - q, 0) (speculative.py:161-166).
// Returns -1 when R <= 0 (the caller falls back to argmax(row)).
__device__ inline int exact_residual_draw(const float* tr, const float* dr, int V, float T,
                                          float zmt, float zmq, double St, double Sq, double u,
                                          double* red_d, int* red_i, double* tsum) {
  const int t = threadIdx.x;
  const int per = (V + WG - 1) / WG;
  const int e0 = t * per, e1 = min(V, e0 + per);
  const double it = 1.0 / St, iq = 1.0 / Sq;
  double s = 0.0;
  for (int e = e0; e < e1; ++e) s += resid(tr[e], dr[e], T, zmt, zmq, it, iq);
  tsum[t] = s;
  const double R = block_sum(s, red_d);
  if (!(R > 0.0)) return -1;
  block_scan(tsum, WG, red_d);            // inclusive prefix of the per-thread sums
  const double prev = t > 0 ? tsum[t - 1] : 0.0;
  int found = INT_MAX;
  if ((prev / R) / (tsum[WG - 1] / R) <= u && (tsum[t] / R) / (tsum[WG - 1] / R) > u) {
    double run = prev;
    for (int e = e0; e < e1; ++e) {
      run += resid(tr[e], dr[e], T, zmt, zmq, it, iq);
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

// ------------------------------------------------------------ 4. draw
__global__ __launch_bounds__(WG) void verify_draw(VerifyArgs A) {
  __shared__ double red_d[2 * NWAVE + 4];
  __shared__ int red_i[2 * NWAVE + 4];
  __shared__ double tsum[WG];
  __shared__ double cm[64];
  __shared__ int s_ch;
  const int b = blockIdx.x;
  const int t = threadIdx.x;
  const float T = A.temperature[b];
  SeqState* sq = A.seq + b;
  if (T == 0.0f || sq->rej < 0) return;
  const int r = sq->rej;
  const int g = A.gamma;
  const float* tr = trow(A, b, r);
  const float* dr = drow(A, b, r);
  const float zmt = sq->Mt / T, zmq = sq->Mq / T;
  const double u = A.u[(size_t)b * (g + 1) + r + 1];
  const double* rm = A.rmass + (size_t)b * A.nchunk;
  int tok = -1;
  int flag = 0;
  double R = 0.0;
  for (int k = 0; k < A.nchunk; ++k) R += rm[k];
  // error of the fp32-term normalisers carries into every p and q
  const double err = sq->exact ? 1e-12 : 2.0 * (tol_norm(zmt) + tol_norm(zmq));
  bool ok = R > err;
  if (ok) {
    if (t == 0) {
      double run = 0.0;
      int k = 0;
      for (; k < A.nchunk - 1; ++k) {
        if ((run + rm[k]) / R > u) break;
        run += rm[k];
      }
      s_ch = k;
      cm[0] = run;
      // distance of u*R to the chunk's edges, relative to R
      double lo_gap = u - run / R, hi_gap = (run + rm[k]) / R - u;
      cm[1] = fmin(k > 0 ? lo_gap : 1.0, k < A.nchunk - 1 ? hi_gap : 1.0);
    }
    __syncthreads();
    const int k = s_ch;
    const double before = cm[0];
    if (cm[1] <= err / R) ok = false;
    if (ok) {
      const int lo = k * VCHUNK, hi = min(A.V, lo + VCHUNK);
      const int per = (hi - lo + WG - 1) / WG;
      const int e0 = lo + t * per, e1 = min(hi, e0 + per);
      const double it = 1.0 / sq->St, iq = 1.0 / sq->Sq;
      double s = 0.0;
      for (int e = e0; e < e1; ++e) s += resid(tr[e], dr[e], T, zmt, zmq, it, iq);
      tsum[t] = s;
      __syncthreads();
      block_scan(tsum, WG, red_d);
      const double prev = before + (t > 0 ? tsum[t - 1] : 0.0);
      int found = INT_MAX;
      double margin = 1.0;
      if (prev / R <= u && (before + tsum[t]) / R > u) {
        double run = prev;
        for (int e = e0; e < e1; ++e) {
          double nx = run + resid(tr[e], dr[e], T, zmt, zmq, it, iq);
          if (nx / R > u) { found = e; margin = fmin(u - run / R, nx / R - u); break; }
          run = nx;
        }
      }
      found = block_min(found, red_i, INT_MAX);
      margin = block_min(margin, red_d, 1.0);
      if (found == INT_MAX || margin <= err / R) ok = false;
      else tok = found;
    }
  }
  if (!ok) {                                            // exact fp64 redo
    double St = exact_row_sum(tr, A.V, T, zmt, red_d);
    double Sq = exact_row_sum(dr, A.V, T, zmq, red_d);
    __syncthreads();
    tok = exact_residual_draw(tr, dr, A.V, T, zmt, zmq, St, Sq, u, red_d, red_i, tsum);
    flag = CX_ROW_FLAG_EXACT;
    if (tok < 0) {                                      // R <= 0: argmax(row), no draw
      tok = row_argmax(tr, A.V, red_d, red_i);
      if (t == 0) A.used[b] = r + 1;
    }
  }
  if (t == 0) {
    A.next_tok[b] = tok;
    A.row_status[b] = CX_ROW_OK | flag | (sq->exact ? CX_ROW_FLAG_EXACT : 0);
  }
}

int launch_verify(const VerifyArgs& A, bool any_stochastic, hipStream_t s) {
  const int nt = A.B * (A.gamma + 1);
  const int nrows = nt + (any_stochastic ? A.B * A.gamma : 0);
  timed_launch(CX_KERNEL_VERIFY_STATS, verify_stats, dim3(nrows * A.nchunk), dim3(WG), 0, s, A);
  timed_launch(CX_KERNEL_VERIFY_REST, verify_decide, dim3(A.B), dim3(WG), 0, s, A);
  if (any_stochastic) {
    timed_launch(CX_KERNEL_VERIFY_REST, verify_residual, dim3(A.B * A.nchunk), dim3(WG), 0, s, A);
    timed_launch(CX_KERNEL_VERIFY_REST, verify_draw, dim3(A.B), dim3(WG), 0, s, A);
  }
  return (int)hipGetLastError();
}

}  // namespace cx
