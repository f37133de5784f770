// cx_finish.hpp -- per-row finisher of the fused sampler.
//
// Runs in the last workgroup of a row.  Merges the slices' statistics,
// gathers the exact region into LDS, sorts it, and applies the reference's
// filters on fp64 probabilities:
//   top-k   sampler.py:76-79  keep every value >= the k-th largest
//   top-p   sampler.py:81-89  shortest prefix (value desc, id asc) with cum >= p
//   min-p   sampler.py:91-93  keep P >= min_p * max P
// then normalises (:123-126) and draws by inverse CDF in token-id order
// (:127, Generator.choice == searchsorted(cumsum/last, u, 'right')).
#pragma once
#include "cx_device.hpp"
#include "cx_internal.hpp"

namespace cx {

__device__ inline void write_row_result(const SampleArgs& A, int row, int status, int token) {
  if (threadIdx.x == 0) {
    A.out_id[row] = token;
    A.row_status[row] = status;
  }
}

// out_probs for rows without a distribution (greedy, argmax fallback): one-hot.
__device__ inline void write_one_hot(const SampleArgs& A, int row, int token) {
  if (!A.out_probs) return;
  float* p = A.out_probs + (size_t)row * A.V;
  for (int i = threadIdx.x; i < A.V; i += WG) p[i] = (i == token) ? 1.0f : 0.0f;
}

// The target-th largest key among the row's candidates with key >= thr
// (MSB-first radix select, 8-bit digits, counts in an LDS histogram).
__device__ inline uint64_t kth_candidate_key(const SampleArgs& A, int row, uint64_t thr,
                                             int target, uint32_t* hist, uint64_t* bcast) {
  const int nsp = A.nsplit;
  const SplitStats* st = A.stats + (size_t)row * nsp;
  uint64_t prefix = 0, pmask = 0;
  int above = 0;
  for (int shift = 56; shift >= 0; shift -= 8) {
    for (int d = threadIdx.x; d < 256; d += WG) hist[d] = 0u;
    __syncthreads();
    for (int s = 0; s < nsp; ++s) {
      const Cand* cs = A.cands + ((size_t)row * nsp + s) * CAPS;
      const int n = st[s].ncand;
      for (int e = threadIdx.x; e < n; e += WG) {
        uint64_t k = cs[e].key;
        if (k >= thr && (k & pmask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
      }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int d = 255;
      for (; d > 0; --d) {
        if (above + (int)hist[d] >= target) break;
        above += (int)hist[d];
      }
      bcast[0] = prefix | ((uint64_t)d << shift);
      bcast[1] = (uint64_t)above;
    }
    __syncthreads();
    prefix = bcast[0];
    above = (int)bcast[1];
    pmask |= 255ull << shift;
    __syncthreads();
  }
  return prefix;
}

// Outcomes of finish_row_fast.
constexpr int FIN_PENDING = 0;   // the exact multi-pass path must take the row
constexpr int FIN_DONE = 1;      // decided and written
constexpr int FIN_REFINE = 2;    // region complete, but a top-p cut lies within the
                                 // normaliser's error bound: decide again with an
                                 // exact fp64 normaliser

// Finish a row from its region (at most CAP entries, CAP / WG per thread).
// S_exact > 0 is the exact fp64 normaliser sum exp((x - M) / T) over the
// row, replacing the slices' streamed sums; the top-p cut is then taken as
// it falls.  Nothing is written unless the outcome is FIN_DONE.
template <int CAP>
__device__ inline int finish_row_fast(const SampleArgs& A, int row, const cx_row_params& P,
                                      unsigned char* dyn, double* red_d, int* red_i,
                                      double S_exact = 0.0) {
  constexpr int R = CAP / WG;
  __shared__ int f_n;
  __shared__ int f_j;
  const int t = threadIdx.x;
  const int nsp = A.nsplit;
  const SplitStats* st = A.stats + (size_t)row * nsp;
  int flags = 0;
  for (int s = 0; s < nsp; ++s) flags |= st[s].flags;

  if (flags & SF_UNSUPPORTED) {
    write_row_result(A, row, CX_ROW_UNSUPPORTED, -1);
    return FIN_DONE;
  }
  if (P.temperature == 0.0) {                      // sampler.py:114-115
    double bv = -__builtin_inf();
    int bi = INT_MAX, ni = INT_MAX;
    for (int s = 0; s < nsp; ++s) {
      if (st[s].best_i != INT_MAX) argmax_merge(bv, bi, st[s].best_v, st[s].best_i);
      ni = min(ni, st[s].nan_i);
    }
    int tok = ni != INT_MAX ? ni : (bi == INT_MAX ? 0 : bi);
    write_row_result(A, row, CX_ROW_GREEDY, tok);
    write_one_hot(A, row, tok);
    return FIN_DONE;
  }

  const double invT = 1.0 / P.temperature;
  double M = -__builtin_inf();
  bool mnan = false;
  for (int s = 0; s < nsp; ++s) {
    mnan |= st[s].m != st[s].m;
    M = st[s].m > M ? st[s].m : M;
  }
  double S = 0.0;
  uint32_t tau = 1u;
  double tol = TOL_S;
  for (int s = 0; s < nsp; ++s) {
    if (st[s].s != 0.0) S += st[s].s * exp((st[s].m - M) * invT);
    tau = max(tau, st[s].tau);
    tol = st[s].tol > tol ? st[s].tol : tol;
  }
  const bool exact = S_exact > 0.0;
  if (exact) S = S_exact;
  // Degenerate rows (NaN / +inf / all -inf), tie floods, typical-p and a
  // possible P**(1/T) underflow (ln V / T > 740) go to the multi-pass kernel.
  if (mnan || !(S > 0.0) || !(S < __builtin_inf()) ||
      (flags & (SF_OVERFLOW | (exact ? 0 : SF_INEXACT))) || P.typical_p < 1.0 ||
      A.logV * invT > 740.0) {
    return FIN_PENDING;
  }
  bool region_incomplete_after_shrink = false;
  const bool region_all_pre = tau <= 1u;
  const uint64_t thr64 = region_all_pre ? 0ull : d2key((double)key2f(tau));

  uint64_t* skey = (uint64_t*)dyn;
  int32_t* sidx = (int32_t*)(dyn + CAP * 8);
  int32_t* saux = sidx + CAP;
  double* sv = (double*)(dyn + CAP * 16);
  double* sc = sv + CAP;

  if (t == 0) f_n = 0;
  __syncthreads();
  for (int s = 0; s < nsp; ++s) {
    const Cand* cs = A.cands + ((size_t)row * nsp + s) * CAPS;
    const int n = st[s].ncand;
    for (int e = t; e < n; e += WG) {
      Cand c = cs[e];
      if (c.key >= thr64) {
        int pos = atomicAdd(&f_n, 1);
        if (pos < CAP) { skey[pos] = c.key; sidx[pos] = c.idx; saux[pos] = 0; }
      }
    }
  }
  __syncthreads();
  int E = f_n;
  if (E > CAP) {
    // Shrink the region to the CAP largest candidates (strictly above the
    // CAP-th key when ties would overflow): it still holds every element of
    // the row above its new threshold.
    __shared__ uint64_t bc[2];
    uint64_t kk = kth_candidate_key(A, row, thr64, CAP, (uint32_t*)sv, bc);
    uint64_t thr2 = kk + 1;
    if (t == 0) f_n = 0;
    __syncthreads();
    for (int s = 0; s < nsp; ++s) {
      const Cand* cs = A.cands + ((size_t)row * nsp + s) * CAPS;
      const int n = st[s].ncand;
      for (int e = t; e < n; e += WG) {
        Cand c = cs[e];
        if (c.key >= thr2) {
          int pos = atomicAdd(&f_n, 1);
          if (pos < CAP) { skey[pos] = c.key; sidx[pos] = c.idx; saux[pos] = 0; }
        }
      }
    }
    __syncthreads();
    E = f_n;
    region_incomplete_after_shrink = true;
  }
  if (E > CAP || E == 0) return FIN_PENDING;
  block_sort<R>(skey, sidx, saux, E);

  const bool region_all = region_all_pre && !region_incomplete_after_shrink;
  // ---- top-k: every value >= the k-th largest (ties kept)
  int nk = E;
  bool complete = region_all;
  if (P.top_k > 0) {
    if (P.top_k <= E) {
      const uint64_t thr = skey[P.top_k - 1];
      if (t == 0) f_j = E;
      __syncthreads();
      for (int j = P.top_k + t; j < E; j += WG)
        if (skey[j] < thr) atomicMin(&f_j, j);
      __syncthreads();
      nk = f_j;
      complete = true;
    } else if (!region_all) {
      return FIN_PENDING;
    }
  }
  // ---- probabilities of the kept prefix
  for (int j = t; j < nk; j += WG) sv[j] = exp((key2d(skey[j]) - M) * invT) / S;
  __syncthreads();
  // ---- top-p on the unrenormalised vector
  if (P.top_p < 1.0) {
    for (int j = t; j < nk; j += WG) sc[j] = sv[j];
    __syncthreads();
    block_scan<R>(sc, nk, red_d);
    if (t == 0) f_j = nk;
    __syncthreads();
    for (int j = t; j < nk; j += WG)
      if (sc[j] >= P.top_p) atomicMin(&f_j, j);
    __syncthreads();
    const int m = f_j;
    bool near;
    if (m < nk) {
      near = fabs(sc[m] - P.top_p) <= tol * sc[m] ||
             (m > 0 && fabs(sc[m - 1] - P.top_p) <= tol * sc[m - 1]);
      nk = m + 1;
      complete = true;
    } else {
      if (!complete) return FIN_PENDING;
      near = fabs(sc[nk - 1] - P.top_p) <= tol * sc[nk - 1];
    }
    if (near && !exact) return FIN_REFINE;
  }
  // ---- min-p relative to the top probability
  if (P.min_p > 0.0) {
    const double floor_p = P.min_p * sv[0];
    if (t == 0) f_j = nk;
    __syncthreads();
    for (int j = t; j < nk; j += WG)
      if (sv[j] < floor_p) atomicMin(&f_j, j);
    __syncthreads();
    if (f_j < nk) { nk = f_j; complete = true; }
    else if (!complete) return FIN_PENDING;
  }
  if (!complete) return FIN_PENDING;

  // ---- normalise and draw in token-id order
  double z = 0.0;
  for (int j = t; j < nk; j += WG) z += sv[j];
  const double Z = block_sum(z, red_d);
  for (int j = t; j < nk; j += WG) { skey[j] = ~(uint64_t)(uint32_t)sidx[j]; saux[j] = j; }
  __syncthreads();
  block_sort<R>(skey, sidx, saux, nk);
  for (int j = t; j < nk; j += WG) sc[j] = sv[saux[j]] / Z;
  __syncthreads();
  block_scan<R>(sc, nk, red_d);
  const double last = sc[nk - 1];
  const double u = A.u[row];
  if (t == 0) f_j = nk - 1;
  __syncthreads();
  for (int j = t; j < nk; j += WG)
    if (sc[j] / last > u) atomicMin(&f_j, j);
  __syncthreads();
  const int tok = sidx[f_j];
  if (A.out_probs) {
    float* p = A.out_probs + (size_t)row * A.V;
    for (int i = t; i < A.V; i += WG) p[i] = 0.0f;
    __syncthreads();
    for (int j = t; j < nk; j += WG) p[sidx[j]] = (float)(sv[saux[j]] / Z);
  }
  write_row_result(A, row, exact ? (CX_ROW_OK | CX_ROW_FLAG_EXACT) : CX_ROW_OK, tok);
  return FIN_DONE;
}

// Finish a row from its slices' statistics and regions; a row this cannot
// decide is marked for the exact-normaliser refinement or, failing that, for
// the exact multi-pass kernel.
template <int CAP>
__device__ inline void finish_row(const SampleArgs& A, int row, const cx_row_params& P,
                                  unsigned char* dyn, double* red_d, int* red_i) {
  const int r = finish_row_fast<CAP>(A, row, P, dyn, red_d, red_i);
  if (r != FIN_DONE) write_row_result(A, row, r == FIN_REFINE ? ROW_REFINE : ROW_PENDING, -1);
}

}  // namespace cx
