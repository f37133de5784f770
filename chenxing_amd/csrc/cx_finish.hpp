// cx_finish.hpp -- region finisher of the fused sampler.
//
// Runs in slow_kernel, one workgroup per row, after the fused kernel has
// written the row's statistics and region (one record per slice).  Merges
// the slices' statistics, gathers the exact region into LDS, and applies
// the reference's filters on fp64 probabilities, with bucketed cuts (a
// sort of the whole region only when a cut's bucket overflows):
//   top-k   sampler.py:76-79  keep every value >= the k-th largest
//   top-p   sampler.py:81-89  shortest prefix (value desc, id asc) with cum >= p;
//                             the cut value's group keeps its survivors spread
//                             over its ids (spread_kept, cx_device.hpp)
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

// ------------------------------------------------------------ bucketed cuts
// The finisher's cuts (the k-th largest value, the top-p prefix, the draw in
// token-id order) without sorting the region: entries go to NBK buckets that
// are monotone in the order (linear in the value, or in the token id); the
// buckets' weights are summed as fixed-point integers with LDS atomics
// (exact, so independent of the order of the additions), scanned, and only
// the bucket that holds the cut is gathered, sorted by one wave and scanned.
// A slot, counted from *counter, for each lane of the wave with p set, in
// lane order: one LDS atomic per wave instead of one per element.  Every
// lane of the wave calls it.
__device__ __forceinline__ int wave_append_slot(bool p, int* counter) {
  const uint64_t b = ballot(p);
  int base = 0;
  if (b) {
    const int first = __builtin_ctzll(b);
    if (lane_id() == first) base = atomicAdd(counter, __popcll(b));
    base = __shfl(base, first);
  }
  return base + lanes_below(b);
}

constexpr int NBK = WG;            // buckets: one per thread in the scan
constexpr int GBK = 64;            // a gathered bucket: one entry per lane
constexpr double FX_MASS = 1152921504606846976.0;   // 2^60: masses sum to <= ~1

struct PrefixCut {
  int found;        // the running weight reaches the target inside the entries
  int overflow;     // the cut's bucket holds more than GBK entries
  int bucket, pos, n;
  double cum;       // running weight up to and including the cut entry
  double prev;      // running weight before it
  double total;     // weight of all eligible entries
  uint64_t key;     // the cut entry's order key and token id
  int32_t idx;
  int g0, g1;       // the cut key's entries: positions [g0, g1) of the sorted bucket
};

// The first eligible entry, in the order (bucket_of ascending, then key
// descending, then id ascending), at which the running weight reaches
// (>= target) or, if strict, passes (> target) the target; a relative
// target is a fraction of the total.  Weights are scaled by `scale` into
// integers (1 for counts).  On return `out` (shared) holds the cut and, with
// `found`, ga[0 .. n) the region indices of the cut bucket's entries in
// order.  All threads; uniform result.  The caller hands over bm zeroed and
// ctr = {0, INT_MAX} (the gather count and the cut bucket), both written
// before a barrier that precedes the call (one barrier less per cut).
template <typename BucketOf, typename KeyOf, typename Weight, typename Elig>
__device__ inline void prefix_cut(int E, const int32_t* sidx, BucketOf bucket_of, KeyOf key_of,
                                  Weight weight, Elig elig, double scale, double target,
                                  bool relative, bool strict, unsigned long long* bm, int* ctr,
                                  uint64_t* gk, int32_t* gi, int32_t* ga, double* red_d,
                                  PrefixCut& out) {
  int& pc_n = ctr[0];
  int& pc_bc = ctr[1];
  const int t = threadIdx.x;
  unsigned long long* red_u = (unsigned long long*)red_d;
  for (int j = t; j < E; j += WG)
    if (elig(j)) atomicAdd(&bm[bucket_of(j)], (unsigned long long)(weight(j) * scale));
  __syncthreads();
  // the cut bucket, by wave 0 alone (lane l scans buckets 16 l .. 16 l + 15
  // and a DPP scan carries the lanes' totals): the first bucket whose running
  // weight reaches the target.  The running weight is monotone, so that
  // bucket is nonempty and the one whose weight before it does not reach
  // the target.
  if (wave_id() == 0) {
    constexpr int PB = NBK / 64;
    const int l = lane_id();
    unsigned long long bw[PB];
    unsigned long long lsum = 0ull;
#pragma unroll
    for (int i = 0; i < PB; ++i) {
      bw[i] = bm[l * PB + i];
      lsum += bw[i];
    }
    const unsigned long long incl = wave_scan_dpp(lsum);
    const unsigned long long all = lane_read((uint64_t)incl, 63);
    const double total = (double)all / scale;
    const double tgt = relative ? target * total : target;
    unsigned long long run = incl - lsum;              // weight before the lane's buckets
    int first = INT_MAX;
    unsigned long long before = 0ull;
#pragma unroll
    for (int i = 0; i < PB; ++i) {
      const unsigned long long bi = run;
      run += bw[i];
      const double be = (double)run / scale;
      if (first == INT_MAX && bw[i] != 0ull && (strict ? be > tgt : be >= tgt)) {
        first = l * PB + i;
        before = bi;
      }
    }
    const uint64_t hb = ballot(first != INT_MAX);
    if (hb) {
      const int fl = __builtin_ctzll(hb);
      if (l == fl) { pc_bc = first; red_u[2 * NWAVE + 1] = before; }
    }
    if (l == 0) red_d[2 * NWAVE + 2] = total;
  }
  __syncthreads();
  const double total = red_d[2 * NWAVE + 2];
  const double tgt = relative ? target * total : target;
  const int bc = pc_bc;
  if (bc == INT_MAX) {
    if (t == 0) { out.found = 0; out.overflow = 0; out.total = total; }
    __syncthreads();
    return;
  }
  // gather the cut bucket
  for (int j0 = 0; j0 < E; j0 += WG) {
    const int j = j0 + t;
    const bool p = j < E && elig(j) && bucket_of(j) == bc;
    const int q = wave_append_slot(p, &pc_n);
    if (p && q < GBK) { gk[q] = key_of(j); gi[q] = sidx[j]; ga[q] = j; }
  }
  __syncthreads();
  const int n = pc_n;
  if (n > GBK) {
    if (t == 0) { out.found = 0; out.overflow = 1; out.total = total; }
    __syncthreads();
    return;
  }
  if (wave_id() == 0) {
    const int l = lane_id();
    // the bucket's n entries in rec_before order: each lane's rank among
    // them (n is usually a few, so n broadcast reads beat a 64-wide
    // sorting network), then each entry written at its rank and read back
    Rec r[1];
    r[0].key = l < n ? gk[l] : 0ull;
    r[0].idx = l < n ? gi[l] : INT_MAX;
    r[0].aux = l < n ? ga[l] : -1;
    int rank = 0;
    for (int j = 0; j < n; ++j) {
      const uint64_t kj = gk[j];
      const int32_t ij = gi[j];
      rank += (kj > r[0].key || (kj == r[0].key && ij < r[0].idx)) ? 1 : 0;
    }
    // every lane's reads above precede the writes (one wave's LDS
    // operations complete in order; the barriers keep the compiler's order)
    __builtin_amdgcn_wave_barrier();
    if (l < n) { gk[rank] = r[0].key; gi[rank] = r[0].idx; ga[rank] = r[0].aux; }
    __builtin_amdgcn_wave_barrier();
    if (l < n) { r[0].key = gk[l]; r[0].idx = gi[l]; r[0].aux = ga[l]; }
    const double w = l < n ? weight(r[0].aux) : 0.0;
    const double incl = wave_scan_dpp(w);
    if (l < n) ga[l] = r[0].aux;
    const unsigned long long bb = red_u[2 * NWAVE + 1];
    const double based = (double)bb / scale;
    const double cum = based + incl, prv = based + (incl - w);
    const uint64_t hb = ballot(l < n && (strict ? cum > tgt : cum >= tgt));
    const int pos = hb ? __builtin_ctzll(hb) : n - 1;
    // equal keys land in one bucket: the cut key's whole group is here,
    // contiguous and in ascending ids
    const uint64_t kpos = lane_read(r[0].key, pos);     // (read by every lane)
    const uint64_t gb = ballot(l < n && r[0].key == kpos);
    if (l == pos) {
      out.found = 1; out.overflow = 0; out.bucket = bc; out.pos = pos; out.n = n;
      out.cum = cum; out.prev = prv; out.total = total; out.key = r[0].key; out.idx = r[0].idx;
      out.g0 = __builtin_ctzll(gb);
      out.g1 = 64 - __builtin_clzll(gb);
    }
  }
  __syncthreads();
}

// Outcomes of finish_row_fast.
constexpr int FIN_PENDING = 0;   // the exact multi-pass path must take the row
constexpr int FIN_DONE = 1;      // decided and written
constexpr int FIN_REFINE = 2;    // region complete, but a top-p cut lies within the
                                 // normaliser's error bound: decide again with an
                                 // exact fp64 normaliser

constexpr int FIN_SORTED = 3;    // (finish_bucketed) a cut bucket overflowed: sort instead

// The filters and the draw of finish_row_fast over the region held in LDS
// (skey, sidx: E entries), with bucketed cuts.  kf, sv and sc are work
// space (kf: kept flags, sv: the entries' probabilities, sc: buckets and the
// gathered bucket).  Returns FIN_SORTED, with nothing written, when a cut's
// bucket holds more than GBK entries (a flood of near-equal values).
__device__ inline int finish_bucketed(const SampleArgs& A, int row, const cx_row_params& P,
                                      const uint64_t* skey, const int32_t* sidx, int32_t* kf,
                                      double* sv, double* sc, int E, bool region_all, double M,
                                      double invT, double S, double tol, bool exact,
                                      double* red_d, int* red_i, const double* tab,
                                      const uint64_t* ext, int* s_ctr) {
  __shared__ PrefixCut pc;
  const int t = threadIdx.x;
  // the gathered bucket, then the buckets of the three cuts (top-k, top-p,
  // draw); the caller cleared the buckets and s_ctr (per cut: gather count,
  // cut bucket) and posted the waves' extremes (ext) before its barrier
  uint64_t* gk = (uint64_t*)sc;
  int32_t* gi = (int32_t*)(gk + GBK);
  int32_t* ga = gi + GBK;
  unsigned long long* bmk = (unsigned long long*)(sc + 2 * GBK);
  unsigned long long* bmp = bmk + NBK;
  unsigned long long* bmd = bmp + NBK;
  // each thread's entries (j = t + i WG, the mapping every pass below
  // keeps): their probabilities and kept flags, read only by this thread
  // until a barrier
  for (int j = t; j < E; j += WG) {
    sv[j] = exp64_neg((key2d(skey[j]) - M) * invT, tab) / S;   // within 1 ulp, as exp
    kf[j] = 1;
  }
  uint64_t kmax = 0ull, kmin = ~0ull;
#pragma unroll
  for (int w = 0; w < NWAVE; ++w) {
    kmax = ext[w] > kmax ? ext[w] : kmax;
    kmin = ext[NWAVE + w] < kmin ? ext[NWAVE + w] : kmin;
  }
  // value buckets: linear in the value, bucket 0 holding the largest
  const double vmax = key2d(kmax), vmin = key2d(kmin);
  double vs = vmax > vmin ? (double)(NBK - 1) / (vmax - vmin) : 0.0;
  if (!(vs < 1e300)) vs = 0.0;
  // (vmax - v) * vs >= 0, or NaN for -inf values when vs == 0: the last bucket
  auto vbucket = [&](int j) {
    const double x = (vmax - key2d(skey[j])) * vs;
    return x < (double)(NBK - 1) ? (int)x : NBK - 1;
  };
  auto vkey = [&](int j) { return skey[j]; };
  // token-id buckets, ascending ids (key ~id orders descending keys as ascending ids)
  auto ibucket = [&](int j) { return (int)(((long long)sidx[j] * NBK) / A.V); };
  auto ikey = [&](int j) { return ~(uint64_t)(uint32_t)sidx[j]; };
  auto one = [&](int) { return 1.0; };
  auto mass = [&](int j) { return sv[j]; };
  auto every = [&](int) { return true; };
  auto kept = [&](int j) { return kf[j] != 0; };

  bool complete = region_all;
  // ---- top-k: every value >= the k-th largest (ties kept)
  if (P.top_k > 0) {
    if (P.top_k <= E) {
      prefix_cut(E, sidx, vbucket, vkey, one, every, 1.0, (double)P.top_k, false, false, bmk,
                 s_ctr, gk, gi, ga, red_d, pc);
      if (pc.overflow || !pc.found) return FIN_SORTED;
      const uint64_t kth = pc.key;
      for (int j = t; j < E; j += WG) kf[j] = skey[j] >= kth;
      __syncthreads();
      complete = true;
    } else if (!region_all) {
      return FIN_PENDING;
    }
  }
  // ---- top-p on the unrenormalised vector: the shortest prefix in (value
  // desc, id asc) order whose running mass reaches top_p; of the cut
  // value's group, the survivors spread over its ids
  if (P.top_p < 1.0) {
    prefix_cut(E, sidx, vbucket, vkey, mass, kept, FX_MASS, P.top_p, false, false, bmp, s_ctr + 2,
               gk, gi, ga, red_d, pc);
    if (pc.overflow) return FIN_SORTED;
    bool near;
    if (pc.found) {
      const double cm = pc.cum, cp = pc.prev;
      near = fabs(cm - P.top_p) <= tol * cm || (cp > 0.0 && fabs(cp - P.top_p) <= tol * cp);
      const int bc = pc.bucket, pos = pc.pos, g0 = pc.g0, g1 = pc.g1, nb = pc.n;
      // entries past the cut bucket dropped; the cut bucket's own (gathered
      // in ga, a disjoint set) kept before the cut value and for its group's
      // survivors
      for (int j = t; j < E; j += WG)
        if (kf[j] && vbucket(j) > bc) kf[j] = 0;
      if (t < nb)
        kf[ga[t]] = t < g0 || (t < g1 && spread_keeps(t - g0, pos + 1 - g0, g1 - g0,
                                                      A.V <= TIE_NET));
      __syncthreads();
      complete = true;
    } else {
      if (!complete) return FIN_PENDING;
      near = fabs(pc.total - P.top_p) <= tol * pc.total;
    }
    if (near && !exact) return FIN_REFINE;
  }
  // ---- min-p relative to the top probability (the largest entry is kept)
  if (P.min_p > 0.0) {
    const double floor_p = P.min_p * (exp((vmax - M) * invT) / S);
    int below = 0;
    for (int j = t; j < E; j += WG)
      if (kf[j] && sv[j] < floor_p) { kf[j] = 0; below = 1; }
    below = block_max(below, red_i, 0);
    if (below) complete = true;
    else if (!complete) return FIN_PENDING;
  }
  if (!complete) return FIN_PENDING;

  // ---- normalise and draw in token-id order: the first id whose running
  // mass passes u times the kept total (Generator.choice)
  // (the draw's target is relative to the kept total: Z itself is needed
  // only for the probabilities written out)
  double z = 0.0;
  int lastk = -1;
  for (int j = t; j < E; j += WG)
    if (kf[j]) { z += sv[j]; lastk = max(lastk, sidx[j]); }
  const double Z = A.out_probs ? block_sum(z, red_d) : 0.0;
  prefix_cut(E, sidx, ibucket, ikey, mass, kept, FX_MASS, A.u[row], true, true, bmd, s_ctr + 4,
             gk, gi, ga, red_d, pc);
  if (pc.overflow) return FIN_SORTED;
  // u beyond the last step by rounding: the last kept id
  const int tok = pc.found ? pc.idx : block_max(lastk, red_i, -1);
  if (A.out_probs) {
    float* p = A.out_probs + (size_t)row * A.V;
    for (int i = t; i < A.V; i += WG) p[i] = 0.0f;
    __syncthreads();
    for (int j = t; j < E; j += WG)
      if (kf[j]) p[sidx[j]] = (float)(sv[j] / Z);
  }
  write_row_result(A, row, exact ? (CX_ROW_OK | CX_ROW_FLAG_EXACT) : CX_ROW_OK, tok);
  return FIN_DONE;
}

// Finish a row from its region (at most CAP entries, CAP / WG per thread).
// S_exact > 0 is the exact fp64 normaliser sum exp((x - M) / T) over the
// row, replacing the slices' streamed sums; so is the sum of the slices'
// own exact fp64 sums when every slice recorded one (SF_EXACT).  With an
// exact normaliser the top-p cut is taken as it falls.  Nothing is written
// unless the outcome is FIN_DONE.
template <int CAP>
__device__ inline int finish_row_fast(const SampleArgs& A, int row, const cx_row_params& P,
                                      unsigned char* dyn, double* red_d, int* red_i,
                                      double S_exact = 0.0) {
  constexpr int R = CAP / WG;
  __shared__ int f_n;
  __shared__ int f_j;
  __shared__ int f_g[2];
  __shared__ SplitStats s_st[SLICE_CAP];
  __shared__ double f_tab[64];                       // EXP64_TAB
  const int t = threadIdx.x;
  const int nsp = A.nsplit;
  const SplitStats* gst = A.stats + (size_t)row * nsp;
  // Every load at once, before anything waits: the slices' records (one
  // thread each, into LDS) and the candidates where the usual layout puts
  // them, entry g of this thread's R at slice g / C, position g % C (C: a
  // slice's share of the capacity, at most one entry per thread, so a
  // single-slice row reads ahead 16 KB, not its whole 64 KB share).
  // Entries past a slice's count are read (the workspace holds CAPS per
  // slice) and dropped below.
  const int C = min(CAP / nsp, WG);
  if (t < nsp) s_st[t] = gst[t];
  if (t < 64) f_tab[t] = EXP64_TAB[t];
  // (a greedy row reads no candidates: its parameters come first)
  const bool stoch = P.temperature != 0.0;
  Cand c[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int g = r * WG + t;
    const int s = g / C;
    c[r].key = 0ull;
    c[r].idx = 0;
    if (stoch && s < nsp) c[r] = A.cands[((size_t)row * nsp + s) * CAPS + (g - s * C)];
  }
  if (t == 0) f_n = 0;
  __syncthreads();
  const SplitStats* st = s_st;
  // the row's scalars, lane s of row 0 taking slice s (every wave; one
  // exponential per lane, not one per slice in turn)
  const int ls = lane_id() & 15;
  const bool lin = ls < nsp;
  const SplitStats& me = st[lin ? ls : 0];
  const int flags = row0_reduce(lin ? me.flags : 0, OpOr());

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
  const uint32_t tau = row0_reduce(lin ? me.tau : 1u, OpMax());
  // Tie floods, typical-p and a possible P**(1/T) underflow (ln V / T >
  // 740) go to the multi-pass kernel; so do degenerate sums (below, once
  // wave 0 has taken them).
  if ((flags & SF_OVERFLOW) || P.typical_p < 1.0 || A.logV * invT > 740.0) return FIN_PENDING;
  // The row's maximum and normaliser: wave 0 alone, after its share of the
  // gather below (the others need only tau), lane s of row 0 taking slice s.
  __shared__ double f_sc[3];
  __shared__ int f_sf[2];
  auto row_sums = [&]() {
    const bool mnan = row0_reduce(lin && me.m != me.m ? 1 : 0, OpOr()) != 0;
    const double M = row0_reduce(lin && me.m == me.m ? me.m : -__builtin_inf(), OpMax());
    const double f = lin ? exp((me.m - M) * invT) : 0.0;     // slice s's sums to M
    double S = row0_reduce(lin && me.s != 0.0 ? me.s * f : 0.0, OpAdd());
    double tol = row0_reduce(lin && me.tol > TOL_S ? me.tol : TOL_S, OpMax());
    bool exact = S_exact > 0.0;
    if (exact) {
      S = S_exact;
    } else if (flags & SF_EXACT) {
      // the slices' fp64 sums (sliced top-p rows), when every slice has one:
      // S = sum over slices of sx_s exp((m_s - M) / T), exact when every
      // slice's is, else within the slices' bounds (split sums)
      const bool mx = lin && (me.flags & SF_EXACT);
      const bool allx = row0_reduce(lin && !mx ? 1 : 0, OpOr()) == 0;
      const double v = mx && me.sx != 0.0 ? me.sx * f : 0.0;
      const double Sx = row0_reduce(v, OpAdd());
      const double Bx = row0_reduce((double)(mx ? me.sxtol : 0.0f) * v, OpAdd());
      if (allx && Sx > 0.0 && Sx < __builtin_inf()) {
        S = Sx;
        if (Bx == 0.0) exact = true;
        else tol = Bx / Sx * 1.000001 + 1e-15;
      }
    }
    if (lane_id() == 0) {
      f_sc[0] = M; f_sc[1] = S; f_sc[2] = tol;
      f_sf[0] = mnan ? 1 : 0; f_sf[1] = exact ? 1 : 0;
    }
  };
  bool region_incomplete_after_shrink = false;
  const bool region_all_pre = tau <= 1u;
  const uint64_t thr64 = region_all_pre ? 0ull : d2key((double)key2f(tau));

  uint64_t* skey = (uint64_t*)dyn;
  int32_t* sidx = (int32_t*)(dyn + CAP * 8);
  int32_t* saux = sidx + CAP;
  double* sv = (double*)(dyn + CAP * 16);
  double* sc = sv + CAP;

  // the loaded candidates at or above the threshold into the region list
  // (the region's extremes taken on the way)
  uint64_t gmax = 0ull, gmin = ~0ull;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int g = r * WG + t;
    const int s = g / C;
    const bool p = s < nsp && g - s * C < st[s].ncand && c[r].key >= thr64;
    const int pos = wave_append_slot(p, &f_n);
    if (p && pos < CAP) { skey[pos] = c[r].key; sidx[pos] = c[r].idx; saux[pos] = 0; }
    if (p) { gmax = c[r].key > gmax ? c[r].key : gmax; gmin = c[r].key < gmin ? c[r].key : gmin; }
  }
  // a slice holding more than C candidates (a flood of ties past the
  // threshold): the rest, slice by slice
  for (int s = 0; s < nsp; ++s) {
    const int n = st[s].ncand;
    for (int e0 = C; e0 < n; e0 += WG) {
      const int e = e0 + t;
      Cand cc;
      cc.key = 0ull;
      cc.idx = 0;
      if (e < n) cc = A.cands[((size_t)row * nsp + s) * CAPS + e];
      const bool p = e < n && cc.key >= thr64;
      const int pos = wave_append_slot(p, &f_n);
      if (p && pos < CAP) { skey[pos] = cc.key; sidx[pos] = cc.idx; saux[pos] = 0; }
      if (p) { gmax = cc.key > gmax ? cc.key : gmax; gmin = cc.key < gmin ? cc.key : gmin; }
    }
  }
  if (wave_id() == 0) row_sums();
  // the waves' extremes and the cuts' cleared buckets, for finish_bucketed,
  // with this barrier (the buckets lie past the region and its values)
  __shared__ uint64_t f_ext[2 * NWAVE];
  __shared__ int f_ctr[6];
  {
    const uint64_t wx = wave_max(gmax), wn = wave_min(gmin);
    if (lane_id() == 0) { f_ext[wave_id()] = wx; f_ext[NWAVE + wave_id()] = wn; }
    static_assert(2 * GBK + 3 * NBK <= FIN_CAP, "finisher scratch");
    unsigned long long* bm0 = (unsigned long long*)(sc + 2 * GBK);
    bm0[t] = 0ull;
    bm0[NBK + t] = 0ull;
    bm0[2 * NBK + t] = 0ull;
    if (t < 6) f_ctr[t] = (t & 1) ? INT_MAX : 0;
  }
  __syncthreads();
  const double M = f_sc[0], S = f_sc[1], tol = f_sc[2];
  const bool exact = f_sf[1] != 0;
  // degenerate rows (NaN / +inf / all -inf) and inexact sums
  if (f_sf[0] || !(S > 0.0) || !(S < __builtin_inf()) || (!exact && (flags & SF_INEXACT)))
    return FIN_PENDING;
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
    gmax = 0ull;
    gmin = ~0ull;
    for (int s = 0; s < nsp; ++s) {
      const Cand* cs = A.cands + ((size_t)row * nsp + s) * CAPS;
      const int n = st[s].ncand;
      for (int e0 = 0; e0 < n; e0 += WG) {
        const int e = e0 + t;
        Cand c;
        c.key = 0ull;
        c.idx = 0;
        if (e < n) c = cs[e];
        const bool p = e < n && c.key >= thr2;
        const int pos = wave_append_slot(p, &f_n);
        if (p && pos < CAP) { skey[pos] = c.key; sidx[pos] = c.idx; saux[pos] = 0; }
        if (p) { gmax = c.key > gmax ? c.key : gmax; gmin = c.key < gmin ? c.key : gmin; }
      }
    }
    const uint64_t wx = wave_max(gmax), wn = wave_min(gmin);
    if (lane_id() == 0) { f_ext[wave_id()] = wx; f_ext[NWAVE + wave_id()] = wn; }
    __syncthreads();
    E = f_n;
    region_incomplete_after_shrink = true;
  }
  if (E > CAP || E == 0) return FIN_PENDING;
  const bool region_all = region_all_pre && !region_incomplete_after_shrink;
  {
    const int rb = finish_bucketed(A, row, P, skey, sidx, saux, sv, sc, E, region_all, M, invT, S,
                                   tol, exact, red_d, red_i, f_tab, f_ext, f_ctr);
    if (rb != FIN_SORTED) return rb;
  }
  // a cut's bucket overflowed (near-equal values): sort the region instead
  block_sort<R>(skey, sidx, saux, E);

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
      // the cut value's group, positions [g0, g1) (ascending ids), keeps
      // m + 1 - g0 members spread over its ids: move them to [g0, m] so the
      // kept entries stay a prefix (the group's probabilities are equal)
      if (t == 0) { f_g[0] = m; f_g[1] = m + 1; }
      __syncthreads();
      for (int j = t; j < nk; j += WG)
        if (skey[j] == skey[m]) { atomicMin(&f_g[0], j); atomicMax(&f_g[1], j + 1); }
      __syncthreads();
      const int g0 = f_g[0], g1 = f_g[1];
      if (g1 > m + 1) {
        const int jg = m + 1 - g0, ng = g1 - g0;
        uint64_t mk[R];
        int32_t mi[R];
#pragma unroll
        for (int q = 0; q < R; ++q) {
          const int j = g0 + q * WG + t;
          mk[q] = j < g1 ? skey[j] : 0ull;
          mi[q] = j < g1 ? sidx[j] : 0;
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < R; ++q) {
          const int r = q * WG + t;
          if (r < ng && spread_keeps(r, jg, ng, A.V <= TIE_NET)) {
            const int d = g0 + (int)spread_kept(r, jg, ng, A.V <= TIE_NET);
            skey[d] = mk[q];
            sidx[d] = mi[q];
          }
        }
        __syncthreads();
      }
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


}  // namespace cx
