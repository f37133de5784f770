// cx_slow.hpp -- exact multi-pass row path (reference chenxing/core/sampler.py:63-127).
//
// Finishes the rows the fused kernel cannot decide: degenerate rows (NaN,
// +inf, all -inf, P**(1/T) underflow), nuclei or top-k sets deeper than the
// fused kernel's region, tie floods, and typical-p.  (A top-p cut within the
// fused normaliser's error bound over a complete region is refined instead:
// exact_norm below, then the region finisher again.)  One workgroup per row;
// every quantity is fp64 and every selection is exact:
//
//   pass A   max / first argmax / first NaN / min of the penalised row
//   pass B   S = sum exp((x - M) / T)  (and the T = 1 sum for the underflow test)
//   select   top-k threshold (count select) and the top-p and typical-p cuts
//            (mass select): histogram passes over an exactly narrowing key
//            range, then the last bucket is gathered into LDS and sorted; a
//            cut inside a group of equal keys keeps j of its n members,
//            spread over their ids (spread_kept, cx_device.hpp)
//   draw     per-wave sums over contiguous id ranges, and a scan in id order
//            of the range that holds u (the passes after a cut visit the row
//            in these wave ranges, so a group member's rank is a running
//            count)
//
// slow_kernel (cx_slow.hip) runs it for the rows the fused path left
// pending.  Rows are re-read from memory for every pass; such rows are rare
// on the fused path's target workloads.
#pragma once
#include "cx_device.hpp"
#include "cx_sampler.h"
#include "cx_internal.hpp"

namespace cx {

constexpr int NB = 1024;             // histogram buckets per pass
constexpr int SCAP = 1024;           // gathered bucket capacity

__device__ __forceinline__ uint32_t s_hash_slot(int id, int ns_log2) {
  return ((uint32_t)id * 0x9E3779B1u) >> (32 - ns_log2);
}

struct SlowRow {
  const cx_row_params* P;
  const void* rowp;
  int bf16;
  int f64;
  bool direct;       // the row holds probabilities: value = mass, no penalties
  int V;
  bool pen;
  const uint32_t* bitmap;
  int nbw;
  const uint32_t* hkey;
  const float* hval;
  int ns_log2;
  double M, invT, S;
};

__device__ __forceinline__ double raw_at(const SlowRow& R, int i) {
  if (R.f64) return ((const double*)R.rowp)[i];
  return R.bf16 ? (double)__uint_as_float((uint32_t)((const uint16_t*)R.rowp)[i] << 16)
                : (double)((const float*)R.rowp)[i];
}

// Penalised fp64 value of element i whose raw value is x (sampler.py:65-72
// + presence/frequency).
__device__ inline double penalise_at(const SlowRow& R, int i, double x) {
  if (R.pen && ((R.bitmap[(i >> 5) & (R.nbw - 1)] >> (i & 31)) & 1u)) {
    const uint32_t mask = (1u << R.ns_log2) - 1;
    uint32_t s = s_hash_slot(i, R.ns_log2);
    for (;;) {
      uint32_t k = R.hkey[s];
      if (k == HEMPTY) break;
      if ((k >> 12) == (uint32_t)i) {
        const cx_row_params& p = *R.P;
        if (p.repetition_penalty != 1.0)
          x = x > 0.0 ? x / p.repetition_penalty : x * p.repetition_penalty;
        x = x - p.frequency_penalty * (double)(k & 0xFFFu);
        x = x - p.presence_penalty;
        break;
      }
      s = (s + 1) & mask;
    }
  }
  return x;
}

__device__ __forceinline__ double value_at(const SlowRow& R, int i) {
  return penalise_at(R, i, raw_at(R, i));
}

// sum over the row's ids [lo, hi) (the whole row by default) of
// exp((x - M) / T), x the penalised fp64 values (the reference's normaliser,
// sampler.py:119-123), in fp64, with the table-driven exp (within 1 ulp;
// every argument is <= 0).  Every thread keeps EXN independent loads in
// flight per step; the result is the same on every thread.
__device__ inline double exact_norm(const SlowRow& R, double M, double invT, double* red_d,
                                   int lo = 0, int hi = INT_MAX) {
  constexpr int EXN = 8;
  __shared__ double etab[64];
  load_exp64_tab(etab);
  const int t = threadIdx.x;
  hi = min(hi, R.V);
  double s = 0.0;
  for (int base = lo; base < hi; base += EXN * WG) {
    double x[EXN];
#pragma unroll
    for (int j = 0; j < EXN; ++j) {
      const int i = base + j * WG + t;
      x[j] = i < hi ? raw_at(R, i) : 0.0;
    }
#pragma unroll
    for (int j = 0; j < EXN; ++j) {
      const int i = base + j * WG + t;
      if (i < hi) s += exp64_neg((penalise_at(R, i, x[j]) - M) * invT, etab);
    }
  }
  return block_sum(s, red_d);
}

__device__ __forceinline__ double mass_of(const SlowRow& R, double v) {
  return R.direct ? v : exp((v - R.M) * R.invT) / R.S;
}

// Boundary of a prefix in (key desc, idx asc) order over the eligible
// elements: keys above k are inside, keys below outside; of the n eligible
// elements whose key equals k, j are inside, spread over their ids (on rows
// of at most TIE_NET ids, its lowest ids) -- the one of rank r (members with
// a lower id before it) is inside iff spread_keeps(r, j, n) (cx_device.hpp).  j >= n: the whole group is inside
// (top-k keeps its ties, and a cut that ends a group splits nothing).
struct Cut {
  uint64_t k;
  int n, j;
  bool net;          // a row of at most TIE_NET ids: the lowest ids survive
};
__device__ __forceinline__ Cut cut_at(uint64_t k) {
  Cut c;
  c.k = k;
  c.n = 0;
  c.j = 0;
  c.net = false;
  return c;
}
__device__ __forceinline__ bool cut_split(const Cut& c) { return c.j < c.n; }
__device__ __forceinline__ bool inside(const Cut& c, uint64_t key, int rank) {
  return key > c.k || (key == c.k && (c.j >= c.n || spread_keeps(rank, c.j, c.n, c.net)));
}

struct Filters {
  Cut rank;          // top-k / top-p prefix (value order)
  double floor_p;    // min-p floor on P (0 = off)
  bool typ;          // typical-p cut active
  double H;          // entropy for the typical order
  Cut tcut;          // typical prefix in (-|log P + H| desc, idx asc) order
  bool want_tk;      // the visits compute the typical order key
  int* b1;           // [NWAVE] rank's group members before each wave range
  int* b2;           // [NWAVE] tcut's group members before each wave range
};

__device__ __forceinline__ uint64_t typ_key(double P, double H) {
  double lp = log(P > 1e-38 ? P : 1e-38);
  return d2key(-fabs(lp + H));
}

struct SlowLds {
  uint32_t* cnt;     // [NB]
  double* mass;      // [NB]
  uint64_t* gk;      // [SCAP]
  int32_t* gi;       // [SCAP]
  int32_t* ga;       // [SCAP]
  double* gm;        // [SCAP]
};

// ---- wave-range traversal
// Once a cut splits a tie group, whether a member is kept depends on how
// many members precede it in id order.  The passes after the cuts therefore
// visit the row in wave ranges: wave w takes ids [w WL, (w + 1) WL) (WL a
// multiple of 64), 64 consecutive ids at a time, lane l id base + l, so a
// member's rank is its wave's base count (Filters::b1, b2) plus a ballot
// prefix.  Control flow is wave-uniform; fn may use wave operations.
__device__ __forceinline__ int wave_span(int V) {
  return ((V + NWAVE * 64 - 1) / (NWAVE * 64)) * 64;
}

// One element as the filters see it.
struct SElem {
  int i;             // token id
  bool valid;        // i < the range's end
  double v;          // penalised fp64 value (the mass itself for direct rows)
  uint64_t key;      // d2key(v)
  double P;          // post-temperature probability
  bool kr;           // kept by top-k, top-p and min-p
  uint64_t tk;       // typical order key (F.want_tk, else 0)
  bool kt;           // kept by every filter
};

// Visits ids [lo, hi) by the calling wave, with r1 / r2 members of the rank
// and typical groups before lo.
template <typename Fn>
__device__ __forceinline__ void visit_range(const SlowRow& R, const Filters& F, int lo, int hi,
                                            int r1, int r2, Fn fn) {
  const int l = lane_id();
  const bool s1 = cut_split(F.rank);
  const bool s2 = F.want_tk && F.typ && cut_split(F.tcut);
  for (int base = lo; base < hi; base += 64) {
    SElem e;
    e.i = base + l;
    e.valid = e.i < hi;
    e.v = e.valid ? value_at(R, e.i) : 0.0;
    e.key = d2key(e.v);
    e.P = mass_of(R, e.v);
    const uint64_t m1 = ballot(s1 && e.valid && e.key == F.rank.k);
    const int rk1 = r1 + lanes_below(m1);
    r1 += __popcll(m1);
    e.kr = e.valid && inside(F.rank, e.key, rk1) && e.P >= F.floor_p;
    e.tk = 0ull;
    e.kt = e.kr;
    if (F.want_tk) {
      e.tk = typ_key(e.P, F.H);
      const uint64_t m2 = ballot(s2 && e.kr && e.tk == F.tcut.k);
      const int rk2 = r2 + lanes_below(m2);
      r2 += __popcll(m2);
      if (F.typ) e.kt = e.kr && inside(F.tcut, e.tk, rk2);
    }
    fn(e);
  }
}
// The whole row, each wave its range.
template <typename Fn>
__device__ __forceinline__ void visit_row(const SlowRow& R, const Filters& F, Fn fn) {
  const int WL = wave_span(R.V), w = wave_id();
  const int lo = min(R.V, w * WL), hi = min(R.V, lo + WL);
  visit_range(R, F, lo, hi, F.b1[w], F.b2[w], fn);
}

// Each wave's count of the elements fn(e) selects, and their exclusive scan
// over the waves into b[NWAVE] (all threads; ends with a barrier).
template <typename Sel>
__device__ __forceinline__ void group_bases(const SlowRow& R, const Filters& F, int* b, Sel sel) {
  int c = 0;
  visit_row(R, F, [&](const SElem& e) { c += __popcll(ballot(e.valid && sel(e))); });
  __shared__ int gb_cnt[NWAVE];
  if (lane_id() == 0) gb_cnt[wave_id()] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int w = 0; w < NWAVE; ++w) { b[w] = run; run += gb_cnt[w]; }
  }
  __syncthreads();
}

// Select the shortest prefix, in (key desc, idx asc) order over the eligible
// elements, that holds `target` elements (COUNT) or `target` mass (MASS):
// the cut key, its group's eligible members n and how many of them the
// prefix takes, j.  Eligible: inside `elig` (a cut that splits no group),
// keyed by value; or with TYP, kept by the rank filters of F, keyed by the
// typical order key.  Returns false if the eligible total never reaches the
// target.
template <bool TYP, bool MASS>
__device__ __forceinline__ bool select_prefix(const SlowRow& R, const Filters& F, const Cut& elig, double target,
                              uint64_t klo, uint64_t khi, SlowLds& L, Cut& out, double* red_d,
                              int* red_i) {
  __shared__ uint64_t sh_u[4];
  __shared__ double sh_d[2];
  __shared__ int sh_i[3];
  const int t = threadIdx.x;
  // the element's order key and weight, if eligible
  auto pick = [&](const SElem& e, uint64_t& key, double& m) -> bool {
    if (TYP) {
      key = e.tk;
      m = e.P;
      return e.kr;
    }
    key = e.key;
    m = MASS ? e.P : 1.0;
    return e.valid && inside(elig, e.key, 0);
  };
  double above = 0.0;                           // count or mass of elements with key > khi
  for (int level = 0; level < 8; ++level) {
    uint64_t D = khi - klo;
    int sh = 0;
    while ((D >> sh) >= (uint64_t)NB) ++sh;
    for (int b = t; b < NB; b += WG) { L.cnt[b] = 0u; L.mass[b] = 0.0; }
    __syncthreads();
    visit_row(R, F, [&](const SElem& e) {
      uint64_t key;
      double m;
      if (pick(e, key, m) && key >= klo && key <= khi) {
        int b = (int)((key - klo) >> sh);
        atomicAdd(&L.cnt[b], 1u);
        if (MASS) atomicAdd(&L.mass[b], m);
      }
    });
    __syncthreads();
    if (t == 0) {
      int b = NB - 1;
      double run = above;
      bool hit = false;
      for (; b >= 0; --b) {
        double w = MASS ? L.mass[b] : (double)L.cnt[b];
        // only a bucket holding elements can complete the prefix (a target of
        // 0 selects the first element, as searchsorted(cum, 0) + 1 does)
        if (L.cnt[b] > 0u && run + w >= target) { hit = true; break; }
        run += w;
      }
      sh_i[0] = hit ? b : -1;
      sh_i[1] = hit ? (int)L.cnt[b] : 0;
      sh_d[0] = run;
    }
    __syncthreads();
    const int bstar = sh_i[0];
    const int nb = sh_i[1];
    if (bstar < 0) return false;
    above = sh_d[0];
    const uint64_t nlo = klo + ((uint64_t)bstar << sh);
    const uint64_t nhi_raw = nlo + (sh >= 64 ? ~0ull : ((1ull << sh) - 1));
    const uint64_t nhi = nhi_raw < khi && nhi_raw >= nlo ? nhi_raw : khi;
    klo = nlo;
    khi = nhi;
    __syncthreads();
    if (nb > SCAP && klo == khi) {
      // one key (and one weight) for the whole bucket: the prefix takes c of
      // its nb members, a count known from the weight
      if (t == 0) {
        const double unit = MASS ? (L.mass[bstar] / (double)nb) : 1.0;
        long c = (long)ceil((target - above) / unit);
        if (c < 1) c = 1;
        if (c > nb) c = nb;
        sh_i[2] = (int)c;
      }
      __syncthreads();
      out.k = klo;
      out.n = nb;
      out.j = sh_i[2];
      out.net = R.V <= TIE_NET;
      __syncthreads();
      return true;
    }
    if (nb <= SCAP) {
      // gather the bucket: the cut key's whole group is in it
      __shared__ int gn;
      if (t == 0) gn = 0;
      __syncthreads();
      visit_row(R, F, [&](const SElem& e) {
        uint64_t key;
        double m;
        if (pick(e, key, m) && key >= klo && key <= khi) {
          int pos = atomicAdd(&gn, 1);
          if (pos < SCAP) {
            L.gk[pos] = key;
            L.gi[pos] = e.i;
            L.gm[pos] = m;
          }
        }
      });
      __syncthreads();
      const int n = min(gn, SCAP);   // >= 1: the bucket was counted non-empty
      for (int j = t; j < n; j += WG) L.ga[j] = j;
      __syncthreads();
      block_sort(L.gk, L.gi, L.ga, n);
      if (t == 0) {
        double run = above;
        int j = 0;
        for (; j < n - 1; ++j) {
          run += L.gm[L.ga[j]];
          if (run >= target) break;
        }
        // the cut key's group: sorted positions [g0, g1)
        int g0 = j, g1 = j + 1;
        while (g0 > 0 && L.gk[g0 - 1] == L.gk[j]) --g0;
        while (g1 < n && L.gk[g1] == L.gk[j]) ++g1;
        sh_u[0] = L.gk[j];
        sh_i[0] = g1 - g0;
        sh_i[1] = j + 1 - g0;
      }
      __syncthreads();
      out.k = sh_u[0];
      out.n = sh_i[0];
      out.j = sh_i[1];
      out.net = R.V <= TIE_NET;
      __syncthreads();
      return true;
    }
  }
  // unreachable for 64-bit keys (each level narrows the range by NB)
  out = cut_at(klo);
  return true;
}

// Bucket of value v in the linear split of [lo, lo + NB / inv): monotone in
// v, clamped to [0, NB).
__device__ __forceinline__ int lin_bucket(double v, double lo, double inv) {
  const double f = (v - lo) * inv;
  return f < 0.0 ? 0 : (f >= (double)(NB - 1) ? NB - 1 : (int)f);
}

// Top-p over a logit row with no top-k before it (sampler.py:81-89): the
// shortest prefix in (value desc, idx asc) order holding `target` mass, as a
// Cut (the cut value's group and how many of it the prefix takes).
// Level 0 splits the values in [vlo, M] linearly into NB buckets (values far
// apart land in different buckets, so the mass atomics rarely collide); a
// level keeps the bucket the cut falls in and splits it again, and a bucket
// of at most SCAP elements is gathered, sorted and scanned.  Every level
// classifies an element by the same chain of bucket tests, so "above",
// "in" and "below" stay consistent across the passes.  Returns false when
// this cannot decide -- the elements at or above vlo hold less than the
// target, or MAXLV levels leave a bucket larger than SCAP -- and the
// caller then runs select_prefix.  tsum: WG doubles of LDS.
__device__ __forceinline__ bool select_mass_linear(const SlowRow& R, double target, double vlo, SlowLds& L,
                                   double* tsum, Cut& out, double* red_d, int* red_i) {
  static_assert(NB == WG, "one bucket per thread");
  constexpr int MAXLV = 4;
  const int t = threadIdx.x;
  double lo[MAXLV], inv[MAXLV];
  int bs[MAXLV];
  if (!(R.M > vlo)) return false;
  lo[0] = vlo;
  inv[0] = (double)NB / (R.M - vlo);
  double above = 0.0;
  for (int lv = 0; lv < MAXLV; ++lv) {
    L.cnt[t] = 0u;
    L.mass[t] = 0.0;
    __syncthreads();
#pragma unroll 4
    for (int i = t; i < R.V; i += WG) {
      const double v = value_at(R, i);
      if (!(v >= vlo)) continue;
      bool in = true;
      for (int m = 0; m < lv; ++m)
        if (lin_bucket(v, lo[m], inv[m]) != bs[m]) { in = false; break; }
      if (!in) continue;
      const int b = lin_bucket(v, lo[lv], inv[lv]);
      atomicAdd(&L.cnt[b], 1u);
      atomicAdd(&L.mass[b], mass_of(R, v));
    }
    __syncthreads();
    // suffix masses: tsum[NB-1-b] = mass[b], inclusive scan
    const uint32_t cb = L.cnt[t];
    const double mb = L.mass[t];
    tsum[NB - 1 - t] = mb;
    __syncthreads();
    block_scan(tsum, NB, red_d);
    const double suf = tsum[NB - 1 - t];             // sum over buckets >= t
    // the cut's bucket: the highest non-empty bucket whose suffix reaches
    // the target (suffix masses only grow toward lower buckets)
    const int cand = (cb > 0u && above + suf >= target) ? t : -1;
    const int bstar = block_max(cand, red_i, -1);
    if (bstar < 0) return false;
    const double above_b = above + (bstar + 1 < NB ? tsum[NB - 2 - bstar] : 0.0);
    const int nb = (int)L.cnt[bstar];
    __syncthreads();
    if (nb <= SCAP) {
      __shared__ int gn;
      if (t == 0) gn = 0;
      __syncthreads();
      for (int i = t; i < R.V; i += WG) {
        const double v = value_at(R, i);
        if (!(v >= vlo)) continue;
        bool in = true;
        for (int m = 0; m < lv; ++m)
          if (lin_bucket(v, lo[m], inv[m]) != bs[m]) { in = false; break; }
        if (!in || lin_bucket(v, lo[lv], inv[lv]) != bstar) continue;
        const int pos = atomicAdd(&gn, 1);
        if (pos < SCAP) { L.gk[pos] = d2key(v); L.gi[pos] = i; L.gm[pos] = mass_of(R, v); }
      }
      __syncthreads();
      const int n = min(gn, SCAP);
      for (int j = t; j < n; j += WG) L.ga[j] = j;
      __syncthreads();
      block_sort(L.gk, L.gi, L.ga, n);
      // masses in sorted order, their prefix sums, and the first position
      // where the running total reaches the target (the last if none does)
      tsum[t] = t < n ? L.gm[L.ga[t]] : 0.0;
      __syncthreads();
      block_scan(tsum, NB, red_d);
      const int hit = (t < n && (above_b + tsum[t] >= target || t == n - 1)) ? t : INT_MAX;
      const int j = block_min(hit, red_i, INT_MAX);
      // the cut value's group (equal values share every level's bucket):
      // sorted positions [g0, g1)
      const uint64_t kj = L.gk[j];
      const bool ing = t < n && L.gk[t] == kj;
      const int g0 = block_min(ing ? t : INT_MAX, red_i, INT_MAX);
      const int g1 = block_max(ing ? t + 1 : 0, red_i, 0);
      out.k = kj;
      out.n = g1 - g0;
      out.j = j + 1 - g0;
      out.net = R.V <= TIE_NET;
      __syncthreads();
      return true;
    }
    if (lv + 1 == MAXLV) return false;
    bs[lv] = bstar;
    lo[lv + 1] = lo[lv] + (double)bstar / inv[lv];
    inv[lv + 1] = inv[lv] * (double)NB;
    above = above_b;
  }
  return false;
}

// Row reader and penalty tables of one row (all WG threads; ends with a
// __syncthreads when tables are built).  The window is the last
// max(64, n_keep) history ids if n_keep > 0, else all of them
// (sampler.py:67); ids outside [0, V) are ignored (:68).  Returns the
// window length; a window longer than WIN_MAX builds no tables (the caller
// reports the row as unsupported).
__device__ inline int slow_setup(const SampleArgs& A, int row, const cx_row_params& P,
                                 unsigned char* dyn, SlowRow& R) {
  const int t = threadIdx.x;
  const int V = A.V;
  R.P = &P;
  R.bf16 = A.bf16;
  R.f64 = A.f64;
  R.direct = false;
  R.V = V;
  R.rowp = (const char*)A.logits +
           (size_t)row * (size_t)A.ld * (A.f64 ? 8 : (A.bf16 ? 2 : 4));
  int wlen = 0, wstart = 0;
  if (A.ldh > 0) {
    int len = max(0, min(A.hist_len[row], (int)A.ldh));
    wstart = P.n_keep > 0 ? max(0, len - max(64, P.n_keep)) : 0;
    wlen = len - wstart;
  }
  R.pen = wlen > 0 && wlen <= WIN_MAX &&
          (P.repetition_penalty != 1.0 || P.presence_penalty != 0.0 ||
           P.frequency_penalty != 0.0);
  uint32_t* bitmap = (uint32_t*)dyn;
  uint32_t* hkey = (uint32_t*)(dyn + A.slow_off_hkey);
  R.bitmap = bitmap;
  R.hkey = hkey;
  R.hval = nullptr;
  R.nbw = A.slow_nbw;
  R.ns_log2 = A.ns_log2;
  R.M = 0.0;
  R.invT = 1.0;
  R.S = 1.0;
  if (R.pen) {
    for (int i = t; i < R.nbw; i += WG) bitmap[i] = 0u;
    for (int i = t; i < A.ns; i += WG) hkey[i] = HEMPTY;
    __syncthreads();
    const int32_t* hrow = A.hist + (size_t)row * A.ldh;
    for (int i = t; i < wlen; i += WG) {
      int id = hrow[wstart + i];
      if (id >= 0 && id < V) {
        atomicOr(&bitmap[(id >> 5) & (R.nbw - 1)], 1u << (id & 31));
        const uint32_t mask = (1u << A.ns_log2) - 1;
        uint32_t s = s_hash_slot(id, A.ns_log2);
        for (;;) {
          uint32_t old = atomicCAS(&hkey[s], HEMPTY, ((uint32_t)id << 12) | 1u);
          if (old == HEMPTY) break;
          if ((old >> 12) == (uint32_t)id) { atomicAdd(&hkey[s], 1u); break; }
          s = (s + 1) & mask;
        }
      }
    }
    __syncthreads();
  }
  return wlen;
}

__device__ inline void slow_lds(const SampleArgs& A, unsigned char* dyn, SlowLds& L) {
  unsigned char* base = dyn + A.slow_off_work;
  L.cnt = (uint32_t*)base;
  L.mass = (double*)(base + NB * 4);
  L.gk = (uint64_t*)(base + NB * 12);
  L.gi = (int32_t*)(base + NB * 12 + SCAP * 8);
  L.ga = (int32_t*)(base + NB * 12 + SCAP * 12);
  L.gm = (double*)(base + NB * 12 + SCAP * 16);
}

// All WG threads of the workgroup; dyn holds the multi-pass layout (slow_*
// offsets of SampleArgs).  Entered after a __syncthreads.
__device__ inline void slow_row(const SampleArgs& A, int row, unsigned char* dyn,
                                      double* red_d, int* red_i) {
  double* tsum = (double*)(dyn + A.slow_off_tsum);
  const int t = threadIdx.x;
  const cx_row_params P = A.prm[row];
  const int V = A.V;

  SlowRow R;
  const int wlen = slow_setup(A, row, P, dyn, R);
  if (wlen > WIN_MAX) {                     // window longer than the LDS index
    if (t == 0) {
      A.out_id[row] = -1;
      A.row_status[row] = CX_ROW_UNSUPPORTED | CX_ROW_FLAG_SLOW;
    }
    return;
  }
  SlowLds L;
  slow_lds(A, dyn, L);

  // ---- pass A: max, min, first argmax, first NaN
  double mx = -__builtin_inf(), mn = __builtin_inf();
  int bi = INT_MAX, ni = INT_MAX;
  double bv = -__builtin_inf();
  for (int i = t; i < V; i += WG) {
    double v = value_at(R, i);
    if (v != v) { ni = min(ni, i); continue; }
    argmax_merge(bv, bi, v, i);
    mx = v > mx ? v : mx;
    mn = v < mn ? v : mn;
  }
  block_argmax(bv, bi, red_d, red_i);
  ni = block_min(ni, red_i, INT_MAX);
  mx = bv;
  mn = block_min(mn, red_d, __builtin_inf());
  const int amax = ni != INT_MAX ? ni : (bi == INT_MAX ? 0 : bi);
  if (P.temperature == 0.0) {                                // sampler.py:114-115
    if (A.out_probs) {
      float* pr = A.out_probs + (size_t)row * V;
      for (int i = t; i < V; i += WG) pr[i] = i == amax ? 1.0f : 0.0f;
    }
    if (t == 0) {
      A.out_id[row] = amax;
      A.row_status[row] = CX_ROW_GREEDY | CX_ROW_FLAG_SLOW;
    }
    return;
  }
  const double invT = 1.0 / P.temperature;
  bool degenerate = ni != INT_MAX || mx == __builtin_inf() || mx == -__builtin_inf();
  R.M = mx;
  R.invT = invT;
  R.S = 1.0;
  // ---- pass B: the normaliser (and the T = 1 sum for the P**(1/T) underflow)
  if (!degenerate) {
    const bool under = P.temperature != 1.0 && log((double)V) * invT > 740.0;
    double s = 0.0, s1 = 0.0;
    for (int i = t; i < V; i += WG) {
      double v = value_at(R, i);
      s += exp((v - mx) * invT);
      if (under) s1 += exp(v - mx);
    }
    R.S = block_sum(s, red_d);
    if (under) {
      double S1 = block_sum(s1, red_d);
      if (pow(1.0 / S1, invT) == 0.0) degenerate = true;
    }
  }
  if (degenerate) {
    // all-NaN probabilities: top-k or min-p zero them and argmax(x) follows
    // (sampler.py:123-125); otherwise numpy's choice raises ValueError.
    const bool am = P.top_k > 0 || P.min_p > 0.0;
    if (A.out_probs) {
      float* pr = A.out_probs + (size_t)row * V;
      for (int i = t; i < V; i += WG) pr[i] = (am && i == amax) ? 1.0f : 0.0f;
    }
    if (t == 0) {
      A.out_id[row] = am ? amax : -1;
      A.row_status[row] = (am ? CX_ROW_ARGMAX : CX_ROW_ERROR) | CX_ROW_FLAG_SLOW;
    }
    return;
  }

  // ---- rank-order filters
  __shared__ int s_b1[NWAVE], s_b2[NWAVE];
  if (t < NWAVE) { s_b1[t] = 0; s_b2[t] = 0; }
  Filters F;
  F.rank = cut_at(0ull);
  F.floor_p = 0.0;
  F.typ = false;
  F.H = 0.0;
  F.tcut = cut_at(0ull);
  F.want_tk = false;
  F.b1 = s_b1;
  F.b2 = s_b2;
  __syncthreads();
  const uint64_t kmax = d2key(mx), kmin = d2key(mn);
  const Cut all = cut_at(0ull);
  if (P.top_k > 0 && P.top_k < V) {                          // sampler.py:76-79
    Cut c;
    select_prefix<false, false>(R, F, all, (double)P.top_k, kmin, kmax, L, c, red_d, red_i);
    F.rank = cut_at(c.k);                                    // ties at the k-th value stay
  }
  if (P.top_p < 1.0) {                                       // sampler.py:81-89
    Cut c;
    // without top-k: linear value buckets from vlo, below which the row
    // holds under a quarter of the mass outside the nucleus
    // (V exp((vlo - M) / T) / S = (1 - top_p) / 4)
    bool done = false;
    if (F.rank.k == 0ull) {
      const double vlo = fmax(mn, mx + P.temperature * log(0.25 * (1.0 - P.top_p) * R.S / (double)V));
      done = select_mass_linear(R, P.top_p, vlo, L, tsum, c, red_d, red_i);
      if (done) F.rank = c;
    }
    if (!done) {
      const uint64_t lo = F.rank.k > kmin ? F.rank.k : kmin;
      if (select_prefix<false, true>(R, F, F.rank, P.top_p, lo, kmax, L, c, red_d, red_i))
        F.rank = c;
    }
    // a cut inside a group of equal values: its members' ranks by wave range
    const uint64_t kc = F.rank.k;
    if (cut_split(F.rank))
      group_bases(R, F, s_b1, [&](const SElem& e) { return e.key == kc; });
  }
  if (P.min_p > 0.0) F.floor_p = P.min_p * (1.0 / R.S);      // sampler.py:91-93
  if (P.typical_p < 1.0) {                                   // sampler.py:95-105
    double h = 0.0;
    uint64_t tlo = ~0ull, thi = 0ull;
    visit_row(R, F, [&](const SElem& e) {
      if (e.kr) h -= e.P * log(e.P > 1e-38 ? e.P : 1e-38);
    });
    F.H = block_sum(h, red_d);
    F.want_tk = true;
    visit_row(R, F, [&](const SElem& e) {
      if (e.kr) {
        tlo = e.tk < tlo ? e.tk : tlo;
        thi = e.tk > thi ? e.tk : thi;
      }
    });
    tlo = block_min<unsigned long long>(tlo, (unsigned long long*)red_d, ~0ull);
    thi = block_max<unsigned long long>(thi, (unsigned long long*)red_d, 0ull);
    Cut c;
    F.typ = select_prefix<true, true>(R, F, all, P.typical_p, tlo, thi, L, c, red_d, red_i);
    F.tcut = c;
    const uint64_t kt = c.k;
    if (F.typ && cut_split(F.tcut))
      group_bases(R, F, s_b2, [&](const SElem& e) { return e.kr && e.tk == kt; });
  }

  // ---- normalise and draw in token-id order (sampler.py:123-127): each
  // wave's kept mass over its range, the range holding u, then a scan of
  // that range in id order
  __shared__ double s_wm[NWAVE];
  __shared__ int s_found;
  const int WL = wave_span(V);
  {
    double m = 0.0;
    visit_row(R, F, [&](const SElem& e) { if (e.kt) m += e.P; });
    m = wave_sum(m);
    if (lane_id() == 0) s_wm[wave_id()] = m;
    if (t == 0) s_found = INT_MAX;
  }
  __syncthreads();
  double Z = 0.0;
  for (int k = 0; k < NWAVE; ++k) Z += s_wm[k];
  if (!(Z > 0.0)) {
    if (A.out_probs) {
      float* pr = A.out_probs + (size_t)row * V;
      for (int i = t; i < V; i += WG) pr[i] = i == amax ? 1.0f : 0.0f;
    }
    if (t == 0) {
      A.out_id[row] = amax;
      A.row_status[row] = CX_ROW_ARGMAX | CX_ROW_FLAG_SLOW;
    }
    return;
  }
  // cdf_i = cumsum(P / Z)_i / cumsum(P / Z)_last; first i with cdf_i > u
  const double u = A.u[row];
  double last = 0.0;
  for (int k = 0; k < NWAVE; ++k) last += s_wm[k] / Z;
  {
    double prev = 0.0;
    int wr = -1;
    for (int k = 0; k < NWAVE && wr < 0; ++k) {
      const double nx = prev + s_wm[k] / Z;
      if (nx / last > u) wr = k;
      else prev = nx;
    }
    if (wave_id() == wr) {
      // the group members before this range, and the running sum
      const int lo = wr * WL, hi = min(V, lo + WL);
      double run = prev;
      int found = INT_MAX;
      visit_range(R, F, lo, hi, F.b1[wr], F.b2[wr], [&](const SElem& e) {
        if (found != INT_MAX) return;
        const double q = e.kt ? e.P / Z : 0.0;
        const double incl = run + wave_scan_dpp(q);
        const uint64_t hb = ballot(q != 0.0 && incl / last > u);
        if (hb) found = __builtin_amdgcn_readlane(e.i, __builtin_ctzll(hb));
        run = __shfl(incl, 63);
      });
      if (lane_id() == 0) s_found = found;
    }
  }
  __syncthreads();
  int found = s_found;
  if (found == INT_MAX) {
    // u beyond the last step by rounding: the last kept id
    int lastk = -1;
    visit_row(R, F, [&](const SElem& e) { if (e.kt) lastk = max(lastk, e.i); });
    found = block_max(lastk, red_i, -1);
  }
  if (A.out_probs) {
    float* pr = A.out_probs + (size_t)row * V;
    visit_row(R, F, [&](const SElem& e) {
      if (e.valid) pr[e.i] = e.kt ? (float)(e.P / Z) : 0.0f;
    });
  }
  if (t == 0) {
    A.out_id[row] = found;
    A.row_status[row] = CX_ROW_OK | CX_ROW_FLAG_SLOW;
  }
}

// Sampler.apply_penalties on elements [i0, i1) of a row (sampler.py:63-73,
// plus presence/frequency): out64 = the fp64 penalised logits.  Every
// workgroup of the row builds the row's tables; workgroup 0 writes the
// row's status (CX_ROW_OK, or CX_ROW_UNSUPPORTED for a window longer than
// WIN_MAX, with nothing written).
__device__ inline void penalties_range(const SampleArgs& A, int row, int i0, int i1,
                                       unsigned char* dyn, bool report) {
  const cx_row_params P = A.prm[row];
  SlowRow R;
  const int wlen = slow_setup(A, row, P, dyn, R);
  const bool ok = wlen <= WIN_MAX;
  if (ok) {
    double* out = A.out64 + (size_t)row * (size_t)A.ldo;
    for (int i = i0 + (int)threadIdx.x; i < i1; i += WG) out[i] = value_at(R, i);
  }
  if (report && threadIdx.x == 0) A.row_status[row] = ok ? CX_ROW_OK : CX_ROW_UNSUPPORTED;
}

// Sampler._truncate on one row of fp64 probabilities (sampler.py:75-106).
// The row's values are the masses themselves (no renormalisation, as in the
// reference, whose top-p and typical cuts accumulate the unnormalised
// input):
//   top-k     keep P >= the k-th largest value (ties kept)         :76-79
//   top-p     shortest prefix in (P desc, id asc) order whose
//             running sum reaches top_p                           :81-89
//   min-p     keep P >= min_p * max P                              :91-93
//   typical   entropy H over the kept values, then the shortest
//             prefix in (|log P + H| asc, id asc) order reaching
//             typical_p                                            :95-105
// out64[i] = P_i where kept, else 0.  Of a group of equal keys that a cut
// splits, the survivors are spread over the group's ids (spread_kept,
// cx_device.hpp; numpy's argsort leaves which ones unspecified).  A row
// holding NaN or a negative value is reported as CX_ROW_ERROR and left
// unwritten.
__device__ inline void truncate_row(const SampleArgs& A, int row, unsigned char* dyn,
                                    double* red_d, int* red_i) {
  const int t = threadIdx.x;
  const cx_row_params P = A.prm[row];
  const int V = A.V;
  SlowRow R;
  R.P = &P;
  R.bf16 = 0;
  R.f64 = 1;
  R.direct = true;
  R.V = V;
  R.rowp = (const char*)A.logits + (size_t)row * (size_t)A.ld * 8;
  R.pen = false;
  R.bitmap = nullptr;
  R.hkey = nullptr;
  R.hval = nullptr;
  R.nbw = 1;
  R.ns_log2 = 0;
  R.M = 0.0;
  R.invT = 1.0;
  R.S = 1.0;
  SlowLds L;
  slow_lds(A, dyn, L);

  double mx = -__builtin_inf(), mn = __builtin_inf();
  int bad = 0;
  for (int i = t; i < V; i += WG) {
    double v = value_at(R, i);
    if (!(v >= 0.0)) { bad = 1; continue; }
    mx = v > mx ? v : mx;
    mn = v < mn ? v : mn;
  }
  bad = block_max(bad, red_i, 0);
  mx = block_max(mx, red_d, -__builtin_inf());
  mn = block_min(mn, red_d, __builtin_inf());
  if (bad) {
    if (t == 0) A.row_status[row] = CX_ROW_ERROR;
    return;
  }
  __shared__ int s_b1[NWAVE], s_b2[NWAVE];
  if (t < NWAVE) { s_b1[t] = 0; s_b2[t] = 0; }
  Filters F;
  F.rank = cut_at(0ull);
  F.floor_p = 0.0;
  F.typ = false;
  F.H = 0.0;
  F.tcut = cut_at(0ull);
  F.want_tk = false;
  F.b1 = s_b1;
  F.b2 = s_b2;
  __syncthreads();
  const uint64_t kmax = d2key(mx), kmin = d2key(mn);
  const Cut all = cut_at(0ull);
  if (P.top_k > 0 && P.top_k < V) {
    Cut c;
    select_prefix<false, false>(R, F, all, (double)P.top_k, kmin, kmax, L, c, red_d, red_i);
    F.rank = cut_at(c.k);
  }
  if (P.top_p < 1.0) {
    Cut c;
    const uint64_t lo = F.rank.k > kmin ? F.rank.k : kmin;
    if (select_prefix<false, true>(R, F, F.rank, P.top_p, lo, kmax, L, c, red_d, red_i))
      F.rank = c;
    const uint64_t kc = F.rank.k;
    if (cut_split(F.rank))
      group_bases(R, F, s_b1, [&](const SElem& e) { return e.key == kc; });
  }
  if (P.min_p > 0.0) F.floor_p = P.min_p * mx;
  if (P.typical_p < 1.0) {
    double h = 0.0;
    uint64_t tlo = ~0ull, thi = 0ull;
    visit_row(R, F, [&](const SElem& e) {
      if (e.kr) h -= e.P * log(e.P > 1e-38 ? e.P : 1e-38);
    });
    F.H = block_sum(h, red_d);
    F.want_tk = true;
    visit_row(R, F, [&](const SElem& e) {
      if (e.kr) {
        tlo = e.tk < tlo ? e.tk : tlo;
        thi = e.tk > thi ? e.tk : thi;
      }
    });
    tlo = block_min<unsigned long long>(tlo, (unsigned long long*)red_d, ~0ull);
    thi = block_max<unsigned long long>(thi, (unsigned long long*)red_d, 0ull);
    Cut c = all;
    if (tlo <= thi)
      F.typ = select_prefix<true, true>(R, F, all, P.typical_p, tlo, thi, L, c, red_d, red_i);
    F.tcut = c;
    const uint64_t kt = c.k;
    if (F.typ && cut_split(F.tcut))
      group_bases(R, F, s_b2, [&](const SElem& e) { return e.kr && e.tk == kt; });
  }
  double* out = A.out64 + (size_t)row * (size_t)A.ldo;
  visit_row(R, F, [&](const SElem& e) {
    if (e.valid) out[e.i] = e.kt ? e.P : 0.0;
  });
  if (t == 0) A.row_status[row] = CX_ROW_OK;
}

}  // namespace cx
