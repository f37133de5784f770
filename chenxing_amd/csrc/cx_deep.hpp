// cx_deep.hpp -- rows whose nucleus is deeper than any region (reference
// chenxing/core/sampler.py:81-93 and :117-127): top-p and min-p rows with no
// top-k, no typical-p and no penalty window, which the fused kernel leaves
// pending because their kept set outgrows its region.  One workgroup per
// row; two passes over the row (three with min-p) and two short ones, in
// place of the multi-pass path's eight or more:
//
//   pass 1  every term e = exp((x - M) / T) <= 1 (M the row maximum the
//           fused kernel found; table-driven fp64 exp): the row's sum S,
//           and a histogram of e over DNB value buckets linear in
//           (M - x) / T on [0, DSPAN).  A bucket sums its terms as integers
//           in its own fixed-point scale (2^-F_b, F_b growing with the
//           bucket's depth, so every term keeps about 42 significant bits and
//           no sum overflows), so the sums do not depend on the order of the
//           atomic additions.  At the end of each wave range (the row split
//           into NWAVE contiguous id ranges) the histogram, summed into
//           coarse buckets, is copied: the mass each range holds per coarse
//           bucket.
//   cut     the first bucket, from the top, whose running sum reaches
//           top_p * S (sampler.py:82-85: cumsum of the sorted
//           probabilities, searchsorted, one past the index)
//   pass 2  the elements of that bucket, gathered, sorted by value
//           (descending) and id (ascending) and scanned: the cut element;
//           of the cut value's group the survivors spread over its ids
//           (spread_kept, cx_device.hpp).  The same pass
//           adds, per range, the terms of the cut's coarse bucket that lie
//           above the cut bucket, so each range's kept mass follows from the
//           copies.  (With min-p, pass 3 instead sums each range's kept terms
//           again, testing e >= min_p per element, sampler.py:91-93.)
//   draw    the range holding u * Z (Z the kept total), then its sixteenth
//           (each wave sums one); one wave scans that sixteenth in id order
//           (sampler.py:126-127: choice == searchsorted(cumsum, u, 'right'))
//
// On bf16 rows a term is the product of three LDS table entries, one per
// part of the value's bits (sign, exponent and the top three mantissa bits;
// the next two; the last two: x = xh + xm + xl exactly), each exp of its
// part (exp((xh - M) / T), exp(xm / T), exp(xl / T)), built once per row:
// no fp64 exp per element.  (Rows whose |x| / T could reach 7000 use the
// exp per element, so no table entry can overflow.)
//
// Each thread reads 32 bytes per pass step (8 fp32 or 16 bf16 values).  On
// 16-byte-aligned rows these are two range-checked buffer loads, issued
// three steps ahead and unpacked only where used, so the loads stay in
// flight; other rows load value by value.
//
// Sums outside the histograms run in a fixed order in fp64.  Each term is
// within 1 ulp, a bucket's integer sum within 2^-42 (relative) of its
// terms' sum, fp64 sums of at most 2^20 terms within 2^20 ulp, and the
// reference's own cumulative sums within 4e-11 (relative) of exact: a
// decision closer to its threshold than 5e-11 of the total returns false
// and the row takes the multi-pass path, as do NaN rows, cuts below the
// bucket span and cut buckets of more elements than the gather holds.
#pragma once
#include "cx_device.hpp"
#include "cx_internal.hpp"

namespace cx {

constexpr int DNB = 4096;                     // value buckets
constexpr int DCB = 64;                       // fine buckets per coarse bucket
constexpr int DNCB = DNB / DCB;               // coarse buckets
constexpr float DSPAN = 40.0f;                // bucket span below M, units of T (exp(-40) ~ 4e-18)
constexpr float DSCALE = DNB / DSPAN;         // buckets per unit
constexpr int DF0 = 42;                       // fixed-point bits of a term at its bucket's top
constexpr double DTOL = 5e-11;                // relative decision margin
constexpr int DCAP = 4 * WG;                  // cut-bucket capacity, fp32 rows (block_sort<4>)
constexpr int DCAP16 = 2 * WG;                // cut-bucket capacity, bf16 rows
constexpr int DW = 8;                         // 32-bit words per thread per step
constexpr int DNV = 16;                       // most values per thread per step (bf16)
// dynamic LDS: h[DNB] u64 | C[NWAVE][DNCB] f64 | X, where X holds the gather
// (gk u64 | gi i32 | ga i32, DCAP entries) on fp32 rows and the three term
// tables (4096 + 2048 + 2048 f64) on bf16 rows, whose gather (DCAP16
// entries) reuses h once the cut bucket is known
constexpr int DEEP_OFF_C = DNB * 8;
constexpr int DEEP_OFF_X = DEEP_OFF_C + NWAVE * DNCB * 8;
constexpr int DEEP_LDS = DEEP_OFF_X + DCAP * 16;
static_assert(DCAP16 * 16 <= DNB * 8 && (4096 + 2048 + 2048) * 8 <= DCAP * 16, "deep LDS layout");

// 16 bytes (vector_size, so host builds of this header compile too)
typedef uint32_t deep_u32x4 __attribute__((vector_size(16)));

// The row as the passes read it.  nv values per thread per step (8 fp32 or
// 16 bf16, 32 bytes), a step covering nv * WG ids.
struct DeepRow {
  __amdgpu_buffer_rsrc_t rs;  // the row, rounded up to 16 bytes (aligned rows)
  const void* p;
  int V, nv, step;
  bool bf16;
};

// The 32 bytes holding values [e0, e0 + nv) (e0 a multiple of nv).  Aligned
// rows: two range-checked 16-byte loads (zeros past the row, no branch), so
// the compiler can keep them in flight; other rows: value by value, zero
// past V.
template <bool VEC>
__device__ __forceinline__ void deep_fetch(const DeepRow& R, int e0, uint32_t (&w)[DW]) {
  if constexpr (VEC) {
    const int off = e0 * (R.bf16 ? 2 : 4);
    const deep_u32x4 a =
        __builtin_bit_cast(deep_u32x4, __builtin_amdgcn_raw_buffer_load_b128(R.rs, off, 0, 0));
    const deep_u32x4 b =
        __builtin_bit_cast(deep_u32x4, __builtin_amdgcn_raw_buffer_load_b128(R.rs, off + 16, 0, 0));
#pragma unroll
    for (int k = 0; k < 4; ++k) { w[k] = a[k]; w[4 + k] = b[k]; }
  } else if (R.bf16) {
    const uint16_t* p = (const uint16_t*)R.p;
#pragma unroll
    for (int k = 0; k < DW; ++k) {
      const uint32_t lo = e0 + 2 * k < R.V ? p[e0 + 2 * k] : 0u;
      const uint32_t hi = e0 + 2 * k + 1 < R.V ? p[e0 + 2 * k + 1] : 0u;
      w[k] = lo | (hi << 16);
    }
  } else {
    const float* p = (const float*)R.p;
#pragma unroll
    for (int k = 0; k < DW; ++k) w[k] = e0 + k < R.V ? __float_as_uint(p[e0 + k]) : 0u;
  }
}
// bf16 code of value j of a fetch (bf16 rows).
__device__ __forceinline__ uint32_t deep_code(const uint32_t (&w)[DW], int j) {
  return (j & 1) ? (w[j >> 1] >> 16) : (w[j >> 1] & 0xFFFFu);
}
// Value j of a fetch.
__device__ __forceinline__ float deep_val(const DeepRow& R, const uint32_t (&w)[DW], int j) {
  if (R.bf16) return __uint_as_float((j & 1) ? (w[j >> 1] & 0xFFFF0000u) : (w[j >> 1] << 16));
  return __uint_as_float(w[j < DW ? j : 0]);
}

// Value bucket of x, or -1 below the span (and for NaN): fp32 arithmetic,
// the same expression in every pass, so an element lands in the same
// bucket each time.
__device__ __forceinline__ int deep_bucket(float x, float Mf, float invTf) {
  const float d = (Mf - x) * invTf;
  return d < DSPAN ? (int)(d * DSCALE) : -1;
}
// Fixed-point exponent of fine bucket b: its terms are at most
// ~exp(-b / DSCALE) = 2^(-b * 0.0140888), so 2^(DF0 + floor(b * 923 / 2^16))
// (923 / 2^16 = 0.0140839) keeps each term below 2^(DF0 + 1) and a sum of at
// most 2^20 of them below 2^63.
__device__ __forceinline__ int deep_scale(int b) { return DF0 + ((b * 923) >> 16); }
// 2^e for |e| < 1023, from its bits
__device__ __forceinline__ double deep_pow2(int e) {
  return __longlong_as_double((long long)(1023 + e) << 52);
}
__device__ __forceinline__ double deep_term(float x, double M, double invT, const double* tab) {
  return exp64_neg(((double)x - M) * invT, tab);
}

// bf16 term tables: ta over code >> 4, tb and tc over (code >> 7) << 2 with
// mantissa bits 3..2, resp. 1..0, of the bf16 code.
__device__ __forceinline__ float bf16_of(uint32_t code) { return __uint_as_float(code << 16); }
__device__ inline void deep_build_tables(double* ta, double* tb, double* tc, double M, double invT,
                                         const double* tab) {
  // (entries of infinite or NaN codes, which no in-span value uses, are 0)
  auto fin = [](double v) { return v == v && v < __builtin_inf() ? v : 0.0; };
  for (int i = threadIdx.x; i < 4096; i += WG)
    ta[i] = fin(exp64(((double)bf16_of((uint32_t)i << 4) - M) * invT, tab));
  for (int i = threadIdx.x; i < 2048; i += WG) {
    const uint32_t hi = (uint32_t)(i >> 2) << 7, lo = (uint32_t)(i & 3);
    // exact differences of bf16 values sharing sign and exponent
    tb[i] = fin(exp64(((double)bf16_of(hi | (lo << 2)) - (double)bf16_of(hi)) * invT, tab));
    tc[i] = fin(exp64(((double)bf16_of(hi | lo) - (double)bf16_of(hi)) * invT, tab));
  }
}
__device__ __forceinline__ double deep_term16(uint32_t code, const double* ta, const double* tb,
                                              const double* tc) {
  const uint32_t se = (code >> 7) << 2;
  return ta[code >> 4] * tb[se | ((code >> 2) & 3u)] * tc[se | (code & 3u)];
}

// Exclusive prefix sum of one fp64 per thread across the workgroup, in a
// fixed order.  scratch: 2 * NWAVE slots.
__device__ __forceinline__ double block_excl_scan_d(double v, double* scratch) {
  double inc = v;
  for (int o = 1; o < 64; o <<= 1) {
    const double w = __shfl_up(inc, o);
    if (lane_id() >= o) inc += w;
  }
  if (lane_id() == 63) scratch[wave_id()] = inc;
  __syncthreads();
  if (threadIdx.x < 64) {
    const double w = threadIdx.x < NWAVE ? scratch[threadIdx.x] : 0.0;
    double y = w;
    for (int o = 1; o < 64; o <<= 1) {
      const double z = __shfl_up(y, o);
      if (lane_id() >= o) y += z;
    }
    if (threadIdx.x < NWAVE) scratch[NWAVE + threadIdx.x] = y - w;
  }
  __syncthreads();
  const double r = scratch[NWAVE + wave_id()] + (inc - v);
  __syncthreads();
  return r;
}

// f(k, w) for every step k < n of a pass over ids from lo on (this
// thread's fetch w from id lo + k * stride + nv * idx on), with the next
// three steps' loads in flight.
template <bool VEC, class F>
__device__ __forceinline__ void deep_stream(const DeepRow& R, int lo, int stride, int idx, int n,
                                            F&& f) {
  const int e = lo + R.nv * idx;
  uint32_t b0[DW], b1[DW], b2[DW], b3[DW];
  deep_fetch<VEC>(R, e, b0);
  deep_fetch<VEC>(R, e + stride, b1);
  deep_fetch<VEC>(R, e + 2 * stride, b2);
  for (int k = 0; k < n; k += 4) {
    deep_fetch<VEC>(R, e + (k + 3) * stride, b3);
    f(k, b0);
    if (k + 1 >= n) break;
    deep_fetch<VEC>(R, e + (k + 4) * stride, b0);
    f(k + 1, b1);
    if (k + 2 >= n) break;
    deep_fetch<VEC>(R, e + (k + 5) * stride, b1);
    f(k + 2, b2);
    if (k + 3 >= n) break;
    deep_fetch<VEC>(R, e + (k + 6) * stride, b2);
    f(k + 3, b3);
  }
}

// Does the row qualify, and its maximum M (from the fused kernel's slice
// records: exact, the raw values being unpenalised).
// (the conditions on the call and the row's parameters alone; a top-k
// bound only where the caller's path applies it: the counted bf16 path)
__device__ inline bool deep_candidate(const SampleArgs& A, int row, const cx_row_params& P,
                                      bool topk_ok = false) {
  if (A.all_slow || A.out_probs) return false;
  if (!(P.temperature > 0.0) || P.typical_p < 1.0) return false;
  if (P.top_k > 0 && P.top_k < A.V && !topk_ok) return false;
  if (A.logV * (1.0 / P.temperature) > 740.0) return false;       // P**(1/T) may underflow
  if (A.ldh > 0 && A.hist_len[row] > 0 &&
      (P.repetition_penalty != 1.0 || P.presence_penalty != 0.0 || P.frequency_penalty != 0.0))
    return false;
  return true;
}
__device__ inline bool deep_eligible(const SampleArgs& A, int row, const cx_row_params& P,
                                     double& M, bool topk_ok = false) {
  if (!deep_candidate(A, row, P, topk_ok)) return false;
  double m = -__builtin_inf();
  for (int s = 0; s < A.nsplit; ++s) {
    const double v = A.stats[(size_t)row * A.nsplit + s].m;
    m = v > m ? v : m;
  }
  M = m;
  return m > -__builtin_inf() && m < __builtin_inf();
}

template <bool VEC>
__device__ __forceinline__ bool deep_row_impl(const SampleArgs& A, int row, const cx_row_params& P,
                                     double M, unsigned char* dyn, double* red_d, int* red_i) {
  __shared__ double tab[64];
  __shared__ double s_d[2 * NWAVE + 4];
  __shared__ double s_wm[NWAVE];                     // kept mass per wave range / sixteenth
  __shared__ unsigned long long s_corr[2 * NWAVE];   // per range: cut coarse bucket, cut bucket
  __shared__ int s_i[4];
  __shared__ int s_g[2];
  const int t = threadIdx.x, l = lane_id(), w = wave_id();
  DeepRow R;
  R.V = A.V;
  R.bf16 = A.bf16 != 0;
  R.nv = R.bf16 ? 16 : 8;
  R.step = R.nv * WG;
  R.p = (const char*)A.logits + (size_t)row * (size_t)A.ld * (R.bf16 ? 2 : 4);
  R.rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(R.p), (short)0,
                                           (R.V * (R.bf16 ? 2 : 4) + 15) & ~15, 0x00020000);
  const int V = R.V, nv = R.nv;
  const double invT = 1.0 / P.temperature;
  const float Mf = (float)M, invTf = (float)invT;
  unsigned long long* h = (unsigned long long*)dyn;
  double* C = (double*)(dyn + DEEP_OFF_C);          // C[r * DNCB + cb]: ranges 0..r, cumulative
  double* ta = (double*)(dyn + DEEP_OFF_X);
  double* tb = ta + 4096;
  double* tc = tb + 2048;
  // the term tables: bf16 rows whose |x| / T stays below 7000
  const bool use_tab = R.bf16 && (fabs(M) + 40.0 * P.temperature) * invT < 7000.0;
  const int cap = R.bf16 ? DCAP16 : DCAP;
  unsigned char* gbase = R.bf16 ? dyn : dyn + DEEP_OFF_X;
  uint64_t* gk = (uint64_t*)gbase;
  int32_t* gi = (int32_t*)(gbase + cap * 8);
  int32_t* ga = (int32_t*)(gbase + cap * 12);
  // wave ranges: NWAVE contiguous id ranges of L ids, L a multiple of the
  // step, so each workgroup step lies in one range
  const int L = ((V + NWAVE * R.step - 1) / (NWAVE * R.step)) * R.step;
  const int nsteps = (V + R.step - 1) / R.step;
  for (int b = t; b < DNB; b += WG) h[b] = 0ull;
  if (t < 2 * NWAVE) s_corr[t] = 0ull;
  if (t == 0) s_i[0] = 0;
  load_exp64_tab(tab);                               // its barrier also orders the clears
  if (use_tab) {
    deep_build_tables(ta, tb, tc, M, invT, tab);
    __syncthreads();
  }

  // ---- pass 1: S and the bucket histograms, copied at each range's end
  double s = 0.0;
  int bad = 0;
  deep_stream<VEC>(R, 0, R.step, t, nsteps, [&](int k, const uint32_t (&wd)[DW]) {
    const int e0 = k * R.step + nv * t;
#pragma unroll
    for (int j = 0; j < DNV; ++j) {
      if (j >= nv || e0 + j >= V) break;
      const float x = deep_val(R, wd, j);
      if (!(x == x) || x > Mf) { bad = 1; continue; }
      const int b = deep_bucket(x, Mf, invTf);
      // (the tables leave out terms below the span: at most V exp(-40) in all)
      const double ev = !use_tab ? deep_term(x, M, invT, tab)
                                 : (b >= 0 ? deep_term16(deep_code(wd, j), ta, tb, tc) : 0.0);
      s += ev;
      if (b >= 0) atomicAdd(h + b, (unsigned long long)(ev * deep_pow2(deep_scale(b))));
    }
    const int r = (k * R.step) / L;
    if ((k + 1) * R.step % L == 0 || k + 1 == nsteps) {
      // the histogram so far, summed into coarse buckets (16 threads each)
      __syncthreads();
      double v = 0.0;
#pragma unroll
      for (int j = 0; j < 4; ++j) v += (double)h[4 * t + j] * deep_pow2(-deep_scale(4 * t + j));
      v = row_reduce(v, OpAdd());
      for (int rr = r; rr < (k + 1 == nsteps ? NWAVE : r + 1); ++rr)
        if ((t & 15) == 0) C[rr * DNCB + (t >> 4)] = v;
      __syncthreads();
    }
  });
  const double S = block_sum(s, s_d);
  if (block_max(bad, red_i, 0)) return false;        // NaN (or a value above M)
  const double tolS = DTOL * S;

  // ---- the cut: first non-empty bucket whose inclusive sum reaches top_p * S
  const bool cut = P.top_p < 1.0;
  float xcut = -__builtin_inff();
  int g0 = 0, gn = 0, gj = 0;                        // the cut value's group: none
  int bs = DNB;                                      // no cut: every bucket above it
  if (cut) {
    const double tgt = P.top_p * S;
    double vb[4];
    double c4 = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      vb[j] = (double)h[4 * t + j] * deep_pow2(-deep_scale(4 * t + j));
      c4 += vb[j];
    }
    double before = block_excl_scan_d(c4, s_d);
    int bstar = INT_MAX;
    double above = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const double incl = before + vb[j];
      if (bstar == INT_MAX && h[4 * t + j] != 0ull && incl >= tgt) {
        bstar = 4 * t + j;
        above = before;
      }
      before = incl;
    }
    bs = block_min(bstar, red_i, INT_MAX);
    if (bs == INT_MAX) return false;                 // the cut lies below the span
    if (bstar == bs) red_d[2 * NWAVE + 2] = above;
    __syncthreads();
    above = red_d[2 * NWAVE + 2];
    __syncthreads();

    // ---- pass 2: gather the cut bucket; per range, the terms of the cut's
    // coarse bucket above it (the copies end at coarse-bucket boundaries)
    const bool corr = P.min_p <= 0.0;
    const int cb0 = (bs / DCB) * DCB;
    const double fc = deep_pow2(deep_scale(cb0));
    unsigned long long acc = 0ull;
    deep_stream<VEC>(R, 0, R.step, t, nsteps, [&](int k, const uint32_t (&wd)[DW]) {
      const int e0 = k * R.step + nv * t;
#pragma unroll
      for (int j = 0; j < DNV; ++j) {
        if (j >= nv) break;
        const float x = deep_val(R, wd, j);
        const int b = e0 + j < V ? deep_bucket(x, Mf, invTf) : -1;
        // the cut bucket's elements, placed by one LDS atomic per wave
        const bool g = b == bs;
        const uint64_t m = ballot(g);
        if (m) {
          int base = 0;
          if (l == 0) base = atomicAdd(s_i, __popcll(m));
          base = __builtin_amdgcn_readfirstlane(base);
          const int pos = base + lanes_below(m);
          if (g && pos < cap) {
            gk[pos] = d2key((double)x);
            gi[pos] = e0 + j;
            ga[pos] = 0;
          }
        }
        if (corr && b >= cb0 && b < bs)
          acc += (unsigned long long)((use_tab ? deep_term16(deep_code(wd, j), ta, tb, tc)
                                               : deep_term(x, M, invT, tab)) * fc);
      }
      if (corr && ((k + 1) * R.step % L == 0 || k + 1 == nsteps)) {
        const unsigned long long m = wave_sum(acc);
        if (l == 0 && m != 0ull) atomicAdd(s_corr + (k * R.step) / L, m);
        acc = 0ull;
      }
    });
    __syncthreads();
    const int ng = s_i[0];
    __syncthreads();
    if (ng > cap) return false;
    block_sort<4>(gk, gi, ga, ng);                   // value descending, id ascending
    // thread t: sorted entries 4t .. 4t+3, their terms and running sums
    double qv[4];
    double s4 = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = 4 * t + j;
      qv[j] = e < ng ? exp64_neg((key2d(gk[e]) - M) * invT, tab) : 0.0;
      s4 += qv[j];
    }
    double run = above + block_excl_scan_d(s4, s_d);
    int jstar = INT_MAX;
    double cprev = 0.0, cstar = 0.0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int e = 4 * t + j;
      const double incl = run + qv[j];
      if (jstar == INT_MAX && e < ng && incl >= tgt) {
        jstar = e;
        cprev = run;
        cstar = incl;
      }
      run = incl;
    }
    const int js = block_min(jstar, red_i, INT_MAX);
    if (js == INT_MAX) return false;
    if (jstar == js) {
      // robust: this element's running sum clearly reaches the target and
      // the one before clearly does not (the first element is always kept)
      const bool first = bs == 0 && js == 0;
      const bool ok = cstar >= tgt + tolS && (first || cprev < tgt - tolS);
      s_i[1] = ok ? 1 : 0;
      s_g[0] = js;
      s_g[1] = js + 1;
      red_d[2 * NWAVE + 2] = key2d(gk[js]);
    }
    __syncthreads();
    if (!s_i[1]) return false;
    // the cut value's group: sorted positions [g0, g1), ascending ids
    {
      const uint64_t kj = gk[js];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = 4 * t + j;
        if (e < ng && gk[e] == kj) { atomicMin(&s_g[0], e); atomicMax(&s_g[1], e + 1); }
      }
    }
    __syncthreads();
    xcut = (float)red_d[2 * NWAVE + 2];
    g0 = s_g[0];
    gn = s_g[1] - g0;
    gj = js + 1 - g0;
    // the kept part of the cut bucket, per range: the entries above the cut
    // value and the group's survivors
    if (corr) {
      const double fb = deep_pow2(deep_scale(bs));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int e = 4 * t + j;
        if (e < g0 || (e < g0 + gn && spread_keeps(e - g0, gj, gn, V <= TIE_NET)))
          atomicAdd(s_corr + NWAVE + gi[e] / L, (unsigned long long)(qv[j] * fb));
      }
    }
    __syncthreads();
  }

  // kept: above the cut value, or in its group among the survivors (the
  // group's member of a given id found by bisection of its sorted ids);
  // with min-p, e >= min_p
  const double minp = P.min_p;
  const double minp_tol = 1e-12 * minp;
  const uint32_t kcut = f2key(xcut);
  auto in_group = [&](int id) -> bool {
    if (gj >= gn) return true;
    int lo = g0, hi = g0 + gn;
    while (lo < hi) {
      const int mid = (lo + hi) >> 1;
      if (gi[mid] < id) lo = mid + 1; else hi = mid;
    }
    return spread_keeps(lo - g0, gj, gn, V <= TIE_NET);
  };
  auto kept_e = [&](float x, int id, int& amb) -> double {
    const uint32_t kx = f2key(x);
    if (!(kx > kcut || (kx == kcut && in_group(id)))) return 0.0;
    const double ev = deep_term(x, M, invT, tab);
    if (minp > 0.0) {
      if (fabs(ev - minp) <= minp_tol) amb = 1;
      if (ev < minp) return 0.0;
    }
    return ev;
  };
  int amb = 0;
  // kept mass of ids [lo, hi) by one wave (hi - lo a multiple of 64 nv), in
  // a fixed order
  auto wave_mass = [&](int lo, int hi) -> double {
    double m = 0.0;
    const int n = hi > lo ? (hi - lo) / (64 * nv) : 0;
    deep_stream<VEC>(R, lo, 64 * nv, l, n, [&](int k, const uint32_t (&wd)[DW]) {
      const int e0 = lo + k * 64 * nv + nv * l;
#pragma unroll
      for (int j = 0; j < DNV; ++j) {
        if (j >= nv) break;
        if (e0 + j < V) m += kept_e(deep_val(R, wd, j), e0 + j, amb);
      }
    });
    return wave_sum(m);
  };

  // ---- each range's kept mass: from the copies (no min-p), or pass 3
  if (minp <= 0.0) {
    if (t < NWAVE) {
      const int cbs = cut ? bs / DCB : DNCB;          // coarse buckets wholly kept
      double m = 0.0;
      for (int cb = 0; cb < cbs; ++cb)
        m += C[t * DNCB + cb] - (t > 0 ? C[(t - 1) * DNCB + cb] : 0.0);
      if (cut)
        m += (double)s_corr[t] * deep_pow2(-deep_scale((bs / DCB) * DCB)) +
             (double)s_corr[NWAVE + t] * deep_pow2(-deep_scale(bs));
      s_wm[t] = m;
    }
    __syncthreads();
  } else {
    const double m = wave_mass(w * L, w * L + L);
    if (l == 0) s_wm[w] = m;
    if (block_max(amb, red_i, 0)) return false;      // an element at the min-p floor
  }
  double Z = 0.0;
  for (int k = 0; k < NWAVE; ++k) Z += s_wm[k];
  if (!(Z > 0.0)) return false;
  const double tolZ = DTOL * Z;
  const double t2 = A.u[row] * Z;
  // the wave range holding t2
  int wr = -1;
  double off = 0.0;
  {
    double o = 0.0;
    for (int k = 0; k < NWAVE && wr < 0; ++k) {
      if (o + s_wm[k] > t2) { wr = k; off = o; }
      o += s_wm[k];
    }
  }
  __syncthreads();
  if (wr < 0) return false;
  // its sixteenth held by each wave
  const int SL = L / NWAVE;
  {
    const double m = wave_mass(wr * L + w * SL, wr * L + (w + 1) * SL);
    if (l == 0) s_wm[w] = m;
  }
  __syncthreads();
  int sr = -1;
  {
    double o = off;
    for (int k = 0; k < NWAVE && sr < 0; ++k) {
      if (o + s_wm[k] > t2) { sr = k; off = o; }
      o += s_wm[k];
    }
  }
  // one wave scans the sixteenth in id order: the first element whose
  // running sum exceeds t2
  if (w == 0) {
    int found = INT_MAX;
    bool ok = false;
    if (sr >= 0) {
      const int lo = wr * L + sr * SL;
      double runw = off;
      for (int base = lo; base < lo + SL && found == INT_MAX; base += 64 * nv) {
        const int e0 = base + nv * l;
        uint32_t wd[DW];
        deep_fetch<VEC>(R, e0, wd);
        double q[DNV];
        double ls = 0.0;
#pragma unroll
        for (int j = 0; j < DNV; ++j) {
          q[j] = j < nv && e0 + j < V ? kept_e(deep_val(R, wd, j), e0 + j, amb) : 0.0;
          ls += q[j];
        }
        double incl = ls;
        for (int o = 1; o < 64; o <<= 1) {
          const double y = __shfl_up(incl, o);
          if (l >= o) incl += y;
        }
        double r = runw + (incl - ls);               // running sum before this lane's elements
        int hit = INT_MAX;
        bool hok = false;
#pragma unroll
        for (int j = 0; j < DNV; ++j) {
          const double ri = r + q[j];
          if (hit == INT_MAX && ri > t2) {
            hit = e0 + j;
            hok = ri > t2 + tolZ && r < t2 - tolZ;
          }
          r = ri;
        }
        found = wave_min(hit);
        if (found != INT_MAX) ok = ballot(hit == found && hok) != 0ull;
        runw += lane_read(incl, 63);
      }
    }
    if (l == 0) s_i[3] = (found != INT_MAX && ok) ? found : -1;
  }
  __syncthreads();
  const int tok = s_i[3];
  if (block_max(amb, red_i, 0) || tok < 0) return false;
  if (t == 0) {
    A.out_id[row] = tok;
    A.row_status[row] = CX_ROW_OK | CX_ROW_FLAG_SLOW | CX_ROW_FLAG_DEEP;
  }
  return true;
}

// The exact normaliser sum over the row's ids [lo, hi) (lo a multiple of
// 16384; the whole row by default) of exp((x - M) / T), in fp64 with the
// table-driven exp, for a row without a penalty window: the passes' stream
// (loads three steps ahead) instead of one load round trip per eight
// elements.  The same value on every thread.
template <bool VEC>
__device__ inline double deep_exact_sum_impl(const SampleArgs& A, int row, double M, double invT,
                                             double* red_d, int lo, int hi) {
  __shared__ double etab[64];
  load_exp64_tab(etab);
  // the row as far as hi: the loads the stream issues past hi return zeros
  // and read nothing (not the next share's logits)
  hi = min(hi, A.V);
  DeepRow R;
  R.V = hi;
  R.bf16 = A.bf16 != 0;
  R.nv = R.bf16 ? 16 : 8;
  R.step = R.nv * WG;
  R.p = (const char*)A.logits + (size_t)row * (size_t)A.ld * (R.bf16 ? 2 : 4);
  R.rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(R.p), (short)0,
                                           (R.V * (R.bf16 ? 2 : 4) + 15) & ~15, 0x00020000);
  const int t = threadIdx.x;
  // per step, the fetch's values as straight-line code (a loop bounded by
  // R.nv, with a break at hi, ran its exps one after another): four
  // accumulators, element j into j % 4, values at or past hi selected away
  double s[4] = {0.0, 0.0, 0.0, 0.0};
  deep_stream<VEC>(R, lo, R.step, t, (hi - lo + R.step - 1) / R.step,
                   [&](int k, const uint32_t (&wd)[DW]) {
    const int e0 = lo + k * R.step + R.nv * t;
    if (R.bf16) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float x = __uint_as_float((j & 1) ? (wd[j >> 1] & 0xFFFF0000u) : (wd[j >> 1] << 16));
        const double e = exp64_neg(((double)x - M) * invT, etab);
        s[j & 3] += e0 + j < hi ? e : 0.0;
      }
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const double e = exp64_neg(((double)__uint_as_float(wd[j]) - M) * invT, etab);
        s[j & 3] += e0 + j < hi ? e : 0.0;
      }
    }
  });
  return block_sum((s[0] + s[1]) + (s[2] + s[3]), red_d);
}
__device__ inline double deep_exact_sum(const SampleArgs& A, int row, double M, double invT,
                                        double* red_d, int lo = 0, int hi = INT_MAX) {
  return A.vec_ok ? deep_exact_sum_impl<true>(A, row, M, invT, red_d, lo, hi)
                  : deep_exact_sum_impl<false>(A, row, M, invT, red_d, lo, hi);
}

// Samples the row and returns true, or returns false with nothing written
// (the caller runs the multi-pass path).  All threads of the workgroup call
// it and get the same result.  dyn: DEEP_LDS bytes; red_d, red_i: >= 2 *
// NWAVE + 4 slots.
__device__ __forceinline__ bool deep_row(const SampleArgs& A, int row, unsigned char* dyn, double* red_d,
                                int* red_i) {
  const cx_row_params P = A.prm[row];
  double M = 0.0;
  if (!deep_eligible(A, row, P, M)) return false;
  return A.vec_ok ? deep_row_impl<true>(A, row, P, M, dyn, red_d, red_i)
                  : deep_row_impl<false>(A, row, P, M, dyn, red_d, red_i);
}

}  // namespace cx
