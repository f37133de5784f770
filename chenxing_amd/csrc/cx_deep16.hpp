// cx_deep16.hpp -- deep-nucleus rows of bf16 logits, by counting values.
//
// A bf16 row holds at most 65536 distinct values and equal values have equal
// terms, so the row's top-p cut follows from how often each value occurs.
// One workgroup per row (finish16_kernel), for the rows deep_eligible admits:
//   pass 1  every element's value counted in LDS: an ordered 16-bit key per
//           bf16 code, two 16-bit counters per word (the counts' total,
//           which a wrapped counter would lower, must equal V).  At the end
//           of each id range (the row split into NWAVE contiguous ranges)
//           the counters of the D16_WIN values below the maximum are copied.
//   cut     each value's mass, count x exp((x - M) / T) in fp64 (within the
//           bucket span below M; terms below it are left out, at most
//           V exp(-40) in all), summed from the top in value order: the
//           value v* at which the running mass reaches top_p * S and the
//           number j of its occurrences kept (sampler.py:81-89), spread
//           over their ids (spread_kept, cx_device.hpp)
//   top-k   the k-th largest element's value from the counts, every value
//           at or above it kept (sampler.py:76-79, ties included); top-p
//           cuts that set unrenormalised, so where its mass falls short of
//           top_p * S the whole set is kept
//   min-p   kept values are those whose term reaches min_p times the top
//           term, 1 (sampler.py:91-93)
//   ranges  per range, the kept mass above v* and the number of v*'s
//           occurrences, whose running count gives each range's share of
//           the j kept occurrences: from the copies when every kept value
//           lies in the copied window, else by a second pass over the row
//   draw    the range holding u * Z (Z the kept total), then its sixteenth
//           (each wave sums one), then one wave's scan of that sixteenth in
//           id order (sampler.py:126-127: choice == searchsorted(cumsum, u,
//           'right'))
// Per element the passes do one LDS atomic, resp. one table read: no exp.
// Sums run in a fixed order in fp64.  A decision closer to its threshold
// than DTOL of the total, or a wrapped counter, returns false with nothing
// written: the caller then takes the bucketed deep path.
#pragma once
#include "cx_deep.hpp"

namespace cx {

constexpr int D16_WORDS = 32768;                  // 65536 16-bit counters
constexpr int D16_TT = D16_WORDS * 4 / 8;         // fp64 term-table entries in the same LDS
static_assert(D16_WORDS * 4 <= FIN_CAP * 32, "deep16 LDS");
constexpr uint32_t D16_NEG_INF = 0x007Fu;         // key of -inf; keys below are NaN codes
constexpr int D16_WIN = 512;                      // values below the maximum copied per range
constexpr int D16_WW = D16_WIN / 2 + 1;           // counter words per copy

// The path's workgroup-shared state (one instance per kernel).
struct Deep16Shared {
  double tab[64];
  double s_d[2 * NWAVE + 4];
  double bm[WG];                                  // mass of each block of 64 keys
  double gt[NWAVE * NWAVE];                       // [range][wave]: kept mass above v* (pass 2)
  int eq[NWAVE * NWAVE];                          // [range][wave]: occurrences of v* (pass 2)
  uint32_t snap[NWAVE * D16_WW];                  // [range]: the window's counters at its end
  uint32_t snapk[NWAVE];                          // [range]: the running maximum's key there
  uint32_t wk[NWAVE];                             // per wave: its running maximum key
  double wm[NWAVE];
  int we[NWAVE];
  double cut[3];                                  // v*'s term; the cut was robust; mass above its block
  int ci[4];                                      // cut block, kc, jk, token
  int kq[2];                                      // top-k: the k-th largest's block, its key
  double kqd[3];                                  // count and mass above that block; mass at or above the key
};

// Key of a bf16 code, ascending in the value (-0 folded onto +0, so equal
// values share a key), and the value of a key.
__device__ __forceinline__ uint32_t d16_key(uint32_t code) {
  code = code == 0x8000u ? 0u : code;
  return (code & 0x8000u) ? (~code & 0xFFFFu) : (code | 0x8000u);
}
__device__ __forceinline__ float d16_val(uint32_t key) {
  const uint32_t code = (key & 0x8000u) ? (key & 0x7FFFu) : (~key & 0xFFFFu);
  return __uint_as_float(code << 16);
}
__device__ __forceinline__ uint32_t d16_half(uint32_t word, uint32_t key) {
  return (word >> ((key & 1u) << 4)) & 0xFFFFu;
}
__device__ __forceinline__ uint32_t d16_count(const uint32_t* cw, uint32_t key) {
  return d16_half(cw[key >> 1], key);
}

// The counter word of the first key of the copied window below key k (the
// window holds keys k - D16_WIN + 1 .. k, from that word on).
__device__ __forceinline__ uint32_t d16_win0(uint32_t k) {
  return k >= (uint32_t)(D16_WIN - 1) ? (k - (D16_WIN - 1)) >> 1 : 0u;
}

template <bool VEC>
__device__ inline bool deep16_row_impl(const SampleArgs& A, int row, const cx_row_params& P,
                                       unsigned char* dyn, double* red_d, int* red_i,
                                       Deep16Shared& sh) {
  const int t = threadIdx.x, l = lane_id(), w = wave_id();
  DeepRow R;
  R.V = A.V;
  R.bf16 = true;
  R.nv = 16;
  R.step = 16 * WG;
  R.p = (const char*)A.logits + (size_t)row * (size_t)A.ld * 2;
  R.rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(R.p), (short)0,
                                           (R.V * 2 + 15) & ~15, 0x00020000);
  const int V = R.V;
  const double invT = 1.0 / P.temperature;
  const int L = ((V + NWAVE * R.step - 1) / (NWAVE * R.step)) * R.step;
  const int nsteps = (V + R.step - 1) / R.step;
  const double* tab = sh.tab;

  uint32_t* cw = (uint32_t*)dyn;
  for (int i = t; i < D16_WORDS; i += WG) cw[i] = 0u;
  for (int i = t; i < NWAVE * NWAVE; i += WG) { sh.gt[i] = 0.0; sh.eq[i] = 0; }
  if (t == 0) { sh.ci[0] = INT_MAX; sh.cut[1] = 0.0; sh.kq[0] = -1; sh.kq[1] = 0; }
  load_exp64_tab(sh.tab);                            // its barrier also orders the clears

  // ---- pass 1: count every value (-inf, a masked token, in a register:
  // masks of more than 65535 ids are common) and find the maximum (the row
  // is not streamed before); at each range's end copy the D16_WIN values
  // below the running maximum.  That covers the final window for every
  // range: the final maximum kM is at least range r's running maximum kr,
  // so the final window starts no lower than r's copy, and a key above kr
  // has no occurrence up to range r's end.
  int ninf = 0;
  uint32_t kmax = 0u;                                // largest key seen: a finite value's or +inf's when any
  deep_stream<VEC>(R, 0, R.step, t, nsteps, [&](int k, const uint32_t (&wd)[DW]) {
    const int e0 = k * R.step + 16 * t;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if (e0 + j < V) {
        const uint32_t key = d16_key(deep_code(wd, j));
        if (key == D16_NEG_INF) ++ninf;
        else atomicAdd(cw + (key >> 1), 1u << ((key & 1u) << 4));
        kmax = key > kmax ? key : kmax;                // (-inf and NaN keys lie below)
      }
    }
    if ((k + 1) * R.step % L == 0 || k + 1 == nsteps) {
      const uint32_t wmax = wave_reduce(kmax, OpMax());
      if (l == 0) sh.wk[w] = wmax;
      __syncthreads();
      uint32_t kr = 0u;
#pragma unroll
      for (int i = 0; i < NWAVE; ++i) kr = sh.wk[i] > kr ? sh.wk[i] : kr;
      const int r = (k * R.step) / L;
      const uint32_t w0 = d16_win0(kr);
      if (t <= (int)((kr >> 1) - w0)) {
        const uint32_t v = cw[w0 + t];
        for (int rr = r; rr < (k + 1 == nsteps ? NWAVE : r + 1); ++rr) sh.snap[rr * D16_WW + t] = v;
      }
      if (t == 0)
        for (int rr = r; rr < (k + 1 == nsteps ? NWAVE : r + 1); ++rr) sh.snapk[rr] = kr;
      __syncthreads();
    }
  });
  ninf = block_sum(ninf, red_i);                     // (its barriers publish snapk)
  // the row's maximum, recorded for the paths that may take the row after
  // this one (the fused kernel did not stream a counted row)
  const uint32_t kM = sh.snapk[NWAVE - 1];
  const double M = kM > D16_NEG_INF ? (double)d16_val(kM) : -__builtin_inf();
  if (t < A.nsplit) A.stats[(size_t)row * A.nsplit + t].m = M;
  if (!(M > -__builtin_inf()) || !(M < __builtin_inf())) return false;
  // the final copied window: counter words kw0 .. kM >> 1
  const uint32_t kw0 = d16_win0(kM);
  // term of a key: 0 below the span (and for -inf)
  auto term = [&](uint32_t key) -> double {
    const double d = (M - (double)d16_val(key)) * invT;
    return d < (double)DSPAN ? exp64_neg(-d, tab) : 0.0;
  };

  // ---- masses of the WG blocks of 64 keys, block b holding keys
  // 65535 - 64 b - l (lane l): descending value in (b, l).  Wave w takes
  // blocks w, w + NWAVE, ... (neighbouring values spread over the waves),
  // a lane a key; a block without counts costs a read and a ballot.
  int n64 = 0, badk = 0;
  for (int q = 0; q < WG / NWAVE; ++q) {
    const int b = w + NWAVE * q;
    const uint32_t key = 65535u - (uint32_t)(64 * b + l);
    const uint32_t n = d16_count(cw, key);
    n64 += (int)n;
    double m = 0.0;
    if (ballot(n != 0u)) {
      if (n) {
        if (key > kM || key < D16_NEG_INF) badk = 1;   // NaN, or a value above M
        else m = (double)n * term(key);
      }
      m = wave_sum(m);
    }
    if (l == 0) sh.bm[b] = m;
  }
  if (block_sum(n64, red_i) + ninf != V) return false;   // a counter wrapped
  if (block_max(badk, red_i, 0)) return false;         // (its barrier publishes bm)
  const double c64 = sh.bm[t];                          // thread t: block t
  const double S = block_sum(c64, sh.s_d);
  if (!(S > 0.0) || !(S < __builtin_inf())) return false;

  // the lowest key inside the span (kept values lie at or above it)
  uint32_t kspan;
  {
    uint32_t lo = D16_NEG_INF + 1, hi = kM;          // kM is inside
    while (lo < hi) {
      const uint32_t mid = (lo + hi) >> 1;
      if ((M - (double)d16_val(mid)) * invT < (double)DSPAN) hi = mid; else lo = mid + 1;
    }
    kspan = lo;
  }
  // top-k (sampler.py:76-79): every value at or above the k-th largest
  // element's is kept, ties included.  kk is that value's key (0: no top-k
  // bound, as when fewer than k values are finite).  Top-p then cuts the
  // post-top-k vector, unrenormalised: where the mass at or above kk clearly
  // falls short of top_p * S the whole top-k set is kept, otherwise the
  // row's cut lies at or above kk, or it is handed back.
  uint32_t kk = 0u;
  bool topk_all = false;
  if (P.top_k > 0 && P.top_k < V) {
    int nb = 0;                                        // block t's count: its 32 counter words
    const uint32_t* bw = cw + (32736 - 32 * t);
    for (int i = 0; i < 32; ++i) nb += (int)((bw[i] & 0xFFFFu) + (bw[i] >> 16));
    const double cbefore = block_excl_scan_d((double)nb, sh.s_d);
    const double mbefore = block_excl_scan_d(c64, sh.s_d);
    const double k = (double)P.top_k;
    if (cbefore < k && cbefore + (double)nb >= k) {
      sh.kq[0] = t;
      sh.kqd[0] = cbefore;
      sh.kqd[1] = mbefore;
    }
    __syncthreads();
    const int kb = sh.kq[0];
    if (kb >= 0) {
      if (w == 0) {
        // the block's keys in descending value: running counts and masses
        const uint32_t key = 65535u - (uint32_t)(64 * kb + l);
        const uint32_t n = d16_count(cw, key);
        const double m = n ? (double)n * term(key) : 0.0;
        double cin = (double)n, min_ = m;
        for (int o = 1; o < 64; o <<= 1) {
          const double yc = __shfl_up(cin, o), ym = __shfl_up(min_, o);
          if (l >= o) { cin += yc; min_ += ym; }
        }
        const uint64_t hit = ballot(sh.kqd[0] + cin >= k);
        if (hit && l == __builtin_ctzll(hit)) {
          sh.kq[1] = (int)key;
          sh.kqd[2] = sh.kqd[1] + min_;
        }
      }
      __syncthreads();
      kk = (uint32_t)sh.kq[1];
      topk_all = !(P.top_p < 1.0) || sh.kqd[2] < P.top_p * S - DTOL * S;
    }
  }
  // kept: key > kc, or key == kc among the jk of its cntc occurrences that survive
  uint32_t kc = kspan - 1;
  int jk = 0;
  double termc = 0.0;
  if (P.top_p < 1.0 && !topk_all) {
    const double tgt = P.top_p * S;
    const double tolS = DTOL * S;
    const double before = block_excl_scan_d(c64, sh.s_d);
    // the block holding the cut (the first, should rounding let two claim)
    if (before < tgt && before + c64 >= tgt) atomicMin(sh.ci, t);
    __syncthreads();
    const int cb = sh.ci[0];
    if (cb == INT_MAX) return false;                 // the cut lies below the span
    if (t == cb) sh.cut[2] = before;
    __syncthreads();
    if (w == 0) {
      // the block's keys, one per lane in descending value: running masses
      const uint32_t key = 65535u - (uint32_t)(64 * cb + l);
      const uint32_t n = d16_count(cw, key);
      const double te = n ? term(key) : 0.0;
      const double m = (double)n * te;
      double incl = m;
      for (int o = 1; o < 64; o <<= 1) {
        const double y = __shfl_up(incl, o);
        if (l >= o) incl += y;
      }
      const double run = sh.cut[2] + (incl - m);    // mass above this lane's key
      const uint64_t hit = ballot(te > 0.0 && run + m >= tgt);
      if (hit && l == __builtin_ctzll(hit)) {
        int j = (int)__builtin_ceil((tgt - run) / te);
        j = j < 1 ? 1 : (j > (int)n ? (int)n : j);
        // robust: the j-th occurrence clearly reaches the target and the
        // element before it clearly does not (the first element is kept)
        const bool first = key == kM && j == 1;
        const bool ok = run + (double)j * te >= tgt + tolS &&
                        (first || run + (double)(j - 1) * te < tgt - tolS);
        sh.ci[1] = (int)key;
        sh.ci[2] = j;
        sh.cut[0] = te;
        sh.cut[1] = ok ? 1.0 : 0.0;
      }
    }
    __syncthreads();
    if (sh.cut[1] == 0.0) return false;
    kc = (uint32_t)sh.ci[1];
    jk = sh.ci[2];
    termc = sh.cut[0];
  }
  if (kc < kk) { kc = kk - 1; jk = 0; termc = 0.0; }   // the top-k bound
  if (P.min_p > 0.0) {
    // the lowest key whose term reaches min_p (the top term is 1)
    const double minp = P.min_p, mtol = 1e-12 * minp;
    uint32_t lo = kspan, hi = kM;
    while (lo < hi) {
      const uint32_t mid = (lo + hi) >> 1;
      if (term(mid) >= minp) hi = mid; else lo = mid + 1;
    }
    if (fabs(term(lo) - minp) <= mtol || (lo > kspan && fabs(term(lo - 1) - minp) <= mtol))
      return false;                                  // a value at the min-p floor
    if (lo > kc) { kc = lo - 1; jk = 0; termc = 0.0; }
  }
  const int cntc = kc == D16_NEG_INF ? ninf : (int)d16_count(cw, kc);
  // terms of the kept values above kc, over the counters: a table by key
  // when it fits, else the three part tables of every bf16 code (a kept
  // range through zero holds the many codes of tiny values)
  const int ntt = (int)(kM - kc);
  const bool dense = ntt <= D16_TT;
  const bool copied = kc >= kw0 * 2u;                // kc and every kept value in the window
  if (!dense && !((fabs(M) + (double)DSPAN * P.temperature) * invT < 7000.0)) return false;
  __syncthreads();                                   // every read of the counters done
  double* tt = (double*)dyn;                         // dense: term of key kc + 1 + i
  double* ta = (double*)dyn;
  double* tb = ta + 4096;
  double* tc = tb + 2048;
  if (dense) {
    for (int i = t; i < ntt; i += WG) tt[i] = term(kc + 1 + (uint32_t)i);
  } else {
    deep_build_tables(ta, tb, tc, M, invT, tab);
  }
  __syncthreads();
  auto kept_term = [&](uint32_t key, uint32_t code) -> double {
    return dense ? tt[key - kc - 1] : deep_term16(code, ta, tb, tc);
  };

  if (copied) {
    // ---- per range, from the copies: wave r takes range r (its counts are
    // the differences of consecutive copies), a lane every 64th kept value
    if (w < NWAVE) {
      // range w's counts: the differences of consecutive copies, each read
      // in its own window (a key above a copy's running maximum has no
      // occurrence there yet)
      const uint32_t* cur = sh.snap + w * D16_WW;
      const uint32_t* prv = w > 0 ? cur - D16_WW : nullptr;
      const uint32_t kc_ = sh.snapk[w], kp_ = w > 0 ? sh.snapk[w - 1] : 0u;
      const uint32_t wc = d16_win0(kc_), wp = d16_win0(kp_);
      auto cnt = [&](uint32_t key) -> int {
        const int a = key <= kc_ ? (int)d16_half(cur[(key >> 1) - wc], key) : 0;
        const int b = prv && key <= kp_ ? (int)d16_half(prv[(key >> 1) - wp], key) : 0;
        return a - b;
      };
      double m = 0.0;
      for (int i = l; i < ntt; i += 64) m += (double)cnt(kc + 1 + (uint32_t)i) * tt[i];
      m = wave_sum(m);
      if (l == 0) {
        sh.wm[w] = m;
        sh.we[w] = cnt(kc);
      }
    }
  } else {
    // ---- pass 2: per range and wave, the kept mass above kc and kc's
    // count (four accumulators, element j into j % 4: shorter add chains,
    // the same order every time)
    double acc[4] = {0.0, 0.0, 0.0, 0.0};
    int ce = 0;
    deep_stream<VEC>(R, 0, R.step, t, nsteps, [&](int k, const uint32_t (&wd)[DW]) {
      const int e0 = k * R.step + 16 * t;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if (e0 + j < V) {
          const uint32_t code = deep_code(wd, j);
          const uint32_t key = d16_key(code);
          if (key > kc) acc[j & 3] += kept_term(key, code);
          else if (key == kc) ++ce;
        }
      }
      if ((k + 1) * R.step % L == 0 || k + 1 == nsteps) {
        const double m = wave_sum((acc[0] + acc[1]) + (acc[2] + acc[3]));
        const int c = wave_sum(ce);
        if (l == 0) {
          sh.gt[((k * R.step) / L) * NWAVE + w] = m;
          sh.eq[((k * R.step) / L) * NWAVE + w] = c;
        }
        acc[0] = acc[1] = acc[2] = acc[3] = 0.0;
        ce = 0;
      }
    });
    __syncthreads();
    // per range: kept mass and v*'s count, in a fixed order
    if (t < NWAVE) {
      double m = 0.0;
      int c = 0;
      for (int k = 0; k < NWAVE; ++k) { m += sh.gt[t * NWAVE + k]; c += sh.eq[t * NWAVE + k]; }
      sh.wm[t] = m;
      sh.we[t] = c;
    }
  }
  __syncthreads();
  // v*'s kept occurrences in the id ranges: of its cntc occurrences jk are
  // kept, spread over their ids -- the first R hold spread_kept(R) of them
  auto kept_between = [&](int r0, int r1) -> int {
    return (int)(spread_kept(r1, jk, cntc, V <= TIE_NET) - spread_kept(r0, jk, cntc, V <= TIE_NET));
  };
  double Z = 0.0;
  {
    int call = 0;
    for (int k = 0; k < NWAVE; ++k) {
      Z += sh.wm[k] + (double)kept_between(call, call + sh.we[k]) * termc;
      call += sh.we[k];
    }
    if (call != cntc) return false;                  // (cannot happen: the passes agree)
  }
  if (!(Z > 0.0)) return false;
  const double tolZ = DTOL * Z;
  const double t2 = A.u[row] * Z;
  // the range holding t2, and the occurrences of v* before it
  int wr = -1, baser = 0;
  double off = 0.0;
  {
    double o = 0.0;
    int before = 0;
    for (int k = 0; k < NWAVE && wr < 0; ++k) {
      const double m = sh.wm[k] + (double)kept_between(before, before + sh.we[k]) * termc;
      if (o + m > t2) { wr = k; off = o; baser = before; }
      o += m;
      before += sh.we[k];
    }
  }
  __syncthreads();
  if (wr < 0) return false;
  // ---- its sixteenths, one per wave
  const int SL = L / NWAVE;
  {
    const int lo = wr * L + w * SL;
    double ma[4] = {0.0, 0.0, 0.0, 0.0};
    int c = 0;
    deep_stream<VEC>(R, lo, 64 * 16, l, SL / (64 * 16), [&](int k, const uint32_t (&wd)[DW]) {
      const int e0 = lo + k * 64 * 16 + 16 * l;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if (e0 + j < V) {
          const uint32_t code = deep_code(wd, j);
          const uint32_t key = d16_key(code);
          if (key > kc) ma[j & 3] += kept_term(key, code);
          else if (key == kc) ++c;
        }
      }
    });
    const double m = wave_sum((ma[0] + ma[1]) + (ma[2] + ma[3]));
    c = wave_sum(c);
    if (l == 0) { sh.wm[w] = m; sh.we[w] = c; }
  }
  __syncthreads();
  int sr = -1, bases = 0;
  {
    double o = off;
    int before = baser;
    for (int k = 0; k < NWAVE && sr < 0; ++k) {
      const double m = sh.wm[k] + (double)kept_between(before, before + sh.we[k]) * termc;
      if (o + m > t2) { sr = k; off = o; bases = before; }
      o += m;
      before += sh.we[k];
    }
  }
  // ---- one wave scans the sixteenth in id order: the first element whose
  // running sum exceeds t2
  if (w == 0) {
    int found = INT_MAX;
    bool ok = false;
    if (sr >= 0) {
      const int lo = wr * L + sr * SL;
      double runw = off;
      int eqw = 0;                                   // occurrences of v* before this block
      for (int base = lo; base < lo + SL && found == INT_MAX; base += 64 * 16) {
        const int e0 = base + 16 * l;
        uint32_t wd[DW];
        deep_fetch<VEC>(R, e0, wd);
        int ne = 0;
#pragma unroll
        for (int j = 0; j < 16; ++j) ne += e0 + j < V && d16_key(deep_code(wd, j)) == kc ? 1 : 0;
        int ie = ne;                                 // inclusive count of v* over the lanes
        for (int o = 1; o < 64; o <<= 1) {
          const int y = __shfl_up(ie, o);
          if (l >= o) ie += y;
        }
        // occurrences of v* before this lane's, as the spread remainder
        int rem = spread_rem(bases + eqw + ie - ne, jk, cntc, V <= TIE_NET);
        double q[16];
        double ls = 0.0;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          double v = 0.0;
          if (e0 + j < V) {
            const uint32_t code = deep_code(wd, j);
            const uint32_t key = d16_key(code);
            if (key > kc) v = kept_term(key, code);
            else if (key == kc) v = spread_step(rem, jk, cntc, V <= TIE_NET) ? termc : 0.0;
          }
          q[j] = v;
          ls += v;
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
        for (int j = 0; j < 16; ++j) {
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
        eqw += lane_read(ie, 63);
      }
    }
    if (l == 0) sh.ci[3] = (found != INT_MAX && ok) ? found : -1;
  }
  __syncthreads();
  const int tok = sh.ci[3];
  if (tok < 0) return false;
  if (t == 0) {
    A.out_id[row] = tok;
    A.row_status[row] = CX_ROW_OK | CX_ROW_FLAG_SLOW | CX_ROW_FLAG_DEEP;
  }
  return true;
}

// Samples a bf16 row that deep_eligible admits by counting its values and
// returns true, or returns false with nothing written (the caller takes the
// bucketed deep path).  All threads of the workgroup call it and get the
// same result.  dyn: FIN_CAP * 32 bytes; red_d, red_i: >= 2 * NWAVE + 4
// slots; sh: the kernel's one Deep16Shared.
__device__ inline bool deep16_row(const SampleArgs& A, int row, unsigned char* dyn, double* red_d,
                                  int* red_i, Deep16Shared& sh) {
  if (!A.bf16) return false;
  const cx_row_params P = A.prm[row];
  if (!deep_candidate(A, row, P, true)) return false;     // (top-k rows too)
  return A.vec_ok ? deep16_row_impl<true>(A, row, P, dyn, red_d, red_i, sh)
                  : deep16_row_impl<false>(A, row, P, dyn, red_d, red_i, sh);
}

}  // namespace cx
