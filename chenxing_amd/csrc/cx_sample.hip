// cx_sample.hip -- fused sampler for gfx950 (reference chenxing/core/sampler.py:63-127).
//
// One launch samples a whole batch.  The grid is B x nsplit workgroups of
// 1024 threads; workgroup (row, s) streams the contiguous slice s of row
// `row` exactly once from HBM with 16-byte nontemporal loads and produces:
//
//   * the penalised maximum and the temperature-scaled normaliser of its
//     slice (online max / sum-exp, fp32 exp2 terms accumulated in fp64),
//     or, for greedy rows, the first argmax;
//   * an exact "region": every element of the slice whose value is >= a
//     threshold tau, collected in per-wave LDS buffers.  Each wave keeps its
//     own threshold, raised by a wave-local radix select whenever its
//     buffer fills, so the hot loop has no workgroup barriers;
//   * the penalised values of its history ids.  Penalties touch only ids in
//     the history window, so the loop tests a bitmap in LDS (one ds_read per
//     16-byte vector) and parks flagged elements; they are re-scored in fp64
//     afterwards from an LDS hash table of (id, count).
//
// The last workgroup of a row to finish (agent-scope counter) runs
// finish_row (cx_finish.hpp).  Rows it cannot decide are marked pending and
// finished by the multi-pass kernel in cx_slow.hip.
#include "cx_device.hpp"
#include "cx_sampler.h"
#include "cx_internal.hpp"
#include "cx_finish.hpp"

namespace cx {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------ penalties
__device__ __forceinline__ uint32_t hash_slot(int id, int ns_log2) {
  return ((uint32_t)id * 0x9E3779B1u) >> (32 - ns_log2);
}

// Insert one window id into the LDS table of (id << 12 | count) words.
__device__ __forceinline__ void hash_insert(uint32_t* hkey, int ns_log2, int id) {
  const uint32_t mask = (1u << ns_log2) - 1;
  uint32_t s = hash_slot(id, ns_log2);
  for (;;) {
    uint32_t old = atomicCAS(&hkey[s], HEMPTY, ((uint32_t)id << 12) | 1u);
    if (old == HEMPTY) return;
    if ((old >> 12) == (uint32_t)id) { atomicAdd(&hkey[s], 1u); return; }
    s = (s + 1) & mask;
  }
}

__device__ __forceinline__ int hash_find(const uint32_t* hkey, int ns_log2, int id) {
  const uint32_t mask = (1u << ns_log2) - 1;
  uint32_t s = hash_slot(id, ns_log2);
  for (;;) {
    uint32_t k = hkey[s];
    if (k == HEMPTY) return -1;
    if ((k >> 12) == (uint32_t)id) return (int)s;
    s = (s + 1) & mask;
  }
}

// Bitmap + hash table for the window ids that fall in [lo, hi)
// (sampler.py:67-68: window of the last max(64, n_keep) ids, out-of-range ids dropped).
__device__ inline void build_penalty_tables(const int32_t* hrow, int wstart, int wlen, int lo,
                                            int hi, uint32_t* bitmap, int nbw, uint32_t* hkey,
                                            int ns, int ns_log2) {
  for (int i = threadIdx.x; i < nbw; i += WG) bitmap[i] = 0u;
  for (int i = threadIdx.x; i < ns; i += WG) hkey[i] = HEMPTY;
  __syncthreads();
  for (int i = threadIdx.x; i < wlen; i += WG) {
    int id = hrow[wstart + i];
    if (id >= lo && id < hi) {
      int r = id - lo;
      atomicOr(&bitmap[(r >> 5) & (nbw - 1)], 1u << (r & 31));
      hash_insert(hkey, ns_log2, id);
    }
  }
  __syncthreads();
}

// fp64 penalised value of a history id: sampler.py:70-72, then the
// presence/frequency extension (identity when both are 0).
__device__ __forceinline__ double penalise(float raw, int cnt, const cx_row_params& p) {
  double x = (double)raw;
  if (p.repetition_penalty != 1.0)
    x = x > 0.0 ? x / p.repetition_penalty : x * p.repetition_penalty;
  x = x - p.frequency_penalty * (double)cnt;
  x = x - p.presence_penalty;
  return x;
}

// ------------------------------------------------------------ loads
template <bool BF16> struct Elem;
template <> struct Elem<false> {
  static constexpr int NE = 4;
  using V = f32x4;
  __device__ static __forceinline__ void unpack(const V& q, float (&x)[NE]) {
    x[0] = q.x; x[1] = q.y; x[2] = q.z; x[3] = q.w;
  }
  __device__ static __forceinline__ float scalar(const void* row, int64_t e) {
    return ((const float*)row)[e];
  }
};
template <> struct Elem<true> {
  static constexpr int NE = 8;
  using V = u32x4;
  __device__ static __forceinline__ void unpack(const V& q, float (&x)[NE]) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      x[2 * j] = __uint_as_float(w[j] << 16);
      x[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
  }
  __device__ static __forceinline__ float scalar(const void* row, int64_t e) {
    return __uint_as_float((uint32_t)((const uint16_t*)row)[e] << 16);
  }
};

// ------------------------------------------------------------ wave candidates
// Wave-uniform state: every lane holds the same n / tau / overflow, and every
// update is made by all 64 lanes from ballots.
struct WaveBuf {
  uint32_t* key;
  int32_t* idx;
  int n;
  uint32_t tau;   // every element seen so far with key >= tau is in the buffer
  int kw;         // entries a compaction keeps
  bool overflow;
};

// Raise tau to the kw-th largest key held (bitwise radix select over the
// buffer with ballot counts) and drop the entries below it.
__device__ __noinline__ void wave_compact(WaveBuf& w) {
  constexpr int PER = CAPW / 64;
  const int l = lane_id();
  uint32_t k[PER];
  int32_t id[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    int pos = l + 64 * e;
    k[e] = pos < w.n ? w.key[pos] : 0u;
    id[e] = pos < w.n ? w.idx[pos] : 0;
  }
  uint32_t prefix = 0;
  for (int bit = 31; bit >= 0; --bit) {
    uint32_t cand = prefix | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int e = 0; e < PER; ++e) cnt += __popcll(ballot(k[e] >= cand));
    if (cnt >= w.kw) prefix = cand;
  }
  if (prefix > w.tau) w.tau = prefix;
  int n = 0;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    bool keep = k[e] >= w.tau && k[e] != 0u;
    uint64_t b = ballot(keep);
    if (keep) {
      int p = n + lanes_below(b);
      w.key[p] = k[e];
      w.idx[p] = id[e];
    }
    n += __popcll(b);
  }
  w.n = n;
}

template <int NE>
__device__ __forceinline__ void wave_insert(WaveBuf& w, const uint32_t (&key)[NE], int64_t e0) {
#pragma unroll
  for (int j = 0; j < NE; ++j) {
    bool p = key[j] >= w.tau;
    uint64_t b = ballot(p);
    if (b == 0) continue;
    int c = __popcll(b);
    if (w.n + c > CAPW) {
      wave_compact(w);
      p = key[j] >= w.tau;
      b = ballot(p);
      c = __popcll(b);
      if (w.n + c > CAPW) { w.overflow = true; continue; }
    }
    if (p) {
      int pos = w.n + lanes_below(b);
      w.key[pos] = key[j];
      w.idx[pos] = (int32_t)(e0 + j);
    }
    w.n += c;
  }
}

// ------------------------------------------------------------ per-thread stream state
struct StochState {
  float m;     // running max of unparked values
  double s;    // sum of exp2((x - m) * c), c = log2(e) / T
};
struct GreedyState {
  float bv;
  int bi;
  int nan_i;
};

// One 16-byte vector (or one scalar, NE == 1).  Called by all 64 lanes of
// the wave; `valid` is false for lanes past the end of the slice.
template <int NE, bool GREEDY>
__device__ __forceinline__ void process_vec(const float (&xin)[NE], int64_t e0, bool valid,
                                            int lo, bool has_pen, const uint32_t* bitmap,
                                            int nbw, const uint32_t* hkey, float* hval,
                                            int ns_log2, float c, StochState& st,
                                            GreedyState& gs, WaveBuf& wb) {
  uint32_t parked = valid ? 0u : 0xFFu;
  if (has_pen && valid) {
    int r = (int)(e0 - lo);
    uint32_t word = bitmap[(r >> 5) & (nbw - 1)];
    uint32_t bits = (word >> (r & 31)) & ((1u << NE) - 1u);
    if (bits) {
#pragma unroll
      for (int j = 0; j < NE; ++j)
        if (bits & (1u << j)) {
          int sl = hash_find(hkey, ns_log2, (int)(e0 + j));
          if (sl >= 0) { hval[sl] = xin[j]; parked |= 1u << j; }
        }
    }
  }
  if (GREEDY) {
#pragma unroll
    for (int j = 0; j < NE; ++j) {
      if (parked & (1u << j)) continue;
      float x = xin[j];
      if (x > gs.bv) { gs.bv = x; gs.bi = (int)(e0 + j); }
      if (x != x && gs.nan_i == INT_MAX) gs.nan_i = (int)(e0 + j);
    }
    return;
  }
  float x[NE];
  float vmax = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < NE; ++j) {
    x[j] = (parked & (1u << j)) ? -__builtin_inff() : xin[j];
    vmax = fmaxf(vmax, x[j]);
  }
  if (vmax > st.m) {
    if (st.s != 0.0) st.s *= exp2((double)(st.m - vmax) * (double)c);
    st.m = vmax;
  }
  const float mm = fmaxf(st.m, -3.402823466e38f);
  float tsum = 0.f;
  uint32_t key[NE];
  uint32_t kmax = 0;
#pragma unroll
  for (int j = 0; j < NE; ++j) {
    tsum += __builtin_amdgcn_exp2f((x[j] - mm) * c);
    key[j] = (parked & (1u << j)) ? 0u : f2key(x[j]);
    kmax = key[j] > kmax ? key[j] : kmax;
  }
  st.s += (double)tsum;
  if (ballot(kmax >= wb.tau)) wave_insert<NE>(wb, key, e0);
}

// ------------------------------------------------------------ the kernel
template <bool BF16>
__global__ __launch_bounds__(WG) void sample_kernel(SampleArgs A) {
  using E = Elem<BF16>;
  constexpr int NE = E::NE;
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ double red_d[2 * NWAVE + 4];
  __shared__ int red_i[2 * NWAVE + 4];
  __shared__ uint32_t w_tau[NWAVE];
  __shared__ int w_n[NWAVE];
  __shared__ int w_ovf[NWAVE];
  __shared__ int s_cnt;
  __shared__ int s_last;

  const int row = blockIdx.x / A.nsplit;
  const int split = blockIdx.x % A.nsplit;
  const int t = threadIdx.x;
  const cx_row_params P = A.prm[row];
  const bool greedy = P.temperature == 0.0;
  const int lo = split * A.split_len;
  const int hi = min(A.V, lo + A.split_len);
  const char* rowp = (const char*)A.logits + (size_t)row * (size_t)A.ld * (BF16 ? 2 : 4);

  int wlen = 0, wstart = 0;
  if (A.ldh > 0) {
    int len = max(0, min(A.hist_len[row], (int)A.ldh));
    wstart = P.n_keep > 0 ? max(0, len - max(64, P.n_keep)) : 0;
    wlen = len - wstart;
  }
  const bool pen_on = wlen > 0 && (P.repetition_penalty != 1.0 || P.presence_penalty != 0.0 ||
                                   P.frequency_penalty != 0.0);
  SplitStats* my = A.stats + (size_t)row * A.nsplit + split;
  Cand* mycand = A.cands + ((size_t)row * A.nsplit + split) * CAPS;

  if (pen_on && wlen > WIN_MAX) {                    // window longer than the LDS table
    if (t == 0) {
      my->flags = SF_UNSUPPORTED; my->ncand = 0; my->tau = 1u;
      my->m = 0; my->s = 0; my->best_i = INT_MAX; my->nan_i = INT_MAX;
    }
  } else {
    uint32_t* bitmap = (uint32_t*)(dyn + A.off_bitmap);
    uint32_t* hkey = (uint32_t*)(dyn + A.off_hkey);
    float* hval = (float*)(dyn + A.off_hval);
    if (pen_on)
      build_penalty_tables(A.hist + (size_t)row * A.ldh, wstart, wlen, lo, hi, bitmap, A.nbw,
                           hkey, A.ns, A.ns_log2);

    WaveBuf wb;
    wb.key = (uint32_t*)(dyn + A.off_wkey) + wave_id() * CAPW;
    wb.idx = (int32_t*)(dyn + A.off_widx) + wave_id() * CAPW;
    wb.n = 0;
    wb.tau = 1u;
    wb.overflow = false;
    // Entries a wave keeps: k for top-k rows; otherwise an equal share of the
    // finisher's sort capacity, so the merged region fits in LDS.
    const int share = max(8, min(KW_MAX, SORT_CAP / (NWAVE * A.nsplit)));
    wb.kw = P.top_k > 0 ? min(P.top_k, KW_MAX) : share;

    const float c = (float)(1.4426950408889634 / (greedy ? 1.0 : P.temperature));
    StochState st{-__builtin_inff(), 0.0};
    GreedyState gs{-__builtin_inff(), INT_MAX, INT_MAX};

    // ---- the slice: aligned 16-byte vectors, then a scalar tail
    const int64_t v0 = A.vec_ok ? lo / NE : 0;
    const int64_t v1 = A.vec_ok ? hi / NE : 0;
    const typename E::V* vp = (const typename E::V*)rowp;
    constexpr int U = BF16 ? 2 : 4;
    for (int64_t base = v0 + t; base - t < v1; base += (int64_t)U * WG) {
      typename E::V q[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int64_t vi = base + (int64_t)u * WG;
        if (vi < v1) q[u] = __builtin_nontemporal_load(&vp[vi]);
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int64_t vi = base + (int64_t)u * WG;
        if (vi - t >= v1) break;                       // uniform: no lane of the wave left
        bool valid = vi < v1;
        float x[NE];
        if (valid) E::unpack(q[u], x);
        else
#pragma unroll
          for (int j = 0; j < NE; ++j) x[j] = -__builtin_inff();
        if (greedy)
          process_vec<NE, true>(x, vi * NE, valid, lo, pen_on, bitmap, A.nbw, hkey, hval,
                                A.ns_log2, c, st, gs, wb);
        else
          process_vec<NE, false>(x, vi * NE, valid, lo, pen_on, bitmap, A.nbw, hkey, hval,
                                 A.ns_log2, c, st, gs, wb);
      }
    }
    {   // scalar elements: [lo, hi) for unaligned rows, else the tail past v1*NE
      const int64_t s0 = A.vec_ok ? (v1 * NE > lo ? v1 * NE : lo) : lo;
      for (int64_t e = s0 + t; e - t < hi; e += WG) {
        bool valid = e < hi;
        float x1[1] = {valid ? E::scalar(rowp, e) : -__builtin_inff()};
        if (greedy)
          process_vec<1, true>(x1, e, valid, lo, pen_on, bitmap, A.nbw, hkey, hval, A.ns_log2,
                               c, st, gs, wb);
        else
          process_vec<1, false>(x1, e, valid, lo, pen_on, bitmap, A.nbw, hkey, hval, A.ns_log2,
                                c, st, gs, wb);
      }
    }

    // Final compaction: each buffer becomes exactly its wave's top-kw (+ ties).
    if (!greedy && wb.n > wb.kw) wave_compact(wb);

    // ---- slice statistics
    if (lane_id() == 0) {
      w_tau[wave_id()] = wb.tau;
      w_n[wave_id()] = wb.n;
      w_ovf[wave_id()] = wb.overflow ? 1 : 0;
    }
    if (t == 0) s_cnt = 0;
    __syncthreads();
    uint32_t tau_s = 1u;
    int ovf = 0;
    for (int w = 0; w < NWAVE; ++w) { tau_s = max(tau_s, w_tau[w]); ovf |= w_ovf[w]; }

    if (greedy) {
      double bv = gs.bi == INT_MAX ? -__builtin_inf() : (double)gs.bv;
      int bi = gs.bi;
      int ni = gs.nan_i;
      if (pen_on)
        for (int sl = t; sl < A.ns; sl += WG) {
          uint32_t k = hkey[sl];
          if (k == HEMPTY) continue;
          int id = (int)(k >> 12);
          double xp = penalise(hval[sl], (int)(k & 0xFFFu), P);
          if (xp != xp) ni = min(ni, id);
          else argmax_merge(bv, bi, xp, id);
        }
      block_argmax(bv, bi, red_d, red_i);
      ni = block_min(ni, red_i, INT_MAX);
      if (t == 0) {
        my->m = 0; my->s = 0; my->best_v = bv; my->best_i = bi; my->nan_i = ni;
        my->tau = 1u; my->ncand = 0; my->flags = 0;
      }
    } else {
      const double invT = 1.0 / P.temperature;
      float Mu = block_max(st.m, (float*)red_d, -__builtin_inff());
      double su = 0.0;
      if (st.s != 0.0) su = st.s * exp2((double)(st.m - Mu) * (double)c);
      double Su = block_sum(su, red_d);
      double mp = -__builtin_inf();
      int pnan = 0;
      if (pen_on)
        for (int sl = t; sl < A.ns; sl += WG) {
          uint32_t k = hkey[sl];
          if (k == HEMPTY) continue;
          double xp = penalise(hval[sl], (int)(k & 0xFFFu), P);
          if (xp != xp) pnan = 1;
          else mp = xp > mp ? xp : mp;
        }
      double Ms = (double)Mu;
      if (pen_on) {
        double Mp = block_max(mp, red_d, -__builtin_inf());
        Ms = Mp > Ms ? Mp : Ms;
        if (block_max(pnan, red_i, 0)) Ms = __builtin_nan("");
      }
      double Ss = Su == 0.0 ? 0.0 : Su * exp(((double)Mu - Ms) * invT);
      const uint64_t thr64 = tau_s <= 1u ? 0ull : d2key((double)key2f(tau_s));
      if (pen_on) {
        double sp = 0.0;
        for (int sl = t; sl < A.ns; sl += WG) {
          uint32_t k = hkey[sl];
          if (k == HEMPTY) continue;
          int id = (int)(k >> 12);
          double xp = penalise(hval[sl], (int)(k & 0xFFFu), P);
          sp += exp((xp - Ms) * invT);
          uint64_t k64 = d2key(xp);
          if (k64 >= thr64 && xp == xp) {
            int pos = atomicAdd(&s_cnt, 1);
            mycand[pos].key = k64;
            mycand[pos].idx = id;
          }
        }
        Ss += block_sum(sp, red_d);
      }
      {   // region entries of this wave's buffer
        const int w = wave_id();
        const uint32_t* wk = (const uint32_t*)(dyn + A.off_wkey) + w * CAPW;
        const int32_t* wi = (const int32_t*)(dyn + A.off_widx) + w * CAPW;
        const int n = w_n[w];
        for (int e = lane_id(); e - lane_id() < n; e += 64) {
          bool keep = e < n && wk[e] >= tau_s;
          uint64_t b = ballot(keep);
          int base = 0;
          if (lane_id() == 0 && b) base = atomicAdd(&s_cnt, (int)__popcll(b));
          base = __shfl(base, 0);
          if (keep) {
            int pos = base + lanes_below(b);
            mycand[pos].key = d2key((double)key2f(wk[e]));
            mycand[pos].idx = wi[e];
          }
        }
      }
      __syncthreads();
      if (t == 0) {
        my->m = Ms; my->s = Ss; my->best_v = 0; my->best_i = INT_MAX; my->nan_i = INT_MAX;
        my->tau = tau_s; my->ncand = s_cnt; my->flags = ovf ? SF_OVERFLOW : 0;
      }
    }
  }

  // ---- the last workgroup of the row finishes it
  __syncthreads();
  if (A.nsplit > 1) {
    if (t == 0) {
      __threadfence();
      int old = __hip_atomic_fetch_add(&A.counters[row], 1, __ATOMIC_ACQ_REL,
                                       __HIP_MEMORY_SCOPE_AGENT);
      s_last = (old == A.nsplit - 1) ? 1 : 0;
      if (s_last)
        __hip_atomic_store(&A.counters[row], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __threadfence();
    }
    __syncthreads();
    if (!s_last) return;
  }
  finish_row(A, row, P, dyn, red_d, red_i);
}

template __global__ void sample_kernel<false>(SampleArgs);
template __global__ void sample_kernel<true>(SampleArgs);

}  // namespace cx

namespace cx {
int launch_sample(const SampleArgs& A, hipStream_t s) {
  const void* fn = A.bf16 ? (const void*)sample_kernel<true> : (const void*)sample_kernel<false>;
  // Raise the dynamic-LDS limit to what this launch needs (static LDS comes on top).
  static int attr_set[2] = {0, 0};
  if (A.lds_bytes > attr_set[A.bf16]) {
    hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, A.lds_bytes);
    if (e != hipSuccess) return (int)e;
    attr_set[A.bf16] = A.lds_bytes;
  }
  if (A.bf16)
    hipLaunchKernelGGL(sample_kernel<true>, dim3(A.B * A.nsplit), dim3(WG), A.lds_bytes, s, A);
  else
    hipLaunchKernelGGL(sample_kernel<false>, dim3(A.B * A.nsplit), dim3(WG), A.lds_bytes, s, A);
  return (int)hipGetLastError();
}
}  // namespace cx
