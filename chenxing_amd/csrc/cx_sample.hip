// cx_sample.hip -- fused sampler for gfx950 (reference chenxing/core/sampler.py:63-127).
//
// One launch samples a whole batch.  The grid is B x nsplit workgroups of
// 1024 threads; workgroup (row, s) streams the contiguous slice s of row
// `row` exactly once from HBM.  The slice is cut into chunks of 64 x U
// 16-byte vectors; each wave streams chunks with nontemporal buffer loads,
// two chunks in flight, taking its next chunk from an LDS counter so the
// waves of a workgroup finish together.  It produces:
//
//   * stochastic rows: the sum of exp2(x * c - R), c = log2(e) / T, over the
//     RAW logits (one fma + one v_exp_f32 per element, fp64 accumulation
//     against a per-lane integer exponent R), and an exact "region": every
//     unpenalised element at or above a threshold, appended to per-wave LDS
//     buffers.  The waves publish their largest lane values in rank-sorted
//     LDS slots and raise a shared threshold to the k-th largest published
//     value, so after the first chunk only a few elements per wave still
//     qualify.  Penalties touch only the history window's ids: their raw
//     logits are gathered at the start, and afterwards each one's raw term
//     is replaced by its penalised term in fp64 -- the hot loop never looks
//     at penalties, except to keep penalised elements out of the region (a
//     bitmap bit, tested only for elements above the threshold);
//   * greedy rows: the first argmax over the unpenalised elements (a bitmap
//     test per vector), merged with the penalised values afterwards.
//
// Top-k rows with one slice and a small region are decided in the same
// workgroup by one wave.  Every other row writes its region and statistics
// (one record per slice) and is finished by slow_kernel (cx_slow.hip), the
// launch that follows this one: the region finisher of cx_finish.hpp, then,
// where that cannot decide, the exact-normaliser refinement or the exact
// multi-pass path.
#include "cx_device.hpp"
#include "cx_sampler.h"
#include "cx_internal.hpp"
#include "cx_finish.hpp"
#include "cx_deep.hpp"
#include "cx_timing.hpp"

namespace cx {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define CX_RELAXED_WG __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP

// The row's scalars -- its 64-byte parameter block, its uniform and its
// history length -- in three scalar loads under one wait (uniform, SGPRs):
// they do not wait behind the vector loads in flight.
struct RowScalars {
  cx_row_params p;
  double u;
  int hlen;
};
__device__ __forceinline__ RowScalars sload_row(const cx_row_params* p, const double* u,
                                                const int32_t* hl) {
  typedef uint32_t u32x16 __attribute__((ext_vector_type(16)));
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  u32x16 v;
  u32x2 uu;
  uint32_t h;
  asm volatile(
      "s_load_dwordx16 %0, %3, 0x0\n\t"
      "s_load_dwordx2 %1, %4, 0x0\n\t"
      "s_load_dword %2, %5, 0x0\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&s"(v), "=&s"(uu), "=&s"(h)
      : "s"(p), "s"(u), "s"(hl));
  RowScalars r;
  r.p = __builtin_bit_cast(cx_row_params, v);
  r.u = __builtin_bit_cast(double, uu);
  r.hlen = (int)h;
  return r;
}

// ------------------------------------------------------------ penalties
// Penalty index of a slice [lo, hi): a bitmap of the window's ids (the
// stream's test), an open-addressing hash of the distinct ids, one word
// (id << 12 | count in the window) and the id's raw logit per slot, and the
// dense list of the occupied slots in insertion order.  Ids are below 2^20
// and counts below 2^12, so no word equals HW_EMPTY.
struct PenIndex {
  CX_LDS uint32_t* bitmap;
  CX_LDS uint32_t* hword;
  CX_LDS float* hval;
  CX_LDS int32_t* dense;
  int nbw;
  int ns, ns_log2;
};
constexpr uint32_t HW_EMPTY = 0xFFFFFFFFu;
constexpr int NSLOT = 4;                        // published lane keys per wave
constexpr int HPT = (WIN_MAX + WG - 1) / WG;   // history entries per thread loaded up front

__device__ __forceinline__ bool pen_bit(const PenIndex& X, int r) {
  return (X.bitmap[r >> 5] >> (r & 31)) & 1u;
}
// The NE penalty bits of the vector starting at slice offset r (a multiple
// of NE, so they share one word), or 0 when !on.  The read is unconditional
// (word 0 when !on) so it needs no branch.
template <int NE>
__device__ __forceinline__ uint32_t pen_bits(const PenIndex& X, bool on, int r) {
  static_assert(32 % NE == 0, "a vector's bits in one word");
  const uint32_t w = X.bitmap[on ? r >> 5 : 0];
  return on ? (w >> (r & 31)) & ((1u << NE) - 1u) : 0u;
}

// Count one more occurrence of id; returns its slot, and in `created`
// whether this call inserted it (one caller per distinct id).  Linear
// probing; the table holds at least twice as many slots as window entries.
__device__ __forceinline__ int pen_insert(const PenIndex& X, int id, bool& created) {
  uint32_t h = ((uint32_t)id * 0x9E3779B1u) >> (32 - X.ns_log2);
  const uint32_t w0 = (uint32_t)id << 12;
  while (true) {
    uint32_t prev = HW_EMPTY;
    created = __hip_atomic_compare_exchange_strong(X.hword + h, &prev, w0, __ATOMIC_RELAXED,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (created || (prev >> 12) == (uint32_t)id) {
      __hip_atomic_fetch_add(X.hword + h, 1u, CX_RELAXED_WG);
      return (int)h;
    }
    h = (h + 1) & (uint32_t)(X.ns - 1);
  }
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
  static constexpr int U = 4;      // vectors per lane per chunk
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
  static constexpr int U = 2;
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

// Buffer descriptor over `bytes` bytes at p: loads past the end return 0, so
// the stream needs no clamped addresses.  Word 3 is the raw-buffer format of
// gfx9 parts.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, bytes, 0x00020000);
}
// 16-byte nontemporal load at byte offset voff (range-checked: past the
// descriptor's end it returns 0 and touches no memory).
template <bool BF16>
__device__ __forceinline__ typename Elem<BF16>::V bload(__amdgpu_buffer_rsrc_t rs, int voff) {
  return __builtin_bit_cast(typename Elem<BF16>::V,
                            __builtin_amdgcn_raw_buffer_load_b128(rs, voff, 0, 2));
}
// The U vectors of this lane in chunk ch: vectors ch * 64U + u * 64 + lane.
// Issued unconditionally, also for chunk ids past the slice (their loads
// return zeros that are never used): the compiler then knows exactly how
// many loads are in flight and waits only for the chunk being consumed.
template <bool BF16>
__device__ __forceinline__ void load_chunk(__amdgpu_buffer_rsrc_t rs, int ch,
                                           typename Elem<BF16>::V (&q)[Elem<BF16>::U]) {
  constexpr int U = Elem<BF16>::U;
#pragma unroll
  for (int u = 0; u < U; ++u) q[u] = bload<BF16>(rs, ((ch * 64 * U + u * 64) + lane_id()) * 16);
}
// Next chunk for this wave from the workgroup's counter.
__device__ __forceinline__ int next_chunk(CX_LDS int* counter) {
  int v = 0;
  if (lane_id() == 0) v = __hip_atomic_fetch_add(counter, 1, CX_RELAXED_WG);
  return __builtin_amdgcn_readfirstlane(v);
}

// The k-th largest of the 64 lane values (1 <= k <= 64): two key bits per
// step, three independent ballot counts each.  Inlined: a call makes the
// callee wait for every load in flight (the calling convention), which in
// the stream would drain the wave's chunk pipeline.
// The k-th largest of the wave's 128 values v1, v2 (two per lane), as
// kth_of_lanes.  With stop > 0 only the key bits from stop up are
// selected: the result is the k-th largest with its lower bits cleared, a
// lower bound of it (the seeds, where a slightly lower first threshold
// costs less than the full selection).
__device__ __forceinline__ uint32_t kth_of_lanes2(uint32_t v1, uint32_t v2, int k, int stop = 0) {
  uint32_t prefix = 0u;
  for (int sh = 30; sh >= stop; sh -= 2) {
    const uint32_t b1 = prefix | (1u << sh), b2 = prefix | (2u << sh), b3 = prefix | (3u << sh);
    const int c3 = __popcll(ballot(v1 >= b3)) + __popcll(ballot(v2 >= b3));
    const int c2 = __popcll(ballot(v1 >= b2)) + __popcll(ballot(v2 >= b2));
    const int c1 = __popcll(ballot(v1 >= b1)) + __popcll(ballot(v2 >= b1));
    prefix = c3 >= k ? b3 : (c2 >= k ? b2 : (c1 >= k ? b1 : prefix));
  }
  return prefix;
}
__device__ __forceinline__ uint32_t kth_of_lanes(uint32_t v, int k, int stop = 0) {
  uint32_t prefix = 0u;
  for (int sh = 30; sh >= stop; sh -= 2) {
    const uint32_t b1 = prefix | (1u << sh), b2 = prefix | (2u << sh), b3 = prefix | (3u << sh);
    const int c3 = __popcll(ballot(v >= b3));
    const int c2 = __popcll(ballot(v >= b2));
    const int c1 = __popcll(ballot(v >= b1));
    prefix = c3 >= k ? b3 : (c2 >= k ? b2 : (c1 >= k ? b1 : prefix));
  }
  return prefix;
}

// ------------------------------------------------------------ wave candidates
// Wave-uniform state: every lane holds the same n / tau / overflow.  tau only
// rises.  `cnt` is the LDS copy of n that lanes bump when they append on
// their own.  `shared` is the slice's shared threshold word: the highest
// proven lower bound of the slice's k-th largest unpenalised value.
struct WaveBuf {
  CX_LDS uint32_t* key;
  CX_LDS int32_t* idx;
  CX_LDS int* cnt;
  CX_LDS uint32_t* shared;
  int n;
  uint32_t tau;   // every unpenalised element seen with key >= tau is held
  float tauf;     // tau as a float; -inf while tau <= 1 (everything)
  int kw;         // entries a compaction keeps
  bool overflow;
  // split normaliser (see XSum): entries [0, xn) of the buffer are already
  // in the wave's exact sum; lossy: an insertion took the one-by-one path,
  // whose compactions the split sum does not follow
  int xn;
  bool lossy;
};

__device__ __forceinline__ void raise_tau(WaveBuf& w, uint32_t t) {
  if (t > w.tau) {
    w.tau = t;
    w.tauf = key2f(t);
  }
}

// State travels by value so nothing of the caller lives in memory.
struct WState {
  int n;
  uint32_t tau;
};

// Raise tau to the kw-th largest key held (bitwise radix select over the
// buffer with ballot counts) and drop the entries below it.  Not inlined: it
// is the cold path of the stream.
__device__ __noinline__ WState wave_compact_call(CX_LDS uint32_t* wkey, CX_LDS int32_t* widx,
                                                 int n, uint32_t tau, int kw, bool share,
                                                 CX_LDS uint32_t* shared) {
  constexpr int PER = CAPW / 64;
  const int l = lane_id();
  // the arguments are wave-uniform: scalar registers keep the radix loop's
  // control and prefix off the vector unit
  n = __builtin_amdgcn_readfirstlane(n);
  kw = __builtin_amdgcn_readfirstlane(kw);
  tau = (uint32_t)__builtin_amdgcn_readfirstlane((int)tau);
  uint32_t k[PER];
  int32_t id[PER];
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    int pos = l + 64 * e;
    k[e] = pos < n ? wkey[pos] : 0u;
    id[e] = pos < n ? widx[pos] : 0;
  }
  // bits above the highest and below the lowest bit in which held keys
  // differ need no radix step (a bf16 value's key has 16 zero low bits)
  uint32_t kand = 0xFFFFFFFFu, kor = 0u;
#pragma unroll
  for (int e = 0; e < PER; ++e)
    if (k[e]) { kand &= k[e]; kor |= k[e]; }
  kand = wave_reduce(kand, OpAnd());
  kor = wave_reduce(kor, OpOr());
  const uint32_t diff = kand ^ kor;
  const int hb = diff ? 31 - __clz(diff) : -1;
  const int lb = diff ? __builtin_ctz(diff) : 0;
  uint32_t prefix = hb < 0 ? kand : (hb == 31 ? 0u : (kand & ~((2u << hb) - 1u)));
  for (int bit = hb; bit >= lb; --bit) {
    uint32_t cand = prefix | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int e = 0; e < PER; ++e) cnt += __popcll(ballot(k[e] >= cand));
    if (cnt >= kw) prefix = cand;
  }
  // the shared low bits: prefix is then the kw-th largest key itself
  if (hb >= 0) prefix |= kand & ((1u << lb) - 1u);
  if (prefix > tau) tau = prefix;
  int m = 0;
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    bool keep = k[e] >= tau && k[e] != 0u;
    uint64_t b = ballot(keep);
    if (keep) {
      int p = m + lanes_below(b);
      wkey[p] = k[e];
      widx[p] = id[e];
    }
    m += __popcll(b);
  }
  // a wave's kw-th largest bounds the slice's k-th largest when kw == k
  if (share && l == 0) __hip_atomic_fetch_max(shared, tau, CX_RELAXED_WG);
  WState r;
  r.n = m;
  r.tau = tau;
  return r;
}

__device__ __forceinline__ void wave_compact(WaveBuf& w, bool share) {
  WState r = wave_compact_call(w.key, w.idx, w.n, w.tau, w.kw, share, w.shared);
  // uniform results: keep them in scalar registers
  w.n = __builtin_amdgcn_readfirstlane(r.n);
  raise_tau(w, (uint32_t)__builtin_amdgcn_readfirstlane((int)r.tau));
}

// Insert one element slot of the wave (key 0 = not a candidate), compacting
// when the buffer is full.  Returns whether this lane's key went in.
__device__ __forceinline__ bool wave_insert1(WaveBuf& w, uint32_t key, int idx, bool share) {
  bool p = key >= w.tau;
  uint64_t b = ballot(p);
  if (b == 0) return false;
  int c = __popcll(b);
  if (w.n + c > CAPW) {
    wave_compact(w, share);
    p = key >= w.tau;
    b = ballot(p);
    c = __popcll(b);
    if (w.n + c > CAPW) { w.overflow = true; return false; }
  }
  if (p) {
    int pos = w.n + lanes_below(b);
    w.key[pos] = key;
    w.idx[pos] = idx;
  }
  w.n += c;
  return p;
}

// ------------------------------------------------------------ shared thresholds
// Every lane keeps ck, the key of the largest unpenalised element it has
// seen at or above its wave's threshold (or in its first chunk): distinct
// lanes hold distinct elements, and ck only grows.
//
// Slot scheme (top-k rows, k <= 64): wave w writes its m = NSLOT largest
// lane keys, rank-sorted, to slots[m w .. m w + m).  Slot j of a wave
// is the (j+1)-th largest lane key, which only grows; a reader that catches
// a wave mid-update therefore never counts more slots >= v than the wave has
// distinct elements >= v, and the k-th largest of the 64 slots is a lower
// bound of the slice's k-th largest unpenalised value.
__device__ __forceinline__ void publish_top(uint32_t ck, int m, CX_LDS uint32_t* slots) {
  uint32_t v = ck;
  for (int j = 0; j < m; ++j) {
    const uint32_t M = wave_reduce(v, OpMax());
    if (lane_id() == 0) slots[j] = M;
    const uint64_t b = ballot(v == M);
    if (lane_id() == __builtin_ctzll(b)) v = 0u;
  }
}
// Minimum scheme (64 < k <= 64 * NWAVE): each wave publishes its r-th largest
// lane key; NWAVE * r distinct elements reach the minimum over the waves.
__device__ __forceinline__ uint32_t pub_min(const CX_LDS uint32_t* w_pub) {
  uint32_t m = lane_id() < NWAVE ? lds_load(w_pub + lane_id()) : 0xFFFFFFFFu;
  for (int o = 32; o > 0; o >>= 1) {
    const uint32_t v = (uint32_t)__shfl_xor((int)m, o);
    m = v < m ? v : m;
  }
  return m;
}
// Publish this wave's values and raise the shared threshold with them.
__device__ __forceinline__ void publish(uint32_t ck, int krow, int pub_r, CX_LDS uint32_t* slots,
                                        CX_LDS uint32_t* w_pub, CX_LDS uint32_t* shared) {
  uint32_t T = 0u;
  if (krow <= 64) {
    publish_top(ck, NSLOT, slots + NSLOT * wave_id());
    T = kth_of_lanes(lds_load(slots + lane_id()), krow);
  } else if (pub_r > 0) {
    const uint32_t th = kth_of_lanes(ck, pub_r);
    if (lane_id() == 0 && th > w_pub[wave_id()]) w_pub[wave_id()] = th;
    T = pub_min(w_pub);
  }
  if (lane_id() == 0 && T > 1u) __hip_atomic_fetch_max(shared, T, CX_RELAXED_WG);
}

// ------------------------------------------------------------ stochastic stream
// The sum is taken against a per-lane integer exponent R: terms
// exp2(x * c - R) stay finite while x <= top = (value that set R) + LIM / c,
// so R moves only on such a jump, and the fp64 sum is then rescaled by an
// exact power of two.  A term's fp32 argument is within half an ulp of LIM
// of the exact one and the 16 terms of a chunk are added in fp32 (15
// roundings) before the fp64 accumulation, so every term is within TOL_T
// of its exact value.
constexpr float LIM = 16.0f;
struct SState {
  float R;      // integer-valued exponent offset (-inf before the first value)
  float nR;     // -R, clamped finite (so -inf values give 0 terms before the first value)
  float top;
  double s;
};

// max of three floats without the NaN quieting fmaxf adds (the stream's sum
// turns NaN on any NaN element anyway)
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
template <int NE>
__device__ __forceinline__ float vec_max(const float (&x)[NE]) {
  if constexpr (NE == 1) {
    return x[0];
  } else {
    float m = max3f(x[0], x[1], x[NE > 2 ? 2 : 1]);
#pragma unroll
    for (int j = 3; j < NE; j += 2) m = max3f(m, x[j], x[j + 1 < NE ? j + 1 : j]);
    return m;
  }
}

__device__ __forceinline__ void rescale(float vmax, float c, float lim, SState& st) {
  if (vmax > st.top) {
    // vmax * c may overflow to +inf: R = +inf, the row's sum turns NaN or 0
    // and the row goes to the multi-pass kernel
    const float Rn = __builtin_ceilf(vmax * c);
    if (st.s != 0.0) st.s = __builtin_ldexp(st.s, (int)fmaxf(st.R - Rn, -2048.0f));
    st.R = Rn;
    st.nR = fminf(-Rn, 3.402823466e38f);
    st.top = vmax + lim;
  }
}

// An exact fp64 running sum of exp((x - m) / T), each term within 1 ulp
// (exp64_neg), against a reference m at or above every summed x (the sum is
// rescaled by exp((m_old - m) / T) when m rises).  Kept only by the
// sliced-launch kernel, for stochastic top-p rows, so that the row's
// normaliser needs no second read of the row, in one of two forms:
//  - full (rows with a penalty window or a top-k): every element of the
//    lane, against the lane's largest value;
//  - split (the other top-p rows): only the elements the wave buffer took,
//    against the wave's largest buffered value.  Each buffered entry is
//    summed once, from the buffer: before a compaction drops entries, and
//    at the stream's end for the rest.  The elements below the wave's
//    threshold when they arrived (SState::t) are summed as the stream sum
//    is, within TOL_S of their exact total, and that total is a small part
//    of a top-p row's normaliser: the buffered elements are the row's
//    largest, which carry the nucleus.  The two add up to the slice's
//    normaliser within TOL_S times the below-threshold part, and the
//    fp64 exponentials are taken for a few entries per lane, not for every
//    element.
struct XSum {
  double s, m;
};
__device__ __forceinline__ void xsum_raise(XSum& xs, double cm, double invT, const double* etab) {
  if (cm > xs.m) {
    if (xs.s != 0.0) xs.s *= exp64_neg((xs.m - cm) * invT, etab);
    xs.m = cm;
  }
}
// Split form: add the exact terms of wave buffer entries [from, to) (bounds
// wave-uniform, to <= CAPW), raising the wave-uniform reference to their
// largest value first.
__device__ __forceinline__ void xsum_entries(const WaveBuf& wb, int from, int to, double invT,
                                             const double* etab, XSum& xs) {
  constexpr int PER = CAPW / 64;
  // entries other lanes of the wave wrote (in order on the hardware; the
  // barrier keeps the compiler from hoisting the reads)
  __builtin_amdgcn_wave_barrier();
  float v[PER];
  float vm = -__builtin_inff();
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int pos = from + lane_id() + 64 * e;
    v[e] = pos < to ? key2f(wb.key[pos]) : -__builtin_inff();
    vm = fmaxf(vm, v[e]);
  }
  xsum_raise(xs, (double)wave_reduce(vm, OpMax()), invT, etab);
  if (!(xs.m > -__builtin_inf())) return;            // nothing buffered yet
#pragma unroll
  for (int e = 0; e < PER; ++e)
    if (v[e] > -__builtin_inff()) xs.s += exp64_neg(((double)v[e] - xs.m) * invT, etab);
}

// Append the candidates of one chunk (some lane of the wave has one: its
// chunk maximum reaches the threshold).  Penalised elements never enter:
// their penalised values join afterwards.
//  - Few flagged lanes (room for all their elements): lanes append on their
//    own through the wave's LDS counter; a slot no lane reaches costs a
//    compare and a branch.
//  - Otherwise each lane marks its element slots at or above the threshold
//    and a wave prefix sum of the marks gives every lane its write offset.
//    When the marks do not fit, the wave compacts first; if they still do
//    not fit the element slots go through wave_insert1 one by one.
template <bool BF16>
__device__ __forceinline__ void append_chunk(WaveBuf& wb,
                                             const float (&xs)[Elem<BF16>::U][Elem<BF16>::NE],
                                             bool flagged, int vb, int nv, int lo, bool pen_on,
                                             const PenIndex& X, bool share, uint32_t& ck,
                                             bool exs, double invT, const double* etab,
                                             XSum& xsum) {
  using E = Elem<BF16>;
  constexpr int NE = E::NE;
  constexpr int U = E::U;
  static_assert(U * NE <= 32, "a lane's element slots in one mask word");
  const int lanes = __popcll(ballot(flagged));
  if (wb.n + lanes * U * NE <= CAPW) {
    if (flagged) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int vi = vb + u * 64;
        const int e0 = vi * NE + lo;
#pragma unroll
        for (int j = 0; j < NE; ++j) {
          if (vi < nv && xs[u][j] >= wb.tauf && !(pen_on && pen_bit(X, e0 + j - lo))) {
            const uint32_t k = f2key(xs[u][j]);
            const int pos = __hip_atomic_fetch_add(wb.cnt, 1, CX_RELAXED_WG);
            wb.key[pos] = k;
            wb.idx[pos] = e0 + j;
            ck = k > ck ? k : ck;
          }
        }
      }
    }
    // the wave's appends precede the read of their count (one wave's LDS
    // operations complete in order; the barrier keeps the compiler from
    // moving the read above them)
    __builtin_amdgcn_wave_barrier();
    wb.n = lds_load(wb.cnt);
    return;
  }
  // this lane's element slots at or above the threshold, unpenalised (the
  // chunk's penalty words are read together: one LDS round trip)
  auto select = [&]() {
    uint32_t m = 0u;
    if (flagged) {
      uint32_t pw[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int vi = vb + u * 64;
        pw[u] = pen_on ? X.bitmap[vi < nv ? (vi * NE) >> 5 : 0] : 0u;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int vi = vb + u * 64;
        const uint32_t pb = pw[u] >> ((vi * NE) & 31);
#pragma unroll
        for (int j = 0; j < NE; ++j)
          if (vi < nv && xs[u][j] >= wb.tauf && !((pb >> j) & 1u)) m |= 1u << (u * NE + j);
      }
    }
    return m;
  };
  uint32_t m = select();
  int c = __popc(m);
  int incl = wave_scan_dpp(c);
  int total = __builtin_amdgcn_readlane(incl, 63);
  if (wb.n + total > CAPW && wb.n > wb.kw) {
    // make room first: keep the kw largest held, raising the threshold (the
    // split sum takes every held entry first, the dropped and the kept)
    if (exs) xsum_entries(wb, wb.xn, wb.n, invT, etab, xsum);
    wave_compact(wb, share);
    if (exs) wb.xn = wb.n;
    // The split sum left this chunk's marked slots out of its
    // below-threshold part: they are written as marked, those under the
    // raised threshold included (the next compaction drops them, summed).
    // Where they no longer fit, the raised threshold selects again and the
    // slots under it are counted nowhere: the slice's split sum is lost.
    if (!exs || wb.n + total > CAPW) {
      if (exs) wb.lossy = true;
      m = select();
      c = __popc(m);
      incl = wave_scan_dpp(c);
      total = __builtin_amdgcn_readlane(incl, 63);
    }
  }
  if (wb.n + total <= CAPW) {
    // each lane writes its slots at its offset in the wave's prefix sum
    const int base = wb.n + incl - c;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e0 = (vb + u * 64) * NE + lo;
#pragma unroll
      for (int j = 0; j < NE; ++j) {
        const int s = u * NE + j;
        if ((m >> s) & 1u) {
          const int pos = base + __popc(m & ((1u << s) - 1u));
          const uint32_t k = f2key(xs[u][j]);
          wb.key[pos] = k;
          wb.idx[pos] = e0 + j;
          ck = k > ck ? k : ck;
        }
      }
    }
    wb.n += total;
    if (lane_id() == 0) *wb.cnt = wb.n;
  } else {
    if (exs) wb.lossy = true;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float (&x)[NE] = xs[u];
      const int vi = vb + u * 64;
      const bool valid = vi < nv;
      const int e0 = vi * NE + lo;
#pragma unroll
      for (int j = 0; j < NE; ++j) {
        uint32_t k = 0u;
        if (valid && x[j] >= wb.tauf && !(pen_on && pen_bit(X, e0 + j - lo))) k = f2key(x[j]);
        if (wave_insert1(wb, k, e0 + j, share)) ck = k > ck ? k : ck;
      }
    }
    if (lane_id() == 0) *wb.cnt = wb.n;
  }
}

// Stream the vectors of a stochastic slice.  Vector i covers elements
// lo + i*NE .. lo + i*NE + NE-1, i < nv.  q and qn hold this wave's first
// two chunks (wave_id() and wave_id() + NWAVE), loaded by the caller.  The
// loop alternates between the two buffers (no register copies, which would
// wait for the chunk still in flight): it consumes one and refills it with
// the chunk after the other, so two chunks stay in flight.  ex, exs: the
// slice keeps the full or the split exact fp64 normaliser (XSum); with the
// split one, st.s sums only the elements below the wave threshold.
template <bool BF16, bool EXACT>
__device__ __forceinline__ void stream_stoch(__amdgpu_buffer_rsrc_t rs,
                                             typename Elem<BF16>::V (&q)[Elem<BF16>::U],
                                             typename Elem<BF16>::V (&qn)[Elem<BF16>::U], int nv,
                                             int lo, bool pen_on, const PenIndex& X, float c,
                                             int krow, int pub_r, CX_LDS int* chunk_ctr,
                                             CX_LDS uint32_t* slots, CX_LDS uint32_t* w_pub,
                                             SState& st, WaveBuf& wb, uint32_t& ck, bool ex,
                                             bool exs, double invT, const double* etab,
                                             XSum& xs) {
  using E = Elem<BF16>;
  using V = typename E::V;
  constexpr int NE = E::NE;
  constexpr int U = E::U;
  constexpr int CH = 64 * U;
  const float lim = LIM / c;
  const bool share = true;
  const int nch = (nv + CH - 1) / CH;
  const int nfull = nv / CH;
  // chunk ids are wave-uniform (SGPRs)
  int ch = __builtin_amdgcn_readfirstlane(wave_id());
  int cn = ch + NWAVE;
  bool fresh = false;              // appended since the last publication
  int it = 0;
  // consume chunk ch from buffer b, refill b with the chunk after cn
  auto step = [&](V (&b)[U]) {
    raise_tau(wb, lds_load(wb.shared));
    // the split sum's tail: elements below the threshold this chunk's
    // appends start from (NaN: every element, the other rows)
    const float tfs = EXACT && exs ? wb.tauf : __builtin_nanf("");
    const int vb = ch * CH + lane_id();
    float x[U][NE];
#pragma unroll
    for (int u = 0; u < U; ++u) E::unpack(b[u], x[u]);
    if (ch >= nfull) {                 // the last, partial chunk
#pragma unroll
      for (int u = 0; u < U; ++u)
#pragma unroll
        for (int j = 0; j < NE; ++j) x[u][j] = vb + u * 64 < nv ? x[u][j] : -__builtin_inff();
    }
    float cmax = vec_max<NE>(x[0]);
#pragma unroll
    for (int u = 1; u < U; ++u) cmax = fmaxf(cmax, vec_max<NE>(x[u]));
    rescale(cmax, c, lim, st);
    float ts = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int j = 0; j < NE; ++j) {
        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(x[u][j], c, st.nR));
        if (EXACT) ts += !(x[u][j] >= tfs) ? e : 0.0f;
        else ts += e;
      }
    st.s += (double)ts;
    // The sum is taken here, before the refill below.  Left free, the
    // compiler sinks it past the refill, the refill then needs registers
    // other than the buffer's, and the loop's back edge copies them over
    // after waiting for every load in flight.
    __asm__ volatile("" : "+v"(st.s));
    if (EXACT && ex) {
      xsum_raise(xs, (double)cmax, invT, etab);
      if (xs.m > -__builtin_inf()) {
        double a = 0.0;
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
          for (int j = 0; j < NE; ++j) a += exp64_neg(((double)x[u][j] - xs.m) * invT, etab);
        xs.s += a;
      }
      __asm__ volatile("" : "+v"(xs.s));
    }
    const bool flagged = cmax >= wb.tauf;
    if (ballot(flagged)) {
      append_chunk<BF16>(wb, x, flagged, vb, nv, lo, pen_on, X, share, ck, EXACT && exs, invT,
                         etab, xs);
      fresh = true;
    }
    const int cnn = cn < nch ? __builtin_amdgcn_readfirstlane(next_chunk(chunk_ctr)) : nch;
    load_chunk<BF16>(rs, cnn, b);      // past the slice: zeros, never consumed
    // after the refill, so both chunks are in flight while the wave
    // publishes (a publish is a few hundred instructions); not once the
    // slice's chunks are all handed out (a raised threshold would filter
    // only the chunks already in flight)
    if ((it == 1 || it == 3) && fresh && cnn < nch) {
      publish(ck, krow, pub_r, slots, w_pub, wb.shared);
      raise_tau(wb, lds_load(wb.shared));
      fresh = false;
    }
    ch = cn;
    cn = cnn;
    ++it;
  };
  while (ch < nch) {
    step(q);
    if (ch >= nch) break;
    step(qn);
  }
}

// Scalar elements [s0, hi) of a stochastic slice (unaligned rows, or the
// tail after the last whole vector).
template <bool BF16, bool EXACT>
__device__ __forceinline__ void stream_scalar(const char* rowp, int s0, int lo, int hi,
                                              bool pen_on, const PenIndex& X, float c, bool share,
                                              SState& st, WaveBuf& wb, uint32_t& ck, bool ex,
                                              double invT, const double* etab, XSum& xs) {
  using E = Elem<BF16>;
  const float lim = LIM / c;
  for (int e = s0 + lane_id() + 64 * wave_id(); e - lane_id() < hi; e += WG) {
    const bool valid = e < hi;
    const float x = valid ? E::scalar(rowp, e) : -__builtin_inff();
    rescale(x, c, lim, st);
    st.s += (double)__builtin_amdgcn_exp2f(__builtin_fmaf(x, c, st.nR));
    if (EXACT && ex) {
      xsum_raise(xs, (double)x, invT, etab);
      if (xs.m > -__builtin_inf()) xs.s += exp64_neg(((double)x - xs.m) * invT, etab);
    }
    uint32_t k = 0u;
    if (valid && x >= wb.tauf && !(pen_on && pen_bit(X, e - lo))) k = f2key(x);
    if (ballot(k != 0u)) {
      if (wave_insert1(wb, k, e, share)) ck = k > ck ? k : ck;
      if (lane_id() == 0) *wb.cnt = wb.n;
    }
  }
}

// ------------------------------------------------------------ greedy stream
struct GreedyState {
  float bv;
  int bi;
  int nan_i;
};

// One vector (or scalar, NE == 1): first argmax over the unpenalised,
// valid elements (penalised ones are merged with their penalised values
// afterwards).
template <int NE>
__device__ __forceinline__ void greedy_vec(const float (&x)[NE], int e0, bool valid, int lo,
                                           bool has_pen, const PenIndex& X, GreedyState& gs) {
  if (!valid) return;
  uint32_t bits = 0u;
  if (has_pen) {
    const int r = e0 - lo;
    bits = (X.bitmap[r >> 5] >> (r & 31)) & ((1u << NE) - 1u);
  }
#pragma unroll
  for (int j = 0; j < NE; ++j) {
    if (bits & (1u << j)) continue;
    if (x[j] > gs.bv) { gs.bv = x[j]; gs.bi = e0 + j; }
    if (x[j] != x[j] && gs.nan_i == INT_MAX) gs.nan_i = e0 + j;
  }
}

template <bool BF16>
__device__ __forceinline__ void stream_greedy(const char* rowp, __amdgpu_buffer_rsrc_t rs,
                                              typename Elem<BF16>::V (&q)[Elem<BF16>::U],
                                              typename Elem<BF16>::V (&qn)[Elem<BF16>::U], int nv,
                                              int lo, int hi, int s0, bool pen_on,
                                              const PenIndex& X, CX_LDS int* chunk_ctr,
                                              GreedyState& gs) {
  using E = Elem<BF16>;
  using V = typename E::V;
  constexpr int NE = E::NE;
  constexpr int U = E::U;
  constexpr int CH = 64 * U;
  const int nch = (nv + CH - 1) / CH;
  int ch = __builtin_amdgcn_readfirstlane(wave_id());
  int cn = ch + NWAVE;
  // the two buffers alternate, as in stream_stoch
  auto step = [&](V (&b)[U]) {
    const int vb = ch * CH + lane_id();
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float x[NE];
      E::unpack(b[u], x);
      const int vi = vb + u * 64;
      greedy_vec<NE>(x, vi * NE + lo, vi < nv, lo, pen_on, X, gs);
    }
    const int cnn = cn < nch ? __builtin_amdgcn_readfirstlane(next_chunk(chunk_ctr)) : nch;
    load_chunk<BF16>(rs, cnn, b);
    ch = cn;
    cn = cnn;
  };
  while (ch < nch) {
    step(q);
    if (ch >= nch) break;
    step(qn);
  }
  for (int e = s0 + threadIdx.x; e < hi; e += WG) {
    float x1[1] = {E::scalar(rowp, e)};
    greedy_vec<1>(x1, e, true, lo, pen_on, X, gs);
  }
}

// ------------------------------------------------------------ top-k finish
// Finish of a top-k row (k <= 64) from its region list (nlist <= LEAN_CAP
// entries with distinct ids, holding every value at or above the k-th
// largest): the list is ranked by value and by id in parallel, then one
// wave cuts top-k (ties kept), top-p and min-p on the rank-ordered top
// entries and draws in token-id order.
struct LeanLds {
  int32_t rv[LEAN_CAP];   // value rank of list entry e (descending, ties by ascending id)
  int32_t ri[LEAN_CAP];   // id rank of list entry e (ascending)
  uint64_t sk[68];        // keys of value ranks 0..64
  int32_t si[68];         // their ids
  int32_t sr[68];         // their id ranks
  double oq[LEAN_CAP];    // normalised kept mass at id rank r (0 where not kept)
  int32_t oid[LEAN_CAP];  // id at id rank r
};

// Waves 1 .. NWAVE-1: each counts, for one group of 64 list entries, the
// entries of one stripe of the list that precede them by value and by id.
// The counts are integers, so the order of the LDS additions does not
// matter.  rv and ri start at zero.
__device__ __forceinline__ void lean_ranks(const CX_LDS uint64_t* gk, const CX_LDS int32_t* gi,
                                           int nlist, CX_LDS LeanLds* L) {
  static_assert(NWAVE == 16 && LEAN_CAP <= 256, "stripe layout");
  // ng groups of 64 entries, per = 15 / ng stripes each; x / per as
  // (x * ceil(2^16 / per)) >> 16, exact for x <= 15 * 256
  const int ng = (nlist + 63) >> 6;
  const int per = ng == 1 ? 15 : (ng == 2 ? 7 : (ng == 3 ? 5 : 3));
  const uint32_t rcp = ng == 1 ? 4370u : (ng == 2 ? 9363u : (ng == 3 ? 13108u : 21846u));
  const int w = wave_id() - 1;
  const int sp = ng == 3 ? (int)(((uint32_t)w * 21846u) >> 16) : w >> (ng == 4 ? 2 : ng - 1);
  const int eg = w - sp * ng;
  if (sp >= per) return;
  const int e = eg * 64 + lane_id();
  const int j0 = (int)(((uint32_t)(sp * nlist) * rcp) >> 16);
  const int j1 = (int)(((uint32_t)((sp + 1) * nlist) * rcp) >> 16);
  const uint64_t ke = e < nlist ? gk[e] : 0ull;
  const int32_t ie = e < nlist ? gi[e] : INT_MAX;
  int cv = 0, ci = 0;
#pragma unroll 4
  for (int j = j0; j < j1; ++j) {
    const uint64_t kj = gk[j];
    const int32_t ij = gi[j];
    cv += (kj > ke || (kj == ke && ij < ie)) ? 1 : 0;
    ci += ij < ie ? 1 : 0;
  }
  if (e < nlist) {
    __hip_atomic_fetch_add(&L->rv[e], cv, CX_RELAXED_WG);
    __hip_atomic_fetch_add(&L->ri[e], ci, CX_RELAXED_WG);
  }
}

// Outcomes of lean_decide.
constexpr int LEAN_PENDING = 0;  // the exact multi-pass path must take the row
constexpr int LEAN_DONE = 1;
constexpr int LEAN_NEAR = 2;     // a top-p cut within the normaliser's error bound

// One wave decides the row from the ranks; Rb and S give probabilities
// exp2(x c - Rb) / S within tol (relative) of the exact ones.  LEAN_NEAR
// sends the row to the exact-normaliser refinement, LEAN_PENDING (more than
// 64 entries tied into the top-k) to the exact path.

__device__ inline int lean_decide(const cx_row_params& P, const CX_LDS uint64_t* gk,
                                  const CX_LDS int32_t* gi, int nlist, double kc, double Rb,
                                  double S, double tol, CX_LDS LeanLds* L, double u, bool net,
                                  int& tok) {
  const int l = lane_id();
  // the top 65 entries in value order, and every id at its id rank
  for (int e = l; e < nlist; e += 64) {
    const int r = L->rv[e], q = L->ri[e];
    const int32_t id = gi[e];
    if (r < 65) { L->sk[r] = gk[e]; L->si[r] = id; L->sr[r] = q; }
    L->oid[q] = id;
    L->oq[q] = 0.0;
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const int E = min(nlist, 64);
  const uint64_t key = l < E ? L->sk[l] : 0ull;
  const int32_t idx = l < E ? L->si[l] : INT_MAX;
  const int32_t rid = l < E ? L->sr[l] : 0;
  // (1) top-k: every entry at or above the k-th largest value
  int n = E;
  if (P.top_k < nlist) {
    const uint64_t kth = lane_read(key, P.top_k - 1);
    n = __popcll(ballot(l < E && key >= kth));
    if (n == 64 && nlist > 64 && L->sk[64] == kth) return LEAN_PENDING;
  }
  // (2) probabilities of the kept prefix; top-p on the unrenormalised vector
  const double Pj = l < n ? exp2(key2d(key) * kc - Rb) / S : 0.0;
  bool keep = l < n;
  if (P.top_p < 1.0) {                                 // sampler.py:81-89
    const double cum = wave_scan_dpp(Pj);
    const uint64_t b = ballot(l < n && cum >= P.top_p);
    bool near;
    if (b) {
      const int mm = __builtin_ctzll(b);
      const double cm = lane_read(cum, mm);
      const double cp = lane_read(cum, mm > 0 ? mm - 1 : 0);
      near = fabs(cm - P.top_p) <= tol * cm || (mm > 0 && fabs(cp - P.top_p) <= tol * cp);
      // the group of the cut entry's value (contiguous lanes, ascending ids,
      // all inside the top-k set) keeps mm + 1 - g0 of its members, spread
      // over its ids
      const uint64_t kcut = lane_read(key, mm);
      const uint64_t g = ballot(l < n && key == kcut);
      const int g0 = __builtin_ctzll(g), g1 = 64 - __builtin_clzll(g);
      keep = l < g0 || (l < g1 && spread_keeps(l - g0, mm + 1 - g0, g1 - g0, net));
    } else {
      const double cl = lane_read(cum, n - 1);
      near = fabs(cl - P.top_p) <= tol * cl;
    }
    if (near) return LEAN_NEAR;                        // exact fp64 normaliser needed
  }
  if (P.min_p > 0.0) {                                 // sampler.py:91-93
    const double floor_p = P.min_p * lane_read(Pj, 0);
    keep = keep && !(Pj < floor_p);
  }
  // (3) normalise and draw in token-id order (sampler.py:123-127; choice ==
  // searchsorted(cumsum / last, u, 'right')): the kept mass goes to its id
  // rank, lane l sums id ranks 4l .. 4l + 3, and a scan over the lanes gives
  // the cumulative mass at every id rank
  const double qv = keep ? Pj : 0.0;
  const double Z = wave_reduce(qv, OpAdd());
  if (keep) L->oq[rid] = qv / Z;
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  static_assert(LEAN_CAP == 4 * 64, "four id ranks per lane");
  double f[4];
  double run = 0.0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = 4 * l + i;
    run += p < nlist ? L->oq[p] : 0.0;
    f[i] = run;
  }
  const double incl = wave_scan_dpp(run);
  double base = __shfl_up(incl, 1);
  if (l == 0) base = 0.0;
  const double last = lane_read(incl, 63);
  int first = INT_MAX;
#pragma unroll
  for (int i = 3; i >= 0; --i)
    if (4 * l + i < nlist && (base + f[i]) / last > u) first = 4 * l + i;
  const uint64_t b = ballot(first != INT_MAX);
  tok = b ? L->oid[lane_read(first, __builtin_ctzll(b))] : wave_reduce(keep ? idx : -1, OpMax());
  return LEAN_DONE;
}

// ------------------------------------------------------------ penalty corrections
// Per wave: the sum of the raw and the penalised terms of the window ids its
// threads own, against the wave's integer exponent offset Rc (every term
// <= 1), and the largest penalised value.
struct PenRec {
  double corr, pr, pmx, Rc;
  double corrx, prx, refx;   // fp64 exact: penalised-minus-raw and raw terms against refx
  int fl, pad;
};

// The penalty work after the stream is shared out dynamically: waves take
// 64-entry groups of the dense list from an LDS counter as their streams
// end, so the waves that finish first do it and the last one usually finds
// nothing left.

// Next group of the dense list for this wave, or -1 when none is left.
__device__ __forceinline__ int next_group(CX_LDS int* ctr, int ngroups) {
  int g = 0;
  if (lane_id() == 0) g = __hip_atomic_fetch_add(ctr, 1, CX_RELAXED_WG);
  g = __builtin_amdgcn_readfirstlane(g);
  return g < ngroups ? g : -1;
}

// The penalty corrections of the groups this wave takes.  Per group: each
// id's raw logit into hval, its penalised value into the region list when
// at or above thr_w, and, against the record's exponent Rc (the running
// ceil(max * c), rescaled exactly when it rises), the raw terms (pr) and
// the penalised-minus-raw terms (corr): fp32 terms each <= 1 and within
// TOL_T of the exact ones.
template <bool BF16, bool EXACT>
__device__ __forceinline__ void pen_correct(const PenIndex& X, int nd, CX_LDS int* gctr,
                                            const char* rowp, const cx_row_params& P, double kc,
                                            double thr_w, CX_LDS uint64_t* lgk,
                                            CX_LDS int32_t* lgi, CX_LDS int* lcnt, PenRec* rec,
                                            bool ex, double invT, const double* etab) {
  double corr = 0.0, pr = 0.0, pmx = -__builtin_inf(), Rc = 0.0;
  XSum cx{0.0, -__builtin_inf()}, px{0.0, -__builtin_inf()};
  int fl = 0;
  bool any = false;
  const int ngroups = (nd + 63) >> 6;
  for (int g = next_group(gctr, ngroups); g >= 0; g = next_group(gctr, ngroups)) {
    const int j = g * 64 + lane_id();
    const bool v = j < nd;
    const int slot = v ? X.dense[j] : 0;
    const uint32_t hw = v ? X.hword[slot] : 0u;
    const float raw = v ? Elem<BF16>::scalar(rowp, (int)(hw >> 12)) : 0.0f;
    const double xp = v ? penalise(raw, (int)(hw & 0xFFFu), P) : -__builtin_inf();
    double pm = -__builtin_inf();
    if (v) {
      X.hval[slot] = raw;
      pm = (double)raw > pm ? (double)raw : pm;
      pm = xp > pm ? xp : pm;
      if (xp >= thr_w) {
        const int pos = __hip_atomic_fetch_add(lcnt, 1, CX_RELAXED_WG);
        if (pos < LEAN_CAP) { lgk[pos] = d2key(xp); lgi[pos] = (int32_t)(hw >> 12); }
      }
    }
    pm = wave_reduce(pm, OpMax());
    // NaN / +-inf windows leave the exponent at 0 (their rows go to the
    // exact kernel)
    const double Rg = (pm > -__builtin_inf() && pm < __builtin_inf()) ? ceil(pm * kc) : 0.0;
    if (!any || Rg > Rc) {
      if (any) {
        const int d = (int)fmax(Rc - Rg, -2048.0);
        corr = corr != 0.0 ? __builtin_ldexp(corr, d) : 0.0;
        pr = pr != 0.0 ? __builtin_ldexp(pr, d) : 0.0;
      }
      Rc = Rg;
      any = true;
    }
    double tr = 0.0, tp = 0.0;
    if (v) {
      tr = (double)__builtin_amdgcn_exp2f((float)((double)raw * kc - Rc));
      tp = (double)__builtin_amdgcn_exp2f((float)(xp * kc - Rc));
      if (xp != xp) fl = 1;
      else pmx = xp > pmx ? xp : pmx;
    }
    corr += wave_reduce(tp - tr, OpAdd());
    pr += wave_reduce(tr, OpAdd());
    if (EXACT && ex && pm > -__builtin_inf() && pm < __builtin_inf()) {
      // the same in fp64 against the running maximum pm
      xsum_raise(cx, pm, invT, etab);
      xsum_raise(px, pm, invT, etab);
      double tpx = 0.0, trx = 0.0;
      if (v && xp == xp) {
        tpx = exp64_neg((xp - cx.m) * invT, etab);
        trx = exp64_neg(((double)raw - cx.m) * invT, etab);
      }
      cx.s += wave_reduce(tpx - trx, OpAdd());
      px.s += wave_reduce(trx, OpAdd());
    }
  }
  pmx = wave_reduce(pmx, OpMax());
  fl = wave_reduce(fl, OpOr());
  if (lane_id() == 0) {
    rec->corr = corr; rec->pr = pr; rec->pmx = pmx; rec->Rc = Rc; rec->fl = fl;
    rec->corrx = cx.s; rec->prx = px.s; rec->refx = cx.m;
  }
}

// ------------------------------------------------------------ the kernel
// EXACT: the kernel of sliced launches (nsplit > 1), whose stochastic top-p
// rows also keep the exact fp64 normaliser of each slice (XSum).
template <bool BF16, bool EXACT>
__global__ __launch_bounds__(WG) void sample_kernel(SampleArgs A) {
  using E = Elem<BF16>;
  constexpr int NE = E::NE;
  constexpr int U = E::U;
  constexpr int CH = 64 * U;
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ double red_d[2 * NWAVE + 4];
  __shared__ int red_i[2 * NWAVE + 4];
  __shared__ double w_s[NWAVE];
  __shared__ PenRec s_pen[NWAVE];
  __shared__ float w_R[NWAVE];
  __shared__ uint32_t w_tau[NWAVE], w_kmx[NWAVE];
  __shared__ int w_fl[NWAVE];
  __shared__ int w_cnt[NWAVE];
  __shared__ uint32_t s_shared;
  __shared__ uint32_t w_pub[NWAVE];
  __shared__ uint32_t slots[4 * NWAVE];
  __shared__ int s_chunk;
  __shared__ int s_cnt;                       // the one-wave top-k finish's list (pen_correct's too)
  __shared__ int s_rcnt;                      // region entries written (general rows)
  __shared__ LeanLds s_lean;

  __shared__ int s_nd;
  __shared__ int s_gctr;
  __shared__ double s_etab[EXACT ? 64 : 1];   // EXP64_TAB, for the exact sums
  __shared__ double w_xs[EXACT ? NWAVE : 1], w_xm[EXACT ? NWAVE : 1];
  const int row = blockIdx.x / A.nsplit;
  const int split = blockIdx.x % A.nsplit;
  const int t = threadIdx.x;
  const int lo = split * A.split_len;
  const int hi = min(A.V, lo + A.split_len);
  const char* rowp = (const char*)A.logits + (size_t)row * (size_t)A.ld * (BF16 ? 2 : 4);
  const bool single = A.nsplit == 1;
  SplitStats* my = A.stats + (size_t)row * A.nsplit + split;
  Cand* mycand = A.cands + ((size_t)row * A.nsplit + split) * CAPS;

  // Vector loads first, before anything waits: the row's first HPT * WG
  // history entries (where the window starts is known only with the
  // parameters), then this wave's first chunk (wave_id; its second,
  // wave_id + NWAVE, follows after the first barrier, and the LDS counter
  // hands out the rest from 2 * NWAVE on).  Every workgroup asks for its
  // first chunks at once when the grid starts: holding the second ones back
  // until the index tables are cleared halves that queue, and the ids and
  // first chunks behind it arrive sooner.  All are unconditional
  // range-checked buffer loads, so waiting for the ids does not wait for
  // the chunks.
  const bool has_hist = A.ldh > 0;
  const int hcov = has_hist ? (int)min((int64_t)HPT * WG, A.ldh) : 0;
  const __amdgpu_buffer_rsrc_t hrs =
      row_rsrc(has_hist ? (const void*)(A.hist + (size_t)row * A.ldh) : nullptr, hcov * 4);
  int32_t hid[HPT];
#pragma unroll
  for (int k = 0; k < HPT; ++k)
    hid[k] = (int)__builtin_amdgcn_raw_buffer_load_b32(hrs, (t + k * WG) * 4, 0, 0);
  const int nv = A.vec_ok ? (hi - lo) / NE : 0;       // whole vectors of the slice
  const int s0 = lo + nv * NE;                         // first scalar element
  const __amdgpu_buffer_rsrc_t rs = row_rsrc(rowp + (size_t)lo * (BF16 ? 2 : 4), nv * 16);
  const int ch0 = __builtin_amdgcn_readfirstlane(wave_id());
  typename E::V q[U], qn[U];
  load_chunk<BF16>(rs, ch0, q);
  // a row's hand-off mark and finish16_kernel's work-item counter start at
  // zero (the workspace may hold a previous call's records of another
  // layout)
  if (split == 0 && t == 0) A.counters[row] = 0;
  if (blockIdx.x == 0 && t == 0) A.counters[A.B] = 0;

  // the row's parameters live in LDS after the first barrier (P), not in
  // registers across the stream; P0 serves the prologue
  __shared__ cx_row_params sP;
  const RowScalars RS = sload_row(A.prm + row, A.u + row,
                                  has_hist ? A.hist_len + row : (const int32_t*)(A.u + row));
  const cx_row_params& P0 = RS.p;
  const double u_row = RS.u;
  const bool greedy = P0.temperature == 0.0;
  int wlen = 0, wstart = 0;
  if (has_hist) {
    const int len = max(0, min(RS.hlen, (int)A.ldh));
    wstart = P0.n_keep > 0 ? max(0, len - max(64, P0.n_keep)) : 0;
    wlen = len - wstart;
  }
  const bool pen_on = wlen > 0 && (P0.repetition_penalty != 1.0 || P0.presence_penalty != 0.0 ||
                                   P0.frequency_penalty != 0.0);
  if (pen_on && wlen > WIN_MAX) {                    // window longer than the LDS index
    if (t == 0) {
      my->flags = SF_UNSUPPORTED; my->ncand = 0; my->tau = 1u;
      my->m = 0; my->s = 0; my->tol = 0; my->best_i = INT_MAX; my->nan_i = INT_MAX;
    }
    if (single) write_row_result(A, row, CX_ROW_UNSUPPORTED, -1);
    return;
  }

  PenIndex X;
  X.bitmap = to_lds((uint32_t*)(dyn + A.off_bitmap));
  X.hword = to_lds((uint32_t*)(dyn + A.off_hword));
  X.hval = to_lds((float*)(dyn + A.off_hval));
  X.dense = to_lds((int32_t*)(dyn + A.off_dense));
  X.nbw = (hi - lo + 31) >> 5;
  X.ns = pen_on ? A.ns : 0;
  X.ns_log2 = A.ns_log2;
  if (t == 0) {
    sP = P0; s_shared = 1u; s_chunk = 2 * NWAVE; s_cnt = 0; s_rcnt = 0; s_nd = 0; s_gctr = 0;
  }
  if (t < LEAN_CAP) { s_lean.rv[t] = 0; s_lean.ri[t] = 0; }
  if (t < NWAVE) { w_pub[t] = 0u; w_cnt[t] = 0; }
  if (t < 4 * NWAVE) slots[t] = 0u;
  if (EXACT && t < 64) s_etab[t] = EXP64_TAB[t];
  if (pen_on) {
    for (int i = t; i < X.nbw; i += WG) X.bitmap[i] = 0u;
    for (int i = t; i < X.ns; i += WG) X.hword[i] = HW_EMPTY;
  }
  __syncthreads();
  const cx_row_params& P = sP;
  // A single-slice bf16 row that may take the counted deep-nucleus path
  // (finish16_kernel counts its values, finding its maximum as it goes, and
  // decides it exactly or hands it to the exact path) is not streamed here:
  // counting reads the row once.  (Its region would be a candidate list its
  // nucleus usually outgrows, or, for top-k above 256, one whose upkeep
  // here, ~50 us a row, costs about what counting the row there does.)
  // Top-k rows up to 64 keep the one-wave finish below, those up to 256 the
  // region finisher.  (Counting every top-k row above 64 left the counting
  // kernel three rounds of workgroups deep: 400 instead of 337 us.)  Such a
  // row has no penalty window, so nothing below is needed for it.
  const bool count_row = BF16 && single && !greedy && !A.out_probs &&
                         !(P.top_k > 0 && P.top_k <= 256) && deep_candidate(A, row, P, true);
  if (count_row) {
    if (t == 0) {
      // no maximum yet (NaN): the counting path finds it and records it
      my->m = __builtin_nan(""); my->s = 0; my->tol = 0; my->best_v = 0;
      my->best_i = INT_MAX; my->nan_i = INT_MAX; my->tau = 1u; my->ncand = 0; my->flags = 0;
      A.out_id[row] = -1;
      A.row_status[row] = ROW_PENDING;
      A.counters[row] = ROW_PENDING | MARK_DEEP | (P.top_k > 0 && P.top_k < A.V ? MARK_TOPK : 0);
    }
    return;
  }
  load_chunk<BF16>(rs, ch0 + NWAVE, qn);
  // index the window entries [wstart, wstart + wlen) whose ids fall in the
  // slice: a bitmap bit and a hash word (id << 12 | count) per distinct id,
  // whose slot its first inserter appends to the dense list
  if (pen_on) {
    const int wend = wstart + wlen;
    auto index_id = [&](int id) {
      if (id >= lo && id < hi) {
        __hip_atomic_fetch_or(X.bitmap + ((id - lo) >> 5), 1u << ((id - lo) & 31), CX_RELAXED_WG);
        bool created;
        const int slot = pen_insert(X, id, created);
        if (created) X.dense[__hip_atomic_fetch_add(to_lds(&s_nd), 1, CX_RELAXED_WG)] = slot;
      }
    };
#pragma unroll
    for (int k = 0; k < HPT; ++k) {
      const int i = t + k * WG;
      if (i >= wstart && i < wend) index_id(hid[k]);
    }
    // windows reaching past the entries loaded up front
    for (int i = max(wstart, HPT * WG) + t; i < wend; i += WG)
      index_id(A.hist[(size_t)row * A.ldh + i]);
  }
  __syncthreads();
  const int nd = pen_on ? s_nd : 0;
  CX_LDS int* const gctr = to_lds(&s_gctr);
  // ---------------------------------------------------------------- greedy
  if (greedy) {
    GreedyState gs{-__builtin_inff(), INT_MAX, INT_MAX};
    stream_greedy<BF16>(rowp, rs, q, qn, nv, lo, hi, s0, pen_on, X, to_lds(&s_chunk), gs);
    double bv = gs.bi == INT_MAX ? -__builtin_inf() : (double)gs.bv;
    int bi = gs.bi;
    int ni = gs.nan_i;
    // the window ids' penalised values (groups of the dense list, taken as
    // the waves' streams end)
    const int ngroups = (nd + 63) >> 6;
    for (int g = next_group(gctr, ngroups); g >= 0; g = next_group(gctr, ngroups)) {
      const int j = g * 64 + lane_id();
      if (j < nd) {
        const uint32_t hw = X.hword[X.dense[j]];
        const int id = (int)(hw >> 12);
        const double xp = penalise(E::scalar(rowp, id), (int)(hw & 0xFFFu), P);
        if (xp != xp) ni = min(ni, id);
        else argmax_merge(bv, bi, xp, id);
      }
    }
    block_argmax(bv, bi, red_d, red_i);
    ni = block_min(ni, red_i, INT_MAX);
    if (single) {
      const int tok = ni != INT_MAX ? ni : (bi == INT_MAX ? 0 : bi);
      write_row_result(A, row, CX_ROW_GREEDY, tok);
      write_one_hot(A, row, tok);
    } else if (t == 0) {
      my->m = 0; my->s = 0; my->tol = 0; my->best_v = bv; my->best_i = bi; my->nan_i = ni;
      my->tau = 1u; my->ncand = 0; my->flags = 0;
    }
    return;
  }

  // ---------------------------------------------------------------- stochastic
  const float c = (float)(1.4426950408889634 / P.temperature);
  const double kc = (double)c;
  // the exact fp64 slice normaliser: sliced top-p rows, whose cut the
  // finisher otherwise could only refine with a second read of the row;
  // split (XSum) for rows with neither a penalty window nor a top-k whose
  // slice is whole vectors, full for the others
  const bool exs = EXACT && P.top_p < 1.0 && P.top_k <= 0 && !pen_on && s0 >= hi;
  const bool ex = EXACT && P.top_p < 1.0 && !exs;
  const double invT = 1.0 / P.temperature;
  const double* etab = EXACT ? (const double*)s_etab : nullptr;
  XSum xs{0.0, -__builtin_inf()};
  WaveBuf wb;
  wb.key = to_lds((uint32_t*)(dyn + A.off_wkey) + wave_id() * CAPW);
  wb.idx = to_lds((int32_t*)(dyn + A.off_widx) + wave_id() * CAPW);
  wb.shared = to_lds(&s_shared);
  wb.cnt = to_lds(&w_cnt[wave_id()]);
  wb.n = 0;
  wb.tau = 1u;
  wb.tauf = -__builtin_inff();
  wb.overflow = false;
  wb.xn = 0;
  wb.lossy = false;
  // Entries a wave keeps: k for top-k rows; otherwise an equal share of the
  // region finisher's capacity, so the merged region fits in its LDS.
  const int share = max(8, min(KW_MAX, FIN_CAP / (NWAVE * A.nsplit)));
  wb.kw = P.top_k > 0 ? min(P.top_k, KW_MAX) : share;
  // elements the shared threshold must leave: k of a top-k row, or for a
  // top-p row 1024 region entries, or the slice's share of the finisher's
  // capacity if that is less (a lower first threshold only adds appends and
  // compactions)
  const int krow = P.top_k > 0 ? P.top_k : min(FIN_CAP / 4, NWAVE * share);
  const int pub_r = krow > 64 && krow <= 64 * NWAVE ? (krow + NWAVE - 1) / NWAVE : 0;
  CX_LDS uint32_t* const lslots = to_lds(slots);
  CX_LDS uint32_t* const lpub = to_lds(w_pub);

  // seed: every lane's largest unpenalised element of its first chunk (a
  // vector's NE penalty bits sit in one bitmap word: one LDS read each),
  // and for wide rows (below) its second largest, in the same pass
  uint32_t ck = 0u, c2 = 0u;
  const bool two = krow > 64 && pub_r >= 32;
  if (wave_id() * CH < nv) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int vi = wave_id() * CH + u * 64 + lane_id();
      float x[NE];
      E::unpack(q[u], x);
      const uint32_t pb = pen_bits<NE>(X, pen_on && vi < nv, vi * NE);
#pragma unroll
      for (int j = 0; j < NE; ++j) {
        const bool ok = vi < nv && x[j] == x[j] && !((pb >> j) & 1u);
        const uint32_t k = ok ? f2key(x[j]) : 0u;
        if (two) c2 = k > ck ? ck : (k > c2 ? k : c2);
        ck = k > ck ? k : ck;
      }
    }
  }
  // The waves' first chunks together set the first threshold: for top-k
  // rows (k <= 64) the k-th largest of the published lane values, for wider
  // rows the smallest of the waves' r-th largest of their lanes' two largest
  // values (every one an element, so each wave holds r elements at or
  // above it).  (A wave's own lane values alone give a threshold too low to
  // keep the first chunks' appends cheap, and with r = 64 the lane maxima
  // alone give their smallest.)
  // (The selections stop at the keys' upper 16 bits: sign, exponent and 7
  // mantissa bits, a threshold lower by at most 1/128 of its magnitude.)
  if (krow <= 64) {
    publish_top(ck, NSLOT, lslots + NSLOT * wave_id());
    __syncthreads();
    raise_tau(wb, kth_of_lanes(lds_load(lslots + lane_id()), krow, 16));
  } else if (pub_r > 0) {
    // for r of 32 and more, the lanes' second largest values too (for
    // smaller r the r-th largest lane maximum is already high)
    const uint32_t th = two ? kth_of_lanes2(ck, c2, pub_r, 16) : kth_of_lanes(ck, pub_r, 16);
    if (lane_id() == 0) lpub[wave_id()] = th;
    __syncthreads();
    raise_tau(wb, pub_min(lpub));
  }

  SState st{-__builtin_inff(), 3.402823466e38f, -__builtin_inff(), 0.0};
  uint64_t* gk = (uint64_t*)(dyn + A.off_gather);
  int32_t* gi = (int32_t*)(dyn + A.off_gather + LEAN_CAP * 8);
  CX_LDS uint64_t* const lgk = to_lds(gk);
  CX_LDS int32_t* const lgi = to_lds(gi);
  CX_LDS int* const lcnt = to_lds(&s_cnt);
  {
    CX_LDS int* const cc = to_lds(&s_chunk);
    stream_stoch<BF16, EXACT>(rs, q, qn, nv, lo, pen_on, X, c, krow, pub_r, cc, lslots, lpub,
                              st, wb, ck, ex, exs, invT, etab, xs);
  }
  if (s0 < hi) {
    raise_tau(wb, lds_load(wb.shared));
    stream_scalar<BF16, EXACT>(rowp, s0, lo, hi, pen_on, X, c, true, st, wb, ck, ex, invT, etab,
                               xs);
  }

  // ---- per wave, after its stream: its region entries into the shared
  // list (the one-wave top-k finish's, so only for its rows), its penalty
  // corrections (with the penalised values at or above its threshold), its
  // sums and state for the combination
  // Top-k rows the rank-parallel finish can take (static conditions).
  const bool lean_static = single && P.top_k > 0 && P.top_k <= 64 && P.typical_p >= 1.0 &&
                           !A.out_probs && A.logV * (1.0 / P.temperature) <= 740.0;
  raise_tau(wb, lds_load(wb.shared));
  // lanes read below the buffer entries other lanes of the wave wrote (in
  // order on the hardware; the barrier keeps the compiler from hoisting)
  __builtin_amdgcn_wave_barrier();
  if (lean_static) {
    const int n = wb.n;
    for (int e = lane_id(); e < n; e += 64) {
      const uint32_t k = wb.key[e];
      if (k >= wb.tau) {
        const int pos = __hip_atomic_fetch_add(lcnt, 1, CX_RELAXED_WG);
        if (pos < LEAN_CAP) { lgk[pos] = d2key((double)key2f(k)); lgi[pos] = wb.idx[e]; }
      }
    }
  }
  if (pen_on) {
    pen_correct<BF16, EXACT>(X, nd, gctr, rowp, P, kc,
                             wb.tau <= 1u ? -__builtin_inf() : (double)wb.tauf, lgk, lgi, lcnt,
                             &s_pen[wave_id()], ex, invT, etab);
  } else if (lane_id() == 0) {
    s_pen[wave_id()].corr = 0.0; s_pen[wave_id()].pr = 0.0; s_pen[wave_id()].pmx = -__builtin_inf();
    s_pen[wave_id()].Rc = 0.0; s_pen[wave_id()].fl = 0;
    s_pen[wave_id()].corrx = 0.0; s_pen[wave_id()].prx = 0.0;
    s_pen[wave_id()].refx = -__builtin_inf();
  }
  // split sum: the entries buffered since the last compaction
  if (EXACT && exs) xsum_entries(wb, wb.xn, wb.n, invT, etab, xs);
  if (EXACT && (ex || exs)) {
    // the wave's exact sum against its largest value
    const double Mw = wave_reduce(xs.m, OpMax());
    double v = xs.s != 0.0 ? xs.s * exp64_neg((xs.m - Mw) * invT, etab) : 0.0;
    v = wave_reduce(v, OpAdd());
    if (lane_id() == 0) { w_xs[wave_id()] = v; w_xm[wave_id()] = Mw; }
  }
  const float Rw = wave_reduce(st.R, OpMax());
  double sl = st.s != 0.0 ? __builtin_ldexp(st.s, (int)fmaxf(st.R - Rw, -2048.0f)) : 0.0;
  sl = wave_reduce(sl, OpAdd());
  const uint32_t kmx_w = wave_reduce(ck, OpMax());
  const int fl = wave_reduce(st.s != st.s ? 1 : 0, OpOr());
  if (krow <= 64 && !lean_static) publish_top(ck, NSLOT, lslots + NSLOT * wave_id());
  if (lane_id() == 0) {
    w_s[wave_id()] = sl;
    w_R[wave_id()] = Rw;
    w_tau[wave_id()] = wb.tau;
    w_kmx[wave_id()] = kmx_w;
    w_fl[wave_id()] = fl | (wb.overflow ? 2 : 0) | (wb.lossy ? 4 : 0);
    w_cnt[wave_id()] = wb.n;
  }
  __syncthreads();
  const int lw = lane_id() & 15;       // lane w of row 0 reads wave w's record

  // ---- top-k finish: wave 0 combines the sums while the other waves rank
  // the region list; then wave 0 decides.  A row it cannot decide (inexact
  // sum, tie flood, long list, near a top-p boundary) is left pending for
  // the exact kernel.
  if (lean_static) {
    CX_LDS LeanLds* const L = to_lds(&s_lean);
    const int nlist = s_cnt;
    const bool list_ok = nlist > 0 && nlist <= LEAN_CAP;
    double Rb = 0.0, Ss = 0.0, tol = 0.0;
    bool ok = false;
    if (wave_id() == 0) {
      // S = sum over waves of 2^(Rw - Rb) s_w + 2^(Rc_w - Rb) corr_w
      const float Rl = w_R[lw];
      const double Rcl = s_pen[lw].Rc;
      const float Rf = row0_reduce(Rl, OpMax());
      const int flw = row0_reduce(w_fl[lw] | s_pen[lw].fl, OpOr());
      Rb = fmax((double)Rf, row0_reduce(Rcl, OpMax()));
      // an exponent offset past +-2^22 leaves fp32 term arguments inexact
      const bool rb_ok = Rf > -__builtin_inff() && fabs(Rb) < 4194304.0;
      double PR = 0.0;
      if (rb_ok) {
        const double sw = w_s[lw];
        const double cw = s_pen[lw].corr, pw = s_pen[lw].pr;
        const int dc = (int)fmax(Rcl - Rb, -2048.0);
        const double term =
            (sw != 0.0 ? __builtin_ldexp(sw, (int)fmax((double)Rl - Rb, -2048.0)) : 0.0) +
            (cw != 0.0 ? __builtin_ldexp(cw, dc) : 0.0);
        Ss = row0_reduce(term, OpAdd());
        PR = row0_reduce(pw != 0.0 ? __builtin_ldexp(pw, dc) : 0.0, OpAdd());
      }
      tol = TOL_S + 2.0 * TOL_T * PR / Ss;
      ok = flw == 0 && rb_ok && Ss > 0.0 && Ss < __builtin_inf() && tol <= TOL_MAX && list_ok;
    } else if (list_ok) {
      lean_ranks(lgk, lgi, nlist, L);
    }
    __syncthreads();
    if (wave_id() != 0) return;
    int tok = -1;
    const int dr = ok ? lean_decide(P, lgk, lgi, nlist, kc, Rb, Ss, tol, L, u_row,
                                    A.V <= TIE_NET, tok)
                      : LEAN_PENDING;
    if (dr == LEAN_NEAR) {
      // the list as the row's region (every element at or above the largest
      // wave threshold), for the exact-normaliser refinement
      uint64_t kmax = 0ull;
      for (int e = lane_id(); e < nlist; e += 64) {
        const uint64_t k = lgk[e];
        mycand[e].key = k;
        mycand[e].idx = lgi[e];
        kmax = k > kmax ? k : kmax;
      }
      kmax = wave_reduce(kmax, OpMax());
      const uint32_t tmax = row0_reduce(w_tau[lw], OpMax());
      if (lane_id() == 0) {
        my->m = key2d(kmax);
        my->s = Ss;
        my->tol = tol;
        my->best_v = 0; my->best_i = INT_MAX; my->nan_i = INT_MAX;
        my->tau = tmax; my->ncand = nlist; my->flags = 0;
      }
    }
    if (lane_id() == 0) {
      const int mark = dr == LEAN_DONE ? 0 : (dr == LEAN_NEAR ? ROW_REFINE : ROW_PENDING);
      A.out_id[row] = dr == LEAN_DONE ? tok : -1;
      A.row_status[row] = mark ? mark : CX_ROW_OK;
      A.counters[row] = mark | (mark && deep_candidate(A, row, P, true) ? MARK_DEEP | MARK_TOPK : 0);
    }
    return;
  }

  // ---- combine: S = sum over waves of 2^(Rw - Rb) s_w + 2^(Rc_w - Rb) corr_w
  const float Rl = w_R[lw];
  const double Rcl = s_pen[lw].Rc;
  uint32_t Tf = row0_reduce(w_tau[lw], OpMax());
  const uint32_t kmx = row0_reduce(w_kmx[lw], OpMax());
  const int flw = row0_reduce(w_fl[lw] | s_pen[lw].fl, OpOr());
  const int anynan = flw & 1, ovf = flw & 2;
  if (krow <= 64) Tf = max(Tf, kth_of_lanes(lds_load(lslots + lane_id()), krow));
  // The slice's sums for its record are taken by wave 0 alone, after its
  // share of the region (below): the other waves need only Tf and kmx.
  double Ss = 0.0, tol = 0.0, Rb = 0.0, Ms = 0.0, Sx = 0.0, xtol = 0.0;
  bool sum_ok = false, xok = false;
  auto slice_sums = [&]() {
    const float Rf = row0_reduce(Rl, OpMax());
    const double PMX = row0_reduce(s_pen[lw].pmx, OpMax());
    Rb = fmax((double)Rf, row0_reduce(Rcl, OpMax()));
    // an exponent offset past +-2^22 leaves fp32 term arguments inexact
    const bool rb_ok = Rf > -__builtin_inff() && fabs(Rb) < 4194304.0;
    double PR = 0.0;
    if (rb_ok) {
      const double sw = w_s[lw];
      const double cw = s_pen[lw].corr, pw = s_pen[lw].pr;
      const int dc = (int)fmax(Rcl - Rb, -2048.0);
      const double term =
          (sw != 0.0 ? __builtin_ldexp(sw, (int)fmax((double)Rl - Rb, -2048.0)) : 0.0) +
          (cw != 0.0 ? __builtin_ldexp(cw, dc) : 0.0);
      Ss = row0_reduce(term, OpAdd());
      PR = row0_reduce(pw != 0.0 ? __builtin_ldexp(pw, dc) : 0.0, OpAdd());
    }
    tol = TOL_S + 2.0 * TOL_T * PR / Ss;
    sum_ok = !anynan && rb_ok && Ss > 0.0 && Ss < __builtin_inf() && tol <= TOL_MAX;
    // the slice's exact fp64 normaliser against its maximum Ms: the waves'
    // sums and their penalty corrections, each rescaled to Ms (lane w of
    // each row of 16 lanes takes wave w).  Kept where the raw terms the
    // corrections replace are not so large that cancelling them loses the
    // sum's precision.
    const double Mu = kmx ? (double)key2f(kmx) : -__builtin_inf();
    Ms = Mu > PMX ? Mu : PMX;
    if (EXACT && ex && sum_ok && Ms > -__builtin_inf() && Ms < __builtin_inf()) {
      const double f = s_pen[lw].refx > -__builtin_inf()
                           ? exp64_neg((s_pen[lw].refx - Ms) * invT, etab) : 0.0;
      const double ws = w_xs[lw];
      const double term = (ws != 0.0 ? ws * exp64_neg((w_xm[lw] - Ms) * invT, etab) : 0.0) +
                          s_pen[lw].corrx * f;
      Sx = row0_reduce(term, OpAdd());
      const double PRx = row0_reduce(s_pen[lw].prx * f, OpAdd());
      xok = Sx > 0.0 && Sx < __builtin_inf() && PRx < 1e5 * Sx;
    }
    if (EXACT && exs && !anynan && rb_ok && !(flw & 4) && Ss < __builtin_inf() &&
        Ms > -__builtin_inf() && Ms < __builtin_inf()) {
      // split (Ss holds only the below-threshold terms, and may be 0): the
      // buffered entries' exact terms plus the below-threshold ones, both
      // against Ms; the bound is TOL_S of the latter (with a margin for the
      // fp64 roundings of the sums)
      const double ws = w_xs[lw];
      const double Sa = row0_reduce(
          ws != 0.0 ? ws * exp64_neg((w_xm[lw] - Ms) * invT, etab) : 0.0, OpAdd());
      const double Stm = Ss != 0.0 ? Ss * exp2(Rb - Ms * kc) : 0.0;
      Sx = Sa + Stm;
      xok = Sx > 0.0 && Sx < __builtin_inf();
      xtol = xok ? TOL_S * Stm / Sx + 1e-12 : 0.0;
    }
  };

  // ---- general: bound the region, write it and the statistics, then finish
  // The region is every buffered entry at or above T, and every element at
  // or above Tf is buffered.  T is the lowest boundary of a 512-bin
  // histogram of the buffered keys in [Tf, kmx] with at most NWAVE * kw
  // entries at or above it (the same bound the waves' own compactions to kw
  // entries gave, in one pass and one barrier).  The bins are the top-k
  // finish's rank counters, zeroed at the start and unused on this path.
  // Whole-row buffers holding no more than the cap in all (most top-k 100
  // rows of a 256000-entry vocabulary) need no histogram: T is Tf.  A
  // slice's buffers nearly always exceed it, so the sliced launch does not
  // test.
  const int cap = NWAVE * wb.kw;
  const uint32_t tlo = Tf > 1u ? Tf : 1u;
  if (!EXACT && row0_reduce(w_cnt[lw], OpAdd()) <= cap) {
    Tf = tlo;
  } else {
    static_assert(2 * LEAN_CAP == 512, "histogram bins");
    CX_LDS int* const bins = to_lds(&s_lean.rv[0]);     // rv, then ri: 512 counters
    const uint32_t lo = tlo;
    const uint32_t d = kmx > lo ? kmx - lo : 0u;
    const int sh = d ? max(0, 23 - (int)__clz(d)) : 0;  // d >> sh < 512
    const uint32_t base = lo >> sh;
    __builtin_amdgcn_wave_barrier();
    for (int e = lane_id(); e < wb.n; e += 64) {
      const uint32_t k = wb.key[e];
      if (k >= lo) __hip_atomic_fetch_add(bins + min((int)((k >> sh) - base), 511), 1,
                                          CX_RELAXED_WG);
    }
    __syncthreads();
    // every wave: lane l holds bins 8l .. 8l + 7; the lowest bin b whose
    // suffix count is at most the cap
    int cb[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) cb[j] = lds_load(bins + 8 * lane_id() + j);
    int lsum = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) lsum += cb[j];
    const int incl = wave_scan_dpp(lsum);
    int cum = __builtin_amdgcn_readlane(incl, 63) - incl;     // entries in the bins above
    int low = 512;
#pragma unroll
    for (int j = 7; j >= 0; --j) {
      cum += cb[j];
      if (cum <= cap) low = 8 * lane_id() + j;
    }
    low = wave_reduce(low, OpMin());
    // all above the cap within the top bin (a flood of near-equal keys):
    // that bin's boundary, the region then over the cap
    low = min(low, 511);
    const uint64_t T = (uint64_t)(base + (uint32_t)low) << sh;
    Tf = T > (uint64_t)lo ? (uint32_t)min(T, (uint64_t)0xFFFFFFFFu) : lo;
  }
  const uint64_t thr64 = Tf <= 1u ? 0ull : d2key((double)key2f(Tf));
  for (int s = t; s < X.ns; s += WG) {
    const uint32_t hw = X.hword[s];
    if (hw == HW_EMPTY) continue;
    const double xp = penalise(X.hval[s], (int)(hw & 0xFFFu), P);
    const uint64_t k64 = d2key(xp);
    if (k64 >= thr64 && xp == xp) {
      const int pos = atomicAdd(&s_rcnt, 1);
      mycand[pos].key = k64;
      mycand[pos].idx = (int32_t)(hw >> 12);
    }
  }
  {
    const int n = wb.n;
    for (int e = lane_id(); e - lane_id() < n; e += 64) {
      const bool keep = e < n && wb.key[e] >= Tf;
      const uint64_t b = ballot(keep);
      int base = 0;
      if (lane_id() == 0 && b) base = atomicAdd(&s_rcnt, (int)__popcll(b));
      base = __shfl(base, 0);
      if (keep) {
        const int pos = base + lanes_below(b);
        mycand[pos].key = d2key((double)key2f(wb.key[e]));
        mycand[pos].idx = wb.idx[e];
      }
    }
  }
  if (wave_id() == 0) slice_sums();
  __syncthreads();
  if (t == 0) {
    // the maximum of the slice's penalised values, and the sums against it
    my->m = Ms;
    my->sx = xok ? Sx : 0.0;
    my->sxtol = (float)(xtol * 1.001);
    my->s = EXACT && exs ? Sx : (sum_ok ? Ss * exp2(Rb - Ms * kc) : Ss);
    my->tol = EXACT && exs ? xtol * 1.001 : tol;
    my->best_v = 0; my->best_i = INT_MAX; my->nan_i = INT_MAX;
    my->tau = Tf; my->ncand = s_rcnt;
    my->flags = (ovf ? SF_OVERFLOW : 0) | ((EXACT && exs ? xok : sum_ok) ? 0 : SF_INEXACT) |
                (xok ? SF_EXACT : 0);
  }
  // The region finisher runs in slow_kernel, after the grid: a kernel
  // boundary makes the slices' records visible across XCDs without
  // per-workgroup cache writebacks, and the finisher's registers stay out of
  // this kernel.  Sliced rows are always finished there; a single-slice row
  // is marked.
  if (single && t == 0) {
    A.row_status[row] = ROW_FINISH;
    // (a top-k row here has a small region: its finisher, not counting, is
    // what it usually needs, so it goes with the rows that cannot go deep)
    A.counters[row] = ROW_FINISH | (deep_candidate(A, row, P) ? MARK_DEEP : 0);
  }
}

template __global__ void sample_kernel<false, false>(SampleArgs);
template __global__ void sample_kernel<true, false>(SampleArgs);
template __global__ void sample_kernel<false, true>(SampleArgs);
template __global__ void sample_kernel<true, true>(SampleArgs);

}  // namespace cx

namespace cx {
int launch_sample(const SampleArgs& A, hipStream_t s) {
  // sliced launches: the kernel that keeps the slices' exact normalisers
  const int v = (A.bf16 ? 1 : 0) + (A.nsplit > 1 ? 2 : 0);
  using K = void (*)(SampleArgs);
  static const K kern[4] = {sample_kernel<false, false>, sample_kernel<true, false>,
                            sample_kernel<false, true>, sample_kernel<true, true>};
  // Raise the dynamic-LDS limit to what this launch needs (static LDS comes on top).
  static int attr_set[4] = {0, 0, 0, 0};
  if (A.lds_bytes > attr_set[v]) {
    hipError_t e = hipFuncSetAttribute((const void*)kern[v],
                                       hipFuncAttributeMaxDynamicSharedMemorySize, A.lds_bytes);
    if (e != hipSuccess) return (int)e;
    attr_set[v] = A.lds_bytes;
  }
  timed_launch(CX_KERNEL_SAMPLE, kern[v], dim3(A.B * A.nsplit), dim3(WG), A.lds_bytes, s, A);
  return (int)hipGetLastError();
}
}  // namespace cx
