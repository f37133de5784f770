// cx_device.hpp -- device building blocks for the gfx950 sampling kernels.
//
// Workgroups are 1024 threads = 16 wave64s.  Everything here is written for
// 64-lane wavefronts: ballots are 64-bit, lane prefix counts use mbcnt, and
// sub-wave exchanges use cross-lane shuffles (ds_swizzle / DPP / bpermute).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <limits.h>

namespace cx {

constexpr int WG = 1024;
constexpr int NWAVE = WG / 64;

// LDS pointers: generic pointers that cross a call or a volatile access
// become flat instructions (which also wait on outstanding global loads);
// address space 3 keeps them ds_* operations.
#define CX_LDS __attribute__((address_space(3)))
// Read-only kernel inputs read through the constant address space: uniform
// reads become scalar loads (SMEM), which complete independently of the
// vector loads in flight.
#define CX_CONST __attribute__((address_space(4)))
template <typename T>
__device__ __forceinline__ T const_load(const T* p) {
  static_assert(sizeof(T) % 4 == 0, "whole dwords");
  T v;
  const CX_CONST uint32_t* s = (const CX_CONST uint32_t*)p;
  uint32_t* d = (uint32_t*)&v;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(T) / 4); ++i) d[i] = s[i];
  return v;
}
template <typename T>
__device__ __forceinline__ CX_LDS T* to_lds(T* p) { return (CX_LDS T*)p; }
template <typename T>
__device__ __forceinline__ T lds_load(const CX_LDS T* p) { return *(const volatile CX_LDS T*)p; }

// ------------------------------------------------------------ orderable keys
// Map a float to an unsigned integer whose unsigned order is the float order
// (-inf < ... < -0 < +0 < ... < +inf).  0 is below every float and serves as
// "no element".
__device__ __forceinline__ uint32_t f2key(float f) {
  uint32_t b = __float_as_uint(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k) {
  uint32_t b = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(b);
}
__device__ __forceinline__ uint64_t d2key(double d) {
  uint64_t b = (uint64_t)__double_as_longlong(d);
  return (b >> 63) ? ~b : (b | (1ull << 63));
}
__device__ __forceinline__ double key2d(uint64_t k) {
  uint64_t b = (k >> 63) ? (k & 0x7fffffffffffffffull) : ~k;
  return __longlong_as_double((long long)b);
}

// ------------------------------------------------------------ lanes
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }
__device__ __forceinline__ uint64_t ballot(bool p) { return __ballot(p); }
__device__ __forceinline__ int lanes_below(uint64_t m) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                   __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}
template <typename T>
__device__ __forceinline__ T uniform(T v) {  // value of the first active lane
  return __shfl(v, __builtin_ctzll(__ballot(1)));
}

template <typename T> __device__ __forceinline__ T wave_max(T v) {
  for (int o = 32; o > 0; o >>= 1) { T w = __shfl_xor(v, o); v = w > v ? w : v; }
  return v;
}
template <typename T> __device__ __forceinline__ T wave_min(T v) {
  for (int o = 32; o > 0; o >>= 1) { T w = __shfl_xor(v, o); v = w < v ? w : v; }
  return v;
}
template <typename T> __device__ __forceinline__ T wave_sum(T v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// (value, index) argmax with NumPy's rule: larger value wins, equal values go
// to the lower index.  NaN is handled separately by the callers.
__device__ __forceinline__ void argmax_merge(double& v, int& i, double w, int j) {
  if (w > v || (w == v && j < i)) { v = w; i = j; }
}
__device__ __forceinline__ void wave_argmax(double& v, int& i) {
  for (int o = 32; o > 0; o >>= 1) {
    double w = __shfl_xor(v, o);
    int j = __shfl_xor(i, o);
    argmax_merge(v, i, w, j);
  }
}

// ------------------------------------------------------------ DPP reductions
// Rotations inside each 16-lane row: one VALU op per 32 bits, no LDS trip.
template <int N> __device__ __forceinline__ uint32_t dpp_ror(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x120 + N, 0xF, 0xF, false);
}
template <int N> __device__ __forceinline__ int dpp_ror(int v) {
  return __builtin_amdgcn_mov_dpp(v, 0x120 + N, 0xF, 0xF, false);
}
template <int N> __device__ __forceinline__ float dpp_ror(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x120 + N, 0xF, 0xF, false));
}
template <int N> __device__ __forceinline__ double dpp_ror(double v) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = dpp_ror<N>((uint32_t)b), hi = dpp_ror<N>((uint32_t)(b >> 32));
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
template <int N> __device__ __forceinline__ uint64_t dpp_ror(uint64_t v) {
  const uint32_t lo = dpp_ror<N>((uint32_t)v), hi = dpp_ror<N>((uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint32_t lane_read(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
__device__ __forceinline__ int lane_read(int v, int l) { return __builtin_amdgcn_readlane(v, l); }
__device__ __forceinline__ float lane_read(float v, int l) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
__device__ __forceinline__ uint64_t lane_read(uint64_t v, int l) {
  const uint32_t lo = lane_read((uint32_t)v, l), hi = lane_read((uint32_t)(v >> 32), l);
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ double lane_read(double v, int l) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = lane_read((uint32_t)b, l), hi = lane_read((uint32_t)(b >> 32), l);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
// Every lane of a 16-lane row receives the row's reduction.
template <typename T, typename Op>
__device__ __forceinline__ T row_reduce(T v, Op op) {
  v = op(v, dpp_ror<8>(v));
  v = op(v, dpp_ror<4>(v));
  v = op(v, dpp_ror<2>(v));
  return op(v, dpp_ror<1>(v));
}
// The whole wave's reduction (uniform); row 0 only: lanes 0-15.
template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
  v = row_reduce(v, op);
  return op(op(lane_read(v, 0), lane_read(v, 16)), op(lane_read(v, 32), lane_read(v, 48)));
}
template <typename T, typename Op>
__device__ __forceinline__ T row0_reduce(T v, Op op) {
  return lane_read(row_reduce(v, op), 0);
}
// Inclusive prefix sum across the 64 lanes with DPP row shifts and row
// broadcasts (no LDS traffic).
template <int CTRL, int ROWS>
__device__ __forceinline__ double dpp_update0(double v) {
  const uint64_t b = (uint64_t)__double_as_longlong(v);
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, ROWS, 0xF, true);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, ROWS, 0xF, true);
  return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double wave_scan_dpp(double v) {
  v += dpp_update0<0x111, 0xF>(v);   // row_shr:1
  v += dpp_update0<0x112, 0xF>(v);   // row_shr:2
  v += dpp_update0<0x114, 0xF>(v);   // row_shr:4
  v += dpp_update0<0x118, 0xF>(v);   // row_shr:8
  v += dpp_update0<0x142, 0xA>(v);   // row_bcast:15 into rows 1 and 3
  v += dpp_update0<0x143, 0xC>(v);   // row_bcast:31 into rows 2 and 3
  return v;
}
template <int CTRL, int ROWS>
__device__ __forceinline__ unsigned long long dpp_update0(unsigned long long b) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)b, CTRL, ROWS, 0xF, true);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(b >> 32), CTRL, ROWS, 0xF, true);
  return ((unsigned long long)hi << 32) | lo;
}
__device__ __forceinline__ unsigned long long wave_scan_dpp(unsigned long long v) {
  v += dpp_update0<0x111, 0xF>(v);
  v += dpp_update0<0x112, 0xF>(v);
  v += dpp_update0<0x114, 0xF>(v);
  v += dpp_update0<0x118, 0xF>(v);
  v += dpp_update0<0x142, 0xA>(v);
  v += dpp_update0<0x143, 0xC>(v);
  return v;
}
__device__ __forceinline__ int wave_scan_dpp(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, true);
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, true);
  return v;
}

struct OpAdd { template <typename T> __device__ T operator()(T a, T b) const { return a + b; } };
struct OpMax { template <typename T> __device__ T operator()(T a, T b) const { return a > b ? a : b; } };
struct OpMin { template <typename T> __device__ T operator()(T a, T b) const { return a < b ? a : b; } };
struct OpOr { template <typename T> __device__ T operator()(T a, T b) const { return a | b; } };
struct OpAnd { template <typename T> __device__ T operator()(T a, T b) const { return a & b; } };

// Block-wide reductions through a small LDS scratch (>= NWAVE slots).
template <typename T>
__device__ __forceinline__ T block_sum(T v, T* scratch) {
  v = wave_sum(v);
  if (lane_id() == 0) scratch[wave_id()] = v;
  __syncthreads();
  T r = 0;
  if (threadIdx.x < 64) {
    r = threadIdx.x < NWAVE ? scratch[threadIdx.x] : T(0);
    r = wave_sum(r);
    if (threadIdx.x == 0) scratch[0] = r;
  }
  __syncthreads();
  r = scratch[0];
  __syncthreads();
  return r;
}
template <typename T>
__device__ __forceinline__ T block_max(T v, T* scratch, T lowest) {
  v = wave_max(v);
  if (lane_id() == 0) scratch[wave_id()] = v;
  __syncthreads();
  if (threadIdx.x < 64) {
    T r = threadIdx.x < NWAVE ? scratch[threadIdx.x] : lowest;
    r = wave_max(r);
    if (threadIdx.x == 0) scratch[0] = r;
  }
  __syncthreads();
  T r = scratch[0];
  __syncthreads();
  return r;
}
template <typename T>
__device__ __forceinline__ T block_min(T v, T* scratch, T highest) {
  v = wave_min(v);
  if (lane_id() == 0) scratch[wave_id()] = v;
  __syncthreads();
  if (threadIdx.x < 64) {
    T r = threadIdx.x < NWAVE ? scratch[threadIdx.x] : highest;
    r = wave_min(r);
    if (threadIdx.x == 0) scratch[0] = r;
  }
  __syncthreads();
  T r = scratch[0];
  __syncthreads();
  return r;
}
__device__ __forceinline__ void block_argmax(double& v, int& i, double* sv, int* si) {
  wave_argmax(v, i);
  if (lane_id() == 0) { sv[wave_id()] = v; si[wave_id()] = i; }
  __syncthreads();
  if (threadIdx.x < 64) {
    double w = threadIdx.x < NWAVE ? sv[threadIdx.x] : -__builtin_inf();
    int j = threadIdx.x < NWAVE ? si[threadIdx.x] : INT_MAX;
    wave_argmax(w, j);
    if (threadIdx.x == 0) { sv[0] = w; si[0] = j; }
  }
  __syncthreads();
  v = sv[0];
  i = si[0];
  __syncthreads();
}

// ------------------------------------------------------------ tie groups
// A prefix cut in (key desc, id asc) order that ends inside a group of equal
// keys keeps j of the group's n members; numpy's argsort (sampler.py:82,103)
// leaves which ones unspecified, and in practice its choice follows its
// algorithm: a row of at most TIE_NET entries is sorted by a compare-exchange
// network, which leaves equal keys mostly in index order, while a longer row
// is partitioned first, which scatters a group's members.  The device
// mirrors that: on rows of at most TIE_NET ids (net) the lowest ids of the
// group survive; on longer rows the survivors are spread evenly over the
// group's ids -- of its first R members (ascending id), spread_kept(R) =
// floor((2 R j + n - 1) / (2 n)) survive.  Either way member r survives iff
// spread_kept(r + 1) > spread_kept(r), and the members of an id range
// [R0, R1) hold spread_kept(R1) - spread_kept(R0) survivors.  (Lowest ids on
// long rows would bias the draw towards low ids at every split group.)
constexpr int TIE_NET = 256;
// (Group sizes are below 2^21, so x = 2 R j + n - 1 < 2^43 is exact in fp64,
// and so is floor(x / 2n) of the correctly rounded quotient: a quotient below
// an integer lies at least 1 / 2n below it, far more than its rounding error
// for x < 2^53.  A 64-bit integer division would expand into a long, register
// hungry sequence at every use.)
__device__ __forceinline__ long long spread_kept(long long R, long long j, long long n, bool net) {
  if (j <= 0 || n <= 0) return 0;
  if (j >= n) return R;
  if (net) return R < j ? R : j;
  const double x = (double)(2 * R * j + n - 1);
  return (long long)floor(x / (double)(2 * n));
}
__device__ __forceinline__ bool spread_keeps(long long r, long long j, long long n, bool net) {
  return spread_kept(r + 1, j, n, net) > spread_kept(r, j, n, net);
}
// The same decision for consecutive members without a division each.  On
// long rows, with x_r = 2 r j + n - 1, member r survives iff (x_r mod 2n) +
// 2j >= 2n, and x_{r+1} mod 2n follows by one addition; on net rows the
// state is the rank itself.  spread_rem gives the state of member r;
// spread_step decides member r from it and advances it to r + 1.
__device__ __forceinline__ int spread_rem(long long r, long long j, long long n, bool net) {
  if (net) return (int)r;
  if (n <= 0) return 0;
  const double x = (double)(2 * r * j + n - 1), d = (double)(2 * n);
  return (int)(x - floor(x / d) * d);
}
__device__ __forceinline__ bool spread_step(int& rem, int j, int n, bool net) {
  if (net) return rem++ < j;
  const bool keep = rem + 2 * j >= 2 * n;
  rem += 2 * j;
  rem -= rem >= 2 * n ? 2 * n : 0;
  return keep;
}

// ------------------------------------------------------------ sort records
// A record orders by key descending, then by idx ascending (a total order:
// tie groups are contiguous and sorted by id, as the tie rule above needs).
struct Rec {
  uint64_t key;
  int32_t idx;
  int32_t aux;
};
__device__ __forceinline__ bool rec_before(const Rec& a, const Rec& b) {
  return a.key > b.key || (a.key == b.key && a.idx < b.idx);
}
__device__ __forceinline__ Rec shfl_xor_rec(const Rec& r, int o) {
  Rec s;
  s.key = __shfl_xor(r.key, o);
  s.idx = __shfl_xor(r.idx, o);
  s.aux = __shfl_xor(r.aux, o);
  return s;
}
// One compare-exchange of element e (held in r) with element e ^ stride
// (held in p) inside a bitonic merge of blocks of `size`.
__device__ __forceinline__ Rec bitonic_pick(const Rec& r, const Rec& p, int e, int stride,
                                            int size) {
  bool lower = (e & stride) == 0;
  bool first_half_desc = (e & size) == 0;
  bool want_first = (lower == first_half_desc);
  bool r_first = rec_before(r, p);
  return (want_first == r_first) ? r : p;
}

// Sort up to 64 * PER records held by one wave in registers into
// rec_before order.  Lane l holds elements l * PER .. l * PER + PER - 1;
// strides below PER swap inside a lane, larger strides use shuffles.
template <int S, int PER>
__device__ __forceinline__ void lane_stage(Rec (&r)[PER], int l, int size) {
  // compare-exchange of in-lane partners j and j ^ S (compile-time indices)
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    if ((j ^ S) > j) {
      const int e = l * PER + j;
      Rec lo = bitonic_pick(r[j], r[j ^ S], e, S, size);
      Rec hi = bitonic_pick(r[j ^ S], r[j], e ^ S, S, size);
      r[j] = lo;
      r[j ^ S] = hi;
    }
  }
}

template <int PER>
__device__ inline void wave_sort(Rec (&r)[PER]) {
  static_assert(PER == 1 || PER == 2 || PER == 4, "PER");
  const int l = lane_id();
  constexpr int NP = 64 * PER;
  for (int size = 2; size <= NP; size <<= 1) {
    for (int stride = size >> 1; stride >= PER; stride >>= 1) {
      const int ls = stride / PER;
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        Rec p = shfl_xor_rec(r[j], ls);
        r[j] = bitonic_pick(r[j], p, l * PER + j, stride, size);
      }
    }
    if constexpr (PER >= 4) {
      if (size >= 4) lane_stage<2, PER>(r, l, size);
    }
    if constexpr (PER >= 2) lane_stage<1, PER>(r, l, size);
  }
}

// Inclusive prefix sum across the 64 lanes of a wave.
__device__ __forceinline__ double wave_incl_scan(double v) {
  for (int o = 1; o < 64; o <<= 1) {
    double w = __shfl_up(v, o);
    if (lane_id() >= o) v += w;
  }
  return v;
}

// Compare-exchange of a thread's own elements j and j ^ JS (elements
// t + j * WG; stride JS * WG), with compile-time register indices.
template <int JS, int R>
__device__ __forceinline__ void own_stage(Rec (&r)[R], const bool (&have)[R], int t, int size) {
#pragma unroll
  for (int j = 0; j < R; ++j) {
    if ((j ^ JS) > j && (j ^ JS) < R && have[j ^ JS]) {
      Rec lo = bitonic_pick(r[j], r[j ^ JS], t + j * WG, JS * WG, size);
      Rec hi = bitonic_pick(r[j ^ JS], r[j], t + (j ^ JS) * WG, JS * WG, size);
      r[j] = lo;
      r[j ^ JS] = hi;
    }
  }
}

// Sort n <= R * WG records held in LDS (k, i, a) into rec_before order.
// Thread t owns elements t + j * WG, j < R.  Strides of WG and more pair a
// thread's own elements, strides from 64 to WG / 2 exchange through LDS,
// smaller strides through cross-lane shuffles.
template <int R = 2>
__device__ __forceinline__ void block_sort(uint64_t* k, int32_t* i, int32_t* a, int n) {
  static_assert(R == 2 || R == 4, "R");
  int np = 2;
  while (np < n) np <<= 1;
  const int t = threadIdx.x;
  for (int e = n + t; e < np; e += WG) { k[e] = 0; i[e] = INT_MAX; a[e] = -1; }
  __syncthreads();
  if (np <= 64) {
    if (t < 64) {
      Rec r;
      bool have = t < np;
      r.key = have ? k[t] : 0;
      r.idx = have ? i[t] : INT_MAX;
      r.aux = have ? a[t] : -1;
      for (int size = 2; size <= np; size <<= 1)
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
          Rec p = shfl_xor_rec(r, stride);
          r = bitonic_pick(r, p, t, stride, size);
        }
      if (have) { k[t] = r.key; i[t] = r.idx; a[t] = r.aux; }
    }
    __syncthreads();
    return;
  }
  // np >= 128 here, so have[j] is uniform across each wave
  Rec r[R];
  bool have[R];
#pragma unroll
  for (int j = 0; j < R; ++j) {
    const int e = t + j * WG;
    have[j] = e < np;
    r[j].key = have[j] ? k[e] : 0;
    r[j].idx = have[j] ? i[e] : INT_MAX;
    r[j].aux = have[j] ? a[e] : -1;
  }
  __syncthreads();
  for (int size = 2; size <= np; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride >= WG) {                       // partner is another of the thread's elements
        if (stride == WG) own_stage<1, R>(r, have, t, size);
        else if constexpr (R >= 4) own_stage<2, R>(r, have, t, size);
      } else if (stride >= 64) {                // partner in another wave: via LDS
#pragma unroll
        for (int j = 0; j < R; ++j)
          if (have[j]) { const int e = t + j * WG; k[e] = r[j].key; i[e] = r[j].idx; a[e] = r[j].aux; }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < R; ++j)
          if (have[j]) {
            const int q = (t + j * WG) ^ stride;
            Rec p; p.key = k[q]; p.idx = i[q]; p.aux = a[q];
            r[j] = bitonic_pick(r[j], p, t + j * WG, stride, size);
          }
        __syncthreads();
      } else {                                  // same wave: shuffles
#pragma unroll
        for (int j = 0; j < R; ++j)
          if (have[j]) {
            Rec p = shfl_xor_rec(r[j], stride);
            r[j] = bitonic_pick(r[j], p, t + j * WG, stride, size);
          }
      }
    }
  }
#pragma unroll
  for (int j = 0; j < R; ++j)
    if (have[j]) { const int e = t + j * WG; k[e] = r[j].key; i[e] = r[j].idx; a[e] = r[j].aux; }
  __syncthreads();
}

// Inclusive prefix sum of v[0..n), n <= R * WG, in place (fp64).  Thread t
// owns elements R t .. R t + R - 1.
template <int R = 2>
__device__ __forceinline__ void block_scan(double* v, int n, double* scratch) {
  static_assert(R == 2 || R == 4, "R");
  const int t = threadIdx.x;
  double x[R];
  double s = 0.0;
#pragma unroll
  for (int j = 0; j < R; ++j) {
    x[j] = R * t + j < n ? v[R * t + j] : 0.0;
    s += x[j];
  }
  double inc = s;                                // inclusive scan across the wave
  for (int o = 1; o < 64; o <<= 1) {
    double w = __shfl_up(inc, o);
    if (lane_id() >= o) inc += w;
  }
  if (lane_id() == 63) scratch[wave_id()] = inc;
  __syncthreads();
  if (t < 64) {
    double w = t < NWAVE ? scratch[t] : 0.0;
    double y = w;
    for (int o = 1; o < 64; o <<= 1) {
      double z = __shfl_up(y, o);
      if (t >= o) y += z;
    }
    if (t < NWAVE) scratch[NWAVE + t] = y - w;   // exclusive wave offsets
  }
  __syncthreads();
  double run = scratch[NWAVE + wave_id()] + (inc - s);
#pragma unroll
  for (int j = 0; j < R; ++j) {
    run += x[j];
    if (R * t + j < n) v[R * t + j] = run;
  }
  __syncthreads();
}


// ------------------------------------------------------------ fp64 exp
// 2^(j/64), j = 0..63, each correctly rounded to fp64.
static __device__ const double EXP64_TAB[64] = {
    1.0, 1.0108892860517005, 1.0218971486541166, 1.0330248790212284,
    1.0442737824274138, 1.0556451783605572, 1.0671404006768237, 1.0787607977571199,
    1.0905077326652577, 1.102382583307841, 1.1143867425958924, 1.1265216186082418,
    1.1387886347566916, 1.1511892299529827, 1.1637248587775775, 1.1763969916502812,
    1.189207115002721, 1.202156731452703, 1.215247359980469, 1.22848053610687,
    1.241857812073484, 1.255380757024691, 1.2690509571917332, 1.2828700160787783,
    1.2968395546510096, 1.3109612115247644, 1.3252366431597413, 1.339667524053303,
    1.3542555469368927, 1.3690024229745905, 1.383909881963832, 1.3989796725383112,
    1.4142135623730951, 1.42961333839197, 1.4451808069770467, 1.460917794180647,
    1.4768261459394993, 1.4929077282912648, 1.5091644275934228, 1.5255981507445384,
    1.5422108254079407, 1.559004400237837, 1.5759808451078865, 1.593142151342267,
    1.6104903319492543, 1.6280274218573478, 1.645755478153965, 1.6636765803267364,
    1.681792830507429, 1.7001063537185235, 1.718619298122478, 1.7373338352737062,
    1.7562521603732995, 1.7753764925265212, 1.7947090750031072, 1.8142521755003989,
    1.8340080864093424, 1.8539791250833855, 1.8741676341103, 1.8945759815869656,
    1.9152065613971474, 1.9360617934922943, 1.9571441241754002, 1.978456026387951,
};

// Copy EXP64_TAB into an LDS array of 64 doubles (all threads; ends with a
// barrier).
__device__ __forceinline__ void load_exp64_tab(double* lds_tab) {
  if (threadIdx.x < 64) lds_tab[threadIdx.x] = EXP64_TAB[threadIdx.x];
  __syncthreads();
}

// exp(x) in fp64 within 1 ulp, by Tang's table-driven method (P. T. P. Tang,
// ACM TOMS 15(2), 1989): x = (64 m + j) ln2/64 + r with |r| <= ln2/128, so
// exp(x) = 2^m 2^(j/64) exp(r), and exp(r) - 1 is its degree-5 Taylor
// polynomial (truncation below 4e-17).  ln2/64 is split into a 36-bit head,
// so k * head is exact for |k| < 2^17, and a tail.  `tab` is EXP64_TAB in
// LDS.  Branch-free, so several calls interleave: x < -745.2 (and -inf)
// gives 0, NaN gives NaN; meant for x <= 709.
__device__ __forceinline__ double exp64(double x, const double* tab) {
  const double xc = __builtin_fmin(__builtin_fmax(x, -745.2), 709.0);   // NaN -> -745.2
  const double kd = __builtin_rint(xc * 92.33248261689366);     // xc * 64 / ln2
  double r = __builtin_fma(-kd, 0.010830424696223417, xc);      // head of ln2/64
  r = __builtin_fma(-kd, 2.572804622327669e-14, r);             // tail of ln2/64
  const int k = (int)kd;
  const double p = r * __builtin_fma(r, __builtin_fma(r, __builtin_fma(r, __builtin_fma(
                           r, 1.0 / 120.0, 1.0 / 24.0), 1.0 / 6.0), 0.5), 1.0);
  const double t = tab[k & 63];
  const double v = __builtin_ldexp(__builtin_fma(t, p, t), k >> 6);
  return x > -745.2 ? v : (x != x ? x : 0.0);
}

// exp(x) for x <= 0 (or -inf), as exp64 without its upper clamp and final
// selects: x below -745.2 gives at most the smallest subnormal instead of 0,
// which no sum of these terms can see.
__device__ __forceinline__ double exp64_neg(double x, const double* tab) {
  const double xc = __builtin_fmax(x, -745.2);
  const double kd = __builtin_rint(xc * 92.33248261689366);
  double r = __builtin_fma(-kd, 0.010830424696223417, xc);
  r = __builtin_fma(-kd, 2.572804622327669e-14, r);
  const int k = (int)kd;
  const double p = r * __builtin_fma(r, __builtin_fma(r, __builtin_fma(r, __builtin_fma(
                           r, 1.0 / 120.0, 1.0 / 24.0), 1.0 / 6.0), 0.5), 1.0);
  const double t = tab[k & 63];
  return __builtin_ldexp(__builtin_fma(t, p, t), k >> 6);
}

// fl32(x / T) for fp32 x and T, given invT = 1 / (double)T: the fp64 product
// is within 2^-52 of x / T, and a quotient of two fp32 values that is not a
// midpoint of fp32 lies at least 2^-48 (relative) from one, so rounding the
// product to fp32 gives the correctly rounded fp32 quotient.
__device__ __forceinline__ double div32(float x, double invT) {
  return (double)(float)((double)x * invT);
}

}  // namespace cx
