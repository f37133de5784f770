// Host emulation of the HIP device subset the sampler's exact path uses:
// one workgroup at a time, one OS thread per work-item, std::barrier for
// __syncthreads, and per-wave exchanges (two wave barriers each) for
// ballots, shuffles, readlane and the DPP moves.
#pragma once
#include <atomic>
#include <barrier>
#include <climits>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>
#define __device__
#define __host__
#define __global__
#define __forceinline__ inline
#define __noinline__
#define __launch_bounds__(x)
#define __align__(x) alignas(x)
#define __shared__ static
struct EmuDim { unsigned x, y, z; };
extern thread_local EmuDim threadIdx;
extern EmuDim blockIdx;
namespace emu {
struct Wave {
  std::barrier<> bar{64};
  uint64_t slot[64];
  const char* site_file[64];
  int site_line[64];
};
extern Wave* waves;          // [16]
extern std::barrier<>* block_bar;
// Where each work-item last entered a barrier or a wave exchange (for the
// driver's watchdog: a workgroup that stops making progress is reported by
// the places its work-items wait at).
struct Where { const char* file; int line; };
extern thread_local Where* where;
inline void at(const char* f, int l) { if (where) { where->file = f; where->line = l; } }
// Every lane of a wave must reach its exchanges together (the emulation
// runs lanes as threads, so a lane that skips or repeats one would pair its
// slots with another exchange's): with EMU_CHECK_SITES set, each exchange
// checks that all 64 lanes came from the same call site and reports the
// first that did not.
void check_sites(int wave_index);
inline int lane() { return threadIdx.x & 63; }
inline Wave& wave() { return waves[threadIdx.x >> 6]; }
// every live lane posts v; f reads the slots; all lanes leave together
template <class F>
inline uint64_t xchg(uint64_t v, F f, const char* file = __builtin_FILE(),
                     int line = __builtin_LINE()) {
  at(file, line);
  Wave& w = wave();
  w.slot[lane()] = v;
  w.site_file[lane()] = file;
  w.site_line[lane()] = line;
  w.bar.arrive_and_wait();
  check_sites((int)(&w - waves));
  uint64_t r = f(w.slot);
  w.bar.arrive_and_wait();
  return r;
}
template <class T> inline uint64_t bits(T v) { uint64_t b = 0; std::memcpy(&b, &v, sizeof(T)); return b; }
template <class T> inline T from(uint64_t b) { T v; std::memcpy(&v, &b, sizeof(T)); return v; }
}  // namespace emu
inline void __syncthreads(const char* file = __builtin_FILE(), int line = __builtin_LINE()) {
  emu::at(file, line);
  emu::block_bar->arrive_and_wait();
}
inline void __threadfence() { std::atomic_thread_fence(std::memory_order_seq_cst); }
inline void __threadfence_block() { std::atomic_thread_fence(std::memory_order_seq_cst); }
inline uint64_t __ballot(int p, const char* file = __builtin_FILE(), int line = __builtin_LINE()) {
  emu::at(file, line);
  const bool me = p != 0;
  emu::Wave& w = emu::wave();
  w.slot[emu::lane()] = me;
  w.site_file[emu::lane()] = file;
  w.site_line[emu::lane()] = line;
  w.bar.arrive_and_wait();
  emu::check_sites((int)(&w - emu::waves));
  uint64_t m = 0;
  for (int l = 0; l < 64; ++l) if (w.slot[l] == 1) m |= 1ull << l;
  w.bar.arrive_and_wait();
  return m;
}
#define EMU_SITE const char* file = __builtin_FILE(), int line = __builtin_LINE()
template <class T> inline T __shfl_xor(T v, int o, int width = 64, EMU_SITE) {
  const int l = emu::lane();
  return emu::from<T>(emu::xchg(emu::bits(v), [&](uint64_t* s) { return s[l ^ o]; }, file, line));
}
template <class T> inline T __shfl_up(T v, unsigned o, int width = 64, EMU_SITE) {
  const int l = emu::lane();
  return emu::from<T>(emu::xchg(emu::bits(v), [&](uint64_t* s) { return (int)l - (int)o >= 0 ? s[l - o] : s[l]; }, file, line));
}
template <class T> inline T __shfl(T v, int src, int width = 64, EMU_SITE) {
  return emu::from<T>(emu::xchg(emu::bits(v), [&](uint64_t* s) { return s[src & 63]; }, file, line));
}
inline int __builtin_amdgcn_readlane(int v, int l, EMU_SITE) {
  return (int)emu::xchg((uint32_t)v, [&](uint64_t* s) { return s[l & 63]; }, file, line);
}
inline int __builtin_amdgcn_readfirstlane(int v, EMU_SITE) {
  return __builtin_amdgcn_readlane(v, 0, file, line);
}
inline uint32_t __builtin_amdgcn_mbcnt_lo(uint32_t m, uint32_t acc) {
  const int l = emu::lane();
  return acc + __builtin_popcount(l >= 32 ? m : (m & ((1u << l) - 1u)));
}
inline uint32_t __builtin_amdgcn_mbcnt_hi(uint32_t m, uint32_t acc) {
  const int l = emu::lane();
  return acc + (l < 32 ? 0 : __builtin_popcount(m & ((1u << (l - 32)) - 1u)));
}
// DPP: row_ror:N (0x121..0x12F), row_shr:N (0x111..0x11F), row_bcast:15 (0x142), row_bcast:31 (0x143)
inline int emu_dpp(int old, int src, int ctrl, int row_mask, bool bound_ctrl, const char* file,
                   int line) {
  const int l = emu::lane();
  const int row = l >> 4, rl = l & 15;
  return (int)emu::xchg((uint32_t)src, [&](uint64_t* s) -> uint64_t {
    if (!((row_mask >> row) & 1)) return (uint32_t)old;
    if (ctrl >= 0x121 && ctrl <= 0x12F) { int n = ctrl - 0x120; return (uint32_t)s[(row << 4) + ((rl - n) & 15)]; }
    if (ctrl >= 0x111 && ctrl <= 0x11F) { int n = ctrl - 0x110; return rl - n >= 0 ? (uint32_t)s[l - n] : (bound_ctrl ? 0u : (uint32_t)old); }
    if (ctrl == 0x142) { return row >= 1 ? (uint32_t)s[(row << 4) - 1] : (bound_ctrl ? 0u : (uint32_t)old); }
    if (ctrl == 0x143) { return row >= 2 ? (uint32_t)s[31] : (bound_ctrl ? 0u : (uint32_t)old); }
    std::fprintf(stderr, "emu: unsupported dpp ctrl %x\n", ctrl); std::abort();
  }, file, line);
}
#define __builtin_amdgcn_mov_dpp(v, ctrl, rm, bm, bc) emu_dpp(0, (v), (ctrl), (rm), (bc), __FILE__, __LINE__)
#define __builtin_amdgcn_update_dpp(old, v, ctrl, rm, bm, bc) emu_dpp((old), (v), (ctrl), (rm), (bc), __FILE__, __LINE__)
#define __builtin_amdgcn_fence(...) (emu::at(__FILE__, __LINE__), emu::wave().bar.arrive_and_wait())
#define __builtin_amdgcn_wave_barrier() (emu::at(__FILE__, __LINE__), emu::wave().bar.arrive_and_wait())
inline int __popcll(uint64_t x) { return __builtin_popcountll(x); }
inline int __popc(uint32_t x) { return __builtin_popcount(x); }
inline int __clz(int x) { return x ? __builtin_clz((unsigned)x) : 32; }
inline float __uint_as_float(uint32_t u) { return emu::from<float>(u); }
inline uint32_t __float_as_uint(float f) { return (uint32_t)emu::bits(f); }
inline float __int_as_float(int u) { return emu::from<float>((uint32_t)u); }
inline int __float_as_int(float f) { return (int)(uint32_t)emu::bits(f); }
inline double __longlong_as_double(long long u) { return emu::from<double>((uint64_t)u); }
inline long long __double_as_longlong(double d) { return (long long)emu::bits(d); }
template <class T> inline T atomicAdd(T* p, T v) { return __atomic_fetch_add(p, v, __ATOMIC_SEQ_CST); }
inline double atomicAdd(double* p, double v) {
  uint64_t* q = (uint64_t*)p;
  uint64_t o = __atomic_load_n(q, __ATOMIC_SEQ_CST);
  for (;;) {
    const uint64_t nb = emu::bits(emu::from<double>(o) + v);
    if (__atomic_compare_exchange_n(q, &o, nb, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST))
      return emu::from<double>(o);
  }
}
template <class T> inline T atomicMin(T* p, T v) {
  T old = __atomic_load_n(p, __ATOMIC_SEQ_CST);
  while (v < old && !__atomic_compare_exchange_n(p, &old, v, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST)) {}
  return old;
}
template <class T> inline T atomicMax(T* p, T v) {
  T old = __atomic_load_n(p, __ATOMIC_SEQ_CST);
  while (v > old && !__atomic_compare_exchange_n(p, &old, v, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST)) {}
  return old;
}
template <class T> inline T atomicOr(T* p, T v) { return __atomic_fetch_or(p, v, __ATOMIC_SEQ_CST); }
template <class T> inline T atomicCAS(T* p, T cmp, T v) {
  __atomic_compare_exchange_n(p, &cmp, v, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST);
  return cmp;
}
// Raw buffer loads: a descriptor is a base and a byte count; dwords past the
// count read as zero and touch no memory.
struct __amdgpu_buffer_rsrc_t { const char* p; int n; };
inline __amdgpu_buffer_rsrc_t __builtin_amdgcn_make_buffer_rsrc(void* p, short, int n, int) {
  return {(const char*)p, n};
}
typedef uint32_t emu_u32x4 __attribute__((vector_size(16)));
inline emu_u32x4 __builtin_amdgcn_raw_buffer_load_b128(__amdgpu_buffer_rsrc_t r, int voff, int soff,
                                                       int) {
  emu_u32x4 v = {0u, 0u, 0u, 0u};
  for (int k = 0; k < 4; ++k) {
    const int o = voff + soff + 4 * k;
    if (o >= 0 && o + 4 <= r.n) { uint32_t w; std::memcpy(&w, r.p + o, 4); v[k] = w; }
  }
  return v;
}
inline uint32_t __builtin_amdgcn_raw_buffer_load_b32(__amdgpu_buffer_rsrc_t r, int voff, int soff,
                                                     int) {
  uint32_t w = 0u;
  const int o = voff + soff;
  if (o >= 0 && o + 4 <= r.n) std::memcpy(&w, r.p + o, 4);
  return w;
}
// Scoped atomics (every scope is the whole process here).  clang has them
// as builtins on every target; g++ gets these.
#ifndef __HIP_MEMORY_SCOPE_WORKGROUP
#define __HIP_MEMORY_SCOPE_SINGLETHREAD 1
#define __HIP_MEMORY_SCOPE_WAVEFRONT 2
#define __HIP_MEMORY_SCOPE_WORKGROUP 3
#define __HIP_MEMORY_SCOPE_AGENT 4
#define __HIP_MEMORY_SCOPE_SYSTEM 5
#endif
#ifndef __clang__
template <class T, class U> inline T emu_rmw(T* p, U v, int op) {
  T o = __atomic_load_n((volatile T*)p, __ATOMIC_SEQ_CST);
  for (;;) {
    T n = op == 0 ? (T)(o + (T)v) : op == 1 ? (o > (T)v ? o : (T)v) : (o < (T)v ? o : (T)v);
    if (__atomic_compare_exchange((T*)p, &o, &n, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST))
      return o;
  }
}
template <class T, class U> inline T __hip_atomic_fetch_add(T* p, U v, int, int) { return emu_rmw(p, v, 0); }
template <class T, class U> inline T __hip_atomic_fetch_max(T* p, U v, int, int) { return emu_rmw(p, v, 1); }
template <class T, class U> inline T __hip_atomic_fetch_min(T* p, U v, int, int) { return emu_rmw(p, v, 2); }
template <class T, class U> inline T __hip_atomic_fetch_or(T* p, U v, int, int) {
  return __atomic_fetch_or(p, (T)v, __ATOMIC_SEQ_CST);
}
template <class T> inline T __hip_atomic_load(T* p, int, int) { return __atomic_load_n(p, __ATOMIC_SEQ_CST); }
template <class T, class U> inline void __hip_atomic_store(T* p, U v, int, int) {
  __atomic_store_n(p, (T)v, __ATOMIC_SEQ_CST);
}
template <class T, class U>
inline bool __hip_atomic_compare_exchange_strong(T* p, T* expected, U desired, int, int, int) {
  T d = (T)desired;
  return __atomic_compare_exchange(p, expected, &d, false, __ATOMIC_SEQ_CST, __ATOMIC_SEQ_CST);
}
#endif
inline float __builtin_amdgcn_exp2f(float x) { return std::exp2(x); }
namespace emu {
// the dynamic LDS of the workgroup being run: an exact-size allocation of
// the bytes its launch requests
extern unsigned char* dyn_lds;
}  // namespace emu
typedef void* hipStream_t;
#include <algorithm>
using std::min;
using std::max;
