// cx_api.hip -- the C-ABI of include/cx_sampler.h: argument checks, launch
// geometry, workspace layout and the host-memory convenience variants.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <algorithm>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "cx_sampler.h"
#include "cx_device.hpp"
#include "cx_internal.hpp"
#include "cx_timing.hpp"

namespace cx {
int launch_sample(const SampleArgs& A, hipStream_t s);
int launch_slow(const SampleArgs& A, hipStream_t s);
int launch_penalties(const SampleArgs& A, hipStream_t s);
int launch_truncate(const SampleArgs& A, hipStream_t s);
int launch_verify(const VerifyArgs& A, bool any_stochastic, hipStream_t s);

static thread_local std::string g_err;

Timing& timing() {
  static Timing t;
  return t;
}

static int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int api_fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

static int hip_fail(hipError_t e, const char* what) {
  return fail(CX_EHIP, "%s: %s", what, hipGetErrorString(e));
}

static int pow2_at_least(long x) {
  int p = 1;
  while (p < x) p <<= 1;
  return p;
}
static int ilog2(int x) {
  int l = 0;
  while ((1 << l) < x) ++l;
  return l;
}

// Penalty hash size and the dynamic LDS layout of the exact multi-pass row
// path: full-row bitmap, hash keys, histogram / gather work area and
// per-thread sums.
static void slow_layout(SampleArgs& A, int32_t V, int64_t ldh) {
  const long win = ldh > 0 ? (ldh < WIN_MAX ? ldh : WIN_MAX) : 0;   // window capacity
  if (ldh > 0) {
    A.ns = pow2_at_least(2 * win > 64 ? 2 * win : 64);
    A.ns_log2 = ilog2(A.ns);
  }
  long bits = ldh > 0 ? pow2_at_least(V) : 32;
  if (bits > (1 << 18)) bits = 1 << 18;
  A.slow_nbw = (int)(bits / 32 > 1 ? bits / 32 : 1);
  size_t so = align_up((size_t)A.slow_nbw * 4, 16);
  A.slow_off_hkey = (int)so;
  so = align_up(so + (size_t)A.ns * 4, 16);
  A.slow_off_work = (int)so;
  so = align_up(so + 1024 * 12 + 1024 * 24, 16);
  A.slow_off_tsum = (int)so;
  so += (size_t)WG * 8;
  A.slow_lds_bytes = (int)so;
}

constexpr int FUSED_LDS_MAX = 150 * 1024;   // fused kernel dynamic LDS (static LDS comes on top)

static int split_len_of(int V, int nsplit) {
  const int per = (V + nsplit - 1) / nsplit;
  return (per + 7) / 8 * 8;
}

// Dynamic LDS layout of the fused kernel for A.split_len and A.ns: the
// penalty index (bitmap of the slice's window ids, hash of (id << 12 | count)
// words, the ids' raw logits and the dense list of occupied slots) and the
// per-wave candidate buffers.
static void fused_layout(SampleArgs& A, int64_t ldh) {
  const long nbw = ldh > 0 ? (A.split_len + 31) / 32 : 0;
  const long nslot = ldh > 0 ? A.ns : 0;
  size_t off = 0;
  A.off_bitmap = 0;
  off = align_up((size_t)nbw * 4, 16);
  A.off_hword = (int)off;
  off += (size_t)nslot * 4;
  A.off_hval = (int)off;
  off += (size_t)nslot * 4;
  A.off_dense = (int)off;
  off = align_up(off + (size_t)nslot * 4, 16);
  A.off_wkey = (int)off;
  off += (size_t)16 * CAPW * 4;
  A.off_widx = (int)off;
  off += (size_t)16 * CAPW * 4;
  A.off_gather = (int)off;
  off += (size_t)LEAN_CAP * 12;
  A.lds_bytes = (int)off;
}

// Slices per row: choose_nsplit's, raised while the fused kernel's LDS
// layout does not fit (its penalty bitmap covers one slice, so a long
// vocabulary with a long history window needs shorter slices).  At
// SLICE_CAP slices every layout fits for V < 2^20.
static int plan_nsplit(int B, int V, int64_t ldh) {
  SampleArgs A;
  memset(&A, 0, sizeof A);
  slow_layout(A, V, ldh);
  int n = choose_nsplit(B, V);
  for (;; ++n) {
    A.split_len = split_len_of(V, n);
    fused_layout(A, ldh);
    if (A.lds_bytes <= FUSED_LDS_MAX || n >= SLICE_CAP) return n;
  }
}

// dtype: 0 fp32, 1 bf16, 2 fp64 (every row on the exact multi-pass path).
static int sample_impl(const void* logits, int dtype, int64_t ld, int32_t B, int32_t V,
                       const int32_t* hist, const int32_t* hist_len, int64_t ldh,
                       const cx_row_params* prm, const double* u, int32_t* out_id,
                       int32_t* row_status, float* out_probs, void* ws, size_t ws_bytes,
                       void* stream) {
  g_err.clear();
  if (B < 0 || V < 1 || ld < V || ldh < 0)
    return fail(CX_EINVAL, "bad shape: B=%d V=%d ld=%lld ldh=%lld", B, V, (long long)ld,
                (long long)ldh);
  if (V >= (1 << 20)) return fail(CX_EINVAL, "V=%d exceeds the 2^20 token-id limit", V);
  if (B == 0) return CX_OK;
  if (!logits || !prm || !u || !out_id || !row_status || !ws)
    return fail(CX_EINVAL, "null pointer argument");
  if (ldh > 0 && (!hist || !hist_len)) return fail(CX_EINVAL, "history pointers are null");
  const int nsplit = plan_nsplit(B, V, ldh);
  const SampleWorkspace L = sample_workspace_layout(B, nsplit);
  if (ws_bytes < L.total)
    return fail(CX_ENOSPACE, "workspace needs %zu bytes, got %zu", L.total, ws_bytes);

  SampleArgs A;
  memset(&A, 0, sizeof A);
  A.logits = logits;
  A.ld = ld;
  A.B = B;
  A.V = V;
  A.hist = hist;
  A.hist_len = hist_len;
  A.ldh = ldh;
  A.prm = prm;
  A.u = u;
  A.out_id = out_id;
  A.row_status = row_status;
  A.out_probs = out_probs;
  char* w = (char*)ws;
  A.counters = (int32_t*)(w + L.off_counters);
  A.stats = (SplitStats*)(w + L.off_stats);
  A.cands = (Cand*)(w + L.off_cands);
  A.nsplit = nsplit;
  A.split_len = split_len_of(V, nsplit);
  A.bf16 = dtype == 1;
  A.f64 = dtype == 2;
  A.all_slow = dtype == 2;
  A.logV = log((double)V);
  const int esz = dtype == 2 ? 8 : (dtype == 1 ? 2 : 4);
  A.vec_ok = (((uintptr_t)logits) % 16 == 0) && ((ld * esz) % 16 == 0);
  slow_layout(A, V, ldh);
  fused_layout(A, ldh);
  if (A.lds_bytes > FUSED_LDS_MAX)
    return fail(CX_EINVAL, "LDS layout too large (%d)", A.lds_bytes);
  hipStream_t s = (hipStream_t)stream;
  int e = 0;
  if (!A.all_slow) {
    e = launch_sample(A, s);
    if (e != 0) return hip_fail((hipError_t)e, "sample launch");
  }
  e = launch_slow(A, s);
  if (e != 0) return hip_fail((hipError_t)e, "slow-path launch");
  return CX_OK;
}

// Sampler.apply_penalties / Sampler._truncate for a batch of rows.
static int rowop_impl(bool trunc, const void* x, int dtype, int64_t ld, int32_t B, int32_t V,
                      const int32_t* hist, const int32_t* hist_len, int64_t ldh,
                      const cx_row_params* prm, double* out, int64_t ldo, int32_t* row_status,
                      void* stream) {
  g_err.clear();
  if (dtype < 0 || dtype > 2) return fail(CX_EINVAL, "dtype must be 0 (fp32), 1 (bf16) or 2 (fp64)");
  if (B < 0 || V < 1 || ld < V || ldo < V || ldh < 0)
    return fail(CX_EINVAL, "bad shape: B=%d V=%d ld=%lld ldo=%lld ldh=%lld", B, V, (long long)ld,
                (long long)ldo, (long long)ldh);
  if (V >= (1 << 20)) return fail(CX_EINVAL, "V=%d exceeds the 2^20 token-id limit", V);
  if (B == 0) return CX_OK;
  if (!x || !prm || !out || !row_status) return fail(CX_EINVAL, "null pointer argument");
  if (ldh > 0 && (!hist || !hist_len)) return fail(CX_EINVAL, "history pointers are null");
  SampleArgs A;
  memset(&A, 0, sizeof A);
  A.logits = x;
  A.ld = ld;
  A.B = B;
  A.V = V;
  A.hist = hist;
  A.hist_len = hist_len;
  A.ldh = trunc ? 0 : ldh;
  A.prm = prm;
  A.row_status = row_status;
  A.bf16 = dtype == 1;
  A.f64 = dtype == 2;
  A.out64 = out;
  A.ldo = ldo;
  slow_layout(A, V, A.ldh);
  hipStream_t s = (hipStream_t)stream;
  int e = trunc ? launch_truncate(A, s) : launch_penalties(A, s);
  if (e != 0) return hip_fail((hipError_t)e, trunc ? "truncate launch" : "penalties launch");
  return CX_OK;
}

static int verify_impl(const float* target, const float* draft, const int32_t* ids,
                       const double* u, const float* temp, int32_t B, int32_t gamma, int32_t V,
                       int32_t* accepted, int32_t* next_tok, int32_t* used, int32_t* status,
                       void* ws, size_t ws_bytes, void* stream, bool any_stoch) {
  g_err.clear();
  if (B < 0 || gamma < 1 || V < 1) return fail(CX_EINVAL, "bad shape B=%d gamma=%d V=%d", B, gamma, V);
  if (gamma > GAMMA_MAX) return fail(CX_EINVAL, "gamma=%d exceeds %d", gamma, GAMMA_MAX);
  if (V > 2 * WG * SUB) return fail(CX_EINVAL, "V=%d exceeds %d", V, 2 * WG * SUB);
  if (B == 0) return CX_OK;
  if (!target || !ids || !u || !temp || !accepted || !next_tok || !used || !status || !ws)
    return fail(CX_EINVAL, "null pointer argument");
  if (any_stoch && !draft) return fail(CX_EINVAL, "draft logits are required for T > 0");
  const VerifyWorkspace L = verify_workspace_layout(B, gamma, V);
  if (ws_bytes < L.total)
    return fail(CX_ENOSPACE, "workspace needs %zu bytes, got %zu", L.total, ws_bytes);
  VerifyArgs A;
  memset(&A, 0, sizeof A);
  A.target = target;
  A.draft = draft;
  A.draft_ids = ids;
  A.u = u;
  A.temperature = temp;
  A.B = B;
  A.gamma = gamma;
  A.V = V;
  A.nchunk = (V + VCHUNK - 1) / VCHUNK;
  A.nsub = (V + SUB - 1) / SUB;
  A.draft_rows = any_stoch ? 1 : 0;
  A.accepted = accepted;
  A.next_tok = next_tok;
  A.used = used;
  A.row_status = status;
  char* w = (char*)ws;
  A.cstats = (ChunkStats*)(w + L.off_cstats);
  A.seq = (SeqState*)(w + L.off_seq);
  A.npart = (NormPart*)(w + L.off_npart);
  A.amb = (AmbEntry*)(w + L.off_amb);
  int e = launch_verify(A, any_stoch, (hipStream_t)stream);
  if (e != 0) return hip_fail((hipError_t)e, "verify launch");
  return CX_OK;
}

// ------------------------------------------------------------ host-call arenas
// Device memory of the host-memory entry points, reused from call to call so
// that a call allocates only when it needs more than any call before it on
// that arena.  One arena per concurrent caller and device: a call takes an
// idle arena of the current device (or makes one) and returns it when done.
// Arenas are held until the process ends; freeing them from a static
// destructor could run after the HIP runtime has shut down.  Each arena has
// its own stream (default priority), so a host call waits only for its own
// copies and kernels.  The workspace part is zero-filled when it is
// allocated and again after a call that failed while using it (the kernels
// need no initial contents there: each call writes what it reads first).
//
// Small calls (a decode step's rows) stage their inputs and outputs through a
// pinned host mirror of the device part: the inputs are packed there with
// memcpy and cross in one copy, the outputs come back in one copy.  Larger
// calls stage their small inputs the same way and send the logits through a
// ring of pinned chunks (below).
constexpr size_t STAGE_MAX = (size_t)8 << 20;

// Logits too large for the mirror cross through a ring of pinned chunks:
// each of up to RING_THREADS host threads fills its own pair of chunks in
// turn (memcpy from the caller's pageable memory) and queues each chunk's
// copy on the arena's stream, so the host copies run in parallel with each
// other and with the DMA engine.  A copy straight from pageable memory goes
// through the runtime's own bounce buffer one piece at a time, at a fraction
// of the link's rate.
constexpr size_t RING_CHUNK = (size_t)4 << 20;
constexpr int RING_THREADS = 8;

struct Arena {
  int dev = -1;
  hipStream_t stream = nullptr;
  char* io = nullptr;          // device part
  size_t io_cap = 0;
  char* host = nullptr;        // pinned mirror of io[0, host_cap)
  size_t host_cap = 0;
  void* ws = nullptr;
  size_t ws_cap = 0;
  bool ws_dirty = false;
  char* ring = nullptr;        // 2 * RING_THREADS pinned chunks of RING_CHUNK bytes
  hipEvent_t ring_ev[2 * RING_THREADS] = {};   // each chunk's last queued copy
};

static std::mutex g_arena_mu;
static std::vector<Arena*> g_arena_idle;

// An arena in use: carves the device part into 256-byte-aligned pieces in
// the order they are taken, and goes back to the idle list when destroyed.
class ArenaLease {
 public:
  ~ArenaLease() {
    if (!a_) return;
    std::lock_guard<std::mutex> g(g_arena_mu);
    g_arena_idle.push_back(a_);
  }
  // io_bytes: the sum of the pieces, each rounded up to 256 bytes; the first
  // stage_bytes of them get a pinned host mirror
  int acquire(size_t io_bytes, size_t ws_bytes, size_t stage_bytes = 0) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    {
      std::lock_guard<std::mutex> g(g_arena_mu);
      for (size_t i = 0; i < g_arena_idle.size(); ++i)
        if (g_arena_idle[i]->dev == dev) {
          a_ = g_arena_idle[i];
          g_arena_idle.erase(g_arena_idle.begin() + i);
          break;
        }
    }
    if (!a_) {
      a_ = new Arena;
      a_->dev = dev;
      if ((e = hipStreamCreateWithFlags(&a_->stream, hipStreamNonBlocking)) != hipSuccess) {
        delete a_;
        a_ = nullptr;
        return hip_fail(e, "hipStreamCreateWithFlags");
      }
    }
    if (io_bytes > a_->io_cap) {
      if (a_->io) (void)hipFree(a_->io);
      a_->io = nullptr;
      a_->io_cap = 0;
      if ((e = hipMalloc((void**)&a_->io, io_bytes)) != hipSuccess) return hip_fail(e, "hipMalloc");
      a_->io_cap = io_bytes;
    }
    if (stage_bytes > a_->host_cap) {
      if (a_->host) (void)hipHostFree(a_->host);
      a_->host = nullptr;
      a_->host_cap = 0;
      if ((e = hipHostMalloc((void**)&a_->host, stage_bytes, hipHostMallocDefault)) != hipSuccess)
        return hip_fail(e, "hipHostMalloc");
      a_->host_cap = stage_bytes;
    }
    if (ws_bytes > a_->ws_cap) {
      if (a_->ws) (void)hipFree(a_->ws);
      a_->ws = nullptr;
      a_->ws_cap = 0;
      if ((e = hipMalloc(&a_->ws, ws_bytes)) != hipSuccess) return hip_fail(e, "hipMalloc");
      a_->ws_cap = ws_bytes;
      a_->ws_dirty = true;
    }
    if (a_->ws_dirty && a_->ws) {
      if ((e = hipMemsetAsync(a_->ws, 0, a_->ws_cap, a_->stream)) != hipSuccess)
        return hip_fail(e, "hipMemsetAsync");
      a_->ws_dirty = false;
    }
    return CX_OK;
  }
  static size_t piece(size_t n) { return (n + 255) & ~(size_t)255; }
  char* take(size_t n) {
    char* p = a_->io + off_;
    off_ += piece(n);
    return p;
  }
  // the pinned mirror of a device piece
  char* host(const void* dev_piece) const { return a_->host + ((const char*)dev_piece - a_->io); }
  void* ws() {
    a_->ws_dirty = true;              // until finish() says the call completed
    return a_->ws;
  }
  size_t ws_cap() const { return a_->ws_cap; }
  hipStream_t stream() const { return a_->stream; }
  // the call completed: no refill before the next call
  void finish() { a_->ws_dirty = false; }

  // Queue the copy of n bytes of host memory to device memory on the
  // arena's stream: through the pinned ring when n spans several chunks,
  // else directly.  Returns once every chunk's copy is queued (the last ones
  // may still be in flight; the host buffer is no longer read).
  int h2d_in(void* dst, const void* src, size_t n) {
    hipError_t e;
    if (n <= RING_CHUNK) {
      if ((e = hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, a_->stream)))
        return hip_fail(e, "hipMemcpyAsync");
      return CX_OK;
    }
    if (!a_->ring) {
      if ((e = hipHostMalloc((void**)&a_->ring, 2 * RING_THREADS * RING_CHUNK,
                             hipHostMallocDefault)) != hipSuccess) {
        a_->ring = nullptr;
        return hip_fail(e, "hipHostMalloc(ring)");
      }
      for (int i = 0; i < 2 * RING_THREADS; ++i)
        if ((e = hipEventCreateWithFlags(&a_->ring_ev[i], hipEventDisableTiming)) != hipSuccess)
          return hip_fail(e, "hipEventCreateWithFlags");
    }
    const size_t nch = (n + RING_CHUNK - 1) / RING_CHUNK;
    const unsigned hc = std::thread::hardware_concurrency();
    const int T = (int)std::min<size_t>(std::min<size_t>(RING_THREADS, nch), hc ? hc : 1);
    std::vector<hipError_t> err(T, hipSuccess);
    auto fill = [&](int t) {
      hipError_t x = hipSetDevice(a_->dev);
      for (size_t j = t, i = 0; x == hipSuccess && j < nch; j += T, ++i) {
        const int b = 2 * t + (int)(i & 1);
        // the chunk's previous copy (of this call, or of an earlier call
        // that failed before its stream was drained) has completed
        if ((x = hipEventSynchronize(a_->ring_ev[b])) != hipSuccess) break;
        const size_t off = j * RING_CHUNK, len = std::min(RING_CHUNK, n - off);
        char* buf = a_->ring + (size_t)b * RING_CHUNK;
        memcpy(buf, (const char*)src + off, len);
        if ((x = hipMemcpyAsync((char*)dst + off, buf, len, hipMemcpyHostToDevice,
                                a_->stream)) != hipSuccess)
          break;
        x = hipEventRecord(a_->ring_ev[b], a_->stream);
      }
      err[t] = x;
    };
    std::vector<std::thread> th;
    for (int t = 1; t < T; ++t) th.emplace_back(fill, t);
    fill(0);
    for (auto& x : th) x.join();
    for (int t = 0; t < T; ++t)
      if (err[t] != hipSuccess) return hip_fail(err[t], "pinned ring copy");
    return CX_OK;
  }

 private:
  Arena* a_ = nullptr;
  size_t off_ = 0;
};

static hipError_t h2d(void* dst, const void* src, size_t n, hipStream_t s) {
  return hipMemcpyAsync(dst, src, n, hipMemcpyHostToDevice, s);
}
static hipError_t d2h(void* dst, const void* src, size_t n, hipStream_t s) {
  return hipMemcpyAsync(dst, src, n, hipMemcpyDeviceToHost, s);
}

// ------------------------------------------------------------ static scratch
// The workspace of cx_sample_f32_noalloc: a file-scope device array (each
// GPU holds its own copy until the process ends).  Its host-side name is
// not a device address; the address is looked up once per device with
// hipGetSymbolAddress and only that address reaches kernels.
constexpr size_t NOALLOC_SCRATCH_BYTES = CX_NOALLOC_SCRATCH_BYTES;
constexpr int NOALLOC_MAX_DEVICES = 64;
static __device__ __align__(256) unsigned char scratch[NOALLOC_SCRATCH_BYTES];
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[NOALLOC_MAX_DEVICES];

// The current device's scratch address, looked up on the first call on that
// device (with the device current, as hipGetSymbolAddress requires).
static int scratch_of_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES)
    return fail(CX_EINVAL, "device %d beyond the %d the static scratch serves", dev,
                NOALLOC_MAX_DEVICES);
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(CX_EHIP, "hipGetSymbolAddress(scratch) returned a null address");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return CX_OK;
}

}  // namespace cx

using namespace cx;

extern "C" {

int cx_sample_f32(const float* logits, int64_t ld, int32_t B, int32_t V, const int32_t* hist,
                  const int32_t* hist_len, int64_t ldh, const cx_row_params* prm, const double* u,
                  int32_t* out_id, int32_t* row_status, float* out_probs, void* workspace,
                  size_t ws_bytes, void* stream) {
  return sample_impl(logits, 0, ld, B, V, hist, hist_len, ldh, prm, u, out_id, row_status,
                     out_probs, workspace, ws_bytes, stream);
}

int cx_sample_f32_noalloc(const float* logits, int64_t ld, int32_t B, int32_t V,
                          const int32_t* hist, const int32_t* hist_len, int64_t ldh,
                          const cx_row_params* prm, const double* u, int32_t* out_id,
                          int32_t* row_status, float* out_probs, void* stream) {
  g_err.clear();
  if (B < 0 || V < 1 || ldh < 0)
    return fail(CX_EINVAL, "bad shape: B=%d V=%d ldh=%lld", B, V, (long long)ldh);
  if (B == 0) return CX_OK;
  if (V >= (1 << 20)) return fail(CX_EINVAL, "V=%d exceeds the 2^20 token-id limit", V);
  const size_t need = sample_workspace_layout(B, plan_nsplit(B, V, ldh)).total;
  if (need > NOALLOC_SCRATCH_BYTES)
    return fail(CX_EINVAL, "B=%d V=%d ldh=%lld needs %zu bytes of scratch; the static scratch "
                "holds %zu", B, V, (long long)ldh, need, NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (int rc = scratch_of_current_device(&ws)) return rc;
  return sample_impl(logits, 0, ld, B, V, hist, hist_len, ldh, prm, u, out_id, row_status,
                     out_probs, ws, NOALLOC_SCRATCH_BYTES, stream);
}

int cx_sample_bf16(const uint16_t* logits, int64_t ld, int32_t B, int32_t V,
                   const int32_t* hist, const int32_t* hist_len, int64_t ldh,
                   const cx_row_params* prm, const double* u, int32_t* out_id,
                   int32_t* row_status, float* out_probs, void* workspace, size_t ws_bytes,
                   void* stream) {
  return sample_impl(logits, 1, ld, B, V, hist, hist_len, ldh, prm, u, out_id, row_status,
                     out_probs, workspace, ws_bytes, stream);
}

int cx_sample_f64(const double* logits, int64_t ld, int32_t B, int32_t V,
                  const int32_t* hist, const int32_t* hist_len, int64_t ldh,
                  const cx_row_params* prm, const double* u, int32_t* out_id,
                  int32_t* row_status, float* out_probs, void* workspace, size_t ws_bytes,
                  void* stream) {
  return sample_impl(logits, 2, ld, B, V, hist, hist_len, ldh, prm, u, out_id, row_status,
                     out_probs, workspace, ws_bytes, stream);
}

size_t cx_sample_workspace_bytes(int32_t B, int32_t V, int64_t ldh) {
  if (B <= 0 || V <= 0 || ldh < 0) return 256;
  return sample_workspace_layout(B, plan_nsplit(B, V, ldh)).total;
}

int cx_sample_host(const void* logits, int32_t dtype, int64_t ld, int32_t B, int32_t V,
                   const int32_t* hist, const int32_t* hist_len, int64_t ldh,
                   const cx_row_params* prm, const double* u, int32_t* out_id,
                   int32_t* row_status, float* out_probs) {
  g_err.clear();
  if (dtype < 0 || dtype > 2) return fail(CX_EINVAL, "dtype must be 0 (fp32), 1 (bf16) or 2 (fp64)");
  if (B < 0 || V < 1 || ld < V || ldh < 0) return fail(CX_EINVAL, "bad shape");
  if (B == 0) return CX_OK;
  if (!logits || !prm || !u || !out_id || !row_status) return fail(CX_EINVAL, "null pointer argument");
  if (ldh > 0 && (!hist || !hist_len)) return fail(CX_EINVAL, "history pointers are null");
  using AL = ArenaLease;
  const size_t esz = dtype == 2 ? 8 : (dtype == 1 ? 2 : 4);
  const size_t nl = (size_t)B * ld * esz, np = sizeof(cx_row_params) * B, nu = 8 * (size_t)B,
               nb = 4 * (size_t)B, nh = ldh > 0 ? (size_t)B * ldh * 4 : 0,
               nhl = ldh > 0 ? nb : 0, npr = out_probs ? (size_t)B * V * 4 : 0;
  // device pieces: the small inputs (and the logits when they fit the
  // mirror), then ids and status (staged together), then the logits that go
  // through the pinned ring, then probs
  const size_t small_in = AL::piece(np) + AL::piece(nu) + AL::piece(nh) + AL::piece(nhl);
  const bool ring = small_in + AL::piece(nl) + 2 * AL::piece(nb) > STAGE_MAX;
  const size_t in_bytes = small_in + (ring ? 0 : AL::piece(nl));
  const size_t staged = in_bytes + 2 * AL::piece(nb);
  const bool stage = staged <= STAGE_MAX;
  ArenaLease L;
  if (int rc = L.acquire(staged + (ring ? AL::piece(nl) : 0) + AL::piece(npr),
                         cx_sample_workspace_bytes(B, V, ldh), stage ? staged : 0))
    return rc;
  char* dp = L.take(np);
  char* du = L.take(nu);
  char* dh = L.take(nh);
  char* dhl = L.take(nhl);
  char* dl = ring ? nullptr : L.take(nl);
  char* did = L.take(nb);
  char* dst = L.take(nb);
  if (ring) dl = L.take(nl);
  char* dpr = out_probs ? L.take(npr) : nullptr;
  const hipStream_t s = L.stream();
  hipError_t e;
  if (stage) {
    memcpy(L.host(dp), prm, np);
    memcpy(L.host(du), u, nu);
    if (ldh > 0) {
      memcpy(L.host(dh), hist, nh);
      memcpy(L.host(dhl), hist_len, nhl);
    }
    if (!ring) memcpy(L.host(dl), logits, nl);
    if ((e = h2d(dp, L.host(dp), in_bytes, s))) return hip_fail(e, "hipMemcpyAsync");
  } else if ((e = h2d(dp, prm, np, s)) || (e = h2d(du, u, nu, s)) ||
             (ldh > 0 && ((e = h2d(dh, hist, nh, s)) || (e = h2d(dhl, hist_len, nhl, s))))) {
    return hip_fail(e, "hipMemcpyAsync");
  }
  if (ring) {
    if (int rc = L.h2d_in(dl, logits, nl)) return rc;
  }
  int rc = sample_impl(dl, dtype, ld, B, V, ldh > 0 ? (const int32_t*)dh : nullptr,
                       ldh > 0 ? (const int32_t*)dhl : nullptr, ldh, (const cx_row_params*)dp,
                       (const double*)du, (int32_t*)did, (int32_t*)dst, (float*)dpr, L.ws(),
                       L.ws_cap(), s);
  if (rc != CX_OK) return rc;
  if (stage) {
    if ((e = d2h(L.host(did), did, 2 * AL::piece(nb), s))) return hip_fail(e, "hipMemcpyAsync");
  } else if ((e = d2h(out_id, did, nb, s)) || (e = d2h(row_status, dst, nb, s))) {
    return hip_fail(e, "hipMemcpyAsync");
  }
  if (out_probs && (e = d2h(out_probs, dpr, npr, s))) return hip_fail(e, "hipMemcpyAsync");
  if ((e = hipStreamSynchronize(s))) return hip_fail(e, "sample kernels");
  L.finish();
  if (stage) {
    memcpy(out_id, L.host(did), nb);
    memcpy(row_status, L.host(dst), nb);
  }
  return CX_OK;
}

int cx_apply_penalties(const void* logits, int32_t dtype, int64_t ld, int32_t B, int32_t V,
                       const int32_t* hist, const int32_t* hist_len, int64_t ldh,
                       const cx_row_params* prm, double* out, int64_t ldo, int32_t* row_status,
                       void* stream) {
  return rowop_impl(false, logits, dtype, ld, B, V, hist, hist_len, ldh, prm, out, ldo,
                    row_status, stream);
}

int cx_truncate_f64(const double* probs, int64_t ld, int32_t B, int32_t V,
                    const cx_row_params* prm, double* out, int64_t ldo, int32_t* row_status,
                    void* stream) {
  return rowop_impl(true, probs, 2, ld, B, V, nullptr, nullptr, 0, prm, out, ldo, row_status,
                    stream);
}

// Host-memory variant of both row operations.
static int rowop_host(bool trunc, const void* x, int32_t dtype, int64_t ld, int32_t B, int32_t V,
                      const int32_t* hist, const int32_t* hist_len, int64_t ldh,
                      const cx_row_params* prm, double* out, int32_t* row_status) {
  g_err.clear();
  if (dtype < 0 || dtype > 2) return fail(CX_EINVAL, "dtype must be 0 (fp32), 1 (bf16) or 2 (fp64)");
  if (B < 0 || V < 1 || ld < V || ldh < 0) return fail(CX_EINVAL, "bad shape");
  if (B == 0) return CX_OK;
  if (!x || !prm || !out || !row_status) return fail(CX_EINVAL, "null pointer argument");
  if (ldh > 0 && (!hist || !hist_len)) return fail(CX_EINVAL, "history pointers are null");
  const size_t esz = dtype == 2 ? 8 : (dtype == 1 ? 2 : 4);
  const size_t nx = (size_t)B * ld * esz, np = sizeof(cx_row_params) * B,
               no = (size_t)B * V * 8, nb = 4 * (size_t)B, nh = ldh > 0 ? (size_t)B * ldh * 4 : 0,
               nhl = ldh > 0 ? nb : 0;
  using AL = ArenaLease;
  ArenaLease L;
  if (int rc = L.acquire(AL::piece(nx) + AL::piece(np) + AL::piece(no) + AL::piece(nb) +
                             AL::piece(nh) + AL::piece(nhl), 0))
    return rc;
  char* dx = L.take(nx);
  char* dp = L.take(np);
  char* dout = L.take(no);
  char* dst = L.take(nb);
  char* dh = ldh > 0 ? L.take(nh) : nullptr;
  char* dhl = ldh > 0 ? L.take(nhl) : nullptr;
  const hipStream_t s = L.stream();
  hipError_t e;
  if ((e = h2d(dp, prm, np, s)) ||
      (ldh > 0 && ((e = h2d(dh, hist, nh, s)) || (e = h2d(dhl, hist_len, nhl, s)))))
    return hip_fail(e, "hipMemcpyAsync");
  if (int rc = L.h2d_in(dx, x, nx)) return rc;
  int rc = rowop_impl(trunc, dx, dtype, ld, B, V, (const int32_t*)dh, (const int32_t*)dhl, ldh,
                      (const cx_row_params*)dp, (double*)dout, V, (int32_t*)dst, s);
  if (rc != CX_OK) return rc;
  if ((e = d2h(out, dout, no, s)) || (e = d2h(row_status, dst, nb, s)))
    return hip_fail(e, "hipMemcpyAsync");
  if ((e = hipStreamSynchronize(s))) return hip_fail(e, trunc ? "truncate kernel" : "penalties kernel");
  L.finish();
  return CX_OK;
}

int cx_apply_penalties_host(const void* logits, int32_t dtype, int64_t ld, int32_t B, int32_t V,
                            const int32_t* hist, const int32_t* hist_len, int64_t ldh,
                            const cx_row_params* prm, double* out, int32_t* row_status) {
  return rowop_host(false, logits, dtype, ld, B, V, hist, hist_len, ldh, prm, out, row_status);
}

int cx_truncate_host(const double* probs, int64_t ld, int32_t B, int32_t V,
                     const cx_row_params* prm, double* out, int32_t* row_status) {
  return rowop_host(true, probs, 2, ld, B, V, nullptr, nullptr, 0, prm, out, row_status);
}

int cx_spec_verify_f32(const float* target, const float* draft, const int32_t* draft_ids,
                       const double* u, const float* temperature, int32_t B, int32_t gamma,
                       int32_t V, int32_t* accepted, int32_t* next_tok, int32_t* used,
                       int32_t* row_status, void* workspace, size_t ws_bytes, void* stream) {
  // The device variant cannot inspect temperatures on the host: it always
  // launches the stochastic stages, which exit at once for greedy rows.
  return verify_impl(target, draft, draft_ids, u, temperature, B, gamma, V, accepted, next_tok,
                     used, row_status, workspace, ws_bytes, stream, draft != nullptr);
}

size_t cx_spec_verify_workspace_bytes(int32_t B, int32_t gamma, int32_t V) {
  if (B <= 0 || gamma <= 0 || V <= 0) return 256;
  return verify_workspace_layout(B, gamma, V).total;
}

int cx_spec_verify_host(const float* target, const float* draft, const int32_t* draft_ids,
                        const double* u, const float* temperature, int32_t B, int32_t gamma,
                        int32_t V, int32_t* accepted, int32_t* next_tok, int32_t* used,
                        int32_t* row_status) {
  g_err.clear();
  if (B < 0 || gamma < 1 || V < 1) return fail(CX_EINVAL, "bad shape");
  if (B == 0) return CX_OK;
  if (!target || !draft_ids || !u || !temperature || !accepted || !next_tok || !used ||
      !row_status)
    return fail(CX_EINVAL, "null pointer argument");
  bool any_stoch = false;
  for (int b = 0; b < B; ++b) any_stoch |= temperature[b] != 0.0f;
  if (any_stoch && !draft) return fail(CX_EINVAL, "draft logits are null with a stochastic row");
  const size_t nt = (size_t)B * (gamma + 1) * V * 4, nd = any_stoch ? (size_t)B * gamma * V * 4 : 0,
               ni = (size_t)B * gamma * 4, nu = (size_t)B * (gamma + 1) * 8, nb = (size_t)B * 4;
  using AL = ArenaLease;
  ArenaLease L;
  if (int rc = L.acquire(AL::piece(nt) + AL::piece(nd) + AL::piece(ni) + AL::piece(nu) +
                             5 * AL::piece(nb),
                         cx_spec_verify_workspace_bytes(B, gamma, V)))
    return rc;
  char* dt = L.take(nt);
  char* dd = any_stoch ? L.take(nd) : nullptr;
  char* di = L.take(ni);
  char* du = L.take(nu);
  char* dT = L.take(nb);
  char* da = L.take(nb);
  char* dn = L.take(nb);
  char* dus = L.take(nb);
  char* dst = L.take(nb);
  const hipStream_t s = L.stream();
  hipError_t e;
  if ((e = h2d(di, draft_ids, ni, s)) || (e = h2d(du, u, nu, s)) ||
      (e = h2d(dT, temperature, nb, s)))
    return hip_fail(e, "hipMemcpyAsync");
  if (int rc = L.h2d_in(dt, target, nt)) return rc;
  if (any_stoch) {
    if (int rc = L.h2d_in(dd, draft, nd)) return rc;
  }
  int rc = verify_impl((const float*)dt, (const float*)dd, (const int32_t*)di,
                       (const double*)du, (const float*)dT, B, gamma, V, (int32_t*)da,
                       (int32_t*)dn, (int32_t*)dus, (int32_t*)dst, L.ws(), L.ws_cap(), s,
                       any_stoch);
  if (rc != CX_OK) return rc;
  if ((e = d2h(accepted, da, nb, s)) || (e = d2h(next_tok, dn, nb, s)) ||
      (e = d2h(used, dus, nb, s)) || (e = d2h(row_status, dst, nb, s)))
    return hip_fail(e, "hipMemcpyAsync");
  if ((e = hipStreamSynchronize(s))) return hip_fail(e, "verify kernels");
  L.finish();
  return CX_OK;
}

int cx_timing_enable(int on) {
  Timing& T = timing();
  std::lock_guard<std::mutex> g(T.mu);
  T.on = on != 0;
  return CX_OK;
}

int cx_timing_read(int32_t kernel, double* total_ms, int64_t* launches) {
  g_err.clear();
  if (kernel < 0 || kernel >= CX_KERNEL_KINDS || !total_ms || !launches)
    return fail(CX_EINVAL, "bad timing query");
  Timing& T = timing();
  std::vector<TimedLaunch> rec;
  {
    std::lock_guard<std::mutex> g(T.mu);
    rec.swap(T.rec[kernel]);
  }
  double sum = 0.0;
  int64_t n = 0;
  int rc = CX_OK;
  for (auto& r : rec) {
    float ms = 0.f;
    hipError_t e = hipEventSynchronize(r.b);
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.a, r.b);
    if (e != hipSuccess) rc = hip_fail(e, "timing events");
    sum += ms;
    ++n;
  }
  {
    std::lock_guard<std::mutex> g(T.mu);
    for (auto& r : rec) { T.pool.push_back(r.a); T.pool.push_back(r.b); }
  }
  *total_ms = sum;
  *launches = n;
  return rc;
}

const char* cx_last_error(void) { return g_err.c_str(); }

const char* cx_version(void) { return "cx_sampler 0.1 gfx950"; }

}  // extern "C"
