// cx_api.hip -- the C-ABI of include/cx_sampler.h: argument checks, launch
// geometry, workspace layout and the host-memory convenience variants.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <mutex>
#include <string>

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

// Device buffer that frees itself.
struct DevBuf {
  void* p = nullptr;
  ~DevBuf() {
    if (p) (void)hipFree(p);
  }
  hipError_t alloc(size_t n) { return hipMalloc(&p, n > 0 ? n : 1); }
};

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
  const size_t esz = dtype == 2 ? 8 : (dtype == 1 ? 2 : 4);
  DevBuf dl, dh, dhl, dp, du, did, dst, dpr, dws;
  hipError_t e;
  const size_t ws = cx_sample_workspace_bytes(B, V, ldh);
  if ((e = dl.alloc((size_t)B * ld * esz)) || (e = dp.alloc(sizeof(cx_row_params) * B)) ||
      (e = du.alloc(8 * (size_t)B)) || (e = did.alloc(4 * (size_t)B)) ||
      (e = dst.alloc(4 * (size_t)B)) || (e = dws.alloc(ws)))
    return hip_fail(e, "hipMalloc");
  if (ldh > 0 && ((e = dh.alloc((size_t)B * ldh * 4)) || (e = dhl.alloc(4 * (size_t)B))))
    return hip_fail(e, "hipMalloc");
  if (out_probs && (e = dpr.alloc((size_t)B * V * 4))) return hip_fail(e, "hipMalloc");
  if ((e = hipMemcpy(dl.p, logits, (size_t)B * ld * esz, hipMemcpyHostToDevice)) ||
      (e = hipMemcpy(dp.p, prm, sizeof(cx_row_params) * B, hipMemcpyHostToDevice)) ||
      (e = hipMemcpy(du.p, u, 8 * (size_t)B, hipMemcpyHostToDevice)) ||
      (e = hipMemset(dws.p, 0, ws)))
    return hip_fail(e, "hipMemcpy");
  if (ldh > 0 && ((e = hipMemcpy(dh.p, hist, (size_t)B * ldh * 4, hipMemcpyHostToDevice)) ||
                  (e = hipMemcpy(dhl.p, hist_len, 4 * (size_t)B, hipMemcpyHostToDevice))))
    return hip_fail(e, "hipMemcpy");
  int rc = sample_impl(dl.p, dtype, ld, B, V, (const int32_t*)dh.p, (const int32_t*)dhl.p, ldh,
                       (const cx_row_params*)dp.p, (const double*)du.p, (int32_t*)did.p,
                       (int32_t*)dst.p, out_probs ? (float*)dpr.p : nullptr, dws.p, ws, nullptr);
  if (rc != CX_OK) return rc;
  if ((e = hipDeviceSynchronize())) return hip_fail(e, "sample kernel");
  if ((e = hipMemcpy(out_id, did.p, 4 * (size_t)B, hipMemcpyDeviceToHost)) ||
      (e = hipMemcpy(row_status, dst.p, 4 * (size_t)B, hipMemcpyDeviceToHost)))
    return hip_fail(e, "hipMemcpy");
  if (out_probs &&
      (e = hipMemcpy(out_probs, dpr.p, (size_t)B * V * 4, hipMemcpyDeviceToHost)))
    return hip_fail(e, "hipMemcpy");
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
  DevBuf dx, dh, dhl, dp, dout, dst;
  hipError_t e;
  if ((e = dx.alloc((size_t)B * ld * esz)) || (e = dp.alloc(sizeof(cx_row_params) * B)) ||
      (e = dout.alloc((size_t)B * V * 8)) || (e = dst.alloc(4 * (size_t)B)))
    return hip_fail(e, "hipMalloc");
  if (ldh > 0 && ((e = dh.alloc((size_t)B * ldh * 4)) || (e = dhl.alloc(4 * (size_t)B))))
    return hip_fail(e, "hipMalloc");
  if ((e = hipMemcpy(dx.p, x, (size_t)B * ld * esz, hipMemcpyHostToDevice)) ||
      (e = hipMemcpy(dp.p, prm, sizeof(cx_row_params) * B, hipMemcpyHostToDevice)))
    return hip_fail(e, "hipMemcpy");
  if (ldh > 0 && ((e = hipMemcpy(dh.p, hist, (size_t)B * ldh * 4, hipMemcpyHostToDevice)) ||
                  (e = hipMemcpy(dhl.p, hist_len, 4 * (size_t)B, hipMemcpyHostToDevice))))
    return hip_fail(e, "hipMemcpy");
  int rc = rowop_impl(trunc, dx.p, dtype, ld, B, V, (const int32_t*)dh.p, (const int32_t*)dhl.p,
                      ldh, (const cx_row_params*)dp.p, (double*)dout.p, V, (int32_t*)dst.p,
                      nullptr);
  if (rc != CX_OK) return rc;
  if ((e = hipDeviceSynchronize())) return hip_fail(e, trunc ? "truncate kernel" : "penalties kernel");
  if ((e = hipMemcpy(out, dout.p, (size_t)B * V * 8, hipMemcpyDeviceToHost)) ||
      (e = hipMemcpy(row_status, dst.p, 4 * (size_t)B, hipMemcpyDeviceToHost)))
    return hip_fail(e, "hipMemcpy");
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
  bool any_stoch = false;
  for (int b = 0; b < B; ++b) any_stoch |= temperature[b] != 0.0f;
  DevBuf dt, dd, di, du, dT, da, dn, dus, dst, dws;
  hipError_t e;
  const size_t nt = (size_t)B * (gamma + 1) * V, nd = (size_t)B * gamma * V;
  const size_t ws = cx_spec_verify_workspace_bytes(B, gamma, V);
  if ((e = dt.alloc(nt * 4)) || (e = di.alloc((size_t)B * gamma * 4)) ||
      (e = du.alloc((size_t)B * (gamma + 1) * 8)) || (e = dT.alloc((size_t)B * 4)) ||
      (e = da.alloc((size_t)B * 4)) || (e = dn.alloc((size_t)B * 4)) ||
      (e = dus.alloc((size_t)B * 4)) || (e = dst.alloc((size_t)B * 4)) || (e = dws.alloc(ws)))
    return hip_fail(e, "hipMalloc");
  if (any_stoch && (e = dd.alloc(nd * 4))) return hip_fail(e, "hipMalloc");
  if ((e = hipMemcpy(dt.p, target, nt * 4, hipMemcpyHostToDevice)) ||
      (e = hipMemcpy(di.p, draft_ids, (size_t)B * gamma * 4, hipMemcpyHostToDevice)) ||
      (e = hipMemcpy(du.p, u, (size_t)B * (gamma + 1) * 8, hipMemcpyHostToDevice)) ||
      (e = hipMemcpy(dT.p, temperature, (size_t)B * 4, hipMemcpyHostToDevice)) ||
      (e = hipMemset(dws.p, 0, ws)))
    return hip_fail(e, "hipMemcpy");
  if (any_stoch && (e = hipMemcpy(dd.p, draft, nd * 4, hipMemcpyHostToDevice)))
    return hip_fail(e, "hipMemcpy");
  int rc = verify_impl((const float*)dt.p, (const float*)dd.p, (const int32_t*)di.p,
                       (const double*)du.p, (const float*)dT.p, B, gamma, V, (int32_t*)da.p,
                       (int32_t*)dn.p, (int32_t*)dus.p, (int32_t*)dst.p, dws.p, ws, nullptr,
                       any_stoch);
  if (rc != CX_OK) return rc;
  if ((e = hipDeviceSynchronize())) return hip_fail(e, "verify kernels");
  if ((e = hipMemcpy(accepted, da.p, (size_t)B * 4, hipMemcpyDeviceToHost)) ||
      (e = hipMemcpy(next_tok, dn.p, (size_t)B * 4, hipMemcpyDeviceToHost)) ||
      (e = hipMemcpy(used, dus.p, (size_t)B * 4, hipMemcpyDeviceToHost)) ||
      (e = hipMemcpy(row_status, dst.p, (size_t)B * 4, hipMemcpyDeviceToHost)))
    return hip_fail(e, "hipMemcpy");
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
