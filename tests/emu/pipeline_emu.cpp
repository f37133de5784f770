#include <mutex>
// Runs what a cx_sample_f32 call runs on the GPU, on the host: the fused
// kernel (sample_kernel, one workgroup per row slice), then slow_kernel (the
// region finisher, the refinement, the deep-nucleus and exact multi-pass
// paths), one workgroup at a time, one OS thread per work-item.  The
// dynamic LDS of each workgroup is an exact-size allocation of the bytes its
// launch requests (the fused layout; max(multi-pass layout, FIN_CAP * 32)
// for slow_kernel), every static LDS array is its own object, and the
// workspace's counters, slice records and regions are separate exact-size
// allocations, so under AddressSanitizer an access past any of them fails
// the run.  The hand-off between the kernels (row status, hand-off marks,
// slice records, regions) is the fused kernel's own output.
// usage: pipeline_emu IN OUT   (written and read by tests/test_emu_pipeline.py)
// The layouts restated below follow cx_api.hip (slow_layout, fused_layout,
// plan_nsplit).
#include <string>
#include "cx_device.hpp"
#include "cx_internal.hpp"
thread_local EmuDim threadIdx;
EmuDim blockIdx;
emu::Wave* emu::waves;
std::barrier<>* emu::block_bar;
thread_local emu::Where* emu::where;

extern "C" void __sanitizer_print_stack_trace();
void emu::check_sites(int wi) {
  static const bool on = getenv("EMU_CHECK_SITES") != nullptr;
  if (!on) return;
  Wave& w = waves[wi];
  int bad = -1;
  for (int l = 1; l < 64 && bad < 0; ++l)
    if (w.site_line[l] != w.site_line[0] || strcmp(w.site_file[l], w.site_file[0]) != 0) bad = l;
  if (bad < 0) return;
  static std::mutex mu;
  std::lock_guard<std::mutex> g(mu);
  const int me = emu::lane();
  if (me != 0 && me != bad) return;
  fprintf(stderr, "wave %d: lanes at different exchanges; lane %d at %s:%d, called from:\n", wi,
          me, w.site_file[me], w.site_line[me]);
  __sanitizer_print_stack_trace();
  if (me == bad) _exit(4);
}
unsigned char* emu::dyn_lds;
using namespace cx;

namespace cx {
template <bool BF16, bool EXACT> void sample_kernel(SampleArgs A);
void slow_kernel(SampleArgs A);
}  // namespace cx

// The launch geometry and LDS layouts of cx_api.hip (slow_layout,
// fused_layout, plan_nsplit), restated for the host.
static int split_len_of(int V, int nsplit) {
  const int per = (V + nsplit - 1) / nsplit;
  return (per + 7) / 8 * 8;
}
static int pow2_at_least(long x) { int p = 1; while (p < x) p <<= 1; return p; }
static int ilog2(int x) { int l = 0; while ((1 << l) < x) ++l; return l; }
static void slow_layout(SampleArgs& A, int32_t V, int64_t ldh) {
  const long win = ldh > 0 ? (ldh < WIN_MAX ? ldh : WIN_MAX) : 0;
  if (ldh > 0) { A.ns = pow2_at_least(2 * win > 64 ? 2 * win : 64); A.ns_log2 = ilog2(A.ns); }
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
constexpr int FUSED_LDS_MAX = 150 * 1024;
static int plan_nsplit(int B, int V, int64_t ldh) {
  // EMU_NSPLIT: force the slice count (long single-slice rows without the
  // batch of 256 rows that gives them)
  if (getenv("EMU_NSPLIT")) return atoi(getenv("EMU_NSPLIT"));
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

template <class T> static T* rd(FILE* f, size_t n) {
  T* p = (T*)malloc(n * sizeof(T) > 0 ? n * sizeof(T) : 1);
  if (n && fread(p, sizeof(T), n, f) != n) { fprintf(stderr, "short read\n"); exit(2); }
  return p;
}

// One workgroup of `kernel` with `lds` bytes of dynamic LDS (garbage-filled,
// as a launch leaves it).
template <class K>
static void run_workgroup(K kernel, const SampleArgs& A, unsigned block, size_t lds) {
  static const bool trace = getenv("EMU_TRACE") != nullptr;
  if (trace) fprintf(stderr, "workgroup %u (lds %zu)\n", block, lds);
  unsigned char* dyn = (unsigned char*)malloc(lds > 0 ? lds : 1);
  for (size_t i = 0; i < lds; ++i) dyn[i] = (unsigned char)(i * 131 + 7 + block);
  emu::dyn_lds = dyn;
  emu::Wave waves[16];
  emu::waves = waves;
  std::barrier<> bb(1024);
  emu::block_bar = &bb;
  blockIdx.x = block;
  std::vector<emu::Where> where(1024, emu::Where{"(start)", 0});
  std::atomic<int> left{1024};
  // watchdog: a workgroup still running after WATCHDOG_S seconds is reported
  // by where its work-items wait, and the run ends
  static const int WATCHDOG_S = getenv("EMU_WATCHDOG") ? atoi(getenv("EMU_WATCHDOG")) : 60;
  std::thread dog([&] {
    for (int s = 0; s < 10 * WATCHDOG_S && left.load() > 0; ++s)
      std::this_thread::sleep_for(std::chrono::milliseconds(100));
    if (left.load() == 0) return;
    fprintf(stderr, "workgroup %u stuck; work-items by their last barrier:\n", block);
    std::vector<std::pair<std::string, int>> seen;
    for (int t = 0; t < 1024; ++t) {
      char buf[256];
      snprintf(buf, sizeof buf, "%s:%d (wave %d)", where[t].file, where[t].line, t >> 6);
      bool found = false;
      for (auto& p : seen) if (p.first == buf) { ++p.second; found = true; }
      if (!found) seen.push_back({buf, 1});
    }
    for (auto& p : seen) fprintf(stderr, "  %4d  %s\n", p.second, p.first.c_str());
    _exit(3);
  });
  std::vector<std::thread> th;
  th.reserve(1024);
  for (int t = 0; t < 1024; ++t)
    th.emplace_back([&, t] {
      threadIdx.x = t;
      emu::where = &where[t];
      kernel(A);
      emu::at("(returned)", 0);
      left.fetch_sub(1);
      waves[t >> 6].bar.arrive_and_drop();
      bb.arrive_and_drop();
    });
  for (auto& h : th) h.join();
  dog.join();
  free(dyn);
}

int main(int argc, char** argv) {
  FILE* in = fopen(argv[1], "rb");
  FILE* out = fopen(argv[2], "wb");
  int32_t ngroups;
  if (fread(&ngroups, 4, 1, in) != 1) return 2;
  for (int g = 0; g < ngroups; ++g) {
    int32_t hdr[3];
    if (fread(hdr, 4, 3, in) != 3) return 2;
    const int B = hdr[0], V = hdr[1], H = hdr[2];
    float* x = rd<float>(in, (size_t)B * V);
    cx_row_params* prm = rd<cx_row_params>(in, B);
    int32_t* hist = H > 0 ? rd<int32_t>(in, (size_t)B * H) : nullptr;
    int32_t* hl = H > 0 ? rd<int32_t>(in, B) : nullptr;
    double* u = rd<double>(in, B);
    int32_t* ids = (int32_t*)malloc(4 * B);
    int32_t* st = (int32_t*)malloc(4 * B);
    const int nsplit = plan_nsplit(B, V, H);
    // the workspace, each part its own exact-size allocation
    int32_t* counters = (int32_t*)malloc(4 * (size_t)(B + 1));
    SplitStats* stats = (SplitStats*)malloc(sizeof(SplitStats) * (size_t)B * nsplit);
    Cand* cands = (Cand*)malloc(sizeof(Cand) * (size_t)B * nsplit * CAPS);
    memset(counters, 0x5a, 4 * (size_t)(B + 1));
    memset(stats, 0x5a, sizeof(SplitStats) * (size_t)B * nsplit);
    SampleArgs A;
    memset(&A, 0, sizeof A);
    A.logits = x; A.ld = V; A.B = B; A.V = V;
    A.hist = hist; A.hist_len = hl; A.ldh = H;
    A.prm = prm; A.u = u; A.out_id = ids; A.row_status = st; A.out_probs = nullptr;
    A.counters = counters; A.stats = stats; A.cands = cands;
    A.nsplit = nsplit;
    A.split_len = split_len_of(V, nsplit);
    A.logV = log((double)V);
    A.vec_ok = (((uintptr_t)x) % 16 == 0) && (((size_t)V * 4) % 16 == 0);
    slow_layout(A, V, H);
    fused_layout(A, H);
    for (unsigned blk = 0; blk < (unsigned)(B * nsplit); ++blk) {
      if (nsplit > 1) run_workgroup(sample_kernel<false, true>, A, blk, A.lds_bytes);
      else run_workgroup(sample_kernel<false, false>, A, blk, A.lds_bytes);
    }
    const size_t slow_lds = (size_t)std::max(A.slow_lds_bytes, FIN_CAP * 32);
    for (unsigned row = 0; row < (unsigned)B; ++row) run_workgroup(slow_kernel, A, row, slow_lds);
    fwrite(ids, 4, B, out);
    fwrite(st, 4, B, out);
    free(x); free(prm); free(hist); free(hl); free(u); free(ids); free(st);
    free(counters); free(stats); free(cands);
    fprintf(stderr, "group V=%d B=%d H=%d nsplit=%d done\n", V, B, H, nsplit);
  }
  fclose(out);
  return 0;
}
