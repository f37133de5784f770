#include <mutex>
// Runs the exact multi-pass row path (slow_row, as slow_kernel runs it for
// fp64 logits: every row) on the host, one workgroup at a time, with every
// buffer an exact-size heap allocation under AddressSanitizer.
// usage: exact_path_emu IN OUT (written and read by tests/test_emu_exact_path.py)
#include "cx_slow.hpp"
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
using namespace cx;

static int pow2_at_least(long x) { int p = 1; while (p < x) p <<= 1; return p; }
static int ilog2(int x) { int l = 0; while ((1 << l) < x) ++l; return l; }
static void slow_layout(SampleArgs& A, int32_t V, int64_t ldh) {   // as cx_api.hip
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

template <class T> static T* rd(FILE* f, size_t n) {
  T* p = (T*)malloc(n * sizeof(T) > 0 ? n * sizeof(T) : 1);
  if (n && fread(p, sizeof(T), n, f) != n) { fprintf(stderr, "short read\n"); exit(2); }
  return p;
}

int main(int argc, char** argv) {
  FILE* in = fopen(argv[1], "rb");
  FILE* out = fopen(argv[2], "wb");
  int32_t ngroups;
  fread(&ngroups, 4, 1, in);
  for (int g = 0; g < ngroups; ++g) {
    int32_t hdr[3];
    fread(hdr, 4, 3, in);
    const int B = hdr[0], V = hdr[1], H = hdr[2];
    float* x = rd<float>(in, (size_t)B * V);
    cx_row_params* prm = rd<cx_row_params>(in, B);
    int32_t* hist = rd<int32_t>(in, (size_t)B * H);
    int32_t* hl = rd<int32_t>(in, B);
    double* u = rd<double>(in, B);
    int32_t* ids = (int32_t*)malloc(4 * B);
    int32_t* st = (int32_t*)malloc(4 * B);
    float* probs = (float*)malloc(sizeof(float) * B * V);
    SampleArgs A;
    memset(&A, 0, sizeof A);
    A.logits = x; A.ld = V; A.B = B; A.V = V; A.hist = hist; A.hist_len = hl; A.ldh = H;
    A.prm = prm; A.u = u; A.out_id = ids; A.row_status = st; A.out_probs = probs;
    A.nsplit = 1; A.all_slow = 1; A.logV = log((double)V);
    slow_layout(A, V, H);
    const size_t lds = A.slow_lds_bytes > FIN_CAP * 32 ? A.slow_lds_bytes : FIN_CAP * 32;
    for (int row = 0; row < B; ++row) {
      unsigned char* dyn = (unsigned char*)malloc(lds);
      for (size_t i = 0; i < lds; ++i) dyn[i] = (unsigned char)(i * 131 + 7);
      emu::Wave waves[16];
      emu::waves = waves;
      std::barrier<> bb(1024);
      emu::block_bar = &bb;
      blockIdx.x = row;
      std::vector<std::thread> th;
      th.reserve(1024);
      for (int t = 0; t < 1024; ++t)
        th.emplace_back([&, t] {
          threadIdx.x = t;
          __shared__ double red_d[2 * NWAVE + 4];
          __shared__ int red_i[2 * NWAVE + 4];
          slow_row(A, row, dyn, red_d, red_i);
          waves[t >> 6].bar.arrive_and_drop();
          bb.arrive_and_drop();
        });
      for (auto& h : th) h.join();
      free(dyn);
    }
    fwrite(ids, 4, B, out);
    fwrite(st, 4, B, out);
    fwrite(probs, 4, (size_t)B * V, out);
    free(x); free(prm); free(hist); free(hl); free(u); free(ids); free(st); free(probs);
    fprintf(stderr, "group V=%d B=%d done\n", V, B);
  }
  fclose(out);
  return 0;
}
