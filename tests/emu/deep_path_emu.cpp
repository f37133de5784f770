#include <mutex>
// Runs a deep-nucleus row path on the host (deep_row, cx_deep.hpp, or with
// MODE 16 deep16_row, cx_deep16.hpp), one workgroup at a time, with every
// buffer an exact-size heap allocation under AddressSanitizer.  Each row's
// maximum goes into its slice record, as the fused kernel leaves it.  Output
// per row: the sampled id, or -2 where the path hands the row back.
// usage: deep_path_emu IN OUT [MODE] (written and read by tests/test_emu_deep_path.py)
#include "cx_deep16.hpp"
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

template <class T> static T* rd(FILE* f, size_t n) {
  T* p = (T*)malloc(n * sizeof(T) > 0 ? n * sizeof(T) : 1);
  if (n && fread(p, sizeof(T), n, f) != n) { fprintf(stderr, "short read\n"); exit(2); }
  return p;
}

int main(int argc, char** argv) {
  FILE* in = fopen(argv[1], "rb");
  FILE* out = fopen(argv[2], "wb");
  const bool counted = argc > 3 && atoi(argv[3]) == 16;
  const size_t lds = counted ? (size_t)FIN_CAP * 32 : (size_t)DEEP_LDS;
  int32_t ngroups;
  if (fread(&ngroups, 4, 1, in) != 1) return 2;
  for (int g = 0; g < ngroups; ++g) {
    int32_t hdr[3];
    if (fread(hdr, 4, 3, in) != 3) return 2;
    const int B = hdr[0], V = hdr[1], bf16 = hdr[2];
    const size_t esz = bf16 ? 2 : 4;
    void* x = rd<unsigned char>(in, (size_t)B * V * esz);
    cx_row_params* prm = rd<cx_row_params>(in, B);
    double* u = rd<double>(in, B);
    int32_t* ids = (int32_t*)malloc(4 * B);
    int32_t* st = (int32_t*)malloc(4 * B);
    SplitStats* stats = (SplitStats*)calloc(B, sizeof(SplitStats));
    std::vector<double> maxes;
    for (int b = 0; b < B; ++b) {
      double m = -INFINITY;
      for (int i = 0; i < V; ++i) {
        const double v = bf16 ? (double)__uint_as_float((uint32_t)((const uint16_t*)x)[(size_t)b * V + i] << 16)
                              : (double)((const float*)x)[(size_t)b * V + i];
        if (v > m) m = v;                       // NaN never wins, as in the fused kernel
      }
      // the counted path finds the maximum itself (the fused kernel leaves
      // NaN for a row it does not stream) and records it for the paths
      // after it: check both
      stats[b].m = counted ? NAN : m;
      maxes.push_back(m);
    }
    SampleArgs A;
    memset(&A, 0, sizeof A);
    A.logits = x; A.ld = V; A.B = B; A.V = V; A.ldh = 0;
    A.prm = prm; A.u = u; A.out_id = ids; A.row_status = st; A.out_probs = nullptr;
    A.nsplit = 1; A.stats = stats; A.bf16 = bf16; A.logV = log((double)V);
    A.vec_ok = ((uintptr_t)x % 16 == 0) && ((size_t)V * esz % 16 == 0);   // as the library sets it
    for (int row = 0; row < B; ++row) {
      unsigned char* dyn = (unsigned char*)malloc(lds);
      for (size_t i = 0; i < lds; ++i) dyn[i] = (unsigned char)(i * 131 + 7);
      emu::Wave waves[16];
      emu::waves = waves;
      std::barrier<> bb(1024);
      emu::block_bar = &bb;
      blockIdx.x = row;
      int decided = -1;
      std::vector<std::thread> th;
      th.reserve(1024);
      for (int t = 0; t < 1024; ++t)
        th.emplace_back([&, t] {
          threadIdx.x = t;
          __shared__ double red_d[2 * NWAVE + 4];
          __shared__ int red_i[2 * NWAVE + 4];
          __shared__ Deep16Shared sh;
          const bool r = counted ? deep16_row(A, row, dyn, red_d, red_i, sh)
                                 : deep_row(A, row, dyn, red_d, red_i);
          if (t == 0) decided = r ? 1 : 0;
          waves[t >> 6].bar.arrive_and_drop();
          bb.arrive_and_drop();
        });
      for (auto& h : th) h.join();
      free(dyn);
      if (!decided) { ids[row] = -2; st[row] = -2; }
      // a counted row's recorded maximum (when it found a finite one)
      if (counted && std::isfinite(maxes[row]) && stats[row].m != maxes[row]) {
        fprintf(stderr, "row %d: recorded maximum %g, the row's is %g\n", row, stats[row].m,
                maxes[row]);
        return 5;
      }
    }
    fwrite(ids, 4, B, out);
    fwrite(st, 4, B, out);
    free(x); free(prm); free(u); free(ids); free(st); free(stats);
    fprintf(stderr, "group V=%d B=%d done\n", V, B);
  }
  fclose(out);
  return 0;
}
