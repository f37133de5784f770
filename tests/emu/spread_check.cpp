// The device's tie-group survivor counts (cx_device.hpp spread_kept,
// spread_keeps, spread_rem / spread_step), compiled for the host and checked
// against the exact integer formula floor((2 R j + n - 1) / (2 n)) (long
// rows) and min(R, j) (rows of at most TIE_NET ids) over random and extreme
// group sizes up to 2^20.  Prints "ok" or the first
// mismatch.
#include "cx_device.hpp"
#include <random>
using namespace cx;

static long long exact(long long R, long long j, long long n) {
  if (j <= 0 || n <= 0) return 0;
  if (j >= n) return R;
  return (2 * R * j + n - 1) / (2 * n);
}

int main() {
  std::mt19937_64 g(12345);
  const long long NMAX = 1 << 20;
  long long checked = 0;
  for (int it = 0; it < 200000; ++it) {
    long long n = it < 1000 ? NMAX - (it % 7) : 1 + (long long)(g() % NMAX);
    long long j = (it % 3 == 0) ? n - 1 - (long long)(g() % 3) : (long long)(g() % (n + 1));
    if (j < 0) j = 0;
    long long R = (long long)(g() % (n + 1));
    for (int net = 0; net < 2; ++net) {
      const long long want_k = net ? (j >= n ? R : (R < j ? R : j)) : exact(R, j, n);
      if (spread_kept(R, j, n, net) != want_k) {
        printf("kept net=%d R=%lld j=%lld n=%lld: %lld != %lld\n", net, R, j, n,
               spread_kept(R, j, n, net), want_k);
        return 1;
      }
      // the incremental form over a run of consecutive members
      if (n > 0 && j > 0) {
        int rem = spread_rem(R, j, n, net);
        for (long long r = R; r < R + 64 && r < n; ++r) {
          const bool want = net ? r < j : exact(r + 1, j, n) > exact(r, j, n);
          if (spread_keeps(r, j, n, net) != want || spread_step(rem, (int)j, (int)n, net) != want) {
            printf("step net=%d r=%lld j=%lld n=%lld\n", net, r, j, n);
            return 1;
          }
          ++checked;
        }
      }
    }
  }
  printf("ok %lld\n", checked);
  return 0;
}
