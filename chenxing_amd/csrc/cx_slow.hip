// cx_slow.hip -- launches the exact multi-pass row path (cx_slow.hpp) for
// the rows the fused sampler left pending.  One workgroup covers
// SLOW_ROWS_PER_WG rows (one: pending rows run in parallel); a workgroup
// whose rows are all decided reads their status words once and exits.
#include "cx_slow.hpp"
#include "cx_timing.hpp"

namespace cx {

constexpr int SLOW_ROWS_PER_WG = 1;

__global__ __launch_bounds__(WG) void slow_kernel(SampleArgs A) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ double red_d[2 * NWAVE + 4];
  __shared__ int red_i[2 * NWAVE + 4];
  __shared__ uint32_t s_pending;
  const int row0 = blockIdx.x * SLOW_ROWS_PER_WG;
  if (threadIdx.x < 64) {
    const int r = row0 + (int)threadIdx.x;
    const bool p = threadIdx.x < SLOW_ROWS_PER_WG && r < A.B && A.row_status[r] == ROW_PENDING;
    const uint64_t b = __ballot(p);
    if (threadIdx.x == 0) s_pending = (uint32_t)b;
  }
  __syncthreads();
  uint32_t pend = s_pending;
  while (pend) {
    const int j = __builtin_ctz(pend);
    pend &= pend - 1;
    slow_row(A, row0 + j, dyn, red_d, red_i);
    __syncthreads();
  }
}

int launch_slow(const SampleArgs& A, hipStream_t s) {
  static int attr = 0;
  if (A.slow_lds_bytes > attr) {
    hipError_t e = hipFuncSetAttribute((const void*)slow_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       A.slow_lds_bytes);
    if (e != hipSuccess) return (int)e;
    attr = A.slow_lds_bytes;
  }
  const int grid = (A.B + SLOW_ROWS_PER_WG - 1) / SLOW_ROWS_PER_WG;
  timed_launch(CX_KERNEL_SAMPLE_SLOW, slow_kernel, dim3(grid), dim3(WG), A.slow_lds_bytes, s, A);
  return (int)hipGetLastError();
}

}  // namespace cx
