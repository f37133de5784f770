// cx_slow.hip -- kernels built on the exact multi-pass row path
// (cx_slow.hpp):
//   slow_kernel       the rows the fused sampler left pending (or, for fp64
//                     logits, every row).  One workgroup per row; a
//                     workgroup whose row is decided reads its status word
//                     and exits.
//   penalties_kernel  Sampler.apply_penalties, grid (rows, chunks of PEN_CHUNK)
//   truncate_kernel   Sampler._truncate, one workgroup per row
#include "cx_slow.hpp"
#include "cx_timing.hpp"

namespace cx {

constexpr int PEN_CHUNK = 16384;     // elements per penalties_kernel workgroup

__global__ __launch_bounds__(WG) void slow_kernel(SampleArgs A) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ double red_d[2 * NWAVE + 4];
  __shared__ int red_i[2 * NWAVE + 4];
  __shared__ int s_pending;
  const int row = blockIdx.x;
  if (threadIdx.x == 0) s_pending = A.all_slow || A.row_status[row] == ROW_PENDING;
  __syncthreads();
  if (s_pending) slow_row(A, row, dyn, red_d, red_i);
}

__global__ __launch_bounds__(WG) void penalties_kernel(SampleArgs A) {
  extern __shared__ __align__(16) unsigned char dyn[];
  const int row = blockIdx.x;
  const int i0 = blockIdx.y * PEN_CHUNK;
  const int i1 = min(A.V, i0 + PEN_CHUNK);
  penalties_range(A, row, i0, i1, dyn, blockIdx.y == 0);
}

__global__ __launch_bounds__(WG) void truncate_kernel(SampleArgs A) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ double red_d[2 * NWAVE + 4];
  __shared__ int red_i[2 * NWAVE + 4];
  truncate_row(A, blockIdx.x, dyn, red_d, red_i);
}

template <typename K>
static int set_lds(K kernel, int bytes, int& attr) {
  if (bytes > attr) {
    hipError_t e = hipFuncSetAttribute((const void*)kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (e != hipSuccess) return (int)e;
    attr = bytes;
  }
  return 0;
}

int launch_slow(const SampleArgs& A, hipStream_t s) {
  static int attr = 0;
  if (int e = set_lds(slow_kernel, A.slow_lds_bytes, attr)) return e;
  timed_launch(CX_KERNEL_SAMPLE_SLOW, slow_kernel, dim3(A.B), dim3(WG), A.slow_lds_bytes, s, A);
  return (int)hipGetLastError();
}

int launch_penalties(const SampleArgs& A, hipStream_t s) {
  static int attr = 0;
  if (int e = set_lds(penalties_kernel, A.slow_lds_bytes, attr)) return e;
  const int nchunk = (A.V + PEN_CHUNK - 1) / PEN_CHUNK;
  timed_launch(CX_KERNEL_PENALTIES, penalties_kernel, dim3(A.B, nchunk), dim3(WG),
               A.slow_lds_bytes, s, A);
  return (int)hipGetLastError();
}

int launch_truncate(const SampleArgs& A, hipStream_t s) {
  static int attr = 0;
  if (int e = set_lds(truncate_kernel, A.slow_lds_bytes, attr)) return e;
  timed_launch(CX_KERNEL_TRUNCATE, truncate_kernel, dim3(A.B), dim3(WG), A.slow_lds_bytes, s, A);
  return (int)hipGetLastError();
}

}  // namespace cx
