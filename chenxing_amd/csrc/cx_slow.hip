// cx_slow.hip -- kernels built on the exact multi-pass row path
// (cx_slow.hpp):
//   slow_kernel       follows every fused launch, one workgroup per row.
//                     Rows the fused kernel left with a region (every row
//                     computed in several slices, and single-slice rows
//                     marked FINISH) get the region finisher; rows it left
//                     for refinement get their normaliser recomputed
//                     exactly in fp64 and the region finished again; pending
//                     rows (or, for fp64 logits, every row) get the exact
//                     multi-pass path, as does any row the steps before
//                     cannot decide; a pending top-p / min-p row without
//                     top-k, typical-p or penalties first tries the
//                     bucketed deep-nucleus path (cx_deep.hpp).  A
//                     workgroup whose row is decided reads its status word
//                     and exits.  In a bf16 call it takes only the rows
//                     finish16_kernel hands back.
//   finish16_kernel   bf16 calls: the finisher and the refinement, then
//                     deep-nucleus rows by counting values (cx_deep16.hpp);
//                     each workgroup takes its row from a counter
//   penalties_kernel  Sampler.apply_penalties, grid (rows, chunks of PEN_CHUNK)
//   truncate_kernel   Sampler._truncate, one workgroup per row
#include "cx_slow.hpp"
#include "cx_deep.hpp"
#include "cx_deep16.hpp"
#include "cx_finish.hpp"
#include "cx_timing.hpp"

namespace cx {

constexpr int PEN_CHUNK = 16384;     // elements per penalties_kernel workgroup

// A row whose region is complete and whose only open question is a top-p
// cut within the streamed normaliser's error bound: the exact fp64
// normaliser over the row (streamed with its loads ahead when the row has no
// penalty window), then the region finished with it.  Returns false, with
// nothing written, if the row still needs the multi-pass path.
__device__ __forceinline__ bool refine_row(const SampleArgs& A, int row, unsigned char* dyn, double* red_d,
                                  int* red_i) {
  const cx_row_params P = A.prm[row];
  SlowRow R;
  const int wlen = slow_setup(A, row, P, dyn, R);
  if (wlen > WIN_MAX || !(P.temperature > 0.0)) return false;
  // the row's maximum penalised value, as the finisher takes it
  double M = -__builtin_inf();
  for (int s = 0; s < A.nsplit; ++s) {
    const double m = A.stats[(size_t)row * A.nsplit + s].m;
    M = m > M ? m : M;
  }
  if (!(M > -__builtin_inf()) || !(M < __builtin_inf())) return false;
  const double S = R.pen || A.f64 ? exact_norm(R, M, 1.0 / P.temperature, red_d)
                                  : deep_exact_sum(A, row, M, 1.0 / P.temperature, red_d);
  __syncthreads();                       // the penalty tables in dyn are dead from here
  if (!(S > 0.0) || !(S < __builtin_inf())) return false;
  return finish_row_fast<FIN_CAP>(A, row, P, dyn, red_d, red_i, S) == FIN_DONE;
}

__global__ __launch_bounds__(WG) void slow_kernel(SampleArgs A) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ double red_d[2 * NWAVE + 4];
  __shared__ int red_i[2 * NWAVE + 4];
  __shared__ int s_state;
  enum { DECIDED, MULTIPASS, REFINE, FINISH };
  const int row = (int)blockIdx.x;
  int state = FINISH;
  // a sliced row's status word is not written by the fused kernel: every
  // sliced row is finished here, with no load before the finisher's own
  if (A.pending_only || A.all_slow || A.nsplit == 1) {
    if (threadIdx.x == 0) {
      const int st = A.row_status[row];
      s_state = A.pending_only ? (st == ROW_PENDING ? MULTIPASS : DECIDED)
                : A.all_slow ? MULTIPASS
                : st == ROW_FINISH ? FINISH
                : st == ROW_PENDING ? MULTIPASS
                : st == ROW_REFINE ? REFINE : DECIDED;
    }
    __syncthreads();
    state = s_state;
  }
  if (state == DECIDED) return;
  if (state == FINISH) {
    const cx_row_params P = A.prm[row];
    const int r = finish_row_fast<FIN_CAP>(A, row, P, dyn, red_d, red_i);
    if (r == FIN_DONE) return;
    state = r == FIN_REFINE ? REFINE : MULTIPASS;
    __syncthreads();
  }
  if (state == REFINE && refine_row(A, row, dyn, red_d, red_i)) return;
  __syncthreads();
  if (deep_row(A, row, dyn, red_d, red_i)) return;
  __syncthreads();
  slow_row(A, row, dyn, red_d, red_i);
}

// finish16_kernel's work items, in the order they are taken: 1 for a row
// that may go deep without a top-k bound (the ones that can be long), 2 for
// one with a top-k bound (counted, its kept set near the top), 3 for
// another row with work; 0 for a row with nothing left to do.  From the
// fused kernel's hand-off marks (one load), which nothing changes during
// the kernel; a sliced row's are all finished, its class from its
// parameters.  A pending row that cannot go deep is left to slow_kernel as
// it is.
__device__ inline int f16_class(const SampleArgs& A, int row) {
  int m;
  if (A.nsplit > 1) {
    const cx_row_params& P = A.prm[row];
    m = ROW_FINISH | (deep_candidate(A, row, P, true) ? MARK_DEEP : 0) |
        (P.top_k > 0 && P.top_k < A.V ? MARK_TOPK : 0);
  } else {
    m = A.counters[row];
  }
  const int mark = m & ~(MARK_DEEP | MARK_TOPK);
  const int deep = !(m & MARK_DEEP) ? 3 : (m & MARK_TOPK) ? 2 : 1;
  if (mark == ROW_FINISH || mark == ROW_REFINE) return deep;
  return mark == ROW_PENDING && deep != 3 ? deep : 0;
}

// The row of item idx of finish16_kernel's list: the class-1 rows in row
// order (n1 of them), then the class-2 rows (n2), then the class-3 rows.
// Every thread gets it.  cnt: NWAVE ints; out: one int.
__device__ inline int f16_item_row(const SampleArgs& A, int idx, int n1, int n2, int* cnt,
                                   int* out) {
  const int want = idx < n1 ? 1 : idx < n1 + n2 ? 2 : 3;
  const int target = idx < n1 ? idx : idx < n1 + n2 ? idx - n1 : idx - n1 - n2;
  const int t = threadIdx.x, w = wave_id();
  int base = 0;                                   // items of that class in earlier chunks
  if (t == 0) *out = -1;                          // (ordered by the loop's first barrier)
  for (int c = 0; c < A.B && base <= target; c += WG) {
    const bool is = c + t < A.B && f16_class(A, c + t) == want;
    const uint64_t b = ballot(is);
    if (lane_id() == 0) cnt[w] = __popcll(b);
    __syncthreads();
    int below = base, tot = 0;
    for (int j = 0; j < NWAVE; ++j) {
      const int n = cnt[j];
      below += j < w ? n : 0;
      tot += n;
    }
    if (is && below + lanes_below(b) == target) *out = c + t;
    base += tot;
    __syncthreads();
  }
  return *out;
}

// In place of slow_kernel's first part for a bf16 call: the region finisher
// and the refinement as there, then, for a row still open, the counted
// deep-nucleus path; a row none of them decides is marked ROW_PENDING for a
// slow_kernel launch that takes only those.  (A kernel without the
// multi-pass path: slow_kernel's register allocation stays as it is, and a
// deep-nucleus row starts counting right after its finisher gives up.)
// Grid B: each workgroup takes the next work item from a counter, in the
// order the workgroups start (f16_class: the rows that may be long, then the
// counted top-k rows, then the finisher rows), so the long rows start
// together on the first workgroups, the others follow on the CUs as they
// free up, and the workgroups left without an item exit last.  (With one
// workgroup per row and kind, blockIdx order, some deep rows started 40 us
// late, behind workgroups that only read a status word and exit.)
__global__ __launch_bounds__(WG) void finish16_kernel(SampleArgs A) {
  extern __shared__ __align__(16) unsigned char dyn[];
  __shared__ double red_d[2 * NWAVE + 4];
  __shared__ int red_i[2 * NWAVE + 4];
  __shared__ Deep16Shared sh;
  __shared__ int s_item[2];
  enum { OPEN, REFINE, FINISH };
  const int t = threadIdx.x;
  if (t == 0) s_item[0] = atomicAdd(A.counters + A.B, 1);
  int n1 = 0, n2 = 0, nw = 0;
  for (int c = 0; c < A.B; c += WG) {
    const int cls = c + t < A.B ? f16_class(A, c + t) : 0;
    n1 += cls == 1;
    n2 += cls == 2;
    nw += cls != 0;
  }
  n1 = block_sum(n1, red_i);                      // (its barriers also publish s_item[0])
  n2 = block_sum(n2, red_i);
  nw = block_sum(nw, red_i);
  const int idx = s_item[0];
  if (idx >= nw) return;
  const int row = f16_item_row(A, idx, n1, n2, red_i, s_item + 1);
  if (row < 0) return;                            // (every workgroup's list is the same)
  const int mark = A.nsplit > 1 ? ROW_FINISH : A.counters[row] & ~(MARK_DEEP | MARK_TOPK);
  int state = mark == ROW_FINISH ? FINISH : mark == ROW_REFINE ? REFINE : OPEN;
  if (state == FINISH) {
    const cx_row_params P = A.prm[row];
    const int r = finish_row_fast<FIN_CAP>(A, row, P, dyn, red_d, red_i);
    if (r == FIN_DONE) return;
    state = r == FIN_REFINE ? REFINE : OPEN;
    __syncthreads();
  }
  if (state == REFINE && refine_row(A, row, dyn, red_d, red_i)) return;
  __syncthreads();
  if (deep16_row(A, row, dyn, red_d, red_i, sh)) return;
  if (t == 0) A.row_status[row] = ROW_PENDING;
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
  static int attr = 0, attr16 = 0;
  // the multi-pass layout, or a refined row's finisher region (which also
  // holds the deep-nucleus paths' tables and counters)
  static_assert(DEEP_LDS <= FIN_CAP * 32, "deep-nucleus LDS");
  const int bytes = max(A.slow_lds_bytes, FIN_CAP * 32);
  if (int e = set_lds(slow_kernel, bytes, attr)) return e;
  SampleArgs A1 = A;
  A1.pending_only = 0;
  if (A.bf16 && !A.all_slow && !A.out_probs) {
    // rows of a bf16 call may take the counted deep-nucleus path:
    // finish16_kernel, then slow_kernel for the rows it hands back
    if (int e = set_lds(finish16_kernel, FIN_CAP * 32, attr16)) return e;
    timed_launch(CX_KERNEL_SAMPLE_SLOW, finish16_kernel, dim3(A.B), dim3(WG), FIN_CAP * 32, s,
                 A1);
    A1.pending_only = 1;
  }
  timed_launch(CX_KERNEL_SAMPLE_SLOW, slow_kernel, dim3(A.B), dim3(WG), bytes, s, A1);
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
