// cx_head.hip -- the LM-head projection with the greedy draw fused, for
// gfx950 (reference chenxing/model/transformer.py:102-104, the last
// hidden state times out_w.T, then chenxing/core/sampler.py:114-115, the
// argmax of the row): the [B, V] logits are never written to HBM.
//
// logits[b, v] = sum_k hidden[b, k] * W[v, k], with bf16 hidden states and
// head weights (row-major [B, D] and [V, D]) and fp32 accumulation on
// MFMA (v_mfma_f32_16x16x32_bf16: A = 16 vocab rows x 32 k, B = 32 k x 16
// batch rows, C = 16 x 16 fp32).  Two stream-ordered launches:
//
//   1. head_tiles   grid (ceil(V / 512), ceil(B / (16 NB))), 16 waves each.
//                   A wave owns 32 vocab rows (two 16-row MFMA tiles) and
//                   the workgroup's 16 NB batch rows, and runs the whole k
//                   loop: the head weights are streamed once from HBM (each
//                   element read by one lane), the hidden states are staged
//                   in LDS once per workgroup.  The
//                   accumulators are reduced in registers and LDS to one
//                   64-bit key per (workgroup, batch row): the orderable
//                   logit above the complement of the vocab id, so the
//                   largest key is the largest logit with the lowest id on
//                   ties, and a NaN logit (key above +inf) the first NaN --
//                   numpy's argmax.
//   2. head_merge   one workgroup per batch row: the largest of its keys.
//
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

#include "cx_device.hpp"
#include "cx_internal.hpp"
#include "cx_sampler.h"
#include "cx_timing.hpp"

namespace cx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int HEAD_WG = 256;                 // merge workgroup
constexpr int HEAD_NW = 16;                  // waves per tile workgroup
constexpr int HEAD_MT = 2;                   // 16-row vocab tiles per wave
constexpr int HEAD_VT = HEAD_NW * 16 * HEAD_MT;   // vocab rows per workgroup
constexpr int HEAD_KB = 128;                 // k per block (4 MFMA slices)
constexpr int HEAD_LDS = 152 * 1024;         // hidden-state chunk in LDS (at most)

struct HeadArgs {
  const uint16_t* hidden;   // [B, ldh] bf16 bits
  const uint16_t* weight;   // [V, ldw] bf16 bits
  int64_t ldh, ldw;
  int B, D, V;
  uint64_t* part;           // [gridDim.x, B] keys
  int nvt;                  // gridDim.x
  int kc;                   // k per LDS chunk of hidden states
  int32_t* out_id;
  float* out_max;           // nullable [B]
  float* out_logits;        // nullable [B, V] (verification)
};

// 16 bytes of head weights: a plain load (the non-temporal form measured
// 0.5 us slower over the 1 GB at B=16)
__device__ __forceinline__ u32x4 ld16(const uint16_t* p) {
  return *(const u32x4*)p;
}

// The 64-bit argmax key of logit x at vocab id v.
__device__ __forceinline__ uint64_t head_key(float x, int v) {
  const uint32_t k = x != x ? 0xFFFFFFFFu : f2key(x);
  return ((uint64_t)k << 32) | (uint32_t)~(uint32_t)v;
}

// One k block of a wave's weights: its two vocab tiles, 4 MFMA slices each.
struct HeadBlock {
  u32x4 w[HEAD_MT][4];
};

__device__ __forceinline__ void head_load(HeadBlock& x, const uint16_t* const (&wp)[HEAD_MT],
                                          int kb) {
#pragma unroll
  for (int m = 0; m < HEAD_MT; ++m)
#pragma unroll
    for (int s = 0; s < 4; ++s) x.w[m][s] = ld16(wp[m] + kb + 32 * s);
}

// The block's MFMAs; the hidden-state operands come from the LDS chunk
// (row r of the chunk at hs + r * hstride, this lane's k offset applied).
template <int NB>
__device__ __forceinline__ void head_mfma(const HeadBlock& x, const CX_LDS uint16_t* hs,
                                          int hstride, int kc, f32x4 (&acc)[HEAD_MT][NB]) {
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    u32x4 h[NB];
#pragma unroll
    for (int n = 0; n < NB; ++n)
      h[n] = *(const CX_LDS u32x4*)(hs + (size_t)16 * n * hstride + kc + 32 * s);
#pragma unroll
    for (int m = 0; m < HEAD_MT; ++m)
#pragma unroll
      for (int n = 0; n < NB; ++n)
        acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            __builtin_bit_cast(bf16x8, x.w[m][s]), __builtin_bit_cast(bf16x8, h[n]), acc[m][n],
            0, 0, 0);
  }
}

// Workgroups of HEAD_NW waves, HEAD_NW * 32 vocab rows.  The hidden states
// of the workgroup's 16 NB batch rows are staged in LDS a chunk of KC k at
// a time (rows padded by 16 bytes so the 16 rows of an MFMA operand fall in
// different banks); each wave streams its weights through a register ring
// of DEPTH blocks, so DEPTH - 1 blocks' loads are in flight while one is
// multiplied.
template <int NB, int DEPTH>
__global__ __launch_bounds__(HEAD_NW * 64) void head_tiles(HeadArgs A) {
  extern __shared__ __align__(16) unsigned char head_lds[];
  __shared__ uint64_t s_key[HEAD_NW][16 * NB];
  CX_LDS uint16_t* const hsh = to_lds((uint16_t*)head_lds);
  const int w = wave_id(), l = lane_id();
  const int g = l >> 4, c = l & 15;
  const int v0 = blockIdx.x * (HEAD_NW * 16 * HEAD_MT) + w * 16 * HEAD_MT;
  const int b0 = blockIdx.y * 16 * NB;
  const int KC = A.kc;                   // k per staged chunk (a multiple of HEAD_KB)
  const int hstride = KC + 8;            // LDS row stride, in bf16
  // the weight rows this lane loads (clamped into the matrix; keys of rows
  // past V are never used); slice s of lane group g is k = kb + 32 s + 8 g
  // + i, so each load instruction reads 64 contiguous bytes of 16 rows
  const uint16_t* wp[HEAD_MT];
#pragma unroll
  for (int m = 0; m < HEAD_MT; ++m)
    wp[m] = A.weight + (size_t)min(v0 + 16 * m + c, A.V - 1) * A.ldw + 8 * g;
  const CX_LDS uint16_t* const hs = hsh + (size_t)c * hstride + 8 * g;
  f32x4 acc[HEAD_MT][NB];
#pragma unroll
  for (int m = 0; m < HEAD_MT; ++m)
#pragma unroll
    for (int n = 0; n < NB; ++n) acc[m][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  HeadBlock ring[DEPTH];
  for (int k0 = 0; k0 < A.D; k0 += KC) {
    const int kn = min(KC, A.D - k0);
    // the chunk's first weight blocks, then the hidden states into LDS
#pragma unroll
    for (int d = 0; d < DEPTH - 1; ++d)
      if (d * HEAD_KB < kn) head_load(ring[d], wp, k0 + d * HEAD_KB);
    if (k0 > 0) __syncthreads();         // every wave is done with the last chunk
    for (int i = threadIdx.x; i < 16 * NB * (kn / 8); i += HEAD_NW * 64) {
      const int r = i / (kn / 8), e = (i % (kn / 8)) * 8;
      const uint16_t* src = A.hidden + (size_t)min(b0 + r, A.B - 1) * A.ldh + k0 + e;
      *(CX_LDS u32x4*)(hsh + (size_t)r * hstride + e) = *(const u32x4*)src;
    }
    __syncthreads();
    for (int kb = 0; kb < kn; kb += DEPTH * HEAD_KB) {
#pragma unroll
      for (int d = 0; d < DEPTH; ++d) {
        const int k = kb + d * HEAD_KB;
        if (k >= kn) break;
        const int kx = k + (DEPTH - 1) * HEAD_KB;
        if (kx < kn) head_load(ring[(d + DEPTH - 1) % DEPTH], wp, k0 + kx);
        head_mfma<NB>(ring[d], hs, hstride, k, acc);
      }
    }
  }
  // lane (g, c) holds logits of vocab rows v0 + 16 m + 4 g + j (j < 4) at
  // batch row b0 + 16 n + c
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    const int b = b0 + 16 * n + c;
    uint64_t key = 0;
#pragma unroll
    for (int m = 0; m < HEAD_MT; ++m)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int v = v0 + 16 * m + 4 * g + j;
        const float x = acc[m][n][j];
        if (v < A.V) {
          const uint64_t k = head_key(x, v);
          key = k > key ? k : key;
          if (A.out_logits && b < A.B) A.out_logits[(size_t)b * A.V + v] = x;
        }
      }
    // the four lane groups of column c
    uint64_t o = __shfl_xor(key, 16);
    key = o > key ? o : key;
    o = __shfl_xor(key, 32);
    key = o > key ? o : key;
    if (g == 0) s_key[w][16 * n + c] = key;
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < 16 * NB && b0 + t < A.B) {
    uint64_t key = s_key[0][t];
#pragma unroll
    for (int k = 1; k < HEAD_NW; ++k) key = s_key[k][t] > key ? s_key[k][t] : key;
    A.part[(size_t)(b0 + t) * A.nvt + blockIdx.x] = key;
  }
}

// One workgroup per batch row: the largest key of its workgroups, four
// loads per thread in flight together.
__global__ __launch_bounds__(HEAD_WG) void head_merge(HeadArgs A) {
  __shared__ uint64_t s_red[HEAD_WG / 64];
  const int b = blockIdx.x;
  const uint64_t* p = A.part + (size_t)b * A.nvt;
  uint64_t key = 0;
  for (int i0 = 0; i0 < A.nvt; i0 += 4 * HEAD_WG) {
    uint64_t k[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = i0 + j * HEAD_WG + (int)threadIdx.x;
      k[j] = i < A.nvt ? p[i] : 0;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) key = k[j] > key ? k[j] : key;
  }
  key = wave_reduce(key, OpMax());
  if (lane_id() == 0) s_red[wave_id()] = key;
  __syncthreads();
  if (threadIdx.x == 0) {
#pragma unroll
    for (int j = 1; j < HEAD_WG / 64; ++j) key = s_red[j] > key ? s_red[j] : key;
    A.out_id[b] = (int32_t)~(uint32_t)key;
    if (A.out_max) {
      const uint32_t k = (uint32_t)(key >> 32);
      A.out_max[b] = k == 0xFFFFFFFFu ? __builtin_nanf("") : key2f(k);
    }
  }
}

// k per LDS chunk for nb batch tiles: the largest multiple of HEAD_KB whose
// padded rows fit HEAD_LDS, at most D.
static int head_kc(int D, int nb) {
  int kc = (HEAD_LDS / (16 * nb * 2) - 8) / HEAD_KB * HEAD_KB;
  return kc < D ? kc : D;
}

int launch_head(const HeadArgs& A0, hipStream_t s) {
  HeadArgs A = A0;
  // 16-row batch tiles per wave (four spill: their accumulators and a ring
  // of two blocks exceed the 128 VGPRs of a 16-wave workgroup)
  const int nb = A.B >= 32 ? 2 : 1;
  A.kc = head_kc(A.D, nb);
  const dim3 grid(A.nvt, (A.B + 16 * nb - 1) / (16 * nb));
  const uint32_t lds = (uint32_t)(16 * nb * (A.kc + 8) * 2);
  const dim3 blk(HEAD_NW * 64);
  using K = void (*)(HeadArgs);
  static const K kern[2] = {head_tiles<1, 3>, head_tiles<2, 2>};
  const int v = nb - 1;
  // the dynamic-LDS limit raised once per variant to the most any launch takes
  static std::once_flag once[2];
  hipError_t err = hipSuccess;
  std::call_once(once[v], [&] {
    err = hipFuncSetAttribute((const void*)kern[v], hipFuncAttributeMaxDynamicSharedMemorySize,
                              HEAD_LDS);
  });
  if (err != hipSuccess) return (int)err;
  timed_launch(CX_KERNEL_LMHEAD, kern[v], grid, blk, lds, s, A);
  timed_launch(CX_KERNEL_LMHEAD_MERGE, head_merge, dim3(A.B), dim3(HEAD_WG), 0, s, A);
  return (int)hipGetLastError();
}

}  // namespace cx

extern "C" {

size_t cx_lmhead_workspace_bytes(int32_t B, int32_t V) {
  if (B <= 0 || V <= 0) return 256;
  return ((size_t)B * ((V + cx::HEAD_VT - 1) / cx::HEAD_VT) * 8 + 255) & ~(size_t)255;
}

int cx_lmhead_argmax_bf16(const uint16_t* hidden, int64_t ldh, const uint16_t* weight,
                          int64_t ldw, int32_t B, int32_t D, int32_t V, int32_t* out_id,
                          float* out_max, float* out_logits, void* workspace, size_t ws_bytes,
                          void* stream) {
  if (B < 0 || V < 1 || D < 1 || ldh < D || ldw < D)
    return cx::api_fail(CX_EINVAL, "bad shape");
  if (B == 0) return CX_OK;
  if (D % cx::HEAD_KB != 0)
    return cx::api_fail(CX_EINVAL, "D (%d) must be a multiple of %d", D, cx::HEAD_KB);
  if (!hidden || !weight || !out_id || !workspace)
    return cx::api_fail(CX_EINVAL, "null pointer argument");
  if ((((uintptr_t)hidden | (uintptr_t)weight) & 15) || ((ldh | ldw) & 7))
    return cx::api_fail(CX_EINVAL, "hidden and weight rows must be 16-byte aligned");
  if (ws_bytes < cx_lmhead_workspace_bytes(B, V))
    return cx::api_fail(CX_ENOSPACE, "workspace holds %zu bytes, needs %zu", ws_bytes,
                        cx_lmhead_workspace_bytes(B, V));
  cx::HeadArgs A;
  A.hidden = hidden; A.weight = weight; A.ldh = ldh; A.ldw = ldw;
  A.B = B; A.D = D; A.V = V;
  A.nvt = (V + cx::HEAD_VT - 1) / cx::HEAD_VT;
  A.part = (uint64_t*)workspace;
  A.out_id = out_id; A.out_max = out_max; A.out_logits = out_logits;
  const int e = cx::launch_head(A, (hipStream_t)stream);
  if (e != 0) return cx::api_fail(CX_EHIP, "lm-head launch: %s", hipGetErrorString((hipError_t)e));
  return CX_OK;
}

}  // extern "C"
