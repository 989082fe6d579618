// Greedy token choice: the index of the largest logit of each row (bf16 logits).
//
// Replaces the greedy branch of Sampler.forward (nanovllm/layers/sampler.py:9-10: logits.float().argmax(dim=-1)).
// bf16 -> fp32 is exact, so comparing the bf16 values is comparing the float ones, and the order is torch's: a NaN
// is larger than any number, equal values (and two NaNs) go to the smaller index -- a strict total order on
// (value, index) pairs, so the maximum is unique and any reduction order finds it.
//
// Each thread visits its elements in increasing index order, so inside a thread "strictly larger, or the first
// NaN" replaces the running best (no index comparison); threads, waves and blocks merge with the full order.
// With a workspace the row is split over S blocks (S * rows >= 512: every CU gets work) whose (value, index)
// results a second launch merges per row; without one, one block per row. At 32 x 151936 (a decode step of
// Qwen3-0.6B) one block per row takes 30 us (32 CUs, each VALU bound), the split form a few us; torch's bf16 ->
// fp32 copy and ArgMaxOps took 6.6 + 59.8 us.
#include <algorithm>
#include <cfloat>

#include "common.h"

namespace nvhip {
namespace {

constexpr int kThreads = 256;

struct Best {
  float v;
  int64_t i;
};

// a beats b in torch's argmax order
__device__ __forceinline__ bool beats(float av, int64_t ai, float bv, int64_t bi) {
  const bool an = av != av, bn = bv != bv;
  if (an || bn) return an && (!bn || ai < bi);
  return av > bv || (av == bv && ai < bi);
}

// x comes after everything b has seen (larger index): it wins if strictly larger, or the first NaN
__device__ __forceinline__ void take_later(Best& b, float x, int64_t i) {
  if (x > b.v || (x != x && b.v == b.v)) b.v = x, b.i = i;
}

__device__ __forceinline__ void merge(Best& b, float v, int64_t i) {
  if (beats(v, i, b.v, b.i)) b.v = v, b.i = i;
}

// Best of elements [lo, hi) of a row (lo a multiple of 8 when VEC), over the block; the result in thread 0.
template <bool VEC>
__device__ __forceinline__ Best block_best(const uint16_t* row, int64_t lo, int64_t hi) {
  const int tid = threadIdx.x;
  Best b{-INFINITY, INT64_MAX};  // loses to every element
  int64_t tail = lo;
  if constexpr (VEC) {
    const int64_t c0 = lo / 8, c1 = hi / 8;  // whole 16-byte chunks
    const u32x4* rv = reinterpret_cast<const u32x4*>(row);
    int64_t c = c0 + tid;
    for (; c + 3 * kThreads < c1; c += 4 * kThreads) {
      u32x4 q[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) q[u] = rv[c + u * kThreads];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        float f[8];
        unpack8(q[u], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) take_later(b, f[e], (c + u * kThreads) * 8 + e);
      }
    }
    for (; c < c1; c += kThreads) {
      float f[8];
      unpack8(rv[c], f);
#pragma unroll
      for (int e = 0; e < 8; ++e) take_later(b, f[e], c * 8 + e);
    }
    tail = c1 * 8;
  }
  // elements past the last whole chunk (all of them without VEC): larger indices than the chunks above
  for (int64_t i = tail + tid; i < hi; i += kThreads) take_later(b, bf16_to_f32(row[i]), i);

#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(b.v, off);
    const int64_t oi = __shfl_xor(b.i, off);
    merge(b, ov, oi);
  }
  __shared__ float sv[kThreads / 64];
  __shared__ int64_t si[kThreads / 64];
  if (tid % 64 == 0) sv[tid / 64] = b.v, si[tid / 64] = b.i;
  __syncthreads();
  if (tid == 0)
    for (int w = 1; w < kThreads / 64; ++w) merge(b, sv[w], si[w]);
  return b;
}

// blockIdx.y = row, blockIdx.x = slice s of `span` elements; S == 1: the index itself, else the slice's best
template <bool VEC>
__global__ __launch_bounds__(kThreads) void argmax_slices_kernel(int64_t* __restrict__ out, Best* __restrict__ part,
                                                                 const uint16_t* __restrict__ x, int64_t n,
                                                                 int64_t stride, int64_t span) {
  const int64_t lo = int64_t(blockIdx.x) * span, hi = std::min(n, lo + span);
  const Best b = block_best<VEC>(x + int64_t(blockIdx.y) * stride, lo, hi);
  if (threadIdx.x == 0) {
    if (gridDim.x == 1) out[blockIdx.y] = b.i < n ? b.i : 0;
    else part[int64_t(blockIdx.y) * gridDim.x + blockIdx.x] = b;
  }
}

// one wave per row: merges the S slice results (S <= 64)
__global__ __launch_bounds__(64) void argmax_merge_kernel(int64_t* __restrict__ out, const Best* __restrict__ part,
                                                          int S, int64_t n) {
  const int l = threadIdx.x;
  Best b = l < S ? part[int64_t(blockIdx.x) * S + l] : Best{-INFINITY, INT64_MAX};
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(b.v, off);
    const int64_t oi = __shfl_xor(b.i, off);
    merge(b, ov, oi);
  }
  if (l == 0) out[blockIdx.x] = b.i < n ? b.i : 0;
}

// slices per row: enough blocks for every CU (rows * S >= 512), slices of at least 4096 elements, S <= 64
int argmax_slices(int64_t rows, int64_t n) {
  int64_t s = (512 + rows - 1) / rows;
  s = std::min<int64_t>(s, (n + 4095) / 4096);
  return int(std::max<int64_t>(1, std::min<int64_t>(s, 64)));
}

}  // namespace
}  // namespace nvhip

extern "C" int64_t nvhip_argmax_workspace_size(int64_t rows, int64_t n) {
  if (rows <= 0 || n <= 0) return 0;
  const int S = nvhip::argmax_slices(rows, n);
  return S > 1 ? rows * S * int64_t(sizeof(nvhip::Best)) : 0;
}

extern "C" int nvhip_argmax_bf16(int64_t* out, const void* logits, int64_t rows, int64_t n, int64_t row_stride,
                                 void* workspace, int64_t workspace_size, void* stream) {
  using namespace nvhip;
  clear_error();
  if (rows < 0 || n <= 0) return invalid("argmax: rows must be >= 0 and n > 0");
  if (row_stride < n) return invalid("argmax: row stride < n");
  if (rows >= 65536) return invalid("argmax: at most 65535 rows");
  if (rows == 0) return NVHIP_OK;
  if (!out || !logits) return invalid("argmax: null pointer");
  int S = argmax_slices(rows, n);
  if (S > 1 && (!workspace || workspace_size < rows * S * int64_t(sizeof(Best)) ||
                (reinterpret_cast<uintptr_t>(workspace) & 15)))
    S = 1;  // no (usable) workspace: one block per row
  const bool vec = aligned16(logits) && row_stride % 8 == 0;
  // slice length: a multiple of 8 (whole chunks) covering n in S slices
  const int64_t span = S == 1 ? n : ((n + S - 1) / S + 7) / 8 * 8;
  S = int((n + span - 1) / span);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* x = static_cast<const uint16_t*>(logits);
  Best* part = static_cast<Best*>(workspace);
  const dim3 grid(static_cast<unsigned>(S), static_cast<unsigned>(rows));
  if (vec) hipLaunchKernelGGL(argmax_slices_kernel<true>, grid, dim3(kThreads), 0, s, out, part, x, n, row_stride, span);
  else hipLaunchKernelGGL(argmax_slices_kernel<false>, grid, dim3(kThreads), 0, s, out, part, x, n, row_stride, span);
  if (int rc = check_launch("argmax")) return rc;
  if (S == 1) return NVHIP_OK;
  hipLaunchKernelGGL(argmax_merge_kernel, dim3(unsigned(rows)), dim3(64), 0, s, out, part, S, n);
  return check_launch("argmax merge");
}
