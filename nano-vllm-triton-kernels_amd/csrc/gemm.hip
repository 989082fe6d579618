// GEMM C = A @ B with fp32 accumulation for gfx950.
//
// Replaces nanovllm/kernels/matmul.py (Triton, :11-99): A [M, K], B [K, N] with arbitrary element strides
// (B = W.t() of an nn.Linear weight [N, K] is the common case), fp32 or bf16 inputs, C [M, N] in the input dtype.
// fp32 inputs: precision "ieee" uses them as they are, "tf32" rounds each input to a 10-bit mantissa
// (round to nearest even) before the products, which is what a tf32 tensor-core product sees.
//
// Kernels:
//   gemm_mfma_nt   bf16, A and B both K-contiguous (sak == 1, sbk == 1): 32x32x16 bf16 MFMA, LDS-staged
//                  double-buffered tiles, GROUP_M-swizzled tile order remapped so that neighbouring tiles share an
//                  XCD (and its L2). See gemm_mfma.inc.
//   gemm_generic   any dtype/strides/precision: 64x64 tile, 4x4 outputs per thread, fp32 FMA.
#include "common.h"

namespace nvhip {
namespace {

constexpr int kBlock = 256;

__device__ __forceinline__ float round_tf32(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7f800000u) == 0x7f800000u) return x;  // inf / nan unchanged
  u += 0xfffu + ((u >> 13) & 1u);
  return __uint_as_float(u & 0xffffe000u);
}

template <typename T>
__device__ __forceinline__ float to_f32(T v);
template <>
__device__ __forceinline__ float to_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t v) { return bf16_to_f32(v); }

template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
template <>
__device__ __forceinline__ uint16_t from_f32<uint16_t>(float v) { return f32_to_bf16(v); }

struct GemmArgs {
  void* c;
  const void* a;
  const void* b;
  int64_t M, N, K;
  int64_t sam, sak, sbk, sbn, scm, scn;
};

// 64x64 output tile per 256-thread block; thread (ty, tx) owns rows ty + 16*i, cols tx + 16*j (i, j < 4).
// K is staged 16 at a time through LDS; out-of-range elements load as 0.
template <typename T, bool TF32>
__global__ __launch_bounds__(kBlock) void gemm_generic(const GemmArgs g) {
  constexpr int BM = 64, BN = 64, BK = 16;
  __shared__ float As[BK][BM + 1];
  __shared__ float Bs[BK][BN + 1];
  const T* A = static_cast<const T*>(g.a);
  const T* B = static_cast<const T*>(g.b);
  T* C = static_cast<T*>(g.c);
  const int64_t m0 = int64_t(blockIdx.y) * BM, n0 = int64_t(blockIdx.x) * BN;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < g.K; k0 += BK) {
    for (int i = threadIdx.x; i < BM * BK; i += kBlock) {
      const int r = i / BK, kk = i % BK;
      const int64_t m = m0 + r, k = k0 + kk;
      float v = (m < g.M && k < g.K) ? to_f32<T>(A[m * g.sam + k * g.sak]) : 0.0f;
      if constexpr (TF32) v = round_tf32(v);
      As[kk][r] = v;
    }
    for (int i = threadIdx.x; i < BN * BK; i += kBlock) {
      const int cidx = i % BN, kk = i / BN;
      const int64_t n = n0 + cidx, k = k0 + kk;
      float v = (n < g.N && k < g.K) ? to_f32<T>(B[k * g.sbk + n * g.sbn]) : 0.0f;
      if constexpr (TF32) v = round_tf32(v);
      Bs[kk][cidx] = v;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < BK; ++kk) {
      float av[4], bv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = As[kk][ty + 16 * i];
#pragma unroll
      for (int j = 0; j < 4; ++j) bv[j] = Bs[kk][tx + 16 * j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(av[i], bv[j], acc[i][j]);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t m = m0 + ty + 16 * i, n = n0 + tx + 16 * j;
      if (m < g.M && n < g.N) C[m * g.scm + n * g.scn] = from_f32<T>(acc[i][j]);
    }
}

template <typename T, bool TF32>
int launch_generic(const GemmArgs& g, hipStream_t s) {
  const int64_t gx = (g.N + 63) / 64, gy = (g.M + 63) / 64;
  if (gx > INT32_MAX || gy > 65535) return invalid("matmul: matrix too large");
  hipLaunchKernelGGL((gemm_generic<T, TF32>), dim3(unsigned(gx), unsigned(gy)), dim3(kBlock), 0, s, g);
  return check_launch("matmul");
}

}  // namespace
}  // namespace nvhip

extern "C" int nvhip_matmul(void* c, const void* a, const void* b, int64_t M, int64_t N, int64_t K, int64_t sam,
                            int64_t sak, int64_t sbk, int64_t sbn, int64_t scm, int64_t scn, int dtype,
                            int precision, void* stream) {
  using namespace nvhip;
  clear_error();
  if (M < 0 || N < 0 || K < 0) return invalid("matmul: negative size");
  if (sam < 0 || sak < 0 || sbk < 0 || sbn < 0 || scm < 0 || scn < 0) return invalid("matmul: negative stride");
  if (dtype != NVHIP_DTYPE_F32 && dtype != NVHIP_DTYPE_BF16) return invalid("matmul: dtype must be fp32 or bf16");
  if (precision != NVHIP_PREC_IEEE && precision != NVHIP_PREC_TF32)
    return invalid("matmul: precision must be ieee or tf32");
  if (M == 0 || N == 0) return NVHIP_OK;
  if (!c || (K > 0 && (!a || !b))) return invalid("matmul: null pointer");
  GemmArgs g{c, a, b, M, N, K, sam, sak, sbk, sbn, scm, scn};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == NVHIP_DTYPE_BF16) return launch_generic<uint16_t, false>(g, s);
  if (precision == NVHIP_PREC_TF32) return launch_generic<float, true>(g, s);
  return launch_generic<float, false>(g, s);
}
