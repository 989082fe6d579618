// Measurement-only kernels for bench.py (libnvhip_bench.so; not part of the nvhip C ABI): the bandwidth ceilings
// the HBM-bound kernels are compared against on the same part.
//
//  nvhip_bench_stream_copy   dst[i] = src[i] over n 16-byte vectors, grid-stride, nontemporal loads and stores:
//                            the plain read + write ceiling for a given byte count (and the known-size kernel that
//                            calibrates rocprof's FETCH_SIZE / WRITE_SIZE counters).
//  nvhip_bench_stream_rw     dst[i] = src[i] (reads_per_write 1) or src[i] ^ src[n + i] (2: two input streams,
//                            as SiLU x Mul reads gate and up) over n 16-byte output vectors, grid-stride,
//                            nontemporal: the ceiling for a kernel's byte counts (read = reads_per_write x write).
//  nvhip_bench_qk_pattern    the memory traffic of nvhip_qk_norm_rope_kv_bf16 (Qwen3 layout, D = 128, write_k off)
//                            with the arithmetic taken out: one 256-thread block per token, LANES = 8 lanes per head
//                            row holding two 16-byte chunks (the halves of RoPE), q rows copied to q_out, k and v rows
//                            to their cache slot (skipped for slot -1), the position, slot and cos/sin row read as the
//                            kernel reads them. What the kernel would take if its math were free.
//  nvhip_bench_hbm_sweep     one point of a sweep for the part's HBM ceiling: a read-only, write-only or 1:1 copy
//                            stream over n 16-byte vectors, `unroll` vectors in flight per lane (the loads of an
//                            iteration issued before its stores), plain / nontemporal / written-through (sc1)
//                            cache policy, a grid-stride grid of `blocks` 256-thread blocks or (blocks 0) a one-shot
//                            grid with one iteration per block.
//  nvhip_bench_mfma_lds      the bf16 MFMA ceiling: each wave issues 8 v_mfma_f32_32x32x16_bf16 per iteration (4
//                            accumulators), with R of them each followed by a 16-byte-per-lane LDS read (R KB per
//                            wave per iteration, R / 8 KB per MFMA) whose value is an operand of the next
//                            iteration's MFMAs, as a GEMM's fragment reads feed its next k step; one block per CU
//                            (96 KB of LDS), per-wave shader-clock and 100 MHz real-time counts around the loop.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace {

using nvhip::u32x4;
typedef float f32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void stream_copy_kernel(u32x4* __restrict__ dst, const u32x4* __restrict__ src,
                                                          int64_t n) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
    __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

template <int R>
__global__ __launch_bounds__(256) void stream_rw_kernel(u32x4* __restrict__ dst, const u32x4* __restrict__ src,
                                                        int64_t n) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride) {
    u32x4 v = __builtin_nontemporal_load(src + i);
    if constexpr (R == 2) v ^= __builtin_nontemporal_load(src + n + i);
    __builtin_nontemporal_store(v, dst + i);
  }
}

struct PatternArgs {
  uint16_t* q_out;
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_stride, k_stride, v_stride;
  const int64_t* positions;
  const int32_t* slots;
  const float* cos_sin;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t num_slots, max_pos;
  int Hq, Hkv;
  uint32_t mix;  // 0 at run time: keeps the cos/sin loads live without changing the copied bits
};

__global__ __launch_bounds__(256) void qk_pattern_kernel(const PatternArgs a) {
  constexpr int D = 128, HALF = 64, LANES = 8;
  const int r = threadIdx.x / LANES, e = (threadIdx.x % LANES) * 8;
  const int R = a.Hq + 2 * a.Hkv;
  if (r >= R) return;
  const int64_t t = blockIdx.x;
  int64_t pos = a.positions[t];
  pos = pos < 0 ? 0 : pos >= a.max_pos ? a.max_pos - 1 : pos;
  int64_t slot = a.slots[t];
  if (slot < 0 || slot >= a.num_slots) slot = -1;
  const uint16_t* src;
  uint16_t* dst;
  if (r < a.Hq) {
    src = a.q + t * a.q_stride + r * D;
    dst = a.q_out + (t * a.Hq + r) * D;
  } else if (r < a.Hq + a.Hkv) {
    if (slot < 0) return;
    src = a.k + t * a.k_stride + (r - a.Hq) * D;
    dst = a.k_cache + slot * (int64_t(a.Hkv) * D) + (r - a.Hq) * D;
  } else {
    if (slot < 0) return;
    src = a.v + t * a.v_stride + (r - a.Hq - a.Hkv) * D;
    dst = a.v_cache + slot * (int64_t(a.Hkv) * D) + (r - a.Hq - a.Hkv) * D;
  }
  // read once, with the nontemporal hint, as the kernel reads its rows
  u32x4 x1 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + e));
  u32x4 x2 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src + HALF + e));
  if (r < a.Hq + a.Hkv) {  // q and k rows read their cos / sin values as the kernel does
    const float* cs = a.cos_sin + pos * D;
    const f32x4 c0 = *reinterpret_cast<const f32x4*>(cs + e), c1 = *reinterpret_cast<const f32x4*>(cs + e + 4);
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(cs + HALF + e);
    const f32x4 s1 = *reinterpret_cast<const f32x4*>(cs + HALF + e + 4);
    x1[0] ^= (__float_as_uint(c0[0]) ^ __float_as_uint(c1[0])) & a.mix;
    x2[0] ^= (__float_as_uint(s0[0]) ^ __float_as_uint(s1[0])) & a.mix;
  }
  __builtin_nontemporal_store(x1, reinterpret_cast<u32x4*>(dst + e));
  __builtin_nontemporal_store(x2, reinterpret_cast<u32x4*>(dst + HALF + e));
}

// MODE 0 read only (the loaded words xor-folded; one store per lane only if the fold hits a value random data does
// not give, so the loads stay live), 1 write only, 2 copy. POL 0 plain loads and stores, 1 nontemporal loads and
// stores, 2 plain loads and written-through stores, 3 nontemporal loads and written-through stores.
template <int MODE, int U, int POL>
__global__ __launch_bounds__(256) void hbm_sweep_kernel(u32x4* __restrict__ dst, const u32x4* __restrict__ src,
                                                        int64_t n, uint32_t salt) {
  const int64_t step = int64_t(gridDim.x) * 256 * U;
  u32x4 fold = {0u, 0u, 0u, 0u};
  for (int64_t base = int64_t(blockIdx.x) * 256 * U + threadIdx.x; base < n; base += step) {
    u32x4 v[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int64_t i = base + int64_t(k) * 256;
      if constexpr (MODE == 1) {
        v[k] = u32x4{uint32_t(i), salt, uint32_t(i) ^ salt, uint32_t(k)};
      } else if (i < n) {
        v[k] = (POL & 1) ? __builtin_nontemporal_load(src + i) : src[i];
      } else {
        v[k] = u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int64_t i = base + int64_t(k) * 256;
      if constexpr (MODE == 0) {
        fold ^= v[k];
      } else if (i < n) {
        if constexpr (POL >= 2) nvhip::store16_wt(dst + i, v[k]);
        else if constexpr (POL == 1) __builtin_nontemporal_store(v[k], dst + i);
        else dst[i] = v[k];
      }
    }
  }
  if constexpr (MODE == 0)
    if (fold[0] == salt && fold[1] == ~salt && fold[2] == salt && fold[3] == ~salt)
      dst[int64_t(blockIdx.x) * 256 + threadIdx.x] = fold;
}

template <int MODE, int U>
void launch_sweep_pol(int pol, dim3 grid, hipStream_t s, u32x4* dst, const u32x4* src, int64_t n) {
  switch (pol) {
    case 0: hipLaunchKernelGGL((hbm_sweep_kernel<MODE, U, 0>), grid, dim3(256), 0, s, dst, src, n, 0x9e3779b9u); break;
    case 1: hipLaunchKernelGGL((hbm_sweep_kernel<MODE, U, 1>), grid, dim3(256), 0, s, dst, src, n, 0x9e3779b9u); break;
    case 2: hipLaunchKernelGGL((hbm_sweep_kernel<MODE, U, 2>), grid, dim3(256), 0, s, dst, src, n, 0x9e3779b9u); break;
    default: hipLaunchKernelGGL((hbm_sweep_kernel<MODE, U, 3>), grid, dim3(256), 0, s, dst, src, n, 0x9e3779b9u);
  }
}

template <int MODE>
void launch_sweep_u(int unroll, int pol, dim3 grid, hipStream_t s, u32x4* dst, const u32x4* src, int64_t n) {
  switch (unroll) {
    case 1: launch_sweep_pol<MODE, 1>(pol, grid, s, dst, src, n); break;
    case 2: launch_sweep_pol<MODE, 2>(pol, grid, s, dst, src, n); break;
    case 4: launch_sweep_pol<MODE, 4>(pol, grid, s, dst, src, n); break;
    default: launch_sweep_pol<MODE, 8>(pol, grid, s, dst, src, n);
  }
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kProbeLds = 96 * 1024;   // dynamic LDS per block: one block per CU
constexpr int kProbeSpan = 64 * 1024;  // bytes the reads cycle through

template <int R>
__global__ __launch_bounds__(1024) void mfma_lds_kernel(int iters, unsigned long long* __restrict__ clocks,
                                                        float* __restrict__ sink) {
  extern __shared__ __align__(16) unsigned char lds[];
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  // bf16 values in [1, 2): the sums stay finite over any iteration count used here
  for (int i = threadIdx.x; i < kProbeSpan / 4; i += blockDim.x)
    reinterpret_cast<uint32_t*>(lds)[i] = 0x3f803f80u + ((i & 0x7f) << 16) + (i >> 7 & 0x7f);
  __syncthreads();
  bf16x8 f[8];
#pragma unroll
  for (int m = 0; m < 8; ++m) f[m] = *reinterpret_cast<const bf16x8*>(lds + m * 1024 + lane * 16);
  f32x16 c[4] = {};
  __syncthreads();
  const unsigned long long t0 = clock64(), w0 = wall_clock64();
  for (int it = 0; it < iters; ++it) {
    const uint32_t off = uint32_t(it * 8 + wave) * 1024u % kProbeSpan;
    bf16x8 nf[R > 0 ? R : 1];
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      c[m % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[m], f[(m + 1) % 8], c[m % 4], 0, 0, 0);
      if (m < R) nf[m] = *reinterpret_cast<const bf16x8*>(lds + (off + m * 3072u) % kProbeSpan + lane * 16);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int m = 0; m < R; ++m) f[m] = nf[m];
  }
  const unsigned long long t1 = clock64(), w1 = wall_clock64();
  float s = 0.0f;
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += c[m][e];
  sink[int64_t(blockIdx.x) * blockDim.x + threadIdx.x] = s;
  if (lane == 0) {
    const int64_t w = int64_t(blockIdx.x) * (blockDim.x / 64) + wave;
    clocks[2 * w] = t1 - t0;
    clocks[2 * w + 1] = w1 - w0;
  }
}

template <int R>
int launch_mfma_lds(int waves, int iters, int blocks, unsigned long long* clocks, float* sink, hipStream_t s) {
  static bool attr = false;
  if (!attr) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(&mfma_lds_kernel<R>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, kProbeLds) != hipSuccess)
      return -2;
    attr = true;
  }
  hipLaunchKernelGGL(mfma_lds_kernel<R>, dim3(blocks), dim3(64 * waves), kProbeLds, s, iters, clocks, sink);
  return 0;
}

}  // namespace

// reads: LDS reads of 16 bytes per lane per 8 MFMAs (0, 2, 4, 6 or 8); waves per block 4, 8 or 16 (1, 2 or 4 per
// SIMD). clocks: 2 x blocks x waves uint64 (shader clocks, 100 MHz ticks per wave); sink: blocks x 64 x waves floats.
extern "C" int nvhip_bench_mfma_lds(int reads, int waves, int iters, int blocks, void* clocks, void* sink,
                                    void* stream) {
  if (!clocks || !sink || iters <= 0 || blocks <= 0 || (waves != 4 && waves != 8 && waves != 16)) return -1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto* c = static_cast<unsigned long long*>(clocks);
  auto* k = static_cast<float*>(sink);
  int rc;
  switch (reads) {
    case 0: rc = launch_mfma_lds<0>(waves, iters, blocks, c, k, s); break;
    case 2: rc = launch_mfma_lds<2>(waves, iters, blocks, c, k, s); break;
    case 4: rc = launch_mfma_lds<4>(waves, iters, blocks, c, k, s); break;
    case 6: rc = launch_mfma_lds<6>(waves, iters, blocks, c, k, s); break;
    case 8: rc = launch_mfma_lds<8>(waves, iters, blocks, c, k, s); break;
    default: return -1;
  }
  if (rc) return rc;
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

// bytes: the stream's length (read-only: bytes read; write-only: bytes written; copy: bytes read = bytes written),
// a multiple of 16. dst must hold `bytes` (read-only: one 16-byte vector per thread of the grid, written only if
// the fold hits the salt pattern). blocks 0: one-shot grid of ceil(n / (256 * unroll)) blocks.
extern "C" int nvhip_bench_hbm_sweep(void* dst, const void* src, int64_t bytes, int mode, int unroll, int policy,
                                     int blocks, void* stream) {
  if (!dst || (mode != 1 && !src) || bytes <= 0 || bytes % 16 || mode < 0 || mode > 2 || policy < 0 ||
      policy > 3 || blocks < 0 || (unroll != 1 && unroll != 2 && unroll != 4 && unroll != 8))
    return -1;
  const int64_t n = bytes / 16;
  const int64_t grid = blocks > 0 ? blocks : (n + 256 * unroll - 1) / (256 * unroll);
  if (grid > INT32_MAX) return -1;
  if (mode == 0 && grid * 256 > n) return -1;  // the read-only kernel's conditional store lands in dst[0, grid * 256)
  hipStream_t s = static_cast<hipStream_t>(stream);
  u32x4* d = static_cast<u32x4*>(dst);
  const u32x4* r = static_cast<const u32x4*>(src);
  const dim3 g(static_cast<unsigned>(grid));
  if (mode == 0) launch_sweep_u<0>(unroll, policy, g, s, d, r, n);
  else if (mode == 1) launch_sweep_u<1>(unroll, policy, g, s, d, r, n);
  else launch_sweep_u<2>(unroll, policy, g, s, d, r, n);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

extern "C" int nvhip_bench_stream_copy(void* dst, const void* src, int64_t bytes, int blocks, void* stream) {
  if (!dst || !src || bytes <= 0 || bytes % 16 || blocks <= 0) return -1;
  hipLaunchKernelGGL(stream_copy_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<u32x4*>(dst), static_cast<const u32x4*>(src), bytes / 16);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

extern "C" int nvhip_bench_stream_rw(void* dst, const void* src, int64_t write_bytes, int reads_per_write,
                                     int blocks, void* stream) {
  if (!dst || !src || write_bytes <= 0 || write_bytes % 16 || blocks <= 0 ||
      (reads_per_write != 1 && reads_per_write != 2))
    return -1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (reads_per_write == 1)
    hipLaunchKernelGGL(stream_rw_kernel<1>, dim3(blocks), dim3(256), 0, s, static_cast<u32x4*>(dst),
                       static_cast<const u32x4*>(src), write_bytes / 16);
  else
    hipLaunchKernelGGL(stream_rw_kernel<2>, dim3(blocks), dim3(256), 0, s, static_cast<u32x4*>(dst),
                       static_cast<const u32x4*>(src), write_bytes / 16);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}

extern "C" int nvhip_bench_qk_pattern(void* q_out, const void* q, const void* k, const void* v, int64_t q_stride,
                                      int64_t k_stride, int64_t v_stride, const int64_t* positions,
                                      const int32_t* slots, const float* cos_sin, int64_t max_pos, void* k_cache,
                                      void* v_cache, int64_t num_slots, int64_t T, int64_t Hq, int64_t Hkv,
                                      void* stream) {
  if (T <= 0 || Hq <= 0 || Hkv <= 0 || (Hq + 2 * Hkv) * 8 > 256 || !q_out || !q || !k || !v || !positions ||
      !slots || !cos_sin || !k_cache || !v_cache || max_pos <= 0)
    return -1;
  PatternArgs a{static_cast<uint16_t*>(q_out), static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                static_cast<const uint16_t*>(v), q_stride, k_stride, v_stride, positions, slots, cos_sin,
                static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), num_slots, max_pos, int(Hq),
                int(Hkv), 0u};
  hipLaunchKernelGGL(qk_pattern_kernel, dim3(unsigned(T)), dim3(256), 0, static_cast<hipStream_t>(stream), a);
  return hipGetLastError() == hipSuccess ? 0 : -2;
}
