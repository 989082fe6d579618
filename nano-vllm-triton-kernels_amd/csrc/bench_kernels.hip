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
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
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

}  // namespace

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
