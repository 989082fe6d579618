// Paged KV-cache write (unfused): the standalone counterpart of the KV half of the fused qk_norm_rope_kv kernel,
// for models whose q/k take another path (qkv bias, no q/k norm).
//
// Replaces store_kvcache() of nanovllm/layers/attention.py:34-41 (its Triton kernel :11-31): token t's row of
// row_elems = Hkv * head_dim elements of key and value (rows at key + t * key_stride, value + t * value_stride,
// elements contiguous) is copied to row slot_mapping[t] of k_cache and v_cache ([num_slots, row_elems]
// contiguous: blocks x block_size slots). Slots outside [0, num_slots) -- the padding value -1 -- are skipped.
//
// Threads take U = 1, 4 or 8 16-byte chunks of the rows, flattened over (token, chunk) with a grid-stride loop, and
// issue all their loads (the slot, read by every thread of its token, and the k / v chunks) before their stores. Rows whose base or stride is not 16-byte aligned go through a 2/4-byte
// element loop instead. The data is copied as raw bits (bf16, fp16 or fp32).
#include <algorithm>

#include "common.h"

namespace nvhip {
namespace {

struct StoreArgs {
  char* kc;
  char* vc;
  const char* k;
  const char* v;
  const int32_t* slots;
  int64_t k_stride, v_stride;  // bytes
  int64_t num_slots, n, row_bytes;
};

template <int U>
__global__ __launch_bounds__(256) void store_kvcache_vec(const StoreArgs g) {
  const int64_t chunks = g.row_bytes / 16, total = g.n * chunks, stride = int64_t(gridDim.x) * 256;
  for (int64_t i0 = int64_t(blockIdx.x) * 256 + threadIdx.x; i0 < total; i0 += stride * U) {
    // U chunks per thread, all loads first: the row loads do not wait for the slot (a padded token's row is read
    // and dropped); the rows are written with the nontemporal hint, as the fused kernel writes its cache rows
    int32_t slot[U];
    int64_t c[U];
    u32x4 kv[U], vv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + u * stride;
      slot[u] = -1;
      if (i < total) {
        const int64_t t = i / chunks;
        c[u] = (i - t * chunks) * 16;
        slot[u] = g.slots[t];
        kv[u] = *reinterpret_cast<const u32x4*>(g.k + t * g.k_stride + c[u]);
        vv[u] = *reinterpret_cast<const u32x4*>(g.v + t * g.v_stride + c[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (slot[u] < 0 || slot[u] >= g.num_slots) continue;
      __builtin_nontemporal_store(kv[u], reinterpret_cast<u32x4*>(g.kc + int64_t(slot[u]) * g.row_bytes + c[u]));
      __builtin_nontemporal_store(vv[u], reinterpret_cast<u32x4*>(g.vc + int64_t(slot[u]) * g.row_bytes + c[u]));
    }
  }
}
template <typename E>
__global__ __launch_bounds__(256) void store_kvcache_elem(const StoreArgs g) {
  const int64_t per = g.row_bytes / int64_t(sizeof(E)), total = g.n * per;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < total; i += int64_t(gridDim.x) * 256) {
    const int64_t t = i / per, e = i - t * per;
    const int32_t slot = g.slots[t];
    if (slot < 0 || slot >= g.num_slots) continue;
    reinterpret_cast<E*>(g.kc + int64_t(slot) * g.row_bytes)[e] = reinterpret_cast<const E*>(g.k + t * g.k_stride)[e];
    reinterpret_cast<E*>(g.vc + int64_t(slot) * g.row_bytes)[e] = reinterpret_cast<const E*>(g.v + t * g.v_stride)[e];
  }
}

}  // namespace
}  // namespace nvhip

extern "C" int nvhip_store_kvcache(void* k_cache, void* v_cache, const void* key, const void* value,
                                   int64_t key_stride, int64_t value_stride, const int32_t* slot_mapping,
                                   int64_t num_slots, int64_t n, int64_t row_elems, int64_t elem_size,
                                   void* stream) {
  using namespace nvhip;
  clear_error();
  if (n < 0 || row_elems < 0 || num_slots < 0) return invalid("store_kvcache: negative size");
  if (elem_size != 2 && elem_size != 4) return invalid("store_kvcache: element size must be 2 or 4 bytes");
  if (key_stride < row_elems || value_stride < row_elems) return invalid("store_kvcache: row stride < row size");
  if (n == 0 || row_elems == 0) return NVHIP_OK;
  if (!k_cache || !v_cache || !key || !value || !slot_mapping) return invalid("store_kvcache: null pointer");
  StoreArgs g{static_cast<char*>(k_cache), static_cast<char*>(v_cache), static_cast<const char*>(key),
              static_cast<const char*>(value), slot_mapping, key_stride * elem_size, value_stride * elem_size,
              num_slots, n, row_elems * elem_size};
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool vec = g.row_bytes % 16 == 0 && g.k_stride % 16 == 0 && g.v_stride % 16 == 0 && aligned16(key) &&
                   aligned16(value) && aligned16(k_cache) && aligned16(v_cache);
  // 16-byte chunks per thread: 8 while that still gives every CU a block (T = 8192 rows of 2 KiB: 14.2 -> 13.2 us,
  // the same-bytes copy 12.8 us; 4 chunks 13.7 us, 16 chunks 13.1 us), 4 at the next size down, else 1
  const int64_t chunks = vec ? n * (g.row_bytes / 16) : 0;
  const int U = chunks >= (int64_t(8) << 16) ? 8 : chunks >= (int64_t(4) << 16) ? 4 : 1;
  const int64_t work = vec ? (chunks + U - 1) / U : n * row_elems;
  const unsigned grid = unsigned(std::min<int64_t>((work + 255) / 256, 1 << 20));
  if (vec && U == 8) hipLaunchKernelGGL(store_kvcache_vec<8>, dim3(grid), dim3(256), 0, s, g);
  else if (vec && U == 4) hipLaunchKernelGGL(store_kvcache_vec<4>, dim3(grid), dim3(256), 0, s, g);
  else if (vec) hipLaunchKernelGGL(store_kvcache_vec<1>, dim3(grid), dim3(256), 0, s, g);
  else if (elem_size == 2) hipLaunchKernelGGL(store_kvcache_elem<uint16_t>, dim3(grid), dim3(256), 0, s, g);
  else hipLaunchKernelGGL(store_kvcache_elem<uint32_t>, dim3(grid), dim3(256), 0, s, g);
  return check_launch("store_kvcache");
}
