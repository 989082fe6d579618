// Fused per-head q/k RMSNorm + RoPE + paged KV-cache write for gfx950.
//
// Replaces nanovllm/kernels/qk_norm_rope_kv.py (Triton, :29-125): everything between qkv_proj and attention in
// Qwen3's attention. Per token t it reads the q, k, v heads straight from their (strided) views of the qkv output
// and writes
//   q_out[t, h]                    normed + rotated q head                                  (always)
//   k_out[t, h]                    normed + rotated k head                                  (if k_out != NULL)
//   k_cache[slot, h], v_cache[slot, h]  normed + rotated k head, raw v head, slot = slot_mapping[t]
//                                  (if caches are given and 0 <= slot < num_slots; -1 = padding, skipped)
//
// Numerics are those of the torch code the kernel replaces (layers/layernorm.py:20-30 rms_forward,
// layers/rotary_embedding.py:6-14 apply_rotary_emb) as torch computes it eagerly on the GPU, bit for bit, with its
// two bf16 roundings:
//   rstd = rsqrt(sum(x^2) / D + eps)                fp32 sum in ATen's order, torch's rsqrt (common.h)
//   n    = bf16(bf16(x * rstd) * w)                 RMSNorm output (bf16, as q_norm/k_norm return it)
//   y1   = bf16(n1*cos - n2*sin), y2 = bf16(n2*cos + n1*sin)   n1/n2 the two halves, products rounded separately
// The file is compiled with -ffp-contract=off so no product is fused into an add (torch rounds each product).
//
// Mapping (wave64): a head row of D bf16 is handled by LANES = D/16 consecutive lanes; lane j of the group holds
// elements [8j, 8j+8) of both halves (two 16-byte loads), so RoPE pairs x1[i] with x2[i] inside the lane and the
// sum of squares is a LANES-wide DPP reduction per half. Row r of a token is q head r (r < Hq), k head r-Hq, or v head
// r-Hq-Hkv (R = Hq + 2*Hkv rows). One block per token (R*LANES threads): for Qwen3-0.6B (Hq 16, Hkv 8, D 128) a
// block is 4 waves (q 0-7, q 8-15, k 0-7, v 0-7), each reading 2 KB and writing 2 KB. Each KV row write is one
// contiguous 256-byte run at slot*Hkv*D + h*D. Very wide models (R*LANES > 1024) use a flattened row space.
#include "common.h"

namespace nvhip {
namespace {

constexpr int kBlock = 256;

struct QkArgs {
  uint16_t* q_out;
  uint16_t* k_out;
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  int64_t q_stride, k_stride, v_stride;
  const int64_t* positions;
  const int32_t* slot_mapping;
  const uint16_t* q_w;
  const uint16_t* k_w;
  const float* cos_sin;
  int64_t cos_sin_stride;
  int64_t max_pos;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t num_slots;
  int64_t total_rows;  // T * (Hq + 2*Hkv)
  int32_t Hq, Hkv, R;  // R = Hq + 2*Hkv rows per token
  float inv_d, eps;
};

// Output stores written through the L2 (store16_wt, common.h): T = 8192, inputs in HBM: 24.1 us, against 25.1 us
// with the nontemporal hint and 27 us with plain stores.
template <bool ALIGNED>
__device__ __forceinline__ void store_out(uint16_t* p, const u32x4& v) {
  if constexpr (ALIGNED) store16_wt(p, v);
  else store8<false>(p, v);
}

// One head row (q, k or v) of token t, handled by the LANES lanes of a group; `sub` is the lane within the group.
template <int D, bool ALIGNED>
__device__ __forceinline__ void process_row(const QkArgs& a, int64_t t, int r, int sub, int64_t pos, int64_t slot) {
  constexpr int HALF = D / 2;
  const int e = sub * 8;  // this lane's first element in each half
  int kind, h;
  const uint16_t* src;
  if (r < a.Hq) {
    kind = 0, h = r;
    src = a.q + t * a.q_stride + int64_t(h) * D;
  } else if (r < a.Hq + a.Hkv) {
    kind = 1, h = r - a.Hq;
    src = a.k + t * a.k_stride + int64_t(h) * D;
  } else {
    kind = 2, h = r - a.Hq - a.Hkv;
    src = a.v + t * a.v_stride + int64_t(h) * D;
  }
  if (kind == 0) slot = -1;
  const int64_t cache_off = slot * (int64_t(a.Hkv) * D) + int64_t(h) * D;

  if (kind == 2) {  // v: raw copy of the head row into the cache
    if (slot < 0) return;
    const u32x4 v1 = load8_once<ALIGNED>(src + e);
    const u32x4 v2 = load8_once<ALIGNED>(src + HALF + e);
    store_out<ALIGNED>(a.v_cache + cache_off + e, v1);
    store_out<ALIGNED>(a.v_cache + cache_off + HALF + e, v2);
    return;
  }
  if (kind == 1 && slot < 0 && a.k_out == nullptr) return;  // a k row with nowhere to go

  const u32x4 xa = load8_once<ALIGNED>(src + e);
  const u32x4 xb = load8_once<ALIGNED>(src + HALF + e);
  const uint16_t* w = kind == 0 ? a.q_w : a.k_w;
  const u32x4 wa = load8<ALIGNED>(w + e);
  const u32x4 wb = load8<ALIGNED>(w + HALF + e);
  const float* cs = a.cos_sin + pos * a.cos_sin_stride;
  float c[8], s[8];
  if constexpr (ALIGNED) {
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    const f32x4 c0 = *reinterpret_cast<const f32x4*>(cs + e), c1 = *reinterpret_cast<const f32x4*>(cs + e + 4);
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(cs + HALF + e);
    const f32x4 s1 = *reinterpret_cast<const f32x4*>(cs + HALF + e + 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) c[i] = c0[i], c[i + 4] = c1[i], s[i] = s0[i], s[i + 4] = s1[i];
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      c[i] = cs[e + i];
      s[i] = cs[HALF + e + i];
    }
  }

  // sum of squares in torch's order, then the norm and the rotation (common.h)
  float x1[8], x2[8];
  unpack8(xa, x1);
  unpack8(xb, x2);
  const float rstd = torch_rsqrt(torch_row_sumsq<D>(x1, x2) * a.inv_d + a.eps);
  u32x4 oa, ob;
  norm_rope16(x1, x2, rstd, wa, wb, c, s, oa, ob);

  if (kind == 0) {
    uint16_t* dst = a.q_out + (t * a.Hq + h) * int64_t(D);
    store_out<true>(dst + e, oa);
    store_out<true>(dst + HALF + e, ob);
    return;
  }
  if (a.k_out != nullptr) {
    uint16_t* dst = a.k_out + (t * a.Hkv + h) * int64_t(D);
    store_out<true>(dst + e, oa);
    store_out<true>(dst + HALF + e, ob);
  }
  if (slot >= 0) {
    store_out<ALIGNED>(a.k_cache + cache_off + e, oa);
    store_out<ALIGNED>(a.k_cache + cache_off + HALF + e, ob);
  }
}

__device__ __forceinline__ int64_t load_position(const QkArgs& a, int64_t t) {
  const int64_t pos = a.positions[t];
  return pos < 0 ? 0 : (pos >= a.max_pos ? a.max_pos - 1 : pos);
}

__device__ __forceinline__ int64_t load_slot(const QkArgs& a, int64_t t) {
  if (a.k_cache == nullptr) return -1;
  const int64_t slot = a.slot_mapping[t];
  return (slot < 0 || slot >= a.num_slots) ? -1 : slot;
}

// One token per block (blockDim = R * LANES rounded up to a whole wave): t is uniform, so the position and the
// slot are scalar loads and no division is needed. Used whenever R * LANES <= 1024.
template <int D, bool ALIGNED>
__global__ __launch_bounds__(1024) void qk_norm_rope_kv_token_kernel(const QkArgs a) {
  constexpr int LANES = D / 16;
  const int r = threadIdx.x / LANES;
  if (r >= a.R) return;  // whole groups leave together
  const int64_t t = blockIdx.x;
  process_row<D, ALIGNED>(a, t, r, threadIdx.x % LANES, load_position(a, t), load_slot(a, t));
}

// Flattened (token, row) space for more than 1024 / LANES rows per token: a 256-thread block covers 256 / LANES
// consecutive rows, which may belong to two tokens.
template <int D, bool ALIGNED>
__global__ __launch_bounds__(kBlock) void qk_norm_rope_kv_kernel(const QkArgs a) {
  constexpr int LANES = D / 16;
  constexpr int ROWS_PER_BLOCK = kBlock / LANES;
  const int64_t g = int64_t(blockIdx.x) * ROWS_PER_BLOCK + threadIdx.x / LANES;
  if (g >= a.total_rows) return;  // whole groups leave together
  const int64_t t = g / a.R;
  process_row<D, ALIGNED>(a, t, int(g - t * a.R), threadIdx.x % LANES, load_position(a, t), load_slot(a, t));
}

template <int D>
int launch(const QkArgs& a, int64_t T, bool aligned, hipStream_t stream) {
  constexpr int LANES = D / 16;
  const int64_t threads = (int64_t(a.R) * LANES + 63) / 64 * 64;
  if (threads <= 1024) {
    if (aligned)
      hipLaunchKernelGGL((qk_norm_rope_kv_token_kernel<D, true>), dim3(unsigned(T)), dim3(unsigned(threads)), 0,
                         stream, a);
    else
      hipLaunchKernelGGL((qk_norm_rope_kv_token_kernel<D, false>), dim3(unsigned(T)), dim3(unsigned(threads)), 0,
                         stream, a);
    return check_launch("qk_norm_rope_kv");
  }
  constexpr int ROWS_PER_BLOCK = kBlock / LANES;
  const int64_t blocks = (a.total_rows + ROWS_PER_BLOCK - 1) / ROWS_PER_BLOCK;
  if (aligned)
    hipLaunchKernelGGL((qk_norm_rope_kv_kernel<D, true>), dim3(unsigned(blocks)), dim3(kBlock), 0, stream, a);
  else
    hipLaunchKernelGGL((qk_norm_rope_kv_kernel<D, false>), dim3(unsigned(blocks)), dim3(kBlock), 0, stream, a);
  return check_launch("qk_norm_rope_kv");
}

}  // namespace
}  // namespace nvhip

extern "C" int nvhip_qk_norm_rope_kv_bf16(void* q_out, void* k_out, const void* q, const void* k, const void* v,
                                          int64_t q_stride, int64_t k_stride, int64_t v_stride,
                                          const int64_t* positions, const int32_t* slot_mapping,
                                          const void* q_weight, const void* k_weight, const float* cos_sin,
                                          int64_t cos_sin_stride, int64_t max_pos, void* k_cache, void* v_cache,
                                          int64_t num_slots, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                                          float eps, void* stream) {
  using namespace nvhip;
  clear_error();
  if (T < 0 || Hq <= 0 || Hkv <= 0 || D <= 0) return invalid("qk_norm_rope_kv: T must be >= 0 and Hq, Hkv, D > 0");
  if (Hq % Hkv != 0) return invalid("qk_norm_rope_kv: Hq must be a multiple of Hkv");
  if (D != 64 && D != 128 && D != 256) return invalid("qk_norm_rope_kv: head_dim must be 64, 128 or 256");
  if (Hq + 2 * Hkv > (1 << 20)) return invalid("qk_norm_rope_kv: too many heads");
  if (T == 0) return NVHIP_OK;
  const bool store = k_cache != nullptr || v_cache != nullptr;
  if (store && (k_cache == nullptr || v_cache == nullptr || slot_mapping == nullptr || num_slots < 0))
    return invalid("qk_norm_rope_kv: k_cache, v_cache and slot_mapping must be given together");
  if (!q_out || !q || !k || !v || !positions || !q_weight || !k_weight || !cos_sin)
    return invalid("qk_norm_rope_kv: null pointer");
  if (max_pos <= 0 || cos_sin_stride < D) return invalid("qk_norm_rope_kv: bad cos_sin cache shape");
  if (q_stride < Hq * D || k_stride < Hkv * D || v_stride < Hkv * D)
    return invalid("qk_norm_rope_kv: token strides must cover all heads");
  if (!aligned16(q_out) || (k_out && !aligned16(k_out)))
    return invalid("qk_norm_rope_kv: outputs must be 16-byte aligned");
  const bool aligned = aligned16(q) && aligned16(k) && aligned16(v) && aligned16(q_weight) &&
                       aligned16(k_weight) && q_stride % 8 == 0 && k_stride % 8 == 0 && v_stride % 8 == 0 &&
                       aligned16(cos_sin) && cos_sin_stride % 4 == 0 &&
                       (!store || (aligned16(k_cache) && aligned16(v_cache)));

  QkArgs a;
  a.q_out = static_cast<uint16_t*>(q_out);
  a.k_out = static_cast<uint16_t*>(k_out);
  a.q = static_cast<const uint16_t*>(q);
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.q_stride = q_stride, a.k_stride = k_stride, a.v_stride = v_stride;
  a.positions = positions;
  a.slot_mapping = store ? slot_mapping : nullptr;
  a.q_w = static_cast<const uint16_t*>(q_weight);
  a.k_w = static_cast<const uint16_t*>(k_weight);
  a.cos_sin = cos_sin;
  a.cos_sin_stride = cos_sin_stride;
  a.max_pos = max_pos;
  a.k_cache = store ? static_cast<uint16_t*>(k_cache) : nullptr;
  a.v_cache = store ? static_cast<uint16_t*>(v_cache) : nullptr;
  a.num_slots = store ? num_slots : 0;
  a.Hq = int32_t(Hq), a.Hkv = int32_t(Hkv), a.R = int32_t(Hq + 2 * Hkv);
  a.total_rows = T * a.R;
  a.inv_d = 1.0f / float(D);
  a.eps = eps;
  const int64_t max_blocks = (a.total_rows + 15) / 16;  // fewest rows per block: 16 (D = 256)
  if (max_blocks > INT32_MAX || T > INT32_MAX) return invalid("qk_norm_rope_kv: too many tokens");

  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (D) {
    case 64: return launch<64>(a, T, aligned, s);
    case 128: return launch<128>(a, T, aligned, s);
    default: return launch<256>(a, T, aligned, s);
  }
}
