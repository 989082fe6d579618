// Shared device helpers and host-side argument checking for the nvhip kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "nvhip.h"

namespace nvhip {

// ---------------------------------------------------------------- host: errors

void set_error(const std::string& msg);
void clear_error();

// Records msg and returns NVHIP_EINVAL.
int invalid(const std::string& msg);

// Checks the launch that was just issued; NVHIP_OK or NVHIP_ELAUNCH with the runtime's message.
int check_launch(const char* kernel);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Paged attention over the sequences of a varlen call that have 1 .. qmax queries (qmax * Hq / Hkv <= 16), with the
// paged decode kernel (paged_attention.hip), for a call with no longer sequence (otherwise the prefill kernel's
// blocks of these sequences run the same decode body, decode_attention.h): sequence b's queries are rows cu_q[b] .. cu_q[b+1]-1 of q / out, its
// keys the first cu_k[b+1] - cu_k[b] tokens of block_table row b, causal aligned to the bottom right. Sequences
// with more queries are not touched. With a workspace of at least paged_decode_varlen_workspace(...) bytes the keys
// of each (sequence, kv head) are split over blocks when there are fewer pairs than CUs (as the decode entry point
// does), merged by a second kernel. Sizes are checked by the caller; returns NVHIP_OK or an error code.
int paged_decode_varlen(uint16_t* out, const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                        const int32_t* block_table, const int32_t* cu_q, const int32_t* cu_k, int num_seqs, int qmax,
                        int Hq, int Hkv, int D, int block_size, int num_blocks, int max_blocks, int64_t q_st,
                        int64_t q_sh, int64_t o_st, int64_t o_sh, float scale, int causal, float* ws, int64_t ws_bytes,
                        hipStream_t s);
// Bytes of workspace paged_decode_varlen can use for num_seqs sequences of at most qmax queries (0: it never splits);
// independent of the context lengths.
int64_t paged_decode_varlen_workspace(int64_t num_seqs, int64_t qmax, int64_t Hq, int64_t Hkv, int64_t D);

// The attention workspaces (decode and prefill entry points) start with kAttnCounterBytes of per-(sequence, kv head)
// counters of the decode attention's in-kernel merge: zero before a call, and every call leaves them zero. Batches
// of up to kBalanceMaxPairs pairs (and 64 sequences) are balanced by length.
constexpr int64_t kBalanceMaxPairs = 512, kAttnCounterBytes = kBalanceMaxPairs * 4;
// Floats per record block of RP rows of the decode attention's split records: whole 128-byte lines when the blocks
// merge in the kernel (each line is written by one block).
constexpr int64_t decode_record_stride(int64_t RP, int64_t D, bool in_kernel) {
  const int64_t f = RP * (2 + D);
  return in_kernel ? (f + 31) / 32 * 32 : f;
}

// Add+RMSNorm (rms_norm.hip) of rows whose x is the sum of `splits` (1..4) fp32 partial products [splits, rows, n]
// (a split-K GEMM's): x = bf16(partials summed in split order), then exactly nvhip_add_rms_norm_bf16 with a
// contiguous residual (res_out may alias r). Only for the n add_rms_norm_partials_supported accepts.
bool add_rms_norm_partials_supported(int64_t n);
int add_rms_norm_partials(uint16_t* y, uint16_t* res_out, const float* xp, int splits, const uint16_t* r,
                          const uint16_t* w, int64_t rows, int64_t n, float eps, hipStream_t s);

// ---------------------------------------------------------------- device: bf16 <-> fp32

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// bf16 bits -> fp32 (exact).
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }

// Two fp32 -> two bf16 packed in one word (a in the low half), round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2 v = __builtin_convertvector((f32x2){a, b}, bf16x2);
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float a) { return uint16_t(pack_bf16x2(a, 0.0f)); }

// fp32 value rounded to the nearest bf16 (as an fp32): the .to(torch.bfloat16) of the torch code.
__device__ __forceinline__ float round_bf16(float a) { return bf16_lo(pack_bf16x2(a, 0.0f)); }

// silu(g) = g / (1 + exp(-g)) rounded to bf16: torch's own silu kernel formula (device expf, correctly rounded
// divide) on a bf16 input, as F.silu(gate) of layers/activation.py:15-18 computes it. Shared by the SiLU x Mul kernel
// and the GEMM epilogue that fuses it, so both give the same bits.
__device__ __forceinline__ float silu_bf16(float g) { return round_bf16(g / (1.0f + expf(-g))); }

// max / sum of v over lanes l and l ^ 32 of the wave, the same bits in both lanes: v_permlane32_swap of v with
// itself returns lanes 0..31 of v in one result and lanes 32..63 in the other (in every lane), a VALU op with no
// LDS round trip.
__device__ __forceinline__ float pair32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// gfx950 transpose read ds_read_b64_tr_b16 from a row-major bf16 tile in LDS: within each 16-lane group, lane i
// receives element i % 4 of the 8-byte chunks addressed by lanes 4j + i / 4 (j = 0..3, its 4 bf16 in that order;
// measured with an in-bounds one-wave probe). Lanes 4j .. 4j+3 addressing row j and 16 consecutive columns hand
// lane i column i of the 4 rows: the layout of an MFMA A/B operand read from a key-major tile.
__device__ __forceinline__ u32x2 lds_read_tr16(const uint16_t* p) {
  const s16x4_t v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_t*)(p));
  return __builtin_bit_cast(u32x2, v);
}

// 8 bf16 (16 bytes) <-> 8 fp32.
__device__ __forceinline__ void unpack8(const u32x4& v, float* f) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = bf16_lo(v[i]);
    f[2 * i + 1] = bf16_hi(v[i]);
  }
}
__device__ __forceinline__ u32x4 pack8(const float* f) {
  u32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
  return v;
}

// Loads/stores of 8 consecutive bf16. ALIGNED: one 16-byte access (pointer must be 16-byte aligned);
// otherwise 8 two-byte accesses.
template <bool ALIGNED>
__device__ __forceinline__ u32x4 load8(const uint16_t* p) {
  if constexpr (ALIGNED) {
    return *reinterpret_cast<const u32x4*>(p);
  } else {
    u32x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = uint32_t(p[2 * i]) | (uint32_t(p[2 * i + 1]) << 16);
    return v;
  }
}
// load8 for data the kernel reads exactly once (activations streamed through): with ALIGNED a 16-byte load with
// the nontemporal hint. Measured per kernel at T = 8192 with the inputs in HBM: the fused q/k norm kernel 26.4 ->
// 25.2 us and SiLU x Mul 28.3 -> 26.5 us use it; RMSNorm (6.6 -> 7.5 us), Add+RMSNorm and store_kvcache were slower
// with it and do not. The hint's loads do not hit in the Infinity Cache: inputs still held there read slower with
// it (the fused kernel at T = 2048 over 136 MB of rotating inputs: 7.3 us plain, 8.9 us nontemporal), and none of
// the sc0 / sc1 / nt cache-policy combinations of a buffer load was faster in both cases.
template <bool ALIGNED>
__device__ __forceinline__ u32x4 load8_once(const uint16_t* p) {
  if constexpr (ALIGNED) return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  else return load8<false>(p);
}

template <bool ALIGNED>
__device__ __forceinline__ void store8(uint16_t* p, const u32x4& v) {
  if constexpr (ALIGNED) {
    *reinterpret_cast<u32x4*>(p) = v;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[2 * i] = uint16_t(v[i]);
      p[2 * i + 1] = uint16_t(v[i] >> 16);
    }
  }
}

// A load from a wave-uniform address through the scalar data cache (s_load): it waits on lgkmcnt instead of
// queueing behind the wave's vector loads in flight, which retire in issue order. Only for data that no wave of the
// running kernel writes: the compiler treats it as constant (and may merge or move such loads across stores), and
// the scalar cache is invalidated when a kernel starts, not by the kernel's own vector stores.
template <typename T>
__device__ __forceinline__ T load_uniform(const T* p) {
  return *(const __attribute__((address_space(4))) T*)p;
}

// 16-byte store (p 16-byte aligned) written through this XCD's L2 at device scope: a buffer store with the sc1
// cache policy. The L2s of the 8 XCDs are not coherent with each other, so when a kernel ends its dirty L2 lines
// are written back before the next kernel starts; with plain or nontemporal stores that write-back runs after the
// last wave (bf16 GEMM at M = 2048, 16 MB of output: 3.0 us from the last block's end to the kernel's end, 0.3 us
// with this store). Used where it measured faster: the fused q/k norm kernel and the MFMA GEMM epilogues. RMSNorm,
// SiLU x Mul and the copy ceilings measured the same or slower, Add+RMSNorm 4 % and store_kvcache 13 % slower.
// The buffer resource is based on the first active lane's address rounded down to 1 GiB; a lane whose address lies
// in another 1 GiB window stores plainly.
__device__ __forceinline__ void store16_wt(void* p, const u32x4& v) {
  typedef float f32x4v __attribute__((ext_vector_type(4)));
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(a >> 32));
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(a)) & 0xC0000000u;
  const uint64_t b = (uint64_t(hi) << 32) | lo;
  if ((a >> 30) == (b >> 30)) {
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(b), (short)0, 0x7fffffff, 0x00020000);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(f32x4v, v), rs, uint32_t(a - b), 0, 16 /* sc1 */);
  } else {
    *reinterpret_cast<u32x4*>(p) = v;
  }
}

// ---------------------------------------------------------------- RMSNorm in torch's GPU order
// The reference's RMSNorm (layers/layernorm.py:20-44) run eagerly on the GPU computes mean(x^2) with ATen's generic
// reduction and rsqrt with ATen's rsqrt kernel. The kernels here reproduce both bit for bit:
//  - torch.rsqrt on a float tensor evaluates the double-precision device rsqrt and rounds it to float;
//  - the mean is an fp32 sum in ATen's order times factor = float(rows) / float(rows * n) (fp32), where the order
//    depends on n and on the number of rows: block width bw (threads per row) from aten_norm_bw(); thread L of a
//    row sums the 4-element vectors L, L + bw, ... (n >= 128; one accumulator per vector component, each from 0,
//    combined as ((a0 + a1) + a2) + a3), or single elements (n < 128); then for bw > 64 t[L] += t[L + off] for
//    off = bw/2 .. 64, then a tree of adjacent lanes (t[L] += t[L + 1], t[L] += t[L + 2], ...).
// A butterfly (xor) reduction gives every lane the value lane 0 of that tree gets (each level adds the same two
// operands), so group_sum below finishes it once each lane holds the partial of adjacent thread(s).

// (float) rsqrt((double) v): torch.rsqrt's result on a float tensor (its kernel calls the double overload).
__device__ __forceinline__ float torch_rsqrt(float v) { return float(rsqrt(double(v))); }

// ATen's threads per row (bw) for the mean over rows of n fp32 values, or 0 when a row is split over the waves of
// a block (then the order is not the one described above). Host-side; a restatement of the launch-shape
// arithmetic of torch's GPU reduction for a contiguous innermost dimension.
inline int aten_norm_bw(int64_t n, int64_t rows) {
  auto last_pow2 = [](int64_t x) { int64_t p = 1; while (p * 2 <= x) p *= 2; return p; };
  const int64_t dim0 = n >= 128 ? n / 4 : n;
  const int64_t d0 = dim0 < 512 ? last_pow2(dim0) : 512, d1 = rows < 512 ? last_pow2(rows) : 512;
  int64_t bw = d0 < 64 ? d0 : 64;
  const int64_t bh = d1 < 512 / bw ? d1 : 512 / bw;
  bw = d0 < 512 / bh ? d0 : 512 / bh;
  const int64_t per_thread = (n + bw - 1) / bw, split_at = bh * 16 < 256 ? bh * 16 : 256;
  if (bh > 1 && per_thread >= split_at) return 0;
  return int(bw);
}
// MeanOps' factor: float(num_outputs) / numel with the int64 numel converted to float.
inline float aten_mean_factor(int64_t n, int64_t rows) { return float(rows) / float(rows * n); }

// Thread partial over one 4-element vector of squares: ((y0 + y1) + y2) + y3.
__device__ __forceinline__ float sumsq4(const float* x) {
  return ((x[0] * x[0] + x[1] * x[1]) + x[2] * x[2]) + x[3] * x[3];
}

// Row layout "T32" for rows of n = 256 K elements (or 128, K = 1, with 16 lanes): a row is owned by 32 aligned
// lanes, lane j holding the 16-byte chunks k = 0 .. K-1 at elements 8 j + 256 k, i.e. the 4-element vectors
// 2 j + 64 k and 2 j + 1 + 64 k. With bw = 64 M, ATen thread 2 j + p + 64 c (p = 0, 1; c < M) owns exactly the
// vectors of chunks c, c + M, c + 2M, ... of parity p, so every thread partial and the bw > 64 halving levels are
// local to lane j, which returns t[2j] + t[2j+1] of the 64-wide tree (the first in-wave level). v[k][e]: element
// e of chunk k (fp32; the squares are formed here, each rounded). group_sum<32> then completes the sum.
template <int K, int M>
__device__ __forceinline__ float t32_partial(const float (*v)[8]) {
  static_assert(M >= 1 && M <= 8 && (M & (M - 1)) == 0 && M <= K, "bw = 64 M with M <= K");
  float t[2][M];
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int c = 0; c < M; ++c) {
      float acc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = v[c][4 * p + i] * v[c][4 * p + i];
#pragma unroll
      for (int k = c + M; k < K; k += M)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] += v[k][4 * p + i] * v[k][4 * p + i];
      t[p][c] = ((acc[0] + acc[1]) + acc[2]) + acc[3];
    }
#pragma unroll
  for (int off = M / 2; off >= 1; off /= 2)
#pragma unroll
    for (int p = 0; p < 2; ++p)
#pragma unroll
      for (int c = 0; c < off; ++c) t[p][c] += t[p][c + off];
  return t[0][0] + t[1][0];
}

// t32_partial for a runtime M (wave-uniform): bw / 64 of the call, 1 .. min(8, K), a power of two.
template <int K>
__device__ __forceinline__ float t32_partial_m(const float (*v)[8], int m) {
  if constexpr (K >= 8)
    if (m >= 8) return t32_partial<K, 8>(v);
  if constexpr (K >= 4)
    if (m >= 4) return t32_partial<K, 4>(v);
  if constexpr (K >= 2)
    if (m >= 2) return t32_partial<K, 2>(v);
  return t32_partial<K, 1>(v);
}

// ---------------------------------------------------------------- device: per-head q/k RMSNorm + RoPE
// The arithmetic of the fused q/k norm (qk_norm_rope_kv.hip) on the 8 + 8 elements one lane holds of a head row:
// x1 = elements [e, e+8) of the first half, x2 = the same offsets of the second half (RoPE pairs x1[i], x2[i]).
// Shared with the decode attention that applies it to its query rows, so both give the same bits.

// This lane's part of the sum of squares of one half, in torch's order for a row of D elements: D >= 128 -- ATen
// threads of one 4-element vector each, the lane's two adjacent ones added (the first tree level); D = 64 -- one
// element per thread, the tree's first three levels over the lane's 8 elements. The D/16 lanes of a row then add
// these parts with group_sum<D/16> for each half, and the two halves' sums are the tree's last level.
template <int D>
__device__ __forceinline__ float half_sumsq8(const float* x) {
  if constexpr (D >= 128) {
    return sumsq4(x) + sumsq4(x + 4);
  } else {
    const float p0 = x[0] * x[0] + x[1] * x[1], p1 = x[2] * x[2] + x[3] * x[3];
    const float p2 = x[4] * x[4] + x[5] * x[5], p3 = x[6] * x[6] + x[7] * x[7];
    return (p0 + p1) + (p2 + p3);
  }
}

// n = bf16(bf16(x * rstd) * w), then y1 = bf16(n1 cos - n2 sin), y2 = bf16(n2 cos + n1 sin), every product rounded
// on its own (w: the weights at the same offsets, c / s: cos and sin of the lane's 8 frequencies); elements 2j and
// 2j+1 of each half share one packed bf16 conversion per rounding step.
__device__ __forceinline__ void norm_rope16(const float* x1, const float* x2, float rstd, const u32x4& wa,
                                            const u32x4& wb, const float* c, const float* s, u32x4& oa, u32x4& ob) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t n1 = pack_bf16x2(x1[2 * j] * rstd, x1[2 * j + 1] * rstd);  // bf16(x * rstd)
    const uint32_t n2 = pack_bf16x2(x2[2 * j] * rstd, x2[2 * j + 1] * rstd);
    const uint32_t m1 = pack_bf16x2(bf16_lo(n1) * bf16_lo(wa[j]), bf16_hi(n1) * bf16_hi(wa[j]));  // bf16(n * w)
    const uint32_t m2 = pack_bf16x2(bf16_lo(n2) * bf16_lo(wb[j]), bf16_hi(n2) * bf16_hi(wb[j]));
    const float a0 = bf16_lo(m1), a1 = bf16_hi(m1), b0 = bf16_lo(m2), b1 = bf16_hi(m2);
    const int i0 = 2 * j, i1 = 2 * j + 1;
    const float p0 = a0 * c[i0], q0 = b0 * s[i0], r0 = b0 * c[i0], u0 = a0 * s[i0];
    const float p1 = a1 * c[i1], q1 = b1 * s[i1], r1 = b1 * c[i1], u1 = a1 * s[i1];
    oa[j] = pack_bf16x2(p0 - q0, p1 - q1);
    ob[j] = pack_bf16x2(r0 + u0, r1 + u1);
  }
}

// ---------------------------------------------------------------- device: merging split attention records
// Element d of row r of one (sequence, kv head) from its context splits' records (fp32 max, sum, two more, O[D] ...
// at rec0 + s * step for split s, the (max, sum) pair first): O = sum_s O_s 2^(m_s - M) / sum_s l_s 2^(m_s - M),
// M = max_s m_s, merged in split order; 0 for a row no split saw (M = -inf). Up to 8 splits' loads issue at once.
// DEVICE_SCOPE: the records were written by other blocks of the running kernel (possibly on other XCDs, whose L2s
// are not coherent with this one): read with device-scope loads (sc1), which do not return this XCD's L2 copy.
template <bool DEVICE_SCOPE = false>
__device__ __forceinline__ float merge_splits(const float* rec0, int64_t step, int splits, int d_off) {
  auto ld = [](const float* p) -> float {
    if constexpr (DEVICE_SCOPE)
      return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
      return *p;
  };
  float num = 0.0f, den = 0.0f;
  if (splits <= 4) {
    float m[4], l[4], o[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      m[u] = -INFINITY, l[u] = o[u] = 0.0f;
      if (u < splits) {
        m[u] = ld(rec0 + u * step);
        l[u] = ld(rec0 + u * step + 1);
        o[u] = ld(rec0 + u * step + d_off);
      }
    }
    float M = -INFINITY;
#pragma unroll
    for (int u = 0; u < 4; ++u) M = fmaxf(M, m[u]);
    if (M != -INFINITY) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        if (u >= splits) break;
        const float f = exp2f(m[u] - M);
        num = __builtin_fmaf(o[u], f, num);
        den = __builtin_fmaf(l[u], f, den);
      }
    }
  } else {  // groups of 8 splits' loads at once (the max is exact in any order; the sums stay in split order)
    constexpr int kG = 8;
    float M = -INFINITY;
    for (int s0 = 0; s0 < splits; s0 += kG) {
      float m[kG];
#pragma unroll
      for (int u = 0; u < kG; ++u) m[u] = s0 + u < splits ? ld(rec0 + (s0 + u) * step) : -INFINITY;
#pragma unroll
      for (int u = 0; u < kG; ++u) M = fmaxf(M, m[u]);
    }
    if (M != -INFINITY) {
      for (int s0 = 0; s0 < splits; s0 += kG) {
        float m[kG], l[kG], o[kG];
#pragma unroll
        for (int u = 0; u < kG; ++u) {
          m[u] = -INFINITY, l[u] = o[u] = 0.0f;
          if (s0 + u < splits) {
            m[u] = ld(rec0 + (s0 + u) * step);
            l[u] = ld(rec0 + (s0 + u) * step + 1);
            o[u] = ld(rec0 + (s0 + u) * step + d_off);
          }
        }
#pragma unroll
        for (int u = 0; u < kG; ++u) {
          if (s0 + u >= splits) break;
          const float f = exp2f(m[u] - M);
          num = __builtin_fmaf(o[u], f, num);
          den = __builtin_fmaf(l[u], f, den);
        }
      }
    }
  }
  return den > 0.0f ? num / den : 0.0f;
}

// ---------------------------------------------------------------- device: reductions

// Sum over aligned groups of LANES consecutive lanes of a wave64 (LANES a power of two, 1..64). Every lane of a
// group gets the same (bitwise) result. Groups of up to 16 use DPP (quad_perm, row_half_mirror, row_mirror),
// wider groups finish with ds_swizzle / bpermute shuffles.
template <int LANES>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(LANES >= 1 && LANES <= 64 && (LANES & (LANES - 1)) == 0, "LANES must be a power of two <= 64");
  if constexpr (LANES >= 2) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
  if constexpr (LANES >= 4) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
  if constexpr (LANES >= 8) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
  if constexpr (LANES >= 16) v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
  if constexpr (LANES >= 32) v += __shfl_xor(v, 16, 64);
  if constexpr (LANES >= 64) v += __shfl_xor(v, 32, 64);
  return v;
}

// Sum of squares of a head row of D elements held as x1 / x2 (8 + 8 elements per lane, D/16 lanes, the fused
// q/k norm's layout) in torch's order: each half's tree over its lanes, then the two halves added.
template <int D>
__device__ __forceinline__ float torch_row_sumsq(const float* x1, const float* x2) {
  return group_sum<D / 16>(half_sumsq8<D>(x1)) + group_sum<D / 16>(half_sumsq8<D>(x2));
}

}  // namespace nvhip
