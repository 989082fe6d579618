// Paged decode attention for gfx950: the step after the fused q/k-norm + RoPE + KV-write kernel.
//
// Replaces flash_attn_with_kvcache(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale, causal=True) as
// nano-vllm calls it (layers/attention.py:80-90): q [num_seqs * q_len, Hq, D] (q_len query tokens per sequence),
// caches [num_blocks, block_size, Hkv, D] (model_runner.py:262-267), block_table [num_seqs, max_blocks] int32 padded
// with -1, cache_seqlens [num_seqs] int32. Query i of a sequence with context length L sees cache tokens
// 0 .. L - q_len + i (the causal mask is aligned to the bottom right); without causal every query sees all L.
// A sequence with L = 0 (batch padding) gets a zero output.
//
// One block per (sequence, kv head), 8 waves; the G = Hq / Hkv query heads of the kv head times the q_len query
// tokens form the R <= 16 "rows" of the block (row = i * G + h). The context is cut into 32-token chunks dealt
// round-robin to the waves. Per chunk a wave
//   1. loads the 32 K rows (MFMA A operand: lane l reads token l % 16 of a 16-token tile, dims 32c + 8 (l / 16) ..
//      +8, straight from the paged cache) and the 32 V rows (lane l reads dims 8 (l % 16) .. +8 of token l / 16 of
//      each group of 4 tokens);
//   2. computes S^T [16 tokens x 16 rows] = K Q^T per tile with v_mfma_f32_16x16x32_bf16 (Q rows as the B operand,
//      held in registers; rows >= R are zero), so lane l holds tokens 4 (l / 16) + r of row l % 16;
//   3. updates the row's running max (fp32, base-2 exponent with the scale folded in), turns the scores into
//      p = 2^(s - max) and hands p and the rescale factor of each row to the other lanes through the wave's own LDS
//      slice;
//   4. accumulates O[row][dims] = O * rescale + sum p * V in fp32 with the lane-owns-8-dims layout of step 1.
// At the end the 4 token groups of a wave are summed with lane shuffles and the 8 waves' (max, sum, O) are merged
// through LDS in wave order (deterministic), O / sum rounded to bf16.
// Tokens past the context, blocks outside [0, num_blocks) and rows past a query's causal limit take no part (their
// K/V are not read; p = 0).
#include "common.h"

namespace nvhip {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kChunk = 32;  // tokens per wave step
constexpr int kWaves = 8;

struct DecodeArgs {
  uint16_t* out;
  const uint16_t* q;
  const uint16_t* kc;
  const uint16_t* vc;
  const int32_t* bt;
  const int32_t* ctx_lens;
  int q_len, Hkv, G, bs, num_blocks, max_blocks;
  int64_t q_st, q_sh, o_st, o_sh;
  float scale_log2;  // softmax scale * log2(e)
  int causal;
};

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ bf16x8_t load_bf16x8(const uint16_t* p) { return *reinterpret_cast<const bf16x8_t*>(p); }

// Element offset of token t's row for this kv head in the caches, or -1 if its block is not a valid block.
// ALIGNED: block_size is a multiple of the chunk, so every token of a chunk lies in the block of the chunk start.
template <int D>
__device__ __forceinline__ int64_t token_row(const DecodeArgs& g, const int32_t* bt_row, int t, int kvh) {
  const int blk = bt_row[t / g.bs];
  if (blk < 0 || blk >= g.num_blocks) return -1;
  return ((int64_t(blk) * g.bs + t % g.bs) * g.Hkv + kvh) * D;
}

template <int D, int RP, bool ALIGNED>
__global__ __launch_bounds__(kWaves * 64) void paged_decode_kernel(const DecodeArgs g) {
  constexpr int KC = D / 32;         // 32-wide dim chunks of a K row (MFMA k steps)
  constexpr int LPT = D / 8;         // lanes per V row in the PV layout
  constexpr int TPI = 64 / LPT;      // tokens per wave instruction in the PV layout
  constexpr int PVI = kChunk / TPI;  // PV steps per chunk
  static_assert(D % 32 == 0 && D <= 256 && RP <= 16, "shape");
  __shared__ float pbuf[kWaves][kChunk][RP];
  __shared__ float cbuf[kWaves][RP];
  __shared__ float red_acc[kWaves][RP][D];
  __shared__ float red_m[kWaves][RP], red_l[kWaves][RP];

  const int b = blockIdx.x / g.Hkv, kvh = blockIdx.x % g.Hkv;
  const int lane = threadIdx.x % 64, wave = threadIdx.x / 64;
  const int rows = g.G * g.q_len;
  const int ctx = min(max(g.ctx_lens[b], 0), g.max_blocks * g.bs);
  const int32_t* bt_row = g.bt + int64_t(b) * g.max_blocks;

  // Q rows as the MFMA B operand: lane l holds row l % 16, dims 32c + 8 (l / 16) .. +8
  const int qrow = lane % 16, q8 = (lane / 16) * 8;
  bf16x8_t qf[KC];
  int row_limit = 0;  // row qrow sees tokens < row_limit
  if (qrow < rows) {
    const int i = qrow / g.G, hh = qrow % g.G;
    const uint16_t* qp = g.q + int64_t(b * g.q_len + i) * g.q_st + int64_t(kvh * g.G + hh) * g.q_sh + q8;
#pragma unroll
    for (int c = 0; c < KC; ++c) qf[c] = load_bf16x8(qp + 32 * c);
    row_limit = g.causal ? min(max(ctx - g.q_len + i + 1, 0), ctx) : ctx;
  } else {
#pragma unroll
    for (int c = 0; c < KC; ++c) qf[c] = bf16x8_t{};
  }

  float m_run = -INFINITY;  // running max of row qrow (the same in the 4 lanes of the row)
  float l_run = 0.0f;       // this lane's part of the row sum
  float acc[RP][8];
#pragma unroll
  for (int r = 0; r < RP; ++r)
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[r][e] = 0.0f;
  const int dg = lane % LPT, ts = lane / LPT;
  const int nchunks = (ctx + kChunk - 1) / kChunk;

  for (int ch = wave; ch < nchunks; ch += kWaves) {
    const int t0 = ch * kChunk;
    int64_t base = -1;  // ALIGNED: row offset of token t0; tokens t0 + j follow at + j * Hkv * D
    if constexpr (ALIGNED) base = token_row<D>(g, bt_row, t0, kvh);
    auto row_of = [&](int t) -> int64_t {
      if (t >= ctx) return -1;
      if constexpr (ALIGNED) return base < 0 ? -1 : base + int64_t(t - t0) * g.Hkv * D;
      return token_row<D>(g, bt_row, t, kvh);
    };
    bf16x8_t kf[2][KC], vf[PVI];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t row = row_of(t0 + 16 * u + lane % 16);
#pragma unroll
      for (int c = 0; c < KC; ++c) kf[u][c] = row >= 0 ? load_bf16x8(g.kc + row + 32 * c + q8) : bf16x8_t{};
    }
#pragma unroll
    for (int it = 0; it < PVI; ++it) {
      const int64_t row = row_of(t0 + it * TPI + ts);
      vf[it] = row >= 0 ? load_bf16x8(g.vc + row + 8 * dg) : bf16x8_t{};
    }
    // scores: lane holds tokens t0 + 16u + 4 (l / 16) + r of row qrow
    f32x4_t s[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      s[u] = f32x4_t{0, 0, 0, 0};
#pragma unroll
      for (int c = 0; c < KC; ++c) s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[u][c], qf[c], s[u], 0, 0, 0);
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = t0 + 16 * u + 4 * (lane / 16) + r;
        const float v = t < row_limit ? s[u][r] * g.scale_log2 : -INFINITY;
        s[u][r] = v;
        tmax = fmaxf(tmax, v);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float resc = exp2f(m_run - m_use);
    m_run = m_new;
    l_run *= resc;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float p = exp2f(s[u][r] - m_use);
        l_run += p;
        if (qrow < RP) pbuf[wave][16 * u + 4 * (lane / 16) + r][qrow] = p;
      }
    if (lane < RP) cbuf[wave][lane] = resc;
    wave_sync();
    float cr[RP];
#pragma unroll
    for (int r = 0; r < RP; ++r) cr[r] = cbuf[wave][r];
#pragma unroll
    for (int r = 0; r < RP; ++r)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[r][e] *= cr[r];
#pragma unroll
    for (int it = 0; it < PVI; ++it) {
      const int tok = it * TPI + ts;
      float pv[RP];
#pragma unroll
      for (int r = 0; r < RP; ++r) pv[r] = pbuf[wave][tok][r];
      float vv[8];
      unpack8(*reinterpret_cast<const u32x4*>(&vf[it]), vv);
#pragma unroll
      for (int r = 0; r < RP; ++r)
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[r][e] = __builtin_fmaf(pv[r], vv[e], acc[r][e]);
    }
    wave_sync();  // pbuf / cbuf are rewritten by the next chunk
  }

  // sum the TPI token groups (lanes dg + LPT * ts) and the row sums (lanes qrow + 16 * j)
#pragma unroll
  for (int off = LPT; off < 64; off *= 2)
#pragma unroll
    for (int r = 0; r < RP; ++r)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[r][e] += __shfl_xor(acc[r][e], off);
  l_run += __shfl_xor(l_run, 16);
  l_run += __shfl_xor(l_run, 32);
  if (ts == 0) {
#pragma unroll
    for (int r = 0; r < RP; ++r)
#pragma unroll
      for (int e = 0; e < 8; ++e) red_acc[wave][r][8 * dg + e] = acc[r][e];
  }
  if (lane < RP) {
    red_m[wave][lane] = m_run;
    red_l[wave][lane] = l_run;
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < rows * D; idx += kWaves * 64) {
    const int r = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, red_m[w][r]);
    float num = 0.0f, den = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        const float f = exp2f(red_m[w][r] - M);
        num = __builtin_fmaf(red_acc[w][r][d], f, num);
        den = __builtin_fmaf(red_l[w][r], f, den);
      }
    }
    const float o = den > 0.0f ? num / den : 0.0f;
    const int i = r / g.G, hh = r % g.G;
    g.out[int64_t(b * g.q_len + i) * g.o_st + int64_t(kvh * g.G + hh) * g.o_sh + d] = f32_to_bf16(o);
  }
}

template <int D, int RP>
int launch_decode(const DecodeArgs& g, int64_t num_seqs, hipStream_t s) {
  const dim3 grid(unsigned(num_seqs * g.Hkv)), block(kWaves * 64);
  if (g.bs % kChunk == 0) hipLaunchKernelGGL((paged_decode_kernel<D, RP, true>), grid, block, 0, s, g);
  else hipLaunchKernelGGL((paged_decode_kernel<D, RP, false>), grid, block, 0, s, g);
  return check_launch("paged_decode_attention");
}

template <int D>
int launch_decode_rows(const DecodeArgs& g, int64_t num_seqs, int rows, hipStream_t s) {
  if (rows <= 1) return launch_decode<D, 1>(g, num_seqs, s);
  if (rows <= 2) return launch_decode<D, 2>(g, num_seqs, s);
  if (rows <= 4) return launch_decode<D, 4>(g, num_seqs, s);
  if (rows <= 8) return launch_decode<D, 8>(g, num_seqs, s);
  if constexpr (D <= 128) return launch_decode<D, 16>(g, num_seqs, s);
  return invalid("paged_decode_attention: at most 8 query rows per kv head with head_dim 256");
}

}  // namespace
}  // namespace nvhip

extern "C" int nvhip_paged_decode_attention_bf16(void* out, const void* q, const void* k_cache, const void* v_cache,
                                                 const int32_t* block_table, const int32_t* context_lens,
                                                 int64_t num_seqs, int64_t q_len, int64_t Hq, int64_t Hkv, int64_t D,
                                                 int64_t block_size, int64_t num_blocks, int64_t max_blocks,
                                                 int64_t q_stride_token, int64_t q_stride_head,
                                                 int64_t out_stride_token, int64_t out_stride_head, float scale,
                                                 int causal, void* stream) {
  using namespace nvhip;
  clear_error();
  if (num_seqs < 0 || q_len < 1 || Hq < 1 || Hkv < 1 || block_size < 1 || num_blocks < 0 || max_blocks < 0)
    return invalid("paged_decode_attention: bad size");
  if (Hq % Hkv != 0) return invalid("paged_decode_attention: Hq must be a multiple of Hkv");
  if (D != 64 && D != 128 && D != 256) return invalid("paged_decode_attention: head_dim must be 64, 128 or 256");
  const int64_t rows = (Hq / Hkv) * q_len;
  if (rows > 16) return invalid("paged_decode_attention: (Hq / Hkv) * q_len must be <= 16");
  if (q_stride_head < D || q_stride_token < Hq * q_stride_head || out_stride_head < D ||
      out_stride_token < Hq * out_stride_head || q_stride_head % 8 != 0 || q_stride_token % 8 != 0)
    return invalid("paged_decode_attention: bad q / out strides (rows of D contiguous, 16-byte aligned)");
  if (num_seqs == 0) return NVHIP_OK;
  if (!out || !q || !block_table || !context_lens || (num_blocks > 0 && (!k_cache || !v_cache)))
    return invalid("paged_decode_attention: null pointer");
  if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache))
    return invalid("paged_decode_attention: q and the caches must be 16-byte aligned");
  if (num_seqs * Hkv > INT32_MAX || num_seqs * q_len > INT32_MAX || max_blocks * block_size > INT32_MAX ||
      num_blocks > INT32_MAX)
    return invalid("paged_decode_attention: size too large");
  DecodeArgs g{static_cast<uint16_t*>(out),
               static_cast<const uint16_t*>(q),
               static_cast<const uint16_t*>(k_cache),
               static_cast<const uint16_t*>(v_cache),
               block_table,
               context_lens,
               int(q_len),
               int(Hkv),
               int(Hq / Hkv),
               int(block_size),
               int(num_blocks),
               int(max_blocks),
               q_stride_token,
               q_stride_head,
               out_stride_token,
               out_stride_head,
               scale * 1.4426950408889634f,
               causal ? 1 : 0};
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (D) {
    case 64: return launch_decode_rows<64>(g, num_seqs, int(rows), s);
    case 128: return launch_decode_rows<128>(g, num_seqs, int(rows), s);
    default: return launch_decode_rows<256>(g, num_seqs, int(rows), s);
  }
}
