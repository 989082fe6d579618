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
//   3. updates the row's running max (fp32, base-2 exponent with the scale folded into one FMA; lazy: the
//      reference max moves only when a score exceeds it by more than 8, so p <= 256 and almost no chunk rescales
//      O) and turns the scores into p = 2^(s - max) in the registers they were computed in: lane l's 8 values of
//      row l % 16 are the B operand of the P.V product, as a bf16 head and a bf16 remainder (two MFMAs; p keeps
//      ~17 bits, where flash-attn rounds it to bf16 once);
//   4. stores its 32 V rows (row layout: lane l reads dims 8 (l % 16) .. +8 of token l / 16 of each group of 4
//      tokens) into its own LDS slice and reads them back as the A operand of O^T [16 dims x 16 rows] += V^T P^T
//      (v_mfma_f32_16x16x32_bf16, one per 16 dims) with the gfx950 transpose read ds_read_b64_tr_b16: within a
//      16-lane group, lane i receives element i % 4 of the 8-byte chunks addressed by lanes 4j + i / 4 (j = 0..3),
//      so lanes addressing 4 consecutive V rows x 16 dims hand each lane 4 tokens of one dim.
// Lane l keeps O^T dims 16 t + 4 (l / 16) + r of row l % 16, so the rescale is lane-local and no in-wave sum is
// needed; at the end the 8 waves' (max, sum, O) are merged through LDS in wave order (deterministic), O / sum
// rounded to bf16.
// The block-table entries of the block's token range are loaded once, one per lane, alongside the context length
// and Q.
// Varlen: a paged prefill call (prefill_attention.hip) hands its sequences with few queries (<= 16 / G each, e.g.
// the decode requests of a mixed step) to this kernel, with per-sequence query rows and context lengths from
// cu_seqlens; the prefill kernel's 128-query tiles would spend a whole tile's work per key on them.
// Small batches: with a caller workspace the context of each (sequence, kv head) is split over several blocks
// (whole 256-token rounds) when there are fewer pairs than CUs; each block writes its merged (max, sum, O) record
// and a second kernel merges the records in split order. Without a workspace one block covers the whole context.
// Tokens past the context, blocks outside [0, num_blocks) and rows past a query's causal limit take no part (their
// K/V are not read; p = 0).
#include <algorithm>

#include "common.h"

namespace nvhip {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kChunk = 32;  // tokens per wave step
constexpr int kWaves = 8;  // waves per block (4 for head_dim 256, whose registers need a whole SIMD per wave)
__host__ __device__ constexpr int block_waves(int D) { return D == 256 ? 4 : kWaves; }

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
  int splits;     // context splits per (sequence, kv head): blocks s = 0 .. splits-1 take tokens
  int split_len;  // [s * split_len, (s + 1) * split_len); a multiple of kChunk * kWaves (so of kChunk * waves)
  float* ws;      // splits > 1: [num_seqs, Hkv, splits, RP, 2 + D] fp32 records (max, sum, O) of each block
  // varlen (the short sequences of a paged prefill call, splits = 1): sequence b's queries are rows cu_q[b] ..
  // cu_q[b+1]-1 of q and out and its context is cu_k[b+1] - cu_k[b] keys; a sequence with no queries or more
  // than q_len is left alone (the prefill kernel takes it). Null: q_len queries per sequence, ctx_lens.
  const int32_t* cu_q;
  const int32_t* cu_k;
  // FUSE kernels (q_len 1, D 64 / 128): q, kn, vn are the raw rows of the qkv projection. The kernel applies the
  // per-head RMSNorm + RoPE of qk_norm_rope_kv (common.h arithmetic, the same bits) to its query rows and to
  // sequence b's new key; the block whose token range holds the new token (position ctx - 1) puts the new key and
  // value row into LDS, uses them in place of what its chunk loads read for that token, and writes them into the
  // cache slot slots[b] for the steps after this one.
  const uint16_t* kn;
  const uint16_t* vn;
  int64_t kn_st, vn_st;
  const int64_t* positions;
  const int32_t* slots;
  const uint16_t* q_w;
  const uint16_t* k_w;
  const float* cos_sin;
  int64_t cs_st, max_pos, num_slots;
  float inv_d, eps;
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


template <int D, int RP, bool ALIGNED, bool FUSE = false>
__global__ __launch_bounds__(block_waves(D) * 64) void paged_decode_kernel(const DecodeArgs g) {
  constexpr int NWV = block_waves(D);
  constexpr int KC = D / 32;         // 32-wide dim chunks of a K row (MFMA k steps of Q.K)
  constexpr int LPT = D / 8;         // lanes per V row in the row layout
  constexpr int TPI = 64 / LPT;      // tokens per wave instruction in the row layout
  constexpr int PVI = kChunk / TPI;  // V load instructions per chunk
  constexpr int DT = D / 16;         // 16-dim tiles of O^T
  constexpr int VPW = D + 16;        // LDS row pitch of a V chunk: the 4 rows of a transpose read hit 32 distinct banks
  constexpr int KPW = D + 8;         // LDS row pitch of a K chunk: the 16 rows of a fragment read hit distinct banks
  static_assert(D % 32 == 0 && D <= 256 && RP <= 16, "shape");
  // LDS: each wave's K and V chunks during the loop, the waves' partial O afterwards (same bytes)
  constexpr int VBYTES = NWV * kChunk * (VPW + KPW) * 2, RBYTES = NWV * RP * D * 4;
  __shared__ __attribute__((aligned(16))) unsigned char smem[VBYTES > RBYTES ? VBYTES : RBYTES];
  __shared__ float red_m[NWV][RP], red_l[NWV][RP];
  __shared__ __attribute__((aligned(16))) uint16_t fresh[FUSE ? 2 * D : 8];  // FUSE: the new key and value rows
  bool fresh_here = false;  // FUSE: this block's token range holds the new token (wave-uniform)

  const int split = blockIdx.x % g.splits, pair = blockIdx.x / g.splits;
  const int b = pair / g.Hkv, kvh = pair % g.Hkv;
  const int lane = threadIdx.x % 64, wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  int q0 = b * g.q_len, lq = g.q_len, ctx;  // the sequence's first query row, its queries and context length
  if (g.cu_q != nullptr) {
    q0 = g.cu_q[b];
    lq = g.cu_q[b + 1] - q0;
    if (lq < 1 || lq > g.q_len) return;  // the whole block: b is uniform
    ctx = min(max(g.cu_k[b + 1] - g.cu_k[b], 0), g.max_blocks * g.bs);
  } else {
    ctx = min(max(g.ctx_lens[b], 0), g.max_blocks * g.bs);
  }
  const int rows = g.G * lq;
  const int32_t* bt_row = g.bt + int64_t(b) * g.max_blocks;
  const int tok_begin = split * g.split_len, blk0 = tok_begin / g.bs;
  // issued together: this split's first 64 block-table entries (one per lane) and the Q rows
  const int bt_lane = blk0 + lane < g.max_blocks ? bt_row[blk0 + lane] : -1;

  // Q rows as the MFMA B operand: lane l holds row l % 16, dims 32c + 8 (l / 16) .. +8
  const int qrow = lane % 16, q8 = (lane / 16) * 8;
  bf16x8_t qf[KC];
  int qi = 0;  // query token of row qrow
  if (qrow < rows) {
    qi = qrow / g.G;
    const int hh = qrow % g.G;
    const uint16_t* qp = g.q + int64_t(q0 + qi) * g.q_st + int64_t(kvh * g.G + hh) * g.q_sh + q8;
#pragma unroll
    for (int c = 0; c < KC; ++c) qf[c] = load_bf16x8(qp + 32 * c);
  } else {
#pragma unroll
    for (int c = 0; c < KC; ++c) qf[c] = bf16x8_t{};
  }
  if constexpr (FUSE) {
    static_assert(D == 64 || D == 128, "fused pre-attention: head_dim 64 or 128");
    const int64_t p = g.positions[b];
    const float* cs = g.cos_sin + (p < 0 ? 0 : p >= g.max_pos ? g.max_pos - 1 : p) * g.cs_st;
    // the query rows: lane group q8 / 8 = j0 holds the elements 8 j of the fused norm's lanes j = j0 + 4 u
    // (chunk u of each half), so the sum of squares is rebuilt in that kernel's DPP order: lanes j ^ 1 and j ^ 2
    // are lane groups 16 and 32 apart, and the last (mirror) step adds the two halves' partial sums
    constexpr int HK = KC / 2;
    float x1[HK][8], x2[HK][8], part[HK];
#pragma unroll
    for (int u = 0; u < HK; ++u) {
      unpack8(__builtin_bit_cast(u32x4, qf[u]), x1[u]);
      unpack8(__builtin_bit_cast(u32x4, qf[u + HK]), x2[u]);
      part[u] = row_sumsq16(x1[u], x2[u]);
      part[u] += __shfl_xor(part[u], 16);
      part[u] += __shfl_xor(part[u], 32);
    }
    const float ss = HK == 1 ? part[0] : part[0] + part[HK - 1];
    const float rstd = 1.0f / sqrtf(ss * g.inv_d + g.eps);
#pragma unroll
    for (int u = 0; u < HK; ++u) {
      const int e = 32 * u + q8;
      const u32x4 wa = *reinterpret_cast<const u32x4*>(g.q_w + e), wb = *reinterpret_cast<const u32x4*>(g.q_w + D / 2 + e);
      float c[8], s[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) c[i] = cs[e + i], s[i] = cs[D / 2 + e + i];
      u32x4 oa, ob;
      norm_rope16(x1[u], x2[u], rstd, wa, wb, c, s, oa, ob);
      qf[u] = qrow < rows ? __builtin_bit_cast(bf16x8_t, oa) : bf16x8_t{};
      qf[u + HK] = qrow < rows ? __builtin_bit_cast(bf16x8_t, ob) : bf16x8_t{};
    }
    // the new key (lanes 0 .. D/16-1 of wave 0, the fused norm's own lane layout) and value (the next D/16 lanes)
    const int32_t slot = g.slots[b];
    const bool writer = ctx > 0 ? (split * g.split_len <= ctx - 1 && ctx - 1 < split * g.split_len + g.split_len)
                                : split == 0;
    const bool store = writer && slot >= 0 && slot < g.num_slots;
    // the new rows stand in for what the chunk loads read at position ctx - 1 when that is the slot they go to (a
    // decode step); otherwise (inconsistent slot, clamped context) they are written before any wave reads
    if (store && ctx > 0 && ctx == g.ctx_lens[b]) {
      const int t = ctx - 1, blk = bt_row[t / g.bs];
      fresh_here = blk >= 0 && int64_t(blk) * g.bs + t % g.bs == slot;
    }
    u32x4 na = {}, nb = {};  // this lane's 8 + 8 elements of the new key (lanes < D/16) or value row
    constexpr int LN = D / 16;
    const int e = 8 * (lane % LN);
    if (store && wave == 0 && lane < D / 8) {
      if (lane < LN) {
        const uint16_t* kr = g.kn + int64_t(b) * g.kn_st + int64_t(kvh) * D;
        float k1[8], k2[8];
        unpack8(*reinterpret_cast<const u32x4*>(kr + e), k1);
        unpack8(*reinterpret_cast<const u32x4*>(kr + D / 2 + e), k2);
        const float kss = group_sum<LN>(row_sumsq16(k1, k2));
        const float krstd = 1.0f / sqrtf(kss * g.inv_d + g.eps);
        const u32x4 wa = *reinterpret_cast<const u32x4*>(g.k_w + e), wb = *reinterpret_cast<const u32x4*>(g.k_w + D / 2 + e);
        float c[8], s[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) c[i] = cs[e + i], s[i] = cs[D / 2 + e + i];
        norm_rope16(k1, k2, krstd, wa, wb, c, s, na, nb);
      } else {
        const uint16_t* vr = g.vn + int64_t(b) * g.vn_st + int64_t(kvh) * D;
        na = *reinterpret_cast<const u32x4*>(vr + e);
        nb = *reinterpret_cast<const u32x4*>(vr + D / 2 + e);
      }
      uint16_t* f = fresh + (lane < LN ? 0 : D);
      *reinterpret_cast<u32x4*>(f + e) = na;
      *reinterpret_cast<u32x4*>(f + D / 2 + e) = nb;
    }
    uint16_t* dst = const_cast<uint16_t*>(lane < LN ? g.kc : g.vc) + int64_t(slot) * g.Hkv * D + int64_t(kvh) * D + e;
    if (store && !fresh_here && wave == 0 && lane < D / 8) {
      *reinterpret_cast<u32x4*>(dst) = na;
      *reinterpret_cast<u32x4*>(dst + D / 2) = nb;
    }
    __syncthreads();  // the new rows are in LDS (or, without fresh_here, in the cache)
    if (fresh_here && wave == 0 && lane < D / 8) {  // for the next steps; this kernel reads them from LDS
      *reinterpret_cast<u32x4*>(dst) = na;
      *reinterpret_cast<u32x4*>(dst + D / 2) = nb;
    }
  }
  // row qrow sees tokens < row_limit
  const int row_limit = qrow >= rows ? 0 : g.causal ? min(max(ctx - lq + qi + 1, 0), ctx) : ctx;

  float m_run = -INFINITY;  // reference max of row qrow (the same in the 4 lanes of the row)
  float l_run = 0.0f;       // this lane's part of the row sum
  f32x4_t acc[DT];          // O^T dims 16 t + 4 (l / 16) + r of row qrow
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x4_t{0, 0, 0, 0};
  const int dg = lane % LPT, ts = lane / LPT;
  const int h4 = lane / 16, l16 = lane % 16;
  uint16_t* vs = reinterpret_cast<uint16_t*>(smem) + wave * kChunk * (VPW + KPW);  // this wave's V chunk
  uint16_t* ks = vs + kChunk * VPW;                                                 // and K chunk
  const int tok_end = min(ctx, tok_begin + g.split_len);
  const int ch_end = (tok_end + kChunk - 1) / kChunk;

  // A chunk's K and V fragments (registers) and which of its tokens are valid. Every load instruction is issued
  // by all lanes (a lane whose token is not valid reads the first 16 bytes of q) and the loaded values are used as
  // they are -- invalid tokens are masked out of the scores, so their p is 0 -- so no select waits on a load.
  struct Tile {
    bf16x8_t k[PVI], v[PVI];  // row layout: dims 8 (l % LPT) .. +8 of token it * TPI + l / LPT
    uint64_t kvalid[2];       // bit j: token t0 + 16u + j has a valid block (from lanes j = 0..15)
  };
  auto row_of = [&](int t, int64_t base, int t0) -> int64_t {
    if (t >= ctx) return -1;
    if constexpr (ALIGNED) return base < 0 ? -1 : base + int64_t(t - t0) * g.Hkv * D;
    return token_row<D>(g, bt_row, t, kvh);
  };
  auto load_tile = [&](Tile& T, int ch) {
    const int t0 = ch * kChunk;
    int64_t base = -1;  // ALIGNED: row offset of token t0; tokens t0 + j follow at + j * Hkv * D
    if constexpr (ALIGNED) {
      const int idx = t0 / g.bs - blk0;
      const int blk = idx < 64 ? __builtin_amdgcn_readlane(bt_lane, idx) : bt_row[t0 / g.bs];
      base = (blk < 0 || blk >= g.num_blocks) ? -1 : ((int64_t(blk) * g.bs + t0 % g.bs) * g.Hkv + kvh) * D;
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) T.kvalid[u] = __ballot(row_of(t0 + 16 * u + lane % 16, base, t0) >= 0);
#pragma unroll
    for (int it = 0; it < PVI; ++it) {
      const int64_t row = row_of(t0 + it * TPI + ts, base, t0);
      T.k[it] = load_bf16x8(row >= 0 ? g.kc + row + 8 * dg : g.q);
      T.v[it] = load_bf16x8(row >= 0 ? g.vc + row + 8 * dg : g.q);
    }
  };
  constexpr float kLazy = 8.0f;
  auto compute_tile = [&](const Tile& T, int ch) {
    const int t0 = ch * kChunk;
    // the chunk's K and V rows into this wave's LDS slices (full cache lines were read); the K rows come back as
    // the A operand of S^T (lane l: token 16u + l % 16, dims 32c + 8 (l / 16) .. +8)
#pragma unroll
    for (int it = 0; it < PVI; ++it) {
      *reinterpret_cast<bf16x8_t*>(ks + (it * TPI + ts) * KPW + 8 * dg) = T.k[it];
      *reinterpret_cast<bf16x8_t*>(vs + (it * TPI + ts) * VPW + 8 * dg) = T.v[it];
    }
    if constexpr (FUSE) {  // the new token's rows from LDS: its cache slot is written only after this kernel read it
      const int r = ctx - 1 - t0;
      if (fresh_here && r >= 0 && r < kChunk && lane < D / 8) {
        *reinterpret_cast<u32x4*>(ks + r * KPW + 8 * lane) = *reinterpret_cast<const u32x4*>(fresh + 8 * lane);
        *reinterpret_cast<u32x4*>(vs + r * VPW + 8 * lane) = *reinterpret_cast<const u32x4*>(fresh + D + 8 * lane);
      }
    }
    wave_sync();
    // scores: lane holds tokens t0 + 16u + 4 (l / 16) + r of row qrow
    f32x4_t s[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      s[u] = f32x4_t{0, 0, 0, 0};
#pragma unroll
      for (int c = 0; c < KC; ++c)
        s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            *reinterpret_cast<const bf16x8_t*>(ks + (16 * u + l16) * KPW + 32 * c + 8 * h4), qf[c], s[u], 0, 0, 0);
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int j = 4 * h4 + r, t = t0 + 16 * u + j;
        if (!(t < row_limit && ((T.kvalid[u] >> j) & 1))) s[u][r] = -INFINITY;
        tmax = fmaxf(tmax, s[u][r]);
      }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
    tmax = pair32_max(tmax) * g.scale_log2;  // the scale is positive
    const bool move = tmax > m_run + kLazy;  // also true for the first finite max (m_run = -inf)
    if (__ballot(move) != 0) {
      const float alpha = move ? exp2f(m_run - tmax) : 1.0f;  // 0 from m_run = -inf
      if (move) m_run = tmax;
      l_run *= alpha;
#pragma unroll
      for (int t = 0; t < DT; ++t) acc[t] *= alpha;
    }
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;
    // P^T as the B operand: k slots 0..3 = tokens 4 h4 + r, 4..7 = tokens 16 + 4 h4 + r, column = row qrow
    float p[8];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        p[4 * u + r] = exp2f(__builtin_fmaf(s[u][r], g.scale_log2, -m_use));
        l_run += p[4 * u + r];
      }
    // p = head + remainder, both bf16: two MFMAs per dim tile keep p to ~2^-17 relative (fp32-like; flash-attn
    // rounds p to bf16 once)
    const u32x4 phi = pack8(p);
    float ph[8];
    unpack8(phi, ph);
#pragma unroll
    for (int e = 0; e < 8; ++e) ph[e] = p[e] - ph[e];
    const bf16x8_t pk = __builtin_bit_cast(bf16x8_t, phi), pr = __builtin_bit_cast(bf16x8_t, pack8(ph));
    // V^T fragments with the transpose read: the lanes of group h4 address rows 4 h4 + i / 4 (slots 0..3) and
    // 16 + 4 h4 + i / 4 (slots 4..7), dims 16 t + 4 (i % 4)
    const uint16_t* v0 = vs + (4 * h4 + l16 / 4) * VPW + 4 * (l16 % 4);
    const uint16_t* v1 = v0 + 16 * VPW;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const u32x2 lo = lds_read_tr16(v0 + 16 * t), hi = lds_read_tr16(v1 + 16 * t);
      const bf16x8_t va = __builtin_bit_cast(bf16x8_t, u32x4{lo[0], lo[1], hi[0], hi[1]});
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pk, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pr, acc[t], 0, 0, 0);
    }
    wave_sync();  // the next chunk rewrites the slice
  };

  // The wave's chunks are first, first + 8, ... (issuing two chunks' loads before computing them, or prefetching
  // the next chunk during the current one, measured no faster: a read-only kernel with this access pattern and
  // no compute takes ~35 us where this one takes ~43 us for 163 MB of K/V).
  for (int ch = tok_begin / kChunk + wave; ch < ch_end; ch += NWV) {
    Tile A;
    load_tile(A, ch);
    compute_tile(A, ch);
  }

  // row sums over the 4 lane groups of the row; each lane's O^T values are its own (no in-wave sum)
  l_run += __shfl_xor(l_run, 16);
  l_run = pair32_sum(l_run);
  __syncthreads();  // every wave is done with its V slice: the partial O reuse those bytes
  float (*red_acc)[RP][D] = reinterpret_cast<float (*)[RP][D]>(smem);
  if (qrow < RP) {
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) red_acc[wave][qrow][16 * t + 4 * h4 + r] = acc[t][r];
    if (h4 == 0) {
      red_m[wave][qrow] = m_run;
      red_l[wave][qrow] = l_run;
    }
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < rows * D; idx += NWV * 64) {
    const int r = idx / D, d = idx % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NWV; ++w) M = fmaxf(M, red_m[w][r]);
    float num = 0.0f, den = 0.0f;
    if (M != -INFINITY) {
#pragma unroll
      for (int w = 0; w < NWV; ++w) {
        const float f = exp2f(red_m[w][r] - M);
        num = __builtin_fmaf(red_acc[w][r][d], f, num);
        den = __builtin_fmaf(red_l[w][r], f, den);
      }
    }
    if (g.splits > 1) {  // this block's record; merged by paged_decode_combine
      float* rec = g.ws + ((int64_t(pair) * g.splits + split) * RP + r) * (2 + D);
      if (d == 0) {
        rec[0] = M;
        rec[1] = den;
      }
      rec[2 + d] = num;
      continue;
    }
    const float o = den > 0.0f ? num / den : 0.0f;
    const int i = r / g.G, hh = r % g.G;
    g.out[int64_t(q0 + i) * g.o_st + int64_t(kvh * g.G + hh) * g.o_sh + d] = f32_to_bf16(o);
  }
}

// Merges the split records of one (sequence, kv head) in split order: O = sum_s O_s 2^(m_s - M) /
// sum_s l_s 2^(m_s - M), M = max_s m_s; a row no split saw (M = -inf) is zero.
template <int D, int RP>
__global__ __launch_bounds__(256) void paged_decode_combine(const DecodeArgs g) {
  const int pair = blockIdx.x, b = pair / g.Hkv, kvh = pair % g.Hkv;
  int q0 = b * g.q_len, lq = g.q_len;  // as in paged_decode_kernel
  if (g.cu_q != nullptr) {
    q0 = g.cu_q[b];
    lq = g.cu_q[b + 1] - q0;
    if (lq < 1 || lq > g.q_len) return;  // no records: the kernel's blocks left this sequence alone
  }
  const int rows = g.G * lq;
  for (int idx = threadIdx.x; idx < rows * D; idx += 256) {
    const int r = idx / D, d = idx % D;
    const float* rec = g.ws + (int64_t(pair) * g.splits * RP + r) * (2 + D);
    const float o = merge_splits(rec, int64_t(RP) * (2 + D), g.splits, 2 + d);
    const int i = r / g.G, hh = r % g.G;
    g.out[int64_t(q0 + i) * g.o_st + int64_t(kvh * g.G + hh) * g.o_sh + d] = f32_to_bf16(o);
  }
}

template <int D, int RP, bool FUSE = false>
int launch_decode(const DecodeArgs& g, int64_t num_seqs, hipStream_t s, bool merge = true) {
  const dim3 grid(unsigned(num_seqs * g.Hkv * g.splits)), block(block_waves(D) * 64);
  if (g.bs % kChunk == 0) hipLaunchKernelGGL((paged_decode_kernel<D, RP, true, FUSE>), grid, block, 0, s, g);
  else hipLaunchKernelGGL((paged_decode_kernel<D, RP, false, FUSE>), grid, block, 0, s, g);
  if (int rc = check_launch("paged_decode_attention")) return rc;
  if (g.splits == 1 || !merge) return NVHIP_OK;
  hipLaunchKernelGGL((paged_decode_combine<D, RP>), dim3(unsigned(num_seqs * g.Hkv)), dim3(256), 0, s, g);
  return check_launch("paged_decode_attention (combine)");
}

template <int D>
int launch_decode_rows(const DecodeArgs& g, int64_t num_seqs, int rows, hipStream_t s, bool merge = true) {
  if (rows <= 1) return launch_decode<D, 1>(g, num_seqs, s, merge);
  if (rows <= 2) return launch_decode<D, 2>(g, num_seqs, s, merge);
  if (rows <= 4) return launch_decode<D, 4>(g, num_seqs, s, merge);
  if (rows <= 8) return launch_decode<D, 8>(g, num_seqs, s, merge);
  return launch_decode<D, 16>(g, num_seqs, s, merge);
}

int rows_padded(int64_t rows) { return rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : rows <= 8 ? 8 : 16; }

// Context split: only when there are fewer (sequence, kv head) pairs than CUs -- every extra block on a CU pays
// the start-up latency of its first loads again (measured: 1 -> 2 -> 4 splits of a 32-sequence batch took 42 ->
// 50 -> 56 us) -- aiming at ~256 blocks in splits of whole 256-token rounds (32 tokens per wave x 8 waves), the
// longest possible context (max_blocks * block_size) setting the count.
void split_policy(int64_t num_seqs, int64_t Hkv, int64_t max_ctx, int& splits, int& split_len) {
  constexpr int64_t kRound = kChunk * kWaves, kTargetBlocks = 256;
  const int64_t pairs = std::max<int64_t>(1, num_seqs * Hkv);
  const int64_t want = std::max<int64_t>(1, (kTargetBlocks + pairs - 1) / pairs);
  int64_t len = std::max<int64_t>(kRound, (max_ctx + want - 1) / want);
  len = (len + kRound - 1) / kRound * kRound;
  const int64_t n = std::max<int64_t>(1, (max_ctx + len - 1) / len);
  splits = int(std::min<int64_t>(n, 1 << 16));
  split_len = int(std::min<int64_t>(len, INT32_MAX / 2));
}

int64_t workspace_bytes(int64_t num_seqs, int64_t q_len, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_ctx) {
  int splits, split_len;
  split_policy(num_seqs, Hkv, max_ctx, splits, split_len);
  if (splits <= 1) return 0;
  return num_seqs * Hkv * splits * rows_padded((Hq / Hkv) * q_len) * (2 + D) * int64_t(sizeof(float));
}

}  // namespace

int64_t paged_decode_varlen_workspace(int64_t num_seqs, int64_t qmax, int64_t Hq, int64_t Hkv, int64_t D) {
  // split_policy makes at most ceil(256 / pairs) splits, whatever the context length
  const int64_t pairs = std::max<int64_t>(1, num_seqs * Hkv), most = (256 + pairs - 1) / pairs;
  if (most <= 1 || qmax < 1 || Hkv < 1) return 0;
  return num_seqs * Hkv * most * rows_padded((Hq / Hkv) * qmax) * (2 + D) * int64_t(sizeof(float));
}

int paged_decode_varlen(uint16_t* out, const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                        const int32_t* block_table, const int32_t* cu_q, const int32_t* cu_k, int num_seqs, int qmax,
                        int Hq, int Hkv, int D, int block_size, int num_blocks, int max_blocks, int64_t q_st,
                        int64_t q_sh, int64_t o_st, int64_t o_sh, float scale, int causal, float* ws, int64_t ws_bytes,
                        DecodeSplits* defer_merge, hipStream_t s) {
  const int G = Hq / Hkv, rows = G * qmax;
  if (qmax < 1 || rows > 16 || (D != 64 && D != 128 && D != 256) ||
      int64_t(num_seqs) * Hkv > INT32_MAX || int64_t(max_blocks) * block_size > INT32_MAX)
    return invalid("prefill_attention: short-sequence path: bad sizes");
  DecodeArgs g{out, q, k_cache, v_cache, block_table, nullptr, qmax, Hkv, G, block_size, num_blocks, max_blocks,
               q_st, q_sh, o_st, o_sh, scale * 1.4426950408889634f, causal ? 1 : 0, 1,
               max_blocks * block_size, nullptr, cu_q, cu_k};
  // the decode entry point's key splits (same policy, so its one-query rows stay bitwise those of a decode call)
  if (ws != nullptr && ws_bytes > 0) {
    int splits, split_len;
    split_policy(num_seqs, Hkv, int64_t(max_blocks) * block_size, splits, split_len);
    const int64_t need = int64_t(num_seqs) * Hkv * splits * rows_padded(rows) * (2 + D) * int64_t(sizeof(float));
    if (splits > 1 && ws_bytes >= need && int64_t(num_seqs) * Hkv * splits <= INT32_MAX) {
      g.splits = splits;
      g.split_len = split_len;
      g.ws = ws;
    }
  }
  const bool merge = defer_merge == nullptr || g.splits == 1;
  if (!merge) *defer_merge = DecodeSplits{g.splits, rows_padded(rows), g.ws};
  switch (D) {
    case 64: return launch_decode_rows<64>(g, num_seqs, rows, s, merge);
    case 128: return launch_decode_rows<128>(g, num_seqs, rows, s, merge);
    default: return launch_decode_rows<256>(g, num_seqs, rows, s, merge);
  }
}

}  // namespace nvhip

extern "C" int64_t nvhip_paged_decode_attention_workspace_size(int64_t num_seqs, int64_t q_len, int64_t Hq,
                                                               int64_t Hkv, int64_t D, int64_t block_size,
                                                               int64_t max_blocks) {
  if (num_seqs <= 0 || q_len < 1 || Hq < 1 || Hkv < 1 || Hq % Hkv != 0 || D < 1 || block_size < 1 || max_blocks < 0)
    return 0;
  return nvhip::workspace_bytes(num_seqs, q_len, Hq, Hkv, D, max_blocks * block_size);
}

extern "C" int nvhip_paged_decode_attention_bf16(void* out, const void* q, const void* k_cache, const void* v_cache,
                                                 const int32_t* block_table, const int32_t* context_lens,
                                                 int64_t num_seqs, int64_t q_len, int64_t Hq, int64_t Hkv, int64_t D,
                                                 int64_t block_size, int64_t num_blocks, int64_t max_blocks,
                                                 int64_t q_stride_token, int64_t q_stride_head,
                                                 int64_t out_stride_token, int64_t out_stride_head, float scale,
                                                 int causal, void* workspace, int64_t workspace_size,
                                                 void* stream) {
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
               causal ? 1 : 0,
               1,
               int(max_blocks * block_size),
               nullptr,
               nullptr,
               nullptr};
  // split the context over several blocks when the caller gave a large enough workspace
  const int64_t need = workspace_bytes(num_seqs, q_len, Hq, Hkv, D, max_blocks * block_size);
  if (need > 0 && workspace && workspace_size >= need) {
    if (reinterpret_cast<uintptr_t>(workspace) % alignof(float) != 0)
      return invalid("paged_decode_attention: workspace must be 4-byte aligned");
    split_policy(num_seqs, Hkv, max_blocks * block_size, g.splits, g.split_len);
    g.ws = static_cast<float*>(workspace);
  }
  if (num_seqs * Hkv * g.splits > INT32_MAX) return invalid("paged_decode_attention: size too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (D) {
    case 64: return launch_decode_rows<64>(g, num_seqs, int(rows), s);
    case 128: return launch_decode_rows<128>(g, num_seqs, int(rows), s);
    default: return launch_decode_rows<256>(g, num_seqs, int(rows), s);
  }
}

extern "C" int nvhip_qk_norm_rope_kv_decode_attention_bf16(
    void* out, const void* q, const void* k, const void* v, int64_t q_stride, int64_t k_stride, int64_t v_stride,
    const int64_t* positions, const int32_t* slot_mapping, const void* q_weight, const void* k_weight,
    const float* cos_sin, int64_t cos_sin_stride, int64_t max_pos, float eps, void* k_cache, void* v_cache,
    const int32_t* block_table, const int32_t* context_lens, int64_t num_seqs, int64_t Hq, int64_t Hkv, int64_t D,
    int64_t block_size, int64_t num_blocks, int64_t max_blocks, int64_t out_stride_token, int64_t out_stride_head,
    float scale, void* workspace, int64_t workspace_size, void* stream) {
  using namespace nvhip;
  clear_error();
  if (num_seqs < 0 || Hq < 1 || Hkv < 1 || block_size < 1 || num_blocks < 1 || max_blocks < 0)
    return invalid("qk_norm_rope_kv_decode_attention: bad size");
  if (Hq % Hkv != 0 || Hq / Hkv > 16)
    return invalid("qk_norm_rope_kv_decode_attention: Hq must be a multiple of Hkv, at most 16 times it");
  if (D != 64 && D != 128) return invalid("qk_norm_rope_kv_decode_attention: head_dim must be 64 or 128");
  if (q_stride < Hq * D || k_stride < Hkv * D || v_stride < Hkv * D || q_stride % 8 || k_stride % 8 || v_stride % 8)
    return invalid("qk_norm_rope_kv_decode_attention: bad q / k / v token strides");
  if (out_stride_head < D || out_stride_token < Hq * out_stride_head)
    return invalid("qk_norm_rope_kv_decode_attention: bad out strides");
  if (max_pos <= 0 || cos_sin_stride < D || cos_sin_stride % 4)
    return invalid("qk_norm_rope_kv_decode_attention: bad cos_sin cache shape");
  if (num_seqs == 0) return NVHIP_OK;
  if (!out || !q || !k || !v || !positions || !slot_mapping || !q_weight || !k_weight || !cos_sin || !k_cache ||
      !v_cache || !block_table || !context_lens)
    return invalid("qk_norm_rope_kv_decode_attention: null pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(q_weight) || !aligned16(k_weight) ||
      !aligned16(cos_sin) || !aligned16(k_cache) || !aligned16(v_cache))
    return invalid("qk_norm_rope_kv_decode_attention: q, k, v, weights, cos_sin and caches must be 16-byte aligned");
  if (num_seqs * Hkv > INT32_MAX || max_blocks * block_size > INT32_MAX || num_blocks > INT32_MAX)
    return invalid("qk_norm_rope_kv_decode_attention: size too large");
  DecodeArgs g{};
  g.out = static_cast<uint16_t*>(out);
  g.q = static_cast<const uint16_t*>(q);
  g.kc = static_cast<const uint16_t*>(k_cache);
  g.vc = static_cast<const uint16_t*>(v_cache);
  g.bt = block_table;
  g.ctx_lens = context_lens;
  g.q_len = 1, g.Hkv = int(Hkv), g.G = int(Hq / Hkv), g.bs = int(block_size), g.num_blocks = int(num_blocks);
  g.max_blocks = int(max_blocks);
  g.q_st = q_stride, g.q_sh = D, g.o_st = out_stride_token, g.o_sh = out_stride_head;
  g.scale_log2 = scale * 1.4426950408889634f;
  g.causal = 1;
  g.splits = 1, g.split_len = int(max_blocks * block_size), g.ws = nullptr;
  g.kn = static_cast<const uint16_t*>(k), g.vn = static_cast<const uint16_t*>(v);
  g.kn_st = k_stride, g.vn_st = v_stride;
  g.positions = positions, g.slots = slot_mapping;
  g.q_w = static_cast<const uint16_t*>(q_weight), g.k_w = static_cast<const uint16_t*>(k_weight);
  g.cos_sin = cos_sin, g.cs_st = cos_sin_stride, g.max_pos = max_pos, g.num_slots = num_blocks * block_size;
  g.inv_d = 1.0f / float(D), g.eps = eps;
  const int64_t need = workspace_bytes(num_seqs, 1, Hq, Hkv, D, max_blocks * block_size);
  if (need > 0 && workspace && workspace_size >= need) {
    if (reinterpret_cast<uintptr_t>(workspace) % alignof(float) != 0)
      return invalid("qk_norm_rope_kv_decode_attention: workspace must be 4-byte aligned");
    split_policy(num_seqs, Hkv, max_blocks * block_size, g.splits, g.split_len);
    g.ws = static_cast<float*>(workspace);
  }
  if (num_seqs * Hkv * g.splits > INT32_MAX) return invalid("qk_norm_rope_kv_decode_attention: size too large");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rows = g.G;
  if (D == 64) {
    if (rows <= 1) return launch_decode<64, 1, true>(g, num_seqs, s);
    if (rows <= 2) return launch_decode<64, 2, true>(g, num_seqs, s);
    if (rows <= 4) return launch_decode<64, 4, true>(g, num_seqs, s);
    if (rows <= 8) return launch_decode<64, 8, true>(g, num_seqs, s);
    return launch_decode<64, 16, true>(g, num_seqs, s);
  }
  if (rows <= 1) return launch_decode<128, 1, true>(g, num_seqs, s);
  if (rows <= 2) return launch_decode<128, 2, true>(g, num_seqs, s);
  if (rows <= 4) return launch_decode<128, 4, true>(g, num_seqs, s);
  if (rows <= 8) return launch_decode<128, 8, true>(g, num_seqs, s);
  return launch_decode<128, 16, true>(g, num_seqs, s);
}
