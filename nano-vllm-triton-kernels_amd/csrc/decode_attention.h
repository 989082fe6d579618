// The paged decode attention's block body (one (sequence, kv head) pair, or one context split of it), shared by
// the decode kernel (paged_attention.hip) and the prefill kernel (prefill_attention.hip), whose blocks of the short
// sequences of a varlen call run it in place of a separate launch. The algorithm is described in
// paged_attention.hip.
#pragma once

#include <type_traits>

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
  float* ws;      // split pairs: fp32 records (max, sum, O[D]) per row, rec_stride floats per (pair, split) block
                  // of RP rows at ws + (pair * rec_splits + split) * rec_stride
  // varlen (the short sequences of a paged prefill call, splits = 1): sequence b's queries are rows cu_q[b] ..
  // cu_q[b+1]-1 of q and out and its context is cu_k[b+1] - cu_k[b] keys; a sequence with no queries or more
  // than q_len is left alone (the prefill kernel takes it). Null: q_len queries per sequence, ctx_lens.
  const int32_t* cu_q;
  const int32_t* cu_k;
  // FUSE kernels (q_len 1, D 64 / 128): q, kn, vn are the raw rows of the qkv projection. The kernel applies the
  // per-head RMSNorm + RoPE of qk_norm_rope_kv (common.h arithmetic, the same bits) to its query rows and to
  // sequence b's new key; in the block whose token range holds the new token (position ctx - 1) the wave whose
  // chunk holds it computes the new key and value rows, uses them in place of what its chunk load read for that
  // token, and writes them into the cache slot slots[b] for the steps after this one.
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
  int rec_splits;      // record blocks per pair
  int64_t rec_stride;  // floats per record block (>= RP * (2 + D))
  // counters != null (ctx_lens calls): the blocks of a split pair merge their records themselves -- each writes
  // its record through to memory, waits for the stores, and bumps the pair's counter; the block that brings it to
  // the pair's split count reads every record with device-scope loads, merges them in split order (the combine
  // kernel's arithmetic) and sets the counter back to 0. The counters are zero between calls.
  uint32_t* counters;
  int num_seqs;
  int balance;  // pieces from balance_pieces (length-aware) instead of splits x split_len
  int halves;   // (with counters; the prefill launch's short sequences) block bid takes half bid % 2 of pair
                // bid / 2: its context cut in the middle
};

// A block's share of one (sequence, kv head) pair: tokens [tok_begin, min(ctx, tok_stop)), split `split` of the
// pair's `nsplit` (nsplit > 1: the pieces' records are merged).
struct Piece {
  int pair, split, nsplit, tok_begin, tok_stop;
};

constexpr int kMinTail = 128;  // a long pair's tail shorter than this stays with its own block

__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ bf16x8_t load_bf16x8(const uint16_t* p) { return *reinterpret_cast<const bf16x8_t*>(p); }
// K / V cache rows, read once per launch, with the nontemporal hint: the loads then neither hit nor fill the Infinity
// Cache, and a batch's cache (~163 MB at batch 32, U[512, 2048] contexts) streams faster from HBM -- per-chunk
// timestamps show every wave waiting 2-4.5 us for each chunk's loads against 0.6 us of compute, and the launch
// took 37.0 us with the hint against 41.7 us without (instrumented builds). A second chunk in flight per wave
// (prefetch) measured slower either way: the chip is at its bandwidth for this pattern while most pairs run.
__device__ __forceinline__ bf16x8_t load_bf16x8_once(const uint16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const bf16x8_t*>(p));
}

// Element offset of token t's row for this kv head in the caches, or -1 if its block is not a valid block.
// ALIGNED: block_size is a multiple of the chunk, so every token of a chunk lies in the block of the chunk start.
template <int D>
__device__ __forceinline__ int64_t token_row(const DecodeArgs& g, const int32_t* bt_row, int t, int kvh) {
  const int blk = bt_row[t / g.bs];
  if (blk < 0 || blk >= g.num_blocks) return -1;
  return ((int64_t(blk) * g.bs + t % g.bs) * g.Hkv + kvh) * D;
}


// Balanced pieces (calls of at most 64 sequences): the n sequences the kernel takes -- a decode call's with a
// non-empty context, the ones with 1 .. q_len queries and keys of a varlen call -- are ranked by context length
// (longest first, ties by index) and rank r < n / 2 is paired with rank n - 1 - r. Empty sequences (batch padding)
// are left out, so padding a batch with them changes no other sequence's pieces. For each kv head the long
// sequence's pair is cut where both blocks get the same work: the long pair's block takes [0, cut), the short
// pair's block takes [cut, ctx_long) and then its own whole context, so that every block of the launch streams
// about (ctx_long + ctx_short) / 2 tokens from the start -- instead of the longest pairs streaming alone at the end
// while the CUs of the short ones idle. Cuts are whole 32-token chunks, moved `shift` tokens towards the long pair's
// block (the short pair's block runs two pieces); a tail under kMinTail tokens is not cut.
// Fills pc with block bid's pieces (the tail first) and returns their count; every wave computes the same plan
// (one context length per lane).
__device__ __forceinline__ int balance_pieces(const DecodeArgs& g, int bid, Piece* pc, int shift) {
  const int lane = threadIdx.x % 64, cap = g.max_blocks * g.bs;
  int c = -1;  // this lane's sequence's context length, -1 if the kernel does not take it
  if (lane < g.num_seqs) {
    if (g.cu_q != nullptr) {
      const int lq = g.cu_q[lane + 1] - g.cu_q[lane];
      if (lq >= 1 && lq <= g.q_len) c = min(max(g.cu_k[lane + 1] - g.cu_k[lane], 0), cap);
    } else {
      c = min(max(g.ctx_lens[lane], 0), cap);
    }
    if (c == 0) c = -1;
  }
  const int n = __popcll(__ballot(c >= 0));
  // unique keys in that order: (c + 1) above 63 - lane (a context of 2^26 - 1 tokens or more ranks as that), so the
  // rank is one compare per sequence; the sequences the kernel does not take (key < 64) rank after the others
  const uint32_t key = (uint32_t(min(c + 1, (1 << 26) - 1)) << 6) | uint32_t(63 - lane);
  const int ns = min(g.num_seqs, 64);
  int rank = 0;
  for (int j = 0; j < ns; ++j) rank += __builtin_amdgcn_readlane(key, j) > key ? 1 : 0;
  const int b = bid / g.Hkv, h = bid % g.Hkv;
  const int rb = __builtin_amdgcn_readlane(rank, b), rp = n - 1 - rb;
  pc[0] = Piece{bid, 0, 1, 0, INT32_MAX};
  if (__builtin_amdgcn_readlane(c, b) < 0) return 1;  // a sequence not taken: its own (empty) pair only
  if (rb == rp) return 1;  // the median of an odd batch
  const int bp = __ffsll((unsigned long long)__ballot(rank == rp)) - 1;
  const int cb = __builtin_amdgcn_readlane(c, b), cp = __builtin_amdgcn_readlane(c, bp);
  const int c_long = rb < rp ? cb : cp, c_short = rb < rp ? cp : cb;
  const int cut = min(c_long, max(kChunk, ((c_long + c_short + 1) / 2 + shift + kChunk - 1) / kChunk * kChunk));
  if (c_long - cut < kMinTail) return 1;
  if (rb < rp) {  // the long pair: its head
    pc[0].nsplit = 2, pc[0].tok_stop = cut;
    return 1;
  }
  pc[1] = pc[0];  // the short pair: the long pair's tail, then its own context
  pc[0] = Piece{bp * g.Hkv + h, 1, 2, cut, INT32_MAX};
  return 2;
}

// Bytes of LDS decode_block uses: every wave's K and V chunk (or, afterwards, its partial O) and the waves' row max
// and sum.
__host__ __device__ constexpr int decode_lds_bytes(int D, int RP, bool) {
  const int nwv = D == 256 ? 4 : 8, vb = nwv * 32 * ((D + 16) + (D + 8)) * 2, rb = nwv * RP * D * 4;
  return (vb > rb ? vb : rb) + 2 * nwv * RP * 4;
}

template <int D, int RP, bool ALIGNED, bool FUSE = false>
__device__ __forceinline__ void decode_piece(const DecodeArgs& g, const Piece& pc, unsigned char* lds) {
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
  static_assert(decode_lds_bytes(D, RP, FUSE) == (VBYTES > RBYTES ? VBYTES : RBYTES) + 2 * NWV * RP * 4,
                "LDS layout");
  unsigned char* smem = lds;  // the waves' K / V chunks, then their partial O
  float (*red_m)[RP] = reinterpret_cast<float (*)[RP]>(lds + (VBYTES > RBYTES ? VBYTES : RBYTES));
  float (*red_l)[RP] = red_m + NWV;
  bool fresh_here = false;  // FUSE: this block's token range holds the new token (wave-uniform)
  u32x4 na = {}, nb = {};    // FUSE: this lane's 8 + 8 elements of the new key (lanes < D/16) or value row

  const int pair = pc.pair, split = pc.split, nsplit = pc.nsplit, tok_begin = pc.tok_begin, tok_stop = pc.tok_stop;
  const int b = pair / g.Hkv, kvh = pair % g.Hkv;
  const int lane = threadIdx.x % 64, wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
  int q0 = b * g.q_len, lq = g.q_len, ctx;  // the sequence's first query row, its queries and context length
  if (g.cu_q != nullptr) {
    q0 = load_uniform(g.cu_q + b);  // b is uniform: the sequence's lengths come through the scalar cache
    lq = load_uniform(g.cu_q + b + 1) - q0;
    if (lq < 1 || lq > g.q_len) return;  // the whole block
    ctx = min(max(load_uniform(g.cu_k + b + 1) - load_uniform(g.cu_k + b), 0), g.max_blocks * g.bs);
  } else {
    ctx = min(max(load_uniform(g.ctx_lens + b), 0), g.max_blocks * g.bs);
  }
  const int rows = g.G * lq;
  const int32_t* bt_row = g.bt + int64_t(b) * g.max_blocks;
  const int blk0 = tok_begin / g.bs;
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
  const int dg = lane % LPT, ts = lane / LPT;
  const int tok_end = min(ctx, tok_stop);
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
  auto load_tile = [&](Tile& T, int ch, bool scalar_bt) {  // scalar_bt: its block-table entry via s_load
    const int t0 = ch * kChunk;
    int64_t base = -1;  // ALIGNED: row offset of token t0; tokens t0 + j follow at + j * Hkv * D
    if constexpr (ALIGNED) {
      const int idx = t0 / g.bs - blk0;
      const int blk = scalar_bt ? load_uniform(bt_row + t0 / g.bs)
                    : idx < 64 ? __builtin_amdgcn_readlane(bt_lane, idx) : bt_row[t0 / g.bs];
      base = (blk < 0 || blk >= g.num_blocks) ? -1 : ((int64_t(blk) * g.bs + t0 % g.bs) * g.Hkv + kvh) * D;
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) T.kvalid[u] = __ballot(row_of(t0 + 16 * u + lane % 16, base, t0) >= 0);
#pragma unroll
    for (int it = 0; it < PVI; ++it) {
      const int64_t row = row_of(t0 + it * TPI + ts, base, t0);
      T.k[it] = load_bf16x8_once(row >= 0 ? g.kc + row + 8 * dg : g.q);
      T.v[it] = load_bf16x8_once(row >= 0 ? g.vc + row + 8 * dg : g.q);
    }
  };
  const int ch0 = tok_begin / kChunk + wave;  // the wave's chunks are ch0, ch0 + NWV, ...
  Tile A;
  bool have = false;  // FUSE: A already holds chunk ch0 (requested during the prologue)
  if constexpr (FUSE) {
    static_assert(D == 64 || D == 128, "fused pre-attention: head_dim 64 or 128");
    constexpr int HK = KC / 2, LN = D / 16;
    // Every input of the prologue is requested before its first wait (vector loads retire in issue order): the
    // sequence's position, cache slot and last block-table entry (scalar loads), the query norm weights, in a block
    // whose range holds the new token that token's key and value rows (lanes 0 .. D/16-1: key, with the key norm
    // weights; the next D/16 lanes: value), and, once the position is in, the cos / sin rows.
    const int64_t p = load_uniform(g.positions + b);
    const int32_t slot = load_uniform(g.slots + b);
    const int blk_last = load_uniform(bt_row + max(ctx - 1, 0) / g.bs);
    const bool writer = ctx > 0 ? (tok_begin <= ctx - 1 && ctx - 1 < tok_stop) : split == 0;
    const int e = 8 * (lane % LN);  // this lane's elements of the new row: e .. e+7 and D/2 + e .. +7
    u32x4 ra = {}, rb = {}, kwa = {}, kwb = {};
    if (writer && lane < D / 8) {
      const uint16_t* r = lane < LN ? g.kn + int64_t(b) * g.kn_st + int64_t(kvh) * D
                                    : g.vn + int64_t(b) * g.vn_st + int64_t(kvh) * D;
      ra = *reinterpret_cast<const u32x4*>(r + e);
      rb = *reinterpret_cast<const u32x4*>(r + D / 2 + e);
      kwa = *reinterpret_cast<const u32x4*>(g.k_w + e);  // used by the key lanes only
      kwb = *reinterpret_cast<const u32x4*>(g.k_w + D / 2 + e);
    }
    u32x4 qwa[HK], qwb[HK];
#pragma unroll
    for (int u = 0; u < HK; ++u) {
      qwa[u] = *reinterpret_cast<const u32x4*>(g.q_w + 32 * u + q8);
      qwb[u] = *reinterpret_cast<const u32x4*>(g.q_w + D / 2 + 32 * u + q8);
    }
    const float* cs = g.cos_sin + (p < 0 ? 0 : p >= g.max_pos ? g.max_pos - 1 : p) * g.cs_st;
    float qcos[HK][8], qsin[HK][8], kcos[8] = {}, ksin[8] = {};
#pragma unroll
    for (int u = 0; u < HK; ++u)
#pragma unroll
      for (int i = 0; i < 8; ++i) qcos[u][i] = cs[32 * u + q8 + i], qsin[u][i] = cs[D / 2 + 32 * u + q8 + i];
    if (writer && lane < LN) {
#pragma unroll
      for (int i = 0; i < 8; ++i) kcos[i] = cs[e + i], ksin[i] = cs[D / 2 + e + i];
    }
    // the new key and value rows go to slot `slot`
    const bool store = writer && slot >= 0 && slot < g.num_slots;
    // the new rows stand in for what the chunk loads read at position ctx - 1 when that is the slot they go to (a
    // decode step); otherwise (inconsistent slot, clamped context) they are written before any wave reads
    if (store && ctx > 0 && ctx == load_uniform(g.ctx_lens + b))
      fresh_here = blk_last >= 0 && int64_t(blk_last) * g.bs + (ctx - 1) % g.bs == slot;
    // the wave's first chunk is requested now, its loads in flight during the arithmetic below (its block-table
    // entry through the scalar cache: no wait on the vector loads); not when the rows must reach the cache first
    if (!(store && !fresh_here) && ch0 < ch_end) {
      load_tile(A, ch0, true);
      have = true;
    }
    // the query rows: lane group q8 / 8 = j0 holds the elements 8 j of the fused norm's lanes j = j0 + 4 u
    // (chunk u of each half), so the sum of squares is rebuilt in that kernel's (torch's) order: per half, lanes
    // j ^ 1 and j ^ 2 are lane groups 16 and 32 apart and j ^ 4 is the other chunk u; then the two halves
    float x1[HK][8], x2[HK][8], p1[HK], p2[HK];
#pragma unroll
    for (int u = 0; u < HK; ++u) {
      unpack8(__builtin_bit_cast(u32x4, qf[u]), x1[u]);
      unpack8(__builtin_bit_cast(u32x4, qf[u + HK]), x2[u]);
      p1[u] = half_sumsq8<D>(x1[u]);
      p2[u] = half_sumsq8<D>(x2[u]);
      p1[u] += __shfl_xor(p1[u], 16);
      p2[u] += __shfl_xor(p2[u], 16);
      p1[u] += __shfl_xor(p1[u], 32);
      p2[u] += __shfl_xor(p2[u], 32);
    }
    const float ss = HK == 1 ? p1[0] + p2[0] : (p1[0] + p1[HK - 1]) + (p2[0] + p2[HK - 1]);
    const float rstd = torch_rsqrt(ss * g.inv_d + g.eps);
#pragma unroll
    for (int u = 0; u < HK; ++u) {
      u32x4 oa, ob;
      norm_rope16(x1[u], x2[u], rstd, qwa[u], qwb[u], qcos[u], qsin[u], oa, ob);
      qf[u] = qrow < rows ? __builtin_bit_cast(bf16x8_t, oa) : bf16x8_t{};
      qf[u + HK] = qrow < rows ? __builtin_bit_cast(bf16x8_t, ob) : bf16x8_t{};
    }
    // computed by the wave whose chunk holds the new token (no block barrier), or by wave 0 when they must reach the
    // cache before any wave reads it
    const int cw = fresh_here ? ((ctx - 1) / kChunk - tok_begin / kChunk) % NWV : 0;
    if (store && wave == cw && lane < D / 8) {
      if (lane < LN) {
        float k1[8], k2[8];
        unpack8(ra, k1);
        unpack8(rb, k2);
        const float krstd = torch_rsqrt(torch_row_sumsq<D>(k1, k2) * g.inv_d + g.eps);
        norm_rope16(k1, k2, krstd, kwa, kwb, kcos, ksin, na, nb);
      } else {
        na = ra, nb = rb;
      }
      // into the cache for the next steps (with fresh_here this kernel takes them from the registers instead)
      uint16_t* dst = const_cast<uint16_t*>(lane < LN ? g.kc : g.vc) + int64_t(slot) * g.Hkv * D +
                      int64_t(kvh) * D + e;
      *reinterpret_cast<u32x4*>(dst) = na;
      *reinterpret_cast<u32x4*>(dst + D / 2) = nb;
    }
    if (store && !fresh_here) __syncthreads();  // block-uniform: the rows are in the cache before any wave reads
  }
  // row qrow sees tokens < row_limit
  const int row_limit = qrow >= rows ? 0 : g.causal ? min(max(ctx - lq + qi + 1, 0), ctx) : ctx;

  float m_run = -INFINITY;  // reference max of row qrow (the same in the 4 lanes of the row)
  float l_run = 0.0f;       // this lane's part of the row sum
  f32x4_t acc[DT];          // O^T dims 16 t + 4 (l / 16) + r of row qrow
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x4_t{0, 0, 0, 0};
  const int h4 = lane / 16, l16 = lane % 16;
  uint16_t* vs = reinterpret_cast<uint16_t*>(smem) + wave * kChunk * (VPW + KPW);  // this wave's V chunk
  uint16_t* ks = vs + kChunk * VPW;                                                 // and K chunk

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
    if constexpr (FUSE) {  // the new token's rows from the registers of this wave (the only one with its chunk)
      const int r = ctx - 1 - t0;
      if (fresh_here && r >= 0 && r < kChunk && lane < D / 8) {
        constexpr int LN = D / 16;
        uint16_t* row = lane < LN ? ks + r * KPW : vs + r * VPW;
        const int e = 8 * (lane % LN);
        *reinterpret_cast<u32x4*>(row + e) = na;
        *reinterpret_cast<u32x4*>(row + D / 2 + e) = nb;
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
  // the next chunk during the current one, measured no faster).
  for (int ch = ch0; ch < ch_end; ch += NWV) {
    if (!have) load_tile(A, ch, false);
    have = false;
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
    if (nsplit > 1) {  // this block's record, merged by paged_decode_combine or below
      float* rec = g.ws + (int64_t(pair) * g.rec_splits + split) * g.rec_stride + r * (2 + D);
      if (g.counters != nullptr) {  // written through the L2 (sc1): the merging block may sit on another XCD
        if (d == 0) {
          __hip_atomic_store(rec, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(rec + 1, den, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __hip_atomic_store(rec + 2 + d, num, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        if (d == 0) {
          rec[0] = M;
          rec[1] = den;
        }
        rec[2 + d] = num;
      }
      continue;
    }
    const float o = den > 0.0f ? num / den : 0.0f;
    const int i = r / g.G, hh = r % g.G;
    g.out[int64_t(q0 + i) * g.o_st + int64_t(kvh * g.G + hh) * g.o_sh + d] = f32_to_bf16(o);
  }
  if (nsplit == 1 || g.counters == nullptr) return;
  // The last block of the pair merges. Every wave waits for its record stores to complete (written through to
  // memory) before the barrier; the counter is a device-scope atomic; the merging block reads the records with
  // device-scope loads after its atomic returned. No L2 write-back or invalidate is needed.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  int* flag = reinterpret_cast<int*>(red_m);  // free: every thread is past the merge loop above
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(g.counters + pair, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old == uint32_t(nsplit - 1);
    if (last) __hip_atomic_store(g.counters + pair, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = last;
  }
  __syncthreads();
  if (!*flag) return;
  const float* recs = g.ws + int64_t(pair) * g.rec_splits * g.rec_stride;
  constexpr int SMEM_FLOATS = (VBYTES > RBYTES ? VBYTES : RBYTES) / 4;
  if (nsplit <= 8 || nsplit * rows * 2 > SMEM_FLOATS) {
    for (int idx = threadIdx.x; idx < rows * D; idx += NWV * 64) {
      const int r = idx / D, d = idx % D;
      const float o = merge_splits<true>(recs + r * (2 + D), g.rec_stride, nsplit, 2 + d);
      const int i = r / g.G, hh = r % g.G;
      g.out[int64_t(q0 + i) * g.o_st + int64_t(kvh * g.G + hh) * g.o_sh + d] = f32_to_bf16(o);
    }
    return;
  }
  // many splits (a few long sequences): merge_splits' arithmetic with fewer round trips to memory -- every split's
  // (max, sum) of every row comes into LDS with one round of device-scope loads, then each (row, dim) sums the
  // splits' O in split order with 16 splits' loads in flight (merge_splits issues 8 at a time, in two passes)
  float* ml = reinterpret_cast<float*>(smem);  // [split][row][max, sum]; the partial O are no longer needed
  for (int i = threadIdx.x; i < nsplit * rows * 2; i += NWV * 64) {
    const int sp = i / (rows * 2), r = (i / 2) % rows, c = i % 2;
    ml[i] = __hip_atomic_load(const_cast<float*>(recs + sp * g.rec_stride + r * (2 + D) + c), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < rows * D; idx += NWV * 64) {
    const int r = idx / D, d = idx % D;
    float M = -INFINITY;
    for (int sp = 0; sp < nsplit; ++sp) M = fmaxf(M, ml[(sp * rows + r) * 2]);
    float num = 0.0f, den = 0.0f;
    if (M != -INFINITY) {
      for (int s0 = 0; s0 < nsplit; s0 += 16) {
        float o[16];
#pragma unroll
        for (int u = 0; u < 16; ++u)
          o[u] = s0 + u < nsplit ? __hip_atomic_load(const_cast<float*>(recs + (s0 + u) * g.rec_stride + r * (2 + D) +
                                                                        2 + d),
                                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                 : 0.0f;
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          if (s0 + u >= nsplit) break;
          const float f = exp2f(ml[((s0 + u) * rows + r) * 2] - M);
          num = __builtin_fmaf(o[u], f, num);
          den = __builtin_fmaf(ml[((s0 + u) * rows + r) * 2 + 1], f, den);
        }
      }
    }
    const float o = den > 0.0f ? num / den : 0.0f;
    const int i = r / g.G, hh = r % g.G;
    g.out[int64_t(q0 + i) * g.o_st + int64_t(kvh * g.G + hh) * g.o_sh + d] = f32_to_bf16(o);
  }
}

// Block bid: split bid % splits of pair bid / splits; or (balance, decode calls) its own pair and then, in a short
// pair's block, a long pair's tail (a barrier between them: the second piece's chunks reuse the LDS of the first's
// merge); or (halves, INLINE: the short sequences of the prefill launch) half bid % 2 of pair bid / 2. Each call of
// the body is a copy of it, so a kernel holds only the modes it runs.
template <int D, int RP, bool ALIGNED, bool FUSE = false, bool INLINE = false>
__device__ __forceinline__ void decode_block(const DecodeArgs& g, const int bid, unsigned char* lds) {
  if constexpr (INLINE) {
    Piece pc{bid, 0, 1, 0, INT32_MAX};
    if (g.halves) {  // the pair's context cut in the middle (whole chunks); a short one stays whole in half 0
      const int pair = bid / 2, half = bid % 2, b = pair / g.Hkv, cap = g.max_blocks * g.bs;
      const int lq = load_uniform(g.cu_q + b + 1) - load_uniform(g.cu_q + b);
      if (lq < 1 || lq > g.q_len) return;
      const int ctx = min(max(load_uniform(g.cu_k + b + 1) - load_uniform(g.cu_k + b), 0), cap);
      const int cut = min(ctx, ((ctx + 1) / 2 + kChunk - 1) / kChunk * kChunk);
      if (ctx - cut < kMinTail) {
        if (half == 1) return;
        pc = Piece{pair, 0, 1, 0, INT32_MAX};
      } else {
        pc = Piece{pair, half, 2, half ? cut : 0, half ? INT32_MAX : cut};
      }
    }
    decode_piece<D, RP, ALIGNED, FUSE>(g, pc, lds);
  } else {
    if (g.balance) {
      Piece pc[2];
      // the cut moves 2 chunks towards the long pair's block: the short pair's block runs a second piece after a
      // barrier, and in the fused kernel that piece repeats the prologue (query norm + RoPE, the new key / value
      // row). Decode step (fused kernel) with moves of 0, 1, 2, 3, 4, 6 chunks: 1825, 1814, 1808, 1800, 1803, 1829
      // us; batch-32 decode attention (plain kernel): 32.8 us up to 2 chunks, 33.6 us at 3. The plain and fused
      // kernels cut alike, so the fused call stays bitwise the two calls.
      const int n = balance_pieces(g, bid, pc, 2 * kChunk);
      decode_piece<D, RP, ALIGNED, FUSE>(g, pc[0], lds);
      if (n > 1) {
        __syncthreads();
        decode_piece<D, RP, ALIGNED, FUSE>(g, pc[1], lds);
      }
      return;
    }
    const int split = bid % g.splits;
    decode_piece<D, RP, ALIGNED, FUSE>(g, Piece{bid / g.splits, split, g.splits, split * g.split_len,
                                                split * g.split_len + g.split_len}, lds);
  }
}

}  // namespace
}  // namespace nvhip
