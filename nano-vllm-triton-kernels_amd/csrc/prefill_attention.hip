// Prefill (variable-length, causal) attention for gfx950.
//
// Replaces flash_attn_varlen_func(q, k, v, max_seqlen_q, cu_seqlens_q, max_seqlen_k, cu_seqlens_k, softmax_scale,
// causal=True, block_table) as nano-vllm calls it for prefill (layers/attention.py:77-83): sequence b owns query
// tokens cu_seqlens_q[b] .. cu_seqlens_q[b+1]-1 of q [Tq, Hq, D] and key tokens 0 .. lk-1, lk = cu_seqlens_k[b+1] -
// cu_seqlens_k[b]; the keys are rows cu_seqlens_k[b] + j of k, v [Tk, Hkv, D], or, with a block table (prefix
// cache, model_runner.py:311-312), cache slot block_table[b][j / block_size] * block_size + j % block_size of the
// paged caches [num_blocks, block_size, Hkv, D]. Query i of a sequence with lq queries sees keys j <= lk - lq + i
// with causal (the mask aligned to the bottom right), all lk keys otherwise. Head h reads kv head h / (Hq / Hkv).
//
// One block (8 waves) per (query tile, sequence, pair of q heads of one kv head): 4 waves and 128 queries per head;
// when Hq / Hkv is odd, one head per block with 8 waves and 256 queries. Wave w of a head owns queries 32w .. 32w+31
// of the tile. The two heads share the K/V tiles (half the K/V traffic of a block per head). Per 64-key tile:
//   1. the K and V tiles go to LDS key-major ([64][D], 16-byte chunks, rows padded);
//   2. S^T [32 keys x 32 queries] = K Q^T per 32-key half with v_mfma_f32_32x32x16_bf16 (K rows from LDS as the A
//      operand, the wave's Q rows from registers as the B operand): lane l holds keys 8 (r / 4) + 4 (l / 32) + r % 4
//      (register r) of query l % 32, so one query's 64 scores sit in lanes l and l ^ 32;
//   3. fp32 online softmax in base 2 per query: the max of the raw scores, then p = 2^(s * scale * log2 e - m) in
//      one FMA and the hardware exp;
//   4. O^T [32 dims x 32 queries] += V^T P^T per 32-dim tile and 16-key step: P (bf16) stays in the registers it was
//      computed in as the B operand, whose 8 k slots of lane l are the keys 4 (l / 32) .. +3 and 8 + 4 (l / 32) ..
//      +3 of the step; the A operand gets the same keys of dim l % 32 from the key-major V tile with two gfx950
//      transpose reads (ds_read_b64_tr_b16, 4 keys each). Each lane keeps one query's O, so the rescale by
//      2^(m_old - m_new) is lane-local.
// A wave's 32 queries use each K and V fragment it reads from LDS twice as often as 16 would, which halves the LDS
// reads per flop; the per-tile work that does not scale with the queries (loads, LDS stores, barriers) is shared by
// twice the flops.
// P is rounded to bf16 for the P.V product (as flash-attn does) and the row sum adds the fp32 p (as flash-attn
// does); scores, softmax and O are fp32; output bf16. The softmax scale must be positive.
// Key splits (with a caller workspace): when the blocks of one pass leave CUs idle and the key ranges are long (a
// prompt chunk over its cached prefix: 2 query tiles x 8 head pairs = 16 blocks streaming thousands of keys each),
// each (query tile, sequence, head group) is cut into key ranges run by separate blocks; each writes its queries'
// (max, sum, O) records and prefill_combine merges them in split order.
#include <algorithm>

#include "decode_attention.h"

namespace nvhip {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kWavesBlock = 8;  // waves per block: 4 per head with two heads, 8 with one
constexpr int kBK = 64;   // keys per tile
constexpr int kThreads = 64 * kWavesBlock;
// queries per block and head (32 per wave)
__host__ __device__ constexpr int block_queries(int heads_per_block) { return 32 * kWavesBlock / heads_per_block; }

struct PrefillArgs {
  uint16_t* out;
  const uint16_t* q;
  const uint16_t* k;  // contiguous [Tk, Hkv, D] rows, or the k cache with a block table
  const uint16_t* v;
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* bt;  // [num_seqs, max_blocks] or null
  int64_t q_st, q_sh, k_st, v_st, o_st, o_sh;
  int Hkv, G, bs, num_blocks, max_blocks;
  float scale_log2;  // softmax scale * log2(e), > 0
  int causal;
  int qtiles, nhg;  // query tiles per sequence (from max_seqlen_q), head groups (Hq / heads per block)
  int lq_skip;      // sequences with 1 .. lq_skip queries are left to the paged decode kernel
  int splits;       // key ranges per (query tile, sequence, head group): split s takes keys s * split_len ..
  int split_len;    // a multiple of kBK
  int Hq;
  int64_t ws_rows;  // Tq: query rows of one split's records
  // splits > 1: fp32 records merged by prefill_combine -- O [splits, Tq, Hq, D] (unnormalised), then (max, sum)
  // [splits, Tq, Hq, 2]
  float* ws;
  // dec_inline: the blocks of the short sequences (1 .. lq_skip queries) run their paged decode attention
  // themselves (one block per (sequence, kv head), dec: its varlen arguments, one split), concurrently with the
  // prefill tiles, instead of a separate launch before this one
  int dec_inline;
  // dec_extra > 0 (dec.halves): the short sequences' (sequence, kv head) pairs are cut in two; the blocks above
  // run the first halves, dec_extra blocks appended to the grid (one per pair of the call) the second halves
  int dec_extra;
  int out_lines;  // out 16-byte aligned with strides in whole 16-byte pieces: the output goes out in whole lines
  DecodeArgs dec;
};

// fp32 elements of one (split, query, head) record: O[D] in the O array, max and row sum in the (max, sum) array.
__host__ __device__ constexpr int record_len(int D) { return D + 2; }

// Element offset of key j of sequence b, kv head kvh, in k (v with v_st): a contiguous row, or (PAGED) the cache
// slot of block blk (-1 if the block is not valid).
template <int D, bool PAGED>
__device__ __forceinline__ int64_t key_row(const PrefillArgs& g, int k0s, int j, int blk, int kvh, int64_t st) {
  if constexpr (!PAGED) return int64_t(k0s + j) * st + int64_t(kvh) * D;
  if (blk < 0 || blk >= g.num_blocks) return -1;
  return ((int64_t(blk) * g.bs + j % g.bs) * g.Hkv + kvh) * D;
}

// HB q heads of one kv head per block (4 waves each, sharing the K/V tiles in LDS).
template <int D, bool PAGED, int HB>
__global__ __launch_bounds__(kThreads) void prefill_attention_kernel(const PrefillArgs g) {
  constexpr int kBQ = block_queries(HB), kHeadThreads = kThreads / HB;
  constexpr int DC = D / 16;   // 16-wide dim steps of Q.K
  constexpr int DT = D / 32;   // 32-dim output tiles
  constexpr int CPR = D / 8;   // 16-byte chunks per K/V row
  constexpr int KP = D + 8;    // K row pitch (elements)
  // V row pitch: D + 32 elements puts the 4 rows of a transpose read 16 (or 48) banks apart, so the 32 lanes of a
  // half-wave (4 keys x 32 dims) hit 64 distinct banks
  constexpr int VP = D + 32;
  constexpr int STAGE = kBK * (KP + VP);  // elements of one LDS stage (K tile, then V tile)
  // LDS: two K/V tile stages, or (paged) the decode attention's buffers for the blocks of short sequences
  constexpr int DEC_BYTES = PAGED ? decode_lds_bytes(D, 16, false) : 0;
  constexpr int LDS_ELEMS = (2 * STAGE * 2 > DEC_BYTES ? 2 * STAGE * 2 : DEC_BYTES) / 2;
  __shared__ __attribute__((aligned(16))) uint16_t lds[LDS_ELEMS];

  // Block order. The ids are dealt round-robin over the 8 XCDs (block b runs on XCD b % 8) and each XCD starts its
  // blocks in id order as CUs free up. When the groups (sequence, head group) divide evenly, XCD x takes whole
  // groups -- all query tiles of a group read the same K/V, which then stays in one XCD's L2 -- namely groups x,
  // x + 8, x + 16, ..., so that every sequence's head groups are spread over the XCDs (contiguous ranges of groups
  // put a mixed step's prefill chunk, the batch's last sequence, on one XCD), and starts them heaviest query tile
  // (most keys) first across its groups, so that no long tile starts late (longest-first list scheduling; starting
  // one group's tiles before the next group's left a third of the CUs idle at the end of a 4 x 2048-token prefill).
  // Otherwise all groups' tiles are dealt heaviest first.
  // With key splits, the (query tile, split) pairs of a group are its tiles, heaviest (latest query tile, first
  // split) first.
  const int ntile = g.qtiles * g.splits;
  const int nblk = int(gridDim.x) - g.dec_extra, ngrp = nblk / ntile;
  if (int(blockIdx.x) >= nblk) {  // a second half of a short sequence's pair (the whole block: uniform)
    if constexpr (PAGED) {
      const int pair = int(blockIdx.x) - nblk;
      if (g.dec.bs % 32 == 0)
        decode_block<D, 16, true, false, true>(g.dec, 2 * pair + 1, reinterpret_cast<unsigned char*>(lds));
      else
        decode_block<D, 16, false, false, true>(g.dec, 2 * pair + 1, reinterpret_cast<unsigned char*>(lds));
    }
    return;
  }
  int grp, ci;
  if (nblk % 8 == 0 && (nblk / 8) % ntile == 0) {
    const int gx = nblk / 8 / ntile, r = blockIdx.x / 8;
    grp = (r % gx) * 8 + blockIdx.x % 8;
    ci = r / gx;
  } else {
    grp = blockIdx.x % ngrp;
    ci = blockIdx.x / ngrp;
  }
  const int qt = g.qtiles - 1 - ci / g.splits, split = ci % g.splits;
  const int b = grp / g.nhg, hg = grp % g.nhg;
  const int h = hg * HB + int(threadIdx.x) / kHeadThreads, kvh = (hg * HB) / g.G;
  const int q0s = g.cu_q[b], lq = g.cu_q[b + 1] - q0s;
  const int k0s = g.cu_k[b], lk = g.cu_k[b + 1] - k0s;
  if (lq >= 1 && lq <= g.lq_skip) {  // the paged decode attention takes this sequence (the whole block: b is uniform)
    // one block per (sequence, kv head) runs the decode attention of the pair (the whole block: b, hg, ci uniform)
    if constexpr (PAGED) {
      if (g.dec_inline && ci == 0 && (hg * HB) % g.G == 0) {
        const int pair = b * g.Hkv + hg * HB / g.G, bid = g.dec.halves ? 2 * pair : pair;
        if (g.dec.bs % 32 == 0) decode_block<D, 16, true, false, true>(g.dec, bid, reinterpret_cast<unsigned char*>(lds));
        else decode_block<D, 16, false, false, true>(g.dec, bid, reinterpret_cast<unsigned char*>(lds));
      }
    }
    return;
  }
  // keys [k_beg, k_stop) of this block: the split's range, cut at the last key its query tile sees
  const int k_beg = split * g.split_len;
  const int k_hi = split == g.splits - 1 ? INT32_MAX : k_beg + g.split_len;  // the last split takes the rest
  const int k_stop = g.causal ? min(min(lk, lk - lq + min(qt * kBQ + kBQ, lq)), k_hi) : min(lk, k_hi);
  if (qt * kBQ >= lq || k_stop <= k_beg) {
    // no keys for this block: zero rows (one pass), or records that say so (the merge then writes zeros)
    const int r = int(threadIdx.x) % kHeadThreads;
    if (qt * kBQ < lq && r < kBQ && qt * kBQ + r < lq) {
      const int64_t row = q0s + qt * kBQ + r;
      if (g.splits > 1) {
        if (row >= g.ws_rows) return;
        const int64_t rec = (int64_t(split) * g.ws_rows + row) * g.Hq + h;
        float* o = g.ws + rec * D;
        for (int d = 0; d < D; ++d) o[d] = 0.0f;
        *reinterpret_cast<f32x2*>(g.ws + int64_t(g.splits) * g.ws_rows * g.Hq * D + 2 * rec) = f32x2{-INFINITY, 0.0f};
      } else {
        uint16_t* o = g.out + row * g.o_st + int64_t(h) * g.o_sh;
        for (int d = 0; d < D; ++d) o[d] = 0;
      }
    }
    return;
  }
  const int tid = threadIdx.x, lane = tid % 64, wave = __builtin_amdgcn_readfirstlane((tid % kHeadThreads) / 64);
  const int ql = lane % 32, hf = lane / 32;
  const int qi_lane = qt * kBQ + 32 * wave + ql;  // this lane's query (B operand column / O column)

  // Q rows of the wave as the B operand: lane l -> query 32 wave + l % 32, dims 16c + 8 (l / 32) .. +8
  bf16x8_t qf[DC];
  {
    const bool ok = qi_lane < lq;
    const uint16_t* qp = g.q + int64_t(q0s + (ok ? qi_lane : 0)) * g.q_st + int64_t(h) * g.q_sh + 8 * hf;
#pragma unroll
    for (int c = 0; c < DC; ++c) qf[c] = ok ? *reinterpret_cast<const bf16x8_t*>(qp + 16 * c) : bf16x8_t{};
  }
  const int diag = lk - lq;  // query i sees keys <= diag + i
  const int limit_lane = g.causal ? diag + qi_lane : lk - 1;      // last key of this lane's query
  const int wave_q0 = qt * kBQ + 32 * wave;                        // the wave's first query

  f32x16_t o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = f32x16_t{};
  float m_run = -INFINITY, l_run = 0.0f;

  // 1. a tile's K and V chunks go global -> registers (all loads of a tile issued together; the next tile's loads
  // are issued before this tile's MFMAs) -> LDS. K and V chunk c: key c / CPR, dims (c % CPR) * 8, stored
  // key-major with one 16-byte write. Invalid keys read the first 16 bytes of q and store zeros.
  constexpr int NT = kThreads;              // threads loading the tiles
  constexpr int NL = kBK * CPR / NT;        // chunks per thread per operand
  static_assert(NL >= 1 && NL * NT == kBK * CPR, "tile chunks per thread");
  struct Regs {
    u32x4 k[NL], v[NL];
    uint32_t kok;  // bit i: the key of chunk i is valid (its K and V rows were read)
    bool all;  // every key of the tile is valid (wave-uniform): no zeroing at the LDS store
  };
  const int32_t* bt_row = PAGED ? g.bt + int64_t(b) * g.max_blocks : nullptr;
  // Contiguous keys: this thread's K / V row addresses at key tile 0; tile kt0 adds kt0 rows (a scalar offset).
  const uint16_t* kbase[NL];
  const uint16_t* vbase[NL];
  if constexpr (!PAGED) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int c = tid + i * NT;
      kbase[i] = g.k + int64_t(k0s + c / CPR) * g.k_st + int64_t(kvh) * D + (c % CPR) * 8;
      vbase[i] = g.v + int64_t(k0s + c / CPR) * g.v_st + int64_t(kvh) * D + (c % CPR) * 8;
    }
  }
  // PAGED: block-table entries of this thread's keys in the tile the next gload call loads (the tiles are loaded
  // in order, the last one repeated), fetched one call ahead: the fetch is issued before that call's data loads and
  // retires with them, so no tile's data loads wait for a block-table load (at 4 key tiles per block, a 256-token
  // chunk over 3840 cached keys, that wait was a memory round trip per tile)
  const int last = (k_stop - 1) / kBK * kBK;
  int kblk_nx[NL];
  auto bt_fetch = [&](int kt0) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int kj = kt0 + (tid + i * NT) / CPR;
      kblk_nx[i] = kj < lk ? bt_row[kj / g.bs] : 0;
    }
  };
  auto gload = [&](Regs& R, int kt0) {
    R.all = kt0 + kBK <= lk;
    R.kok = 0;
    if constexpr (!PAGED) {
      if (R.all) {  // every row valid: the addresses are the bases plus a per-tile offset
#pragma unroll
        for (int i = 0; i < NL; ++i) {
          R.k[i] = *reinterpret_cast<const u32x4*>(kbase[i] + int64_t(kt0) * g.k_st);
          R.v[i] = *reinterpret_cast<const u32x4*>(vbase[i] + int64_t(kt0) * g.v_st);
        }
        return;
      }
    }
    // block-table entries of this thread's keys (PAGED: fetched by the previous call), then the entries of the
    // tile the next call loads, then every data load back to back
    int kblk[NL];
#pragma unroll
    for (int i = 0; i < NL; ++i) kblk[i] = PAGED ? kblk_nx[i] : 0;
    if constexpr (PAGED) bt_fetch(min(kt0 + kBK, last));
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int c = tid + i * NT;
      const int kj = kt0 + c / CPR;
      const int64_t krow = kj < lk ? key_row<D, PAGED>(g, k0s, kj, kblk[i], kvh, g.k_st) : -1;
      const int64_t vrow = kj < lk ? key_row<D, PAGED>(g, k0s, kj, kblk[i], kvh, g.v_st) : -1;
      R.kok |= uint32_t(krow >= 0) << i;  // krow and vrow are valid together
      R.k[i] = *reinterpret_cast<const u32x4*>(krow >= 0 ? g.k + krow + (c % CPR) * 8 : g.q);
      R.v[i] = *reinterpret_cast<const u32x4*>(vrow >= 0 ? g.v + vrow + (c % CPR) * 8 : g.q);
    }
    if constexpr (PAGED) R.all = false;  // a block-table entry may be invalid
  };
  // every key of the tile at kt0 is valid: the bases plus a per-tile offset (contiguous keys only)
  auto gload_full = [&](Regs& R, int kt0) {
    R.all = true;
    R.kok = 0;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      R.k[i] = *reinterpret_cast<const u32x4*>(kbase[i] + int64_t(kt0) * g.k_st);
      R.v[i] = *reinterpret_cast<const u32x4*>(vbase[i] + int64_t(kt0) * g.v_st);
    }
  };
  auto lstore_full = [&](const Regs& R, int stage) {  // R holds a tile whose keys are all valid
    uint16_t* Ks = lds + stage * STAGE;
    uint16_t* Vs = Ks + kBK * KP;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int c = tid + i * NT;
      *reinterpret_cast<u32x4*>(&Ks[(c / CPR) * KP + (c % CPR) * 8]) = R.k[i];
      *reinterpret_cast<u32x4*>(&Vs[(c / CPR) * VP + (c % CPR) * 8]) = R.v[i];
    }
  };
  auto lstore = [&](const Regs& R, int stage) {
    uint16_t* Ks = lds + stage * STAGE;
    uint16_t* Vs = Ks + kBK * KP;
    const bool all = R.all;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int c = tid + i * NT;
      const u32x4 zero = u32x4{0, 0, 0, 0};
      const bool ok = all || ((R.kok >> i) & 1);
      *reinterpret_cast<u32x4*>(&Ks[(c / CPR) * KP + (c % CPR) * 8]) = ok ? R.k[i] : zero;
      *reinterpret_cast<u32x4*>(&Vs[(c / CPR) * VP + (c % CPR) * 8]) = ok ? R.v[i] : zero;
    }
  };

  // 2.-4. per tile: S^T of both 32-key halves, one online-softmax step over the tile's 64 keys, O^T += V^T P^T
  // (the p of the second half are computed under the P.V MFMAs of the first). Rescaling is lazy: a query's
  // reference max m_run only moves when a score exceeds it by more than kLazy (base 2), so p <= 2^kLazy; O and the
  // row sum carry the same factor, which cancels in O / sum, and almost every tile after the first skips the O
  // rescale (one wave-uniform branch per tile).
  constexpr float kLazy = 8.0f;
  auto tile = [&](int kt0, int stage) {
    const uint16_t* Ks = lds + stage * STAGE;
    const uint16_t* Vs = Ks + kBK * KP;
    // S^T per 32-key half: lane holds keys kt0 + 32 u + 8 (r / 4) + 4 hf + r % 4 of query qi_lane. All K fragments
    // of the tile are read before the first MFMA, so the MFMAs wait for LDS latency once, not once each.
    bf16x8_t kf[2][DC];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int c = 0; c < DC; ++c)
        kf[u][c] = *reinterpret_cast<const bf16x8_t*>(&Ks[(32 * u + ql) * KP + 8 * hf + 16 * c]);
    f32x16_t s[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      s[u] = f32x16_t{};
#pragma unroll
      for (int c = 0; c < DC; ++c) s[u] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[u][c], qf[c], s[u], 0, 0, 0);
    }
    // V^T fragments of both halves (A operands of O^T += V^T P^T): dim 32 t + l % 32, keys 32 u + 16 j + 4 hf .. +3
    // and 32 u + 16 j + 8 + 4 hf .. +3, by transpose reads (lane i of a 16-lane group addresses key i / 4 of the 4,
    // dims 4 (i % 4) .. +3 of the group's 16, and receives dim i of the 4 keys); read here so that they are in flight
    // during the softmax
    const uint16_t* vt0 = Vs + (4 * hf + (lane % 16) / 4) * VP + 16 * (ql / 16) + 4 * (lane % 4);
    u32x4 vf[2][DT][2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const uint16_t* vr = vt0 + (32 * u + 16 * j) * VP + 32 * t;
          const u32x2 lo = lds_read_tr16(vr), hi = lds_read_tr16(vr + 8 * VP);
          vf[u][t][j] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
    // issue order: the 8 K reads of half 0, then its MFMAs each followed by a K read of half 1, then the MFMAs of
    // half 1 interleaved with the max of half 0 (VALU work under the matrix cores), then the V reads
    __builtin_amdgcn_sched_group_barrier(0x100, DC, 0);
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
#pragma unroll
    for (int c = 0; c < DC; ++c) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 4 * DT, 0);
    // Only a tile that reaches past the key count or past the causal limit of the wave's first query needs the
    // mask (wave-uniform test); key offsets within the tile are compile-time constants per register.
    const bool full = kt0 + kBK <= lk && (!g.causal || kt0 + kBK - 1 <= diag + wave_q0);
    const int lim = min(lk - 1, limit_lane) - kt0 - 4 * hf;  // largest visible offset 32 u + 8 (r / 4) + r % 4
    // max of the tile's raw scores (the scale is positive)
    float tmax = -INFINITY;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      if (!full) {
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (32 * u + 8 * (r / 4) + r % 4 > lim) s[u][r] = -INFINITY;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, s[u][r]);
    }
    tmax = pair32_max(tmax) * g.scale_log2;
    const bool move = tmax > m_run + kLazy;  // also true for the first finite max (m_run = -inf)
    if (__ballot(move) != 0) {
      const float alpha = move ? __builtin_amdgcn_exp2f(m_run - tmax) : 1.0f;  // 0 from m_run = -inf
      if (move) m_run = tmax;
      l_run *= alpha;
#pragma unroll
      for (int t = 0; t < DT; ++t) o[t] *= alpha;
    }
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;
    // p = 2^(s * scale_log2 - m) in one FMA and v_exp_f32 (arguments <= kLazy; only results below the fp32 normal
    // range, which flush to 0, differ from exp2f), as bf16 packed per 16-key step in the k-slot order of P.V
    bf16x8_t pf[2][2];
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        float p[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[u][8 * j + e], g.scale_log2, -m_use));
          l_run += p[e];
        }
        pf[u][j] = __builtin_bit_cast(bf16x8_t, pack8(p));
      }
    // O^T += V^T P^T; the p of half 1 are computed under the MFMAs of half 0
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int t = 0; t < DT; ++t)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, vf[u][t][j]), pf[u][j], o[t], 0,
                                                         0, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, 28, 1);
#pragma unroll
    for (int i = 0; i < 2 * DT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
      __builtin_amdgcn_sched_group_barrier(0x002, 4, 1);
    }
  };
  // Two LDS stages: while the waves compute tile i from one, the loads of tile i + 1 (issued a tile earlier) are
  // stored into the other and the loads of tile i + 2 are issued; one barrier per tile. Past the last tile the last
  // one is loaded and stored again, unused (every load is issued unconditionally so the compiler's waits are exact).
  // The first tile is peeled: the loads of tiles 0 and 1 both go out before the first wait, so tile 1's are in
  // flight during the prologue and tile 0 (with one set of tile registers, tile 1's loads went out after tile 0's
  // LDS store and were waited for after a single tile of work).
  {
    Regs A;
    if constexpr (PAGED) bt_fetch(k_beg);
    gload(A, k_beg);
    {
      Regs B;
      gload(B, min(k_beg + kBK, last));
      lstore(A, 0);
      __syncthreads();
      tile(k_beg, 0);
      lstore(B, 1);
    }
    gload(A, min(k_beg + 2 * kBK, last));
    __syncthreads();
    int stage = 1;
    int kt0 = k_beg + kBK;
    if constexpr (!PAGED) {
      // while the tile stored next and the one loaded next are both whole (every key valid), the loop body holds
      // only their loads and stores: the general loader's per-key row arithmetic and the zeroing selects, which the
      // compiler executes on every tile when the two paths share the body, are left to the last tiles
      for (; kt0 < k_stop && min(kt0 + 2 * kBK, last) + kBK <= lk; kt0 += kBK) {
        tile(kt0, stage);
        lstore_full(A, stage ^ 1);
        gload_full(A, min(kt0 + 2 * kBK, last));
        __syncthreads();
        stage ^= 1;
      }
    }
    for (; kt0 < k_stop; kt0 += kBK) {
      tile(kt0, stage);
      lstore(A, stage ^ 1);
      gload(A, min(kt0 + 2 * kBK, last));
      __syncthreads();
      stage ^= 1;
    }
  }

  // row sums over the two lane halves of the query; lane l holds O^T dims 32 t + 8 (r / 4) + 4 hf + r % 4 of query
  // qi_lane
  l_run = pair32_sum(l_run);
  if (g.splits > 1) {
    // this split's records of the wave's queries: the reference max and the row sum, and O unnormalised. O goes out
    // in whole 128-byte lines written through the L2: each half of the dims passes through the wave's own part of
    // the LDS (free after the loop's last barrier), a lane holding dims 32 t + 8 (r / 4) + 4 hf + r % 4 of its query
    // and a store instruction then covering D / 2 consecutive floats of 64 * 16 / (2 D) queries. Stored from the
    // MFMA layout (32-byte pieces of 32 records per instruction, (max, sum) beside O) the records' dirty lines were
    // written back after the last block: a 256-token chunk over 3840 cached keys 34.1 -> 32.2 us, a fresh
    // 2048-token prompt (2 splits) 62.7 -> 59.8 us, 256 over 1792 33.0 -> 29.8 us (whole lines with plain stores:
    // 32.5 / 61.8 / 31.3 us).
    const int nq = min(32, min(lq, int(min<int64_t>(g.ws_rows - q0s, INT32_MAX))) - wave_q0);  // wave-uniform
    if (nq <= 0) return;
    const int64_t rec0 = (int64_t(split) * g.ws_rows + q0s + wave_q0) * g.Hq + h;  // record of the first query
    if (hf == 0 && ql < nq)
      *reinterpret_cast<f32x2*>(g.ws + int64_t(g.splits) * g.ws_rows * g.Hq * D + 2 * (rec0 + int64_t(ql) * g.Hq)) =
          f32x2{m_run, l_run};
    constexpr int HD = D / 2, RP = HD + 4;  // dims per pass, LDS row pitch (floats)
    constexpr int CH = HD / 4, PER = 32 * CH / 64;  // 16-byte chunks per query and pass, per lane and pass
    static_assert(kThreads / 64 * 32 * RP * 4 <= LDS_ELEMS * 2, "record staging exceeds the LDS");
    float* wl = reinterpret_cast<float*>(lds) + (tid / 64) * 32 * RP;
#pragma unroll
    for (int hv = 0; hv < 2; ++hv) {
#pragma unroll
      for (int t = hv * DT / 2; t < (hv + 1) * DT / 2; ++t)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr)
          *reinterpret_cast<f32x4_t*>(wl + ql * RP + 32 * (t - hv * DT / 2) + 8 * rr + 4 * hf) =
              f32x4_t{o[t][4 * rr], o[t][4 * rr + 1], o[t][4 * rr + 2], o[t][4 * rr + 3]};
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int c = lane + 64 * i, qq = c / CH, cc = c % CH;
        const u32x4 x = *reinterpret_cast<const u32x4*>(wl + qq * RP + 4 * cc);
        if (qq < nq) store16_wt(g.ws + (rec0 + int64_t(qq) * g.Hq) * D + hv * HD + 4 * cc, x);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
    return;
  }
  const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
  if (g.out_lines) {
    // the wave's 32 output rows pass through its own part of the LDS, so that a store instruction covers whole
    // rows (D bf16 each, 16-byte pieces of 64 * 8 / D queries), written through the L2. Against the rows stored
    // straight from the MFMA layout (8-byte pieces of 32 rows per instruction): 4 x 2048 tokens 82.2 -> 77.3 us
    // (whole lines with plain stores: 78.1), 8 x 512 25.6 -> 21.6 us (23.0), 16 x 256 19.9 -> 15.7 us (17.5); the
    // 256-token mixed step 2170 -> 2160-2167 us per step (plain stores 2155-2205: within its run-to-run spread).
    const int nq = min(32, lq - wave_q0);  // wave-uniform
    if (nq <= 0) return;
    constexpr int RP = D / 2 + 4, CH = D / 8, PER = 32 * CH / 64;  // u32 row pitch, 16-byte pieces per row, per lane
    static_assert(kThreads / 64 * 32 * RP * 4 <= LDS_ELEMS * 2, "output staging exceeds the LDS");
    uint32_t* wl = reinterpret_cast<uint32_t*>(lds) + (tid / 64) * 32 * RP;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr)
        *reinterpret_cast<u32x2*>(wl + ql * RP + 16 * t + 4 * rr + 2 * hf) =
            u32x2{pack_bf16x2(o[t][4 * rr] * inv, o[t][4 * rr + 1] * inv),
                  pack_bf16x2(o[t][4 * rr + 2] * inv, o[t][4 * rr + 3] * inv)};
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    uint16_t* ob = g.out + int64_t(q0s + wave_q0) * g.o_st + int64_t(h) * g.o_sh;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int c = lane + 64 * i, qq = c / CH, cc = c % CH;
      const u32x4 x = *reinterpret_cast<const u32x4*>(wl + qq * RP + 4 * cc);
      if (qq < nq) store16_wt(ob + int64_t(qq) * g.o_st + 8 * cc, x);
    }
    return;
  }
  if (qi_lane >= lq) return;
  uint16_t* op = g.out + int64_t(q0s + qi_lane) * g.o_st + int64_t(h) * g.o_sh + 4 * hf;
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int rr = 0; rr < 4; ++rr)
      *reinterpret_cast<u32x2*>(op + 32 * t + 8 * rr) =
          u32x2{pack_bf16x2(o[t][4 * rr] * inv, o[t][4 * rr + 1] * inv),
                  pack_bf16x2(o[t][4 * rr + 2] * inv, o[t][4 * rr + 3] * inv)};
}

// Merges the split records of every query of the sequences the prefill kernel took, in split order:
// O = sum_s O_s 2^(m_s - M) / sum_s l_s 2^(m_s - M), M = max_s m_s; a query no split saw (M = -inf) is zero.
// One wave per two (query, head) pairs p0 = 2 w, p0 + 1 (pair = query * Hq + head; records of consecutive pairs are
// adjacent), 4 waves per block (block x: sequence x / per_seq, its waves 4 (x % per_seq) ..): lane s < splits reads
// split s's (max, sum) of both pairs (all at once), the weights come back to the whole wave with readlane, and half
// h of the wave sums pair p0 + h, D / 32 dims per lane (one 16-byte load per split at D = 128), eight splits' loads
// in flight at a time. (One wave per pair, 8-byte loads, four splits at a time: the merge of a 256-token chunk over
// 3840 cached keys, 16 splits, read its 34.6 MB of records at ~5 TB/s.)
template <int D>
__global__ __launch_bounds__(256) void prefill_combine(const PrefillArgs g, int per_seq) {
  constexpr int DPL = D / 32, SB = 8;
  static_assert(DPL == 2 || DPL == 4, "head_dim 64 or 128");
  const int b = blockIdx.x / per_seq;
  const int lane = threadIdx.x % 64, hh = lane / 32;
  const int p0 = ((blockIdx.x % per_seq) * 4 + int(threadIdx.x) / 64) * 2;
  const int q0s = g.cu_q[b], lq = g.cu_q[b + 1] - q0s;
  if (lq <= g.lq_skip) return;  // the decode kernel wrote these rows (or there are none)
  const int64_t rows_left = min<int64_t>(lq, g.ws_rows - q0s);  // queries of the sequence that have records
  const bool ok0 = p0 < rows_left * g.Hq, ok1 = p0 + 1 < rows_left * g.Hq;
  if (!ok0) return;  // the wave's first pair is past the sequence's queries (wave-uniform)
  const int64_t step = g.ws_rows * g.Hq;  // records of one split
  const int64_t rec0 = int64_t(q0s) * g.Hq + p0;
  const float* ml = g.ws + g.splits * step * D + 2 * rec0;  // (max, sum) of pair p0, split 0
  const bool mine = lane < g.splits;  // splits <= 64 (host)
  f32x2 ml0 = {-INFINITY, 0.0f}, ml1 = {-INFINITY, 0.0f};
  if (mine) ml0 = *reinterpret_cast<const f32x2*>(ml + 2 * lane * step);
  if (mine && ok1) ml1 = *reinterpret_cast<const f32x2*>(ml + 2 + 2 * lane * step);
  float M0 = ml0[0], M1 = ml1[0];
#pragma unroll
  for (int off = 32; off >= 1; off /= 2) M0 = fmaxf(M0, __shfl_xor(M0, off)), M1 = fmaxf(M1, __shfl_xor(M1, off));
  const float f0 = M0 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml0[0] - M0);  // 0 for a split that saw nothing
  const float f1 = M1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml1[0] - M1);
  float den0 = ml0[1] * f0, den1 = ml1[1] * f1;
#pragma unroll
  for (int off = 32; off >= 1; off /= 2) den0 += __shfl_xor(den0, off), den1 += __shfl_xor(den1, off);
  const bool mine_pair = hh == 0 || ok1;
  const float* rp = g.ws + (rec0 + hh) * D + (lane % 32) * DPL;
  float num[DPL] = {};
  for (int sp0 = 0; sp0 < g.splits; sp0 += SB) {
    float v[SB][DPL];
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      const int sp = min(sp0 + u, g.splits - 1);
      if (mine_pair) {
        if constexpr (DPL == 4) {
          const f32x4_t x = *reinterpret_cast<const f32x4_t*>(rp + sp * step * D);
          v[u][0] = x[0], v[u][1] = x[1], v[u][2] = x[2], v[u][3] = x[3];
        } else {
          const f32x2 x = *reinterpret_cast<const f32x2*>(rp + sp * step * D);
          v[u][0] = x[0], v[u][1] = x[1];
        }
      } else {
#pragma unroll
        for (int e = 0; e < DPL; ++e) v[u][e] = 0.0f;
      }
    }
#pragma unroll
    for (int u = 0; u < SB; ++u) {
      if (sp0 + u >= g.splits) break;  // uniform
      const float w0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f0), sp0 + u));
      const float w1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, f1), sp0 + u));
      const float w = hh ? w1 : w0;
#pragma unroll
      for (int e = 0; e < DPL; ++e) num[e] = __builtin_fmaf(v[u][e], w, num[e]);
    }
  }
  if (!mine_pair) return;
  const float den = hh ? den1 : den0;
  const float inv = den > 0.0f ? 1.0f / den : 0.0f;
  const int pr = p0 + hh, i = pr / g.Hq, h = pr % g.Hq;
  uint16_t* o = g.out + int64_t(q0s + i) * g.o_st + int64_t(h) * g.o_sh + (lane % 32) * DPL;
  if constexpr (DPL == 4)
    *reinterpret_cast<u32x2*>(o) =
        u32x2{pack_bf16x2(num[0] * inv, num[1] * inv), pack_bf16x2(num[2] * inv, num[3] * inv)};
  else
    *reinterpret_cast<uint32_t*>(o) = pack_bf16x2(num[0] * inv, num[1] * inv);
}

// Key splits: only when the blocks of one pass (query tiles x sequences x head groups) leave CUs idle and the
// sequences bring long key ranges (a chunk of a prompt over its cached prefix, a single long prompt): aiming at
// ~256 blocks with at least 4 key tiles (256 keys) per split, the longest key range (max_seqlen_k) setting the
// count.
void prefill_split_policy(int64_t blocks, int64_t max_seqlen_k, int& splits, int& split_len) {
  constexpr int64_t kCUs = 256, kMinKeys = 4 * kBK;
  splits = 1;
  split_len = int(std::min<int64_t>(std::max<int64_t>(max_seqlen_k, 1), INT32_MAX / 2));
  if (blocks <= 0 || blocks >= kCUs || max_seqlen_k < 2 * kMinKeys) return;
  const int64_t want = std::min<int64_t>(std::min<int64_t>((kCUs + blocks - 1) / blocks, max_seqlen_k / kMinKeys), 64);
  if (want < 2) return;
  int64_t len = (max_seqlen_k + want - 1) / want;
  len = (len + kBK - 1) / kBK * kBK;
  splits = int((max_seqlen_k + len - 1) / len);
  split_len = int(len);
}

int prefill_heads_per_block(int64_t Hq, int64_t Hkv) { return (Hq / Hkv) % 2 == 0 ? 2 : 1; }

int64_t prefill_workspace_bytes(int64_t num_seqs, int64_t max_seqlen_q, int64_t max_seqlen_k, int64_t Hq,
                                int64_t Hkv, int64_t D, int64_t total_q) {
  const int hb = prefill_heads_per_block(Hq, Hkv);
  const int64_t qtiles = (max_seqlen_q + block_queries(hb) - 1) / block_queries(hb);
  int splits, split_len;
  prefill_split_policy(qtiles * num_seqs * (Hq / hb), max_seqlen_k, splits, split_len);
  if (splits <= 1) return 0;
  const double bytes = double(splits) * double(total_q) * double(Hq) * record_len(int(D)) * sizeof(float);
  if (bytes > double(int64_t(1) << 40)) return 0;  // no split rather than a workspace past 1 TiB
  return int64_t(splits) * total_q * Hq * record_len(int(D)) * int64_t(sizeof(float));
}

// Queries per sequence the paged decode kernel takes in a call with a block table (0: none): sequences with at
// most 16 / G queries, unless the call has one sequence with more (nothing for that kernel then).
int64_t short_queries(int64_t num_seqs, int64_t total_q, int64_t Hq, int64_t Hkv, int64_t max_seqlen_q) {
  const int64_t G = Hq / Hkv;
  if (G > 16 || (num_seqs == 1 && total_q > 16 / G)) return 0;
  return std::min<int64_t>(16 / G, max_seqlen_q);
}

// Workspace: kAttnCounterBytes of counters (the decode attention's in-kernel merge: zero before a call, left
// zero), the prefill kernel's split records, then (16-byte aligned) the short sequences' decode records -- those of
// the paged decode kernel's splits (no longer sequence in the call), or those of the length-balanced pieces that
// the prefill kernel's blocks of the short sequences run (a longer sequence in the call).
int64_t decode_workspace_offset(int64_t prefill_bytes) { return kAttnCounterBytes + (prefill_bytes + 15) / 16 * 16; }

// The short sequences' decode attention inside the prefill launch cuts each (sequence, kv head) pair's context in
// two (halves) for at most kBalanceMaxPairs pairs (the counters): two record blocks of 16 rows per pair.
bool inline_halves(int64_t num_seqs, int64_t Hkv) { return num_seqs * Hkv <= kBalanceMaxPairs; }
int64_t inline_halves_bytes(int64_t num_seqs, int64_t Hkv, int64_t D) {
  return 2 * num_seqs * Hkv * decode_record_stride(16, D, true) * int64_t(sizeof(float));
}

int64_t total_workspace_bytes(int64_t num_seqs, int64_t max_seqlen_q, int64_t max_seqlen_k, int64_t Hq, int64_t Hkv,
                              int64_t D, int64_t total_q) {
  const int64_t pre = prefill_workspace_bytes(num_seqs, max_seqlen_q, max_seqlen_k, Hq, Hkv, D, total_q);
  const int64_t qs = short_queries(num_seqs, total_q, Hq, Hkv, max_seqlen_q);
  int64_t dec = qs > 0 ? paged_decode_varlen_workspace(num_seqs, qs, Hq, Hkv, D) : 0;
  if (qs > 0 && max_seqlen_q > qs && inline_halves(num_seqs, Hkv))
    dec = std::max(dec, inline_halves_bytes(num_seqs, Hkv, D));
  if (pre == 0 && dec == 0) return 0;
  return decode_workspace_offset(pre) + dec;
}

}  // namespace
}  // namespace nvhip

extern "C" int64_t nvhip_prefill_attention_workspace_size(int64_t num_seqs, int64_t max_seqlen_q,
                                                          int64_t max_seqlen_k, int64_t Hq, int64_t Hkv, int64_t D,
                                                          int64_t total_q) {
  if (num_seqs <= 0 || max_seqlen_q <= 0 || max_seqlen_k <= 0 || Hq < 1 || Hkv < 1 || Hq % Hkv != 0 ||
      (D != 64 && D != 128) || total_q <= 0)
    return 0;
  return nvhip::total_workspace_bytes(num_seqs, max_seqlen_q, max_seqlen_k, Hq, Hkv, D, total_q);
}

extern "C" int nvhip_prefill_attention_bf16(void* out, const void* q, const void* k, const void* v,
                                            const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                            int64_t num_seqs, int64_t max_seqlen_q, int64_t max_seqlen_k,
                                            int64_t total_q, int64_t Hq, int64_t Hkv, int64_t D,
                                            int64_t q_stride_token, int64_t q_stride_head, int64_t k_stride_token,
                                            int64_t v_stride_token, int64_t out_stride_token,
                                            int64_t out_stride_head, const int32_t* block_table, int64_t block_size,
                                            int64_t num_blocks, int64_t max_blocks, float scale, int causal,
                                            void* workspace, int64_t workspace_size, void* stream) {
  using namespace nvhip;
  clear_error();
  if (num_seqs < 0 || max_seqlen_q < 0 || max_seqlen_k < 0 || total_q < 0 || Hq < 1 || Hkv < 1)
    return invalid("prefill_attention: bad size");
  if (!(scale > 0.0f) || scale == INFINITY) return invalid("prefill_attention: softmax_scale must be positive");
  if (Hq % Hkv != 0) return invalid("prefill_attention: Hq must be a multiple of Hkv");
  if (D != 64 && D != 128) return invalid("prefill_attention: head_dim must be 64 or 128");
  if (q_stride_head < D || q_stride_token < Hq * q_stride_head || out_stride_head < D ||
      out_stride_token < Hq * out_stride_head || q_stride_head % 8 || q_stride_token % 8 || out_stride_head % 4 ||
      out_stride_token % 4)
    return invalid("prefill_attention: bad q / out strides");
  if (block_table == nullptr && (k_stride_token < Hkv * D || v_stride_token < Hkv * D || k_stride_token % 8 ||
                                 v_stride_token % 8))
    return invalid("prefill_attention: bad k / v strides");
  if (block_table != nullptr && (block_size < 1 || num_blocks < 1 || max_blocks < 1))
    return invalid("prefill_attention: bad block table shape");
  if (num_seqs == 0 || max_seqlen_q == 0 || total_q == 0) return NVHIP_OK;
  if (!out || !q || !k || !v || !cu_seqlens_q || !cu_seqlens_k) return invalid("prefill_attention: null pointer");
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || reinterpret_cast<uintptr_t>(out) % 8)
    return invalid("prefill_attention: q, k, v must be 16-byte and out 8-byte aligned");
  const int hb = prefill_heads_per_block(Hq, Hkv);  // q heads per block
  const int64_t qtiles = (max_seqlen_q + block_queries(hb) - 1) / block_queries(hb);
  if (qtiles > INT32_MAX || num_seqs > INT32_MAX || num_blocks > INT32_MAX ||
      max_blocks * block_size > INT32_MAX || max_seqlen_k > INT32_MAX / 2)
    return invalid("prefill_attention: size too large");
  PrefillArgs g{};
  g.out = static_cast<uint16_t*>(out);
  g.q = static_cast<const uint16_t*>(q);
  g.k = static_cast<const uint16_t*>(k);
  g.v = static_cast<const uint16_t*>(v);
  g.cu_q = cu_seqlens_q;
  g.cu_k = cu_seqlens_k;
  g.bt = block_table;
  g.q_st = q_stride_token;
  g.q_sh = q_stride_head;
  g.k_st = block_table ? Hkv * D : k_stride_token;
  g.v_st = block_table ? Hkv * D : v_stride_token;
  g.o_st = out_stride_token;
  g.o_sh = out_stride_head;
  g.Hkv = int(Hkv);
  g.G = int(Hq / Hkv);
  g.bs = int(block_size);
  g.num_blocks = int(num_blocks);
  g.max_blocks = int(max_blocks);
  g.scale_log2 = scale * 1.4426950408889634f;
  g.causal = causal ? 1 : 0;
  g.qtiles = int(qtiles);
  g.nhg = int(Hq / hb);
  g.lq_skip = 0;
  g.Hq = int(Hq);
  g.ws_rows = total_q;
  g.out_lines = aligned16(out) && out_stride_token % 8 == 0 && out_stride_head % 8 == 0;
  const int64_t base_blocks = qtiles * num_seqs * (Hq / hb);
  // split the keys over several blocks when the caller gave a large enough workspace
  g.splits = 1;
  g.split_len = int(std::max<int64_t>(max_seqlen_k, 1));
  const int64_t need = prefill_workspace_bytes(num_seqs, max_seqlen_q, max_seqlen_k, Hq, Hkv, D, total_q);
  if (workspace && reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
    return invalid("prefill_attention: workspace must be 256-byte aligned");
  if (need > 0 && workspace && workspace_size >= kAttnCounterBytes + need) {
    prefill_split_policy(base_blocks, max_seqlen_k, g.splits, g.split_len);
    g.ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + kAttnCounterBytes);
  }
  const int64_t blocks = base_blocks * g.splits;
  if (blocks + num_seqs * Hkv > INT32_MAX) return invalid("prefill_attention: size too large");
  const dim3 block(static_cast<unsigned>(kThreads));
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool paged = block_table != nullptr;
  // With the cache (a mixed step, a prefix-cache chunk), sequences with at most 16 / G queries -- the decode
  // requests of a mixed step -- run in the paged decode kernel, one block per (sequence, kv head) streaming its
  // keys; the prefill kernel's blocks for them return at once.
  const int64_t qs = paged ? short_queries(num_seqs, total_q, Hq, Hkv, max_seqlen_q) : 0;
  if (qs > 0) {
    g.lq_skip = int(qs);
    // its key splits use the part of the workspace after the prefill kernel's records
    const int64_t off = decode_workspace_offset(need);
    float* dws = workspace && workspace_size > off ? reinterpret_cast<float*>(static_cast<char*>(workspace) + off)
                                                   : nullptr;
    // When some sequence has more queries the prefill kernel is launched and its blocks of the short sequences run
    // their decode attention (unsplit) alongside the prefill tiles; otherwise the decode kernel runs alone, its
    // contexts split over blocks with the workspace
    const int64_t G = Hq / Hkv;
    if (max_seqlen_q > g.lq_skip && G * g.lq_skip <= 16) {
      DecodeArgs& d = g.dec;
      d.out = static_cast<uint16_t*>(out), d.q = static_cast<const uint16_t*>(q);
      d.kc = static_cast<const uint16_t*>(k), d.vc = static_cast<const uint16_t*>(v), d.bt = block_table;
      d.q_len = g.lq_skip, d.Hkv = int(Hkv), d.G = int(G), d.bs = int(block_size), d.num_blocks = int(num_blocks);
      d.max_blocks = int(max_blocks);
      d.q_st = q_stride_token, d.q_sh = q_stride_head, d.o_st = out_stride_token, d.o_sh = out_stride_head;
      d.scale_log2 = scale * 1.4426950408889634f, d.causal = causal ? 1 : 0;
      d.splits = 1, d.split_len = int(max_blocks * block_size);
      d.cu_q = cu_seqlens_q, d.cu_k = cu_seqlens_k;
      // each pair's context cut in two when the workspace holds the counters and the halves' records: the pairs
      // stream on twice the CUs (the second halves in blocks appended to the grid, which start as the short
      // sequences' idle query-tile blocks exit -- not in those blocks, which would hold back the long sequence's
      // last tiles), merged inside the launch
      if (inline_halves(num_seqs, Hkv) && dws != nullptr &&
          workspace_size - off >= inline_halves_bytes(num_seqs, Hkv, D)) {
        d.halves = 1, d.num_seqs = int(num_seqs);
        d.counters = static_cast<uint32_t*>(workspace), d.ws = dws;
        d.rec_splits = 2, d.rec_stride = decode_record_stride(16, D, true);
        g.dec_extra = int(num_seqs * Hkv);
      }
      g.dec_inline = 1;
    }
    if (!g.dec_inline) {
      return paged_decode_varlen(static_cast<uint16_t*>(out), static_cast<const uint16_t*>(q),
                                 static_cast<const uint16_t*>(k), static_cast<const uint16_t*>(v), block_table,
                                 cu_seqlens_q, cu_seqlens_k, int(num_seqs), g.lq_skip, int(Hq), int(Hkv), int(D),
                                 int(block_size), int(num_blocks), int(max_blocks), q_stride_token, q_stride_head,
                                 out_stride_token, out_stride_head, scale, causal, dws,
                                 dws ? workspace_size - off : 0, s);
    }
  }
  const dim3 grid(static_cast<unsigned>(blocks + g.dec_extra));
#define NVHIP_PREFILL_LAUNCH(DD, PG, HBV) hipLaunchKernelGGL((prefill_attention_kernel<DD, PG, HBV>), grid, block, 0, s, g)
  if (hb == 2 && D == 64 && paged) NVHIP_PREFILL_LAUNCH(64, true, 2);
  else if (hb == 2 && D == 64) NVHIP_PREFILL_LAUNCH(64, false, 2);
  else if (hb == 2 && paged) NVHIP_PREFILL_LAUNCH(128, true, 2);
  else if (hb == 2) NVHIP_PREFILL_LAUNCH(128, false, 2);
  else if (D == 64 && paged) NVHIP_PREFILL_LAUNCH(64, true, 1);
  else if (D == 64) NVHIP_PREFILL_LAUNCH(64, false, 1);
  else if (paged) NVHIP_PREFILL_LAUNCH(128, true, 1);
  else NVHIP_PREFILL_LAUNCH(128, false, 1);
#undef NVHIP_PREFILL_LAUNCH
  if (int rc = check_launch("prefill_attention")) return rc;
  if (g.splits == 1) return NVHIP_OK;
  const int64_t per_seq = (max_seqlen_q * Hq + 7) / 8;  // blocks of 4 waves of two (query, head) pairs per sequence
  if (num_seqs * per_seq > INT32_MAX) return invalid("prefill_attention: size too large");
  const dim3 cgrid(static_cast<unsigned>(num_seqs * per_seq));
  if (D == 64) hipLaunchKernelGGL((prefill_combine<64>), cgrid, dim3(256), 0, s, g, int(per_seq));
  else hipLaunchKernelGGL((prefill_combine<128>), cgrid, dim3(256), 0, s, g, int(per_seq));
  return check_launch("prefill_attention (combine)");
}
