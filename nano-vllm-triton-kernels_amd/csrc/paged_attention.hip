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
// Work split (with a caller workspace): with fewer pairs than CUs the context of each (sequence, kv head) is split
// over several blocks (whole 256-token rounds); with 256 to 512 pairs of at most 64 sequences the batch is
// balanced by length -- the longest and shortest sequences paired, the long pair's tail run by the short pair's
// block before its own context -- because one block per pair leaves the longest pairs streaming alone at the end
// (batch 32, contexts U[512, 2048]: 36.6 -> 34.8 us). The blocks of a split pair each write their merged (max,
// sum, O) record through the L2 (sc1 stores), wait for the stores and bump the pair's counter (a device-scope
// atomic); the block that completes the count reads the records with device-scope loads and merges them in split
// order, so no second launch is needed (the XCDs' L2s are not coherent with each other, and agent-scope fences --
// a write-back and an invalidate of the whole L2 -- measured 30-400 us per call; the stores, atomic and loads of
// this hand-off measured ~2.6 us at the end of the pair). Without a workspace one block covers the whole context.
// Per-block timestamps of the balanced launch show the blocks' work equal to +-8 % but their loop times spread
// 3.6-6.3 us per 256 tokens: under full load the pairs of kv heads 1 and 5 stream ~25 % slower (their 256-byte
// slices of the 2 KiB token rows sit on busier HBM channels; with kv heads and XCDs decoupled the difference
// follows the head), which a static balance cannot see.
// Tokens past the context, blocks outside [0, num_blocks) and rows past a query's causal limit take no part (their
// K/V are not read; p = 0).
#include <algorithm>
#include <mutex>
#include <string>

#include "decode_attention.h"

namespace nvhip {
namespace {

template <int D, int RP, bool ALIGNED, bool FUSE = false>
__global__ __launch_bounds__(block_waves(D) * 64) void paged_decode_kernel(const DecodeArgs g) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[decode_lds_bytes(D, RP, FUSE)];
  decode_block<D, RP, ALIGNED, FUSE>(g, blockIdx.x, lds);
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
    const float* rec = g.ws + int64_t(pair) * g.rec_splits * g.rec_stride + r * (2 + D);
    const float o = merge_splits(rec, g.rec_stride, g.splits, 2 + d);
    const int i = r / g.G, hh = r % g.G;
    g.out[int64_t(q0 + i) * g.o_st + int64_t(kvh * g.G + hh) * g.o_sh + d] = f32_to_bf16(o);
  }
}

template <int D, int RP, bool FUSE = false>
int launch_decode(const DecodeArgs& args, int64_t num_seqs, hipStream_t s) {
  DecodeArgs g = args;
  g.rec_splits = g.balance ? 2 : g.splits;
  g.rec_stride = decode_record_stride(RP, D, g.counters != nullptr);
  const int64_t blocks = num_seqs * g.Hkv * g.splits;  // balance: one block per pair (splits = 1)
  const dim3 grid(static_cast<unsigned>(blocks)), block(block_waves(D) * 64);
  if (g.bs % kChunk == 0) hipLaunchKernelGGL((paged_decode_kernel<D, RP, true, FUSE>), grid, block, 0, s, g);
  else hipLaunchKernelGGL((paged_decode_kernel<D, RP, false, FUSE>), grid, block, 0, s, g);
  if (int rc = check_launch("paged_decode_attention")) return rc;
  if (g.splits == 1 || g.counters != nullptr) return NVHIP_OK;
  hipLaunchKernelGGL((paged_decode_combine<D, RP>), dim3(unsigned(num_seqs * g.Hkv)), dim3(256), 0, s, g);
  return check_launch("paged_decode_attention (combine)");
}

template <int D>
int launch_decode_rows(const DecodeArgs& g, int64_t num_seqs, int rows, hipStream_t s) {
  if (rows <= 1) return launch_decode<D, 1>(g, num_seqs, s);
  if (rows <= 2) return launch_decode<D, 2>(g, num_seqs, s);
  if (rows <= 4) return launch_decode<D, 4>(g, num_seqs, s);
  if (rows <= 8) return launch_decode<D, 8>(g, num_seqs, s);
  return launch_decode<D, 16>(g, num_seqs, s);
}

int rows_padded(int64_t rows) { return rows <= 1 ? 1 : rows <= 2 ? 2 : rows <= 4 ? 4 : rows <= 8 ? 8 : 16; }

// The batch size a plan is chosen for: num_seqs rounded up the way nano-vllm pads a decode batch to the sizes its
// graphs are recorded for (1, 2, 4, 8, then multiples of 16; model_runner.py:27-29). A batch and the same batch
// padded with empty sequences (context 0) then get the same plan, and since empty sequences take no part in the
// length balance (balance_pieces), the real sequences' outputs are bitwise the same either way.
int64_t plan_batch(int64_t num_seqs) {
  if (num_seqs <= 2) return num_seqs;
  if (num_seqs <= 8) return num_seqs <= 4 ? 4 : 8;
  return (num_seqs + 15) / 16 * 16;
}

// Context split: only when there are fewer (sequence, kv head) pairs than CUs -- every extra block on a CU pays
// the start-up latency of its first loads again (measured: 1 -> 2 -> 4 splits of a 32-sequence batch took 42 ->
// 50 -> 56 us) -- aiming at ~256 blocks in splits of whole 256-token rounds (32 tokens per wave x 8 waves), the
// longest possible context (max_blocks * block_size) and the padded batch size (plan_batch) setting the count.
void split_policy(int64_t num_seqs, int64_t Hkv, int64_t max_ctx, int& splits, int& split_len) {
  constexpr int64_t kRound = kChunk * kWaves, kTargetBlocks = 256;
  const int64_t pairs = std::max<int64_t>(1, plan_batch(num_seqs) * Hkv);
  const int64_t want = std::max<int64_t>(1, (kTargetBlocks + pairs - 1) / pairs);
  int64_t len = std::max<int64_t>(kRound, (max_ctx + want - 1) / want);
  len = (len + kRound - 1) / kRound * kRound;
  const int64_t n = std::max<int64_t>(1, (max_ctx + len - 1) / len);
  splits = int(std::min<int64_t>(n, 1 << 16));
  split_len = int(std::min<int64_t>(len, INT32_MAX / 2));
}

// Decode calls with context lengths (not varlen), the pair counts those of the padded batch (plan_batch): fewer
// pairs than CUs -> splits x split_len (split_policy); 256 to 512 pairs of at most 64 sequences -> balance
// (length-aware: long and short sequences paired, the long pair's tail taken by the short pair's block,
// balance_pieces);
// either way the blocks of a split pair merge their records in the kernel. Workspace: kAttnCounterBytes of counters
// (zero between calls; a fixed region, so that one workspace can serve calls of any shape), then the record blocks.
struct DecodePlan {
  int splits = 1, split_len = 0, balance = 0;
  int64_t counter_bytes = 0, bytes = 0;
};
DecodePlan decode_plan(int64_t num_seqs, int64_t q_len, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_ctx) {
  DecodePlan p;
  split_policy(num_seqs, Hkv, max_ctx, p.splits, p.split_len);
  const int64_t pairs = num_seqs * Hkv, round = kChunk * block_waves(int(D)), nb = plan_batch(num_seqs);
  int64_t blocks = 0;
  if (p.splits > 1) {
    blocks = pairs * p.splits;
  } else if (nb >= 2 && nb <= 64 && nb * Hkv <= kBalanceMaxPairs && max_ctx >= 2 * round) {
    p.balance = 1;
    blocks = pairs * 2;
  }
  if (blocks == 0) return p;
  p.counter_bytes = kAttnCounterBytes;  // splits x split_len: fewer than 256 pairs; balance: at most 512
  p.bytes = p.counter_bytes + blocks * decode_record_stride(rows_padded((Hq / Hkv) * q_len), D, true) *
                                   int64_t(sizeof(float));
  return p;
}
int64_t workspace_bytes(int64_t num_seqs, int64_t q_len, int64_t Hq, int64_t Hkv, int64_t D, int64_t max_ctx) {
  return decode_plan(num_seqs, q_len, Hq, Hkv, D, max_ctx).bytes;
}
// Points g at the workspace when it is large enough (counters first, records after them).
int use_workspace(DecodeArgs& g, const DecodePlan& p, int64_t num_seqs, void* workspace, int64_t workspace_size,
                  const char* what) {
  if (p.bytes == 0 || workspace == nullptr || workspace_size < p.bytes) return NVHIP_OK;
  if (reinterpret_cast<uintptr_t>(workspace) % 256 != 0)
    return invalid(std::string(what) + ": workspace must be 256-byte aligned");
  g.splits = p.splits, g.split_len = p.split_len, g.balance = p.balance;
  g.counters = static_cast<uint32_t*>(workspace);
  g.ws = reinterpret_cast<float*>(static_cast<char*>(workspace) + p.counter_bytes);
  g.num_seqs = int(num_seqs);
  return NVHIP_OK;
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
                        hipStream_t s) {
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
  switch (D) {
    case 64: return launch_decode_rows<64>(g, num_seqs, rows, s);
    case 128: return launch_decode_rows<128>(g, num_seqs, rows, s);
    default: return launch_decode_rows<256>(g, num_seqs, rows, s);
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
  // split contexts over several blocks when the caller gave a large enough workspace
  const DecodePlan plan = decode_plan(num_seqs, q_len, Hq, Hkv, D, max_blocks * block_size);
  if (int rc = use_workspace(g, plan, num_seqs, workspace, workspace_size, "paged_decode_attention")) return rc;
  if (num_seqs * Hkv * g.splits * 2 > INT32_MAX) return invalid("paged_decode_attention: size too large");
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
  const DecodePlan plan = decode_plan(num_seqs, 1, Hq, Hkv, D, max_blocks * block_size);
  if (int rc = use_workspace(g, plan, num_seqs, workspace, workspace_size, "qk_norm_rope_kv_decode_attention"))
    return rc;
  if (num_seqs * Hkv * g.splits * 2 > INT32_MAX) return invalid("qk_norm_rope_kv_decode_attention: size too large");
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

// ------------------------------------------------------------------------------------------------------------
// Allocation-free variant: the pair counters and split records live in `scratch`, a file-scope device array (each
// GPU the library runs on holds its own copy until the process ends; zero at load, and every call leaves its
// counters zero). The plan above makes at most 2 * kBalanceMaxPairs = 1024 record blocks (2 per pair of at most 512
// pairs when balancing; fewer than 512 with splits x split_len, which needs fewer than 256 padded pairs and makes
// at most ceil(256 / padded pairs) splits), each of at most decode_record_stride(16, 256) fp32 (16 rows of
// 2 + D <= 258 floats, rounded to whole 128-byte lines: 16.1 KiB), after kAttnCounterBytes (2 KiB) of counters:
// kScratchBytes (16.1 MiB) covers every size it can choose, and a larger need is refused. In host code `scratch` is
// only a stand-in for the symbol: its device address on the current GPU comes from hipGetSymbolAddress, looked up
// once per device on the first call made with that device current, and only that address reaches the kernels.
namespace nvhip {
namespace {
constexpr int64_t kScratchRecordBlocks = 2 * kBalanceMaxPairs;
constexpr int64_t kScratchBytes =
    kAttnCounterBytes + kScratchRecordBlocks * decode_record_stride(16, 256, true) * int64_t(sizeof(float));
static_assert(kScratchBytes % 256 == 0 && kScratchBytes < (int64_t(17) << 20), "scratch size");
constexpr int kScratchDevices = 64;
}  // namespace
}  // namespace nvhip

static __device__ __align__(256) float scratch[nvhip::kScratchBytes / sizeof(float)];

namespace nvhip {
namespace {
std::mutex g_scratch_mu;
float* g_scratch_ptr[kScratchDevices] = {};

// This GPU's scratch address (the current device's), or an error code.
int scratch_address(float** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices)
    return invalid("paged_decode_attention_noalloc: no usable current device");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || p == nullptr)
      return invalid(std::string("paged_decode_attention_noalloc: hipGetSymbolAddress failed: ") +
                     hipGetErrorString(err));
    g_scratch_ptr[dev] = static_cast<float*>(p);
  }
  *ptr = g_scratch_ptr[dev];
  return NVHIP_OK;
}
}  // namespace
}  // namespace nvhip

extern "C" int nvhip_paged_decode_attention_bf16_noalloc(void* out, const void* q, const void* k_cache,
                                                         const void* v_cache, const int32_t* block_table,
                                                         const int32_t* context_lens, int64_t num_seqs,
                                                         int64_t q_len, int64_t Hq, int64_t Hkv, int64_t D,
                                                         int64_t block_size, int64_t num_blocks, int64_t max_blocks,
                                                         int64_t q_stride_token, int64_t q_stride_head,
                                                         int64_t out_stride_token, int64_t out_stride_head,
                                                         float scale, int causal, void* stream) {
  using namespace nvhip;
  clear_error();
  const int64_t need = nvhip_paged_decode_attention_workspace_size(num_seqs, q_len, Hq, Hkv, D, block_size,
                                                                   max_blocks);
  if (need > kScratchBytes)
    return invalid("paged_decode_attention_noalloc: the split records need " + std::to_string(need) +
                   " bytes, more than the " + std::to_string(kScratchBytes) + "-byte scratch");
  float* ws = nullptr;
  if (need > 0 && num_seqs > 0)
    if (int rc = scratch_address(&ws)) return rc;
  return nvhip_paged_decode_attention_bf16(out, q, k_cache, v_cache, block_table, context_lens, num_seqs, q_len, Hq,
                                           Hkv, D, block_size, num_blocks, max_blocks, q_stride_token,
                                           q_stride_head, out_stride_token, out_stride_head, scale, causal, ws, need,
                                           stream);
}
