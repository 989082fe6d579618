/*
 * nvhip.h — C ABI of the MI355X (gfx950) kernels behind nano-vllm's kernel_backend="hip".
 *
 * One entry point per kernel family of nano-vllm's nanovllm/kernels/ package. Every entry point
 *   - takes raw device pointers, int64 sizes/strides (in elements), scalars and a hipStream_t (passed as void*);
 *   - launches asynchronously on that stream and returns 0 on success, or a negative NVHIP_E* code;
 *   - never allocates, synchronises or touches global mutable device state, so it may be recorded into a HIP graph
 *     (nvhip_paged_decode_attention_bf16_noalloc alone uses a device array of the library, see there);
 *   - on failure stores a message readable with nvhip_last_error() (thread-local, valid until the next call).
 * bf16 tensors are passed as void* holding IEEE bfloat16 values (torch.bfloat16).
 * Size 0 (T == 0, rows == 0, M*N == 0) is a valid no-op that launches nothing.
 */
#ifndef NVHIP_H
#define NVHIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NVHIP_OK 0
#define NVHIP_EINVAL -1   /* bad argument: null pointer, bad size/stride/shape, unsupported dtype */
#define NVHIP_ELAUNCH -2  /* the HIP runtime refused the launch */

#define NVHIP_DTYPE_F32 0
#define NVHIP_DTYPE_BF16 1

#define NVHIP_PREC_IEEE 0 /* fp32 inputs used as they are */
#define NVHIP_PREC_TF32 1 /* fp32 inputs rounded to a 10-bit mantissa (tf32) before the products */

/* ABI version (bumped on any signature change). */
int nvhip_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* nvhip_last_error(void);

/*
 * Fused per-head q/k RMSNorm + RoPE + paged KV-cache write (Qwen3 attention pre-segment).
 * Replaces qk_norm_rope_kv() of nanovllm/kernels/qk_norm_rope_kv.py:92-125 (its Triton kernel :45-82).
 *   q [T, Hq, D], k, v [T, Hkv, D] bf16: row t at ptr + t*{q,k,v}_stride, head h at + h*D, elements contiguous.
 *   positions [T] int64 (clamped to [0, max_pos)); cos_sin [max_pos, D] fp32 rows of (cos | sin), row stride
 *   cos_sin_stride; q_weight, k_weight [D] bf16; eps the RMSNorm epsilon.
 *   q_out [T, Hq, D] bf16 contiguous (always written).
 *   k_out [T, Hkv, D] bf16 contiguous, or NULL (= write_k False).
 *   k_cache, v_cache [num_slots, Hkv, D] bf16 contiguous (blocks x block_size slots), or both NULL (no store; then
 *   slot_mapping may be NULL). slot_mapping [T] int32: token t goes to slot slot_mapping[t]; slots outside
 *   [0, num_slots) (the padding value -1) are skipped.
 * Supported D: 64, 128, 256. Numerics: see the kernel source.
 */
int nvhip_qk_norm_rope_kv_bf16(void* q_out, void* k_out, const void* q, const void* k, const void* v,
                               int64_t q_stride, int64_t k_stride, int64_t v_stride, const int64_t* positions,
                               const int32_t* slot_mapping, const void* q_weight, const void* k_weight,
                               const float* cos_sin, int64_t cos_sin_stride, int64_t max_pos, void* k_cache,
                               void* v_cache, int64_t num_slots, int64_t T, int64_t Hq, int64_t Hkv, int64_t D,
                               float eps, void* stream);

/*
 * RMSNorm over the last dim: y = bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w).
 * Replaces rms_norm() of nanovllm/kernels/rms_norm.py:83-98 (its Triton kernel :34-54).
 *   x: groups x rows_per_group rows of n bf16; row (g, r) at x + g*group_stride + r*row_stride (elements
 *   contiguous). A 2-D [rows, n] input is groups=rows, rows_per_group=1, row_stride=0.
 *   y: [groups*rows_per_group, n] bf16 contiguous. w: [n] bf16.
 */
int nvhip_rms_norm_bf16(void* y, const void* x, const void* w, int64_t groups, int64_t rows_per_group,
                        int64_t group_stride, int64_t row_stride, int64_t n, float eps, void* stream);

/*
 * Add + RMSNorm: s = fp32(x) + fp32(residual); residual_out = bf16(s); y = bf16(bf16(s * rsqrt(mean(s^2)+eps)) * w).
 * Replaces fused_add_rms_norm() of nanovllm/kernels/rms_norm.py:101-111 (its Triton kernel :57-80).
 *   x, residual [rows, n] bf16 with row strides x_stride, r_stride (elements contiguous).
 *   y, residual_out [rows, n] bf16 contiguous. residual_out may equal residual (in place) when r_stride == n.
 */
int nvhip_add_rms_norm_bf16(void* y, void* residual_out, const void* x, const void* residual, const void* w,
                            int64_t rows, int64_t x_stride, int64_t r_stride, int64_t n, float eps, void* stream);

/*
 * SiLU x Mul: out = bf16(bf16(silu(fp32(gate))) * up), gate = x[:, :n], up = x[:, n:2n].
 * Replaces silu_and_mul() of nanovllm/kernels/swiglu.py:34-43 (its Triton kernel :19-31).
 *   x [rows, 2n] bf16, row stride x_stride (elements contiguous); out [rows, n] bf16 contiguous.
 */
int nvhip_silu_mul_bf16(void* out, const void* x, int64_t rows, int64_t x_stride, int64_t n, void* stream);

/*
 * GEMM: C[M, N] = A[M, K] @ B[K, N], fp32 accumulation, C in the input dtype (fp32 or bf16).
 * Replaces matmul() of nanovllm/kernels/matmul.py:84-99 (its Triton kernel :33-81).
 *   Element (i, j) of X lives at X + i*s_x0 + j*s_x1 (any non-negative strides, e.g. B = W.t() of a [N, K]
 *   weight: sbk = 1, sbn = K). precision: NVHIP_PREC_IEEE or NVHIP_PREC_TF32 (fp32 only; ignored for bf16).
 */
int nvhip_matmul(void* c, const void* a, const void* b, int64_t M, int64_t N, int64_t K, int64_t sam, int64_t sak,
                 int64_t sbk, int64_t sbn, int64_t scm, int64_t scn, int dtype, int precision, void* stream);

/*
 * GEMM with the SiLU x Mul epilogue (the gate_up projection of an MLP and its activation in one launch):
 * out[M, N2] = bf16(bf16(silu(bf16(A Wg^T))) * bf16(A Wu^T)), W = [Wg; Wu] of shape [2*N2, K] (an nn.Linear
 * gate_up weight), fp32 accumulation; bitwise nvhip_silu_mul_bf16 applied to the nvhip_matmul result.
 * Not in the reference's kernels (its matmul.py:3-4 plans this epilogue as the next step).
 *   A [M, K] bf16 row stride sam; W row stride swn (K-contiguous rows, K % 8 == 0, 16-byte aligned rows);
 *   out row stride som (elements contiguous).
 */
int nvhip_matmul_silu_mul_bf16(void* out, const void* a, const void* w, int64_t M, int64_t N2, int64_t K,
                               int64_t sam, int64_t swn, int64_t som, void* stream);

/*
 * RMSNorm (or Add+RMSNorm) of the rows of x fused into the projection that follows it, for decode batches
 * (1 <= M <= 32): out = matmul(norm, W^T), or with silu != 0 the SiLU x Mul epilogue of
 * nvhip_matmul_silu_mul_bf16 (W = [Wg; Wu] of shape [2N, K]), where norm = RMSNorm(x + residual) and
 * residual_out = bf16(x + residual) -- or norm = RMSNorm(x) when residual is null. One launch, bitwise
 * nvhip_add_rms_norm_bf16 / nvhip_rms_norm_bf16 followed by nvhip_matmul / nvhip_matmul_silu_mul_bf16.
 * Not in the reference's kernels: the norm that precedes a projection in models/qwen3.py:166-183
 * (input_layernorm -> qkv_proj, post_attention_layernorm -> gate_up_proj) moved into the projection.
 *   x [M, K] row stride sx; residual [M, K] row stride sr, or null (then residual_out is null too);
 *   residual_out [M, K] contiguous, not overlapping x or residual (every block reads them); norm_w [K];
 *   W [N or 2N, K] row stride swn; out [M, N] row stride som. K = 1024 or 2048; 16-byte aligned, K-contiguous
 *   rows; row strides multiples of 8. Anything else is rejected (NVHIP_EINVAL): run the two launches.
 */
int nvhip_rms_norm_matmul_bf16(void* out, void* residual_out, const void* x, const void* residual,
                               const void* norm_w, float eps, const void* w, int64_t M, int64_t N, int64_t K,
                               int64_t sx, int64_t sr, int64_t swn, int64_t som, int silu, void* stream);

/*
 * Paged KV-cache write (unfused).
 * Replaces store_kvcache() of nanovllm/layers/attention.py:34-41 (its Triton kernel :11-31).
 *   key, value: n rows of row_elems elements (Hkv * head_dim) at ptr + t*stride (elements contiguous).
 *   k_cache, v_cache: [num_slots, row_elems] contiguous (blocks x block_size slots). Row t goes to slot
 *   slot_mapping[t] (int32); slots outside [0, num_slots) (the padding value -1) are skipped.
 *   elem_size: 2 (bf16 / fp16) or 4 (fp32) bytes; the bits are copied unchanged.
 */
int nvhip_store_kvcache(void* k_cache, void* v_cache, const void* key, const void* value, int64_t key_stride,
                        int64_t value_stride, const int32_t* slot_mapping, int64_t num_slots, int64_t n,
                        int64_t row_elems, int64_t elem_size, void* stream);

/*
 * Paged decode attention over the KV cache that nvhip_qk_norm_rope_kv_bf16 writes.
 * Replaces flash_attn_with_kvcache(q, k_cache, v_cache, cache_seqlens=context_lens, block_table=block_table,
 * softmax_scale=scale, causal=True) as called at nanovllm/layers/attention.py:84-90 (decode branch).
 *   q, out: [num_seqs * q_len, Hq, D] bf16; token b*q_len + i, head h at ptr + token*stride_token + h*stride_head,
 *   elements contiguous (16-byte aligned rows). k_cache, v_cache: [num_blocks, block_size, Hkv, D] bf16 contiguous.
 *   block_table: [num_seqs, max_blocks] int32 (entries past a sequence's blocks unused; -1 padding allowed).
 *   context_lens: [num_seqs] int32 cache tokens per sequence, including the q_len new ones (0 = padding: zero
 *   output). Query i sees cache tokens < context_len - q_len + i + 1 when causal, all context_len otherwise.
 *   Blocks outside [0, num_blocks) are skipped. D: 64, 128, 256; (Hq / Hkv) * q_len <= 16 (8 for D = 256).
 *   workspace: device memory of at least nvhip_paged_decode_attention_workspace_size(...) bytes, 256-byte
 *   aligned, ZERO-FILLED before its first use (its first 2 KiB are per-(sequence, kv head) counters; every call
 *   leaves them zero again, so a workspace is zeroed once and kept; calls that share it must be ordered on one
 *   stream). With it, fewer (sequence, kv head) pairs than CUs split each context over several blocks, and 256 to
 *   512 pairs of at most 64 sequences are balanced by length (the longest and shortest sequences paired, the
 *   long pair's tail taken by the short pair's block); the blocks of a split pair merge their (max, sum, O)
 *   records themselves, in split order (the last to finish, found with a device-scope counter). NULL (or too
 *   small) runs one block per (sequence, kv head).
 * Numerics: fp32 scores and softmax (exp2 with the scale folded in), fp32 P*V accumulation, bf16 output.
 */
int nvhip_paged_decode_attention_bf16(void* out, const void* q, const void* k_cache, const void* v_cache,
                                      const int32_t* block_table, const int32_t* context_lens, int64_t num_seqs,
                                      int64_t q_len, int64_t Hq, int64_t Hkv, int64_t D, int64_t block_size,
                                      int64_t num_blocks, int64_t max_blocks, int64_t q_stride_token,
                                      int64_t q_stride_head, int64_t out_stride_token, int64_t out_stride_head,
                                      float scale, int causal, void* workspace, int64_t workspace_size,
                                      void* stream);

/*
 * nvhip_paged_decode_attention_bf16 without a workspace argument and without any allocation: the pair counters and
 * split records go to a device array of this library (16.1 MiB per GPU, zero at load, held until the process ends;
 * its address on the current device is looked up once per device with hipGetSymbolAddress). No counterpart in the
 * reference: for callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments, plan and results as nvhip_paged_decode_attention_bf16 given a
 * zero-filled workspace of nvhip_paged_decode_attention_workspace_size(...) bytes; a need beyond the array is
 * refused (NVHIP_EINVAL; the plan never asks for more). All calls on one GPU share the array: calls that overlap in
 * time on one GPU (different streams without ordering) race on it. Every call leaves the counters zero.
 */
int nvhip_paged_decode_attention_bf16_noalloc(void* out, const void* q, const void* k_cache, const void* v_cache,
                                              const int32_t* block_table, const int32_t* context_lens,
                                              int64_t num_seqs, int64_t q_len, int64_t Hq, int64_t Hkv, int64_t D,
                                              int64_t block_size, int64_t num_blocks, int64_t max_blocks,
                                              int64_t q_stride_token, int64_t q_stride_head,
                                              int64_t out_stride_token, int64_t out_stride_head, float scale,
                                              int causal, void* stream);

/*
 * Variable-length (prefill) attention.
 * Replaces flash_attn_varlen_func(q, k, v, max_seqlen_q, cu_seqlens_q, max_seqlen_k, cu_seqlens_k, softmax_scale,
 * causal, block_table) as called at nanovllm/layers/attention.py:77-83 (prefill branch).
 *   q, out: [total_q, Hq, D] bf16 (token / head strides in elements, rows of D contiguous); sequence b owns tokens
 *   cu_seqlens_q[b] .. cu_seqlens_q[b+1]-1 (int32 [num_seqs + 1]); max_seqlen_q bounds their count.
 *   Keys of sequence b: lk = cu_seqlens_k[b+1] - cu_seqlens_k[b] (max_seqlen_k bounds it). Without a block table,
 *   key j is row cu_seqlens_k[b] + j of k, v [Tk, Hkv, D] (token strides k_stride_token, v_stride_token). With a
 *   block table ([num_seqs, max_blocks] int32, prefix cache / mixed steps), k and v are the paged caches
 *   [num_blocks, block_size, Hkv, D] and key j is slot block_table[b][j / block_size] * block_size + j % block_size
 *   (invalid blocks are skipped); then sequences with at most 16 / (Hq / Hkv) queries (decode requests of a mixed
 *   step) are computed by the paged decode kernel inside this call.
 *   Query i of a sequence with lq queries sees keys j <= lk - lq + i when causal, all lk otherwise; a query that
 *   sees no key gets zeros. Head h reads kv head h / (Hq / Hkv). D: 64, 128.
 *   workspace: device memory of at least nvhip_prefill_attention_workspace_size(...) bytes, 256-byte aligned,
 *   whose first 2 KiB are ZERO before its first use (the counters of the decode attention's in-kernel merge; every
 *   call leaves them zero, and the same workspace may serve nvhip_paged_decode_attention_bf16 calls), or NULL /
 *   too small: then the keys of a sequence are never split over blocks. With it, few query tiles over long key
 *   ranges (a prompt chunk over its cached prefix) are spread over the CUs in key ranges whose partial results a
 *   second kernel merges; with a block table and only short sequences, their contexts are split as
 *   nvhip_paged_decode_attention_bf16 splits them (fewer (sequence, kv head) pairs than CUs); with short sequences
 *   beside longer ones (a mixed step) each short (sequence, kv head) context is cut in two halves, the second ones
 *   in blocks appended to the launch, merged inside it. Calls that share a workspace must be ordered on one stream.
 * Numerics: fp32 scores and online softmax, P rounded to bf16 for P.V (as flash-attn), fp32 accumulation, bf16 out.
 */
int nvhip_prefill_attention_bf16(void* out, const void* q, const void* k, const void* v, const int32_t* cu_seqlens_q,
                                 const int32_t* cu_seqlens_k, int64_t num_seqs, int64_t max_seqlen_q,
                                 int64_t max_seqlen_k, int64_t total_q, int64_t Hq, int64_t Hkv, int64_t D,
                                 int64_t q_stride_token, int64_t q_stride_head, int64_t k_stride_token,
                                 int64_t v_stride_token, int64_t out_stride_token, int64_t out_stride_head,
                                 const int32_t* block_table, int64_t block_size, int64_t num_blocks,
                                 int64_t max_blocks, float scale, int causal, void* workspace,
                                 int64_t workspace_size, void* stream);

/*
 * Bytes of workspace nvhip_prefill_attention_bf16 uses for these sizes (0: it does not split). Host-only, no GPU
 * work. An addition of this library (flash-attn allocates its own split buffers).
 */
int64_t nvhip_prefill_attention_workspace_size(int64_t num_seqs, int64_t max_seqlen_q, int64_t max_seqlen_k,
                                               int64_t Hq, int64_t Hkv, int64_t D, int64_t total_q);

/*
 * Bytes of workspace nvhip_paged_decode_attention_bf16 uses for these sizes (0: one block per (sequence, kv head)).
 * Host-only, no GPU work. An addition of this library (the reference has no workspace: flash-attn allocates its
 * own).
 */
int64_t nvhip_paged_decode_attention_workspace_size(int64_t num_seqs, int64_t q_len, int64_t Hq, int64_t Hkv,
                                                    int64_t D, int64_t block_size, int64_t max_blocks);

/*
 * A projection followed by the Add+RMSNorm that consumes it (o_proj -> post_attention_layernorm, down_proj -> the
 * next layer's input_layernorm in models/qwen3.py:176-209): h = bf16(x W^T), s = fp32(h) + fp32(residual),
 * residual_out = bf16(s), y = bf16(bf16(s * rstd) * norm_w) -- nvhip_matmul then nvhip_add_rms_norm_bf16.
 * Not in the reference's kernels: the epilogue side of the GEMM fusions of matmul.py:3-4, for the longer inputs of
 * mixed steps and prompt chunks (M > 32). When the product's 64x64 tiles leave CUs idle (N = 1024 / 2048 / 4096,
 * M up to a few hundred) its K is split over up to 4 block ranges whose fp32 partial products the norm kernel sums
 * in split order before rounding h to bf16: no extra launch, and h then differs from nvhip_matmul's only by that
 * summation order (within fp32 rounding; deterministic). Otherwise the two launches, bitwise.
 *   x [M, K] row stride x_stride, W [N, K] row stride w_stride (K-contiguous, 16-byte aligned rows, K % 8 == 0);
 *   residual, residual_out and y [M, N] contiguous, 16-byte aligned (residual_out may be residual); norm_w [N].
 *   workspace: at least nvhip_matmul_add_rms_norm_workspace_size(M, N, K) bytes, 16-byte aligned (required;
 *   contents need no initialisation). Calls that share a workspace must be ordered on one stream.
 */
int nvhip_matmul_add_rms_norm_bf16(void* y, void* residual_out, const void* x, const void* weight,
                                   const void* residual, const void* norm_w, float eps, int64_t M, int64_t N,
                                   int64_t K, int64_t x_stride, int64_t w_stride, void* workspace,
                                   int64_t workspace_size, void* stream);

/* Bytes of workspace nvhip_matmul_add_rms_norm_bf16 needs for these sizes. Host-only, no GPU work. */
int64_t nvhip_matmul_add_rms_norm_workspace_size(int64_t M, int64_t N, int64_t K);

/*
 * Decode with one token per sequence: nvhip_qk_norm_rope_kv_bf16 (q_out not written, no k_out) followed by
 * nvhip_paged_decode_attention_bf16 (q_len 1, causal), in one launch. Not in the reference's kernels: its decode
 * step runs qk_norm_rope_kv.py:92-125 and then flash_attn_with_kvcache (layers/attention.py:84-90) on the result.
 * Each attention block (sequence b, kv head h) normalises and rotates its q rows with the arithmetic of the fused
 * kernel (the same bits) and the block whose key range holds the new token (position context_lens[b] - 1) writes
 * the new key (normed, rotated) and value of head h into slot slot_mapping[b] (skipped outside [0, num_blocks *
 * block_size)) before it reads the cache; the output is bitwise that of the two calls when slot_mapping[b] is
 * the slot of sequence b's position context_lens[b] - 1 in its block table (as every decode step builds it). A slot
 * outside that layout is still written, but ordered before the reads of the writing block only: another block that
 * reads it in the same launch (another context split or balanced piece of the pair, another sequence) may see the
 * old row.
 *   q [num_seqs, Hq, D], k, v [num_seqs, Hkv, D]: the raw rows of the qkv projection (token strides q_stride,
 *   k_stride, v_stride, multiples of 8; heads contiguous; 16-byte aligned). positions int64, slot_mapping int32
 *   [num_seqs]; q_weight, k_weight [D]; cos_sin [max_pos, cos_sin_stride] fp32 (cos | sin); caches, block_table,
 *   context_lens, out, scale and workspace (nvhip_paged_decode_attention_workspace_size with q_len 1) as for
 *   nvhip_paged_decode_attention_bf16. D: 64 or 128; Hq / Hkv <= 16.
 */
int nvhip_qk_norm_rope_kv_decode_attention_bf16(
    void* out, const void* q, const void* k, const void* v, int64_t q_stride, int64_t k_stride, int64_t v_stride,
    const int64_t* positions, const int32_t* slot_mapping, const void* q_weight, const void* k_weight,
    const float* cos_sin, int64_t cos_sin_stride, int64_t max_pos, float eps, void* k_cache, void* v_cache,
    const int32_t* block_table, const int32_t* context_lens, int64_t num_seqs, int64_t Hq, int64_t Hkv, int64_t D,
    int64_t block_size, int64_t num_blocks, int64_t max_blocks, int64_t out_stride_token, int64_t out_stride_head,
    float scale, void* workspace, int64_t workspace_size, void* stream);

/*
 * Greedy sampling: out[r] = the index of the largest of logits[r, 0 .. n) (int64), for bf16 logits with row
 * stride row_stride (elements). Replaces the greedy branch of Sampler.forward (nanovllm/layers/sampler.py:9-10,
 * logits.float().argmax(dim=-1)) and returns the same index: a NaN counts as the largest value, ties go to the
 * smallest index. rows < 65536. workspace (16-byte aligned, contents need no initialisation) of
 * nvhip_argmax_workspace_size(rows, n) bytes lets each row be split over several blocks and merged by a second
 * launch; with a NULL (or too small) workspace one block reads each row.
 */
int64_t nvhip_argmax_workspace_size(int64_t rows, int64_t n);
int nvhip_argmax_bf16(int64_t* out, const void* logits, int64_t rows, int64_t n, int64_t row_stride,
                      void* workspace, int64_t workspace_size, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NVHIP_H */
