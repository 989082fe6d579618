"""Attention over the paged KV cache: the HIP replacements of the two flash-attn calls in nano-vllm's layers.

flash_attn_varlen_func (prefill, nanovllm/layers/attention.py:77-83): variable-length causal attention over the
new tokens' own k, v, or -- with a block table (the prefix cache, a mixed prefill + decode step) -- over the paged
caches. Kernel: csrc/prefill_attention.hip; with a block table, the sequences that bring at most 16 / (Hq / Hkv)
queries (a mixed step's decode requests) run inside the same call in the paged decode kernel.

flash_attn_with_kvcache (decode):

nanovllm/layers/attention.py:84-90 reshapes q to [num_seqs, q_len, Hq, D] and calls
    flash_attn_with_kvcache(q, k_cache, v_cache, cache_seqlens=context_lens, block_table=block_tables,
                            softmax_scale=scale, causal=True)
on the paged cache [num_blocks, block_size, Hkv, D] that the fused qk_norm_rope_kv kernel writes. The function
below takes the same arguments and returns the same [num_seqs, q_len, Hq, D] output (query i of a sequence sees the
cache up to context_len - q_len + i with causal=True; a sequence with context_len 0 gets zeros). The kernel is
csrc/paged_attention.hip.
"""
import torch

import nanovllm_hip.ops  # noqa: F401  (registers torch.ops.nvhip)


def flash_attn_with_kvcache(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                            cache_seqlens: torch.Tensor, block_table: torch.Tensor, softmax_scale: float | None = None,
                            causal: bool = False) -> torch.Tensor:
    """q [num_seqs, q_len, Hq, D] bf16 -> o [num_seqs, q_len, Hq, D] bf16, attending over the paged caches."""
    assert q.dim() == 4 and q.dtype == torch.bfloat16, (q.shape, q.dtype)
    num_seqs, q_len, Hq, D = q.shape
    assert k_cache.dim() == 4 and k_cache.shape == v_cache.shape and k_cache.shape[3] == D, (k_cache.shape, D)
    assert k_cache.dtype == v_cache.dtype == torch.bfloat16
    assert k_cache.is_contiguous() and v_cache.is_contiguous()
    assert Hq % k_cache.shape[2] == 0, (Hq, k_cache.shape[2])
    assert block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.shape[0] == num_seqs
    assert cache_seqlens.dtype == torch.int32 and cache_seqlens.shape == (num_seqs,)
    block_table = block_table.contiguous()
    cache_seqlens = cache_seqlens.contiguous()
    if q.stride(-1) != 1 or q.stride(1) != Hq * q.stride(2) or q.stride(0) != q_len * q.stride(1):
        q = q.contiguous()
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    o = torch.ops.nvhip.paged_decode_attention(q.view(num_seqs * q_len, Hq, D), k_cache, v_cache, block_table,
                                               cache_seqlens, q_len, scale, causal)
    return o.view(num_seqs, q_len, Hq, D)


paged_decode_attention = flash_attn_with_kvcache


def qk_norm_rope_kv_decode_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, positions: torch.Tensor,
                                     q_weight: torch.Tensor, k_weight: torch.Tensor, eps: float,
                                     cos_sin_cache: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                                     slot_mapping: torch.Tensor, cache_seqlens: torch.Tensor,
                                     block_table: torch.Tensor, softmax_scale: float | None = None) -> torch.Tensor:
    """One decode token per sequence: qk_norm_rope_kv(q, k, v, ...) (writing the new k / v into the caches)
    followed by flash_attn_with_kvcache(q_out, k_cache, v_cache, cache_seqlens, block_table, causal=True), in one
    launch -> o [B, Hq, D]. q [B, Hq, D], k / v [B, Hkv, D] the raw (strided) views of the qkv projection, the other
    arguments those of the two calls. The normed and rotated q / k are bitwise those of qk_norm_rope_kv and the
    output that of the two-step sequence; q_out is not written. Falls back to the two calls for layouts the fused
    kernel does not take (head_dim other than 64 / 128, unaligned rows, more than 16 q heads per kv head)."""
    from nanovllm_hip.kernels.qk_norm_rope_kv import qk_norm_rope_kv
    B, Hq, D = q.shape
    Hkv = k.shape[1]
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    cs = cos_sin_cache.reshape(cos_sin_cache.shape[0], -1)
    assert block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.shape[0] == B
    assert cache_seqlens.dtype == torch.int32 and cache_seqlens.shape == (B,)
    assert k_cache.dim() == 4 and k_cache.shape == v_cache.shape and k_cache.shape[3] == D
    assert k_cache.dtype == v_cache.dtype == torch.bfloat16
    ok = (D in (64, 128) and Hq % Hkv == 0 and Hq // Hkv <= 16 and k.shape == v.shape == (B, Hkv, D)
          and all(t.dtype == torch.bfloat16 and t.stride(2) == 1 and t.stride(1) == D and t.stride(0) % 8 == 0
                  and t.data_ptr() % 16 == 0 for t in (q, k, v))
          and q_weight.is_contiguous() and k_weight.is_contiguous() and q_weight.data_ptr() % 16 == 0
          and k_weight.data_ptr() % 16 == 0 and cs.dtype == torch.float32 and cs.stride(1) == 1
          and cs.shape[1] == D and cs.stride(0) % 4 == 0 and cs.data_ptr() % 16 == 0
          and k_cache.is_contiguous() and v_cache.is_contiguous() and k_cache.shape[2:] == (Hkv, D)
          and positions.dtype == torch.int64 and positions.shape == (B,) and slot_mapping.dtype == torch.int32
          and slot_mapping.shape == (B,) and cache_seqlens.dtype == torch.int32 and block_table.dtype == torch.int32)
    if not ok:
        q_out, _ = qk_norm_rope_kv(q, k, v, positions, q_weight, k_weight, eps, cos_sin_cache, k_cache, v_cache,
                                   slot_mapping, False)
        return flash_attn_with_kvcache(q_out.view(B, 1, Hq, D), k_cache, v_cache, cache_seqlens, block_table, scale,
                                       causal=True).view(B, Hq, D)
    return torch.ops.nvhip.qk_norm_rope_kv_decode_attention(
        q, k, v, positions.contiguous(), q_weight, k_weight, float(eps), cs, k_cache, v_cache,
        slot_mapping.contiguous(), cache_seqlens.contiguous(), block_table.contiguous(), scale)


def flash_attn_varlen_func(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, max_seqlen_q: int,
                           cu_seqlens_q: torch.Tensor, max_seqlen_k: int, cu_seqlens_k: torch.Tensor,
                           softmax_scale: float | None = None, causal: bool = False,
                           block_table: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """q [Tq, Hq, D] bf16 -> o [Tq, Hq, D]. Without block_table k, v are [Tk, Hkv, D] (the new tokens' own keys);
    with it they are the paged caches [num_blocks, block_size, Hkv, D]. Query i of a sequence with lq queries and
    lk keys sees keys j <= lk - lq + i when causal. out: an optional [Tq, Hq, D] bf16 tensor (dims contiguous,
    8-byte aligned rows) the result is written into and returned -- an addition of this package, so that a caller
    with a fixed output buffer (piecewise graphs) needs no copy."""
    assert q.dim() == 3 and q.dtype == torch.bfloat16 and q.stride(-1) == 1, (q.shape, q.dtype)
    Tq, Hq, D = q.shape
    assert k.dtype == v.dtype == torch.bfloat16 and k.shape == v.shape and k.shape[-1] == D
    assert cu_seqlens_q.dtype == cu_seqlens_k.dtype == torch.int32 and cu_seqlens_q.shape == cu_seqlens_k.shape
    if block_table is None:
        assert k.dim() == 3 and k.stride(-1) == 1 and v.stride(-1) == 1
        assert k.stride(1) == D and v.stride(1) == D, "heads of a k/v row must be contiguous"
        Hkv = k.shape[1]
    else:
        assert k.dim() == 4 and k.is_contiguous() and v.is_contiguous()
        assert block_table.dtype == torch.int32 and block_table.dim() == 2
        assert block_table.shape[0] == cu_seqlens_q.shape[0] - 1
        block_table = block_table.contiguous()
        Hkv = k.shape[2]
    assert Hq % Hkv == 0, (Hq, Hkv)
    if q.stride(1) % 8 or q.stride(0) % 8:
        q = q.contiguous()
    scale = D ** -0.5 if softmax_scale is None else float(softmax_scale)
    if out is not None:
        assert out.shape == q.shape and out.dtype == torch.bfloat16 and out.stride(2) == 1, (out.shape, out.stride())
        assert out.stride(1) % 4 == 0 and out.stride(0) % 4 == 0 and out.data_ptr() % 8 == 0
        torch.ops.nvhip.prefill_attention_out(q, k, v, cu_seqlens_q.contiguous(), cu_seqlens_k.contiguous(),
                                              int(max_seqlen_q), int(max_seqlen_k), scale, causal, block_table, out)
        return out
    return torch.ops.nvhip.prefill_attention(q, k, v, cu_seqlens_q.contiguous(), cu_seqlens_k.contiguous(),
                                             int(max_seqlen_q), int(max_seqlen_k), scale, causal, block_table)
