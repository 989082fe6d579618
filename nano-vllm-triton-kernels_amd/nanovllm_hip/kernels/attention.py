"""Paged decode attention: the HIP replacement of the flash_attn_with_kvcache call in nano-vllm's decode path.

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
