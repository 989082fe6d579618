"""Unfused paged KV-cache write: the HIP replacement of store_kvcache in nanovllm/layers/attention.py:34-41.

Same call, same checks: key/value [N, Hkv, head_dim] with contiguous heads (rows may be strided views of the qkv
projection), caches whose slot rows are Hkv * head_dim contiguous elements, slot_mapping [N] int32 with -1 =
padding (skipped). The kernel is csrc/store_kvcache.hip.
"""
import torch

import nanovllm_hip.ops  # noqa: F401  (registers torch.ops.nvhip)


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor) -> None:
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == D and v_cache.stride(1) == D
    assert slot_mapping.numel() == N
    assert value.shape == key.shape and key.dtype == value.dtype == k_cache.dtype == v_cache.dtype
    assert k_cache.is_contiguous() and v_cache.is_contiguous() and k_cache.shape == v_cache.shape
    assert slot_mapping.dtype == torch.int32
    torch.ops.nvhip.store_kvcache(key, value, k_cache, v_cache, slot_mapping.contiguous())
