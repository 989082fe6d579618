"""Fused q/k RMSNorm + RoPE + paged KV-cache write: the HIP replacement of nanovllm/kernels/qk_norm_rope_kv.py.

Same call as the reference's qk_norm_rope_kv (qk_norm_rope_kv.py:92-125), same assertions, same outputs:
  q_out [T, Hq, D]  normed + rotated q, contiguous
  k_out [T, Hkv, D] normed + rotated k if write_k, else None
  k_cache/v_cache   normed + rotated k and raw v written at slot_mapping[t] (slot -1 skipped), unless the caches
                    are empty (numel() == 0), then nothing is stored
Numerics: layers/layernorm.py rms_forward then layers/rotary_embedding.py apply_rotary_emb (see
csrc/qk_norm_rope_kv.hip). kv_per_prog and num_warps were the Triton launch knobs; they are accepted and ignored
(the HIP launch shape depends only on head_dim).
"""
import torch

import nanovllm_hip.ops  # noqa: F401  (registers torch.ops.nvhip)


def qk_norm_rope_kv(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, positions: torch.Tensor,
    q_weight: torch.Tensor, k_weight: torch.Tensor, eps: float, cos_sin_cache: torch.Tensor,
    k_cache: torch.Tensor, v_cache: torch.Tensor, slot_mapping: torch.Tensor | None, write_k: bool,
    kv_per_prog: int | None = None, num_warps: int | None = None,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """q: [T, Hq, D], k, v: [T, Hkv, D] bf16, each with contiguous heads (any token stride: views of the qkv
    output work). positions: [T] int64. cos_sin_cache: [max_pos, 1, D] fp32 (cos | sin). k_cache, v_cache:
    [blocks, block_size, Hkv, D] contiguous, or empty (nothing stored). slot_mapping: [T] int32, -1 = don't store.
    Returns (q_out, k_out or None)."""
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    assert q.dtype == k.dtype == v.dtype == torch.bfloat16 and k.shape == v.shape == (T, Hkv, D)
    assert Hq % Hkv == 0 and D in (64, 128, 256), (Hq, Hkv, D)
    for x in (q, k, v):
        assert x.stride(2) == 1 and x.stride(1) == D
    assert positions.shape == (T,) and positions.dtype == torch.int64
    assert cos_sin_cache.dtype == torch.float32 and cos_sin_cache.shape[-1] == D and cos_sin_cache.stride(-1) == 1
    assert all(s == 1 for s in cos_sin_cache.shape[1:-1]), cos_sin_cache.shape
    assert q_weight.dtype == k_weight.dtype == torch.bfloat16 and q_weight.shape == k_weight.shape == (D,)
    assert q_weight.is_contiguous() and k_weight.is_contiguous()
    store = k_cache.numel() > 0
    if store:
        assert k_cache.is_contiguous() and v_cache.is_contiguous() and k_cache.shape[-2:] == (Hkv, D)
        assert v_cache.shape == k_cache.shape and k_cache.dtype == v_cache.dtype == torch.bfloat16
        assert slot_mapping is not None and slot_mapping.shape == (T,) and slot_mapping.dtype == torch.int32
    q_out, k_out = torch.ops.nvhip.qk_norm_rope_kv(q, k, v, positions, q_weight, k_weight, float(eps), cos_sin_cache,
                                                   k_cache, v_cache, slot_mapping if store else None, bool(write_k))
    return q_out, (k_out if write_k else None)
