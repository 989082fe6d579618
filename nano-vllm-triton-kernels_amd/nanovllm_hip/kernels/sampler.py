"""Greedy sampling: the HIP replacement of the greedy branch of Sampler.forward (nanovllm/layers/sampler.py:9-10,
`logits.float().argmax(dim=-1)`), reading the bf16 logits of the LM head directly (no fp32 copy). Same index as
torch: a NaN counts as the largest value, ties go to the smallest index. The kernel is csrc/sampler.hip.
"""
import torch

import nanovllm_hip.ops  # noqa: F401  (registers torch.ops.nvhip)


def greedy_sample(logits: torch.Tensor) -> torch.Tensor:
    """logits [num_seqs, vocab] bf16 (rows may be strided, elements contiguous) -> token ids [num_seqs] int64."""
    assert logits.dim() == 2 and logits.stride(-1) == 1, "logits must be [rows, vocab] with contiguous rows"
    assert logits.dtype == torch.bfloat16, "greedy_sample takes the bf16 logits of the LM head"
    assert logits.shape[1] > 0
    return torch.ops.nvhip.argmax(logits)
