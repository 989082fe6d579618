"""SiLU-and-multiply: the HIP replacement of nanovllm/kernels/swiglu.py (same call, same output).

out = bf16(silu(fp32(gate))) * up for x = [gate | up] in the last dim (numerics of layers/activation.py:15-18,
see csrc/silu_mul.hip).
"""
import torch

import nanovllm_hip.ops  # noqa: F401  (registers torch.ops.nvhip)


def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """silu(x[..., :n]) * x[..., n:] for x [..., 2 * n] with a contiguous last dim."""
    if x.dim() != 2 or x.stride(-1) != 1:
        x = x.reshape(-1, x.shape[-1]).contiguous()
    assert x.dtype == torch.bfloat16 and x.shape[1] % 2 == 0, (x.dtype, x.shape)
    return torch.ops.nvhip.silu_and_mul(x)
