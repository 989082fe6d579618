"""GEMM C = A @ B with fp32 accumulation: the HIP replacement of nanovllm/kernels/matmul.py (same call, same output).

A [M, K], B [K, N] with any strides (e.g. B = weight.t() of an nn.Linear weight [N, K]); fp32 or bf16; C [M, N]
in A's dtype. input_precision only matters for fp32 inputs: "ieee" = fp32 products, "tf32" = inputs rounded to a
10-bit mantissa first (see csrc/gemm.hip).
"""
import torch

import nanovllm_hip.ops  # noqa: F401  (registers torch.ops.nvhip)


def matmul(a: torch.Tensor, b: torch.Tensor, input_precision: str = "ieee") -> torch.Tensor:
    """a [M, K] @ b [K, N] -> [M, N] in a's dtype."""
    assert a.ndim == 2 and b.ndim == 2 and a.shape[1] == b.shape[0], (a.shape, b.shape)
    assert a.dtype == b.dtype and a.dtype in (torch.float32, torch.bfloat16), (a.dtype, b.dtype)
    assert input_precision in ("ieee", "tf32")
    return torch.ops.nvhip.matmul(a, b, input_precision)
