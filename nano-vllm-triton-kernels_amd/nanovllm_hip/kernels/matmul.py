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


def matmul_silu_and_mul(x: torch.Tensor, gate_up_weight: torch.Tensor) -> torch.Tensor:
    """silu_and_mul(matmul(x, gate_up_weight.t())) in one launch: x [M, K] bf16, gate_up_weight [2 * I, K] bf16 (the
    MergedColumnParallelLinear weight, gate rows then up rows) -> [M, I]. Bitwise the two-step result (csrc/gemm.hip
    SILU epilogue). Falls back to the two launches when the rows are not 16-byte aligned / K % 8 != 0."""
    assert x.ndim == 2 and gate_up_weight.ndim == 2 and x.shape[1] == gate_up_weight.shape[1]
    assert x.dtype == gate_up_weight.dtype == torch.bfloat16 and gate_up_weight.shape[0] % 2 == 0
    K = x.shape[1]
    ok = (x.stride(1) == 1 and gate_up_weight.stride(1) == 1 and K % 8 == 0 and x.stride(0) % 8 == 0
          and gate_up_weight.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0 and gate_up_weight.data_ptr() % 16 == 0)
    if not ok:
        from nanovllm_hip.kernels.swiglu import silu_and_mul
        return silu_and_mul(matmul(x, gate_up_weight.t()))
    return torch.ops.nvhip.matmul_silu_mul(x, gate_up_weight)
