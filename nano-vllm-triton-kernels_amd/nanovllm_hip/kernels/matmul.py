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


def _fusable(x, residual, norm_w, weight):
    M, K = x.shape
    tensors = [x, norm_w, weight] + ([residual] if residual is not None else [])
    return (1 <= M <= 32 and K in (1024, 2048) and x.dtype == norm_w.dtype == weight.dtype == torch.bfloat16
            and all(t.stride(-1) == 1 and t.data_ptr() % 16 == 0 for t in tensors)
            and all(t.stride(0) % 8 == 0 for t in tensors if t.dim() == 2))


def rms_norm_matmul(x: torch.Tensor, norm_w: torch.Tensor, eps: float, weight: torch.Tensor,
                    silu: bool = False) -> torch.Tensor:
    """matmul(rms_norm(x, norm_w, eps), weight.t()) -- or matmul_silu_and_mul of it when silu -- in one launch for
    decode batches (x [M, K] with M <= 32, K = 1024 or 2048); weight [N, K] ([2 * I, K] with silu). Bitwise the
    two-launch result, which it falls back to for other shapes (the norm that precedes a projection,
    models/qwen3.py:166-183, moved into it)."""
    assert x.ndim == 2 and weight.ndim == 2 and x.shape[1] == weight.shape[1] and norm_w.shape == (x.shape[1],)
    if not _fusable(x, None, norm_w, weight):
        from nanovllm_hip.kernels.rms_norm import rms_norm
        h = rms_norm(x, norm_w, eps)
        return matmul_silu_and_mul(h, weight) if silu else matmul(h, weight.t())
    out, _ = torch.ops.nvhip.rms_norm_matmul(x, None, norm_w, float(eps), weight, silu)
    return out


def matmul_add_rms_norm(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor, norm_w: torch.Tensor,
                        eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """fused_add_rms_norm(matmul(x, weight.t()), residual, norm_w, eps) -> (normed, new residual): a projection
    and the Add+RMSNorm that consumes it (o_proj -> post_attention_layernorm, down_proj -> the next
    input_layernorm, models/qwen3.py:176-209). For inputs whose 64x64 tiles leave CUs idle (M of a mixed step or
    a prompt chunk, hidden 1024 / 2048 / 4096) the projection's K is split over blocks and the norm kernel sums the
    fp32 partial products before rounding them to bf16 (deterministic; equal to the two-step result up to that fp32
    summation order); otherwise bitwise the two steps. x [M, K], weight [N, K], residual [M, N], all bf16."""
    assert x.ndim == 2 and weight.ndim == 2 and x.shape[1] == weight.shape[1]
    assert residual.shape == (x.shape[0], weight.shape[0]) and norm_w.shape == (weight.shape[0],)
    K = x.shape[1]
    ok = (x.dtype == weight.dtype == residual.dtype == norm_w.dtype == torch.bfloat16 and x.stride(1) == 1
          and weight.stride(1) == 1 and K % 8 == 0 and x.stride(0) % 8 == 0 and weight.stride(0) % 8 == 0
          and residual.is_contiguous() and norm_w.is_contiguous()
          and all(t.data_ptr() % 16 == 0 for t in (x, weight, residual, norm_w)))
    if not ok:
        from nanovllm_hip.kernels.rms_norm import fused_add_rms_norm
        return fused_add_rms_norm(matmul(x, weight.t()), residual, norm_w, eps)
    return torch.ops.nvhip.matmul_add_rms_norm(x, weight, residual, norm_w, float(eps))


def add_rms_norm_matmul(x: torch.Tensor, residual: torch.Tensor, norm_w: torch.Tensor, eps: float,
                        weight: torch.Tensor, silu: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """(matmul(RMSNorm(x + residual), weight.t()), x + residual) -- the product as matmul_silu_and_mul when silu --
    in one launch for decode batches (M <= 32, K = 1024 or 2048); the new residual is a new tensor. Bitwise
    fused_add_rms_norm followed by matmul / matmul_silu_and_mul, which it falls back to for other shapes."""
    assert x.ndim == 2 and x.shape == residual.shape and weight.ndim == 2 and x.shape[1] == weight.shape[1]
    assert norm_w.shape == (x.shape[1],)
    if not _fusable(x, residual, norm_w, weight):
        from nanovllm_hip.kernels.rms_norm import fused_add_rms_norm
        h, res = fused_add_rms_norm(x, residual, norm_w, eps)
        return (matmul_silu_and_mul(h, weight) if silu else matmul(h, weight.t())), res
    return torch.ops.nvhip.rms_norm_matmul(x, residual, norm_w, float(eps), weight, silu)
