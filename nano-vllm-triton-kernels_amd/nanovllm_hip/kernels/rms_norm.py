"""RMSNorm and Add+RMSNorm: the HIP replacement of nanovllm/kernels/rms_norm.py (same calls, same outputs).

  rms_norm(x, w, eps)                      y = bf16(x * rsqrt(mean(x^2) + eps)) * w          (rms_norm.py:83-98)
  fused_add_rms_norm(x, residual, w, eps)  (RMSNorm(x + residual), x + residual), sum in fp32 (rms_norm.py:101-111)
  fused_add_rms_norm_(x, residual, w, eps) the same with the new residual written into `residual` (no counterpart in
                                           the reference; the decoder layer never reads the old residual again)
Numerics: layers/layernorm.py:20-44 (see csrc/rms_norm.hip).
"""
import torch

import nanovllm_hip.ops  # noqa: F401  (registers torch.ops.nvhip)


def rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm over the last dim. x: [rows, n] or [T, H, n] with a contiguous last dim (any other strides)."""
    n = x.shape[-1]
    if x.dim() != 3 and x.dim() != 2 or x.stride(-1) != 1:
        x = x.reshape(-1, n).contiguous()
    assert x.dtype == w.dtype == torch.bfloat16 and w.shape == (n,) and w.is_contiguous(), (x.dtype, w.dtype, w.shape)
    return torch.ops.nvhip.rms_norm(x, w, float(eps))


def _check_add(x, residual, w):
    assert x.shape == residual.shape and x.dim() == 2 and x.stride(-1) == 1 and residual.stride(-1) == 1
    assert x.dtype == residual.dtype == w.dtype == torch.bfloat16 and w.shape == (x.shape[1],) and w.is_contiguous()


def fused_add_rms_norm(x: torch.Tensor, residual: torch.Tensor, w: torch.Tensor,
                       eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(RMSNorm(x + residual), x + residual), the sum in fp32. x, residual: [rows, n] with a contiguous last dim."""
    _check_add(x, residual, w)
    return torch.ops.nvhip.fused_add_rms_norm(x, residual, w, float(eps))


def fused_add_rms_norm_(x: torch.Tensor, residual: torch.Tensor, w: torch.Tensor,
                        eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """fused_add_rms_norm with the new residual stored in place into `residual` (which must be contiguous).
    Returns (y, residual)."""
    _check_add(x, residual, w)
    assert residual.is_contiguous()
    return torch.ops.nvhip.fused_add_rms_norm_(x, residual, w, float(eps)), residual
