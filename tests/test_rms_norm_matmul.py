"""The norm fused into the following decode GEMM (nvhip_rms_norm_matmul_bf16) on the GPU: bitwise the two-launch
result -- fused_add_rms_norm (or rms_norm) then matmul / matmul_silu_and_mul -- for the output and the new
residual, at the Qwen3-0.6B projections that follow a norm (qkv N = 4096, gate_up with the SiLU epilogue N = 3072)
and ragged shapes, M = 1 .. 32, K = 1024 and 2048; plus the fp64 oracle of the norm and the product, the
fallback for M > 32 and the argument checks of the entry point."""
import math

import pytest
import torch

import oracle
from nanovllm_hip import kernels as hip

pytestmark = pytest.mark.gpu

DEV = "cuda"


def case(M, K, N, silu, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    r = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    nw = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16).to(DEV)
    w = (torch.randn(2 * N if silu else N, K, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(DEV)
    return x, r, nw, w


@pytest.mark.parametrize("M", [1, 5, 16, 17, 32])
@pytest.mark.parametrize("K,N,silu", [(1024, 4096, False), (1024, 3072, True), (1024, 1000, False),
                                      (2048, 1024, False), (2048, 136, True)])
@pytest.mark.parametrize("add", [True, False])
def test_bitwise_the_two_launch_result(M, K, N, silu, add):
    x, r, nw, w = case(M, K, N, silu, seed=M * 100 + K + N + int(silu) + 7 * int(add))
    eps = 1e-6
    if add:
        h, res_ref = hip.fused_add_rms_norm(x, r, nw, eps)
    else:
        h, res_ref = hip.rms_norm(x, nw, eps), None
    ref = hip.matmul_silu_and_mul(h, w) if silu else hip.matmul(h, w.t())
    out, res = torch.ops.nvhip.rms_norm_matmul(x, r if add else None, nw, eps, w, silu)   # the fused launch itself
    torch.cuda.synchronize()
    assert out.shape == ref.shape and torch.equal(out, ref)
    if add:
        assert torch.equal(res, res_ref)


def test_wrappers_and_oracle():
    """add_rms_norm_matmul / rms_norm_matmul against the fp64 oracle of the norm and the product."""
    M, K, N = 32, 1024, 4096
    x, r, nw, w = case(M, K, N, False, seed=3)
    out, res = hip.add_rms_norm_matmul(x, r, nw, 1e-6, w)
    y_ref, res_ref = oracle.add_rms_forward(x.cpu(), r.cpu(), nw.cpu(), 1e-6)
    assert torch.equal(res.cpu(), res_ref)
    ref = oracle.matmul_fp64(y_ref, w.cpu().t())
    torch.testing.assert_close(out.cpu().double(), ref, rtol=1.6e-2, atol=1e-2)
    out2 = hip.rms_norm_matmul(x, nw, 1e-6, w)
    ref2 = oracle.matmul_fp64(oracle.rms_forward(x.cpu(), nw.cpu(), 1e-6), w.cpu().t())
    torch.testing.assert_close(out2.cpu().double(), ref2, rtol=1.6e-2, atol=1e-2)


def test_more_rows_fall_back_to_two_launches():
    x, r, nw, w = case(48, 1024, 512, True, seed=5)
    out, res = hip.add_rms_norm_matmul(x, r, nw, 1e-6, w, silu=True)
    h, res_ref = hip.fused_add_rms_norm(x, r, nw, 1e-6)
    assert torch.equal(out, hip.matmul_silu_and_mul(h, w)) and torch.equal(res, res_ref)


def test_rejects_overlapping_residual_out():
    from nanovllm_hip import _lib
    x, r, nw, w = case(8, 1024, 256, False, seed=9)
    out = torch.empty(8, 256, dtype=torch.bfloat16, device=DEV)
    status = _lib.lib().nvhip_rms_norm_matmul_bf16(out.data_ptr(), r.data_ptr(), x.data_ptr(), r.data_ptr(),
                                                   nw.data_ptr(), 1e-6, w.data_ptr(), 8, 256, 1024, 1024, 1024,
                                                   1024, 256, 0, _lib.stream_of(x))
    assert status == _lib.NVHIP_EINVAL and b"overlap" in _lib.lib().nvhip_last_error()
