"""A projection followed by the Add+RMSNorm that consumes it (nvhip_matmul_add_rms_norm_bf16) on the GPU: bitwise
matmul then fused_add_rms_norm where the product is not split; where it is (mixed-step and prompt-chunk rows,
N = 1024 / 2048), the split-K partial products summed by the norm kernel against the fp32 product and the two-step
result, determinism, every split count, and the decoder layer's use in the harness."""
import math

import pytest
import torch

from nanovllm_hip import _lib
from nanovllm_hip import kernels as hip

pytestmark = pytest.mark.gpu

DEV = "cuda"


def case(M, K, N, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    x = torch.randn(M, K, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(N, K, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(DEV)
    r = torch.randn(M, N, generator=g).to(torch.bfloat16).to(DEV)
    nw = (1 + 0.1 * torch.randn(N, generator=g)).to(torch.bfloat16).to(DEV)
    return x, w, r, nw


def splits(M, N, K):
    """Split count the entry point uses, read back from its workspace size (fp32 partials vs the bf16 product)."""
    ws = _lib.lib().nvhip_matmul_add_rms_norm_workspace_size(M, N, K)
    return ws // (M * N * 4) if ws >= 2 * M * N * 4 else 1


def two_step(x, w, r, nw, eps):
    return hip.fused_add_rms_norm(hip.matmul(x, w.t()), r, nw, eps)


@pytest.mark.parametrize("M,K,N", [(1, 1024, 1024), (32, 2048, 1024), (1024, 1024, 1024), (2048, 3072, 1024),
                                   (300, 1024, 3072), (64, 1000, 1024), (100, 2048, 960)])
def test_bitwise_two_steps_without_split(M, K, N):
    assert splits(M, N, K) == 1
    x, w, r, nw = case(M, K, N, seed=M + K + N)
    y, res = torch.ops.nvhip.matmul_add_rms_norm(x, w, r, nw, 1e-6)
    y_ref, res_ref = two_step(x, w, r, nw, 1e-6)
    assert torch.equal(y, y_ref) and torch.equal(res, res_ref)


@pytest.mark.parametrize("M,K,N,S", [(256, 2048, 1024, 4), (256, 3072, 1024, 4), (33, 1024, 1024, 4),
                                     (100, 3072, 1024, 4), (512, 2048, 1024, 2), (320, 3072, 1024, 3),
                                     (256, 1024, 2048, 2), (40, 2048, 4096, 4)])
def test_split_products_summed_by_the_norm(M, K, N, S):
    assert splits(M, N, K) == S
    x, w, r, nw = case(M, K, N, seed=7 * M + K + N)
    eps = 1e-6
    y, res = torch.ops.nvhip.matmul_add_rms_norm(x, w, r, nw, eps)
    y2, res2 = torch.ops.nvhip.matmul_add_rms_norm(x, w, r, nw, eps)
    assert torch.equal(y, y2) and torch.equal(res, res2)          # deterministic (fixed split order)
    # fp32 reference of the whole chain (the product rounded to bf16, as the GEMM output is)
    h = (x.float() @ w.float().t()).to(torch.bfloat16).float()
    s = h + r.float()
    torch.testing.assert_close(res.float(), s.to(torch.bfloat16).float(), rtol=1.6e-2, atol=1e-2)
    rstd = torch.rsqrt(s.pow(2).mean(-1, keepdim=True) + eps)
    y_ref = ((s * rstd).to(torch.bfloat16).float() * nw.float()).to(torch.bfloat16)
    torch.testing.assert_close(y.float(), y_ref.float(), rtol=1.6e-2, atol=1e-2)
    # the two-step result differs only by the fp32 summation order of the product: nearly all bits equal
    y_ref2, res_ref2 = two_step(x, w, r, nw, eps)
    assert (res == res_ref2).float().mean().item() > 0.95
    torch.testing.assert_close(y.float(), y_ref2.float(), rtol=1.6e-2, atol=1e-2)


def test_in_place_residual_and_wrapper():
    M, K, N = 256, 2048, 1024
    x, w, r, nw = case(M, K, N, seed=3)
    y_ref, res_ref = torch.ops.nvhip.matmul_add_rms_norm(x, w, r, nw, 1e-6)
    y, res = hip.matmul_add_rms_norm(x, w, r, nw, 1e-6)
    assert torch.equal(y, y_ref) and torch.equal(res, res_ref)
    # residual_out == residual through the C ABI
    lib = _lib.lib()
    ws = torch.empty(lib.nvhip_matmul_add_rms_norm_workspace_size(M, N, K) // 4, dtype=torch.float32, device=DEV)
    y2 = torch.empty_like(y)
    rr = r.clone()
    st = lib.nvhip_matmul_add_rms_norm_bf16(y2.data_ptr(), rr.data_ptr(), x.data_ptr(), w.data_ptr(), rr.data_ptr(),
                                            nw.data_ptr(), 1e-6, M, N, K, K, K, ws.data_ptr(), ws.numel() * 4,
                                            _lib.stream_of(x))
    _lib.check(st, "matmul_add_rms_norm")
    assert torch.equal(y2, y_ref) and torch.equal(rr, res_ref)
    # strided x (a column slice) falls back to the two steps in the wrapper
    xs = torch.randn(M, K + 8, device=DEV).to(torch.bfloat16)[:, 1:K + 1]
    y3, res3 = hip.matmul_add_rms_norm(xs, w, r, nw, 1e-6)
    y3_ref, res3_ref = two_step(xs, w, r, nw, 1e-6)
    assert torch.equal(y3, y3_ref) and torch.equal(res3, res3_ref)


def test_rejects_small_workspace_and_bad_rows():
    lib = _lib.lib()
    M, K, N = 256, 2048, 1024
    x, w, r, nw = case(M, K, N, seed=4)
    y = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    need = lib.nvhip_matmul_add_rms_norm_workspace_size(M, N, K)
    ws = torch.empty(need // 4, dtype=torch.float32, device=DEV)

    def call(ws_size=need, xs=K, k=K):
        return lib.nvhip_matmul_add_rms_norm_bf16(y.data_ptr(), r.data_ptr(), x.data_ptr(), w.data_ptr(),
                                                  r.data_ptr(), nw.data_ptr(), 1e-6, M, N, k, xs, K,
                                                  ws.data_ptr(), ws_size, _lib.stream_of(x))
    assert call(ws_size=need - 16) == _lib.NVHIP_EINVAL and b"workspace" in lib.nvhip_last_error()
    assert call(xs=K - 8) == _lib.NVHIP_EINVAL
    assert call(k=K - 4) == _lib.NVHIP_EINVAL
