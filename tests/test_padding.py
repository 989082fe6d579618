"""Padding a decode batch to its graph bucket leaves the real rows' results bitwise unchanged (GPU).

nano-vllm pads a decode batch of B sequences to the next size its graphs are recorded for (1, 2, 4, 8, then
multiples of 16; model_runner.py:27-29) with empty requests: context length 0, block-table rows of -1, slot -1.
The reference's scripts/check_padding.py asks whether that changes the real rows' results, for flash-attn's decode
call and the projections of Qwen3. Here the same question is asserted for the HIP path: the paged decode attention
(its plan is chosen for the padded batch size and empty sequences take no part in the length balance), the fused
q/k norm + RoPE + KV write + decode attention (output and both caches), the M <= 32 GEMMs (plain and with the SiLU
epilogue) and the norm-fused decode GEMMs. Those last ones reproduce torch's RMSNorm bit for bit, and torch's own
mean of squares changes its summation order with the row count (ATen's launch shape for n = 1024: 1-3, 4-7 and
>= 8 rows); where the two row counts give ATen the same launch shape the padded call must be bitwise the unpadded
one, otherwise each must be bitwise the two-launch sequence at its own size.
"""
import pytest
import torch

import oracle
from nanovllm_hip.kernels.attention import flash_attn_with_kvcache, qk_norm_rope_kv_decode_attention
from nanovllm_hip.kernels.matmul import (add_rms_norm_matmul, matmul, matmul_silu_and_mul, rms_norm_matmul)
from nanovllm_hip.kernels.rms_norm import fused_add_rms_norm, rms_norm

pytestmark = pytest.mark.gpu
DEV = "cuda"
HQ, HKV, D, BS = 16, 8, 128, 256


def bucket(b):
    """nano-vllm's graph batch sizes (model_runner.py:27-29 with max_bs 512): 1, 2, 4, 8, 16, 32, 48, ..."""
    return next(x for x in [1, 2, 4, 8] + list(range(16, 513, 16)) if x >= b)


SIZES = [(b, bucket(b)) for b in (3, 5, 9, 17, 33)]


def decode_case(b, p, seed, lens=None, width=None):
    """q for p rows, caches, a block table and context lengths whose first b rows are real requests (contexts
    U[512, 2048] unless given) and whose other rows are padding (context 0, table rows of -1)."""
    g = torch.Generator("cpu").manual_seed(seed)
    lens = torch.randint(512, 2049, (b,), generator=g).tolist() if lens is None else lens
    need = [(n + BS - 1) // BS for n in lens]
    width = max(need) if width is None else width
    nb = sum(need) + 1
    kc = torch.randn(nb, BS, HKV, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, BS, HKV, D, generator=g).to(torch.bfloat16)
    perm = torch.randperm(nb, generator=g)
    bt = torch.full((p, width), -1, dtype=torch.int32)
    used = 0
    for i, k in enumerate(need):
        bt[i, :k] = perm[used:used + k].to(torch.int32)
        used += k
    ctx = torch.tensor(lens + [0] * (p - b), dtype=torch.int32)
    return g, kc.to(DEV), vc.to(DEV), bt.to(DEV), ctx.to(DEV), lens


@pytest.mark.parametrize("b,p", SIZES)
def test_decode_attention_padding(b, p):
    g, kc, vc, bt, ctx, _ = decode_case(b, p, seed=b)
    q = torch.randn(p, 1, HQ, D, generator=g).to(torch.bfloat16).to(DEV)
    alone = flash_attn_with_kvcache(q[:b], kc, vc, ctx[:b], bt[:b], D ** -0.5, True)
    padded = flash_attn_with_kvcache(q, kc, vc, ctx, bt, D ** -0.5, True)
    torch.cuda.synchronize()
    assert torch.equal(padded[:b], alone), f"{b} -> {p}: real rows differ"
    assert torch.all(padded[b:] == 0), "padding rows must be zero"


@pytest.mark.parametrize("b,p", [(3, 4), (17, 32)])
def test_decode_attention_padding_equal_contexts(b, p):
    """The reference script's own layout: every real context 300 tokens, block tables 17 entries wide."""
    g, kc, vc, bt, ctx, _ = decode_case(b, p, seed=100 + b, lens=[300] * b, width=17)
    q = torch.randn(p, 1, HQ, D, generator=g).to(torch.bfloat16).to(DEV)
    alone = flash_attn_with_kvcache(q[:b], kc, vc, ctx[:b], bt[:b], D ** -0.5, True)
    padded = flash_attn_with_kvcache(q, kc, vc, ctx, bt, D ** -0.5, True)
    torch.cuda.synchronize()
    assert torch.equal(padded[:b], alone)


@pytest.mark.parametrize("b,p", SIZES)
def test_fused_decode_attention_padding(b, p):
    g, kc, vc, bt, ctx, lens = decode_case(b, p, seed=50 + b)
    W = (HQ + 2 * HKV) * D + 64
    qkv = torch.randn(p, W, generator=g).to(torch.bfloat16).to(DEV)
    q = qkv[:, :HQ * D].view(p, HQ, D)
    k = qkv[:, HQ * D:(HQ + HKV) * D].view(p, HKV, D)
    v = qkv[:, (HQ + HKV) * D:(HQ + 2 * HKV) * D].view(p, HKV, D)
    btc = bt.cpu()
    pos = torch.tensor([n - 1 for n in lens] + [0] * (p - b), dtype=torch.int64, device=DEV)
    slots = torch.tensor([int(btc[i, (n - 1) // BS]) * BS + (n - 1) % BS for i, n in enumerate(lens)] +
                         [-1] * (p - b), dtype=torch.int32, device=DEV)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(DEV)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(DEV)
    cs = oracle.rope_cos_sin_cache(D, 4096, 1e6).to(DEV)
    kc1, vc1, kc2, vc2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    alone = qk_norm_rope_kv_decode_attention(q[:b], k[:b], v[:b], pos[:b], qw, kw, 1e-6, cs, kc1, vc1, slots[:b],
                                             ctx[:b], bt[:b], D ** -0.5)
    padded = qk_norm_rope_kv_decode_attention(q, k, v, pos, qw, kw, 1e-6, cs, kc2, vc2, slots, ctx, bt, D ** -0.5)
    torch.cuda.synchronize()
    assert torch.equal(padded[:b], alone), f"{b} -> {p}: real rows differ"
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2), "the padded call wrote other cache rows"


GEMMS = {"qkv": (1024, 4096), "gate_up": (1024, 6144), "down": (3072, 1024), "o_proj": (2048, 1024)}


@pytest.mark.parametrize("name", list(GEMMS))
def test_decode_gemm_padding(name):
    K, N = GEMMS[name]
    g = torch.Generator("cpu").manual_seed(len(name))
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    for b, p in [(1, 1), (3, 4), (5, 8), (9, 16), (17, 32)]:
        x = torch.randn(p, K, generator=g).to(torch.bfloat16).to(DEV)
        assert torch.equal(matmul(x, w.t())[:b], matmul(x[:b], w.t())), f"{name} {b} -> {p}"
        if name == "gate_up":
            assert torch.equal(matmul_silu_and_mul(x, w)[:b], matmul_silu_and_mul(x[:b], w)), f"silu {b} -> {p}"


def same_aten_order(n, rows_a, rows_b):
    return oracle.aten_reduce.reduce_config(n, rows_a) == oracle.aten_reduce.reduce_config(n, rows_b)


@pytest.mark.parametrize("name,silu", [("qkv", False), ("gate_up", True)])
def test_norm_fused_decode_gemm_padding(name, silu):
    K, N = GEMMS[name]
    g = torch.Generator("cpu").manual_seed(7 + len(name))
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).to(DEV)
    nw = (1 + 0.1 * torch.randn(K, generator=g)).to(torch.bfloat16).to(DEV)
    prod = (lambda h: matmul_silu_and_mul(h, w)) if silu else (lambda h: matmul(h, w.t()))
    seen_same = seen_diff = False
    for b, p in [(3, 4), (5, 8), (9, 16), (17, 32)]:
        x = torch.randn(p, K, generator=g).to(torch.bfloat16).to(DEV)
        r = torch.randn(p, K, generator=g).to(torch.bfloat16).to(DEV)
        y_p = rms_norm_matmul(x, nw, 1e-6, w, silu)
        y_b = rms_norm_matmul(x[:b], nw, 1e-6, w, silu)
        z_p, res_p = add_rms_norm_matmul(x, r, nw, 1e-6, w, silu)
        z_b, res_b = add_rms_norm_matmul(x[:b], r[:b], nw, 1e-6, w, silu)
        assert torch.equal(res_p[:b], res_b)  # the new residual is an exactly rounded sum either way
        if same_aten_order(K, b, p):
            seen_same = True
            assert torch.equal(y_p[:b], y_b), f"{name} {b} -> {p}"
            assert torch.equal(z_p[:b], z_b), f"{name} add {b} -> {p}"
        else:  # torch's own RMSNorm sums the rows in another order at the two sizes: each is its two-launch result
            seen_diff = True
            for rows, y, z in ((b, y_b, z_b), (p, y_p, z_p)):
                assert torch.equal(y, prod(rms_norm(x[:rows], nw, 1e-6)))
                h, _ = fused_add_rms_norm(x[:rows], r[:rows], nw, 1e-6)
                assert torch.equal(z, prod(h))
    assert seen_same and seen_diff
