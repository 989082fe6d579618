"""GPU parity of the unfused paged KV write (nvhip_store_kvcache) against the oracle's store_kvcache.

The reference: nanovllm/layers/attention.py:11-41 (one program per token, skip slot -1, row of Hkv * head_dim at
slot * row). The bar is bit-exact: every written cache row equals its key/value row, every other slot keeps its
previous contents. Cases: the Qwen3-0.6B prefill batch (8192 tokens, k/v strided views of the qkv projection output,
512 blocks x 256 slots, 10 % padding), decode sizes, an odd row stride (element loop), fp32, slots outside the
cache, N = 0, graph capture and replay.
"""
import pytest
import torch

import oracle
from nanovllm_hip.kernels import store_kvcache

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make(N, Hkv=8, D=128, blocks=64, bs=256, pad=64, dtype=torch.bfloat16, seed=0, frac_pad=0.1):
    g = torch.Generator("cpu").manual_seed(seed)
    buf = torch.randn(N, (16 + 2 * Hkv) * D + pad, generator=g).to(dtype)
    k = buf[:, 16 * D:(16 + Hkv) * D].view(N, Hkv, D)
    v = buf[:, (16 + Hkv) * D:(16 + 2 * Hkv) * D].view(N, Hkv, D)
    slots = torch.randperm(blocks * bs, generator=g)[:N].to(torch.int32)
    slots[torch.rand(N, generator=g) < frac_pad] = -1
    kc = torch.randn(blocks, bs, Hkv, D, generator=g).to(dtype)
    vc = torch.randn(blocks, bs, Hkv, D, generator=g).to(dtype)
    return buf, k, v, kc, vc, slots


def check(k, v, kc, vc, slots):
    ref_k, ref_v = kc.clone(), vc.clone()
    oracle.store_kvcache(k, v, ref_k, ref_v, slots)
    dk, dv = kc.to(DEV), vc.to(DEV)
    store_kvcache(k.to(DEV) if k.is_contiguous() else k, v.to(DEV) if v.is_contiguous() else v, dk, dv,
                  slots.to(DEV))
    assert torch.equal(dk.cpu(), ref_k) and torch.equal(dv.cpu(), ref_v)


@pytest.mark.parametrize("N", [1, 32, 2048, 3001, 8192])  # 3001: the last threads of a 4-chunk stride run short
def test_qwen3_strided_views(N):
    buf, k, v, kc, vc, slots = make(N, blocks=max(64, N // 256 + 8), seed=N)
    dbuf = buf.to(DEV)
    dk = dbuf[:, 16 * 128:24 * 128].view(N, 8, 128)
    dv = dbuf[:, 24 * 128:32 * 128].view(N, 8, 128)
    ref_k, ref_v = kc.clone(), vc.clone()
    oracle.store_kvcache(k, v, ref_k, ref_v, slots)
    ck, cv = kc.to(DEV), vc.to(DEV)
    store_kvcache(dk, dv, ck, cv, slots.to(DEV))
    assert torch.equal(ck.cpu(), ref_k) and torch.equal(cv.cpu(), ref_v)


def test_odd_row_stride_takes_the_element_loop():
    g = torch.Generator("cpu").manual_seed(3)
    buf = torch.randn(100, 8 * 128 * 2 + 1, generator=g).to(torch.bfloat16)
    k = buf[:, 1:1 + 1024].view(100, 8, 128)          # stride 2049: rows not 16-byte aligned
    v = buf[:, 1 + 1024:1 + 2048].view(100, 8, 128)
    kc = torch.randn(4, 64, 8, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(4, 64, 8, 128, generator=g).to(torch.bfloat16)
    slots = torch.randperm(256, generator=g)[:100].to(torch.int32)
    ref_k, ref_v = kc.clone(), vc.clone()
    oracle.store_kvcache(k, v, ref_k, ref_v, slots)
    dbuf = buf.to(DEV)
    ck, cv = kc.to(DEV), vc.to(DEV)
    store_kvcache(dbuf[:, 1:1 + 1024].view(100, 8, 128), dbuf[:, 1 + 1024:1 + 2048].view(100, 8, 128), ck, cv,
                  slots.to(DEV))
    assert torch.equal(ck.cpu(), ref_k) and torch.equal(cv.cpu(), ref_v)


def test_fp32_and_other_head_shapes():
    _, k, v, kc, vc, slots = make(300, Hkv=2, D=64, dtype=torch.float32, seed=5)
    check(k.contiguous(), v.contiguous(), kc, vc, slots)


def test_slots_outside_the_cache_are_skipped():
    _, k, v, kc, vc, slots = make(64, seed=7, frac_pad=0.0)
    slots[::4] = 64 * 256 + 5        # past the end
    slots[1::4] = -7                 # negative, not -1
    ref_k, ref_v = kc.clone(), vc.clone()
    keep = (slots >= 0) & (slots < 64 * 256)
    oracle.store_kvcache(k[keep], v[keep], ref_k, ref_v, slots[keep])
    ck, cv = kc.to(DEV), vc.to(DEV)
    store_kvcache(k.contiguous().to(DEV), v.contiguous().to(DEV), ck, cv, slots.to(DEV))
    assert torch.equal(ck.cpu(), ref_k) and torch.equal(cv.cpu(), ref_v)


def test_empty_batch_is_a_no_op():
    kc = torch.randn(2, 16, 8, 128).to(torch.bfloat16).to(DEV)
    before = kc.clone()
    e = torch.empty(0, 8, 128, dtype=torch.bfloat16, device=DEV)
    store_kvcache(e, e, kc, kc.clone(), torch.empty(0, dtype=torch.int32, device=DEV))
    assert torch.equal(kc, before)


def test_graph_replay():
    _, k, v, kc, vc, slots = make(512, seed=9)
    ref_k, ref_v = kc.clone(), vc.clone()
    oracle.store_kvcache(k, v, ref_k, ref_v, slots)
    dk, dv, ds = k.contiguous().to(DEV), v.contiguous().to(DEV), slots.to(DEV)
    ck, cv = kc.to(DEV), vc.to(DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        store_kvcache(dk, dv, ck, cv, ds)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        store_kvcache(dk, dv, ck, cv, ds)
    for rep in range(3):
        ck.copy_(kc.to(DEV))
        cv.copy_(vc.to(DEV))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(ck.cpu(), ref_k) and torch.equal(cv.cpu(), ref_v), rep
