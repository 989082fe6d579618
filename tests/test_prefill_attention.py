"""GPU parity of the prefill (varlen) attention (nvhip_prefill_attention_bf16) against the oracle.

The oracle restates flash_attn_varlen_func as nanovllm/layers/attention.py:77-83 calls it (fp32 from the same bf16
inputs). The kernel rounds P to bf16 for P.V (as flash-attn does); tolerance: the bf16 output tolerance rtol 1.6e-2,
atol 1e-2. Cases: a Qwen3-0.6B prefill batch (16 q / 8 kv heads, head_dim 128, k and v strided views of the qkv
projection output), the prefix cache (keys through a block table of 256- and 16-slot blocks, NaN in unused slots),
head_dim 64, GQA ratios 1 / 4 / 8, non-causal, more queries than keys (rows that see nothing are zero), an empty
sequence, graph capture and replay; mixed steps over the cache, whose sequences with <= 16 / G queries run in the
paged decode kernel (bitwise the decode attention's rows for one-query sequences); chunks over long prefixes and
long prompts whose keys are split over blocks and merged (with and without the cache, causal and not, in graphs);
seeded random batches over the cache.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import paged_decode_abi
from nanovllm_hip.kernels.attention import flash_attn_varlen_func

pytestmark = pytest.mark.gpu
DEV = "cuda"


def cu(lens):
    return torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32)


def contiguous_case(lens, Hq=16, Hkv=8, D=128, seed=0, pad=64):
    g = torch.Generator("cpu").manual_seed(seed)
    T = sum(lens)
    buf = torch.randn(T, (Hq + 2 * Hkv) * D + pad, generator=g).to(torch.bfloat16)
    q = buf[:, :Hq * D].view(T, Hq, D)
    k = buf[:, Hq * D:(Hq + Hkv) * D].view(T, Hkv, D)
    v = buf[:, (Hq + Hkv) * D:(Hq + 2 * Hkv) * D].view(T, Hkv, D)
    return buf, q, k, v


def check(q, k, v, cq, ck, causal=True, block_table=None, scale=None):
    D = q.shape[-1]
    scale = D ** -0.5 if scale is None else scale
    lq = (cq[1:] - cq[:-1]).tolist()
    lk = (ck[1:] - ck[:-1]).tolist()
    out = flash_attn_varlen_func(q.to(DEV), k.to(DEV), v.to(DEV), max(lq), cq.to(DEV), max(lk), ck.to(DEV), scale,
                                 causal, None if block_table is None else block_table.to(DEV))
    ref = oracle.varlen_attention(q, k, v, cq, ck, scale, causal, block_table)
    out = out.cpu()
    assert out.shape == q.shape and torch.isfinite(out.float()).all()
    torch.testing.assert_close(out.float(), ref.float(), rtol=1.6e-2, atol=1e-2)
    return out, ref


def test_qwen3_prefill_batch_strided_views():
    lens = [100, 300, 513, 1000]
    buf, q, k, v = contiguous_case(lens, seed=1)
    dbuf = buf.to(DEV)
    T = sum(lens)
    dq = dbuf[:, :2048].view(T, 16, 128)
    dk = dbuf[:, 2048:3072].view(T, 8, 128)
    dv = dbuf[:, 3072:4096].view(T, 8, 128)
    cq = cu(lens)
    out = flash_attn_varlen_func(dq, dk, dv, 1000, cq.to(DEV), 1000, cq.to(DEV), 128 ** -0.5, True)
    ref = oracle.varlen_attention(q, k, v, cq, cq, 128 ** -0.5, True)
    torch.testing.assert_close(out.cpu().float(), ref.float(), rtol=1.6e-2, atol=1e-2)


@pytest.mark.parametrize("lens", [[1], [63, 64, 65], [2, 129, 31, 250]])
def test_lengths_around_tiles(lens):
    _, q, k, v = contiguous_case(lens, seed=len(lens))
    check(q.contiguous(), k.contiguous(), v.contiguous(), cu(lens), cu(lens))


@pytest.mark.parametrize("block_size", [256, 16])
def test_prefix_cache_block_table(block_size):
    """lq new tokens attend over lk >= lq cached keys read through the block table (NaN in unused slots)."""
    g = torch.Generator("cpu").manual_seed(block_size)
    lq, lk = [37, 1, 200], [300, 70, 200]
    Hq, Hkv, D = 16, 8, 128
    nb = sum((n + block_size - 1) // block_size for n in lk) + 3
    kc = torch.full((nb, block_size, Hkv, D), float("nan")).to(torch.bfloat16)
    vc = kc.clone()
    perm = torch.randperm(nb, generator=g)
    maxb = max((n + block_size - 1) // block_size for n in lk)
    bt = torch.full((3, maxb), -1, dtype=torch.int32)
    used = 0
    for b, n in enumerate(lk):
        for c in range((n + block_size - 1) // block_size):
            blk = int(perm[used]); used += 1
            bt[b, c] = blk
            cnt = min(n - c * block_size, block_size)
            kc[blk, :cnt] = torch.randn(cnt, Hkv, D, generator=g).to(torch.bfloat16)
            vc[blk, :cnt] = torch.randn(cnt, Hkv, D, generator=g).to(torch.bfloat16)
    q = torch.randn(sum(lq), Hq, D, generator=g).to(torch.bfloat16)
    check(q, kc, vc, cu(lq), cu(lk), True, bt)


def paged_case(lq, lk, block_size, Hq=16, Hkv=8, D=128, seed=0):
    """q [sum(lq), Hq, D] and paged caches holding lk[b] keys of sequence b through a random block table (NaN in
    the unused slots)."""
    g = torch.Generator("cpu").manual_seed(seed)
    nb = sum((n + block_size - 1) // block_size for n in lk) + 3
    kc = torch.full((nb, block_size, Hkv, D), float("nan")).to(torch.bfloat16)
    vc = kc.clone()
    perm = torch.randperm(nb, generator=g)
    maxb = max(max((n + block_size - 1) // block_size for n in lk), 1)
    bt = torch.full((len(lk), maxb), -1, dtype=torch.int32)
    used = 0
    for b, n in enumerate(lk):
        for c in range((n + block_size - 1) // block_size):
            blk = int(perm[used]); used += 1
            bt[b, c] = blk
            cnt = min(n - c * block_size, block_size)
            kc[blk, :cnt] = torch.randn(cnt, Hkv, D, generator=g).to(torch.bfloat16)
            vc[blk, :cnt] = torch.randn(cnt, Hkv, D, generator=g).to(torch.bfloat16)
    q = torch.randn(sum(lq), Hq, D, generator=g).to(torch.bfloat16)
    return q, kc, vc, bt


@pytest.mark.parametrize("block_size", [256, 16])
def test_mixed_step_short_sequences(block_size):
    """A mixed step: decode requests (1 query), short runs of 2 .. 9 queries and prefill chunks over the cache.
    Sequences with <= 16 / G queries (8 here) take the paged decode kernel, the rest the prefill kernel; an
    empty sequence and one with no cached keys are in the batch too."""
    lq = [1, 1, 40, 1, 3, 8, 9, 1, 0, 130, 2]
    lk = [700, 1, 300, 1500, 90, 8, 1000, 257, 0, 130, 0]
    q, kc, vc, bt = paged_case(lq, lk, block_size, seed=block_size + 1)
    out, _ = check(q, kc, vc, cu(lq), cu(lk), True, bt)
    assert torch.all(out[-2:] == 0)     # the last sequence has no keys


def test_decode_only_varlen_equals_decode_attention():
    """Every sequence with one query: the varlen call runs only the paged decode kernel, whose rows are bitwise
    those of the decode entry point with one block per (sequence, kv head) (32 sequences x 8 kv heads: the varlen
    call does not split the contexts), and within the bf16 tolerance of flash_attn_with_kvcache, which balances the
    long and short contexts of such a batch over the blocks."""
    from nanovllm_hip.kernels.attention import flash_attn_with_kvcache
    g = torch.Generator("cpu").manual_seed(12)
    lk = torch.randint(1, 2049, (32,), generator=g).tolist()
    lq = [1] * len(lk)
    q, kc, vc, bt = paged_case(lq, lk, 256, seed=11)
    out, _ = check(q, kc, vc, cu(lq), cu(lk), True, bt)
    lens = torch.tensor(lk, dtype=torch.int32, device=DEV)
    qd = q.to(DEV).view(len(lk), 1, 16, 128)
    single, _ = paged_decode_abi(qd, kc.to(DEV), vc.to(DEV), lens, bt.to(DEV), 128 ** -0.5, True, workspace=False)
    assert torch.equal(out, single.view(-1, 16, 128).cpu())
    dec = flash_attn_with_kvcache(qd, kc.to(DEV), vc.to(DEV), lens, bt.to(DEV), 128 ** -0.5, causal=True)
    torch.testing.assert_close(dec.view(-1, 16, 128).cpu().float(), out.float(), rtol=1.6e-2, atol=1e-2)


def test_few_decode_sequences_split_like_the_decode_call():
    """5 one-query sequences (40 (sequence, kv head) pairs, fewer than the CUs): the varlen call's short-sequence
    path splits the contexts over blocks with the decode call's policy and workspace layout, so its rows stay
    bitwise those of flash_attn_with_kvcache, which splits them too."""
    from nanovllm_hip.kernels.attention import flash_attn_with_kvcache
    lk = [2000, 37, 1025, 512, 1800]
    lq = [1] * len(lk)
    q, kc, vc, bt = paged_case(lq, lk, 256, seed=13)
    out, _ = check(q, kc, vc, cu(lq), cu(lk), True, bt)
    dec = flash_attn_with_kvcache(q.to(DEV).view(len(lk), 1, 16, 128), kc.to(DEV), vc.to(DEV),
                                  torch.tensor(lk, dtype=torch.int32, device=DEV), bt.to(DEV), 128 ** -0.5,
                                  causal=True)
    assert torch.equal(out, dec.view(-1, 16, 128).cpu())


def test_out_buffer_gets_the_same_rows():
    """out= writes the result into a caller's buffer (a view of a larger one here) with the bits of the returned
    tensor, for the prefill kernel's and the short-sequence path's rows."""
    from nanovllm_hip.kernels.attention import flash_attn_varlen_func
    lq, lk = [1, 40, 1, 3], [700, 300, 1500, 90]
    q, kc, vc, bt = paged_case(lq, lk, 256, seed=14)
    q, kc, vc, bt = q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV)
    cq, ck = cu(lq).to(DEV), cu(lk).to(DEV)
    want = flash_attn_varlen_func(q, kc, vc, max(lq), cq, max(lk), ck, 128 ** -0.5, True, bt)
    buf = torch.full((q.shape[0] + 5, 16, 128), 7.0, dtype=torch.bfloat16, device=DEV)
    got = flash_attn_varlen_func(q, kc, vc, max(lq), cq, max(lk), ck, 128 ** -0.5, True, bt, out=buf[2:2 + q.shape[0]])
    assert got.data_ptr() == buf[2:].data_ptr() and torch.equal(got, want)
    assert torch.all(buf[:2] == 7) and torch.all(buf[2 + q.shape[0]:] == 7)


@pytest.mark.parametrize("layout", ["head_stride_132", "offset_8_bytes"])
def test_out_not_in_16_byte_pieces(layout):
    """An out buffer whose rows do not start on 16-byte boundaries (head stride 132, or the whole view 8 bytes off)
    takes the kernel's per-lane 8-byte stores instead of the rows staged through the LDS and stored as whole lines:
    the same bits either way, for contiguous keys (causal, partial query tiles) and for keys split over blocks."""
    for split in (False, True):
        if split:
            lq, lk = [256], [4096]
            q, kc, vc, bt = paged_case(lq, lk, 256, seed=21)
            args = (max(lq), cu(lq).to(DEV), max(lk), cu(lk).to(DEV), 128 ** -0.5, True, bt.to(DEV))
            q, k, v = q.to(DEV), kc.to(DEV), vc.to(DEV)
        else:
            lens = [70, 300, 129]
            _, q, k, v = contiguous_case(lens, seed=22)
            q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
            args = (max(lens), cu(lens).to(DEV), max(lens), cu(lens).to(DEV), 128 ** -0.5, True)
        want = flash_attn_varlen_func(q, k, v, *args)
        T = q.shape[0]
        if layout == "head_stride_132":
            buf = torch.full((T, 16, 132), 7.0, dtype=torch.bfloat16, device=DEV)
            out = buf[:, :, :128]
        else:
            buf = torch.full((T * 16 * 128 + 4,), 7.0, dtype=torch.bfloat16, device=DEV)
            out = buf[4:].view(T, 16, 128)
            assert out.data_ptr() % 16 == 8
        got = flash_attn_varlen_func(q, k, v, *args, out=out)
        assert got.data_ptr() == out.data_ptr() and torch.equal(got, want)
        if layout == "head_stride_132":
            assert torch.all(buf[:, :, 128:] == 7)
        else:
            assert torch.all(buf[:4] == 7)


def test_chunk_over_a_long_prefix_splits_the_keys():
    """A 256-token chunk over 3840 cached keys: 16 blocks would stream 4096 keys each, so the call splits the keys
    into 16 ranges (256 blocks) and merges them (workspace query pinned on the CPU)."""
    from nanovllm_hip import _lib
    assert _lib.lib().nvhip_prefill_attention_workspace_size(1, 256, 4096, 16, 8, 128, 256) > 0
    q, kc, vc, bt = paged_case([256], [4096], 256, seed=21)
    check(q, kc, vc, cu([256]), cu([4096]), True, bt)


def test_split_keys_with_decode_rows_and_causal_limits():
    """Key splits together with the short-sequence path in one call over the cache: one-query sequences, a chunk
    over a long prefix and a sequence whose later splits see no key for its first queries."""
    lq = [1, 1, 300, 1, 40]
    lk = [900, 50, 3000, 2000, 1200]
    q, kc, vc, bt = paged_case(lq, lk, 16, seed=22)
    check(q, kc, vc, cu(lq), cu(lk), True, bt)


def test_split_keys_without_cache_non_causal_and_head_dim_64():
    # one fresh 1100-token prompt (9 query tiles x 8 head pairs: 4 key splits), causal
    _, q, k, v = contiguous_case([1100], seed=23)
    check(q.contiguous(), k.contiguous(), v.contiguous(), cu([1100]), cu([1100]))
    # non-causal, head_dim 64, 4 q heads per kv head: 100 queries over 1500 keys
    g = torch.Generator("cpu").manual_seed(24)
    q = torch.randn(100, 16, 64, generator=g).to(torch.bfloat16)
    k = torch.randn(1500, 4, 64, generator=g).to(torch.bfloat16)
    v = torch.randn(1500, 4, 64, generator=g).to(torch.bfloat16)
    check(q, k, v, cu([100]), cu([1500]), causal=False)


def test_split_graph_replay_matches_eager():
    q, kc, vc, bt = paged_case([256], [4096], 256, seed=25)
    q, kc, vc, bt = q.to(DEV), kc.to(DEV), vc.to(DEV), bt.to(DEV)
    cq, ck = cu([256]).to(DEV), cu([4096]).to(DEV)
    eager = flash_attn_varlen_func(q, kc, vc, 256, cq, 4096, ck, 0.1, True, bt)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        flash_attn_varlen_func(q, kc, vc, 256, cq, 4096, ck, 0.1, True, bt)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = flash_attn_varlen_func(q, kc, vc, 256, cq, 4096, ck, 0.1, True, bt)
    for rep in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep


@pytest.mark.parametrize("seed", range(10))
def test_random_varlen_batches(seed):
    """Seeded random batches over the cache: 1-6 sequences mixing empty, one-query, short (<= 16 / G queries, the
    decode kernel's) and long query runs over prefixes of 0-1200 cached keys; block sizes 16 / 64 / 256; GQA ratios
    1 / 2 / 4; head_dim 64 / 128; causal or not. Some batches split their keys over blocks."""
    rng = np.random.default_rng(1000 + seed)
    Hq, Hkv = [(16, 8), (8, 8), (16, 4)][seed % 3]
    D = 128 if seed % 2 == 0 else 64
    bs = [16, 64, 256][seed % 3]
    n = int(rng.integers(1, 7))
    lq, lk = [], []
    for _ in range(n):
        kind = rng.integers(0, 4)
        q = [0, 1, int(rng.integers(2, 9)), int(rng.integers(9, 200))][kind]
        lq.append(q)
        lk.append(q + int(rng.integers(0, 1201)))
    causal = bool(seed % 4 != 3)
    q, kc, vc, bt = paged_case(lq, lk, bs, Hq=Hq, Hkv=Hkv, D=D, seed=2000 + seed)
    check(q, kc, vc, cu(lq), cu(lk), causal, bt)


def test_head_dim_64_and_gqa():
    for Hq, Hkv, D in [(8, 8, 64), (16, 4, 128), (16, 2, 64)]:
        _, q, k, v = contiguous_case([90, 200], Hq=Hq, Hkv=Hkv, D=D, seed=Hq + Hkv + D)
        check(q.contiguous(), k.contiguous(), v.contiguous(), cu([90, 200]), cu([90, 200]))


def test_odd_group_size_one_head_per_block():
    # Hq / Hkv odd: one q head per block, 256-query tiles; lengths past one and two tiles
    for Hq, Hkv, D, lens in [(6, 2, 128, [600, 37]), (3, 1, 64, [257, 513])]:
        _, q, k, v = contiguous_case(lens, Hq=Hq, Hkv=Hkv, D=D, seed=Hq * 7 + D)
        check(q.contiguous(), k.contiguous(), v.contiguous(), cu(lens), cu(lens))


def test_non_causal_and_more_queries_than_keys():
    _, q, k, v = contiguous_case([50, 120], seed=3)
    check(q.contiguous(), k.contiguous(), v.contiguous(), cu([50, 120]), cu([50, 120]), causal=False)
    g = torch.Generator("cpu").manual_seed(9)
    q = torch.randn(40, 16, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(10, 8, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(10, 8, 128, generator=g).to(torch.bfloat16)
    out, _ = check(q, k, v, cu([40]), cu([10]), causal=True)   # queries 0..29 see no key
    assert torch.all(out[:30] == 0)


def test_empty_sequence_in_the_batch():
    _, q, k, v = contiguous_case([30, 0, 70], seed=5)
    check(q.contiguous(), k.contiguous(), v.contiguous(), cu([30, 0, 70]), cu([30, 0, 70]))


def test_graph_replay_matches_eager():
    lens = [200, 333]
    _, q, k, v = contiguous_case(lens, seed=6)
    q, k, v = q.contiguous().to(DEV), k.contiguous().to(DEV), v.contiguous().to(DEV)
    cq = cu(lens).to(DEV)
    eager = flash_attn_varlen_func(q, k, v, 333, cq, 333, cq, 0.1, True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        flash_attn_varlen_func(q, k, v, 333, cq, 333, cq, 0.1, True)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = flash_attn_varlen_func(q, k, v, 333, cq, 333, cq, 0.1, True)
    for rep in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep
