"""GPU parity of the paged decode attention (nvhip_paged_decode_attention_bf16) against the oracle.

The oracle restates flash_attn_with_kvcache as nanovllm/layers/attention.py:84-90 calls it (fp32 from the same
bf16 inputs). Tolerance: the bf16 output tolerance rtol 1.6e-2, atol 1e-2. Cases: the Qwen3-0.6B decode batch
(32 sequences, 16 q heads, 8 kv heads, head_dim 128, 256-slot blocks, contexts of 512..2048 tokens); context lengths
around the 32-token chunk and the block size, 0 (padding) and 1; block sizes that are not a multiple of 32; head_dim
64 and 256; GQA ratios 1, 4, 8; several query tokens per sequence with and without the causal mask; NaN in the
unused slots of a sequence's last block and in blocks no sequence owns; graph capture and replay; ragged batches of
1 .. 512 sequences (empty contexts among them) with and without the context split, repeated bitwise.
"""
import math

import pytest
import torch

import oracle
from helpers import paged_decode_abi
from nanovllm_hip.kernels.attention import flash_attn_with_kvcache

pytestmark = pytest.mark.gpu
DEV = "cuda"


def make_case(lens, q_len=1, Hq=16, Hkv=8, D=128, block_size=256, seed=0, spare_blocks=3, nan_unused=True):
    g = torch.Generator("cpu").manual_seed(seed)
    num_seqs = len(lens)
    need = [max(1, (n + block_size - 1) // block_size) for n in lens]
    num_blocks = sum(need) + spare_blocks
    kc = torch.randn(num_blocks, block_size, Hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(num_blocks, block_size, Hkv, D, generator=g).to(torch.bfloat16)
    perm = torch.randperm(num_blocks, generator=g)
    maxb = max(need)
    bt = torch.full((num_seqs, maxb), -1, dtype=torch.int32)
    used = 0
    for b, nb in enumerate(need):
        bt[b, :nb] = perm[used:used + nb].to(torch.int32)
        used += nb
    if nan_unused:
        for b, n in enumerate(lens):   # slots past the context in the sequence's last block
            last = int(bt[b, max(n - 1, 0) // block_size])
            if n % block_size:
                kc[last, n % block_size:] = float("nan")
                vc[last, n % block_size:] = float("nan")
        for blk in perm[used:]:          # blocks no sequence owns
            kc[blk] = float("nan")
            vc[blk] = float("nan")
    q = torch.randn(num_seqs, q_len, Hq, D, generator=g).to(torch.bfloat16)
    return q, kc, vc, torch.tensor(lens, dtype=torch.int32), bt


def run_and_check(q, kc, vc, lens, bt, causal=True, scale=None):
    D = q.shape[-1]
    scale = D ** -0.5 if scale is None else scale
    out = flash_attn_with_kvcache(q.to(DEV), kc.to(DEV), vc.to(DEV), lens.to(DEV), bt.to(DEV), scale, causal)
    ref = oracle.paged_decode_attention(q, kc, vc, lens, bt, scale, causal)
    out = out.cpu()
    assert out.shape == q.shape and out.dtype == torch.bfloat16
    assert torch.isfinite(out.float()).all()
    torch.testing.assert_close(out.float(), ref.float(), rtol=1.6e-2, atol=1e-2)
    return out, ref


def test_qwen3_decode_batch():
    g = torch.Generator("cpu").manual_seed(7)
    lens = torch.randint(512, 2049, (32,), generator=g).tolist()
    out, ref = run_and_check(*make_case(lens))
    # fp32 inside, one bf16 rounding at the end: nearly every element is the correctly rounded oracle value
    assert (out == ref).float().mean() > 0.97


@pytest.mark.parametrize("block_size", [256, 32, 16, 8])
def test_context_lengths_around_chunks_and_blocks(block_size):
    lens = [1, 2, 31, 32, 33, 63, 64, 65, 255, 256, 257, 300, 511, 513]
    run_and_check(*make_case(lens, block_size=block_size, seed=block_size))


def test_padding_sequence_gets_zeros():
    q, kc, vc, lens, bt = make_case([40, 0, 70], nan_unused=False)
    out, _ = run_and_check(q, kc, vc, lens, bt)
    assert torch.all(out[1] == 0)


@pytest.mark.parametrize("D", [64, 256])
def test_head_dims(D):
    run_and_check(*make_case([5, 100, 700], D=D, Hq=8, Hkv=4, seed=D))


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (16, 4), (16, 2)])
def test_gqa_ratios(Hq, Hkv):
    run_and_check(*make_case([77, 300, 1000], Hq=Hq, Hkv=Hkv, seed=Hq * 10 + Hkv))


@pytest.mark.parametrize("q_len,causal", [(2, True), (3, True), (4, False), (8, True)])
def test_several_query_tokens(q_len, causal):
    run_and_check(*make_case([q_len, 50, 290, 1024], q_len=q_len, Hq=16, Hkv=8, seed=q_len), causal=causal)


def test_sixteen_rows_per_kv_head():
    run_and_check(*make_case([20, 600], q_len=2, Hq=8, Hkv=1, seed=3))


def test_strided_q_view():
    """q as a view of a wider buffer (per-token stride > Hq * D) is accepted (copied by the wrapper)."""
    q, kc, vc, lens, bt = make_case([100, 200])
    wide = torch.zeros(2, 1, 16, 160, dtype=torch.bfloat16)
    wide[..., :128] = q
    run_and_check(wide[..., :128], kc, vc, lens, bt)


def test_graph_replay_matches_eager():
    q, kc, vc, lens, bt = make_case([300, 700, 1500, 64], seed=11)
    q, kc, vc, lens, bt = (t.to(DEV) for t in (q, kc, vc, lens, bt))
    eager = flash_attn_with_kvcache(q, kc, vc, lens, bt, 128 ** -0.5, True)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        flash_attn_with_kvcache(q, kc, vc, lens, bt, 128 ** -0.5, True)
    torch.cuda.current_stream().wait_stream(s)
    with torch.cuda.graph(graph):
        out = flash_attn_with_kvcache(q, kc, vc, lens, bt, 128 ** -0.5, True)
    for rep in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), rep


def test_rejects_bad_arguments():
    q, kc, vc, lens, bt = (t.to(DEV) for t in make_case([10, 20]))
    with pytest.raises(AssertionError):
        flash_attn_with_kvcache(q.float(), kc, vc, lens, bt, 0.1, True)
    with pytest.raises(ValueError):   # 32 rows per kv head
        flash_attn_with_kvcache(q.repeat(1, 2, 1, 1), kc[:, :, :1].contiguous(), vc[:, :, :1].contiguous(), lens, bt,
                                0.1, True)


def balanced_lens(kind):
    g = torch.Generator("cpu").manual_seed(len(kind))
    if kind == "qwen3_b32":      # the decode step's batch: contexts U[512, 2048]
        return torch.randint(512, 2049, (32,), generator=g).tolist()
    if kind == "qwen3_b64":
        return torch.randint(512, 2049, (64,), generator=g).tolist()
    if kind == "odd_33":         # the median sequence is not paired
        return torch.randint(1, 3001, (33,), generator=g).tolist()
    if kind == "equal":          # nothing to cut: every pair whole in its own block
        return [1000] * 40
    if kind == "empty_and_long":  # empty and one-token contexts paired with the longest ones
        return [0, 1, 4000, 3500, 0, 2] + torch.randint(1, 1500, (26,), generator=g).tolist()
    raise ValueError(kind)


@pytest.mark.parametrize("kind,q_len,Hq,Hkv,D,bs", [
    ("qwen3_b32", 1, 16, 8, 128, 256), ("odd_33", 1, 16, 8, 128, 256), ("equal", 1, 16, 8, 128, 256),
    ("empty_and_long", 1, 16, 8, 128, 256), ("qwen3_b32", 3, 16, 8, 128, 256),
    ("qwen3_b32", 1, 16, 8, 128, 16),    # 16-slot blocks: chunks and cuts cross cache blocks
    ("qwen3_b64", 1, 16, 4, 64, 32),     # 4 kv heads (256 pairs), head_dim 64
    ("qwen3_b32", 1, 32, 16, 128, 256),  # 16 kv heads: 512 pairs
    ("qwen3_b32", 1, 16, 8, 256, 32),    # head_dim 256: 4-wave blocks, 128-token rounds
])
def test_balanced_batches(kind, q_len, Hq, Hkv, D, bs):
    """256 .. 512 (sequence, kv head) pairs with a workspace: long and short contexts are paired and the long
    pair's tail runs in the short pair's block, the two pieces merged inside the kernel by whichever block finishes
    last. The oracle's values at the bf16 tolerance, the one-block-per-pair path's too, the same bits on a second
    call, the workspace counters zero after each call (checked in paged_decode_abi)."""
    lens = balanced_lens(kind)
    q, kc, vc, lt, bt = make_case(lens, q_len=q_len, Hq=Hq, Hkv=Hkv, D=D, block_size=bs, seed=len(lens) + q_len,
                                  nan_unused=False)
    ref = oracle.paged_decode_attention(q, kc, vc, lt, bt, 0.1, True)
    dev = [t.to(DEV) for t in (q, kc, vc, lt, bt)]
    bal, need = paged_decode_abi(*dev, 0.1, True, workspace=True)
    again, _ = paged_decode_abi(*dev, 0.1, True, workspace=True)
    single, _ = paged_decode_abi(*dev, 0.1, True, workspace=False)
    assert need > 0
    assert torch.equal(bal, again)
    for out in (bal, single):
        torch.testing.assert_close(out.cpu().float(), ref.float(), rtol=1.6e-2, atol=1e-2)
    for b, n in enumerate(lens):
        if n == 0:
            assert torch.all(bal[b] == 0)
    if kind == "equal":
        assert torch.equal(bal, single)  # no pair is cut: the same blocks' arithmetic


@pytest.mark.parametrize("B,max_len,block_size,seed", [
    (1, 100, 256, 1),      # 8 (sequence, kv head) pairs of at most 4 chunks
    (3, 20000, 256, 2),    # 24 pairs of up to 625 chunks: many splits each
    (20, 300, 16, 3),      # 160 pairs, 16-slot blocks
    (64, 1200, 256, 4),    # 512 pairs: the pairs of the sequences above the mean context cut in two
    (512, 64, 32, 5),      # 4096 short pairs
])
def test_ragged_batches(B, max_len, block_size, seed):
    """Ragged batches (context lengths 0 .. max_len, a tenth of them 0), with and without a workspace: the oracle's
    values, zeros for empty contexts, and the same bits on a second call."""
    g = torch.Generator("cpu").manual_seed(seed)
    lens = torch.randint(0, max_len + 1, (B,), generator=g)
    lens[torch.rand(B, generator=g) < 0.1] = 0
    lens = lens.tolist()
    q, kc, vc, lt, bt = make_case(lens, block_size=block_size, seed=seed, nan_unused=False)
    ref = oracle.paged_decode_attention(q, kc, vc, lt, bt, 0.1, True)
    dev = [t.to(DEV) for t in (q, kc, vc, lt, bt)]
    split, need = paged_decode_abi(*dev, 0.1, True, workspace=True)
    again, _ = paged_decode_abi(*dev, 0.1, True, workspace=True)
    single, _ = paged_decode_abi(*dev, 0.1, True, workspace=False)
    if 256 <= B * 8 <= 512:
        assert need > 0                    # a batch of 256 to 512 pairs: the long pairs cut in two
    if B * 8 > 512:
        assert need == 0                   # more pairs: one block each
    if B == 3:
        assert need > 0                    # few pairs over long contexts: split
    assert torch.equal(split, again)
    for out in (split, single):
        torch.testing.assert_close(out.cpu().float(), ref.float(), rtol=1.6e-2, atol=1e-2)
    for b, n in enumerate(lens):
        if n == 0:
            assert torch.all(split[b] == 0) and torch.all(single[b] == 0)


@pytest.mark.parametrize("lens", [[300, 2048, 1, 777, 256, 512, 0, 1500], [5000, 17, 4096]])
def test_split_and_single_pass_agree_with_oracle(lens):
    """The split-context path (workspace) and the one-block path (no workspace) both match the oracle."""
    q, kc, vc, lt, bt = make_case(lens, seed=len(lens))
    ref = oracle.paged_decode_attention(q, kc, vc, lt, bt, 0.1, True)
    dev = [t.to(DEV) for t in (q, kc, vc, lt, bt)]
    split, need = paged_decode_abi(*dev, 0.1, True, workspace=True)
    single, _ = paged_decode_abi(*dev, 0.1, True, workspace=False)
    assert need > 0
    for out in (split, single):
        torch.testing.assert_close(out.cpu().float(), ref.float(), rtol=1.6e-2, atol=1e-2)
