"""Mixed prefill + decode steps and their piecewise graphs (nanovllm_hip/harness/mixed.py).

CPU: the flat batch layout of a mixed step against values worked out by hand from nano-vllm's rules
(model_runner.py:32-64: slots across block boundaries, cu_seqlens_k up to each request's last query, which rows
get logits); the fp32 varlen paged attention against the one-sequence prefill and the decode attention it
generalises; the segment runner (eager, padded to a bucket) against the unpadded forward, torch backend.

GPU: a mixed step of three decode requests, a first prefill chunk and a second prefill chunk (its first chunk
already cached), hip backend, HIP varlen paged attention: the piecewise graphs replay exactly (bitwise) what the
same segments give eagerly at the same padded size, hidden states and KV cache; a second, smaller step replays the
same bucket's graphs; the padded step agrees with the unpadded eager forward, and with the torch backend (fp32
attention, torch layers) within bf16 rounding.
"""
import pytest
import torch

from nanovllm_hip.harness.mixed import Piecewise, Request, mixed_batch, mixed_buckets, prepare_mixed
from nanovllm_hip.harness.qwen3 import Context, Qwen3, Qwen3Config, paged_decode_attention, prefill_attention, \
    varlen_paged_attention


def test_mixed_batch_layout():
    reqs = [Request(tokens=[5, 6, 7, 8, 9], block_table=[2, 7], num_cached=4),                 # decode
            Request(tokens=list(range(20, 30)), block_table=[3, 0, 5], num_cached=3, num_scheduled=6),  # mid chunk
            Request(tokens=[40, 41], block_table=[1], num_cached=0, num_scheduled=2)]          # whole prompt
    b = mixed_batch(reqs, block_size=4)
    assert b["input_ids"] == [9, 23, 24, 25, 26, 27, 28, 40, 41]
    assert b["positions"] == [4, 3, 4, 5, 6, 7, 8, 0, 1]
    # decode token at position 4 -> block 7, offset 0; the chunk's positions 3..8 -> 3*4+3, block 0 (0..3), 5*4+0
    assert b["slot_mapping"] == [28, 15, 0, 1, 2, 3, 20, 4, 5]
    assert b["cu_seqlens_q"] == [0, 1, 7, 9]
    assert b["cu_seqlens_k"] == [0, 5, 14, 16]
    assert b["logits_indices"] == [0, 8]        # the decode row; the chunk that ends its prompt (not the mid chunk)
    assert (b["max_seqlen_q"], b["max_seqlen_k"]) == (6, 9)


def test_mixed_buckets():
    assert mixed_buckets() == [64, 128, 192, 256, 320, 384, 448, 512]
    assert mixed_buckets(200) == [64, 128, 192, 200]


def _cache_with(k_seq, v_seq, table, num_blocks, bs):
    hkv, d = k_seq.shape[1], k_seq.shape[2]
    kc = torch.zeros(num_blocks, bs, hkv, d, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    for p in range(k_seq.shape[0]):
        kc[table[p // bs], p % bs] = k_seq[p]
        vc[table[p // bs], p % bs] = v_seq[p]
    return kc, vc


def test_varlen_paged_attention_reduces_to_prefill_and_decode():
    g = torch.Generator().manual_seed(0)
    hq, hkv, d, bs = 4, 2, 16, 8
    lk = 21
    k = torch.randn(lk, hkv, d, generator=g).bfloat16()
    v = torch.randn(lk, hkv, d, generator=g).bfloat16()
    table = [3, 0, 5]
    kc, vc = _cache_with(k, v, table, 6, bs)
    bt = torch.tensor([table], dtype=torch.int32)
    scale = d ** -0.5
    # whole sequence as queries: the one-sequence causal prefill
    q = torch.randn(lk, hq, d, generator=g).bfloat16()
    cu_q = torch.tensor([0, lk], dtype=torch.int32)
    got = varlen_paged_attention(q, kc, vc, bt, cu_q, cu_q, scale)
    assert torch.equal(got, prefill_attention(q, k, v, scale))
    # one query (the last token): the decode attention over the whole context
    q1 = q[-1:]
    got1 = varlen_paged_attention(q1, kc, vc, bt, torch.tensor([0, 1], dtype=torch.int32),
                                  torch.tensor([0, lk], dtype=torch.int32), scale)
    want1 = paged_decode_attention(q1, kc, vc, bt, torch.tensor([lk], dtype=torch.int32), scale)
    torch.testing.assert_close(got1.float(), want1.float(), rtol=0, atol=1e-2)
    # the last 5 queries of the sequence, bottom-right aligned: rows of the full prefill
    cu5 = torch.tensor([0, 5], dtype=torch.int32)
    got5 = varlen_paged_attention(q[-5:], kc, vc, bt, cu5, torch.tensor([0, lk], dtype=torch.int32), scale)
    assert torch.equal(got5, prefill_attention(q, k, v, scale)[-5:])


def _tiny_cfg(layers=2):
    return Qwen3Config(vocab_size=300, hidden_size=64, intermediate_size=96, num_hidden_layers=layers,
                       num_attention_heads=4, num_key_value_heads=2, head_dim=16, max_position_embeddings=512)


def _prefill_eager(model, tokens, table, bs, backend, attention, device, start=0):
    """Writes the KV of tokens[start:] (positions start..) through a one-sequence prefill (no prefix)."""
    n = len(tokens) - start
    pos = torch.arange(start, len(tokens), device=device)
    slots = torch.tensor([table[p // bs] * bs + p % bs for p in range(start, len(tokens))], dtype=torch.int32,
                         device=device)
    model.forward(torch.tensor(tokens[start:], device=device), pos, Context(True, slots), backend, attention)
    return n


def _scenario(model, bs, device, backend, attention, seed=1, n_decode=3, first_chunk=40, second=(64, 56)):
    """Requests of a mixed step: n_decode decode requests whose prompts are cached, a first prefill chunk and a
    second chunk of a request whose first chunk is cached. Returns the requests."""
    g = torch.Generator().manual_seed(seed)
    vocab = model.cfg.vocab_size
    next_block = iter(torch.randperm(model.kv[0][0].shape[0], generator=g).tolist())
    reqs = []
    for i in range(n_decode):
        plen = int(torch.randint(20, 300, (1,), generator=g))
        toks = torch.randint(0, vocab, (plen + 1,), generator=g).tolist()
        table = [next(next_block) for _ in range((plen + 1 + bs - 1) // bs)]
        _prefill_eager(model, toks[:plen], table, bs, backend, attention, device)
        reqs.append(Request(toks, table, num_cached=plen))
    toks = torch.randint(0, vocab, (first_chunk + 30,), generator=g).tolist()
    reqs.append(Request(toks, [next(next_block) for _ in range((len(toks) + bs - 1) // bs)], 0, first_chunk))
    done, chunk = second
    toks = torch.randint(0, vocab, (done + chunk,), generator=g).tolist()
    table = [next(next_block) for _ in range((len(toks) + bs - 1) // bs)]
    _prefill_eager(model, toks[:done], table, bs, backend, attention, device)
    reqs.append(Request(toks, table, done, chunk))
    return reqs


def test_piecewise_eager_matches_forward_cpu():
    torch.manual_seed(0)
    bs = 16
    model = Qwen3(_tiny_cfg(), "cpu", seed=3)
    model.allocate_kv_cache(64, bs)
    reqs = _scenario(model, bs, "cpu", "torch", "torch", n_decode=2, first_chunk=9, second=(20, 11))
    ids, pos, ctx, logits_idx = prepare_mixed(reqs, bs, "cpu")
    assert ids.shape[0] == 22
    want = model.forward(ids, pos, ctx, "torch", "torch")
    pw = Piecewise(model, [16, 32], backend="torch", attention="torch")
    got = pw.run(ids, pos, ctx)            # padded to 32 tokens, segments run eagerly
    assert got.shape == want.shape
    torch.testing.assert_close(got.float(), want.float(), rtol=2e-2, atol=2e-2)
    assert logits_idx.tolist() == [0, 1, 21]


@pytest.mark.gpu
def test_piecewise_graphs_mixed_step():
    dev = torch.device("cuda:0")
    bs = 256
    cfg = Qwen3Config(num_hidden_layers=3)
    model = Qwen3(cfg, dev, seed=0)
    cache = model.allocate_kv_cache(24, bs)
    reqs = _scenario(model, bs, dev, "hip", "hip")
    ids, pos, ctx, logits_idx = prepare_mixed(reqs, bs, dev)
    n = ids.shape[0]
    assert n == 3 + 40 + 56
    before = cache.clone()

    eager_pw = Piecewise(model, [64, 128], backend="hip", attention="hip")
    h_pe = eager_pw.run(ids, pos, ctx).clone()
    cache_pe = cache.clone()
    cache.copy_(before)

    pw = Piecewise(model, [64, 128], backend="hip", attention="hip")
    pw.record()
    cache.copy_(before)                      # recording ran the segments only; attention never ran
    h_pg = pw.run(ids, pos, ctx).clone()
    torch.cuda.synchronize()
    assert torch.equal(h_pg, h_pe)
    assert torch.equal(cache, cache_pe)
    # replays again with other inputs in between: same bits
    cache.copy_(before)
    assert torch.equal(pw.run(ids, pos, ctx), h_pe)

    # The graph = eager pair above is the reference's contract (tests/test_greedy.py:110-112, MUST_MATCH
    # mixed_graph = mixed_eager, where mixed_eager pads to the same token counts). The unpadded eager forward runs
    # the same kernels on 99 instead of 128 rows, where the GEMM tiles and the projections' K splits are chosen
    # for that M, so it is compared within bf16 tolerance.
    cache.copy_(before)
    h_eager = model.forward(ids, pos, ctx, "hip", "hip")
    torch.testing.assert_close(h_pg.float(), h_eager.float(), rtol=2e-2, atol=2e-2)

    # torch backend (torch layers, fp32 varlen attention) on the same step and cache: bf16 rounding differences only
    cache.copy_(before)
    h_torch = model.forward(ids, pos, ctx, "torch", "torch").float()
    rel = ((h_pg.float() - h_torch).norm() / h_torch.norm()).item()
    assert rel < 3e-2, rel

    # a second, smaller step (70 tokens) replays the same bucket's graphs
    cache.copy_(before)
    reqs2 = reqs[:2] + [Request(reqs[3].tokens, reqs[3].block_table, 0, 68)]
    ids2, pos2, ctx2, _ = prepare_mixed(reqs2, bs, dev)
    assert ids2.shape[0] == 70
    h2_pg = pw.run(ids2, pos2, ctx2).clone()
    cache2_pg = cache.clone()
    cache.copy_(before)
    h2_pe = eager_pw.run(ids2, pos2, ctx2)
    assert torch.equal(h2_pg, h2_pe)
    assert torch.equal(cache, cache2_pg)
    # logits rows: the three decode rows and the last row of the chunk that ends its prompt (not the first chunk)
    assert logits_idx.tolist() == [0, 1, 2, n - 1]
