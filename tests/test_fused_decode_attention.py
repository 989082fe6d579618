"""The decode step's q/k norm + RoPE + KV write fused into the paged decode attention
(nvhip_qk_norm_rope_kv_decode_attention_bf16) on the GPU: bitwise qk_norm_rope_kv followed by
flash_attn_with_kvcache -- the attention output and both caches -- at the Qwen3-0.6B attention shape with and
without the context split of small batches, block sizes that do and do not hold whole 32-token chunks, head_dim
64 with 4 q heads per kv head, padding slots, slots outside the decode layout, and the wrapper's fallback for
head_dim 256."""
import pytest
import torch

from nanovllm_hip.kernels.attention import flash_attn_with_kvcache, qk_norm_rope_kv_decode_attention
from nanovllm_hip.kernels.qk_norm_rope_kv import qk_norm_rope_kv

pytestmark = pytest.mark.gpu

DEV = "cuda"


def case(lens, Hq=16, Hkv=8, D=128, bs=256, seed=0, pad=()):
    """Raw q/k/v views of a qkv buffer for one new token per sequence (position len - 1), caches holding the
    earlier tokens, a shuffled block table, the slots of the new tokens (-1 for the sequences in pad)."""
    g = torch.Generator("cpu").manual_seed(seed)
    B = len(lens)
    need = [(n + bs - 1) // bs for n in lens]
    nb = sum(need) + 2
    kc = torch.randn(nb, bs, Hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, bs, Hkv, D, generator=g).to(torch.bfloat16)
    perm = torch.randperm(nb, generator=g)
    maxb = max(max(need), 1)
    bt = torch.zeros(B, maxb, dtype=torch.int32)
    used = 0
    for b, n in enumerate(need):
        for c in range(n):
            bt[b, c] = int(perm[used]); used += 1
    W = (Hq + 2 * Hkv) * D + 64
    qkv = torch.randn(B, W, generator=g).to(torch.bfloat16)
    q = qkv[:, :Hq * D].view(B, Hq, D)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].view(B, Hkv, D)
    v = qkv[:, (Hq + Hkv) * D:(Hq + 2 * Hkv) * D].view(B, Hkv, D)
    pos = torch.tensor([max(n - 1, 0) for n in lens], dtype=torch.int64)
    slots = torch.tensor([-1 if (b in pad or n == 0) else int(bt[b, (n - 1) // bs]) * bs + (n - 1) % bs
                          for b, n in enumerate(lens)], dtype=torch.int32)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    inv = 1.0 / (1e6 ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    ang = torch.arange(4096, dtype=torch.float64)[:, None] * inv[None, :]
    cos_sin = torch.cat([ang.cos(), ang.sin()], -1).float().unsqueeze(1)
    t = lambda x: x.to(DEV)
    return (t(qkv), t(q), t(k), t(v), t(pos), t(slots), t(qw), t(kw), t(cos_sin), t(kc), t(vc), t(bt),
            torch.tensor(lens, dtype=torch.int32, device=DEV))


def both(c, eps=1e-6):
    qkv, q, k, v, pos, slots, qw, kw, cs, kc, vc, bt, lens = c
    B, Hq, D = q.shape
    kc1, vc1, kc2, vc2 = kc.clone(), vc.clone(), kc.clone(), vc.clone()
    q_out, _ = qk_norm_rope_kv(q, k, v, pos, qw, kw, eps, cs, kc1, vc1, slots, False)
    ref = flash_attn_with_kvcache(q_out.view(B, 1, Hq, D), kc1, vc1, lens, bt, D ** -0.5, causal=True)
    got = qk_norm_rope_kv_decode_attention(q, k, v, pos, qw, kw, eps, cs, kc2, vc2, slots, lens, bt, D ** -0.5)
    return got, ref.view(B, Hq, D), (kc1, vc1), (kc2, vc2)


@pytest.mark.parametrize("B,bs", [(32, 256), (32, 16), (5, 256), (3, 48)])
def test_bitwise_the_two_calls(B, bs):
    g = torch.Generator("cpu").manual_seed(B * 1000 + bs)
    lens = torch.randint(1, 2049, (B,), generator=g).tolist()
    got, ref, c1, c2 = both(case(lens, bs=bs, seed=B + bs))
    assert torch.equal(got, ref)
    assert torch.equal(c1[0], c2[0]) and torch.equal(c1[1], c2[1])


def test_head_dim_64_gqa_and_padding():
    lens = [700, 1, 33, 0, 256, 257]
    got, ref, c1, c2 = both(case(lens, Hq=16, Hkv=4, D=64, bs=32, seed=5, pad=(3,)))
    assert torch.equal(got, ref)
    assert torch.equal(c1[0], c2[0]) and torch.equal(c1[1], c2[1])
    assert torch.all(got[3] == 0)


def test_fallback_for_head_dim_256():
    lens = [300, 40]
    got, ref, c1, c2 = both(case(lens, Hq=8, Hkv=2, D=256, bs=32, seed=6))
    assert torch.equal(got, ref)
    assert torch.equal(c1[0], c2[0]) and torch.equal(c1[1], c2[1])


@pytest.mark.parametrize("B", [3, 32])
def test_slot_in_another_sequences_context(B):
    """A slot inside another sequence's context (B = 32: the length-balanced launch, whose blocks run pieces of
    two pairs): the new rows still land in the cache bitwise as the two calls write them, and every sequence whose
    context does not hold that slot gets the two calls' output bitwise. The sequence that reads the slot is
    outside the guarantee (its block may run before or after the writing block), so only its finiteness is
    checked."""
    g = torch.Generator("cpu").manual_seed(40 + B)
    lens = [300, 900, 45] if B == 3 else torch.randint(64, 2049, (B,), generator=g).tolist()
    c = list(case(lens, seed=9 + B))
    bt, slots = c[11].cpu(), c[5].clone()
    bs = c[9].shape[1]
    reader, writer, tok = 0, B - 1, 7
    slots[writer] = int(bt[reader, tok // bs]) * bs + tok % bs
    c[5] = slots
    got, ref, c1, c2 = both(tuple(c))
    assert torch.equal(c1[0], c2[0]) and torch.equal(c1[1], c2[1])
    others = [b for b in range(B) if b != reader]
    assert torch.equal(got[others], ref[others])
    assert torch.isfinite(got[reader].float()).all()


def test_graph_replay_matches_eager():
    lens = [1500, 90, 2048, 5]
    c = case(lens, seed=7)
    qkv, q, k, v, pos, slots, qw, kw, cs, kc, vc, bt, ln = c
    eager = qk_norm_rope_kv_decode_attention(q, k, v, pos, qw, kw, 1e-6, cs, kc, vc, slots, ln, bt, 128 ** -0.5)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = qk_norm_rope_kv_decode_attention(q, k, v, pos, qw, kw, 1e-6, cs, kc, vc, slots, ln, bt, 128 ** -0.5)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_slot_that_is_not_the_new_position():
    """A slot other than the cache slot of position len - 1 (not a decode step's layout): the kernel writes it
    before reading the cache, as the two calls do, so the rows and caches still match them bitwise."""
    lens = [300, 900, 45]
    c = list(case(lens, seed=8))
    bt, kc = c[11], c[9]
    used = set(bt.flatten().tolist())
    spare = next(i for i in range(kc.shape[0]) if i not in used)
    slots = c[5].clone()
    slots[1] = spare * kc.shape[1] + 3
    c[5] = slots
    got, ref, c1, c2 = both(tuple(c))
    assert torch.equal(got, ref)
    assert torch.equal(c1[0], c2[0]) and torch.equal(c1[1], c2[1])
