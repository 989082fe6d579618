"""GPU parity of the fused q/k RMSNorm + RoPE + paged-KV write (nvhip_qk_norm_rope_kv_bf16) against the CPU oracle.

Structure of the reference's tests/test_kernels_qk_rope_kv.py, with the oracle (the reference's torch code restated,
run on the CPU on the same seeded inputs) as the referee:
  torch eager  q_out, k_out and both caches bitwise equal to the reference's torch composition (q_norm / k_norm,
               rotary_emb, store_kvcache) run eagerly on the same GPU, and to oracle.qk_norm_rope_kv with
               gpu_numerics (its CPU restatement: ATen's GPU summation order, torch.rsqrt's double evaluation).
  norm stage   the kernel with an identity rotation table (cos = 1, sin = 0, all positions 0) outputs exactly its
               normed q and k: within MAX_ULP = 2 bf16 ulps of the CPU oracle's rms_forward (the reference's bar).
  rope stage   the kernel's real output equals, bitwise, the oracle's RoPE applied to the kernel's own normed q/k.
  KV write     written k rows equal k_out bitwise, v rows equal v bitwise, every unnamed row is untouched.
  end to end   q_out / k_out within the task's bf16 tolerance (rtol 1.6e-2, atol 1e-2) of the oracle.
Cases: the reference's grid (tokens 1/7/128/4097 x random/arange positions, every 5th slot -1, random cache
contents) plus the MI355X workload (tokens 1/32/2048/8192, qkv a view of a [T, 4096+64] buffer, 4 sequences
with contiguous positions, 512 x 256-slot cache, 10% padding slots), other head layouts and the edge cases.
"""
import os

import numpy as np
import pytest
import torch

import oracle
from helpers import (BLOCK, EPS, HEAD_DIM, KV_HEADS, MAX_POS, Q_HEADS, THETA, bf16_randn, max_ulp, norm_weight,
                     random_block_table_slots)
from nanovllm_hip.kernels import qk_norm_rope_kv

pytestmark = pytest.mark.gpu

MAX_ULP = 2
RTOL, ATOL = 1.6e-2, 1e-2
DEV = "cuda"
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "qk_norm_rope_kv_t16.npz")

_cos_sin = {}


def cos_sin_cache(d=HEAD_DIM):
    if d not in _cos_sin:
        _cos_sin[d] = oracle.rope_cos_sin_cache(d, MAX_POS, THETA)
    return _cos_sin[d]


def identity_table(d):
    return torch.cat([torch.ones(d // 2), torch.zeros(d // 2)]).view(1, 1, d)


class Case:
    """One set of inputs, on the CPU (for the oracle) and on the GPU (same values)."""

    def __init__(self, tokens, seed, hq=Q_HEADS, hkv=KV_HEADS, d=HEAD_DIM, pad=0, offset=0, positions=None,
                 slots=None, num_blocks=None, cache_init="randn"):
        g = torch.Generator("cpu").manual_seed(seed)
        self.T, self.hq, self.hkv, self.d = tokens, hq, hkv, d
        width = (hq + 2 * hkv) * d
        buf = bf16_randn((tokens, offset + width + pad), g)
        self.buf_cpu = buf
        self.q_w, self.k_w = norm_weight(d, g), norm_weight(d, g)
        self.positions = positions if positions is not None else torch.randint(0, MAX_POS, (tokens,), generator=g)
        if num_blocks is None:
            num_blocks = max(1, (2 * tokens + BLOCK - 1) // BLOCK)
        self.num_blocks = num_blocks
        if slots is None:
            slots = torch.randperm(num_blocks * BLOCK, generator=g)[:tokens].to(torch.int32)
            slots[4::5] = -1
        self.slots = slots
        self.offset = offset
        shape = (num_blocks, BLOCK, hkv, d)
        if cache_init == "randn":  # generated on the GPU (large caches), copied back for the oracle when needed
            gg = torch.Generator(DEV).manual_seed(seed + 1)
            self.cache0 = torch.randn((2,) + shape, device=DEV, generator=gg).to(torch.bfloat16)
        else:
            self.cache0 = torch.zeros((2,) + shape, device=DEV, dtype=torch.bfloat16)
        self.buf_dev = buf.to(DEV)

    def views(self, buf):
        T, hq, hkv, d, o = self.T, self.hq, self.hkv, self.d, self.offset
        q = buf[:, o:o + hq * d].view(T, hq, d) if T else buf[:, :hq * d].reshape(0, hq, d)
        k = buf[:, o + hq * d:o + (hq + hkv) * d]
        v = buf[:, o + (hq + hkv) * d:o + (hq + 2 * hkv) * d]
        return q, k.view(T, hkv, d) if T else k.reshape(0, hkv, d), v.view(T, hkv, d) if T else v.reshape(0, hkv, d)

    def run(self, identity_rope=False, write_k=True, store=True):
        q, k, v = self.views(self.buf_dev)
        cache = self.cache0.clone()
        positions, table = self.positions, cos_sin_cache(self.d)
        if identity_rope:
            positions, table = torch.zeros_like(positions), identity_table(self.d)
        kc, vc = (cache[0], cache[1]) if store else (torch.empty(0, device=DEV), torch.empty(0, device=DEV))
        q_out, k_out = qk_norm_rope_kv(q, k, v, positions.to(DEV), self.q_w.to(DEV), self.k_w.to(DEV), EPS,
                                       table.to(DEV), kc, vc, self.slots.to(DEV) if store else None, write_k)
        return q_out, k_out, cache

    def oracle_norms(self):
        q, k, _ = self.views(self.buf_cpu)
        return oracle.rms_forward(q, self.q_w, EPS), oracle.rms_forward(k, self.k_w, EPS)

    def oracle_end_to_end(self):
        q, k, v = self.views(self.buf_cpu)
        empty = torch.empty(0)
        return oracle.qk_norm_rope_kv(q, k, v, self.positions, self.q_w, self.k_w, EPS, cos_sin_cache(self.d),
                                      empty, empty, None, True)


def check_kv_write(case, k_out, cache):
    """Written rows hold k_out / v bitwise; every other row keeps its initial contents."""
    hkv, d = case.hkv, case.d
    slots = case.slots.to(DEV).long()
    real = slots >= 0
    _, _, v = case.views(case.buf_dev)
    k_rows = cache[0].view(-1, hkv, d)
    v_rows = cache[1].view(-1, hkv, d)
    assert torch.equal(k_rows[slots[real]], k_out[real]), "k cache rows differ from k_out"
    assert torch.equal(v_rows[slots[real]], v[real]), "v cache rows differ from v"
    untouched = torch.ones(k_rows.shape[0], dtype=torch.bool, device=DEV)
    untouched[slots[real]] = False
    for i in range(2):
        assert torch.equal(cache[i].view(-1, hkv, d)[untouched], case.cache0[i].view(-1, hkv, d)[untouched])


def check_torch_eager(case, q_out, k_out, cache):
    """Bitwise the reference's torch code run eagerly on the GPU, and its CPU restatement with GPU numerics."""
    q, k, v = case.views(case.buf_dev)
    cache_t = case.cache0.clone()
    q_t, k_t = oracle.qk_norm_rope_kv(q, k, v, case.positions.clamp(max=MAX_POS - 1).to(DEV), case.q_w.to(DEV),
                                      case.k_w.to(DEV), EPS, cos_sin_cache(case.d).to(DEV), cache_t[0], cache_t[1],
                                      case.slots.to(DEV), True)
    assert torch.equal(q_out, q_t) and torch.equal(k_out, k_t), "not bitwise torch-eager on the GPU"
    assert torch.equal(cache, cache_t), "caches differ from torch-eager's store_kvcache"
    qc, kc, vc = case.views(case.buf_cpu)
    empty = torch.empty(0)
    q_c, k_c = oracle.qk_norm_rope_kv(qc, kc, vc, case.positions.clamp(max=MAX_POS - 1), case.q_w, case.k_w, EPS,
                                      cos_sin_cache(case.d), empty, empty, None, True, gpu_numerics=True)
    assert torch.equal(q_out.cpu(), q_c) and torch.equal(k_out.cpu(), k_c)


def check_case(case):
    # norm stage
    q_n, k_n, _ = case.run(identity_rope=True)
    q_ref, k_ref = case.oracle_norms()
    assert max_ulp(q_n, q_ref) <= MAX_ULP, "q norm"
    assert max_ulp(k_n, k_ref) <= MAX_ULP, "k norm"
    # rope stage: bitwise vs the oracle's rotation of the kernel's own normed values
    q_out, k_out, cache = case.run()
    qr, kr = oracle.rotary_forward(case.positions, q_n.cpu(), k_n.cpu(), cos_sin_cache(case.d))
    assert torch.equal(q_out.cpu(), qr), "q rope stage not bitwise"
    assert torch.equal(k_out.cpu(), kr), "k rope stage not bitwise"
    # KV write
    check_kv_write(case, k_out, cache)
    check_torch_eager(case, q_out, k_out, cache)
    # end to end
    q_e, k_e = case.oracle_end_to_end()
    check_end_to_end(q_out, q_e, q_n, q_ref)
    check_end_to_end(k_out, k_e, k_n, k_ref)


def check_end_to_end(out, ref, normed, normed_ref):
    """out within (RTOL, ATOL) of the oracle, except where the kernel's normed input pair (n1[i], n2[i]) differs
    from the oracle's (an fp32 summation-order flip of one bf16 rounding, bounded by the norm stage): RoPE's
    subtraction can turn such a 1-ulp input difference into a large relative error of a near-zero output."""
    out, ref = out.cpu().float(), ref.float()
    bad = ~torch.isclose(out, ref, rtol=RTOL, atol=ATOL)
    if not bad.any():
        return
    half = out.shape[-1] // 2
    differs = normed.cpu() != normed_ref
    pair = differs[..., :half] | differs[..., half:]
    explained = torch.cat([pair, pair], dim=-1)
    assert not (bad & ~explained).any(), f"{int((bad & ~explained).sum())} elements outside tolerance"
    assert bad.float().mean() < 1e-4, f"{int(bad.sum())} of {bad.numel()} elements outside tolerance"


# ------------------------------------------------------------------ the reference's case grid

REF_TOKENS = [1, 7, 128, 4097]
REF_CASES = [(t, rp) for t in REF_TOKENS for rp in (True, False)]


@pytest.mark.parametrize("tokens,random_positions", REF_CASES,
                         ids=[f"tokens={t}-{'random' if rp else 'arange'}" for t, rp in REF_CASES])
def test_reference_grid(tokens, random_positions):
    positions = None if random_positions else torch.arange(tokens)
    check_case(Case(tokens, seed=tokens * 2 + random_positions, positions=positions))


# ------------------------------------------------------------------ the MI355X workload (prefill and decode)

@pytest.mark.parametrize("tokens", [1, 32, 2048, 8192])
def test_workload(tokens):
    g = torch.Generator("cpu").manual_seed(100 + tokens)
    slots, positions = random_block_table_slots(tokens, 512, g, num_seqs=min(4, tokens), pad_frac=0.1)
    check_case(Case(tokens, seed=tokens, pad=64, positions=positions, slots=slots, num_blocks=512))


# ------------------------------------------------------------------ golden fixture (16 tokens)

def test_golden_t16():
    z = np.load(GOLDEN)
    u16 = lambda name: torch.from_numpy(z[name].astype(np.int16)).view(torch.bfloat16)
    qkv = u16("qkv").to(DEV)
    T, D, Hq, Hkv = 16, 128, 16, 8
    q, k, v = (t.view(T, -1, D) for t in qkv.split([Hq * D, Hkv * D, Hkv * D], dim=-1))
    slots = torch.from_numpy(z["slot_mapping"]).to(DEV)
    positions = torch.from_numpy(z["positions"]).to(DEV)
    qw, kw, eps = u16("q_weight").to(DEV), u16("k_weight").to(DEV), float(z["eps"])

    def run(pos, table):
        kc = torch.zeros(64, 256, Hkv, D, dtype=torch.bfloat16, device=DEV)
        vc = torch.zeros_like(kc)
        q_out, k_out = qk_norm_rope_kv(q, k, v, pos, qw, kw, eps, table.to(DEV), kc, vc, slots, True)
        return q_out, k_out, kc, vc

    q_n, k_n, _, _ = run(torch.zeros_like(positions), identity_table(D))
    assert max_ulp(q_n, u16("q_normed")) <= MAX_ULP and max_ulp(k_n, u16("k_normed")) <= MAX_ULP
    q_out, k_out, kc, vc = run(positions, cos_sin_cache())
    assert torch.equal(q_out.cpu(), u16("q_out_gpu")) and torch.equal(k_out.cpu(), u16("k_out_gpu"))
    check_end_to_end(q_out, u16("q_out"), q_n, u16("q_normed"))
    check_end_to_end(k_out, u16("k_out"), k_n, u16("k_normed"))
    rows = slots.long()
    assert torch.equal(vc.view(-1, Hkv, D)[rows].cpu(), u16("v_cache_rows"))
    assert torch.equal(kc.view(-1, Hkv, D)[rows], k_out)
    check_end_to_end(kc.view(-1, Hkv, D)[rows], u16("k_cache_rows"), k_n, u16("k_normed"))


# ------------------------------------------------------------------ other head layouts and the edge cases

@pytest.mark.parametrize("hq,hkv,d", [(32, 8, 128), (40, 8, 128), (4, 4, 128), (16, 8, 64), (8, 2, 256),
                                      (2, 1, 128)])
def test_head_layouts(hq, hkv, d):
    check_case(Case(37, seed=hq * 7 + hkv + d, hq=hq, hkv=hkv, d=d))


@pytest.mark.parametrize("seed", range(8))
def test_random_layouts(seed):
    """Seeded random cases: token counts 1-700, head layouts including very wide ones (more than 1024 / (D / 16)
    rows per token: the flattened (token, row) kernel), row padding, 2-byte-offset views and random slots / -1
    padding."""
    rng = np.random.default_rng(500 + seed)
    layouts = [(16, 8, 128), (128, 8, 128), (64, 8, 256), (6, 2, 64), (32, 4, 128), (8, 8, 256), (96, 16, 128),
               (2, 2, 64)]
    hq, hkv, d = layouts[seed]
    tokens = int(rng.integers(1, 701))
    check_case(Case(tokens, seed=3000 + seed, hq=hq, hkv=hkv, d=d, pad=int(rng.integers(0, 3)) * 8,
                    offset=int(seed % 4 == 1)))


def test_unaligned_views():
    # q/k/v start 2 bytes into the buffer: the kernel takes its unaligned (2-byte access) path
    check_case(Case(45, seed=5, offset=1, pad=3))


def test_write_k_false_and_no_cache():
    case = Case(33, seed=9)
    q_a, k_a, cache_a = case.run(write_k=True)
    q_b, k_b, cache_b = case.run(write_k=False)
    assert k_b is None and torch.equal(q_a, q_b) and torch.equal(cache_a, cache_b)
    q_c, k_c, cache_c = case.run(write_k=True, store=False)
    assert torch.equal(q_a, q_c) and torch.equal(k_a, k_c) and torch.equal(cache_c, case.cache0)
    q_d, k_d, _ = case.run(write_k=False, store=False)
    assert k_d is None and torch.equal(q_a, q_d)


def test_zero_tokens():
    case = Case(0, seed=1, num_blocks=1)
    q_out, k_out, cache = case.run()
    assert q_out.shape == (0, Q_HEADS, HEAD_DIM) and k_out.shape == (0, KV_HEADS, HEAD_DIM)
    assert torch.equal(cache, case.cache0)


def test_all_slots_padding():
    case = Case(20, seed=3, slots=torch.full((20,), -1, dtype=torch.int32))
    q_out, k_out, cache = case.run()
    assert torch.equal(cache, case.cache0)
    q_e, k_e = case.oracle_end_to_end()
    q_n, _, _ = case.run(identity_rope=True)
    check_end_to_end(q_out, q_e, q_n, case.oracle_norms()[0])


def test_out_of_range_slots_and_positions_are_guarded():
    # Slots outside [0, num_slots) are skipped like -1 (the reference would write out of bounds); positions past
    # the table are clamped to its last row (the reference would read out of bounds).
    T = 8
    nslots = 2 * BLOCK
    slots = torch.tensor([0, nslots, -7, 5, nslots + 100, 7, -1, 9], dtype=torch.int32)
    pos = torch.tensor([0, 1, 2, MAX_POS + 3, 4, MAX_POS - 1, 6, 10 ** 9], dtype=torch.int64)
    case = Case(T, seed=11, slots=slots, positions=pos, num_blocks=2)
    q_out, k_out, cache = case.run()
    valid = torch.tensor([True, False, False, True, False, True, False, True])
    ref_case = Case(T, seed=11, slots=torch.where(valid, slots, torch.tensor(-1, dtype=torch.int32)),
                    positions=pos.clamp(max=MAX_POS - 1), num_blocks=2)
    q_r, k_r, cache_r = ref_case.run()
    assert torch.equal(q_out, q_r) and torch.equal(k_out, k_r) and torch.equal(cache, cache_r)


def test_graph_capture_replay():
    """Recorded into a HIP graph, replayed several times with new inputs copied into the static buffers, with
    eager work and synchronisation between replays: every replay equals the eager call."""
    case = Case(64, seed=21)
    q, k, v = case.views(case.buf_dev)
    positions = case.positions.to(DEV)
    slots = case.slots.to(DEV)
    cache = case.cache0.clone()
    table = cos_sin_cache().to(DEV)
    qw, kw = case.q_w.to(DEV), case.k_w.to(DEV)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        qk_norm_rope_kv(q, k, v, positions, qw, kw, EPS, table, cache[0], cache[1], slots, True)  # warm up
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_q, out_k = qk_norm_rope_kv(q, k, v, positions, qw, kw, EPS, table, cache[0], cache[1], slots, True)
    g = torch.Generator("cpu").manual_seed(5)
    for _ in range(4):
        case.buf_dev.copy_(bf16_randn(case.buf_dev.shape, g))
        positions.copy_(torch.randint(0, MAX_POS, (64,), generator=g))
        cache.copy_(case.cache0)
        graph.replay()
        torch.cuda.synchronize()
        eager_cache = case.cache0.clone()
        e_q, e_k = qk_norm_rope_kv(q, k, v, positions, qw, kw, EPS, table, eager_cache[0], eager_cache[1], slots,
                                   True)
        torch.cuda.synchronize()
        assert torch.equal(out_q, e_q) and torch.equal(out_k, e_k) and torch.equal(cache, eager_cache)
