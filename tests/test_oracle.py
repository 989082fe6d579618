"""Pins the CPU oracle (oracle/torch_ref.py) independently of its own formulas (CPU only).

The reference ships no golden vectors for this path, so each oracle function is checked against what the
mathematics fixes, chosen so that a plausible slip (a dropped term, a wrong sign, a swapped half, a wrong index or
divisor, a missing rounding, a transposed operand) fails at least one check:
  rms_forward       hand-computed known answers; float64 closed form; float64 emulation of the rounding points;
                    power-of-two scale invariance (eps = 0); eps visible on tiny rows
  add_rms_forward   residual = exact float64 sum rounded once; y = RMSNorm of the *unrounded* sum; r = 0 reduces to
                    rms_forward
  rope table        float64 cos/sin of p / theta^(2i/D) at small p; layout [max_pos, 1, (cos | sin)]
  apply_rotary_emb  identity table; complex multiplication (x1 + i x2) e^{i angle} in float64; norm preservation;
                    dot products depend only on the position difference; hand-computed 90-degree rotation
  store_kvcache     brute-force per-element loop with the flat slot formula block * block_size + offset
  qk_norm_rope_kv   identity rotation reduces it to the norms; cache rows equal k_out / raw v; empty cache no-op
  silu_and_mul      float64 closed form; known answers at 0 and large |g|; gate/up order
  matmul_fp64       brute-force triple loop on the reference's tiny shapes
  paged_decode_attention  float64 torch SDPA on the gathered, GQA-expanded K/V with an explicit bottom-right mask;
                    equal keys give the mean of exactly the visible values (visible count, head mapping); a dominant
                    key one past the causal limit does not leak in, one at the limit wins; relocating blocks, -1
                    padding and NaN in unused slots change nothing; an empty context gives zeros
"""
import math

import numpy as np
import pytest
import torch

import oracle

BF16 = torch.bfloat16


def bits_f32_to_bf16_round(x32: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even), returned as float32. Independent of torch."""
    u = np.ascontiguousarray(x32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32)


def f64(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.float64).numpy()


def ulps(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    def line(t):
        i = t.contiguous().view(torch.int16).to(torch.int32)
        return torch.where(i < 0, -(i & 0x7FFF), i)
    return (line(a) - line(b)).abs()


# ------------------------------------------------------------------ RMSNorm

def test_rms_known_answer():
    # x = [3, 4, 0, 0], eps = 0: mean(x^2) = 25/4, x * rsqrt = [1.2, 1.6, 0, 0] -> bf16 [1.203125, 1.6015625, 0, 0]
    # (a divisor of n-1 would give 1.039/1.386; a mean of |x| 1.714/2.286)
    x = torch.tensor([[3.0, 4.0, 0.0, 0.0]], dtype=BF16)
    y = oracle.rms_forward(x, torch.ones(4, dtype=BF16), 0.0)
    assert y.tolist() == [[1.203125, 1.6015625, 0.0, 0.0]]
    # weight 2 doubles exactly; a weight on one column touches only that column
    y2 = oracle.rms_forward(x, torch.tensor([2.0, 1.0, 1.0, 1.0], dtype=BF16), 0.0)
    assert y2.tolist() == [[2.40625, 1.6015625, 0.0, 0.0]]
    # constant row: x * rsqrt(x^2 + eps) ~ 1 -> y = w; zero row stays 0 (eps keeps it finite)
    w = torch.tensor([0.5, -1.25, 3.0, 1.0], dtype=BF16)
    yc = oracle.rms_forward(torch.full((1, 4), 7.0, dtype=BF16), w, 1e-6)
    assert torch.equal(yc[0], w)
    assert torch.equal(oracle.rms_forward(torch.zeros(1, 4, dtype=BF16), w, 1e-6), torch.zeros(1, 4, dtype=BF16))


@pytest.mark.parametrize("n", [128, 1024])
def test_rms_closed_form_float64(n):
    g = torch.Generator().manual_seed(n)
    x = torch.randn(64, n, generator=g)
    x[1] *= 1e-3  # mean(x^2) ~ 1e-6: eps = 1e-6 changes the result by ~sqrt(2), so a dropped eps fails
    x[2] *= 300.0
    x = x.to(BF16)
    w = (1 + 0.1 * torch.randn(n, generator=g)).to(BF16)
    eps = 1e-6
    xd = f64(x)
    y64 = xd / np.sqrt((xd ** 2).mean(axis=-1, keepdims=True) + eps) * f64(w)
    y = oracle.rms_forward(x, w, eps)
    ref = torch.from_numpy(bits_f32_to_bf16_round(y64.astype(np.float32))).to(BF16)
    assert int(ulps(y, ref).max()) <= 2


@pytest.mark.parametrize("n", [128, 1024])
def test_rms_rounding_points(n):
    """Float64 emulation of the rounding points: n = bf16(fp32(x * rstd)), y = bf16(fp32(n * w)). The float64 sum of
    squares is order-free, so the torch oracle must agree bitwise on all but a few elements (a summation-order flip);
    a missing rounding before the weight multiply would differ on a large fraction."""
    g = torch.Generator().manual_seed(7 + n)
    x = torch.randn(256, n, generator=g).to(BF16)
    w = (1 + 0.1 * torch.randn(n, generator=g)).to(BF16)
    eps = 1e-6
    xd = f64(x)
    mean = np.float32((xd ** 2).mean(axis=-1, keepdims=True))
    rstd = (np.float32(1.0) / np.sqrt(mean + np.float32(eps), dtype=np.float32)).astype(np.float32)
    normed = bits_f32_to_bf16_round((xd.astype(np.float32) * rstd).astype(np.float32))
    y = bits_f32_to_bf16_round((normed * f64(w).astype(np.float32)).astype(np.float32))
    got = oracle.rms_forward(x, w, eps).float().numpy()
    assert np.mean(got == y) > 0.999
    assert np.max(np.abs(got - y) / np.maximum(np.abs(y), 1e-30)) < 2 ** -6  # at most a couple of bf16 steps


def test_rms_scale_invariance():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(32, 128, generator=g).to(BF16)
    w = (1 + 0.1 * torch.randn(128, generator=g)).to(BF16)
    y = oracle.rms_forward(x, w, 0.0)
    for k in (-6, -1, 3, 9):
        assert torch.equal(oracle.rms_forward(x * (2.0 ** k), w, 0.0), y)


def test_rms_strided_3d_view_equals_rows():
    g = torch.Generator().manual_seed(4)
    qkv = torch.randn(5, 32 * 128, generator=g).to(BF16)
    w = (1 + 0.1 * torch.randn(128, generator=g)).to(BF16)
    q = qkv[:, :16 * 128].view(5, 16, 128)
    assert torch.equal(oracle.rms_forward(q, w, 1e-6).reshape(80, 128),
                       oracle.rms_forward(q.reshape(80, 128).contiguous(), w, 1e-6))


# ------------------------------------------------------------------ torch's GPU order (oracle.aten_reduce)
# Bitwise against torch's own GPU mean in tests/test_norm_act.py (GPU); here: the launch shapes and hand-derived
# known answers that a plausible slip in the restatement (sequential or pairwise order inside a thread, the wrong
# threads per row for small row counts, the element loop of narrow rows) changes.

@pytest.mark.parametrize("n,rows,expected", [
    (64, 1, (False, 64)), (64, 2048, (False, 64)), (100, 8, (False, 64)), (128, 1, (True, 32)),
    (128, 4096, (True, 32)), (1024, 1, (True, 256)), (1024, 3, (True, 256)), (1024, 4, (True, 128)),
    (1024, 7, (True, 128)), (1024, 8, (True, 64)), (1024, 8192, (True, 64)), (2048, 1, (True, 512)),
    (2048, 2, (True, 256)), (4096, 1, (True, 512)), (2560, 100, (True, 64))])
def test_aten_launch_shapes(n, rows, expected):
    assert oracle.aten_reduce.reduce_config(n, rows) == expected


def test_aten_launch_shapes_not_restated():
    for n, rows in ((8192, 8), (130, 8)):  # a row split over waves; misaligned vector loads
        with pytest.raises(NotImplementedError):
            oracle.aten_reduce.reduce_config(n, rows)


def test_aten_order_known_answers():
    big = np.float32(2 ** 24)  # 2^24 + 1 is a tie between 2^24 and 2^24 + 2 and rounds to 2^24 (even)
    # n = 128 (32 threads, one 4-vector each): ((2^24 + 1) + 1) + 1 = 2^24; pairs would give 2^24 + 2
    y = np.zeros((1, 128), np.float32)
    y[0, :4] = [big, 1, 1, 1]
    assert oracle.aten_reduce.row_sum(y)[0] == big
    # n = 64 (64 threads of one element, then a tree of adjacent pairs): (2^24 + 1) + (1 + 1) = 2^24 + 2
    y = np.zeros((1, 64), np.float32)
    y[0, :4] = [big, 1, 1, 1]
    assert oracle.aten_reduce.row_sum(y)[0] == big + 2
    # n = 1024: y[0] = 2^24, y[1..3] = 2, y[256] = y[512] = y[768] = 1 (exact sum 2^24 + 9)
    y = np.zeros((1, 1024), np.float32)
    y[0, :4] = [big, 2, 2, 2]
    y[0, [256, 512, 768]] = 1
    # >= 8 rows, 64 threads: thread 0 sums component 0 over vectors 0, 64, 128, 192 first: 2^24 (three ties),
    # then ((2^24 + 2) + 2) + 2
    assert oracle.aten_reduce.row_sum(y, 8)[0] == big + 6
    # 4..7 rows, 128 threads: thread 0 = vectors 0 and 128 -> 2^24 + 6, thread 64 = vectors 64 and 192 -> 2,
    # halving step: 2^24 + 8
    assert oracle.aten_reduce.row_sum(y, 4)[0] == big + 8
    # 1..3 rows, 256 threads: thread 0 = 2^24 + 6, + thread 128 (1) = 2^24 + 7 -> tie -> 2^24 + 8, + (1 + 1)
    assert oracle.aten_reduce.row_sum(y, 1)[0] == big + 10
    # the mean factor for a power-of-two width is 1/n exactly, whatever the row count
    assert oracle.aten_reduce.mean_factor(1024, 12345) == np.float32(1 / 1024)


@pytest.mark.parametrize("n", [64, 100, 128, 1024, 2560, 4096])
@pytest.mark.parametrize("rows", [1, 4, 8])
def test_aten_order_sums_every_term_once(n, rows):
    # every element counted once: within the fp32 error bound of a sum of n positive terms of the float64 sum
    rng = np.random.default_rng(n + rows)
    y = rng.random((rows, n)).astype(np.float32) + 0.5
    s = oracle.aten_reduce.row_sum(y).astype(np.float64)
    exact = y.astype(np.float64).sum(axis=1)
    assert np.all(np.abs(s - exact) <= n * 2.0 ** -23 * exact)
    y2 = y.copy()
    y2[:, n // 2] += 1.0  # one term changed by 1 moves the sum by ~1
    assert np.all(np.abs(oracle.aten_reduce.row_sum(y2) - s - 1.0) < 1e-2 * exact.max() / n + 1e-3 * exact.max())


def test_gpu_numerics_norms_close_to_cpu_oracle():
    g = torch.Generator().manual_seed(8)
    for rows, n in ((3, 1024), (33, 1024), (40, 128)):
        x = torch.randn(rows, n, generator=g).to(BF16)
        r = torch.randn(rows, n, generator=g).to(BF16)
        w = (1 + 0.1 * torch.randn(n, generator=g)).to(BF16)
        assert int(ulps(oracle.rms_forward_gpu(x, w, 1e-6), oracle.rms_forward(x, w, 1e-6)).max()) <= 2
        y, s = oracle.add_rms_forward_gpu(x, r, w, 1e-6)
        y_c, s_c = oracle.add_rms_forward(x, r, w, 1e-6)
        assert int(ulps(y, y_c).max()) <= 2 and torch.equal(s, s_c)
        y0, _ = oracle.add_rms_forward_gpu(x, torch.zeros_like(x), w, 1e-6)
        assert torch.equal(y0, oracle.rms_forward_gpu(x, w, 1e-6))


# ------------------------------------------------------------------ Add + RMSNorm

def test_add_rms_residual_and_unrounded_sum():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(128, 1024, generator=g).to(BF16)
    r = torch.randn(128, 1024, generator=g).to(BF16)
    w = (1 + 0.1 * torch.randn(1024, generator=g)).to(BF16)
    y, res = oracle.add_rms_forward(x, r, w, 1e-6)
    s64 = f64(x) + f64(r)  # exact: two bf16 values always sum exactly in float64
    assert np.array_equal(res.float().numpy(), bits_f32_to_bf16_round(s64.astype(np.float32)))
    y64 = s64 / np.sqrt((s64 ** 2).mean(axis=-1, keepdims=True) + 1e-6) * f64(w)
    ref = torch.from_numpy(bits_f32_to_bf16_round(y64.astype(np.float32))).to(BF16)
    assert int(ulps(y, ref).max()) <= 2
    # normalising the rounded residual instead would be a different function: it must differ somewhere
    assert not torch.equal(y, oracle.rms_forward(res, w, 1e-6))
    # r = 0: plain RMSNorm, bitwise
    y0, res0 = oracle.add_rms_forward(x, torch.zeros_like(x), w, 1e-6)
    assert torch.equal(y0, oracle.rms_forward(x, w, 1e-6)) and torch.equal(res0, x)


# ------------------------------------------------------------------ RoPE

def test_rope_table_layout_and_values():
    D, max_pos, base = 128, 40960, 1e6
    cache = oracle.rope_cos_sin_cache(D, max_pos, base)
    assert cache.shape == (max_pos, 1, D) and cache.dtype == torch.float32
    p = np.arange(0, 17, dtype=np.float64)[:, None]
    inv = base ** (-np.arange(0, D, 2, dtype=np.float64) / D)
    ang = p * inv[None, :]
    np.testing.assert_allclose(cache[:17, 0, :D // 2].double().numpy(), np.cos(ang), atol=5e-6)
    np.testing.assert_allclose(cache[:17, 0, D // 2:].double().numpy(), np.sin(ang), atol=5e-6)
    # row 0 is the identity rotation; frequency 0 turns by exactly one radian per position
    assert torch.equal(cache[0, 0], torch.cat([torch.ones(D // 2), torch.zeros(D // 2)]))
    np.testing.assert_allclose(cache[1000, 0, 0].item(), math.cos(1000.0), atol=1e-4)


def test_rope_identity_and_known_rotation():
    g = torch.Generator().manual_seed(6)
    x = torch.randn(3, 4, 8, generator=g).to(BF16)
    ones, zeros = torch.ones(4), torch.zeros(4)
    assert torch.equal(oracle.apply_rotary_emb(x, ones, zeros), x)
    # 90 degrees (cos 0, sin 1): (x1, x2) -> (-x2, x1)
    y = oracle.apply_rotary_emb(x, zeros, ones)
    assert torch.equal(y, torch.cat([-x[..., 4:], x[..., :4]], dim=-1))


def test_rope_complex_form_and_invariants():
    D = 128
    cache = oracle.rope_cos_sin_cache(D, 40960, 1e6)
    g = torch.Generator().manual_seed(8)
    T = 64
    q = torch.randn(T, 4, D, generator=g).to(BF16)
    k = torch.randn(T, 4, D, generator=g).to(BF16)
    pos = torch.randint(0, 40960, (T,), generator=g)
    qr, kr = oracle.rotary_forward(pos, q, k, cache)
    cs = cache[pos].double().numpy()  # [T, 1, D]
    c, s = cs[..., :D // 2], cs[..., D // 2:]
    z = f64(q)[..., :D // 2] + 1j * f64(q)[..., D // 2:]
    zr = z * (c + 1j * s)
    want = np.concatenate([zr.real, zr.imag], axis=-1)
    got = f64(qr)
    assert np.all(np.abs(got - want) <= 2 ** -8 * np.abs(want) + 1e-5)
    # rotation keeps each (x1[i], x2[i]) pair's length
    np.testing.assert_allclose(np.abs(zr), np.abs(f64(qr)[..., :D // 2] + 1j * f64(qr)[..., D // 2:]),
                               rtol=2 ** -7, atol=1e-6)
    # q.k after rotation depends only on the position difference
    p1, p2 = torch.full((T,), 1000), torch.full((T,), 990)
    a1, b1 = oracle.rotary_forward(p1, q, k, cache)
    a2, b2 = oracle.rotary_forward(p1 + 3000, q, k, cache)
    _, b3 = oracle.rotary_forward(p2 + 3000, q, k, cache)
    _, b4 = oracle.rotary_forward(p2, q, k, cache)
    d1 = (f64(a1) * f64(b4)).sum(-1)
    d2 = (f64(a2) * f64(b3)).sum(-1)
    np.testing.assert_allclose(d1, d2, atol=0.1 * np.sqrt(D))


# ------------------------------------------------------------------ KV scatter

def test_store_kvcache_brute_force():
    g = torch.Generator().manual_seed(9)
    T, blocks, bs, hkv, d = 6, 3, 4, 2, 4
    k = torch.randn(T, hkv, d, generator=g).to(BF16)
    v = torch.randn(T, hkv, d, generator=g).to(BF16)
    slots = torch.tensor([5, -1, 0, 11, 7, -1], dtype=torch.int32)
    kc = torch.randn(blocks, bs, hkv, d, generator=g).to(BF16)
    vc = torch.randn(blocks, bs, hkv, d, generator=g).to(BF16)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    oracle.store_kvcache(k, v, kc, vc, slots)
    flat_k, flat_v = kc_ref.view(-1), vc_ref.view(-1)
    for t in range(T):
        s = int(slots[t])
        if s == -1:
            continue
        block, off = divmod(s, bs)
        for h in range(hkv):
            for i in range(d):
                flat_k[((block * bs + off) * hkv + h) * d + i] = k[t, h, i]
                flat_v[((block * bs + off) * hkv + h) * d + i] = v[t, h, i]
    assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref)
    assert torch.equal(kc[2, 3], k[3]) and torch.equal(vc[1, 1], v[0])  # slot 11 = block 2 offset 3; 5 = 1, 1


def test_fused_composition():
    g = torch.Generator().manual_seed(10)
    T, Hq, Hkv, D = 9, 4, 2, 128
    qkv = torch.randn(T, (Hq + 2 * Hkv) * D, generator=g).to(BF16)
    q, k, v = (t.view(T, -1, D) for t in qkv.split([Hq * D, Hkv * D, Hkv * D], dim=-1))
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(BF16)
    pos = torch.randint(0, 100, (T,), generator=g)
    slots = torch.tensor([3, -1, 0, 7, 12, 5, -1, 9, 15], dtype=torch.int32)
    cache = torch.randn(2, 4, 4, Hkv, D, generator=g).to(BF16)
    kc, vc = cache[0].clone(), cache[1].clone()
    table = oracle.rope_cos_sin_cache(D, 128, 1e6)
    q_out, k_out = oracle.qk_norm_rope_kv(q, k, v, pos, qw, kw, 1e-6, table, kc, vc, slots, True)
    # identity table: the outputs are the norms
    ident = torch.cat([torch.ones(D // 2), torch.zeros(D // 2)]).view(1, 1, D)
    qi, ki = oracle.qk_norm_rope_kv(q, k, v, torch.zeros_like(pos), qw, kw, 1e-6, ident, torch.empty(0),
                                    torch.empty(0), None, True)
    assert torch.equal(qi, oracle.rms_forward(q, qw, 1e-6)) and torch.equal(ki, oracle.rms_forward(k, kw, 1e-6))
    # cache rows: rotated k and raw v at the named slots, the rest untouched
    keep = slots >= 0
    assert torch.equal(kc.view(-1, Hkv, D)[slots[keep].long()], k_out[keep])
    assert torch.equal(vc.view(-1, Hkv, D)[slots[keep].long()], v[keep])
    untouched = torch.ones(16, dtype=torch.bool)
    untouched[slots[keep].long()] = False
    assert torch.equal(kc.view(-1, Hkv, D)[untouched], cache[0].view(-1, Hkv, D)[untouched])
    # write_k False -> None; empty cache -> nothing stored
    q2, k2 = oracle.qk_norm_rope_kv(q, k, v, pos, qw, kw, 1e-6, table, torch.empty(0), torch.empty(0), None, False)
    assert k2 is None and torch.equal(q2, q_out)


# ------------------------------------------------------------------ SiLU x Mul

def test_silu_closed_form_and_known_answers():
    g = torch.Generator().manual_seed(11)
    x = torch.randn(64, 2 * 3072, generator=g).to(BF16)
    out = oracle.silu_and_mul(x)
    gate, up = f64(x[:, :3072]), f64(x[:, 3072:])
    silu32 = (gate / (1 + np.exp(-gate))).astype(np.float32)
    want = bits_f32_to_bf16_round((bits_f32_to_bf16_round(silu32) * up.astype(np.float32)).astype(np.float32))
    got = out.float().numpy()
    assert np.mean(got == want) > 0.999
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) < 2 ** -6
    kat = torch.tensor([[0.0, 20.0, -100.0, 1.0, 3.0, 0.5, 2.0, 1.0]], dtype=BF16)
    y = oracle.silu_and_mul(kat)
    assert y[0, 0].item() == 0.0  # silu(0) = 0
    assert y[0, 1].item() == 10.0  # silu(20) = 20 in bf16, times 0.5
    assert abs(y[0, 2].item()) < 1e-30  # silu(-100) ~ -4e-42
    assert y[0, 3].item() == 0.73046875  # bf16(1/(1+e^-1) = 0.7310586) = 0.73046875, times 1
    # gate | up order: swapping the halves changes the result
    assert not torch.equal(oracle.silu_and_mul(torch.cat([x[:, 3072:], x[:, :3072]], 1)), out)


# ------------------------------------------------------------------ GEMM reference

@pytest.mark.parametrize("M,N,K", [(3, 5, 2), (7, 33, 65)])
def test_matmul_fp64_brute_force(M, N, K):
    g = torch.Generator().manual_seed(M * N * K)
    a = torch.randn(M, K, generator=g)
    b = torch.randn(N, K, generator=g).t()  # B = W.t(): a transposed operand
    c = oracle.matmul_fp64(a, b).numpy()
    al, bl = a.tolist(), b.tolist()
    for i in range(M):
        for j in range(N):
            assert abs(c[i, j] - math.fsum(al[i][kk] * bl[kk][j] for kk in range(K))) < 1e-9
    assert c.shape == (M, N)


# ------------------------------------------------------------------ paged decode attention

def _paged_setup(num_seqs=3, q_len=1, Hq=4, Hkv=2, D=16, block_size=8, lens=(5, 17, 9), seed=0, num_blocks=12):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(num_seqs, q_len, Hq, D, generator=g, dtype=torch.float64)
    kc = torch.randn(num_blocks, block_size, Hkv, D, generator=g, dtype=torch.float64)
    vc = torch.randn(num_blocks, block_size, Hkv, D, generator=g, dtype=torch.float64)
    perm = torch.randperm(num_blocks, generator=g)
    maxb = max((n + block_size - 1) // block_size for n in lens)
    bt = torch.full((num_seqs, maxb), -1, dtype=torch.int32)
    used = 0
    for b, n in enumerate(lens):
        nb = (n + block_size - 1) // block_size
        bt[b, :nb] = perm[used:used + nb].to(torch.int32)
        used += nb
    return q, kc, vc, torch.tensor(lens, dtype=torch.int32), bt


def _gather(cache, bt_row, n, block_size):
    j = torch.arange(n)
    return cache.reshape(-1, *cache.shape[2:])[bt_row.long()[j // block_size] * block_size + j % block_size]


@pytest.mark.parametrize("q_len,causal", [(1, True), (3, True), (3, False)])
def test_paged_attention_matches_sdpa_float64(q_len, causal):
    """Against torch's scaled_dot_product_attention in float64 on the gathered, GQA-expanded K/V with an explicit
    bottom-right causal mask."""
    q, kc, vc, lens, bt = _paged_setup(q_len=q_len)
    scale = 0.3
    out = oracle.paged_decode_attention(q, kc, vc, lens, bt, scale, causal, compute_dtype=torch.float64)
    for b in range(q.shape[0]):
        n = int(lens[b])
        k = _gather(kc, bt[b], n, 8).repeat_interleave(2, dim=1).permute(1, 0, 2)   # [Hq, n, D]
        v = _gather(vc, bt[b], n, 8).repeat_interleave(2, dim=1).permute(1, 0, 2)
        mask = torch.ones(q_len, n, dtype=torch.bool)
        if causal:
            mask = torch.arange(n)[None, :] <= (n - q_len + torch.arange(q_len))[:, None]
        ref = torch.nn.functional.scaled_dot_product_attention(q[b].permute(1, 0, 2), k, v, attn_mask=mask,
                                                               scale=scale)
        torch.testing.assert_close(out[b], ref.permute(1, 0, 2), rtol=1e-12, atol=1e-12)


def test_paged_attention_uniform_keys_average_visible_values():
    """Equal keys: every visible token gets the same weight, so query i of a causal step with L tokens returns the
    mean of the first L - q_len + i + 1 values -- pins the visible count of each query and the GQA head mapping."""
    q, kc, vc, lens, bt = _paged_setup(q_len=3)
    kc[:] = 0.7
    out = oracle.paged_decode_attention(q, kc, vc, lens, bt, 0.5, True, compute_dtype=torch.float64)
    for b in range(3):
        n = int(lens[b])
        v = _gather(vc, bt[b], n, 8)                                               # [n, Hkv, D]
        for i in range(3):
            visible = n - 3 + i + 1
            for h in range(4):
                expect = v[:visible, h // 2].mean(dim=0)
                torch.testing.assert_close(out[b, i, h], expect, rtol=1e-12, atol=1e-12)


def test_paged_attention_causal_boundary_and_layout_invariance():
    """A dominant key right after a query's last visible token must not leak in, one at the last visible token
    must win; moving blocks (and the table with them), -1 padding and NaN in unused slots change nothing."""
    q, kc, vc, lens, bt = _paged_setup(q_len=2, lens=(20, 20, 20), num_blocks=10)
    bs = 8
    base = oracle.paged_decode_attention(q, kc, vc, lens, bt, 1.0, True, compute_dtype=torch.float64)
    # query 0 sees tokens <= 18; plant at token 19 a key aligned with query 1's head 0 (score ~ 50 |q|, far above
    # the others) -> query 0 unchanged, query 1 head 0 returns that token's value
    big_k = kc.clone()
    slot = int(bt[0, 19 // bs]) * bs + 19 % bs
    big_k.view(-1, 2, 16)[slot, 0] = 50 * q[0, 1, 0] / q[0, 1, 0].norm()
    out = oracle.paged_decode_attention(q, big_k, vc, lens, bt, 1.0, True, compute_dtype=torch.float64)
    torch.testing.assert_close(out[0, 0], base[0, 0])
    torch.testing.assert_close(out[0, 1, 0], vc.view(-1, 2, 16)[slot, 0], rtol=1e-9, atol=1e-9)
    # relocate every block to a new physical block, fill the unused slots and the old blocks with NaN
    perm = torch.randperm(10, generator=torch.Generator().manual_seed(5))
    kc2 = torch.full((20, bs, 2, 16), float("nan"), dtype=torch.float64)
    vc2 = kc2.clone()
    bt2 = bt.clone()
    for b in range(3):
        for c in range(bt.shape[1]):
            if bt[b, c] >= 0:
                dst = int(perm[bt[b, c]]) + 10
                kc2[dst], vc2[dst] = kc[bt[b, c]], vc[bt[b, c]]
                bt2[b, c] = dst
    for b in range(3):   # slots past the context inside the last block hold NaN
        last = (20 - 1) // bs
        kc2[bt2[b, last], 20 % bs:] = float("nan")
        vc2[bt2[b, last], 20 % bs:] = float("nan")
    out2 = oracle.paged_decode_attention(q, kc2, vc2, lens, bt2, 1.0, True, compute_dtype=torch.float64)
    torch.testing.assert_close(out2, base, rtol=0, atol=0)


def test_paged_attention_empty_context_is_zero():
    q, kc, vc, lens, bt = _paged_setup()
    lens[1] = 0
    out = oracle.paged_decode_attention(q, kc, vc, lens, bt, 1.0, True, compute_dtype=torch.float64)
    assert torch.all(out[1] == 0)


# ------------------------------------------------------------------ varlen (prefill) attention

def _varlen_setup(lq=(5, 17, 1), lk=None, Hq=4, Hkv=2, D=16, seed=0):
    g = torch.Generator().manual_seed(seed)
    lk = lq if lk is None else lk
    cq = torch.tensor([0] + list(np.cumsum(lq)), dtype=torch.int32)
    ck = torch.tensor([0] + list(np.cumsum(lk)), dtype=torch.int32)
    q = torch.randn(int(cq[-1]), Hq, D, generator=g, dtype=torch.float64)
    k = torch.randn(int(ck[-1]), Hkv, D, generator=g, dtype=torch.float64)
    v = torch.randn(int(ck[-1]), Hkv, D, generator=g, dtype=torch.float64)
    return q, k, v, cq, ck


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("lq,lk", [((5, 17, 1), None), ((3, 4), (10, 4)), ((6,), (2,))])
def test_varlen_attention_matches_sdpa_float64(lq, lk, causal):
    """Per sequence against float64 scaled_dot_product_attention with an explicit bottom-right mask (prefix keys
    when lk > lq; queries with no visible key give zeros, which SDPA leaves as NaN)."""
    q, k, v, cq, ck = _varlen_setup(lq, lk)
    out = oracle.varlen_attention(q, k, v, cq, ck, 0.25, causal, compute_dtype=torch.float64)
    for b in range(len(lq)):
        q0, q1, k0, k1 = int(cq[b]), int(cq[b + 1]), int(ck[b]), int(ck[b + 1])
        nq, nk = q1 - q0, k1 - k0
        mask = torch.ones(nq, nk, dtype=torch.bool)
        if causal:
            mask = torch.arange(nk)[None, :] <= (nk - nq + torch.arange(nq))[:, None]
        ref = torch.nn.functional.scaled_dot_product_attention(
            q[q0:q1].permute(1, 0, 2), k[k0:k1].repeat_interleave(2, dim=1).permute(1, 0, 2),
            v[k0:k1].repeat_interleave(2, dim=1).permute(1, 0, 2), attn_mask=mask, scale=0.25).permute(1, 0, 2)
        seen = mask.any(dim=1)
        torch.testing.assert_close(out[q0:q1][seen], ref[seen], rtol=1e-12, atol=1e-12)
        assert torch.all(out[q0:q1][~seen] == 0)


def test_varlen_attention_causal_closed_forms():
    """Equal keys: query i of a sequence with lq queries and lk keys returns the mean of the first lk - lq + i + 1
    values; with lq == lk the first query returns exactly value 0."""
    q, k, v, cq, ck = _varlen_setup((4, 7), (9, 7))
    k[:] = 0.5
    out = oracle.varlen_attention(q, k, v, cq, ck, 1.0, True, compute_dtype=torch.float64)
    for b, (nq, nk) in enumerate([(4, 9), (7, 7)]):
        for i in range(nq):
            vis = nk - nq + i + 1
            expect = v[int(ck[b]):int(ck[b]) + vis].mean(dim=0).repeat_interleave(2, dim=0)
            torch.testing.assert_close(out[int(cq[b]) + i], expect, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(out[int(cq[1])], v[int(ck[1])].repeat_interleave(2, dim=0), rtol=0, atol=0)


def test_varlen_with_block_table_equals_contiguous_and_decode():
    """Keys read through a block table (the prefix cache) give the contiguous result; one query per sequence over
    the paged cache is exactly the decode attention."""
    q, k, v, cq, ck = _varlen_setup((3, 1, 5), (20, 9, 5), seed=4)
    bs = 4
    lk = [20, 9, 5]
    nb = sum((n + bs - 1) // bs for n in lk) + 2
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(1))
    kc = torch.full((nb, bs, 2, 16), float("nan"), dtype=torch.float64)
    vc = kc.clone()
    bt = torch.full((3, 5), -1, dtype=torch.int32)
    used = 0
    for b, n in enumerate(lk):
        for c in range((n + bs - 1) // bs):
            blk = int(perm[used]); used += 1
            bt[b, c] = blk
            rows = slice(int(ck[b]) + c * bs, int(ck[b]) + min(n, (c + 1) * bs))
            cnt = rows.stop - rows.start
            kc[blk, :cnt], vc[blk, :cnt] = k[rows], v[rows]
    ref = oracle.varlen_attention(q, k, v, cq, ck, 0.3, True, compute_dtype=torch.float64)
    paged = oracle.varlen_attention(q, kc, vc, cq, ck, 0.3, True, block_table=bt, compute_dtype=torch.float64)
    torch.testing.assert_close(paged, ref, rtol=0, atol=0)
    # one query per sequence == decode attention over the same cache
    q1 = torch.stack([q[int(cq[b + 1]) - 1] for b in range(3)])          # the last query of each sequence
    cq1 = torch.arange(4, dtype=torch.int32)
    dec = oracle.paged_decode_attention(q1[:, None], kc, vc, torch.tensor(lk, dtype=torch.int32), bt, 0.3, True,
                                        compute_dtype=torch.float64)[:, 0]
    var = oracle.varlen_attention(q1, kc, vc, cq1, ck, 0.3, True, block_table=bt, compute_dtype=torch.float64)
    torch.testing.assert_close(var, dec, rtol=0, atol=0)
