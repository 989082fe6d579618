"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py from the oracle) are
reproduced by the oracle from their stored inputs (CPU only). The GPU tests check the HIP kernels against the same
files."""
import math
import os

import numpy as np
import torch

import oracle

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def u16(z, name):
    return torch.from_numpy(z[name].astype(np.int16)).view(torch.bfloat16)


def test_qk_norm_rope_kv_fixture():
    z = np.load(os.path.join(HERE, "qk_norm_rope_kv_t16.npz"))
    T, Hq, Hkv, D = 16, 16, 8, 128
    qkv = u16(z, "qkv")
    assert qkv.shape == (T, (Hq + 2 * Hkv) * D)
    q, k, v = (t.view(T, -1, D) for t in qkv.split([Hq * D, Hkv * D, Hkv * D], dim=-1))
    slots = torch.from_numpy(z["slot_mapping"])
    positions = torch.from_numpy(z["positions"])
    assert slots.dtype == torch.int32 and len(set(slots.tolist())) == T and positions.max() < 4096
    kc = torch.zeros(64, 256, Hkv, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    qw, kw, eps = u16(z, "q_weight"), u16(z, "k_weight"), float(z["eps"])
    q_out, k_out = oracle.qk_norm_rope_kv(q, k, v, positions, qw, kw, eps, oracle.rope_cos_sin_cache(D, 40960, 1e6),
                                          kc, vc, slots, True)
    assert torch.equal(q_out, u16(z, "q_out")) and torch.equal(k_out, u16(z, "k_out"))
    empty = torch.empty(0)
    q_g, k_g = oracle.qk_norm_rope_kv(q, k, v, positions, qw, kw, eps, oracle.rope_cos_sin_cache(D, 40960, 1e6),
                                      empty, empty, None, True, gpu_numerics=True)
    assert torch.equal(q_g, u16(z, "q_out_gpu")) and torch.equal(k_g, u16(z, "k_out_gpu"))
    assert torch.equal(oracle.rms_forward(q, qw, eps), u16(z, "q_normed"))
    assert torch.equal(oracle.rms_forward(k, kw, eps), u16(z, "k_normed"))
    rows = slots.long()
    assert torch.equal(kc.view(-1, Hkv, D)[rows], u16(z, "k_cache_rows"))
    assert torch.equal(vc.view(-1, Hkv, D)[rows], u16(z, "v_cache_rows"))
    assert torch.equal(u16(z, "v_cache_rows"), v)


def test_norm_act_fixture():
    z = np.load(os.path.join(HERE, "norm_act_t16.npz"))
    for n in (1024, 128):
        x, r, w = u16(z, f"x_{n}"), u16(z, f"r_{n}"), u16(z, f"w_{n}")
        assert torch.equal(oracle.rms_forward(x, w, 1e-6), u16(z, f"rms_{n}"))
        y, s = oracle.add_rms_forward(x, r, w, 1e-6)
        assert torch.equal(y, u16(z, f"add_y_{n}")) and torch.equal(s, u16(z, f"add_res_{n}"))
        assert torch.equal(oracle.rms_forward_gpu(x, w, 1e-6), u16(z, f"rms_gpu_{n}"))
        assert torch.equal(oracle.add_rms_forward_gpu(x, r, w, 1e-6)[0], u16(z, f"add_y_gpu_{n}"))
    assert torch.equal(oracle.silu_and_mul(u16(z, "gate_up")), u16(z, "silu"))


def test_matmul_fixture():
    z = np.load(os.path.join(HERE, "matmul_small.npz"))
    for (M, N, K) in ((7, 33, 65), (20, 40, 300)):
        a, w = torch.from_numpy(z[f"a_f32_{M}_{N}_{K}"]), torch.from_numpy(z[f"w_f32_{M}_{N}_{K}"])
        np.testing.assert_allclose(oracle.matmul_fp64(a, w.t()).numpy(), z[f"c_f64_{M}_{N}_{K}"], rtol=1e-12,
                                   atol=1e-12 * math.sqrt(K))
        ab, wb = u16(z, f"a_bf16_{M}_{N}_{K}"), u16(z, f"w_bf16_{M}_{N}_{K}")
        np.testing.assert_allclose(oracle.matmul_fp64(ab, wb.t()).numpy(), z[f"cb_f64_{M}_{N}_{K}"], rtol=1e-12,
                                   atol=1e-12 * math.sqrt(K))
