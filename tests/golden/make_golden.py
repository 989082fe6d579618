"""Writes the golden fixtures of tests/golden/ from the CPU oracle (run from the repo root:
`python tests/golden/make_golden.py`). The reference ships no fixtures for this path; these pin the oracle's outputs
on small seeded inputs so that the oracle (tests/test_golden.py) and the HIP kernels (GPU tests) are checked
against the same committed numbers. bf16 tensors are stored as their uint16 bit patterns.

  qk_norm_rope_kv_t16.npz  fused qk-norm + RoPE + paged-KV write, Qwen3-0.6B attention shape, 16 tokens: qkv
                           [16, 4096] ~N(0,1), norm weights 1+0.1*N(0,1), eps 1e-6, positions U[0, 4096), RoPE
                           theta 1e6 / max_pos 40960, caches [64, 256, 8, 128] zero-initialised, 16 distinct random
                           slots. Outputs: q_out, k_out, the normed q/k (before RoPE) and the written
                           cache rows.
  norm_act_t16.npz         rms_norm / fused_add_rms_norm at hidden 1024 and 128, silu_and_mul at 2 x 3072, 16 rows.
  The *_gpu arrays are the same outputs with the numerics torch gives the reference's code on the GPU
  (oracle.rms_forward_gpu: ATen's GPU summation order, torch.rsqrt's double evaluation), which the kernels match
  bit for bit.
  matmul_small.npz         fp32 and bf16 A @ B for (M, N, K) = (7, 33, 65) and (20, 40, 300); B stored [N, K].
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def make_qk(seed=0):
    g = torch.Generator("cpu").manual_seed(seed)
    T, Hq, Hkv, D, eps = 16, 16, 8, 128, 1e-6
    qkv = torch.randn(T, (Hq + 2 * Hkv) * D, generator=g).to(torch.bfloat16)
    q_w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    k_w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    positions = torch.randint(0, 4096, (T,), generator=g)
    slots = torch.randperm(64 * 256, generator=g)[:T].to(torch.int32)
    q, k, v = (t.view(T, -1, D) for t in qkv.split([Hq * D, Hkv * D, Hkv * D], dim=-1))
    cos_sin = oracle.rope_cos_sin_cache(D, 40960, 1e6)
    k_cache = torch.zeros(64, 256, Hkv, D, dtype=torch.bfloat16)
    v_cache = torch.zeros_like(k_cache)
    q_out, k_out = oracle.qk_norm_rope_kv(q, k, v, positions, q_w, k_w, eps, cos_sin, k_cache, v_cache, slots, True)
    empty = torch.empty(0)
    q_gpu, k_gpu = oracle.qk_norm_rope_kv(q, k, v, positions, q_w, k_w, eps, cos_sin, empty, empty, None, True,
                                          gpu_numerics=True)
    rows = slots.long()
    return dict(qkv=bits(qkv), q_weight=bits(q_w), k_weight=bits(k_w), positions=positions.numpy(),
                slot_mapping=slots.numpy(), eps=np.float32(eps), q_out=bits(q_out), k_out=bits(k_out),
                q_out_gpu=bits(q_gpu), k_out_gpu=bits(k_gpu),
                q_normed=bits(oracle.rms_forward(q, q_w, eps)), k_normed=bits(oracle.rms_forward(k, k_w, eps)),
                k_cache_rows=bits(k_cache.view(-1, Hkv, D)[rows]), v_cache_rows=bits(v_cache.view(-1, Hkv, D)[rows]))


def make_norm_act(seed=1):
    g = torch.Generator("cpu").manual_seed(seed)
    out = {}
    for n in (1024, 128):
        x = torch.randn(16, n, generator=g).to(torch.bfloat16)
        r = torch.randn(16, n, generator=g).to(torch.bfloat16)
        w = (1 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16)
        y_add, s = oracle.add_rms_forward(x, r, w, 1e-6)
        out.update({f"x_{n}": bits(x), f"r_{n}": bits(r), f"w_{n}": bits(w),
                    f"rms_{n}": bits(oracle.rms_forward(x, w, 1e-6)), f"add_y_{n}": bits(y_add),
                    f"add_res_{n}": bits(s), f"rms_gpu_{n}": bits(oracle.rms_forward_gpu(x, w, 1e-6)),
                    f"add_y_gpu_{n}": bits(oracle.add_rms_forward_gpu(x, r, w, 1e-6)[0])})
    gu = torch.randn(16, 6144, generator=g).to(torch.bfloat16)
    out.update(gate_up=bits(gu), silu=bits(oracle.silu_and_mul(gu)))
    return out


def make_matmul(seed=2):
    g = torch.Generator("cpu").manual_seed(seed)
    out = {}
    for (M, N, K) in ((7, 33, 65), (20, 40, 300)):
        a = torch.randn(M, K, generator=g)
        w = torch.randn(N, K, generator=g)
        out[f"a_f32_{M}_{N}_{K}"] = a.numpy()
        out[f"w_f32_{M}_{N}_{K}"] = w.numpy()
        out[f"c_f64_{M}_{N}_{K}"] = oracle.matmul_fp64(a, w.t()).numpy()
        ab, wb = a.to(torch.bfloat16), w.to(torch.bfloat16)
        out[f"a_bf16_{M}_{N}_{K}"] = bits(ab)
        out[f"w_bf16_{M}_{N}_{K}"] = bits(wb)
        out[f"cb_f64_{M}_{N}_{K}"] = oracle.matmul_fp64(ab, wb.t()).numpy()
    return out


def main():
    np.savez_compressed(os.path.join(HERE, "qk_norm_rope_kv_t16.npz"), **make_qk())
    np.savez_compressed(os.path.join(HERE, "norm_act_t16.npz"), **make_norm_act())
    np.savez_compressed(os.path.join(HERE, "matmul_small.npz"), **make_matmul())
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
