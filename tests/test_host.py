"""Host-side behaviour of the Python layer (CPU only): the reference's argument assertions, output shapes through
the ops' fake (meta) implementations, and no CPU fallback (CPU tensors are refused by the dispatcher)."""
import pytest
import torch

from nanovllm_hip.kernels import fused_add_rms_norm, matmul, qk_norm_rope_kv, rms_norm, silu_and_mul

BF16 = torch.bfloat16


def qk_args(device="meta", T=5, Hq=16, Hkv=8, D=128, store=True, dtype=BF16):
    qkv = torch.empty(T, (Hq + 2 * Hkv) * D + 64, dtype=dtype, device=device)
    q = qkv[:, :Hq * D].view(T, Hq, D)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].view(T, Hkv, D)
    v = qkv[:, (Hq + Hkv) * D:(Hq + 2 * Hkv) * D].view(T, Hkv, D)
    cache = (torch.empty(4, 256, Hkv, D, dtype=BF16, device=device) if store
             else torch.empty(0, device=device))
    return dict(q=q, k=k, v=v, positions=torch.empty(T, dtype=torch.int64, device=device),
                q_weight=torch.empty(D, dtype=BF16, device=device), k_weight=torch.empty(D, dtype=BF16, device=device),
                eps=1e-6, cos_sin_cache=torch.empty(40960, 1, D, device=device), k_cache=cache,
                v_cache=cache.clone() if store else cache,
                slot_mapping=torch.empty(T, dtype=torch.int32, device=device) if store else None, write_k=True)


def test_qk_shapes_through_fake_impl():
    q_out, k_out = qk_norm_rope_kv(**qk_args())
    assert q_out.shape == (5, 16, 128) and k_out.shape == (5, 8, 128) and q_out.is_contiguous()
    a = qk_args()
    a["write_k"] = False
    assert qk_norm_rope_kv(**a)[1] is None
    q_out, k_out = qk_norm_rope_kv(**qk_args(store=False))
    assert q_out.shape == (5, 16, 128)


@pytest.mark.parametrize("bad", ["dtype", "head_dim", "gqa", "stride", "positions", "cache", "slots", "table"])
def test_qk_assertions(bad):
    a = qk_args()
    if bad == "dtype":
        a = qk_args(dtype=torch.float16)
    elif bad == "head_dim":
        a = qk_args(D=96)
    elif bad == "gqa":
        a = qk_args(Hq=12, Hkv=8)
    elif bad == "stride":
        a["q"] = torch.empty(5, 128, 16, dtype=BF16, device="meta").transpose(1, 2)
    elif bad == "positions":
        a["positions"] = a["positions"].to(torch.int32)
    elif bad == "cache":
        a["k_cache"] = torch.empty(4, 256, 8, 256, dtype=BF16, device="meta")[..., :128]
    elif bad == "slots":
        a["slot_mapping"] = None
    elif bad == "table":
        a["cos_sin_cache"] = torch.empty(40960, 1, 128, dtype=BF16, device="meta")
    with pytest.raises(AssertionError):
        qk_norm_rope_kv(**a)


def test_norm_silu_matmul_shapes_and_assertions():
    x = torch.empty(7, 1024, dtype=BF16, device="meta")
    w = torch.empty(1024, dtype=BF16, device="meta")
    assert rms_norm(x, w, 1e-6).shape == (7, 1024)
    assert rms_norm(torch.empty(7, 16, 128, dtype=BF16, device="meta"), w[:128], 1e-6).shape == (7, 16, 128)
    y, s = fused_add_rms_norm(x, x, w, 1e-6)
    assert y.shape == s.shape == (7, 1024)
    assert silu_and_mul(torch.empty(7, 6144, dtype=BF16, device="meta")).shape == (7, 3072)
    a = torch.empty(32, 1024, dtype=BF16, device="meta")
    b = torch.empty(4096, 1024, dtype=BF16, device="meta").t()
    assert matmul(a, b).shape == (32, 4096)
    with pytest.raises(AssertionError):
        fused_add_rms_norm(x, torch.empty(7, 512, dtype=BF16, device="meta"), w, 1e-6)
    with pytest.raises(AssertionError):
        rms_norm(x.float(), w, 1e-6)
    with pytest.raises(AssertionError):
        matmul(a, b.float())
    with pytest.raises(AssertionError):
        matmul(a, b, input_precision="bf16x3")
    with pytest.raises(AssertionError):
        matmul(a, torch.empty(512, 4096, dtype=BF16, device="meta"))


def test_no_cpu_fallback():
    """The ops have no CPU kernel: CPU tensors fail loudly in the dispatcher instead of running a slow path."""
    x = torch.randn(4, 256).to(BF16)
    w = torch.ones(256, dtype=BF16)
    with pytest.raises(NotImplementedError):
        rms_norm(x, w, 1e-6)
    with pytest.raises(NotImplementedError):
        silu_and_mul(x)
    with pytest.raises(NotImplementedError):
        matmul(x, x.t())
    with pytest.raises(NotImplementedError):
        qk_norm_rope_kv(**qk_args(device="cpu"))


def test_model_latches_the_kernel_backend_at_construction():
    # the reference's layers read nanovllm.kernels.backend once, in __init__ (layers/layernorm.py:18); so does the
    # harness model, and a later change of the module value does not reach a model already built
    import nanovllm_hip.kernels as kernels
    from nanovllm_hip.harness.qwen3 import Qwen3, Qwen3Config
    cfg = Qwen3Config(vocab_size=64, hidden_size=64, intermediate_size=128, num_hidden_layers=1,
                      num_attention_heads=2, num_key_value_heads=1, head_dim=64, max_position_embeddings=16)
    old = kernels.backend
    try:
        kernels.backend = "compile"
        model = Qwen3(cfg, "meta")
        kernels.backend = "hip"
        assert model.kernel_backend == "torch"
        assert Qwen3(cfg, "meta").kernel_backend == "hip"
        assert Qwen3(cfg, "meta", kernel_backend="compile").kernel_backend == "torch"
        kernels.backend = "triton"
        with pytest.raises(ValueError):
            Qwen3(cfg, "meta")
    finally:
        kernels.backend = old
