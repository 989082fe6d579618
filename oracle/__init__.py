"""CPU oracle for the nano-vllm kernel path — TEST INFRASTRUCTURE ONLY.

A plain-torch fp32 restatement of the reference's eager torch code (the code its Triton kernels replace), run on
CPU tensors with the same rounding points. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it, and only as the reference results are compared with or as the timed CPU baseline; the product path
(nanovllm_hip) never calls it.

Functions and the reference code each one follows (paths in R3pere/nano-vllm-triton-kernels):
  rms_forward        nanovllm/layers/layernorm.py:20-30   (RMSNorm.rms_forward)
  add_rms_forward    nanovllm/layers/layernorm.py:32-44   (RMSNorm.add_rms_forward)
  rms_forward_gpu, add_rms_forward_gpu
                     the same two functions with the numerics torch gives them when they run eagerly on the GPU
                     (the reference's torch path on an MI355X): the mean of squares in ATen's GPU summation order
                     (aten_reduce, restated from torch's open-source ATen/native/hip/Reduce.cuh) and torch.rsqrt's
                     double-precision evaluation rounded to float
  rope_cos_sin_cache nanovllm/layers/rotary_embedding.py:19-35 (RotaryEmbedding.__init__ cache)
  apply_rotary_emb   nanovllm/layers/rotary_embedding.py:6-14
  rotary_forward     nanovllm/layers/rotary_embedding.py:37-48 (RotaryEmbedding.forward)
  store_kvcache      nanovllm/layers/attention.py:11-41   (store_kvcache_kernel / store_kvcache)
  qk_norm_rope_kv    nanovllm/models/qwen3.py:89-105 + nanovllm/layers/attention.py:64-76 (the unfused composition
                     that nanovllm/kernels/qk_norm_rope_kv.py:92-125 replaces)
  silu_and_mul       nanovllm/layers/activation.py:15-18
  matmul_fp64        tests/test_kernels_matmul.py:52 (A.double() @ B.double())
  paged_decode_attention  nanovllm/layers/attention.py:84-90 (flash_attn_with_kvcache on the paged cache, decode),
                     slot formula model_runner.py:340; flash-attn is not vendored in the reference (an unpinned
                     pyproject dependency), so its documented semantics (bottom-right causal mask, GQA head h -> kv
                     head h // (Hq / Hkv)) are restated and pinned by float64 SDPA, closed forms and invariants
  varlen_attention   nanovllm/layers/attention.py:77-83 (flash_attn_varlen_func, prefill, with the prefix-cache block
                     table of model_runner.py:311-312); pinned like the decode attention and by agreeing with it on
                     one-query sequences

How each is pinned (tests/test_oracle.py): closed forms in float64, hand-computed known answers, invariants
(identity rotation, norm preservation, relative-position dependence, scale invariance), and brute-force loops on
tiny inputs. The reference ships no golden vectors for this path.
"""
from oracle import aten_reduce  # noqa: F401
from oracle.torch_ref import (  # noqa: F401
    add_rms_forward,
    add_rms_forward_gpu,
    rms_forward_gpu,
    apply_rotary_emb,
    matmul_fp64,
    paged_decode_attention,
    varlen_attention,
    qk_norm_rope_kv,
    rms_forward,
    rope_cos_sin_cache,
    rotary_forward,
    silu_and_mul,
    store_kvcache,
)
