"""The HIP kernels with the call signatures of nano-vllm's nanovllm/kernels package.

`backend` plays the role of nanovllm/kernels/__init__.py:5 (set from Config.kernel_backend, model_runner.py:83):
a model reads it once when it is built, as the reference's layers do in __init__ (layers/layernorm.py:18,
layers/activation.py:13, models/qwen3.py:73), and dispatches on the value it latched ("hip" selects these kernels;
"compile" keeps the layers' own torch code). The harness model nanovllm_hip.harness.qwen3.Qwen3 latches it so.
"""
from nanovllm_hip.kernels.matmul import (add_rms_norm_matmul, matmul, matmul_add_rms_norm,  # noqa: F401
                                          matmul_silu_and_mul, rms_norm_matmul)
from nanovllm_hip.kernels.qk_norm_rope_kv import qk_norm_rope_kv  # noqa: F401
from nanovllm_hip.kernels.rms_norm import fused_add_rms_norm, fused_add_rms_norm_, rms_norm  # noqa: F401
from nanovllm_hip.kernels.sampler import greedy_sample  # noqa: F401
from nanovllm_hip.kernels.store_kvcache import store_kvcache  # noqa: F401
from nanovllm_hip.kernels.swiglu import silu_and_mul  # noqa: F401

BACKENDS = ("compile", "hip")
backend = "hip"
