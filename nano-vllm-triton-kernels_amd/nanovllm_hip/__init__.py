"""nanovllm_hip — MI355X (gfx950) HIP kernels for nano-vllm's kernel path, behind kernel_backend="hip".

nanovllm_hip.kernels mirrors nano-vllm's nanovllm/kernels package (same function names, arguments, return values
and assertion behaviour): qk_norm_rope_kv, rms_norm, fused_add_rms_norm, silu_and_mul, matmul. They run through
the `nvhip` torch custom ops (nanovllm_hip.ops) on the C-ABI library libnvhip.so (include/nvhip.h).
"""
