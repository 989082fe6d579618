"""End-to-end decode harness: a random-init Qwen3-0.6B-shaped model whose layers call the HIP kernels (backend
"hip") or the layers' own torch code (backend "torch"), a paged KV cache, prefill + greedy decode, HIP-graph
decode steps, token agreement between the backends, per-step time and kernel count (nanovllm_hip.harness.decode).
"""
