"""End-to-end greedy decode through the HIP kernels (GPU): a random-init Qwen3-0.6B-shaped model (2 layers here, to
keep the test short; bench runs of the harness use all 28), batch 4, prompts of 100-300 random tokens, paged KV in
256-slot blocks, 8 decode steps, eager and HIP-graph decode, with the HIP paged decode attention (and once with the
fp32 torch attention) shared by both backends; the hip backend's projections and LM head through the HIP GEMM (and
once through torch's F.linear).

Checks: the graph replay gives exactly the eager tokens (both backends); the hip backend's tokens equal the
torch-eager backend's, except where the torch backend's own logits had the two candidates within one bf16 step of
each other (a tie broken by a last-bit difference: nano-vllm's tests/test_greedy.py also reports cross-backend
agreement rather than requiring it); the hip decode step launches fewer kernels than the torch one (the fused
pre-attention kernel replaces q_norm, k_norm, rotary and the KV scatter).
"""
import pytest

from nanovllm_hip.harness import decode

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("attention,linear,fp32_logits", [("hip", "hip", False), ("hip", "hip", True),
                                                           ("hip", "torch", False), ("torch", "torch", False)])
def test_decode_hip_vs_torch(attention, linear, fp32_logits):
    args = ["--layers", "2", "--batch", "4", "--steps", "8", "--min-len", "100", "--max-len", "300", "--reps", "2",
            "--attention", attention, "--linear", linear]
    out = decode.main(args + (["--fp32-logits"] if fp32_logits else []))
    assert out["graph_equals_eager"] == {"hip": True, "torch": True}
    agree = out["tokens_hip_vs_torch_eager"]
    if agree["identical"] != agree["total"]:
        for req, d in out["divergence"].items():
            assert d["logit_gap"] <= 0.0625, (req, d)
    g = out["decode_step_graph"]
    assert g["hip"]["kernels"] < g["torch"]["kernels"]
