"""End-to-end greedy decode through the HIP kernels (GPU): a random-init Qwen3-0.6B-shaped model, paged KV in
256-slot blocks, eager and HIP-graph decode, the "hip" backend against the "torch" backend (the layers' own torch
code run eagerly -- the torch-eager path the reference's kernels stand in for).

With --linear torch both backends run the same projections (torch's F.linear) and differ only in the four kernels
of the path (RMSNorm, Add+RMSNorm, the fused q/k norm + RoPE + KV write, SiLU x Mul; with the HIP attention also the
decode step's fused pre-attention + attention launch). Those are bitwise torch-eager on the GPU, so every generated
token must be identical: the full-size case is the batch-32 greedy decode of Qwen3-0.6B (28 layers, 32 requests with
prompts of U[512, 2048] random ids, 32 decode steps: 1056 tokens). With --linear hip the projections run on the HIP
GEMM, whose fp32 sums are in another order than hipBLASLt's: tokens may then differ where the torch backend's own top two logits
are within a bf16 step (nano-vllm's tests/test_greedy.py reports cross-backend agreement rather than requiring it
for that reason); every such divergence must be such a near-tie. In every mode the graph replay gives exactly the
eager tokens (the reference's MUST_MATCH pairs), and the hip decode step launches fewer kernels than the torch one.
"""
import pytest

from nanovllm_hip.harness import decode

pytestmark = pytest.mark.gpu


def run(args):
    out = decode.main(args)
    print({k: out[k] for k in ("tokens_hip_vs_torch_eager", "graph_equals_eager", "decode_step_graph")}, flush=True)
    assert out["graph_equals_eager"] == {"hip": True, "torch": True}
    g = out["decode_step_graph"]
    assert g["hip"]["kernels"] < g["torch"]["kernels"]
    return out


def check_near_ties(out):
    agree = out["tokens_hip_vs_torch_eager"]
    if agree["identical"] != agree["total"]:
        for req, d in out["divergence"].items():
            assert d["logit_gap"] <= 0.0625, (req, d)


@pytest.mark.parametrize("attention,linear,fp32_logits", [("hip", "hip", False), ("hip", "hip", True),
                                                           ("hip", "torch", False), ("torch", "torch", False)])
def test_decode_small(attention, linear, fp32_logits):
    args = ["--layers", "2", "--batch", "4", "--steps", "8", "--min-len", "100", "--max-len", "300", "--reps", "2",
            "--attention", attention, "--linear", linear]
    out = run(args + (["--fp32-logits"] if fp32_logits else []))
    if linear == "torch":
        agree = out["tokens_hip_vs_torch_eager"]
        assert agree["identical"] == agree["total"], out["divergence"]
    else:
        check_near_ties(out)


def test_decode_batch32_full_model_token_identical():
    """The batch-32 greedy decode at full size: the four kernels only (--linear torch), 32 decode steps after
    the first token: 32 x 33 tokens, every one identical to the torch-eager backend's."""
    out = run(["--layers", "28", "--batch", "32", "--steps", "32", "--min-len", "512", "--max-len", "2048",
               "--reps", "2", "--linear", "torch"])
    agree = out["tokens_hip_vs_torch_eager"]
    assert agree["total"] == 32 * 33
    assert agree["identical"] == agree["total"], out["divergence"]


def test_decode_batch32_full_model_hip_gemm():
    """The same decode with the HIP GEMM for every projection and the LM head: graph = eager, and every request
    that diverges from torch-eager does so at a near-tie of the torch backend's logits."""
    out = run(["--layers", "28", "--batch", "32", "--steps", "32", "--min-len", "512", "--max-len", "2048",
               "--reps", "2", "--linear", "hip"])
    check_near_ties(out)
