"""Greedy sampling (csrc/sampler.hip, nvhip_argmax_bf16) against the reference's greedy branch, run by torch on the
same GPU tensor: `logits.float().argmax(dim=-1)` (nanovllm/layers/sampler.py:9-10). The index must be identical:
random logits at the Qwen3 vocabulary (151936) for 1, 32 and 300 rows, exact ties (the first index wins), NaNs
(the first NaN wins), rows of -inf or of one repeated value, widths that are not a multiple of 8, strided rows
(16-byte aligned and not), a replayed HIP graph, and the C ABI without a workspace (one block per row)."""
import pytest
import torch

from nanovllm_hip.kernels import greedy_sample

pytestmark = pytest.mark.gpu

DEV = "cuda"
V = 151936


def ref(logits):
    return logits.float().argmax(dim=-1)


def randn(rows, n, seed, scale=4.0):
    g = torch.Generator("cpu").manual_seed(seed)
    return (scale * torch.randn(rows, n, generator=g)).to(torch.bfloat16).to(DEV)


@pytest.mark.parametrize("rows", [1, 32, 300])
def test_random_logits_at_the_vocabulary_size(rows):
    x = randn(rows, V, rows)
    assert torch.equal(greedy_sample(x), ref(x))


def test_ties_go_to_the_first_index():
    # bf16 logits of small integers: many exact ties of the maximum in every row
    g = torch.Generator("cpu").manual_seed(1)
    x = torch.randint(-20, 21, (64, V), generator=g).to(torch.bfloat16).to(DEV)
    got = greedy_sample(x)
    assert torch.equal(got, ref(x))
    x = torch.zeros(8, V, dtype=torch.bfloat16, device=DEV)
    for r, cols in enumerate([[5, 9], [151935, 0], [1023, 1024, 8191], [8, 7]]):
        x[r, cols] = 3.0
    assert torch.equal(greedy_sample(x), ref(x))
    assert greedy_sample(x)[:4].tolist() == [5, 0, 1023, 7]


def test_nan_counts_as_the_largest():
    x = randn(16, V, 2)
    x[0, 77] = float("nan")
    x[1, 151935] = float("nan")
    x[2, 4000] = float("nan")
    x[2, 3999] = float("nan")
    x[3, 12] = float("inf")
    x[3, 13] = float("nan")
    x[4, 100] = float("inf")
    got = greedy_sample(x)
    assert torch.equal(got, ref(x))
    assert got[:5].tolist() == [77, 151935, 3999, 13, 100]


def test_constant_and_minus_inf_rows():
    x = torch.full((4, 1000), float("-inf"), dtype=torch.bfloat16, device=DEV)
    x[1] = 0.0
    x[2] = -0.0
    x[3, 500] = 0.0
    x[3, 499] = -0.0
    assert torch.equal(greedy_sample(x), ref(x))
    assert greedy_sample(x).tolist() == [0, 0, 0, 499]


@pytest.mark.parametrize("n,pad", [(1, 0), (7, 0), (1001, 0), (8192, 0), (1001, 13), (V, 64), (V, 3)])
def test_widths_and_strided_rows(n, pad):
    base = randn(40, n + pad, n + pad)
    x = base[:, :n]
    assert torch.equal(greedy_sample(x), ref(x))
    y = base[1:, pad:pad + n] if pad else base[1:, :n]  # a row start that is not 16-byte aligned when pad % 8
    assert torch.equal(greedy_sample(y), ref(y))


def test_no_rows():
    assert greedy_sample(torch.empty(0, 10, dtype=torch.bfloat16, device=DEV)).shape == (0,)


def test_graph_replay_matches_eager():
    x = randn(32, V, 3)
    eager = greedy_sample(x)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = greedy_sample(x)
    for i in range(3):
        x.copy_(randn(32, V, 10 + i))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref(x))
    assert eager.shape == out.shape


@pytest.mark.parametrize("rows,n", [(32, V), (3, 1001), (600, 4096)])
def test_one_block_per_row_without_workspace(rows, n):
    """The C ABI without a workspace (one block per row) gives the split launch's index."""
    from nanovllm_hip import _lib
    x = randn(rows, n, 7)
    x[0, n // 3] = float("nan")
    out = torch.empty(rows, dtype=torch.int64, device=DEV)
    rc = _lib.lib().nvhip_argmax_bf16(out.data_ptr(), x.data_ptr(), rows, n, x.stride(0), None, 0,
                                      torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    assert torch.equal(out, ref(x))
    assert torch.equal(out, greedy_sample(x))
