"""GPU parity of the GEMM (nvhip_matmul) against float64.

The reference's tests/test_kernels_matmul.py: torch.testing.assert_close(C, A.double() @ B.double()) with
  fp32 "ieee": rtol 1e-4,   atol 1e-4 * sqrt(K)
  fp32 "tf32": rtol 1e-2,   atol 1e-2 * sqrt(K)
  bf16:        rtol 1.6e-2, atol 1e-2 * sqrt(K)
over its shape grid (M = 1 decode rows, sizes that are not multiples of any tile, K < one K-tile) for B row-major
and B = W.t() of an nn.Linear weight, plus the guard that "ieee" is not silently tf32. Added: the Qwen3-0.6B
projection shapes at M = 32, 256 and 2048 (bf16, B = W.t(), A ~N(0,1)/sqrt(K)), rows independent of the tile
shape M selects, fp32 4096^3, strided/offset views and the committed golden products.
"""
import math
import os

import numpy as np
import pytest
import torch

import oracle
from nanovllm_hip.kernels import matmul

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = {
    ("fp32", "ieee"): (1e-4, 1e-4),
    ("fp32", "tf32"): (1e-2, 1e-2),
    ("bf16", "ieee"): (1.6e-2, 1e-2),
}
DTYPES = {"fp32": torch.float32, "bf16": torch.bfloat16}
SHAPES = [(1, 1024, 4096), (1, 3072, 1024), (7, 33, 65), (17, 129, 257), (100, 300, 70), (127, 255, 1000),
          (512, 512, 512), (1000, 1000, 1000), (3, 5, 2), (130, 260, 36), (20, 100, 200), (77, 1000, 1024)]
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "matmul_small.npz")


def check(a, b, prec, rtol_atol):
    c = matmul(a, b, input_precision=prec)
    assert c.shape == (a.shape[0], b.shape[1]) and c.dtype == a.dtype
    ref = oracle.matmul_fp64(a.cpu(), b.cpu())
    rtol, atol = rtol_atol
    torch.testing.assert_close(c.cpu().double(), ref, rtol=rtol, atol=atol * math.sqrt(max(a.shape[1], 1)))


@pytest.mark.parametrize("b_transposed", [False, True])
@pytest.mark.parametrize("dtype,prec", list(TOL))
@pytest.mark.parametrize("M,N,K", SHAPES)
def test_matmul(M, N, K, dtype, prec, b_transposed):
    g = torch.Generator("cpu").manual_seed(0)
    a = torch.randn(M, K, generator=g).to(DTYPES[dtype]).to(DEV)
    if b_transposed:
        b = torch.randn(N, K, generator=g).to(DTYPES[dtype]).to(DEV).t()
    else:
        b = torch.randn(K, N, generator=g).to(DTYPES[dtype]).to(DEV)
    check(a, b, prec, TOL[(dtype, prec)])


@pytest.mark.parametrize("M,N,K", [(33, 4096, 1024), (300, 1024, 3072), (256, 6144, 1024), (2048, 4096, 1024),
                                   (2048, 1024, 2048), (300, 200, 136), (65, 1000, 1000), (64, 8, 8)])
def test_n_contiguous_b_is_bitwise_the_k_contiguous_product(M, N, K):
    """bf16 with B row-major ([K, N], N-contiguous: the reference test's layout) runs the MFMA tile kernel with B
    staged as it lies and read through transpose reads; for M > 32 (M > 256 when K >= 2048) the K-contiguous layout
    of the same B runs the same tile shape and k order, so the two products are bitwise equal (and within the bf16
    tolerance of fp64).
    Covers N not a multiple of the tile (column clamp), K not a multiple of 64 (zero tail) and a strided B."""
    g = torch.Generator("cpu").manual_seed(M + N + K)
    a = (torch.randn(M, K, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(DEV)
    wide = torch.randn(K, N + 64, generator=g).to(torch.bfloat16).to(DEV)
    for b in (wide[:, :N].contiguous(), wide[:, :N]):   # row stride N, then N + 64
        c = matmul(a, b)
        ref_nt = matmul(a, b.t().contiguous().t())      # the same B, K-contiguous
        assert torch.equal(c, ref_nt)
    torch.testing.assert_close(c.cpu().double(), oracle.matmul_fp64(a.cpu(), b.cpu()), rtol=1.6e-2,
                               atol=1e-2 * math.sqrt(K))


def test_ieee_is_not_tf32():
    g = torch.Generator("cpu").manual_seed(0)
    a = torch.randn(256, 4096, generator=g).to(DEV)
    b = torch.randn(4096, 256, generator=g).to(DEV)
    ref = oracle.matmul_fp64(a.cpu(), b.cpu())
    err_ieee = (matmul(a, b, "ieee").cpu().double() - ref).abs().max().item()
    err_tf32 = (matmul(a, b, "tf32").cpu().double() - ref).abs().max().item()
    assert err_ieee < 1e-2 < err_tf32, (err_ieee, err_tf32)


QWEN_SHAPES = {"qkv": (1024, 4096), "gate_up": (1024, 6144), "down": (3072, 1024), "o_proj": (2048, 1024)}


@pytest.mark.parametrize("M", [32, 48, 64, 256, 2048])
@pytest.mark.parametrize("layer", list(QWEN_SHAPES))
def test_qwen_projection_shapes(layer, M):
    K, N = QWEN_SHAPES[layer]
    g = torch.Generator("cpu").manual_seed(M + K + N)
    a = (torch.randn(M, K, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(DEV)
    w = torch.randn(N, K, generator=g).to(torch.bfloat16).to(DEV)
    c = matmul(a, w.t())
    ref = oracle.matmul_fp64(a.cpu(), w.cpu().t())
    # |C| ~ 1 here (A is scaled by 1/sqrt(K)): the bf16 tolerance with atol 1e-2
    torch.testing.assert_close(c.cpu().double(), ref, rtol=1.6e-2, atol=1e-2)


@pytest.mark.parametrize("layer", list(QWEN_SHAPES))
def test_rows_do_not_depend_on_the_tile_choice(layer):
    """Every MFMA tile shape (32x64 or 64x64 with 4 k-tiles of loads in flight while they fit one round on the CUs,
    the cost model's larger tiles beyond) sums each output in the same k order, so a row of C has the same bits
    whatever M selects: rows of products with 48, 64, 100, 256 and 512 rows equal those rows of the 2048-row
    product. With
    K >= 2048 (down, o_proj) up to 256 rows run the skinny kernels' row tiles instead, whose block shapes also share
    one k order: there rows of 100- and 256-row products equal those of the 64-row product, and 512 rows equal the
    2048-row product."""
    K, N = QWEN_SHAPES[layer]
    g = torch.Generator("cpu").manual_seed(K + N)
    a = (torch.randn(2048, K, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(DEV)
    w = torch.randn(N, K, generator=g).to(torch.bfloat16).to(DEV)
    full = matmul(a, w.t())
    if K >= 2048:
        assert torch.equal(matmul(a[:512], w.t()), full[:512])
        rows64 = matmul(a[:64], w.t())
        for M in (100, 256):
            c = matmul(a[:M], w.t())
            assert torch.equal(c[:64], rows64), M
            ref = oracle.matmul_fp64(a[:M].cpu(), w.cpu().t())
            torch.testing.assert_close(c.cpu().double(), ref, rtol=1.6e-2, atol=1e-2)
        return
    for M in (48, 64, 100, 256, 512):
        assert torch.equal(matmul(a[:M], w.t()), full[:M]), M


@pytest.mark.parametrize("layer", ["down", "o_proj"])
def test_long_k_up_to_64_rows_run_in_row_tiles(layer):
    """33 to 64 rows with K >= 2048 run the decode kernels' 16-row tiles as grid rows, so a row's bits depend only
    on its tile: rows of 48- and 64-row products equal those of the 32-row product and of each other (a batch padded
    from 33 to 48 rows keeps its real rows), and the product is within the bf16 tolerance of fp64."""
    K, N = QWEN_SHAPES[layer]
    g = torch.Generator("cpu").manual_seed(K * 3 + N)
    a = (torch.randn(64, K, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(DEV)
    w = torch.randn(N, K, generator=g).to(torch.bfloat16).to(DEV)
    full = matmul(a, w.t())
    assert torch.equal(matmul(a[:32], w.t()), full[:32])
    assert torch.equal(matmul(a[:48], w.t()), full[:48])
    padded = torch.cat([a[:33], torch.zeros(15, K, dtype=a.dtype, device=DEV)])
    assert torch.equal(matmul(padded, w.t())[:33], matmul(a[:33], w.t()))
    ref = oracle.matmul_fp64(a.cpu(), w.cpu().t())
    torch.testing.assert_close(full.cpu().double(), ref, rtol=1.6e-2, atol=1e-2)


@pytest.mark.parametrize("M,N,K", [(77, 1000, 2056), (200, 520, 4104), (45, 3000, 2048)])
def test_long_k_row_tiles_ragged(M, N, K):
    """The 33-256-row, K >= 2048 route on ragged sizes: rows past M, columns past N (not a multiple of the 16- or
    32-column block), K ending inside a staged round; within the bf16 tolerance of fp64, and its first 32 rows
    bitwise the 32-row product's (every skinny block shape sums a column in the same k order)."""
    g = torch.Generator("cpu").manual_seed(M + N + K)
    a = (torch.randn(M, K, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(DEV)
    w = torch.randn(N, K, generator=g).to(torch.bfloat16).to(DEV)
    c = matmul(a, w.t())
    ref = oracle.matmul_fp64(a.cpu(), w.cpu().t())
    torch.testing.assert_close(c.cpu().double(), ref, rtol=1.6e-2, atol=1e-2)
    assert torch.equal(c[:32], matmul(a[:32], w.t()))


@pytest.mark.parametrize("M", [1, 17, 32])
@pytest.mark.parametrize("K", [776, 1024, 2048, 2056, 3072, 4104])
def test_decode_column_tilings_agree_bitwise(M, K):
    """M <= 32: the 8-wave block tilings sum a column in the same k order, so a column has the same bits in an
    8-column block (staged through LDS from K = 2048 on, N = 1024; K = 2056 / 4104 end in a partial round) and in a
    16-column block (N = 4096: the whole K staged in one LDS round up to K = 1024, K = 776 ending inside it;
    fragments loaded straight from memory beyond); the 4-wave 64-column blocks of LM-head-wide outputs (staged through LDS) agree
    with each other whatever the output width (151 936 = the Qwen3 vocabulary, 131 176 = 2049 blocks and a ragged one) and with the
    fp64 product."""
    g = torch.Generator(DEV).manual_seed(M * 131 + K)
    a = (torch.randn(M, K, generator=g, device=DEV) / math.sqrt(K)).to(torch.bfloat16)
    w = torch.randn(151936, K, generator=g, device=DEV).to(torch.bfloat16)
    mid = matmul(a, w[:4096].t())
    narrow = matmul(a, w[:1024].t())
    assert torch.equal(mid[:, :1024], narrow)
    wide = matmul(a, w.t())
    wide2 = matmul(a, w[:131176].t())
    assert torch.equal(wide[:, :131176], wide2)
    ref = oracle.matmul_fp64(a.cpu(), w[:4096].cpu().t())
    torch.testing.assert_close(wide[:, :4096].cpu().double(), ref, rtol=1.6e-2, atol=1e-2)


@pytest.mark.parametrize("M", [1, 17, 32])
def test_decode_tiles_wide_and_narrow_outputs(M):
    """M <= 32 picks its block tile by the output width: 64 columns for an LM-head-wide output (151 936 = the Qwen3
    vocabulary, not a multiple of 64), one 16-row tile x 8 columns for N = 1024, and the ragged tails of both."""
    for N, K in [(151936, 1024), (1024, 3072), (1000, 72)]:
        g = torch.Generator("cpu").manual_seed(M * 7 + N + K)
        a = (torch.randn(M, K, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(DEV)
        w = torch.randn(N, K, generator=g).to(torch.bfloat16).to(DEV)
        c = matmul(a, w.t())
        ref = oracle.matmul_fp64(a.cpu(), w.cpu().t())
        torch.testing.assert_close(c.cpu().double(), ref, rtol=1.6e-2, atol=1e-2)


def test_fp32_4096_cube():
    g = torch.Generator("cpu").manual_seed(4096)
    a = torch.randn(4096, 4096, generator=g).to(DEV)
    b = torch.randn(4096, 4096, generator=g).to(DEV)
    c = matmul(a, b, "ieee")
    # float64 reference on the GPU (a 4096^3 float64 product is minutes on the CPU)
    ref = a.double() @ b.double()
    torch.testing.assert_close(c.double(), ref, rtol=1e-4, atol=1e-4 * 64)


@pytest.mark.parametrize("M,N,K,b_transposed,prec", [
    (4096, 4096, 2048, False, "tf32"), (4096, 4096, 2048, True, "ieee"), (4096, 4096, 2048, True, "tf32"),
    (4000, 4100, 1000, False, "ieee"), (4000, 4100, 1000, True, "tf32"),  # partial tiles, K not a multiple of 32
])
def test_fp32_large_tiles(M, N, K, b_transposed, prec):
    """Products with at least 256 tiles of 256 x 256 take the 16-wave kernel with 16-byte fragment reads (k
    permuted within groups of 8): both B layouts, both precisions, ragged edges and a K tail, against float64 on the
    GPU at the reference's tolerances."""
    g = torch.Generator("cpu").manual_seed(M + N + K)
    a = torch.randn(M, K, generator=g).to(DEV)
    b = torch.randn(N, K, generator=g).to(DEV).t() if b_transposed else torch.randn(K, N, generator=g).to(DEV)
    c = matmul(a, b, prec)
    ref = a.double() @ b.double()
    rtol, atol = TOL[("fp32", prec)]
    torch.testing.assert_close(c.double(), ref, rtol=rtol, atol=atol * math.sqrt(K))
    if prec == "ieee":  # and not silently tf32: a tf32 product of the same inputs is off by far more
        assert (c.double() - ref).abs().max().item() < 1e-2 < (matmul(a, b, "tf32").double() - ref).abs().max().item()


def test_strided_views_and_empty():
    g = torch.Generator("cpu").manual_seed(5)
    big_a = torch.randn(70, 300, generator=g).to(torch.bfloat16).to(DEV)
    big_b = torch.randn(300, 310, generator=g).to(torch.bfloat16).to(DEV)
    check(big_a[3:60, 7:263], big_b[:256, 9:130], "ieee", TOL[("bf16", "ieee")])  # offset views, odd strides
    check(big_a[::2, :128], big_b[10:138, ::2], "ieee", TOL[("bf16", "ieee")])  # non-unit strides
    check(big_a.float()[:, :64], big_b.float()[:64, :33].t().contiguous().t(), "ieee", TOL[("fp32", "ieee")])
    z = matmul(big_a[:, :0], big_b[:0, :5])
    assert z.shape == (70, 5) and not z.any()
    assert matmul(big_a[:0], big_b[:300, :5]).shape == (0, 5)


def test_golden_small():
    z = np.load(GOLDEN)
    for (M, N, K) in ((7, 33, 65), (20, 40, 300)):
        a = torch.from_numpy(z[f"a_f32_{M}_{N}_{K}"]).to(DEV)
        w = torch.from_numpy(z[f"w_f32_{M}_{N}_{K}"]).to(DEV)
        ref = torch.from_numpy(z[f"c_f64_{M}_{N}_{K}"])
        torch.testing.assert_close(matmul(a, w.t()).cpu().double(), ref, rtol=1e-4, atol=1e-4 * math.sqrt(K))
        ab = torch.from_numpy(z[f"a_bf16_{M}_{N}_{K}"].astype(np.int16)).view(torch.bfloat16).to(DEV)
        wb = torch.from_numpy(z[f"w_bf16_{M}_{N}_{K}"].astype(np.int16)).view(torch.bfloat16).to(DEV)
        refb = torch.from_numpy(z[f"cb_f64_{M}_{N}_{K}"])
        torch.testing.assert_close(matmul(ab, wb.t()).cpu().double(), refb, rtol=1.6e-2, atol=1e-2 * math.sqrt(K))


@pytest.mark.parametrize("M", [1, 5, 16, 17, 32, 33, 64, 100, 256, 2048])
@pytest.mark.parametrize("I,K", [(3072, 1024), (40, 64), (300, 136), (1024, 2048), (512, 3072)])
def test_matmul_silu_mul_is_bitwise_the_two_step_result(M, I, K):
    """The fused gate_up + SiLU x Mul equals silu_and_mul(matmul(x, w.t())) bit for bit (same per-column k order,
    same rounding points; K >= 2048 covers the skinny kernels' row tiles up to 256 rows, which both calls pick from
    M, K and the W rows alike); the two-step result itself is checked against the oracle elsewhere."""
    from nanovllm_hip.kernels import matmul_silu_and_mul, silu_and_mul
    g = torch.Generator("cpu").manual_seed(M * 7 + I)
    x = (torch.randn(M, K, generator=g) / math.sqrt(K)).to(torch.bfloat16).to(DEV)
    w = torch.randn(2 * I, K, generator=g).to(torch.bfloat16).to(DEV)
    fused = matmul_silu_and_mul(x, w)
    two_step = silu_and_mul(matmul(x, w.t()))
    assert fused.shape == (M, I)
    assert torch.equal(fused, two_step)
    # and against the oracle composition (float64 product rounded to bf16, then the reference's silu * up)
    ref = oracle.silu_and_mul(oracle.matmul_fp64(x.cpu(), w.cpu().t()).to(torch.bfloat16))
    torch.testing.assert_close(fused.cpu().float(), ref.float(), rtol=1.6e-2, atol=2e-2)
