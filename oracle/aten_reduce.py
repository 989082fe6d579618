"""The summation order of torch's GPU `mean` over the last dim (TEST INFRASTRUCTURE ONLY: see __init__).

The reference's RMSNorm (nanovllm/layers/layernorm.py:26 and :40) computes `x.pow(2).mean(dim=-1, keepdim=True)`
on fp32 rows. Run eagerly on an MI355X that is ATen's generic GPU reduction (torch's open-source
ATen/native/hip/Reduce.cuh, ROCm build, 64-lane wavefronts) with MeanOps (ReduceMomentKernel: a plain fp32 sum,
then `sum * factor`, factor = float(num_outputs) / numel in fp32). Its order of fp32 additions depends on the row
width n and on the number of rows (the launch configuration does), so an fp32 sum in any other order differs in
the last bits and the normalised bf16 values differ now and then.

This module restates that order with numpy float32 arithmetic (every add rounded to nearest even, as on the GPU)
for the configurations where one thread-block row reduces one output (no split of a row over waves or blocks):

  setReduceConfig:  vectorised loads of 4 fp32 when n >= 128 (dim0 = n // 4 vectors), else one element per step;
                    d0 = last_pow2(dim0) capped at 512, d1 = last_pow2(rows) capped at 512;
                    bw = min(d0, 64); bh = min(d1, 512 // bw); bw = min(d0, 512 // bh)   (block = bw x bh threads)
  thread reduce:    thread L of a row takes vectors L, L + bw, L + 2 bw, ...; four accumulators (one per vector
                    component, or per unrolled step), each summed sequentially from 0; then ((a0 + a1) + a2) + a3
  block_x_reduce:   bw > 64: t[L] += t[L + off] for off = bw/2 .. 64 (shared memory); then within the wave
                    t[L] += t[L + off] for off = 1, 2, 4, .. (shuffle down, increasing offsets on ROCm) -- lane 0
                    ends with the pairwise sum of adjacent lanes
  mean:             t[0] * factor

Every function takes float32 numpy arrays and returns float32 results. Pinned in tests/test_oracle.py (brute force
and closed forms on the CPU) and, on the GPU, bitwise against torch's own `mean` (tests/test_norm_act.py).
"""
import numpy as np

WARP = 64
MAX_THREADS = 512  # mnt_wrapper<float>::MAX_NUM_THREADS


def _last_pow2(x: int) -> int:
    return 1 << (int(x).bit_length() - 1)


def reduce_config(n: int, rows: int):
    """(vectorised, bw): how ATen's GPU reduction splits `rows` rows of n contiguous fp32 values. Raises
    NotImplementedError for the configurations that split a row over the waves of a block (very wide rows)."""
    if n <= 0 or rows <= 0:
        raise ValueError("n and rows must be positive")
    vec = n >= 128
    if vec and n % 4:
        raise NotImplementedError("rows of n >= 128 that are not a multiple of 4 (misaligned vector loads)")
    dim0 = n // 4 if vec else n
    d0 = _last_pow2(dim0) if dim0 < MAX_THREADS else MAX_THREADS
    d1 = _last_pow2(rows) if rows < MAX_THREADS else MAX_THREADS
    bw = min(d0, WARP)
    bh = min(d1, MAX_THREADS // bw)
    bw = min(d0, MAX_THREADS // bh)
    values_per_thread = -(-n // bw)
    if bh > 1 and values_per_thread >= min(bh * 16, 256):
        raise NotImplementedError("a row split over the waves of a block")
    return vec, bw


def thread_partials(y: np.ndarray, bw: int, vec: bool) -> np.ndarray:
    """t[r, L]: what thread L of row r holds after its own loop and the combination of its four accumulators."""
    y = np.asarray(y, dtype=np.float32)
    rows, n = y.shape
    acc = np.zeros((rows, bw, 4), np.float32)
    if vec:
        V = n // 4
        yv = y.reshape(rows, V, 4)
        for lo in range(0, V, bw):
            hi = min(V, lo + bw)
            acc[:, :hi - lo, :] += yv[:, lo:hi, :]
    else:
        # thread_reduce_impl with vt0 = 4: steps of 4 * bw while idx + 3 bw < n, then a tail of up to 4 loads
        for L in range(bw):
            idx = L
            while idx + 3 * bw < n:
                for i in range(4):
                    acc[:, L, i] += y[:, idx + i * bw]
                idx += 4 * bw
            for i in range(4):
                if idx >= n:
                    break
                acc[:, L, i] += y[:, idx]
                idx += bw
    return ((acc[:, :, 0] + acc[:, :, 1]) + acc[:, :, 2]) + acc[:, :, 3]


def block_tree(t: np.ndarray) -> np.ndarray:
    """The block's combination of the thread partials t [rows, bw] -> [rows]: shared-memory halving down to one
    wave, then the in-wave tree of adjacent pairs that lane 0 ends with."""
    t = np.asarray(t, dtype=np.float32)
    bw = t.shape[1]
    off = bw // 2
    while off >= WARP:
        t = t[:, :off] + t[:, off:2 * off]
        off //= 2
    while t.shape[1] > 1:
        t = t[:, 0::2] + t[:, 1::2]
    return t[:, 0]


def row_sum(y: np.ndarray, rows_in_call: int | None = None) -> np.ndarray:
    """ATen's fp32 sum of each row of y [rows, n] in its GPU order. rows_in_call: the number of rows of the whole
    reduction when y is a slice of it (the order depends on it); defaults to y's rows."""
    y = np.asarray(y, dtype=np.float32)
    vec, bw = reduce_config(y.shape[1], rows_in_call or y.shape[0])
    return block_tree(thread_partials(y, bw, vec))


def mean_factor(n: int, rows: int) -> np.float32:
    """MeanOps' factor: float(num_outputs) / numel, the int64 numel converted to float first."""
    return np.float32(rows) / np.float32(rows * n)


def mean_sq(x: np.ndarray, rows_in_call: int | None = None) -> np.ndarray:
    """`x.pow(2).mean(dim=-1)` of fp32 rows x [rows, n] as torch computes it on the GPU: fp32 squares, ATen's sum
    order, times the fp32 factor."""
    x = np.asarray(x, dtype=np.float32)
    rows = rows_in_call or x.shape[0]
    return row_sum(x * x, rows) * mean_factor(x.shape[1], rows)
