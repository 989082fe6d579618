"""Benchmark of the HIP kernel path on one MI355X: prints ONE JSON line.

Headline (`value`): the fused q/k RMSNorm + RoPE + paged-KV write at T = 8192 tokens, Qwen3-0.6B attention shape
(16 q heads, 8 kv heads, head_dim 128), in GB/s of algorithmic bytes:
  qkv a strided view of a [T, 4096 + 64] bf16 buffer; positions contiguous over 4 sequences of T/4 tokens; a
  512-block x 256-slot paged cache; every slot valid (the reference's microbenchmark layout); write_k False.
  bytes/launch = T * (4096 q read + 4096 q_out write + 8 position + 4 slot + 512 cos/sin)
                 + n_valid * (2048 k read + 2048 v read + 2048 k cache write + 2048 v cache write) + 512 weights
               = 16 908 * T + 512 with every slot valid (the reference's formula, scripts/bench_qk_rope_kv.py:50-52).
One step = one launch over the T tokens. NSETS = 8 input/output sets (each with its own block table) rotate from
launch to launch, 544 MB of qkv in all (twice the 256 MiB Infinity Cache), so the reads come from HBM; after
warm-up launches (--warmup of them and at least 50 ms) and a synchronize, 64 untimed launches are queued (one
replay of a HIP graph of them) and then exactly --steps launches are timed with HIP events on the stream they run
on (the host submits them while the GPU still runs the queued ones, so the timed region holds the launches back to
back and no submission gap).

Also reported (under "extra"): the ceilings of the headline on this part -- its own launch shape and memory pattern
with the arithmetic removed (libnvhip_bench.so's nvhip_bench_qk_pattern) and a plain nontemporal copy of the same
byte count; the same kernel at T = 1, 32, 2048, and at T = 2048 with write_k (the prefill setting of the
reference's README table; at T = 2048 enough sets rotate -- 32 -- that the reads come from HBM, as for the headline); the unfused KV write (store_kvcache, bytes =
T * (2 * 2048 read + 2 * 2048 written + 4 slot)) at T = 8192; RMSNorm, Add+RMSNorm and SiLU x Mul at T = 8192
(hidden 1024, gate_up 2 x 3072) in GB/s; the bf16 GEMM at the Qwen3-0.6B projection shapes, M = 2048 in TFLOP/s
and M = 32 in GB/s (weights rotated through >= 512 MiB of copies so they come from HBM); the fp32 4096^3 GEMM;
the paged decode attention of one layer for 32 sequences with contexts of 512..2048 tokens, in GB/s; the causal
prefill attention of one layer over 4 sequences of 2048 tokens and of a 256-token chunk over 3840 cached keys, in
TFLOP/s; the end-to-end decode step of a
random-init Qwen3-0.6B-shaped model (batch 32, HIP graph: us per step, tokens/s, kernel nodes); a 256-token mixed
step of the same model (16 decode requests + a 240-token prefill chunk), eager and from piecewise graphs.
The CPU baseline is the oracle (the reference's torch code restated, fp32 math, on the host cores this process may
use, the count stated) on a bounded sample of the same workload, with CPU lines for RMSNorm, Add+RMSNorm, SiLU x Mul
and the fp32 GEMM (torch.matmul) beside it.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--tokens 8192] [--no-cpu] [--no-extra] [--no-e2e]
       (profiling modes: --profile, --profile-gemm, --profile-e2e, --profile-prefill, --profile-chunk,
       --profile-mixed)
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "nano-vllm-triton-kernels_amd"))
sys.path.insert(0, ROOT)

METRIC = "qk-norm+RoPE+KV-write GB/s (%HBM peak) at T=8192; bf16 GEMM TFLOP/s"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3
HQ, HKV, D, MAX_POS, THETA, BLOCK, EPS = 16, 8, 128, 40960, 1e6, 256, 1e-6
NUM_BLOCKS = 512
PAD = 64
NSETS = 8  # rotating input sets: 8 x 68 MB of qkv for the headline, twice the 256 MiB Infinity Cache
MALL_BYTES = 256 * 2 ** 20  # the Infinity Cache (memory-attached last-level cache) of the part
WARM_S = 0.05  # minimum warm-up wall time of every measurement (clock ramp)
GEMM_SHAPES = {"qkv": (1024, 4096), "gate_up": (1024, 6144), "down": (3072, 1024), "o_proj": (2048, 1024)}  # (K, N)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "qk_norm_rope_kv_t8192_traffic.json")


def fused_bytes(T, n_valid, write_k=False):
    return T * (HQ * D * 2 * 2 + 8 + 4 + D * 4) + n_valid * (4 * HKV * D * 2) + (HKV * D * 2 if write_k else 0) * T \
        + 2 * D * 2


def block_table_slots(T, g, torch):
    """Slots of 4 sequences of T/4 tokens in random distinct blocks, and their contiguous positions."""
    nseq = min(4, T)
    lens = [T // nseq + (1 if i < T % nseq else 0) for i in range(nseq)]
    perm = torch.randperm(NUM_BLOCKS, generator=g)
    slots, positions, used = [], [], 0
    for n in lens:
        nb = (n + BLOCK - 1) // BLOCK
        blocks = perm[used:used + nb]
        used += nb
        off = torch.arange(n)
        slots.append(blocks[off // BLOCK] * BLOCK + off % BLOCK)
        start = int(torch.randint(0, 4096, (1,), generator=g))
        positions.append(start + off)
    return torch.cat(slots).to(torch.int32), torch.cat(positions).to(torch.int64)


class FusedWorkload:
    def __init__(self, T, dev, torch, oracle, seed=0, nsets=None):
        g = torch.Generator("cpu").manual_seed(seed)
        self.T = T
        self.nsets = NSETS if nsets is None else nsets
        self.sets = []
        for _ in range(self.nsets):
            buf = torch.randn(T, (HQ + 2 * HKV) * D + PAD, generator=g).to(torch.bfloat16).to(dev)
            q = buf[:, :HQ * D].view(T, HQ, D)
            k = buf[:, HQ * D:(HQ + HKV) * D].view(T, HKV, D)
            v = buf[:, (HQ + HKV) * D:(HQ + 2 * HKV) * D].view(T, HKV, D)
            slots, positions = block_table_slots(T, g, torch)
            self.sets.append(dict(buf=buf, q=q, k=k, v=v, slots=slots.to(dev), positions=positions.to(dev)))
        self.q_w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(dev)
        self.k_w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(dev)
        self.cos_sin = oracle.rope_cos_sin_cache(D, MAX_POS, THETA).to(dev)
        self.k_cache = torch.zeros(NUM_BLOCKS, BLOCK, HKV, D, dtype=torch.bfloat16, device=dev)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.n_valid = T

    def call(self, i, qk_norm_rope_kv, write_k=False):
        s = self.sets[i % self.nsets]
        return qk_norm_rope_kv(s["q"], s["k"], s["v"], s["positions"], self.q_w, self.k_w, EPS, self.cos_sin,
                               self.k_cache, self.v_cache, s["slots"], write_k)

    def pattern(self, i, bench_lib, torch):
        """The same launch through nvhip_bench_qk_pattern: the kernel's loads and stores without its arithmetic."""
        s = self.sets[i % self.nsets]
        if "q_out" not in s:
            s["q_out"] = torch.empty(self.T, HQ, D, dtype=torch.bfloat16, device=s["buf"].device)
        rc = bench_lib.nvhip_bench_qk_pattern(
            s["q_out"].data_ptr(), s["q"].data_ptr(), s["k"].data_ptr(), s["v"].data_ptr(), s["q"].stride(0),
            s["k"].stride(0), s["v"].stride(0), s["positions"].data_ptr(), s["slots"].data_ptr(),
            self.cos_sin.data_ptr(), MAX_POS, self.k_cache.data_ptr(), self.v_cache.data_ptr(), NUM_BLOCKS * BLOCK,
            self.T, HQ, HKV, torch.cuda.current_stream().cuda_stream)
        assert rc == 0, rc


def bench_lib():
    """libnvhip_bench.so (measurement-only kernels, built with the library), loaded after torch."""
    import ctypes
    path = os.path.join(ROOT, "nano-vllm-triton-kernels_amd", "nanovllm_hip", "libnvhip_bench.so")
    lib = ctypes.CDLL(path)
    p, i64, i = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.nvhip_bench_stream_copy.argtypes = [p, p, i64, i, p]
    lib.nvhip_bench_stream_rw.argtypes = [p, p, i64, i, i, p]
    lib.nvhip_bench_qk_pattern.argtypes = [p, p, p, p, i64, i64, i64, p, p, p, i64, p, p, i64, i64, i64, i64, p]
    lib.nvhip_bench_mfma_lds.argtypes = [i, i, i, i, p, p, p]
    return lib


def stream_copy(torch, lib, dst, src, nbytes):
    """Plain nontemporal 16-byte copy of nbytes, 8 blocks of 256 threads per CU (grid-stride)."""
    rc = lib.nvhip_bench_stream_copy(dst.data_ptr(), src.data_ptr(), nbytes, 2048,
                                     torch.cuda.current_stream().cuda_stream)
    assert rc == 0, rc


def copy_ceiling_us(torch, dev, write_bytes, reads_per_write, steps, windows=1):
    """Microseconds per call of a plain nontemporal stream over NSETS rotating buffer pairs that reads
    reads_per_write x write_bytes and writes write_bytes (nvhip_bench_stream_rw, 8 blocks of 256 threads per CU, or
    one 16-byte vector per thread for small streams): the ceiling of an HBM-bound kernel with those byte counts, its
    launch ramp and drain included (the median of `windows` timed windows)."""
    lib = bench_lib()
    write_bytes = -(-write_bytes // 16) * 16
    blocks = max(1, min(2048, -(-write_bytes // (16 * 256))))
    bufs = [(torch.empty(write_bytes, dtype=torch.uint8, device=dev),
             torch.empty(write_bytes * reads_per_write, dtype=torch.uint8, device=dev)) for _ in range(NSETS)]

    def fn(i):
        dst, src = bufs[i % NSETS]
        rc = lib.nvhip_bench_stream_rw(dst.data_ptr(), src.data_ptr(), write_bytes, reads_per_write, blocks,
                                       torch.cuda.current_stream().cuda_stream)
        assert rc == 0, rc
    ms = sorted(time_graph(torch, fn, NSETS, max(40, steps), 20, WARM_S)[0] for _ in range(windows))[windows // 2]
    del bufs
    return ms * 1e3


HBM_SWEEP_POLICIES = {0: "plain", 1: "nontemporal", 2: "plain loads, written-through stores",
                      3: "nontemporal loads, written-through stores"}


def hbm_ceiling(torch, dev, table=False, moved=2 ** 30):
    """This part's HBM ceiling: the best of a sweep of read-only, write-only and 1:1 copy streams
    (libnvhip_bench.so's nvhip_bench_hbm_sweep) that move `moved` bytes per launch (default 1 GiB; copy: half read,
    half written) over rotating buffers of >= 1 GiB in all, four times the 256 MiB Infinity Cache: 1, 2, 4 or 8
    16-byte vectors in flight per lane; plain, nontemporal or written-through cache policies; grid-stride grids of 1,
    2, 4, 8 or 16 256-thread blocks per CU or a one-shot grid. Each point is the best of 3 windows of 8 eager
    launches (4 for 1 GiB) after a 20 ms warm-up of that point. Returns the best point per mode (and every point
    when table)."""
    lib = bench_lib()
    import ctypes
    lib.nvhip_bench_hbm_sweep.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    moved = moved // 65536 * 65536  # whole 256-thread x 8-vector iterations of both halves
    nrot = max(1, -(-(2 ** 30) // moved))
    bufs = [(torch.full((moved,), 1, dtype=torch.uint8, device=dev), torch.full((moved,), 2, dtype=torch.uint8,
                                                                               device=dev)) for _ in range(nrot)]
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    stream = torch.cuda.current_stream()
    launches = 4 if nrot == 1 else 8
    points = []
    for mode, name in ((0, "read"), (1, "write"), (2, "copy")):
        nbytes = moved if mode < 2 else moved // 2
        pols = (0, 1) if mode == 0 else (0, 1, 2) if mode == 1 else (0, 1, 2, 3)
        for unroll in (1, 2, 4, 8):
            for pol in pols:
                for bpc in (1, 2, 4, 8, 16, 0):
                    blocks = bpc * cus
                    if mode == 0 and blocks * 256 * 16 > nbytes:
                        continue

                    def fn(i):
                        a, b = bufs[i % nrot]
                        return lib.nvhip_bench_hbm_sweep(b.data_ptr(), None if mode == 1 else a.data_ptr(), nbytes,
                                                         mode, unroll, pol, blocks, stream.cuda_stream)
                    t0, i = time.perf_counter(), 0
                    while time.perf_counter() - t0 < 0.02:
                        assert fn(i) == 0
                        i += 1
                        if i % 64 == 0:
                            torch.cuda.synchronize()
                    torch.cuda.synchronize()
                    best = None
                    for _ in range(3):
                        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                        for j in range(nrot):  # queued ahead of the start event
                            assert fn(j) == 0
                        e0.record(stream)
                        for j in range(launches):
                            assert fn(j) == 0
                        e1.record(stream)
                        e1.synchronize()
                        us = e0.elapsed_time(e1) * 1e3 / launches
                        best = us if best is None else min(best, us)
                    total = nbytes * (2 if mode == 2 else 1)
                    points.append({"mode": name, "unroll": unroll, "policy": HBM_SWEEP_POLICIES[pol],
                                   "blocks_per_cu": bpc or "one-shot", "us": round(best, 2),
                                   "GB/s": round(total / (best * 1e-6) / 1e9, 1)})
    del bufs
    torch.cuda.empty_cache()
    out = {"bytes_per_launch": moved, "rotating_buffers": nrot, "points": len(points)}
    for name in ("read", "write", "copy"):
        top = max((p for p in points if p["mode"] == name), key=lambda p: p["GB/s"])
        out[name] = {k: v for k, v in top.items() if k != "mode"}
        out[name]["frac_hbm"] = round(top["GB/s"] / HBM_PEAK_GBS, 4)
    if table:
        out["table"] = points
    return out


def mfma_ceiling(torch, dev, iters=20000):
    """The bf16 MFMA ceiling of this part (libnvhip_bench.so's nvhip_bench_mfma_lds): one block per CU whose waves
    issue v_mfma_f32_32x32x16_bf16 back to back, with 0, 2, 4, 6 or 8 KB of LDS fragment reads per 8 MFMAs (a GEMM
    wave tile of 64 x 64 reads 1 KB per MFMA, 64 x 128 0.75 KB, 128 x 128 0.5 KB), at 1, 2 or 4 waves per SIMD.
    Per point, the best of 3 timed launches after 2 untimed ones: TFLOP/s over the launch (HIP events), the shader
    clock (per-wave s_memtime cycles over s_memrealtime ticks) and the MFMA pipe's busy fraction per clock (a
    32x32x16 MFMA holds a SIMD's pipe for 32 cycles)."""
    lib = bench_lib()
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    stream = torch.cuda.current_stream()
    rows = []
    for waves in (4, 8, 16):
        clocks = torch.zeros(2 * cus * waves, dtype=torch.int64, device=dev)
        sink = torch.empty(cus * waves * 64, dtype=torch.float32, device=dev)
        for reads in (0, 2, 4, 6, 8):
            def launch():
                rc = lib.nvhip_bench_mfma_lds(reads, waves, iters, cus, clocks.data_ptr(), sink.data_ptr(),
                                              stream.cuda_stream)
                assert rc == 0, rc
            for _ in range(2):
                launch()
            best = None
            for _ in range(3):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                launch()
                e1.record(stream)
                e1.synchronize()
                ms = e0.elapsed_time(e1)
                c = clocks.view(-1, 2).double().mean(0).tolist()
                pt = (ms, c[0], c[1])
                best = pt if best is None or ms < best[0] else best
            ms, cyc, ticks = best
            flops = cus * waves * iters * 8 * 32 * 32 * 16 * 2
            rows.append({"waves_per_simd": waves // 4, "lds_kb_per_mfma": reads / 8, "ms": round(ms, 4),
                         "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
                         "frac_2p5": round(flops / (ms * 1e-3) / 2.5e15, 4),
                         "clock_ghz": round(cyc / (ticks * 10.0), 3),
                         "mfma_pipe_busy": round(iters * 8 * (waves // 4) * 32 / cyc, 4)})
    return {"iters": iters, "blocks": cus, "points": rows}


def time_graph(torch, fn, n_calls, steps, warmup, min_warm_s=0.0):
    """Records n_calls calls of fn(i) into one HIP graph, replays it (warmup + steps calls, rounded up to whole
    replays) and returns the average milliseconds per call, timed with events on the replay stream.

    min_warm_s: keep warming up until that much wall time has passed. The GPU raises its clocks over several
    milliseconds of load, and a measurement that starts right after host-side set-up (where the GPU idled) reads
    10-20 % slow for a compute-bound kernel; the extras use 50 ms so that every kernel and its torch comparison
    start from the same state."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(n_calls):
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(n_calls):
            fn(i)
    reps_warm = max(1, -(-warmup // n_calls))
    reps = max(1, -(-steps // n_calls))
    t0 = time.perf_counter()
    for _ in range(reps_warm):
        graph.replay()
    torch.cuda.synchronize()
    batch = reps_warm
    while time.perf_counter() - t0 < min_warm_s:
        for _ in range(batch):
            graph.replay()
        torch.cuda.synchronize()
        batch *= 2
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    # one untimed lead-in replay, then the start event in stream order behind it: the host submits the timed
    # replay while the GPU still runs the lead-in, so the timed region holds the calls and no idle submission gap
    graph.replay()
    start.record(stream)
    for _ in range(reps):
        graph.replay()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / (reps * n_calls), reps * n_calls


def paired_ms(torch, fn, fn_ref, n_calls, steps, warmup):
    """Compute-bound GEMM launches beside the vendor library's: the two timed alternately, twice each (ours,
    theirs, ours, theirs, each with its own warm-up), and the faster window of each kept: the chip's clock under
    such load drifts between windows (two windows of the same launch measured up to 9 % apart in one process, for
    ours and for hipBLASLt's alike)."""
    runs = [time_graph(torch, f, n_calls, steps, warmup, WARM_S)[0] for _ in range(2) for f in (fn, fn_ref)]
    return min(runs[0], runs[2]), min(runs[1], runs[3])


def time_steps(torch, fn, steps, warmup, min_warm_s, lead=64):
    """Exactly `steps` eager calls fn(0) .. fn(steps - 1), timed with HIP events on the current stream: warm-up calls
    first (at least `warmup` of them and min_warm_s of wall time: the clock ramp), a synchronize, then one replay of
    a HIP graph of `lead` calls queued ahead of the start event (one host call: ~1.5 ms of GPU work however slow the
    host's per-call submission is, e.g. under a profiler), so the GPU runs the timed calls back to back while the host
    submits them. Returns (milliseconds per call, host submission microseconds per timed call). The timed calls are
    eager launches: a 20-node graph replay of the same calls measured 0.3-0.8 us slower per call than 40- or 200-node
    replays and than eager calls, whose time matches the kernel trace's mean duration."""
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    # the lead-in graph is recorded first, so that nothing leaves the GPU idle between the warm-up calls, the lead-in
    # replay and the timed calls (recording it after the warm-up left the GPU idle for the few milliseconds the
    # recording takes, and the timed calls then started on a cooling clock)
    fn(0)  # one eager call before the recording (lazy set-up happens outside it)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            for j in range(lead):
                fn(j)
    torch.cuda.synchronize()
    i, t0 = 0, time.perf_counter()
    while i < warmup or time.perf_counter() - t0 < min_warm_s:
        fn(i)
        i += 1
        if i % 256 == 0:
            torch.cuda.synchronize()
    graph.replay()
    start.record(stream)
    h0 = time.perf_counter()
    for j in range(steps):
        fn(j)
    host_us = (time.perf_counter() - h0) * 1e6 / steps
    end.record(stream)
    end.synchronize()
    del graph
    return start.elapsed_time(end) / steps, host_us


def host_cores():
    """(threads to use, description): the CPUs this process may run on (its affinity set), capped by the cgroup CPU
    quota when there is one, with os.cpu_count() stated beside them."""
    n = os.cpu_count() or 1
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else n
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()
            if q != "max":
                quota = max(1, int(int(q) // int(period)))
    except (OSError, ValueError):
        pass
    threads = min(usable, quota) if quota else usable
    return threads, f"os.cpu_count()={n}, affinity {usable} CPUs, cgroup quota {quota or 'none'}"


def cpu_median(fn, budget_s, min_calls=3):
    fn()  # warm up
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < min_calls:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_extra(torch, oracle, budget_s=3.0):
    """The oracle's RMSNorm, Add+RMSNorm, SiLU x Mul at T = 8192 (hidden 1024, gate_up 2 x 3072) and the fp32 GEMM
    (torch.matmul on the CPU) at the qkv shape at M = 2048 and at 4096^3, each the median of a ~3 s sample."""
    g = torch.Generator("cpu").manual_seed(4)
    T, H, I = 8192, 1024, 3072
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    r = torch.randn(T, H, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16)
    gu = torch.randn(T, 2 * I, generator=g).to(torch.bfloat16)
    out = {}
    for name, fn, nbytes in (("rms_norm_T8192", lambda: oracle.rms_forward(x, w, EPS), (2 * T * H + H) * 2),
                             ("fused_add_rms_norm_T8192", lambda: oracle.add_rms_forward(x, r, w, EPS),
                              (4 * T * H + H) * 2),
                             ("silu_and_mul_T8192", lambda: oracle.silu_and_mul(gu), 3 * T * I * 2)):
        med, n = cpu_median(fn, budget_s)
        out[name] = {"GB/s": round(nbytes / med / 1e9, 2), "ms": round(med * 1e3, 2), "calls": n}
    for name, (M, N, K) in (("gemm_fp32_qkv_M2048", (2048, 4096, 1024)), ("gemm_fp32_4096", (4096, 4096, 4096))):
        a = torch.randn(M, K, generator=g)
        b = torch.randn(K, N, generator=g)
        med, n = cpu_median(lambda: torch.matmul(a, b), budget_s, min_calls=2)
        out[name] = {"TFLOP/s": round(2 * M * N * K / med / 1e12, 3), "ms": round(med * 1e3, 1), "calls": n}
    return out


def cpu_baseline(torch, oracle, T, budget_s=12.0):
    """The oracle (torch CPU, fp32 math) on the same fused workload, timed on the host cores."""
    threads, cores_desc = host_cores()
    torch.set_num_threads(threads)
    g = torch.Generator("cpu").manual_seed(1)
    buf = torch.randn(T, (HQ + 2 * HKV) * D + PAD, generator=g).to(torch.bfloat16)
    q = buf[:, :HQ * D].view(T, HQ, D)
    k = buf[:, HQ * D:(HQ + HKV) * D].view(T, HKV, D)
    v = buf[:, (HQ + HKV) * D:(HQ + 2 * HKV) * D].view(T, HKV, D)
    slots, positions = block_table_slots(T, g, torch)
    qw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16)
    cos_sin = oracle.rope_cos_sin_cache(D, MAX_POS, THETA)
    kc = torch.zeros(NUM_BLOCKS, BLOCK, HKV, D, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    run = lambda: oracle.qk_norm_rope_kv(q, k, v, positions, qw, kw, EPS, cos_sin, kc, vc, slots, False)
    med, calls = cpu_median(run, budget_s, min_calls=5)
    return {"value": round(fused_bytes(T, T) / med / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": f"oracle qk_norm_rope_kv (torch CPU fp32) at T={T}, {calls} calls in ~{budget_s:.0f} s, "
                      f"median {med * 1e3:.1f} ms/call, {torch.get_num_threads()} threads ({cores_desc})",
            "extra": cpu_extra(torch, oracle)}


def ceilings(torch, kernels, wl, steps, head_gbs):
    """Bandwidth ceilings for the headline, measured on this part: the headline's own launch shape and memory
    pattern with the arithmetic removed (nvhip_bench_qk_pattern), and a plain nontemporal copy moving the same
    number of bytes (half read, half written), both over rotating buffers like the headline."""
    lib = bench_lib()
    nbytes = fused_bytes(wl.T, wl.n_valid)
    ms, _ = time_steps(torch, lambda i: wl.pattern(i, lib, torch), max(40, steps), 20, WARM_S)
    pat = nbytes / (ms * 1e-3) / 1e9
    half = nbytes // 2 // 16 * 16
    bufs = [(torch.empty(half, dtype=torch.uint8, device=wl.cos_sin.device),
             torch.empty(half, dtype=torch.uint8, device=wl.cos_sin.device)) for _ in range(NSETS)]
    ms_c, _ = time_steps(torch, lambda i: stream_copy(torch, lib, bufs[i % NSETS][0], bufs[i % NSETS][1], half),
                      max(40, steps), 20, WARM_S)
    cp = 2 * half / (ms_c * 1e-3) / 1e9
    del bufs
    return {"qk_pattern_copy_T8192": {"us": round(ms * 1e3, 3), "GB/s": round(pat, 1),
                                      "frac_hbm": round(pat / HBM_PEAK_GBS, 4),
                                      "headline_frac_of_it": round(head_gbs / pat, 4)},
            "stream_copy_same_bytes": {"us": round(ms_c * 1e3, 3), "GB/s": round(cp, 1),
                                       "frac_hbm": round(cp / HBM_PEAK_GBS, 4), "bytes": 2 * half}}


def extras(torch, oracle, kernels, dev, steps):
    out = {}
    for T in (1, 32, 2048):
        # T = 2048: enough input sets (>= 2x the 256 MiB Infinity Cache, as for the headline) that every call reads
        # from HBM; T = 1 / 32 are launch-latency bound and keep NSETS
        nsets = NSETS if T <= 32 else max(NSETS, -(-(2 * MALL_BYTES) // (T * (HQ + 2 * HKV) * D * 2)))
        wl = FusedWorkload(T, dev, torch, oracle, seed=T, nsets=nsets)
        # launch-latency bound launches vary from window to window (3.3 vs 5.2 us at T = 32 back to back): the
        # median of 5 windows
        windows = 5 if T <= 32 else 1
        ms = sorted(time_graph(torch, lambda i: wl.call(i, kernels.qk_norm_rope_kv), nsets, max(40, steps), 20,
                               WARM_S)[0] for _ in range(windows))[windows // 2]
        out[f"qk_norm_rope_kv_T{T}"] = {"us": round(ms * 1e3, 3),
                                        "GB/s": round(fused_bytes(T, T) / (ms * 1e-3) / 1e9, 1), "sets": nsets}
        if T == 2048:  # the kernel's memory pattern with the arithmetic removed, over the same rotating sets
            lib = bench_lib()
            ms_p, _ = time_graph(torch, lambda i: wl.pattern(i, lib, torch), nsets, max(40, steps), 20, WARM_S)
            out["qk_pattern_copy_T2048"] = {"us": round(ms_p * 1e3, 3),
                                            "GB/s": round(fused_bytes(T, T) / (ms_p * 1e-3) / 1e9, 1),
                                            "fused_frac_of_it": round(ms_p / ms, 4)}
        if T == 2048:  # prefill setting of the reference's README table: k_out written too
            ms, _ = time_graph(torch, lambda i: wl.call(i, kernels.qk_norm_rope_kv, True), nsets, max(40, steps),
                               20, WARM_S)
            nb = fused_bytes(T, T, write_k=True)
            out["qk_norm_rope_kv_T2048_write_k"] = {"us": round(ms * 1e3, 3), "bytes": nb,
                                                    "GB/s": round(nb / (ms * 1e-3) / 1e9, 1)}
    wl = FusedWorkload(8192, dev, torch, oracle, seed=5)
    ms, _ = time_graph(torch, lambda i: kernels.store_kvcache(wl.sets[i % NSETS]["k"], wl.sets[i % NSETS]["v"],
                                                              wl.k_cache, wl.v_cache, wl.sets[i % NSETS]["slots"]),
                       NSETS, max(40, steps), 20, WARM_S)
    nbytes = 8192 * (4 * HKV * D * 2 + 4)
    gbs = nbytes / (ms * 1e-3) / 1e9
    cp = copy_ceiling_us(torch, dev, 8192 * 2 * HKV * D * 2, 1, steps)
    out["store_kvcache_T8192"] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                                  "copy_us": round(cp, 3), "frac_of_copy": round(cp / (ms * 1e3), 4)}
    del wl
    T, H, I = 8192, 1024, 3072
    g = torch.Generator("cpu").manual_seed(2)
    xs = [torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev) for _ in range(NSETS)]
    rs = [torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev) for _ in range(NSETS)]
    gus = [torch.randn(T, 2 * I, generator=g).to(torch.bfloat16).to(dev) for _ in range(NSETS)]
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)
    # (name, call, algorithmic bytes, bytes written, reads per byte written) -- the last two size the copy ceiling
    for name, fn, nbytes, wbytes, rpw in (
            ("rms_norm_T8192", lambda i: kernels.rms_norm(xs[i], w, EPS), (2 * T * H + H) * 2, T * H * 2, 1),
            ("fused_add_rms_norm_T8192", lambda i: kernels.fused_add_rms_norm(xs[i], rs[i], w, EPS),
             (4 * T * H + H) * 2, 2 * T * H * 2, 1),
            ("silu_and_mul_T8192", lambda i: kernels.silu_and_mul(gus[i]), 3 * T * I * 2, T * I * 2, 2)):
        ms, _ = time_graph(torch, fn, NSETS, max(40, steps), 20, WARM_S)
        gbs = nbytes / (ms * 1e-3) / 1e9
        cp = copy_ceiling_us(torch, dev, wbytes, rpw, steps, windows=3)  # the median: one window read 16.9 vs 6 us
        out[name] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                     "copy_us": round(cp, 3), "frac_of_copy": round(cp / (ms * 1e3), 4)}
    del xs, rs, gus
    # decode batches (T = 1, 32): launch-latency bound; the median of 5 timed windows, each beside the same-bytes copy
    for T in (1, 32):
        xs = [torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev) for _ in range(NSETS)]
        rs = [torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev) for _ in range(NSETS)]
        gus = [torch.randn(T, 2 * I, generator=g).to(torch.bfloat16).to(dev) for _ in range(NSETS)]
        for name, fn, nbytes, wbytes, rpw in (
                ("rms_norm", lambda i: kernels.rms_norm(xs[i], w, EPS), (2 * T * H + H) * 2, T * H * 2, 1),
                ("fused_add_rms_norm", lambda i: kernels.fused_add_rms_norm(xs[i], rs[i], w, EPS),
                 (4 * T * H + H) * 2, 2 * T * H * 2, 1),
                ("silu_and_mul", lambda i: kernels.silu_and_mul(gus[i]), 3 * T * I * 2, T * I * 2, 2)):
            ms = sorted(time_graph(torch, fn, NSETS, max(40, steps), 20, WARM_S)[0] for _ in range(5))[2]
            cp = copy_ceiling_us(torch, dev, wbytes, rpw, steps, windows=5)
            out[f"{name}_T{T}"] = {"us": round(ms * 1e3, 3), "GB/s": round(nbytes / (ms * 1e-3) / 1e9, 1),
                                   "copy_us": round(cp, 3), "frac_of_copy": round(cp / (ms * 1e3), 4)}
        del xs, rs, gus
    # the per-head q norm of the attention: rows of 128 in a strided [T, 16, 128] view of the qkv output (T = 8192)
    T = 8192
    bufs = [torch.randn(T, (HQ + 2 * HKV) * D + PAD, generator=g).to(torch.bfloat16).to(dev) for _ in range(NSETS)]
    qs = [bb[:, :HQ * D].view(T, HQ, D) for bb in bufs]
    wq = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(dev)
    ms, _ = time_graph(torch, lambda i: kernels.rms_norm(qs[i], wq, EPS), NSETS, max(40, steps), 20, WARM_S)
    nbytes = (2 * T * HQ * D + D) * 2
    gbs = nbytes / (ms * 1e-3) / 1e9
    cp = copy_ceiling_us(torch, dev, T * HQ * D * 2, 1, steps)
    out["rms_norm_q_heads_T8192"] = {"us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
                                     "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "rows": T * HQ, "n": D,
                                     "copy_us": round(cp, 3), "frac_of_copy": round(cp / (ms * 1e3), 4)}
    del bufs, qs
    for layer, (K, N) in GEMM_SHAPES.items():
        M = 2048
        a = (torch.randn(M, K, generator=g) / K ** 0.5).to(torch.bfloat16).to(dev)
        wt = torch.randn(N, K, generator=g).to(torch.bfloat16).to(dev)
        b = wt.t()
        ms, ms_ref = paired_ms(torch, lambda i: kernels.matmul(a, b), lambda i: torch.nn.functional.linear(a, wt),
                               4, max(40, steps), 20)
        tf = 2 * M * N * K / (ms * 1e-3) / 1e12
        out[f"gemm_bf16_{layer}_M{M}"] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 1),
                                           "frac_mfma": round(tf / BF16_PEAK_TFLOPS, 4),
                                           "torch_linear_us": round(ms_ref * 1e3, 2)}
        del a, wt, b
    # B row-major ([K, N], N-contiguous: the layout of the reference's own matmul test) at 2048 x 4096 x 1024
    M, N, K = 2048, 4096, 1024
    a = (torch.randn(M, K, generator=g) / K ** 0.5).to(torch.bfloat16).to(dev)
    b = torch.randn(K, N, generator=g).to(torch.bfloat16).to(dev)
    ms, ms_ref = paired_ms(torch, lambda i: kernels.matmul(a, b), lambda i: torch.matmul(a, b), 4, max(40, steps), 20)
    tf = 2 * M * N * K / (ms * 1e-3) / 1e12
    out["gemm_bf16_b_rowmajor_2048x4096x1024"] = {"us": round(ms * 1e3, 2), "TFLOP/s": round(tf, 1),
                                                  "frac_mfma": round(tf / BF16_PEAK_TFLOPS, 4),
                                                  "torch_matmul_us": round(ms_ref * 1e3, 2)}
    del a, b
    # decode-sized GEMMs are weight-bandwidth bound: rotate over enough weight copies (>= 512 MiB) that every call
    # reads its weight from HBM, as a decode step over 28 layers does
    # M = 32 (a decode batch), and M = 64 (a batch of 33-64 rows; their inputs from a generator of their own, so the
    # extras after them see the same inputs as without them)
    g64 = torch.Generator().manual_seed(64)
    for layer, M in [(name, 32) for name in GEMM_SHAPES] + [(name, 64) for name in GEMM_SHAPES]:
        K, N = GEMM_SHAPES[layer]
        nw = -(-(512 * 2 ** 20) // (N * K * 2))
        gl = g if M == 32 else g64
        a = (torch.randn(M, K, generator=gl) / K ** 0.5).to(torch.bfloat16).to(dev)
        w0 = torch.randn(N, K, generator=gl).to(torch.bfloat16).to(dev)
        ws = [w0.clone() for _ in range(nw)]
        ms, _ = time_graph(torch, lambda i: kernels.matmul(a, ws[i].t()), nw, max(nw, steps), nw, WARM_S)
        ms_ref, _ = time_graph(torch, lambda i: torch.nn.functional.linear(a, ws[i]), nw, max(nw, steps), nw, WARM_S)
        nbytes = 2 * (M * K + N * K + M * N)
        gbs = nbytes / (ms * 1e-3) / 1e9
        out[f"gemm_bf16_{layer}_M{M}"] = {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                                         "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                                         "torch_linear_us": round(ms_ref * 1e3, 2)}
        del a, w0, ws
    out["paged_decode_attention_B32"] = decode_attention(torch, dev, steps, g)
    # a small batch of long contexts: each (sequence, kv head) split over 8 blocks, merged inside the launch
    out["paged_decode_attention_B4_4k_8k"] = decode_attention(torch, dev, steps, g, batch=4, min_len=4096,
                                                              max_len=8192)
    out["prefill_attention_4x2048"] = prefill_attention(torch, dev, steps, g)
    out["prefill_chunk256_over_3840"] = prefill_chunk_over_prefix(torch, dev, steps, g)
    n = 4096
    a = torch.randn(n, n, generator=g).to(dev)
    b = torch.randn(n, n, generator=g).to(dev)
    ms, ms_ref = paired_ms(torch, lambda i: kernels.matmul(a, b), lambda i: torch.matmul(a, b), 1, 5, 2)
    tf = 2 * n ** 3 / (ms * 1e-3) / 1e12
    out["gemm_fp32_ieee_4096"] = {"us": round(ms * 1e3, 1), "TFLOP/s": round(tf, 1),
                                  "frac_fp32_peak": round(tf / FP32_PEAK_TFLOPS, 4),
                                  "torch_matmul_us": round(ms_ref * 1e3, 1)}
    return out


def decode_attention(torch, dev, steps, g, batch=32, min_len=512, max_len=2048, profile=False):
    """Paged decode attention of one Qwen3-0.6B layer for `batch` sequences with contexts U[min_len, max_len] (one
    query token each; the headline decode case: 32 sequences, U[512, 2048]), NSETS caches rotated so that the K/V
    (~170 MB per set at batch 32) come from HBM.
    bytes = sum(ctx) * Hkv * D * 2 (k, v) * 2 B + q read + out write + context lengths + block-table entries."""
    from nanovllm_hip.kernels.attention import flash_attn_with_kvcache
    lens = torch.randint(min_len, max_len + 1, (batch,), generator=g)
    need = [(int(n) + BLOCK - 1) // BLOCK for n in lens]
    nb = sum(need)
    sets = []
    for _ in range(NSETS):
        kc = torch.empty(nb, BLOCK, HKV, D, dtype=torch.bfloat16, device=dev).normal_()
        vc = torch.empty_like(kc).normal_()
        perm = torch.randperm(nb, generator=g)
        bt = torch.zeros(batch, max(need), dtype=torch.int32)
        used = 0
        for b, k in enumerate(need):
            bt[b, :k] = perm[used:used + k].to(torch.int32)
            used += k
        q = torch.randn(batch, 1, HQ, D, generator=g).to(torch.bfloat16).to(dev)
        sets.append((q, kc, vc, lens.to(torch.int32).to(dev), bt.to(dev)))
    scale = D ** -0.5
    ctx = int(lens.sum())
    nbytes = ctx * HKV * D * 2 * 2 + 2 * batch * HQ * D * 2 + batch * 4 + sum(need) * 4
    if profile:  # for rocprofv3 counter runs: `steps` eager launches over the sets, then the calibration copies
        for i in range(steps):
            flash_attn_with_kvcache(*sets[i % NSETS], scale, True)
        torch.cuda.synchronize()
        lib = bench_lib()
        n = 256 * 2 ** 20
        src = torch.ones(n // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            stream_copy(torch, lib, dst, src, n)
        torch.cuda.synchronize()
        print(f"profile: {steps} x paged decode attention (batch {batch}, {ctx} context tokens, {nbytes} algorithmic "
              f"bytes each); 5 x stream copy of {n} bytes", flush=True)
        return None
    ms, _ = time_graph(torch, lambda i: flash_attn_with_kvcache(*sets[i % NSETS], scale, True), NSETS,
                       max(40, steps), 8, WARM_S)
    gbs = nbytes / (ms * 1e-3) / 1e9
    del sets
    return {"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "context_tokens": ctx, "bytes": nbytes}


def profile_warmup(torch, call):
    """Eager calls until WARM_S of wall time has passed (the GPU raises its clocks over several milliseconds of
    load), for the kernel traces: their summaries average the calls after these. Returns the number of calls."""
    n, t0 = 0, time.perf_counter()
    while n < 4 or time.perf_counter() - t0 < WARM_S:
        for _ in range(4):
            call()
        n += 4
        torch.cuda.synchronize()
    return n


def prefill_attention(torch, dev, steps, g, nseq=4, L=2048, profile=False):
    """Causal prefill attention of one Qwen3-0.6B layer over nseq sequences of L tokens (k, v views of the qkv
    output). flops = 4 * D * Hq * sum over queries of the keys each sees (L (L + 1) / 2 per sequence)."""
    from nanovllm_hip.kernels.attention import flash_attn_varlen_func
    T = nseq * L
    buf = torch.randn(T, (HQ + 2 * HKV) * D + PAD, generator=g).to(torch.bfloat16).to(dev)
    q = buf[:, :HQ * D].view(T, HQ, D)
    k = buf[:, HQ * D:(HQ + HKV) * D].view(T, HKV, D)
    v = buf[:, (HQ + HKV) * D:(HQ + 2 * HKV) * D].view(T, HKV, D)
    cu = torch.arange(0, T + 1, L, dtype=torch.int32, device=dev)
    if profile:  # for a rocprofv3 kernel trace: warm-up launches (the clock ramp), then `steps` eager launches
        warm = profile_warmup(torch, lambda: flash_attn_varlen_func(q, k, v, L, cu, L, cu, D ** -0.5, True))
        for _ in range(steps):
            flash_attn_varlen_func(q, k, v, L, cu, L, cu, D ** -0.5, True)
        torch.cuda.synchronize()
        print(f"profile: {warm} warm-up, then {steps} prefill attention launches ({nseq} x {L} tokens)", flush=True)
        return None
    ms, _ = time_graph(torch, lambda i: flash_attn_varlen_func(q, k, v, L, cu, L, cu, D ** -0.5, True), 4,
                       max(20, steps // 4), 4, WARM_S)
    flops = 4 * D * HQ * nseq * L * (L + 1) // 2
    tf = flops / (ms * 1e-3) / 1e12
    return {"us": round(ms * 1e3, 1), "TFLOP/s": round(tf, 1), "frac_mfma": round(tf / BF16_PEAK_TFLOPS, 4)}


def prefill_chunk_over_prefix(torch, dev, steps, g, chunk=256, prefix=3840, profile=False):
    """Causal attention of one Qwen3-0.6B layer for a `chunk`-token piece of a prompt over its `prefix` cached keys
    (chunked prefill / prefix cache: the keys come through a block table of the paged 256-slot cache). flops = 4 *
    D * Hq * sum over the chunk's queries of the keys each sees."""
    from nanovllm_hip.kernels.attention import flash_attn_varlen_func
    lk = prefix + chunk
    nb = (lk + BLOCK - 1) // BLOCK
    kc = torch.randn(nb, BLOCK, HKV, D, generator=g).to(torch.bfloat16).to(dev)
    vc = torch.randn(nb, BLOCK, HKV, D, generator=g).to(torch.bfloat16).to(dev)
    bt = torch.randperm(nb, generator=g).to(torch.int32).view(1, nb).to(dev)
    q = torch.randn(chunk, HQ, D, generator=g).to(torch.bfloat16).to(dev)
    cq = torch.tensor([0, chunk], dtype=torch.int32, device=dev)
    ck = torch.tensor([0, lk], dtype=torch.int32, device=dev)
    if profile:  # for a rocprofv3 kernel trace: warm-up calls (the clock ramp), then `steps` eager calls
        warm = profile_warmup(torch, lambda: flash_attn_varlen_func(q, kc, vc, chunk, cq, lk, ck, D ** -0.5, True, bt))
        for _ in range(steps):
            flash_attn_varlen_func(q, kc, vc, chunk, cq, lk, ck, D ** -0.5, True, bt)
        torch.cuda.synchronize()
        print(f"profile: {warm} warm-up, then {steps} prefill attention calls ({chunk}-token chunk over {prefix} "
              f"cached keys)", flush=True)
        return None
    ms, _ = time_graph(torch, lambda i: flash_attn_varlen_func(q, kc, vc, chunk, cq, lk, ck, D ** -0.5, True, bt), 4,
                       max(20, steps // 4), 4, WARM_S)
    flops = 4 * D * HQ * sum(prefix + i + 1 for i in range(chunk))
    tf = flops / (ms * 1e-3) / 1e12
    return {"us": round(ms * 1e3, 1), "TFLOP/s": round(tf, 1), "frac_mfma": round(tf / BF16_PEAK_TFLOPS, 4)}


def e2e_decode_step(torch, dev, batch=32, layers=28, min_len=512, max_len=2048, reps=20, profile_replays=0):
    """One decode step of a random-init Qwen3-0.6B-shaped model (28 layers, tied embeddings, bf16) for 32 sequences
    with prompts of U[512, 2048] random ids in 256-slot paged blocks, through the hip backend (the HIP kernels for
    the norms, the fused pre-attention kernel, every projection and the LM head, gate_up with the SiLU epilogue, the
    paged decode attention), replayed from a HIP graph: microseconds per step, tokens per second, kernel nodes.
    The prompts are prefilled first (HIP prefill attention) so the caches hold real K/V."""
    from nanovllm_hip.harness.decode import Batch, DecodeStep, graph_nodes, prefill, replay_us
    from nanovllm_hip.harness.qwen3 import Qwen3, Qwen3Config
    cfg = Qwen3Config(num_hidden_layers=layers)
    model = Qwen3(cfg, dev, seed=0)
    b = Batch(cfg, batch, 4, min_len, max_len, 0, dev)
    model.allocate_kv_cache(b.num_blocks)
    first, _ = prefill(model, b, "hip")
    step = DecodeStep(model, b, "hip")
    with torch.inference_mode():
        step.set_inputs(first, 0)
        step.capture()
    if profile_replays:  # for a rocprofv3 kernel trace: eager-synchronised replays, nothing else launched
        torch.cuda.synchronize()
        for _ in range(profile_replays):
            step.graph.replay()
        torch.cuda.synchronize()
        print(f"profile: {profile_replays} decode-step graph replays", flush=True)
    us = replay_us(step, reps)
    kernels_n, nodes = graph_nodes(step.graph)
    out = {"us": round(us, 1), "tokens_per_s": round(batch / (us * 1e-6), 1), "kernels": kernels_n,
           "context_tokens": sum(b.lens), "batch": batch, "layers": layers}
    del step, model
    torch.cuda.empty_cache()
    return out


def e2e_mixed_step(torch, dev, decodes=16, chunk=240, layers=28, min_len=512, max_len=2048, reps=20):
    """One mixed step of the same model: `decodes` decode requests (prompts of U[512, 2048] random ids, prefilled
    first) and a `chunk`-token prefill chunk, 256 tokens in all, through the hip backend with the HIP varlen paged
    attention. Timed as piecewise HIP graphs (one per segment between two attentions, the attentions eager) and
    as the same segments run eagerly: microseconds per step."""
    from nanovllm_hip.harness.decode import Batch, prefill
    from nanovllm_hip.harness.mixed import Piecewise, Request, prepare_mixed
    from nanovllm_hip.harness.qwen3 import Qwen3, Qwen3Config
    cfg = Qwen3Config(num_hidden_layers=layers)
    model = Qwen3(cfg, dev, seed=0)
    b = Batch(cfg, decodes, 4, min_len, max_len, 0, dev)
    model.allocate_kv_cache(b.num_blocks + 1)
    first, _ = prefill(model, b, "hip")
    reqs = [Request(p.tolist() + [t], tab, len(p)) for p, tab, t in zip(b.prompts, b.tables, first)]
    g = torch.Generator().manual_seed(5)
    reqs.append(Request(torch.randint(0, cfg.vocab_size, (chunk,), generator=g).tolist(), [b.num_blocks], 0, chunk))
    ids, pos, ctx, _ = prepare_mixed(reqs, 256, dev)
    n = ids.shape[0]
    out = {"tokens": n, "decode_requests": decodes, "prefill_chunk": chunk, "layers": layers}
    for name, pw in (("eager_us", Piecewise(model, [n])), ("piecewise_graph_us", Piecewise(model, [n]))):
        if name == "piecewise_graph_us":
            pw.record()
        for _ in range(3):
            pw.run(ids, pos, ctx)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            pw.run(ids, pos, ctx)
        end.record()
        end.synchronize()
        out[name] = round(start.elapsed_time(end) * 1e3 / reps, 1)
        del pw
    del model
    torch.cuda.empty_cache()
    return out


def profile_run(torch, oracle, kernels, wl, steps):
    """Eager launches for rocprofv3 counter runs (no graph): the headline kernel, then the other HBM-bound kernels
    at their bench sizes (RMSNorm / Add+RMSNorm / SiLU x Mul / store_kvcache at T = 8192, the fused kernel at
    T = 2048 with write_k), `steps` launches each, then 5 plain copies of 256 MiB (nvhip_bench_stream_copy: 256 MiB
    read + 256 MiB written each) that calibrate the byte counters."""
    for i in range(steps):
        wl.call(i, kernels.qk_norm_rope_kv)
    torch.cuda.synchronize()
    dev = wl.k_cache.device
    g = torch.Generator("cpu").manual_seed(2)
    T, H, I = 8192, HQ * D // 2, 3 * HQ * D // 2
    xs = [torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev) for _ in range(2)]
    w = (1 + 0.1 * torch.randn(H, generator=g)).to(torch.bfloat16).to(dev)
    gus = [torch.randn(T, 2 * I, generator=g).to(torch.bfloat16).to(dev) for _ in range(2)]
    for i in range(steps):
        kernels.rms_norm(xs[i % 2], w, EPS)
    for i in range(steps):
        kernels.fused_add_rms_norm(xs[i % 2], xs[(i + 1) % 2], w, EPS)
    for i in range(steps):
        kernels.silu_and_mul(gus[i % 2])
    for i in range(steps):
        s = wl.sets[i % NSETS]
        kernels.store_kvcache(s["k"], s["v"], wl.k_cache, wl.v_cache, s["slots"])
    torch.cuda.synchronize()
    del xs, gus
    wl2 = FusedWorkload(2048, dev, torch, oracle, seed=2048)
    for i in range(steps):
        wl2.call(i, kernels.qk_norm_rope_kv, True)
    torch.cuda.synchronize()
    lib = bench_lib()
    n = 256 * 2 ** 20
    src = torch.ones(n // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(5):
        stream_copy(torch, lib, dst, src, n)
    torch.cuda.synchronize()
    print(f"profile: {steps} x qk_norm_rope_kv (T={wl.T}, {fused_bytes(wl.T, wl.n_valid)} algorithmic bytes each); "
          f"{steps} x rms_norm ({(2 * T * H + H) * 2} B), fused_add_rms_norm ({(4 * T * H + H) * 2} B), "
          f"silu_and_mul ({3 * T * I * 2} B), store_kvcache ({T * (4 * HKV * D * 2 + 4)} B) at T={T}; {steps} x "
          f"qk_norm_rope_kv T=2048 write_k ({fused_bytes(2048, 2048, True)} B); 5 x stream copy of {n} bytes",
          flush=True)


def profile_gemm(torch, kernels, dev, steps, M):
    g = torch.Generator("cpu").manual_seed(3)
    for layer, (K, N) in GEMM_SHAPES.items():
        a = (torch.randn(M, K, generator=g) / K ** 0.5).to(torch.bfloat16).to(dev)
        w0 = torch.randn(N, K, generator=g).to(torch.bfloat16).to(dev)
        # up to a few hundred rows the weight stream matters: rotate over >= 512 MiB of weight copies so each call
        # reads its weight from HBM, as a step over 28 layers does
        ws = [w0.clone() for _ in range(-(-(512 * 2 ** 20) // (N * K * 2)))] if M <= 256 else [w0]
        # all of ours, then all of torch's: neither reads a weight copy the other has just brought into the caches
        for i in range(steps):
            kernels.matmul(a, ws[i % len(ws)].t())
        torch.cuda.synchronize()
        for i in range(steps):
            torch.nn.functional.linear(a, ws[i % len(ws)])
        torch.cuda.synchronize()
        print(f"profile: {steps} x matmul, then {steps} x F.linear, {layer} {M}x{N}x{K}, {len(ws)} weight copies",
              flush=True)
        del ws, w0, a


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=2000)
    p.add_argument("--tokens", type=int, default=8192)
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-extra", action="store_true", help="only the headline kernel")
    p.add_argument("--no-e2e", action="store_true", help="skip the end-to-end decode step (part of the extras)")
    p.add_argument("--profile-gemm", action="store_true",
                   help="for rocprofv3 runs: --steps eager launches of the bf16 GEMM at each Qwen3-0.6B projection "
                        "shape (M = --gemm-m), each followed by torch.nn.functional.linear on the same tensors")
    p.add_argument("--gemm-m", type=int, default=2048, help="M of the --profile-gemm products")
    p.add_argument("--profile-e2e", action="store_true",
                   help="for rocprofv3 kernel traces: build the Qwen3-0.6B-shaped model, prefill, capture the batch-32 "
                        "decode step and replay it --steps times, then print the e2e line")
    p.add_argument("--profile-prefill", action="store_true",
                   help="for rocprofv3 kernel traces: --steps eager launches of the prefill attention (4 x 2048 "
                        "tokens, one Qwen3-0.6B layer)")
    p.add_argument("--profile-chunk", action="store_true",
                   help="for rocprofv3 kernel traces: --steps eager calls of the prefill attention for a 256-token "
                        "chunk over 3840 cached keys (one Qwen3-0.6B layer)")
    p.add_argument("--profile-decode", action="store_true",
                   help="for rocprofv3 counter runs: --steps eager launches of the batch-32 paged decode attention "
                        "(one Qwen3-0.6B layer, contexts U[512, 2048], the sets rotated), then 5 plain copies of 256 "
                        "MiB that calibrate the byte counters")
    p.add_argument("--profile-mixed", action="store_true",
                   help="for rocprofv3 kernel traces: build the model, prefill 16 requests, then time the 256-token "
                        "mixed step (16 decodes + a 240-token chunk) --steps times eagerly and --steps times from "
                        "piecewise graphs, and print the mixed-step line")
    p.add_argument("--profile", action="store_true",
                   help="for rocprofv3 counter runs: --steps eager launches of the headline kernel (no graph), of "
                        "RMSNorm / Add+RMSNorm / SiLU x Mul / store_kvcache at T=8192 and of the fused kernel at "
                        "T=2048 with write_k, then 5 plain copies of 256 MiB (256 MiB read + 256 MiB written each) "
                        "to calibrate the byte counters; prints the launch list instead of the JSON line")
    p.add_argument("--hbm-sweep", action="store_true",
                   help="only the HBM ceiling sweep (read-only, write-only and copy streams), every point printed, "
                        "at 1 GiB per launch and at the headline's bytes per launch")
    p.add_argument("--mfma-probe", action="store_true",
                   help="only the bf16 MFMA ceiling probe (MFMA issue with 0-1 KB of LDS reads per MFMA, 1-4 waves "
                        "per SIMD), every point printed")
    args = p.parse_args()
    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus}: only one GPU is measured (the kernel path has no collective: under "
              "tensor parallelism each rank runs these kernels on its own head / column shard). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import oracle
    import nanovllm_hip.kernels as kernels

    dev = torch.device("cuda:0")
    if args.hbm_sweep:
        print(json.dumps(hbm_ceiling(torch, dev, table=True)), flush=True)
        print(json.dumps(hbm_ceiling(torch, dev, table=True, moved=fused_bytes(args.tokens, args.tokens))),
              flush=True)
        return
    if args.mfma_probe:
        print(json.dumps(mfma_ceiling(torch, dev)), flush=True)
        return
    if args.profile_gemm:
        profile_gemm(torch, kernels, dev, args.steps, args.gemm_m)
        return
    if args.profile_prefill:
        prefill_attention(torch, dev, args.steps, torch.Generator().manual_seed(0), profile=True)
        return
    if args.profile_chunk:
        prefill_chunk_over_prefix(torch, dev, args.steps, torch.Generator().manual_seed(0), profile=True)
        return
    if args.profile_mixed:
        print(json.dumps(e2e_mixed_step(torch, dev, reps=args.steps)), flush=True)
        return
    if args.profile_decode:
        decode_attention(torch, dev, args.steps, torch.Generator("cpu").manual_seed(1234), profile=True)
        return
    if args.profile_e2e:
        print(json.dumps(e2e_decode_step(torch, dev, profile_replays=args.steps)), flush=True)
        return
    T = args.tokens
    wl = FusedWorkload(T, dev, torch, oracle)
    if args.profile:
        profile_run(torch, oracle, kernels, wl, args.steps)
        return
    # exactly --steps launches (the NSETS sets in turn) recorded into one graph; one replay is timed
    ms, host_us = time_steps(torch, lambda i: wl.call(i, kernels.qk_norm_rope_kv), args.steps, args.warmup, WARM_S)
    steps_done = args.steps
    nbytes = fused_bytes(T, wl.n_valid)
    gbs = nbytes / (ms * 1e-3) / 1e9
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("bytes_per_launch")
    result = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps_done,
        "warmup": args.warmup, "ms_per_step": round(ms, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": f"qk_norm_rope_kv Qwen3-0.6B attention (Hq 16, Hkv 8, D 128), T={T}, qkv view of "
                               f"[T, 4096+{PAD}], 4 sequences, 512x256-slot paged KV, all slots valid, write_k=False",
                   "tokens": T, "bytes_per_step": nbytes, "rotating_sets": NSETS,
                   "rotating_read_bytes": NSETS * T * ((HQ + 2 * HKV) * D + PAD) * 2,
                   "timing": f"{steps_done} eager launches timed with HIP events behind a queued graph of 64 "
                             f"untimed launches; host submission {host_us:.1f} us per launch"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic},
    }
    if not args.no_extra:
        result["extra"] = ceilings(torch, kernels, wl, args.steps, gbs)
        result["extra"]["hbm_ceiling"] = hbm_ceiling(torch, dev)
        # the same sweep at the headline's bytes per launch (138.5 MB: the launch ramp and drain at that size)
        result["extra"]["hbm_ceiling_headline_bytes"] = hbm_ceiling(torch, dev, moved=fused_bytes(T, wl.n_valid))
        result["extra"].update(extras(torch, oracle, kernels, dev, args.steps))
        if not args.no_e2e:
            result["extra"]["e2e_decode_step"] = e2e_decode_step(torch, dev)
            result["extra"]["e2e_mixed_step"] = e2e_mixed_step(torch, dev)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(torch, oracle, T)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
