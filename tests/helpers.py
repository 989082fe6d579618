"""Shared input builders and comparison metrics for the tests (inputs are generated on the CPU with a seeded
torch.Generator, so the CPU oracle and the GPU see the same values)."""
import torch

HEAD_DIM, Q_HEADS, KV_HEADS, MAX_POS, THETA, BLOCK = 128, 16, 8, 40960, 1e6, 256
HIDDEN, INTERMEDIATE = 1024, 3072
EPS = 1e-6


def ulp_line(t: torch.Tensor) -> torch.Tensor:
    """bf16 bit patterns mapped to a monotonic integer line (the reference tests' metric,
    tests/test_kernels_qk_rope_kv.py:46-51)."""
    i = t.detach().cpu().contiguous().view(torch.int16).to(torch.int32)
    return torch.where(i < 0, -(i & 0x7FFF), i)


def ulp_diff(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    return (ulp_line(a) - ulp_line(b)).abs()


def max_ulp(a: torch.Tensor, b: torch.Tensor) -> int:
    assert a.shape == b.shape, (a.shape, b.shape)
    d = ulp_diff(a, b)
    return int(d.max()) if d.numel() else 0


def bf16_randn(shape, g, scale=1.0):
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def norm_weight(n, g):
    return (1 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16)


def random_block_table_slots(T, num_blocks, g, num_seqs=4, pad_frac=0.0):
    """Slots of T tokens split into num_seqs equal-ish sequences, each in its own random distinct blocks
    (slot = block * BLOCK + offset, as model_runner.py:303-310 builds them), with about pad_frac of the entries
    set to -1 (padding). Also returns the positions (contiguous per sequence)."""
    lens = [T // num_seqs + (1 if i < T % num_seqs else 0) for i in range(num_seqs)]
    perm = torch.randperm(num_blocks, generator=g).tolist()
    slots, positions = [], []
    for n in lens:
        nb = (n + BLOCK - 1) // BLOCK
        blocks, perm = perm[:nb], perm[nb:]
        assert len(blocks) == nb, "cache too small for the requested tokens"
        start = int(torch.randint(0, 1024, (1,), generator=g))
        for i in range(n):
            slots.append(blocks[i // BLOCK] * BLOCK + i % BLOCK)
            positions.append(start + i)
    slots = torch.tensor(slots, dtype=torch.int32)
    positions = torch.tensor(positions, dtype=torch.int64)
    if pad_frac > 0 and T > 0:
        pad = torch.rand(T, generator=g) < pad_frac
        slots[pad] = -1
    return slots, positions


def paged_decode_abi(q, kc, vc, lens, bt, scale, causal, workspace):
    """Calls nvhip_paged_decode_attention_bf16 directly: workspace False -> one block per (sequence, kv head);
    True -> a zero-filled workspace of the size the entry point asks for (its context splits, or the length-aware
    balance of 256 .. 512 pairs). Returns the output and the workspace size."""
    from nanovllm_hip import _lib
    num_seqs, q_len, Hq, D = q.shape
    qf = q.reshape(num_seqs * q_len, Hq, D)
    out = torch.empty_like(qf)
    lib = _lib.lib()
    need = lib.nvhip_paged_decode_attention_workspace_size(num_seqs, q_len, Hq, kc.shape[2], D, kc.shape[1],
                                                           bt.shape[1])
    # zero-filled: the entry point's per-pair counters must be zero before a call (each call leaves them zero)
    ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=q.device) if workspace else None
    status = lib.nvhip_paged_decode_attention_bf16(
        out.data_ptr(), qf.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(), lens.data_ptr(), num_seqs,
        q_len, Hq, kc.shape[2], D, kc.shape[1], kc.shape[0], bt.shape[1], qf.stride(0), qf.stride(1),
        out.stride(0), out.stride(1), scale, int(causal), ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0, _lib.stream_of(q))
    _lib.check(status, "paged_decode_attention")
    if ws is not None:  # the call leaves the per-pair counters (the workspace's first num_seqs x Hkv words) zero
        assert not torch.any(ws[:num_seqs * kc.shape[2] * 4]).item()
    return out.view(q.shape), need
