"""Torch restatement of the reference's eager code for the kernel path (TEST INFRASTRUCTURE ONLY: see __init__).

Every function takes and returns torch tensors and runs on whatever device its inputs are on (CPU for the oracle;
the GPU tests may also run it on the GPU to get torch's own GPU rounding). bf16 activations, fp32 arithmetic, and
a bf16 rounding exactly where the reference's torch code has a `.to(bfloat16)` or a bf16 multiply.
"""
import torch

from oracle import aten_reduce

BF16 = torch.bfloat16


def rms_forward(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """RMSNorm of the last dim (layers/layernorm.py:20-30): y = bf16(x * rsqrt(mean(x^2) + eps)) * weight.

    x: bf16 [..., n] (any strides); weight: bf16 [n]. The fp32 normalised value is rounded to x's dtype before
    the weight multiply, and that multiply is a bf16 x bf16 product (computed in fp32, rounded to bf16)."""
    xf = x.to(torch.float32)
    mean_sq = xf.pow(2).mean(dim=-1, keepdim=True)
    normed = xf * torch.rsqrt(mean_sq + eps)
    return normed.to(x.dtype).mul_(weight)  # in place: the product keeps x's dtype whatever weight's dtype


def add_rms_forward(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """Add + RMSNorm (layers/layernorm.py:32-44). Returns (y, new_residual).

    s = fp32(x) + fp32(residual); new_residual = bf16(s); y = RMSNorm of the *unrounded* fp32 s."""
    s = x.to(torch.float32) + residual.to(torch.float32)
    new_residual = s.to(x.dtype)
    mean_sq = s.pow(2).mean(dim=-1, keepdim=True)
    normed = s * torch.rsqrt(mean_sq + eps)
    return normed.to(x.dtype).mul_(weight), new_residual


def _gpu_rstd(s: torch.Tensor, eps: float) -> torch.Tensor:
    """rsqrt(mean(s^2) + eps) per row of the fp32 CPU tensor s [..., n] with torch's GPU numerics: the mean in
    ATen's GPU summation order for that many rows (oracle.aten_reduce), the fp32 add of eps, and torch.rsqrt's
    double-precision evaluation rounded to float."""
    n = s.shape[-1]
    rows = s.reshape(-1, n)
    mean = torch.from_numpy(aten_reduce.mean_sq(rows.numpy(), rows.shape[0]))
    var = mean + torch.tensor(eps, dtype=torch.float32)
    return torch.rsqrt(var.double()).float().reshape(*s.shape[:-1], 1)


def rms_forward_gpu(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """rms_forward (layers/layernorm.py:20-30) as torch computes it eagerly on an MI355X, restated on the CPU: the
    same rounding points as rms_forward, with the GPU's mean and rsqrt (_gpu_rstd). x [..., n] bf16 on the CPU; the
    rows of the call are all of x's rows (a [T, H, n] view is T * H rows)."""
    xf = x.to(torch.float32)
    return (xf * _gpu_rstd(xf, eps)).to(x.dtype).mul_(weight)


def add_rms_forward_gpu(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    """add_rms_forward (layers/layernorm.py:32-44) with torch's GPU numerics (see rms_forward_gpu)."""
    s = x.to(torch.float32) + residual.to(torch.float32)
    return (s * _gpu_rstd(s, eps)).to(x.dtype).mul_(weight), s.to(x.dtype)


def rope_cos_sin_cache(head_size: int, max_position: int, base: float) -> torch.Tensor:
    """The rotary table (layers/rotary_embedding.py:19-35): [max_position, 1, head_size] fp32, row p = (cos | sin)
    of p * inv_freq, inv_freq[i] = 1 / base^(2i / head_size), all computed in fp32."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_size, 2, dtype=torch.float32) / head_size))
    pos = torch.arange(max_position, dtype=torch.float32)
    angles = pos[:, None] * inv_freq[None, :]  # fp32 outer product, as the reference's einsum "i,j -> ij"
    return torch.cat((angles.cos(), angles.sin()), dim=-1).unsqueeze(1)


def apply_rotary_emb(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE (layers/rotary_embedding.py:6-14): halves x1, x2 of fp32(x);
    y1 = x1*cos - x2*sin, y2 = x2*cos + x1*sin, each product a separately rounded fp32 tensor; result in x's dtype."""
    x1, x2 = torch.chunk(x.to(torch.float32), 2, dim=-1)
    y1 = x1 * cos - x2 * sin
    y2 = x2 * cos + x1 * sin
    return torch.cat((y1, y2), dim=-1).to(x.dtype)


def rotary_forward(positions: torch.Tensor, q: torch.Tensor, k: torch.Tensor, cos_sin_cache: torch.Tensor):
    """RotaryEmbedding.forward (layers/rotary_embedding.py:37-48): the table row of each token's position,
    broadcast over heads, applied to q [T, Hq, D] and k [T, Hkv, D]."""
    cos_sin = cos_sin_cache[positions]  # [T, 1, D]
    cos, sin = cos_sin.chunk(2, dim=-1)
    return apply_rotary_emb(q, cos, sin), apply_rotary_emb(k, cos, sin)


def store_kvcache(k: torch.Tensor, v: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                  slot_mapping: torch.Tensor) -> None:
    """Paged KV write (layers/attention.py:11-41), in place: for each token t with slot s = slot_mapping[t] != -1,
    the whole [Hkv, D] row of k[t] / v[t] goes to slot s of the caches [blocks, block_size, Hkv, D]
    (flat slot index s = block * block_size + offset). Rows of tokens with slot -1 are not written."""
    hkv, d = k.shape[1], k.shape[2]
    keep = slot_mapping != -1
    slots = slot_mapping[keep].long()
    k_cache.view(-1, hkv, d)[slots] = k[keep]
    v_cache.view(-1, hkv, d)[slots] = v[keep]


def qk_norm_rope_kv(q, k, v, positions, q_weight, k_weight, eps, cos_sin_cache, k_cache, v_cache, slot_mapping,
                    write_k, gpu_numerics=False):
    """The unfused pre-attention composition (models/qwen3.py:89-105 then layers/attention.py:64-76):
    q_norm and k_norm (rms_forward per head row), rotary_emb, then store_kvcache of the rotated k and raw v.
    Mutates the caches (unless they are empty); returns (q_out [T, Hq, D] contiguous, k_out or None).
    gpu_numerics: the norms as torch computes them on the GPU (rms_forward_gpu; CPU tensors only)."""
    norm = rms_forward_gpu if gpu_numerics else rms_forward
    qn = norm(q, q_weight, eps)
    kn = norm(k, k_weight, eps)
    q_out, k_rot = rotary_forward(positions, qn, kn, cos_sin_cache)
    if k_cache.numel() > 0:
        store_kvcache(k_rot, v, k_cache, v_cache, slot_mapping)
    return q_out.contiguous(), (k_rot.contiguous() if write_k else None)


def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    """SiluAndMul (layers/activation.py:15-18): gate, up = halves of the last dim; silu(gate) in fp32 rounded to
    x's dtype, times up (a bf16 product)."""
    gate, up = x.chunk(2, -1)
    return torch.nn.functional.silu(gate) * up


def matmul_fp64(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """The GEMM reference of tests/test_kernels_matmul.py:52: exact-ish float64 product of the inputs."""
    return a.double() @ b.double()


def paged_decode_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, context_lens: torch.Tensor,
                           block_table: torch.Tensor, scale: float, causal: bool = True,
                           compute_dtype=torch.float32) -> torch.Tensor:
    """The decode call of layers/attention.py:84-90, flash_attn_with_kvcache(q, k_cache, v_cache,
    cache_seqlens=context_lens, block_table=block_table, softmax_scale=scale, causal=True), restated.

    q [num_seqs, q_len, Hq, D]; caches [num_blocks, block_size, Hkv, D] (model_runner.py:262-267); block_table
    [num_seqs, max_blocks] int32; context_lens [num_seqs] int32. Cache token j of sequence b is slot
    block_table[b, j // block_size] * block_size + j % block_size (model_runner.py:340). Query i of a sequence with
    L cached tokens sees tokens j <= L - q_len + i when causal (the mask is aligned to the bottom right, as the comment
    at attention.py:86 says), all L otherwise; head h reads kv head h // (Hq / Hkv). softmax(q.k * scale) @ v in
    compute_dtype, output in q's dtype; a query that sees no token gets zeros."""
    num_seqs, q_len, Hq, D = q.shape
    block_size, Hkv = k_cache.shape[1], k_cache.shape[2]
    g = Hq // Hkv
    out = torch.zeros(q.shape, dtype=compute_dtype)
    kf = k_cache.reshape(-1, Hkv, D)
    vf = v_cache.reshape(-1, Hkv, D)
    for b in range(num_seqs):
        L = int(context_lens[b])
        if L <= 0:
            continue
        j = torch.arange(L)
        slots = block_table[b].long()[j // block_size] * block_size + j % block_size
        kb = kf[slots].to(compute_dtype).repeat_interleave(g, dim=1)   # [L, Hq, D]
        vb = vf[slots].to(compute_dtype).repeat_interleave(g, dim=1)
        qb = q[b].to(compute_dtype)                                    # [q_len, Hq, D]
        s = torch.einsum("ihd,jhd->hij", qb, kb) * scale               # [Hq, q_len, L]
        if causal:
            limit = L - q_len + torch.arange(q_len)                    # last visible token of query i
            s = s.masked_fill(j[None, None, :] > limit[None, :, None], float("-inf"))
        p = torch.softmax(s, dim=-1)
        p = torch.nan_to_num(p, nan=0.0)                               # queries that see nothing
        out[b] = torch.einsum("hij,jhd->ihd", p, vb)
    return out.to(q.dtype)


def varlen_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cu_seqlens_q: torch.Tensor,
                     cu_seqlens_k: torch.Tensor, scale: float, causal: bool = True,
                     block_table: torch.Tensor | None = None, compute_dtype=torch.float32) -> torch.Tensor:
    """The prefill call of layers/attention.py:77-83, flash_attn_varlen_func(q, k, v, max_seqlen_q, cu_seqlens_q,
    max_seqlen_k, cu_seqlens_k, softmax_scale=scale, causal=True, block_table), restated.

    q [Tq, Hq, D]; sequence b owns query rows cu_seqlens_q[b] .. cu_seqlens_q[b+1]-1 and lk = cu_seqlens_k[b+1] -
    cu_seqlens_k[b] keys: rows cu_seqlens_k[b] + j of k, v [Tk, Hkv, D], or with a block table (the prefix cache,
    model_runner.py:311-312) slots block_table[b][j // bs] * bs + j % bs of the caches [blocks, bs, Hkv, D]. Query i
    sees keys j <= lk - lq + i when causal (bottom-right alignment), all lk otherwise; head h reads kv head
    h // (Hq / Hkv); a query that sees no key gets zeros. softmax(q.k * scale) @ v in compute_dtype."""
    Tq, Hq, D = q.shape
    out = torch.zeros(q.shape, dtype=compute_dtype)
    for b in range(cu_seqlens_q.numel() - 1):
        q0, q1 = int(cu_seqlens_q[b]), int(cu_seqlens_q[b + 1])
        k0, k1 = int(cu_seqlens_k[b]), int(cu_seqlens_k[b + 1])
        lq, lk = q1 - q0, k1 - k0
        if lq <= 0 or lk <= 0:
            continue
        if block_table is None:
            kb, vb = k[k0:k1], v[k0:k1]
        else:
            bs, hkv = k.shape[1], k.shape[2]
            j = torch.arange(lk)
            slots = block_table[b].long()[j // bs] * bs + j % bs
            kb, vb = k.reshape(-1, hkv, D)[slots], v.reshape(-1, hkv, D)[slots]
        g = Hq // kb.shape[1]
        kb = kb.to(compute_dtype).repeat_interleave(g, dim=1)
        vb = vb.to(compute_dtype).repeat_interleave(g, dim=1)
        s = torch.einsum("ihd,jhd->hij", q[q0:q1].to(compute_dtype), kb) * scale
        if causal:
            limit = lk - lq + torch.arange(lq)
            s = s.masked_fill(torch.arange(lk)[None, None, :] > limit[None, :, None], float("-inf"))
        p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
        out[q0:q1] = torch.einsum("hij,jhd->ihd", p, vb)
    return out.to(q.dtype)
