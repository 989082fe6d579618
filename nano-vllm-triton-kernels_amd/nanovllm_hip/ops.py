"""PyTorch custom ops (namespace `nvhip`) over the C-ABI kernels of libnvhip.so.

Each op has a CUDA (= ROCm/HIP device) implementation that allocates its outputs with torch's caching allocator and
launches the kernel on torch's current stream through ctypes, and a fake (meta) implementation so torch.compile and
graph capture can trace it. There is no CPU implementation: CPU tensors raise in the dispatcher.

The user-facing functions with the reference's signatures are in nanovllm_hip.kernels; these ops take the already
validated, normalised arguments.
"""
import torch

from nanovllm_hip import _lib

_DEF = torch.library.Library("nvhip", "DEF")

_DEF.define(
    "qk_norm_rope_kv(Tensor q, Tensor k, Tensor v, Tensor positions, Tensor q_weight, Tensor k_weight, float eps, "
    "Tensor cos_sin_cache, Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor? slot_mapping, bool write_k) "
    "-> (Tensor, Tensor)")
_DEF.define("rms_norm(Tensor x, Tensor w, float eps) -> Tensor")
_DEF.define("fused_add_rms_norm(Tensor x, Tensor residual, Tensor w, float eps) -> (Tensor, Tensor)")
_DEF.define("fused_add_rms_norm_(Tensor x, Tensor(a!) residual, Tensor w, float eps) -> Tensor")
_DEF.define("silu_and_mul(Tensor x) -> Tensor")
_DEF.define("matmul(Tensor a, Tensor b, str input_precision) -> Tensor")
_DEF.define("matmul_silu_mul(Tensor a, Tensor w) -> Tensor")
_DEF.define("rms_norm_matmul(Tensor x, Tensor? residual, Tensor norm_w, float eps, Tensor w, bool silu) "
            "-> (Tensor, Tensor)")
_DEF.define("matmul_add_rms_norm(Tensor x, Tensor w, Tensor residual, Tensor norm_w, float eps) -> (Tensor, Tensor)")
_DEF.define("qk_norm_rope_kv_decode_attention(Tensor q, Tensor k, Tensor v, Tensor positions, Tensor q_w, Tensor k_w, "
            "float eps, Tensor cos_sin, Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor slot_mapping, "
            "Tensor cache_seqlens, Tensor block_table, float scale) -> Tensor")
_DEF.define("prefill_attention(Tensor q, Tensor k, Tensor v, Tensor cu_seqlens_q, Tensor cu_seqlens_k, "
            "int max_seqlen_q, int max_seqlen_k, float scale, bool causal, Tensor? block_table) -> Tensor")
_DEF.define("prefill_attention_out(Tensor q, Tensor k, Tensor v, Tensor cu_seqlens_q, Tensor cu_seqlens_k, "
            "int max_seqlen_q, int max_seqlen_k, float scale, bool causal, Tensor? block_table, "
            "Tensor(a!) out) -> ()")
_DEF.define("store_kvcache(Tensor key, Tensor value, Tensor(a!) k_cache, Tensor(b!) v_cache, "
            "Tensor slot_mapping) -> ()")
_DEF.define("paged_decode_attention(Tensor q, Tensor k_cache, Tensor v_cache, Tensor block_table, "
            "Tensor context_lens, int q_len, float scale, bool causal) -> Tensor")
_DEF.define("argmax(Tensor logits) -> Tensor")


# ------------------------------------------------------------------ qk_norm_rope_kv

def _qk_outputs(q, k, write_k):
    T, Hq, D = q.shape
    q_out = q.new_empty((T, Hq, D))
    k_out = k.new_empty((T, k.shape[1], D)) if write_k else k.new_empty((0,))
    return q_out, k_out


def _qk_norm_rope_kv_impl(q, k, v, positions, q_weight, k_weight, eps, cos_sin_cache, k_cache, v_cache,
                          slot_mapping, write_k):
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    q_out, k_out = _qk_outputs(q, k, write_k)
    store = k_cache.numel() > 0
    cs = cos_sin_cache
    status = _lib.lib().nvhip_qk_norm_rope_kv_bf16(
        q_out.data_ptr(), k_out.data_ptr() if write_k else None,
        q.data_ptr(), k.data_ptr(), v.data_ptr(), q.stride(0), k.stride(0), v.stride(0),
        positions.data_ptr(), slot_mapping.data_ptr() if store else None,
        q_weight.data_ptr(), k_weight.data_ptr(), cs.data_ptr(), cs.stride(0), cs.shape[0],
        k_cache.data_ptr() if store else None, v_cache.data_ptr() if store else None,
        k_cache.numel() // (Hkv * D) if store else 0,
        T, Hq, Hkv, D, float(eps), _lib.stream_of(q))
    _lib.check(status, "qk_norm_rope_kv")
    return q_out, k_out


_DEF.impl("qk_norm_rope_kv", _qk_norm_rope_kv_impl, "CUDA")


@torch.library.register_fake("nvhip::qk_norm_rope_kv")
def _qk_norm_rope_kv_fake(q, k, v, positions, q_weight, k_weight, eps, cos_sin_cache, k_cache, v_cache,
                          slot_mapping, write_k):
    return _qk_outputs(q, k, write_k)


# ------------------------------------------------------------------ rms_norm / fused_add_rms_norm

def _rms_norm_impl(x, w, eps):
    n = x.shape[-1]
    if x.dim() == 2:
        groups, rows_per_group, group_stride, row_stride = x.shape[0], 1, x.stride(0), 0
    else:
        groups, rows_per_group, group_stride, row_stride = x.shape[0], x.shape[1], x.stride(0), x.stride(1)
    y = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    status = _lib.lib().nvhip_rms_norm_bf16(y.data_ptr(), x.data_ptr(), w.data_ptr(), groups, rows_per_group,
                                            group_stride, row_stride, n, float(eps), _lib.stream_of(x))
    _lib.check(status, "rms_norm")
    return y


_DEF.impl("rms_norm", _rms_norm_impl, "CUDA")


@torch.library.register_fake("nvhip::rms_norm")
def _rms_norm_fake(x, w, eps):
    return torch.empty(x.shape, dtype=x.dtype, device=x.device)


def _add_rms(x, residual, w, eps, res_out):
    rows, n = x.shape
    y = torch.empty((rows, n), dtype=x.dtype, device=x.device)
    status = _lib.lib().nvhip_add_rms_norm_bf16(y.data_ptr(), res_out.data_ptr(), x.data_ptr(), residual.data_ptr(),
                                                w.data_ptr(), rows, x.stride(0), residual.stride(0), n, float(eps),
                                                _lib.stream_of(x))
    _lib.check(status, "fused_add_rms_norm")
    return y


def _fused_add_rms_norm_impl(x, residual, w, eps):
    s = torch.empty(x.shape, dtype=x.dtype, device=x.device)
    return _add_rms(x, residual, w, eps, s), s


def _fused_add_rms_norm_inplace_impl(x, residual, w, eps):
    return _add_rms(x, residual, w, eps, residual)


_DEF.impl("fused_add_rms_norm", _fused_add_rms_norm_impl, "CUDA")
_DEF.impl("fused_add_rms_norm_", _fused_add_rms_norm_inplace_impl, "CUDA")


@torch.library.register_fake("nvhip::fused_add_rms_norm")
def _fused_add_rms_norm_fake(x, residual, w, eps):
    return torch.empty(x.shape, dtype=x.dtype, device=x.device), torch.empty(x.shape, dtype=x.dtype, device=x.device)


@torch.library.register_fake("nvhip::fused_add_rms_norm_")
def _fused_add_rms_norm_inplace_fake(x, residual, w, eps):
    return torch.empty(x.shape, dtype=x.dtype, device=x.device)


# ------------------------------------------------------------------ silu_and_mul

def _silu_and_mul_impl(x):
    rows, n = x.shape[0], x.shape[1] // 2
    out = torch.empty((rows, n), dtype=x.dtype, device=x.device)
    status = _lib.lib().nvhip_silu_mul_bf16(out.data_ptr(), x.data_ptr(), rows, x.stride(0), n, _lib.stream_of(x))
    _lib.check(status, "silu_and_mul")
    return out


_DEF.impl("silu_and_mul", _silu_and_mul_impl, "CUDA")


@torch.library.register_fake("nvhip::silu_and_mul")
def _silu_and_mul_fake(x):
    return torch.empty((x.shape[0], x.shape[1] // 2), dtype=x.dtype, device=x.device)


# ------------------------------------------------------------------ matmul

def _matmul_impl(a, b, input_precision):
    M, K = a.shape
    N = b.shape[1]
    c = torch.empty((M, N), dtype=a.dtype, device=a.device)
    dtype = _lib.DTYPE_BF16 if a.dtype == torch.bfloat16 else _lib.DTYPE_F32
    prec = _lib.PREC_TF32 if input_precision == "tf32" else _lib.PREC_IEEE
    status = _lib.lib().nvhip_matmul(c.data_ptr(), a.data_ptr(), b.data_ptr(), M, N, K, a.stride(0), a.stride(1),
                                     b.stride(0), b.stride(1), c.stride(0), c.stride(1), dtype, prec,
                                     _lib.stream_of(a))
    _lib.check(status, "matmul")
    return c


_DEF.impl("matmul", _matmul_impl, "CUDA")


@torch.library.register_fake("nvhip::matmul")
def _matmul_fake(a, b, input_precision):
    return torch.empty((a.shape[0], b.shape[1]), dtype=a.dtype, device=a.device)


# ------------------------------------------------------------------ paged decode attention

# The attention workspaces (decode and prefill): they start with the decode attention's per-pair counters, which
# must be zero before a call and which every call leaves zero, so one workspace is zero-filled once and kept per
# device, for both ops (a graph captured after an eager warm-up call reuses it, so the zero fill is not captured).
# Attention calls on one device must therefore not run concurrently on unordered streams. A workspace is never
# freed: a captured graph keeps using its address (a larger need adds a new one).
_ATTN_WS = {}


def _attn_workspace(device, nbytes):
    if nbytes <= 0:
        return None
    held = _ATTN_WS.setdefault(device.index, [])
    if not held or held[-1].numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            # a zero fill recorded into the graph would run only at replay, after eager calls that already used the
            # new workspace's uninitialised counters
            raise RuntimeError(
                f"nvhip attention: a {nbytes}-byte workspace is needed inside a graph capture, but the workspace "
                f"held for this device is {held[-1].numel() if held else 0} bytes; run the same call once eagerly "
                f"before capturing it")
        held.append(torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device))
    return held[-1]


def _paged_decode_attention_impl(q, k_cache, v_cache, block_table, context_lens, q_len, scale, causal):
    T, Hq, D = q.shape
    num_blocks, block_size, Hkv = k_cache.shape[0], k_cache.shape[1], k_cache.shape[2]
    num_seqs, max_blocks = context_lens.shape[0], block_table.shape[1]
    out = torch.empty((T, Hq, D), dtype=q.dtype, device=q.device)
    lib = _lib.lib()
    ws_bytes = lib.nvhip_paged_decode_attention_workspace_size(num_seqs, q_len, Hq, Hkv, D, block_size, max_blocks)
    ws = _attn_workspace(q.device, ws_bytes)
    status = lib.nvhip_paged_decode_attention_bf16(
        out.data_ptr(), q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(),
        context_lens.data_ptr(), num_seqs, q_len, Hq, Hkv, D, block_size, num_blocks, max_blocks,
        q.stride(0), q.stride(1), out.stride(0), out.stride(1), scale, int(causal),
        ws.data_ptr() if ws is not None else None, ws_bytes if ws is not None else 0, _lib.stream_of(q))
    _lib.check(status, "paged_decode_attention")
    return out


_DEF.impl("paged_decode_attention", _paged_decode_attention_impl, "CUDA")


@torch.library.register_fake("nvhip::paged_decode_attention")
def _paged_decode_attention_fake(q, k_cache, v_cache, block_table, context_lens, q_len, scale, causal):
    return torch.empty(q.shape, dtype=q.dtype, device=q.device)


# ------------------------------------------------------------------ store_kvcache

def _store_kvcache_impl(key, value, k_cache, v_cache, slot_mapping):
    n, row = key.shape[0], key.shape[1] * key.shape[2]
    num_slots = k_cache.numel() // row if row else 0
    status = _lib.lib().nvhip_store_kvcache(k_cache.data_ptr(), v_cache.data_ptr(), key.data_ptr(), value.data_ptr(),
                                            key.stride(0), value.stride(0), slot_mapping.data_ptr(), num_slots, n,
                                            row, key.element_size(), _lib.stream_of(key))
    _lib.check(status, "store_kvcache")


_DEF.impl("store_kvcache", _store_kvcache_impl, "CUDA")


@torch.library.register_fake("nvhip::store_kvcache")
def _store_kvcache_fake(key, value, k_cache, v_cache, slot_mapping):
    return None


# ------------------------------------------------------------------ GEMM + SiLU x Mul epilogue

def _matmul_silu_mul_impl(a, w):
    M, K = a.shape
    N2 = w.shape[0] // 2
    out = torch.empty((M, N2), dtype=a.dtype, device=a.device)
    status = _lib.lib().nvhip_matmul_silu_mul_bf16(out.data_ptr(), a.data_ptr(), w.data_ptr(), M, N2, K, a.stride(0),
                                                   w.stride(0), out.stride(0), _lib.stream_of(a))
    _lib.check(status, "matmul_silu_mul")
    return out


_DEF.impl("matmul_silu_mul", _matmul_silu_mul_impl, "CUDA")


@torch.library.register_fake("nvhip::matmul_silu_mul")
def _matmul_silu_mul_fake(a, w):
    return torch.empty((a.shape[0], w.shape[0] // 2), dtype=a.dtype, device=a.device)


# ------------------------------------------------------------------ RMSNorm / Add+RMSNorm fused into the next GEMM

def _rms_norm_matmul_impl(x, residual, norm_w, eps, w, silu):
    M, K = x.shape
    N = w.shape[0] // 2 if silu else w.shape[0]
    out = torch.empty((M, N), dtype=x.dtype, device=x.device)
    res_out = torch.empty_like(x, memory_format=torch.contiguous_format) if residual is not None else x.new_empty((0,))
    status = _lib.lib().nvhip_rms_norm_matmul_bf16(
        out.data_ptr(), res_out.data_ptr() if residual is not None else None, x.data_ptr(),
        residual.data_ptr() if residual is not None else None, norm_w.data_ptr(), eps, w.data_ptr(), M, N, K,
        x.stride(0), residual.stride(0) if residual is not None else 0, w.stride(0), out.stride(0),
        int(silu), _lib.stream_of(x))
    _lib.check(status, "rms_norm_matmul")
    return out, res_out


_DEF.impl("rms_norm_matmul", _rms_norm_matmul_impl, "CUDA")


@torch.library.register_fake("nvhip::rms_norm_matmul")
def _rms_norm_matmul_fake(x, residual, norm_w, eps, w, silu):
    N = w.shape[0] // 2 if silu else w.shape[0]
    out = torch.empty((x.shape[0], N), dtype=x.dtype, device=x.device)
    return out, (torch.empty_like(x) if residual is not None else x.new_empty((0,)))


# ------------------------------------------------------------------ GEMM followed by the Add+RMSNorm that consumes it

def _matmul_add_rms_norm_impl(x, w, residual, norm_w, eps):
    M, K = x.shape
    N = w.shape[0]
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    res_out = torch.empty((M, N), dtype=x.dtype, device=x.device)
    lib = _lib.lib()
    ws_bytes = lib.nvhip_matmul_add_rms_norm_workspace_size(M, N, K)
    ws = torch.empty((max(ws_bytes, 16) + 3) // 4, dtype=torch.float32, device=x.device)
    status = lib.nvhip_matmul_add_rms_norm_bf16(
        y.data_ptr(), res_out.data_ptr(), x.data_ptr(), w.data_ptr(), residual.data_ptr(), norm_w.data_ptr(), eps,
        M, N, K, x.stride(0), w.stride(0), ws.data_ptr(), ws.numel() * 4, _lib.stream_of(x))
    _lib.check(status, "matmul_add_rms_norm")
    return y, res_out


_DEF.impl("matmul_add_rms_norm", _matmul_add_rms_norm_impl, "CUDA")


@torch.library.register_fake("nvhip::matmul_add_rms_norm")
def _matmul_add_rms_norm_fake(x, w, residual, norm_w, eps):
    out = torch.empty((x.shape[0], w.shape[0]), dtype=x.dtype, device=x.device)
    return out, torch.empty_like(out)


# ------------------------------------------------------------------ fused q/k norm + RoPE + KV write + decode attention

def _qk_norm_rope_kv_decode_attention_impl(q, k, v, positions, q_w, k_w, eps, cos_sin, k_cache, v_cache,
                                           slot_mapping, cache_seqlens, block_table, scale):
    B, Hq, D = q.shape
    num_blocks, block_size, Hkv = k_cache.shape[0], k_cache.shape[1], k_cache.shape[2]
    max_blocks = block_table.shape[1]
    out = torch.empty((B, Hq, D), dtype=q.dtype, device=q.device)
    lib = _lib.lib()
    ws_bytes = lib.nvhip_paged_decode_attention_workspace_size(B, 1, Hq, Hkv, D, block_size, max_blocks)
    ws = _attn_workspace(q.device, ws_bytes)
    cs = cos_sin.reshape(cos_sin.shape[0], -1)
    status = lib.nvhip_qk_norm_rope_kv_decode_attention_bf16(
        out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), q.stride(0), k.stride(0), v.stride(0),
        positions.data_ptr(), slot_mapping.data_ptr(), q_w.data_ptr(), k_w.data_ptr(), cs.data_ptr(), cs.stride(0),
        cs.shape[0], eps, k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(), cache_seqlens.data_ptr(),
        B, Hq, Hkv, D, block_size, num_blocks, max_blocks, out.stride(0), out.stride(1), scale,
        ws.data_ptr() if ws is not None else None, ws_bytes if ws is not None else 0, _lib.stream_of(q))
    _lib.check(status, "qk_norm_rope_kv_decode_attention")
    return out


_DEF.impl("qk_norm_rope_kv_decode_attention", _qk_norm_rope_kv_decode_attention_impl, "CUDA")


@torch.library.register_fake("nvhip::qk_norm_rope_kv_decode_attention")
def _qk_norm_rope_kv_decode_attention_fake(q, k, v, positions, q_w, k_w, eps, cos_sin, k_cache, v_cache,
                                           slot_mapping, cache_seqlens, block_table, scale):
    return torch.empty(q.shape, dtype=q.dtype, device=q.device)


# ------------------------------------------------------------------ prefill (varlen) attention

def _prefill_attention_impl(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, scale, causal,
                            block_table):
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    _prefill_attention_out_impl(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, scale, causal,
                                block_table, out)
    return out


def _prefill_attention_out_impl(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, scale, causal,
                                block_table, out):
    """Writes the attention into out [Tq, Hq, D] (rows of Hq * D contiguous heads: out.stride(2) == 1)."""
    Tq, Hq, D = q.shape
    if block_table is None:
        Hkv, bt, bs, nb, mb = k.shape[1], None, 0, 0, 0
        k_st, v_st = k.stride(0), v.stride(0)
    else:
        Hkv, bt, bs, nb, mb = k.shape[2], block_table.data_ptr(), k.shape[1], k.shape[0], block_table.shape[1]
        k_st = v_st = Hkv * D
    num_seqs = cu_seqlens_q.shape[0] - 1
    lib = _lib.lib()
    ws_bytes = lib.nvhip_prefill_attention_workspace_size(num_seqs, max_seqlen_q, max_seqlen_k, Hq, Hkv, D, Tq)
    ws = _attn_workspace(q.device, ws_bytes)
    status = lib.nvhip_prefill_attention_bf16(
        out.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(),
        num_seqs, max_seqlen_q, max_seqlen_k, Tq, Hq, Hkv, D, q.stride(0), q.stride(1), k_st, v_st, out.stride(0),
        out.stride(1), bt, bs, nb, mb, scale, int(causal), ws.data_ptr() if ws is not None else None,
        ws_bytes if ws is not None else 0, _lib.stream_of(q))
    _lib.check(status, "prefill_attention")


_DEF.impl("prefill_attention", _prefill_attention_impl, "CUDA")
_DEF.impl("prefill_attention_out", _prefill_attention_out_impl, "CUDA")


@torch.library.register_fake("nvhip::prefill_attention")
def _prefill_attention_fake(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, scale, causal,
                            block_table):
    return torch.empty(q.shape, dtype=q.dtype, device=q.device)


# ------------------------------------------------------------------ greedy sampling (argmax over the vocabulary)

def _argmax_impl(logits):
    rows, n = logits.shape
    out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    ws_bytes = _lib.lib().nvhip_argmax_workspace_size(rows, n)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device=logits.device)
    status = _lib.lib().nvhip_argmax_bf16(out.data_ptr(), logits.data_ptr(), rows, n, logits.stride(0),
                                          ws.data_ptr(), ws_bytes, _lib.stream_of(logits))
    _lib.check(status, "argmax")
    return out


_DEF.impl("argmax", _argmax_impl, "CUDA")


@torch.library.register_fake("nvhip::argmax")
def _argmax_fake(logits):
    return torch.empty(logits.shape[0], dtype=torch.int64, device=logits.device)
