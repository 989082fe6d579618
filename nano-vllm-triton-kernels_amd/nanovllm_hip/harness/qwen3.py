"""Qwen3 decoder (random init) whose layers dispatch to the HIP kernels or to their own torch code.

The call sites mirror nano-vllm's: RMSNorm.forward (layers/layernorm.py:46-58), SiluAndMul.forward
(layers/activation.py:20-23), Qwen3Attention.pre_attn + Attention.forward with the fused path
(models/qwen3.py:89-105, layers/attention.py:64-92) and the decoder layer (models/qwen3.py:166-183).

backend "hip"   : rms_norm / fused_add_rms_norm_ (residual in place) / silu_and_mul / qk_norm_rope_kv from
                  nanovllm_hip.kernels (the fused kernel does q/k norm, RoPE and the KV write in one launch).
backend "torch" : the layers' own torch code run eagerly (what the reference's "compile" backend compiles), with
                  the unfused q_norm, k_norm, rotary and KV scatter.
The projections and the tied LM head use the HIP GEMM (nanovllm_hip.kernels.matmul, the wiring of linear.py:51,
:73, :153 and embed_head.py:63; gate_up with the SiLU x Mul epilogue) in the hip backend, with the norm before the
qkv and gate_up projections inside those GEMMs for decode batches (rms_norm_matmul / add_rms_norm_matmul, bitwise
the separate launches), and torch's F.linear in the torch backend; forward(..., linear="torch") makes the hip
backend use F.linear, the separate norms and the separate silu_and_mul, so that token differences come only from
the four kernels.
Both backends share the embedding and the attention. The attention is chosen apart
from the backend: "torch" = the fp32 code below (prefill and decode), "hip" = the HIP attention kernels
(nanovllm_hip.kernels.attention): flash_attn_varlen_func for prefill and mixed steps (layers/attention.py:77-83),
flash_attn_with_kvcache for decode steps (:84-90) -- or, in the hip backend, the decode step's fused q/k norm + RoPE
+ KV write + attention launch.
"""
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from nanovllm_hip import kernels as hip
from nanovllm_hip.kernels.attention import (flash_attn_varlen_func, flash_attn_with_kvcache,
                                            qk_norm_rope_kv_decode_attention)


@dataclass
class Qwen3Config:
    """Qwen3-0.6B shapes."""
    vocab_size: int = 151936
    hidden_size: int = 1024
    intermediate_size: int = 3072
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1e6
    max_position_embeddings: int = 40960
    init_std: float = 0.02


@dataclass
class Context:
    """Per-forward batch layout (the fields of nano-vllm's utils/context.py this model reads).

    Prefill without block_tables: one sequence, its own keys. Prefill with block_tables (a mixed step or a prefix
    cache, model_runner.py:489-496): varlen over the paged cache, sequence s has queries cu_seqlens_q[s] ..
    cu_seqlens_q[s+1] and keys 0 .. cu_seqlens_k[s+1] - cu_seqlens_k[s] (this step's KV is stored first)."""
    is_prefill: bool
    slot_mapping: torch.Tensor          # [T] int32, -1 = no KV write
    context_lens: torch.Tensor | None = None   # decode: [B] int32
    block_tables: torch.Tensor | None = None   # decode / varlen prefill: [B, max_blocks] int32 (padded with -1)
    cu_seqlens_q: torch.Tensor | None = None   # varlen prefill: [B + 1] int32
    cu_seqlens_k: torch.Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0


# ------------------------------------------------------------------ torch code of the layers (backend "torch")

def rms_forward(x, w, eps):
    """layers/layernorm.py:20-30 as it runs eagerly."""
    orig = x.dtype
    x = x.float()
    var = x.pow(2).mean(dim=-1, keepdim=True)
    x = x * torch.rsqrt(var + eps)
    return x.to(orig).mul_(w)


def add_rms_forward(x, residual, w, eps):
    """layers/layernorm.py:32-44: normalises the unrounded fp32 sum, returns (y, bf16 sum)."""
    orig = x.dtype
    s = x.float() + residual.float()
    residual = s.to(orig)
    var = s.pow(2).mean(dim=-1, keepdim=True)
    s = s * torch.rsqrt(var + eps)
    return s.to(orig).mul_(w), residual


def rope_table(head_dim, max_pos, base):
    """layers/rotary_embedding.py:19-35: [max_pos, 1, head_dim] fp32 (cos | sin)."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
    t = torch.arange(max_pos, dtype=torch.float)
    freqs = t[:, None] * inv_freq[None, :]
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1).unsqueeze_(1)


def apply_rope(x, cos, sin):
    """layers/rotary_embedding.py:6-14."""
    x1, x2 = torch.chunk(x.float(), 2, dim=-1)
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1).to(x.dtype)


def store_kvcache(k, v, k_cache, v_cache, slot_mapping):
    """layers/attention.py:11-41: token t's [Hkv, D] rows go to slot slot_mapping[t] of the caches. The harness never
    pads its batches (no slot -1), so this is a plain scatter and can be recorded into a graph."""
    hkv, d = k.shape[1], k.shape[2]
    idx = slot_mapping.long()
    k_cache.view(-1, hkv, d)[idx] = k
    v_cache.view(-1, hkv, d)[idx] = v


# ------------------------------------------------------------------ attention shared by both backends

def prefill_attention(q, k, v, scale):
    """Causal attention of one sequence (no prefix cache) in fp32: q [L, Hq, D], k, v [L, Hkv, D] -> [L, Hq, D]."""
    L, hq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    qf = q.float().view(L, hkv, g, d).permute(1, 2, 0, 3).contiguous()      # [Hkv, G, L, D]
    kt = k.float().permute(1, 2, 0).contiguous().unsqueeze(1)              # [Hkv, 1, D, L]
    vf = v.float().permute(1, 0, 2).contiguous().unsqueeze(1)              # [Hkv, 1, L, D]
    s = torch.matmul(qf, kt) * scale                                       # [Hkv, G, L, L]
    causal = torch.ones(L, L, dtype=torch.bool, device=q.device).tril_()
    s.masked_fill_(~causal, float("-inf"))
    o = torch.matmul(torch.softmax(s, dim=-1), vf)                         # [Hkv, G, L, D]
    return o.permute(2, 0, 1, 3).reshape(L, hq, d).to(q.dtype)


def paged_decode_attention(q, k_cache, v_cache, block_tables, context_lens, scale):
    """One query token per sequence against its paged cache, fp32, static shapes (graph-capturable):
    q [B, Hq, D]; caches [blocks, block_size, Hkv, D]; block_tables [B, max_blocks]; context_lens [B]."""
    B, hq, d = q.shape
    bs, hkv = k_cache.shape[1], k_cache.shape[2]
    g = hq // hkv
    L = block_tables.shape[1] * bs
    kk = k_cache[block_tables.long()].view(B, L, hkv, d)                   # gather by block table
    vv = v_cache[block_tables.long()].view(B, L, hkv, d)
    kt = kk.float().permute(0, 2, 3, 1).contiguous()                       # [B, Hkv, D, L]
    vf = vv.float().permute(0, 2, 1, 3).contiguous()                       # [B, Hkv, L, D]
    qf = q.float().view(B, hkv, g, d)                                      # [B, Hkv, G, D]
    s = torch.matmul(qf, kt) * scale                                       # [B, Hkv, G, L]
    valid = torch.arange(L, device=q.device)[None, :] < context_lens[:, None]
    s.masked_fill_(~valid[:, None, None, :], float("-inf"))
    o = torch.matmul(torch.softmax(s, dim=-1), vf)                         # [B, Hkv, G, D]
    return o.reshape(B, hq, d).to(q.dtype)


def varlen_paged_attention(q, k_cache, v_cache, block_tables, cu_seqlens_q, cu_seqlens_k, scale):
    """Varlen causal attention over the paged cache in fp32 (the flash_attn_varlen_func call with block_table of
    layers/attention.py:77-83): sequence s's queries are the last lq of its lk cached tokens, query i sees keys
    0 .. lk - lq + i. Eager only (the loop reads the sequence bounds on the host)."""
    hq, d = q.shape[1], q.shape[2]
    bs, hkv = k_cache.shape[1], k_cache.shape[2]
    g = hq // hkv
    cq, ck = cu_seqlens_q.tolist(), cu_seqlens_k.tolist()
    out = torch.empty_like(q)
    for s in range(len(cq) - 1):
        lq, lk = cq[s + 1] - cq[s], ck[s + 1] - ck[s]
        nb = (lk + bs - 1) // bs
        blocks = block_tables[s, :nb].long()
        kk = k_cache[blocks].reshape(nb * bs, hkv, d)[:lk].float()          # [lk, Hkv, D]
        vv = v_cache[blocks].reshape(nb * bs, hkv, d)[:lk].float()
        qf = q[cq[s]:cq[s + 1]].float().view(lq, hkv, g, d).permute(1, 2, 0, 3).contiguous()  # [Hkv, G, lq, D]
        kt = kk.permute(1, 2, 0).contiguous().unsqueeze(1)                  # [Hkv, 1, D, lk]
        vf = vv.permute(1, 0, 2).contiguous().unsqueeze(1)                  # [Hkv, 1, lk, D]
        sc = torch.matmul(qf, kt) * scale                                   # [Hkv, G, lq, lk]
        allowed = torch.arange(lk, device=q.device)[None, :] <= (lk - lq + torch.arange(lq, device=q.device))[:, None]
        sc.masked_fill_(~allowed, float("-inf"))
        o = torch.matmul(torch.softmax(sc, dim=-1), vf)                     # [Hkv, G, lq, D]
        out[cq[s]:cq[s + 1]] = o.permute(2, 0, 1, 3).reshape(lq, hq, d).to(q.dtype)
    return out


def hip_linear(x, w):
    """nn.Linear without bias through the HIP GEMM: x [T, in] @ w[out, in]^T (B = w.t(), the K-contiguous layout)."""
    return hip.matmul(x, w.t())


@dataclass
class Deferred:
    """The projection x @ weight^T, not computed yet: post_attn hands its down projection to the Add+RMSNorm that
    consumes it (the next layer's input norm or the final norm), which runs both in one call
    (hip.matmul_add_rms_norm)."""
    x: torch.Tensor
    weight: torch.Tensor


# ------------------------------------------------------------------ the model

class Qwen3:
    """Random-init Qwen3 weights (bf16) and the forward pass with backend dispatch. Tied embeddings.

    The kernel backend is latched when the model is built, as the reference's layers read nanovllm.kernels.backend
    in __init__ (layers/layernorm.py:18, layers/activation.py:13, models/qwen3.py:73): from nanovllm_hip.kernels
    .backend ("hip" -> this package's kernels, "compile" -> the layers' torch code, here "torch") unless
    kernel_backend names one. forward() runs the latched backend; its `backend` argument overrides it per call
    (the decode harness runs both backends on one set of weights)."""

    def __init__(self, cfg: Qwen3Config, device, seed=0, kernel_backend=None):
        self.cfg = cfg
        latched = hip.backend if kernel_backend is None else kernel_backend
        if latched not in hip.BACKENDS + ("torch",):
            raise ValueError(f"kernel backend {latched!r}: expected one of {hip.BACKENDS}")
        self.kernel_backend = "torch" if latched == "compile" else latched
        g = torch.Generator(device="cpu").manual_seed(seed)
        std = cfg.init_std
        H, D, hq, hkv, I = cfg.hidden_size, cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads, \
            cfg.intermediate_size

        def randn(*shape, scale=std):
            return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16).to(device)

        def norm_w(n):
            return (1 + 0.1 * torch.randn(n, generator=g)).to(torch.bfloat16).to(device)

        self.embed = randn(cfg.vocab_size, H)
        self.layers = []
        for _ in range(cfg.num_hidden_layers):
            self.layers.append(dict(
                input_norm=norm_w(H), post_norm=norm_w(H), q_norm=norm_w(D), k_norm=norm_w(D),
                qkv=randn((hq + 2 * hkv) * D, H), o=randn(H, hq * D),
                gate_up=randn(2 * I, H), down=randn(H, I)))
        self.final_norm_w = norm_w(H)
        self.cos_sin = rope_table(D, cfg.max_position_embeddings, cfg.rope_theta).to(device)
        self.kv = None  # [(k_cache, v_cache)] per layer
        self.scale = D ** -0.5

    def allocate_kv_cache(self, num_blocks, block_size=256):
        c = self.cfg
        shape = (2, c.num_hidden_layers, num_blocks, block_size, c.num_key_value_heads, c.head_dim)
        cache = torch.zeros(shape, dtype=torch.bfloat16, device=self.embed.device)
        self.kv = [(cache[0, i], cache[1, i]) for i in range(c.num_hidden_layers)]
        return cache

    def pre_attn(self, li, positions, h, residual, backend, linear="hip"):
        """Layer li up to its attention (models/qwen3.py:185-197 with Qwen3Attention.pre_attn :89-105): the input
        norm and the qkv projection, plus the q/k norms and RoPE in the torch backend. Returns (q, k, v, residual):
        strided [T, heads, D] views of the projection output. In the hip backend q and k are not normed or rotated
        yet -- the fused kernel in attn() does that together with the KV write, as the reference's fused_norm_rope
        path does. Reads nothing of the batch layout (Context), so a piecewise graph can record it."""
        c, L = self.cfg, self.layers[li]
        eps, hq, hkv, D = c.rms_norm_eps, c.num_attention_heads, c.num_key_value_heads, c.head_dim
        # hip backend with the HIP GEMM: the norm runs inside the projection that follows it (one launch, bitwise
        # the norm then the GEMM) for decode batches, and as the two launches for longer inputs
        if backend == "hip" and linear == "hip":
            if residual is None:
                residual = h
                qkv = hip.rms_norm_matmul(h, L["input_norm"], eps, L["qkv"])
            elif isinstance(h, Deferred):  # the previous layer's down projection, then this norm, then qkv
                h, residual = hip.matmul_add_rms_norm(h.x, h.weight, residual, L["input_norm"], eps)
                qkv = hip_linear(h, L["qkv"])
            else:
                qkv, residual = hip.add_rms_norm_matmul(h, residual, L["input_norm"], eps, L["qkv"])
        else:
            if residual is None:
                residual = h
                h = hip.rms_norm(h, L["input_norm"], eps) if backend == "hip" else \
                    rms_forward(h, L["input_norm"], eps)
            elif backend == "hip":
                h, residual = hip.fused_add_rms_norm_(h, residual, L["input_norm"], eps)
            else:
                h, residual = add_rms_forward(h, residual, L["input_norm"], eps)
            qkv = F.linear(h, L["qkv"])
        q, k, v = qkv.split([hq * D, hkv * D, hkv * D], dim=-1)
        q, k, v = q.view(-1, hq, D), k.view(-1, hkv, D), v.view(-1, hkv, D)
        if backend != "hip":
            q = rms_forward(q, L["q_norm"], eps)
            k = rms_forward(k, L["k_norm"], eps)
            cos, sin = self.cos_sin[positions].chunk(2, dim=-1)
            q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
        return q, k, v, residual

    def attn(self, li, q, k, v, positions, ctx: Context, backend, attention="torch", out=None):
        """Attention.forward of layer li (layers/attention.py:64-92): the KV write (hip: the fused q/k norm + RoPE
        + KV-write kernel) and the attention over the batch layout in ctx -> o [T, Hq, D], written into out when
        given (the varlen hip attention writes it there directly; the other paths copy)."""
        o = self._attn(li, q, k, v, positions, ctx, backend, attention, out)
        if out is not None and o.data_ptr() != out.data_ptr():
            out.copy_(o)
            return out
        return o

    def _attn(self, li, q, k, v, positions, ctx: Context, backend, attention, out):
        c, L = self.cfg, self.layers[li]
        hq, D = c.num_attention_heads, c.head_dim
        k_cache, v_cache = self.kv[li]
        varlen = ctx.is_prefill and ctx.block_tables is not None
        if backend == "hip" and attention == "hip" and not ctx.is_prefill and q.shape[0] == ctx.context_lens.shape[0]:
            # one decode token per sequence: the q/k norm + RoPE + KV write and the attention in one launch
            return qk_norm_rope_kv_decode_attention(q, k, v, positions, L["q_norm"], L["k_norm"], c.rms_norm_eps,
                                                    self.cos_sin, k_cache, v_cache, ctx.slot_mapping,
                                                    ctx.context_lens, ctx.block_tables, self.scale)
        if backend == "hip":
            write_k = ctx.is_prefill and not varlen     # only a prefill without the cache reads k from here
            q, k_out = hip.qk_norm_rope_kv(q, k, v, positions, L["q_norm"], L["k_norm"], c.rms_norm_eps,
                                           self.cos_sin, k_cache, v_cache, ctx.slot_mapping, write_k)
            if write_k:
                k = k_out
        else:
            store_kvcache(k, v, k_cache, v_cache, ctx.slot_mapping)
        if varlen and attention == "hip":
            return flash_attn_varlen_func(q, k_cache, v_cache, ctx.max_seqlen_q, ctx.cu_seqlens_q, ctx.max_seqlen_k,
                                          ctx.cu_seqlens_k, self.scale, causal=True, block_table=ctx.block_tables,
                                          out=out)
        if varlen:
            return varlen_paged_attention(q, k_cache, v_cache, ctx.block_tables, ctx.cu_seqlens_q, ctx.cu_seqlens_k,
                                          self.scale)
        if ctx.is_prefill and attention == "hip":
            T = q.shape[0]
            cu = torch.tensor([0, T], dtype=torch.int32, device=q.device)
            return flash_attn_varlen_func(q, k, v, T, cu, T, cu, self.scale, causal=True)
        if ctx.is_prefill:
            return prefill_attention(q, k, v, self.scale)
        if attention == "hip":
            B = ctx.context_lens.shape[0]
            return flash_attn_with_kvcache(q.view(B, -1, hq, D), k_cache, v_cache, ctx.context_lens,
                                           ctx.block_tables, self.scale, causal=True).view(-1, hq, D)
        return paged_decode_attention(q, k_cache, v_cache, ctx.block_tables, ctx.context_lens, self.scale)

    def post_attn(self, li, o, residual, backend, linear="hip"):
        """Layer li after its attention (models/qwen3.py:199-209): o_proj, the post-attention norm and the MLP.
        Returns (h, residual); like pre_attn it reads nothing of the batch layout. With the hip backend and GEMM
        and more than 32 tokens, o_proj runs with the norm that consumes it and h is the down projection Deferred
        to the next norm (pre_attn / final_norm), which runs with it."""
        c, L = self.cfg, self.layers[li]
        eps, hq, D = c.rms_norm_eps, c.num_attention_heads, c.head_dim
        lin = hip_linear if backend == "hip" and linear == "hip" else F.linear
        o2 = o.reshape(o.shape[0], hq * D)
        if backend == "hip" and linear == "hip" and o2.shape[0] > 32:
            h, residual = hip.matmul_add_rms_norm(o2, L["o"], residual, L["post_norm"], eps)
            return Deferred(hip.matmul_silu_and_mul(h, L["gate_up"]), L["down"]), residual
        h = lin(o2, L["o"])
        if backend == "hip" and linear == "hip":   # norm, gate_up and SiLU x Mul in one launch for decode batches
            h, residual = hip.add_rms_norm_matmul(h, residual, L["post_norm"], eps, L["gate_up"], silu=True)
        elif backend == "hip":
            h, residual = hip.fused_add_rms_norm_(h, residual, L["post_norm"], eps)
            h = hip.silu_and_mul(lin(h, L["gate_up"]))
        else:
            h, residual = add_rms_forward(h, residual, L["post_norm"], eps)
            gate, up = F.linear(h, L["gate_up"]).chunk(2, -1)
            h = F.silu(gate) * up
        return lin(h, L["down"]), residual

    def final_norm(self, h, residual, backend):
        """The model's last Add+RMSNorm (models/qwen3.py:232) -> hidden states [T, hidden]."""
        if isinstance(h, Deferred):
            return hip.matmul_add_rms_norm(h.x, h.weight, residual, self.final_norm_w, self.cfg.rms_norm_eps)[0]
        if backend == "hip":
            return hip.fused_add_rms_norm_(h, residual, self.final_norm_w, self.cfg.rms_norm_eps)[0]
        return add_rms_forward(h, residual, self.final_norm_w, self.cfg.rms_norm_eps)[0]

    def forward(self, input_ids, positions, ctx: Context, backend: str | None = None, attention: str = "torch",
                linear: str = "hip"):
        """Returns the final hidden states [T, hidden] (after the last norm). backend None: the latched one."""
        backend = self.kernel_backend if backend is None else backend
        h, residual = F.embedding(input_ids, self.embed), None
        for li in range(len(self.layers)):
            q, k, v, residual = self.pre_attn(li, positions, h, residual, backend, linear)
            o = self.attn(li, q, k, v, positions, ctx, backend, attention)
            h, residual = self.post_attn(li, o, residual, backend, linear)
        return self.final_norm(h, residual, backend)

    def logits(self, h, fp32=False, backend="torch", linear="hip", as_float=True):
        """Tied LM head (embed_head.py:56-68): bf16 like the reference (then fp32 for sampling, sampler.py:9; with
        as_float=False the bf16 logits themselves), or with fp32=True the same product in fp32, which removes the
        exact ties of bf16-rounded logits. The hip backend's bf16 head is the HIP GEMM (unless linear="torch")."""
        if fp32:
            return F.linear(h.float(), self.embed.float())
        out = hip_linear(h, self.embed) if backend == "hip" and linear == "hip" else F.linear(h, self.embed)
        return out.float() if as_float else out


def num_params(cfg: Qwen3Config) -> int:
    H, D, hq, hkv, I = cfg.hidden_size, cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads, \
        cfg.intermediate_size
    per_layer = (hq + 2 * hkv) * D * H + H * hq * D + 2 * I * H + H * I + 2 * H + 2 * D
    return cfg.vocab_size * H + cfg.num_hidden_layers * per_layer + H


__all__ = ["Qwen3Config", "Context", "Qwen3", "num_params", "varlen_paged_attention"]
