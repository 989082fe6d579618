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
from the backend: "torch" = the fp32 code below (prefill and decode), "hip" = the HIP paged decode attention
(nanovllm_hip.kernels.attention, the flash_attn_with_kvcache call of layers/attention.py:84-90) for decode steps,
the fp32 code for prefill.
"""
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from nanovllm_hip import kernels as hip
from nanovllm_hip.kernels.attention import flash_attn_varlen_func, flash_attn_with_kvcache


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
    """Per-forward batch layout (the fields of nano-vllm's utils/context.py this model reads)."""
    is_prefill: bool
    slot_mapping: torch.Tensor          # [T] int32, -1 = no KV write
    context_lens: torch.Tensor | None = None   # decode: [B] int32
    block_tables: torch.Tensor | None = None   # decode: [B, max_blocks] int32 (padded with 0)


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


def hip_linear(x, w):
    """nn.Linear without bias through the HIP GEMM: x [T, in] @ w[out, in]^T (B = w.t(), the K-contiguous layout)."""
    return hip.matmul(x, w.t())


# ------------------------------------------------------------------ the model

class Qwen3:
    """Random-init Qwen3 weights (bf16) and the forward pass with backend dispatch. Tied embeddings."""

    def __init__(self, cfg: Qwen3Config, device, seed=0):
        self.cfg = cfg
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
        self.final_norm = norm_w(H)
        self.cos_sin = rope_table(D, cfg.max_position_embeddings, cfg.rope_theta).to(device)
        self.kv = None  # [(k_cache, v_cache)] per layer
        self.scale = D ** -0.5

    def allocate_kv_cache(self, num_blocks, block_size=256):
        c = self.cfg
        shape = (2, c.num_hidden_layers, num_blocks, block_size, c.num_key_value_heads, c.head_dim)
        cache = torch.zeros(shape, dtype=torch.bfloat16, device=self.embed.device)
        self.kv = [(cache[0, i], cache[1, i]) for i in range(c.num_hidden_layers)]
        return cache

    def forward(self, input_ids, positions, ctx: Context, backend: str, attention: str = "torch",
                linear: str = "hip"):
        """Returns the final hidden states [T, hidden] (after the last norm)."""
        c = self.cfg
        lin = hip_linear if backend == "hip" and linear == "hip" else F.linear
        eps = c.rms_norm_eps
        hq, hkv, D = c.num_attention_heads, c.num_key_value_heads, c.head_dim
        h = F.embedding(input_ids, self.embed)
        residual = None
        # hip backend with the HIP GEMM: each norm runs inside the projection that follows it (one launch; bitwise
        # the norm then the GEMM) for decode batches, and as the two launches for longer inputs
        fuse = backend == "hip" and linear == "hip"
        for li, L in enumerate(self.layers):
            k_cache, v_cache = self.kv[li]
            # input_layernorm + qkv projection; q/k/v are strided views of the projection output
            if fuse:
                if residual is None:
                    residual = h
                    qkv = hip.rms_norm_matmul(h, L["input_norm"], eps, L["qkv"])
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
                qkv = lin(h, L["qkv"])
            q, k, v = qkv.split([hq * D, hkv * D, hkv * D], dim=-1)
            q, k, v = q.view(-1, hq, D), k.view(-1, hkv, D), v.view(-1, hkv, D)
            if backend == "hip":
                q, k_out = hip.qk_norm_rope_kv(q, k, v, positions, L["q_norm"], L["k_norm"], eps, self.cos_sin,
                                               k_cache, v_cache, ctx.slot_mapping, ctx.is_prefill)
                if ctx.is_prefill:
                    k = k_out
            else:
                q = rms_forward(q, L["q_norm"], eps)
                k = rms_forward(k, L["k_norm"], eps)
                cos, sin = self.cos_sin[positions].chunk(2, dim=-1)
                q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
                store_kvcache(k, v, k_cache, v_cache, ctx.slot_mapping)
            if ctx.is_prefill and attention == "hip":
                T = q.shape[0]
                cu = torch.tensor([0, T], dtype=torch.int32, device=q.device)
                o = flash_attn_varlen_func(q, k, v, T, cu, T, cu, self.scale, causal=True)
            elif ctx.is_prefill:
                o = prefill_attention(q, k, v, self.scale)
            elif attention == "hip":
                B = ctx.context_lens.shape[0]
                o = flash_attn_with_kvcache(q.view(B, -1, hq, D), k_cache, v_cache, ctx.context_lens,
                                            ctx.block_tables, self.scale, causal=True).view(-1, hq, D)
            else:
                o = paged_decode_attention(q, k_cache, v_cache, ctx.block_tables, ctx.context_lens, self.scale)
            h = lin(o.reshape(o.shape[0], hq * D), L["o"])
            # post_attention_layernorm + MLP
            if fuse:   # norm, gate_up projection and SiLU x Mul in one launch (bitwise the three-step result)
                h, residual = hip.add_rms_norm_matmul(h, residual, L["post_norm"], eps, L["gate_up"], silu=True)
            elif backend == "hip":
                h, residual = hip.fused_add_rms_norm_(h, residual, L["post_norm"], eps)
                h = hip.silu_and_mul(lin(h, L["gate_up"]))
            else:
                h, residual = add_rms_forward(h, residual, L["post_norm"], eps)
                gate, up = F.linear(h, L["gate_up"]).chunk(2, -1)
                h = F.silu(gate) * up
            h = lin(h, L["down"])
        if backend == "hip":
            h, _ = hip.fused_add_rms_norm_(h, residual, self.final_norm, eps)
        else:
            h, _ = add_rms_forward(h, residual, self.final_norm, eps)
        return h

    def logits(self, h, fp32=False, backend="torch", linear="hip"):
        """Tied LM head (embed_head.py:56-68): bf16 like the reference (then fp32 for sampling), or with fp32=True
        the same product in fp32, which removes the exact ties of bf16-rounded logits. The hip backend's bf16 head
        is the HIP GEMM (unless linear="torch")."""
        if fp32:
            return F.linear(h.float(), self.embed.float())
        if backend == "hip" and linear == "hip":
            return hip_linear(h, self.embed).float()
        return F.linear(h, self.embed).float()


def num_params(cfg: Qwen3Config) -> int:
    H, D, hq, hkv, I = cfg.hidden_size, cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads, \
        cfg.intermediate_size
    per_layer = (hq + 2 * hkv) * D * H + H * hq * D + 2 * I * H + H * I + 2 * H + 2 * D
    return cfg.vocab_size * H + cfg.num_hidden_layers * per_layer + H


__all__ = ["Qwen3Config", "Context", "Qwen3", "num_params"]
