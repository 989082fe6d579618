"""Mixed prefill + decode steps with piecewise HIP graphs, on the harness's Qwen3 model.

nano-vllm runs a step that mixes decode requests and prefill chunks as one varlen batch over the paged cache
(model_runner.py:32-64 `mixed_batch`, :489-496 `prepare_mixed`). Its piecewise mode (:543-591 `run_segment` /
`run_piecewise`, buckets :139-149, recording :680-689) records everything between two attentions as a graph per
(token bucket, segment) and runs only the attentions eagerly, on the real tokens. The segments never read the batch
layout, so one recording serves every mixed step padded to the bucket.

Here the segments are the model's pre_attn / post_attn (qwen3.py in this package) with the hip backend's kernels:
norms, GEMMs (SiLU x Mul in the gate_up epilogue) and, for the hip backend, q/k/v left un-normed so that the
attention step runs the fused q/k norm + RoPE + KV-write kernel followed by the varlen paged attention. Instead of
copying q / k / v / residual into fixed buffers after every segment (what the reference does), each segment's
outputs stay in the graph's own memory: segment i + 1 was recorded reading segment i's outputs, so a replay
chain passes them along in place, and the eager attention reads them as views.
"""
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from nanovllm_hip.harness.qwen3 import Context, Qwen3


@dataclass
class Request:
    """One request of a mixed step: all its tokens so far, its cache blocks and how many tokens are cached.
    num_scheduled > 0: a prefill chunk (tokens num_cached .. num_cached + num_scheduled); 0: a decode request,
    whose query is its last token (position len(tokens) - 1, not cached yet)."""
    tokens: list
    block_table: list
    num_cached: int
    num_scheduled: int = 0

    @property
    def is_prefill(self):
        return self.num_scheduled > 0


def mixed_batch(reqs, block_size):
    """The flat batch of a mixed step as Python lists (model_runner.py:32-64 with no draft tokens): per request its
    query tokens, their positions and slots; cu_seqlens_k counts each request's whole length up to its last query;
    logits_indices = the decode rows and the last row of a prefill chunk that ends its prompt."""
    input_ids, positions, slots, logits_indices = [], [], [], []
    cu_q, cu_k = [0], [0]
    for r in reqs:
        if r.is_prefill:
            start, end = r.num_cached, r.num_cached + r.num_scheduled
        else:
            start, end = len(r.tokens) - 1, len(r.tokens)
        input_ids.extend(r.tokens[start:end])
        positions.extend(range(start, end))
        slots.extend(r.block_table[p // block_size] * block_size + p % block_size for p in range(start, end))
        q0 = cu_q[-1]
        cu_q.append(q0 + end - start)
        cu_k.append(cu_k[-1] + end)
        if not r.is_prefill:
            logits_indices.append(q0)
        elif end == len(r.tokens):
            logits_indices.append(cu_q[-1] - 1)
    return dict(input_ids=input_ids, positions=positions, slot_mapping=slots, logits_indices=logits_indices,
                cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
                max_seqlen_q=max(b - a for a, b in zip(cu_q, cu_q[1:])),
                max_seqlen_k=max(b - a for a, b in zip(cu_k, cu_k[1:])))


def prepare_mixed(reqs, block_size, device):
    """(input_ids, positions, Context, logits_indices) on `device` for a mixed step (model_runner.py:489-496)."""
    b = mixed_batch(reqs, block_size)
    max_blocks = max(len(r.block_table) for r in reqs)
    tables = torch.tensor([r.block_table + [-1] * (max_blocks - len(r.block_table)) for r in reqs],
                          dtype=torch.int32, device=device)

    def dev(x, dtype):
        return torch.tensor(x, dtype=dtype, device=device)

    ctx = Context(True, dev(b["slot_mapping"], torch.int32), block_tables=tables,
                  cu_seqlens_q=dev(b["cu_seqlens_q"], torch.int32), cu_seqlens_k=dev(b["cu_seqlens_k"], torch.int32),
                  max_seqlen_q=b["max_seqlen_q"], max_seqlen_k=b["max_seqlen_k"])
    return dev(b["input_ids"], torch.int64), dev(b["positions"], torch.int64), ctx, \
        dev(b["logits_indices"], torch.int64)


def mixed_buckets(max_num_batched_tokens=512):
    """Token counts mixed steps are padded to: every 64 up to min(max_num_batched_tokens, 512)
    (model_runner.py:139-149)."""
    most = min(max_num_batched_tokens, 512)
    return list(range(64, most, 64)) + [most]


class Piecewise:
    """Runs mixed steps of `model` segment by segment (model_runner.py:543-591): segment 0 = embedding + layer 0 up
    to its attention, segment i = the rest of layer i - 1 + layer i up to its attention, segment L = the rest of
    the last layer + the final norm. After record() the segments of each bucket are replayed from their graphs;
    before, the same code runs eagerly on the same padded shapes (the reference's enforce_eager)."""

    def __init__(self, model: Qwen3, buckets, backend="hip", linear="hip", attention="hip"):
        c = model.cfg
        self.model, self.buckets = model, list(buckets)
        self.backend, self.linear, self.attention = backend, linear, attention
        n, dev = self.buckets[-1], model.embed.device
        self.input_ids = torch.zeros(n, dtype=torch.int64, device=dev)
        self.positions = torch.zeros(n, dtype=torch.int64, device=dev)
        self.o = torch.zeros(n, c.num_attention_heads, c.head_dim, dtype=torch.bfloat16, device=dev)
        self.outs = {}      # (bucket, i) -> outputs of segment i: (q, k, v, residual), or (hidden,) for the last
        self.graphs = {}    # (bucket, i) -> torch.cuda.CUDAGraph
        self.pool = None

    @property
    def num_segments(self):
        return len(self.model.layers) + 1

    def segment(self, i, n):
        """Segment i for n (padded) tokens; reads input_ids / positions / o and segment i - 1's outputs."""
        m, L = self.model, len(self.model.layers)
        if i == 0:
            h, residual = F.embedding(self.input_ids[:n], m.embed), None
        else:
            h, residual = m.post_attn(i - 1, self.o[:n], self.outs[(n, i - 1)][3], self.backend, self.linear)
        if i == L:
            self.outs[(n, i)] = (m.final_norm(h, residual, self.backend),)
        else:
            self.outs[(n, i)] = m.pre_attn(i, self.positions[:n], h, residual, self.backend, self.linear)

    @torch.inference_mode()
    def record(self):
        """Records every segment of every bucket as a graph, largest bucket first, in one memory pool. Each segment
        runs eagerly once before its recording (warm-up), so the recording reads the previous segment's recorded
        outputs."""
        for n in reversed(self.buckets):
            for i in range(self.num_segments):
                self.segment(i, n)
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, pool=self.pool):
                    self.segment(i, n)
                if self.pool is None:
                    self.pool = g.pool()
                self.graphs[(n, i)] = g
        torch.cuda.synchronize()

    @torch.inference_mode()
    def run(self, input_ids, positions, ctx: Context):
        """Hidden states [n, hidden] of a mixed step of n tokens (a view of a buffer the next step overwrites).
        Padded rows (token 0 at position 0) never reach the attention: it gets the first n rows, writes no KV for
        the rest, and their attention output is zero."""
        n = input_ids.shape[0]
        if n > self.buckets[-1]:  # the reference runs such a step eagerly, unpadded (model_runner.py:516-519)
            raise ValueError(f"{n} tokens exceed the largest bucket ({self.buckets[-1]}): run model.forward")
        bucket = next(b for b in self.buckets if b >= n)
        self.input_ids[:n] = input_ids
        self.input_ids[n:bucket] = 0
        self.positions[:n] = positions
        self.positions[n:bucket] = 0
        self.o[n:bucket] = 0
        for i in range(self.num_segments):
            if i:
                q, k, v, _ = self.outs[(bucket, i - 1)]
                self.model.attn(i - 1, q[:n], k[:n], v[:n], self.positions[:n], ctx, self.backend, self.attention,
                                out=self.o[:n])
            if self.graphs:
                self.graphs[(bucket, i)].replay()
            else:
                self.segment(i, bucket)
        return self.outs[(bucket, self.num_segments - 1)][0][:n]


__all__ = ["Request", "mixed_batch", "prepare_mixed", "mixed_buckets", "Piecewise"]
