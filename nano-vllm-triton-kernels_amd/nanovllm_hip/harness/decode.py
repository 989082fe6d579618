"""Fixed-batch greedy decode of a random-init Qwen3 model with the "hip" and "torch" backends.

Like nano-vllm's scripts/bench_decode.py: B requests with random prompts are prefilled (one sequence at a time,
eagerly), then every request gets one token per decode step. The decode step (model forward for the B last tokens,
tied LM head, greedy argmax -- in the hip backend the HIP argmax over the bf16 logits, in the torch backend
logits.float().argmax(-1), sampler.py:9-10) runs eagerly and as a recorded HIP graph whose static inputs are
refreshed before each replay (model_runner.py:372-392, :647-698). Paged KV with 256-slot blocks; each request owns ceil((len + steps + 1) / 256)
distinct random blocks.

Reported: the generated tokens of each backend and mode, token agreement (hip vs torch eager, hip graph vs hip
eager), for each request that diverges the first divergent step and the torch backend's logit gap between the two
candidates there (a near-tie flipped by a last-bit difference has a tiny gap), the graph replay time per decode step
and the number of kernel nodes in each decode graph.

The attention (shared by both backends) is the HIP prefill and paged decode attention by default (--attention
torch: the harness's fp32 torch code). The hip backend's projections and LM head use the HIP GEMM by
default (--linear torch: torch's F.linear, as in the torch backend).

Usage: python -m nanovllm_hip.harness.decode [--batch 32] [--steps 32] [--layers 28] [--min-len 512]
                                             [--max-len 2048] [--seed 0] [--reps 20] [--fp32-logits]
                                             [--attention hip|torch] [--linear hip|torch]
"""
import argparse
import ctypes
import json
import time

import torch

from nanovllm_hip.harness.qwen3 import Context, Qwen3, Qwen3Config
from nanovllm_hip.kernels.sampler import greedy_sample

BLOCK = 256


class Batch:
    def __init__(self, cfg, batch, steps, min_len, max_len, seed, device):
        g = torch.Generator("cpu").manual_seed(seed + 1)
        self.lens = torch.randint(min_len, max_len + 1, (batch,), generator=g).tolist()
        self.prompts = [torch.randint(0, cfg.vocab_size, (n,), generator=g) for n in self.lens]
        need = [(n + steps + 1 + BLOCK - 1) // BLOCK for n in self.lens]
        self.num_blocks = sum(need)
        perm = torch.randperm(self.num_blocks, generator=g).tolist()
        self.tables, used = [], 0
        for nb in need:
            self.tables.append(perm[used:used + nb])
            used += nb
        self.max_blocks = max(need)
        padded = [t + [-1] * (self.max_blocks - len(t)) for t in self.tables]  # -1 padding (model_runner.py:273)
        self.block_tables = torch.tensor(padded, dtype=torch.int32, device=device)
        self.device = device

    def slots(self, i, positions):
        t = self.tables[i]
        return torch.tensor([t[p // BLOCK] * BLOCK + p % BLOCK for p in positions], dtype=torch.int32)


@torch.inference_mode()
def prefill(model, batch, backend, fp32_logits=False, reference=None, linear="hip", attention="hip"):
    """Prefills every request; returns its first generated token (greedy) and, where it differs from
    reference[i], this backend's logit gap between its token and the reference's."""
    first, gaps = [], {}
    for i, prompt in enumerate(batch.prompts):
        n = len(prompt)
        ctx = Context(True, batch.slots(i, range(n)).to(batch.device))
        h = model.forward(prompt.to(batch.device), torch.arange(n, device=batch.device), ctx, backend, attention,
                          linear)
        logits = model.logits(h[-1:], fp32_logits, backend, linear)[0]
        tok = int(logits.argmax())
        if reference is not None and reference[i] != tok:
            gaps[i] = {"step": "prefill", "logit_gap": round(float(logits[tok] - logits[reference[i]]), 5)}
        first.append(tok)
    return first, gaps


class DecodeStep:
    """Static input buffers of one decode step and the step itself (eager or replayed from a graph)."""

    def __init__(self, model, batch, backend, fp32_logits=False, attention="hip", linear="hip"):
        self.model, self.batch, self.backend, self.fp32_logits = model, batch, backend, fp32_logits
        self.attention, self.linear = attention, linear
        B, dev = len(batch.lens), batch.device
        self.input_ids = torch.zeros(B, dtype=torch.int64, device=dev)
        self.positions = torch.zeros(B, dtype=torch.int64, device=dev)
        self.slot_mapping = torch.zeros(B, dtype=torch.int32, device=dev)
        self.context_lens = torch.zeros(B, dtype=torch.int32, device=dev)
        self.graph = None
        self.out = None

    def set_inputs(self, tokens, step):
        b = self.batch
        pos = [n + step for n in b.lens]
        self.input_ids.copy_(torch.tensor(tokens, dtype=torch.int64))
        self.positions.copy_(torch.tensor(pos, dtype=torch.int64))
        self.slot_mapping.copy_(torch.tensor([b.tables[i][p // BLOCK] * BLOCK + p % BLOCK for i, p in enumerate(pos)],
                                             dtype=torch.int32))
        self.context_lens.copy_(torch.tensor([p + 1 for p in pos], dtype=torch.int32))

    def forward(self):
        ctx = Context(False, self.slot_mapping, self.context_lens, self.batch.block_tables)
        h = self.model.forward(self.input_ids, self.positions, ctx, self.backend, self.attention, self.linear)
        if self.backend == "hip" and not self.fp32_logits:
            # greedy sampling on the bf16 logits (csrc/sampler.hip): the index of logits.float().argmax(-1)
            logits = self.model.logits(h, False, self.backend, self.linear, as_float=False)
            return logits, greedy_sample(logits)
        logits = self.model.logits(h, self.fp32_logits, self.backend, self.linear)
        return logits, logits.argmax(dim=-1)

    def capture(self):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.forward()  # warm-up outside the graph (allocations, library handles)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(self.graph):
            self.out = self.forward()
        self.graph.instantiate()

    def run(self):
        if self.graph is None:
            return self.forward()
        self.graph.replay()
        return self.out


@torch.inference_mode()
def decode(model, batch, first, steps, backend, use_graph, reference=None, fp32_logits=False, attention="hip",
           linear="hip"):
    """Greedy decode of `steps` tokens after `first`; returns (tokens [B][steps], divergence info vs reference)."""
    step = DecodeStep(model, batch, backend, fp32_logits, attention, linear)
    if use_graph:
        step.set_inputs(first, 0)
        step.capture()
    B = len(batch.lens)
    tokens, cur = [], list(first)
    diverged = {}
    for s in range(steps):
        step.set_inputs(cur, s)
        logits, nxt = step.run()
        nxt = nxt.tolist()
        if reference is not None:
            for b in range(B):
                if b not in diverged and reference[b][s] != nxt[b]:
                    gap = float(logits[b, nxt[b]].float() - logits[b, reference[b][s]].float())
                    diverged[b] = {"step": s, "logit_gap": round(gap, 5)}
        tokens.append(nxt)
        cur = nxt
    return [list(t) for t in zip(*tokens)], diverged, step


def graph_nodes(graph):
    """(kernel nodes, all nodes) of a captured torch CUDAGraph (keep_graph=True), via hipGraphGetNodes."""
    hip = ctypes.CDLL("libamdhip64.so.7")
    raw = ctypes.c_void_p(graph.raw_cuda_graph())
    n = ctypes.c_size_t(0)
    if hip.hipGraphGetNodes(raw, None, ctypes.byref(n)) != 0:
        return None, None
    nodes = (ctypes.c_void_p * n.value)()
    hip.hipGraphGetNodes(raw, nodes, ctypes.byref(n))
    kernels = 0
    for node in nodes:
        t = ctypes.c_int(-1)
        hip.hipGraphNodeGetType(ctypes.c_void_p(node), ctypes.byref(t))
        kernels += t.value == 0  # hipGraphNodeTypeKernel
    return kernels, n.value


def replay_us(step, reps, warm=10):
    """Average microseconds per replay of the captured step, after `warm` untimed replays (the GPU raises its
    clocks over the first milliseconds of load)."""
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(warm):
        step.graph.replay()
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        step.graph.replay()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) * 1e3 / reps


def agreement(a, b):
    same = sum(x == y for ra, rb in zip(a, b) for x, y in zip(ra, rb))
    total = sum(len(r) for r in a)
    return same, total


def main(argv=None):
    p = argparse.ArgumentParser()
    p.add_argument("--batch", type=int, default=32)
    p.add_argument("--steps", type=int, default=32)
    p.add_argument("--layers", type=int, default=28)
    p.add_argument("--min-len", type=int, default=512)
    p.add_argument("--max-len", type=int, default=2048)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--reps", type=int, default=20)
    p.add_argument("--fp32-logits", action="store_true", help="LM head in fp32 (both backends)")
    p.add_argument("--attention", choices=("hip", "torch"), default="hip",
                   help="decode attention of both backends: HIP paged kernel or the fp32 torch code")
    p.add_argument("--linear", choices=("hip", "torch"), default="hip",
                   help="projections and LM head of the hip backend: HIP GEMM or torch F.linear")
    args = p.parse_args(argv)
    f32, att, lin = args.fp32_logits, args.attention, args.linear
    dev = torch.device("cuda:0")
    cfg = Qwen3Config(num_hidden_layers=args.layers)
    t0 = time.time()
    model = Qwen3(cfg, dev, seed=args.seed)
    batch = Batch(cfg, args.batch, args.steps, args.min_len, args.max_len, args.seed, dev)
    out = {"config": {"model": "Qwen3-0.6B shapes, random init", "layers": args.layers, "batch": args.batch,
                      "steps": args.steps, "prompt_lens": [args.min_len, args.max_len], "kv_blocks": batch.num_blocks,
                      "block_size": BLOCK, "lm_head": "fp32" if f32 else "bf16",
                      "decode_attention": att, "hip_backend_linear": lin}}
    print(f"model + batch ready in {time.time() - t0:.1f}s; prompts {sum(batch.lens)} tokens", flush=True)

    # hip backend: prefill, eager decode, graph decode from the same KV state
    cache = model.allocate_kv_cache(batch.num_blocks)
    first_h, _ = prefill(model, batch, "hip", f32, linear=lin, attention=att)
    snapshot = cache.clone()
    tok_h, _, _ = decode(model, batch, first_h, args.steps, "hip", use_graph=False, fp32_logits=f32, attention=att,
                         linear=lin)
    cache.copy_(snapshot)
    tok_hg, _, step_hg = decode(model, batch, first_h, args.steps, "hip", use_graph=True, fp32_logits=f32,
                                attention=att, linear=lin)
    print("hip backend done", flush=True)
    # torch backend (the reference): eager decode, compared step by step with the hip tokens (while a request's
    # history is identical its logits are directly comparable), then graph decode
    cache.zero_()
    first_t, div_prefill = prefill(model, batch, "torch", f32, reference=first_h, attention=att)
    snapshot.copy_(cache)
    tok_t, div, _ = decode(model, batch, first_t, args.steps, "torch", use_graph=False, reference=tok_h,
                        fp32_logits=f32, attention=att)
    cache.copy_(snapshot)
    tok_tg, _, step_tg = decode(model, batch, first_t, args.steps, "torch", use_graph=True, fp32_logits=f32,
                                attention=att)
    print("torch backend done", flush=True)
    div = {b: d for b, d in div.items() if first_h[b] == first_t[b]}
    div.update(div_prefill)

    full_t = [[f] + t for f, t in zip(first_t, tok_t)]
    full_h = [[f] + t for f, t in zip(first_h, tok_h)]
    same, total = agreement(full_h, full_t)
    out["first_token_agreement"] = sum(a == b for a, b in zip(first_h, first_t))
    out["tokens_hip_vs_torch_eager"] = {"identical": same, "total": total,
                                        "requests_identical": sum(a == b for a, b in zip(full_h, full_t))}
    out["graph_equals_eager"] = {"hip": tok_hg == tok_h, "torch": tok_tg == tok_t}
    out["divergence"] = {str(b): d for b, d in sorted(div.items())}
    k_h, n_h = graph_nodes(step_hg.graph)
    k_t, n_t = graph_nodes(step_tg.graph)
    out["decode_step_graph"] = {
        "hip": {"us": round(replay_us(step_hg, args.reps), 1), "kernels": k_h, "nodes": n_h},
        "torch": {"us": round(replay_us(step_tg, args.reps), 1), "kernels": k_t, "nodes": n_t}}
    print(json.dumps(out), flush=True)
    return out


if __name__ == "__main__":
    main()
