"""nvhip_paged_decode_attention_bf16_noalloc (GPU): the paged decode attention whose pair counters and split records
live in the library's own device scratch array instead of a caller workspace. Called through the C ABI, it must
give bitwise the output of nvhip_paged_decode_attention_bf16 with a zero-filled workspace of the size that entry
point asks for (the same plan, the same kernels), on calls in a row -- a balanced batch of 32 sequences, then
smaller batches with context splits and shorter contexts, so stale records or counters of a call would show; and
recorded into a HIP graph after an eager warm-up call (which looks up the scratch address), whose replays, with new
queries copied into the captured input between them and eager calls of both entry points in between, must each
give bitwise the workspace entry point's output for those queries.
(Its refusal of sizes beyond the scratch cannot be reached with valid arguments: the plan never needs more than
the 16.1 MiB the array holds.)"""
import pytest
import torch

from nanovllm_hip import _lib

pytestmark = pytest.mark.gpu

DEV = "cuda"
HQ, HKV, D, BS = 16, 8, 128, 256


def noalloc_fn():
    return _lib.lib().nvhip_paged_decode_attention_bf16_noalloc


def make_case(seed, batch, max_ctx):
    g = torch.Generator("cpu").manual_seed(seed)
    lens = torch.randint(max_ctx // 2, max_ctx + 1, (batch,), generator=g)
    max_blocks = (max_ctx + BS - 1) // BS
    nb = batch * max_blocks
    kc = torch.randn(nb, BS, HKV, D, generator=g).to(torch.bfloat16).to(DEV)
    vc = torch.randn(nb, BS, HKV, D, generator=g).to(torch.bfloat16).to(DEV)
    bt = torch.randperm(nb, generator=g).to(torch.int32).view(batch, max_blocks).to(DEV)
    q = torch.randn(batch, HQ, D, generator=g).to(torch.bfloat16).to(DEV)
    return q, kc, vc, bt, lens.to(torch.int32).to(DEV), max_blocks


def call(fn, case, out, extra):
    q, kc, vc, bt, lens, max_blocks = case
    B = q.shape[0]
    args = [out.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(), bt.data_ptr(), lens.data_ptr(), B, 1, HQ,
            HKV, D, BS, kc.shape[0], max_blocks, HQ * D, D, HQ * D, D, D ** -0.5, 1]
    return fn(*args, *extra, torch.cuda.current_stream().cuda_stream)


def test_noalloc_equals_workspace_entry_point_on_calls_in_a_row():
    lib = _lib.lib()
    fn = noalloc_fn()
    for seed, batch, max_ctx in ((3, 32, 2048), (1, 4, 4096), (2, 2, 1100)):
        case = make_case(seed, batch, max_ctx)
        need = lib.nvhip_paged_decode_attention_workspace_size(batch, 1, HQ, HKV, D, BS, case[5])
        assert need > 0, "the case must split its contexts (the scratch is used)"
        ws = torch.zeros(need, dtype=torch.uint8, device=DEV)  # its counters must start at zero
        ref = torch.empty(batch, HQ, D, dtype=torch.bfloat16, device=DEV)
        _lib.check(call(lib.nvhip_paged_decode_attention_bf16, case, ref, [ws.data_ptr(), need]), "workspace call")
        out = torch.full((batch, HQ, D), float("nan"), dtype=torch.bfloat16, device=DEV)
        _lib.check(call(fn, case, out, []), "noalloc call")
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"batch {batch}: differs from the workspace entry point"


def test_noalloc_graph_replays_equal_workspace_entry_point():
    lib = _lib.lib()
    fn = noalloc_fn()
    case = make_case(5, 32, 2048)  # balanced batch: records merged inside the launch through the scratch counters
    q, max_blocks = case[0], case[5]
    need = lib.nvhip_paged_decode_attention_workspace_size(32, 1, HQ, HKV, D, BS, max_blocks)
    assert need > 0
    ws = torch.zeros(need, dtype=torch.uint8, device=DEV)
    out = torch.empty(32, HQ, D, dtype=torch.bfloat16, device=DEV)
    _lib.check(call(fn, case, out, []), "eager warm-up")  # scratch address looked up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.check(call(fn, case, out, []), "captured call")
    g = torch.Generator("cpu").manual_seed(11)
    other = make_case(6, 4, 4096)  # an eager call of another plan between the replays, through the same scratch
    other_out = torch.empty(4, HQ, D, dtype=torch.bfloat16, device=DEV)
    for rep in range(3):
        q.copy_(torch.randn(32, HQ, D, generator=g).to(torch.bfloat16))
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        ref = torch.empty_like(out)
        _lib.check(call(lib.nvhip_paged_decode_attention_bf16, case, ref, [ws.data_ptr(), need]), "workspace call")
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep}: differs from the workspace entry point"
        _lib.check(call(fn, other, other_out, []), "eager noalloc call between replays")
        torch.cuda.synchronize()


def test_noalloc_rejects_bad_arguments_before_launching():
    fn = noalloc_fn()
    B, max_blocks = 4, 16  # would split: the arguments are checked before the scratch is used
    args = [None, None, None, None, None, None, B, 1, HQ, HKV, D, BS, 1, max_blocks, HQ * D, D, HQ * D, D, 0.1, 1,
            None]
    assert fn(*args) == _lib.NVHIP_EINVAL and "null pointer" in _lib.lib().nvhip_last_error().decode()
    args[10] = 96  # head_dim
    assert fn(*args) == _lib.NVHIP_EINVAL and "head_dim" in _lib.lib().nvhip_last_error().decode()
