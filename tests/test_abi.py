"""The C-ABI library (CPU only, no kernel launches): libnvhip.so loads, exports every function include/nvhip.h
declares with the argument count the Python binding uses, and rejects bad arguments before launching anything
(those paths return before any HIP call, so they run without a GPU)."""
import ctypes
import os
import re

import pytest

from nanovllm_hip import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nvhip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(?:const\s+)?\w+\s*\*?\s*(nvhip_\w+)\s*\(([^)]*)\)\s*;", text, flags=re.M):
        args = m.group(2).strip()
        out[m.group(1)] = 0 if args in ("", "void") else len(args.split(","))
    return out


def test_header_declares_the_five_kernels():
    names = set(declared_functions())
    assert {"nvhip_qk_norm_rope_kv_bf16", "nvhip_rms_norm_bf16", "nvhip_add_rms_norm_bf16", "nvhip_silu_mul_bf16",
            "nvhip_matmul", "nvhip_last_error", "nvhip_abi_version"} <= names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    decl = declared_functions()
    for name, nargs in decl.items():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no Python binding"
        assert len(_lib.SIGNATURES[name]) == nargs, f"{name}: header has {nargs} args"
    assert set(_lib.SIGNATURES) == set(decl)
    assert lib.nvhip_abi_version() == _lib.ABI_VERSION


def _err():
    return _lib.lib().nvhip_last_error().decode()


def test_qk_rejects_bad_arguments_without_launching():
    f = _lib.lib().nvhip_qk_norm_rope_kv_bf16
    P = None
    common = dict(q_stride=4096, k_stride=4096, v_stride=4096, cs_stride=128, max_pos=40960, num_slots=0)

    def call(T=4, Hq=16, Hkv=8, D=128, k_cache=None, v_cache=None, slot=None, q_stride=4096):
        return f(P, P, P, P, P, q_stride, common["k_stride"], common["v_stride"], P, slot, P, P, P,
                 common["cs_stride"], common["max_pos"], k_cache, v_cache, 16, T, Hq, Hkv, D, 1e-6, P)

    assert call(D=96) == _lib.NVHIP_EINVAL and "head_dim" in _err()
    assert call(Hq=12, Hkv=8) == _lib.NVHIP_EINVAL and "multiple" in _err()
    assert call(T=-1) == _lib.NVHIP_EINVAL
    assert call(k_cache=ctypes.c_void_p(16)) == _lib.NVHIP_EINVAL and "together" in _err()
    assert call(T=0) == _lib.NVHIP_OK and _err() == ""  # T = 0: nothing to do, nothing launched
    assert call() == _lib.NVHIP_EINVAL and "null" in _err()


def test_norm_silu_matmul_reject_bad_arguments_without_launching():
    lib = _lib.lib()
    assert lib.nvhip_rms_norm_bf16(None, None, None, 4, 1, 1024, 0, 0, 1e-6, None) == _lib.NVHIP_EINVAL
    assert lib.nvhip_rms_norm_bf16(None, None, None, 0, 1, 1024, 0, 1024, 1e-6, None) == _lib.NVHIP_OK
    assert lib.nvhip_rms_norm_bf16(None, None, None, 4, 1, 1024, 0, 1024, 1e-6, None) == _lib.NVHIP_EINVAL
    assert "null" in _err()
    assert lib.nvhip_add_rms_norm_bf16(None, None, None, None, None, 4, 512, 1024, 1024, 1e-6, None) == \
        _lib.NVHIP_EINVAL and "stride" in _err()
    assert lib.nvhip_add_rms_norm_bf16(None, None, None, None, None, 0, 1024, 1024, 1024, 1e-6, None) == _lib.NVHIP_OK
    assert lib.nvhip_silu_mul_bf16(None, None, 4, 100, 64, None) == _lib.NVHIP_EINVAL
    assert lib.nvhip_silu_mul_bf16(None, None, 0, 128, 64, None) == _lib.NVHIP_OK
    m = lib.nvhip_matmul
    assert m(None, None, None, 4, 4, 4, 4, 1, 4, 1, 4, 1, 7, 0, None) == _lib.NVHIP_EINVAL and "dtype" in _err()
    assert m(None, None, None, 4, 4, 4, 4, 1, 4, 1, 4, 1, 0, 5, None) == _lib.NVHIP_EINVAL and "precision" in _err()
    assert m(None, None, None, 4, 4, 4, -4, 1, 4, 1, 4, 1, 0, 0, None) == _lib.NVHIP_EINVAL
    assert m(None, None, None, 0, 4, 4, 4, 1, 4, 1, 4, 1, 1, 0, None) == _lib.NVHIP_OK
    assert m(None, None, None, 4, 4, 4, 4, 1, 4, 1, 4, 1, 1, 0, None) == _lib.NVHIP_EINVAL and "null" in _err()


def test_check_maps_status_to_exceptions():
    lib = _lib.lib()
    lib.nvhip_silu_mul_bf16(None, None, 4, 100, 64, None)
    with pytest.raises(ValueError, match="stride"):
        _lib.check(_lib.NVHIP_EINVAL, "silu")
    with pytest.raises(_lib.KernelError):
        _lib.check(_lib.NVHIP_ELAUNCH, "silu")
    _lib.check(_lib.NVHIP_OK, "silu")


def test_attention_store_and_fused_gemm_reject_bad_arguments_without_launching():
    lib = _lib.lib()
    P = None
    dec = lib.nvhip_paged_decode_attention_bf16

    def decode(num_seqs=2, q_len=1, Hq=16, Hkv=8, D=128, bs=256, nb=4, mb=2, qst=2048, qsh=128, ost=2048, osh=128):
        return dec(P, P, P, P, P, P, num_seqs, q_len, Hq, Hkv, D, bs, nb, mb, qst, qsh, ost, osh, 0.1, 1, P, 0, P)

    assert decode(Hq=12) == _lib.NVHIP_EINVAL and "multiple" in _err()
    assert decode(D=96) == _lib.NVHIP_EINVAL and "head_dim" in _err()
    assert decode(q_len=3, Hq=16, Hkv=2) == _lib.NVHIP_EINVAL and "<= 16" in _err()   # 24 rows per kv head
    assert decode(qsh=100) == _lib.NVHIP_EINVAL and "strides" in _err()
    assert decode(num_seqs=0) == _lib.NVHIP_OK
    assert decode() == _lib.NVHIP_EINVAL and "null" in _err()
    ws = lib.nvhip_paged_decode_attention_workspace_size
    # 256 pairs: 512 counters (2 KiB) + 2 record blocks per pair of 2 rows x (2 + 128) fp32 in 128-byte lines
    assert ws(32, 1, 16, 8, 128, 256, 8) == 2048 + 256 * 2 * 288 * 4
    assert ws(1, 1, 16, 8, 128, 256, 64) > 0                  # one long sequence: split over blocks
    assert ws(1, 1, 16, 8, 128, 256, 64) == 2048 + 8 * 32 * 288 * 4    # 8 pairs x 32 splits of 512 tokens
    assert ws(520, 1, 16, 8, 128, 256, 8) == 0                # 4160 pairs: one block each
    assert ws(1, 1, 16, 8, 128, 256, 1) == 0                  # 8 pairs of one 256-token round: nothing to split
    assert ws(0, 1, 16, 8, 128, 256, 8) == 0

    pre = lib.nvhip_prefill_attention_bf16

    def prefill(num_seqs=2, maxq=64, Hq=16, Hkv=8, D=128, kst=4160, bt=None, bs=0, nb=0, mb=0, scale=0.1,
                ws=None, ws_size=0):
        return pre(P, P, P, P, P, P, num_seqs, maxq, 300, 128, Hq, Hkv, D, 4160, 128, kst, kst, 2048, 128, bt, bs,
                   nb, mb, scale, 1, ws, ws_size, P)

    assert prefill(D=256) == _lib.NVHIP_EINVAL and "head_dim" in _err()
    assert prefill(kst=1000) == _lib.NVHIP_EINVAL and "k / v strides" in _err()
    assert prefill(bt=ctypes.c_void_p(64), bs=0) == _lib.NVHIP_EINVAL and "block table" in _err()
    assert prefill(maxq=0) == _lib.NVHIP_OK
    assert prefill(scale=0.0) == _lib.NVHIP_EINVAL and "softmax_scale" in _err()
    assert prefill(scale=-0.1) == _lib.NVHIP_EINVAL and "softmax_scale" in _err()
    assert prefill() == _lib.NVHIP_EINVAL and "null" in _err()

    # key splits of the prefill attention: only when few blocks meet long key ranges
    pws = lib.nvhip_prefill_attention_workspace_size
    rec = (128 + 2) * 4                                       # bytes of one (split, query, head) record: O, max, sum
    dec = (2 + 128) * 4 * 16                                  # one short-sequence split record: 16 rows (8 queries x G 2)
    cnt = 2048                                                # the decode attention's counters, first
    # 4 x 16 query tiles x 8 head pairs fill the CUs: no prefill split, but room for the short-sequence path's
    # splits (4 sequences x 8 kv heads = 32 pairs: at most 8 splits each)
    assert pws(4, 2048, 2048, 16, 8, 128, 8192) == cnt + 4 * 8 * 8 * dec
    # a mixed step: 136 pairs, at most 2 splits -- or the balanced pieces' 2 records per pair
    assert pws(17, 240, 2048, 16, 8, 128, 256) == cnt + 17 * 8 * 2 * dec
    assert pws(32, 1, 2048, 16, 8, 128, 32) == 0              # 256 pairs: no split anywhere
    assert pws(1, 256, 300, 16, 8, 128, 256) == 0             # keys too few to split
    assert pws(1, 256, 4096, 16, 8, 128, 256) == cnt + 16 * 256 * 16 * rec    # chunk over a prefix: 16 splits of 256
    assert pws(1, 2048, 2048, 16, 8, 128, 2048) == cnt + 2 * 2048 * 16 * rec  # one long prompt: 2 splits of 1024
    assert pws(1, 256, 4096, 16, 8, 256, 256) == 0            # head_dim 256 is not supported

    st = lib.nvhip_store_kvcache
    assert st(P, P, P, P, 1024, 1024, P, 64, 4, 1024, 3, P) == _lib.NVHIP_EINVAL and "element size" in _err()
    assert st(P, P, P, P, 512, 1024, P, 64, 4, 1024, 2, P) == _lib.NVHIP_EINVAL and "stride" in _err()
    assert st(P, P, P, P, 1024, 1024, P, 64, 0, 1024, 2, P) == _lib.NVHIP_OK
    assert st(P, P, P, P, 1024, 1024, P, 64, 4, 1024, 2, P) == _lib.NVHIP_EINVAL and "null" in _err()

    fm = lib.nvhip_matmul_silu_mul_bf16
    assert fm(P, P, P, 4, 8, 12, 16, 16, 8, P) == _lib.NVHIP_EINVAL and "null" in _err()
    assert fm(ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), 4, 8, 12, 16, 16, 8, P) == \
        _lib.NVHIP_EINVAL and "K % 8" in _err()
    assert fm(P, P, P, 0, 8, 16, 16, 16, 8, P) == _lib.NVHIP_OK


def test_rms_norm_matmul_rejects_bad_arguments_without_launching():
    f = _lib.lib().nvhip_rms_norm_matmul_bf16
    A = ctypes.c_void_p(1 << 20)   # 16-byte aligned stand-ins: every call below returns before touching them
    B = ctypes.c_void_p(2 << 20)

    def call(M=32, N=4096, K=1024, res=A, res_out=B, x=ctypes.c_void_p(3 << 20), sx=1024, silu=0):
        return f(ctypes.c_void_p(4 << 20), res_out, x, res, ctypes.c_void_p(5 << 20), 1e-6,
                 ctypes.c_void_p(6 << 20), M, N, K, sx, 1024, 1024, N, silu, None)

    assert call(M=33) == _lib.NVHIP_EINVAL and "32 rows" in _err()
    assert call(K=1000) == _lib.NVHIP_EINVAL and "1024 or 2048" in _err()
    assert call(res_out=None) == _lib.NVHIP_EINVAL and "residual_out" in _err()
    assert call(res=None) == _lib.NVHIP_EINVAL and "residual_out" in _err()     # residual_out without residual
    assert call(sx=1000) == _lib.NVHIP_EINVAL and "strides" in _err()
    assert call(x=ctypes.c_void_p((3 << 20) + 8)) == _lib.NVHIP_EINVAL and "aligned" in _err()
    assert call(res_out=ctypes.c_void_p((1 << 20) + 2048 * 16)) == _lib.NVHIP_EINVAL and "overlap" in _err()
    assert call(M=0) == _lib.NVHIP_OK and _err() == ""


def test_argmax_rejects_bad_arguments_without_launching():
    f = _lib.lib().nvhip_argmax_bf16
    P = None
    assert f(P, P, -1, 10, 10, P, 0, P) == _lib.NVHIP_EINVAL
    assert f(P, P, 4, 0, 10, P, 0, P) == _lib.NVHIP_EINVAL
    assert f(P, P, 4, 10, 9, P, 0, P) == _lib.NVHIP_EINVAL and "stride" in _err()
    assert f(P, P, 65536, 10, 10, P, 0, P) == _lib.NVHIP_EINVAL and "rows" in _err()
    assert f(P, P, 4, 10, 10, P, 0, P) == _lib.NVHIP_EINVAL and "null" in _err()
    assert f(P, P, 0, 10, 10, P, 0, P) == _lib.NVHIP_OK and _err() == ""  # no rows: nothing launched
    ws = _lib.lib().nvhip_argmax_workspace_size
    assert ws(32, 151936) == 32 * 16 * 16  # 16 slices of 9496 logits per row, 16 bytes each
    assert ws(1, 100) == 0 and ws(4096, 151936) == 0 and ws(0, 10) == 0
