"""Loader of libnvhip.so, the C-ABI HIP kernel library (declared in include/nvhip.h).

The library is built in-tree (csrc/Makefile) next to this file. There is no fallback: if it is missing or does not
load, every kernel call raises. torch is imported first so that the library binds to the HIP runtime torch already
loaded (both carry the soname libamdhip64.so.7): one runtime, one set of streams.
"""
import ctypes
import os

import torch  # noqa: F401  (must be loaded before the HIP library, see above)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libnvhip.so")
ABI_VERSION = 7

NVHIP_OK = 0
NVHIP_EINVAL = -1
NVHIP_ELAUNCH = -2
DTYPE_F32 = 0
DTYPE_BF16 = 1
PREC_IEEE = 0
PREC_TF32 = 1

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_f = ctypes.c_float
_i = ctypes.c_int

# name -> argument types, in the order of include/nvhip.h
SIGNATURES = {
    "nvhip_abi_version": [],
    "nvhip_last_error": [],
    "nvhip_qk_norm_rope_kv_bf16": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _i64, _i64, _p, _p,
                                   _i64, _i64, _i64, _i64, _i64, _f, _p],
    "nvhip_rms_norm_bf16": [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _f, _p],
    "nvhip_add_rms_norm_bf16": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _f, _p],
    "nvhip_silu_mul_bf16": [_p, _p, _i64, _i64, _i64, _p],
    "nvhip_matmul": [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i, _i, _p],
    "nvhip_paged_decode_attention_bf16": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                          _i64, _i64, _i64, _i64, _f, _i, _p, _i64, _p],
    "nvhip_paged_decode_attention_workspace_size": [_i64, _i64, _i64, _i64, _i64, _i64, _i64],
    "nvhip_paged_decode_attention_bf16_noalloc": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                                  _i64, _i64, _i64, _i64, _i64, _f, _i, _p],
    "nvhip_store_kvcache": [_p, _p, _p, _p, _i64, _i64, _p, _i64, _i64, _i64, _i64, _p],
    "nvhip_matmul_silu_mul_bf16": [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _p],
    "nvhip_prefill_attention_bf16": [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                     _i64, _i64, _i64, _i64, _p, _i64, _i64, _i64, _f, _i, _p, _i64, _p],
    "nvhip_prefill_attention_workspace_size": [_i64, _i64, _i64, _i64, _i64, _i64, _i64],
    "nvhip_rms_norm_matmul_bf16": [_p, _p, _p, _p, _p, _f, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i, _p],
    "nvhip_matmul_add_rms_norm_bf16": [_p, _p, _p, _p, _p, _p, _f, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "nvhip_matmul_add_rms_norm_workspace_size": [_i64, _i64, _i64],
    "nvhip_qk_norm_rope_kv_decode_attention_bf16": [_p, _p, _p, _p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _i64, _i64,
                                                    _f, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64,
                                                    _i64, _i64, _f, _p, _i64, _p],
    "nvhip_argmax_workspace_size": [_i64, _i64],
    "nvhip_argmax_bf16": [_p, _p, _i64, _i64, _i64, _p, _i64, _p],
}
RESTYPES = {"nvhip_last_error": ctypes.c_char_p, "nvhip_paged_decode_attention_workspace_size": ctypes.c_int64,
            "nvhip_prefill_attention_workspace_size": ctypes.c_int64,
            "nvhip_matmul_add_rms_norm_workspace_size": ctypes.c_int64, "nvhip_argmax_workspace_size": ctypes.c_int64}

_lib = None


class KernelError(RuntimeError):
    """A kernel launch was refused by the HIP runtime."""


def lib() -> ctypes.CDLL:
    """The loaded library (loaded on first use). Raises if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built: run `make -C <package>/csrc` (or __graft_entry__.build())")
        handle = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = RESTYPES.get(name, ctypes.c_int)
        version = handle.nvhip_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libnvhip.so ABI version {version}, expected {ABI_VERSION}: rebuild it")
        _lib = handle
    return _lib


def check(status: int, what: str) -> None:
    """Turns a negative status into ValueError (bad argument) or KernelError (launch failure)."""
    if status == NVHIP_OK:
        return
    msg = lib().nvhip_last_error().decode(errors="replace") or what
    if status == NVHIP_EINVAL:
        raise ValueError(msg)
    raise KernelError(msg)


def stream_of(t: torch.Tensor) -> int:
    """hipStream_t (as an int) of torch's current stream on t's device."""
    return torch.cuda.current_stream(t.device).cuda_stream
