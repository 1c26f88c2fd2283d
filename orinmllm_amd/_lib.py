"""ctypes binding of liborin_attn.so (the C ABI of include/orin_attn.h).

The library is built in-tree by ``python -m orinmllm_amd.build`` (or
``__graft_entry__.build()``).  Loading fails loudly when it is missing: there is
no CPU fallback for any entry point.
"""
from __future__ import annotations

import ctypes as C
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "liborin_attn.so")

DTYPE_FP32 = 1
DTYPE_FP16 = 4
DTYPE_BF16 = 5

OK = 0
ERR_INVALID_ARG = -1
ERR_UNSUPPORTED = -2
ERR_WORKSPACE = -3
ERR_LAUNCH = -4

i32, i64, f32, sz, vp = C.c_int32, C.c_int64, C.c_float, C.c_size_t, C.c_void_p

# name -> (restype, argtypes); the order matches include/orin_attn.h.
SIGNATURES = {
    "orin_attn_abi_version": (C.c_int, []),
    "orin_attn_status_string": (C.c_char_p, [C.c_int]),
    "orin_attn_last_hip_error": (C.c_char_p, []),
    "orin_mha_kernel": (C.c_int, [i32, i32, i32, i32, i32, i32, i32, vp, vp, vp, vp, vp, vp]),
    "orin_mha_kernel_gpu_pos": (C.c_int, [vp, i32, i32, i32, i32, i32, i32, vp, vp, vp, vp, vp, vp]),
    "orin_batched_mha": (C.c_int, [i32, i32, i32, i32, i32, i32, i32, i32, i32, vp, vp, vp, vp, vp, vp]),
    "orin_flash_attention_prefill": (C.c_int, [i32, i32, i32, i32, i32, i32, i32, i32, i32, vp, vp, vp, vp, i32, vp]),
    "orin_flash_attention_prefill_qk_norm_rope": (C.c_int, [i32, i32, i32, i32, i32, i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, f32, i32, vp]),
    "orin_flash_attention_decode": (C.c_int, [i32, i32, i32, i32, i32, i32, i32, i32, vp, vp, vp, vp, i32, vp]),
    "orin_flash_attention_decode_gpu_pos": (C.c_int, [vp, i32, i32, i32, i32, i32, i32, i32, vp, vp, vp, vp, i32, vp]),
    "orin_flash_attention_decode_gpu_pos_noalloc": (C.c_int, [vp, i32, i32, i32, i32, i32, i32, i32, vp, vp, vp, vp, i32, vp]),
    "orin_flash_attention_decode_noalloc_max_bytes": (sz, []),
    "orin_flash_attention_decode_workspace_size": (sz, [i32, i32, i32]),
    "orin_flash_attention_prefill_workspace_size": (sz, [i32, i32, i32, i32, i32, i32]),
    "orin_attn_workspace_reserve": (C.c_int, [sz]),
    "orin_attn_workspace_reserve_stream": (C.c_int, [sz, sz, vp]),
    "orin_attn_workspace_release": (C.c_int, []),
    "orin_attn_workspace_release_stream": (C.c_int, [vp]),
    "orin_attn_decode_workspace_size": (sz, [i32, i32, i32, i32, i32, i32]),
    "orin_attn_decode_split_tokens": (i32, [i32, i32, i32, i32, i32]),
    "orin_attn_decode_split_tokens_for_total": (i32, [i32, i32, i32, i32, i64]),
    "orin_attn_decode": (C.c_int, [vp, vp, vp, vp, i32, i32, i32, i32, i64, i64, vp, i32, i32, f32, i32, vp, sz, vp]),
    "orin_attn_decode_paged": (C.c_int, [vp, vp, vp, vp, i32, i32, i32, i32, vp, i32, i32, i32, vp, i32, i32, f32, i32, vp, sz, vp]),
    "orin_vision_attention_pretransposed": (C.c_int, [vp, vp, vp, vp, vp, vp, i32, i32, i32, f32, i32, vp]),
    "orin_vision_attention_varlen": (C.c_int, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, f32, i32, vp]),
    "orin_batched_matmul": (C.c_int, [vp, vp, vp, i32, i32, i32, f32, i32, vp]),
    "orin_copy_to_kv_cache": (C.c_int, [vp, vp, vp, i32, i32, i32, i32, vp]),
    "orin_kv_cache_write_paged": (C.c_int, [vp, vp, i64, vp, vp, vp, i32, i32, i32, i32, i32, i32, vp]),
    "orin_kv_cache_convert": (C.c_int, [vp, i64, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp]),
    "orin_rope_sin_cos_cache": (C.c_int, [vp, vp, i32, i32, f32, vp]),
    "orin_qk_norm_rope": (C.c_int, [vp, vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, vp, i32, i32, i32, i32, f32, i32, vp]),
    "orin_vision_split_rope_transpose": (C.c_int, [vp, vp, vp, vp, vp, vp, i32, i32, i32, i32, vp]),
}


class OrinAttnError(RuntimeError):
    def __init__(self, fn: str, status: int, detail: str = ""):
        self.status = status
        msg = f"{fn} failed: {status_string(status)} ({status})"
        if detail:
            msg += f": {detail}"
        super().__init__(msg)


_lock = threading.Lock()
_lib = None


def load(path: str = LIB_PATH) -> C.CDLL:
    """Load liborin_attn.so once and attach the argument types of every entry point."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise OSError(
                f"{path} is missing: build the HIP library first "
                "(python -m orinmllm_amd.build); there is no CPU fallback"
            )
        lib = C.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def status_string(status: int) -> str:
    return load().orin_attn_status_string(status).decode()


def check(fn: str, status: int) -> None:
    if status != OK:
        detail = load().orin_attn_last_hip_error().decode() if status == ERR_LAUNCH else ""
        raise OrinAttnError(fn, status, detail)
