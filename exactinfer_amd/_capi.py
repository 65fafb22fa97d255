"""ctypes binding of libei_attn.so (the C ABI declared in include/ei_attn.h).

Loading fails loudly: there is no fallback path.  torch is imported first so that the
library binds to the HIP runtime torch already loaded (both carry the soname
libamdhip64.so.7), which keeps device pointers and streams shared.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (must precede the library load, see module docstring)

import os

# EI_ATTN_LIB may point at an alternative build of the same library (e.g. an instrumented one)
LIB_PATH = Path(os.environ.get("EI_ATTN_LIB") or Path(__file__).resolve().parent / "libei_attn.so")

# every symbol include/ei_attn.h declares (checked by tests/test_capi_exports.py)
EXPORTS = (
    "ei_last_error", "ei_abi_version", "ei_rope_table_fill", "ei_headnorm_rope", "ei_kv_append", "ei_qkv_prepare",
    "ei_attn_decode_ws_bytes", "ei_attn_workspace_init", "ei_attn_decode", "ei_attn_decode_batched",
    "ei_decode_step", "ei_decode_step_noalloc", "ei_attn_decode_paged", "ei_decode_step_paged", "ei_attn_prefill", "ei_attn_prefill_ws_bytes", "ei_attn_prefill_split", "ei_prefill_step", "ei_prefill_step_paged", "ei_qkv_project", "ei_stream_ceiling", "ei_synth_fill",
    "ei_attn_workspace_status", "ei_decode_status_check", "ei_read_ceiling",
    "ei_qkv_project_max_rows",
    # include/ei_gguf.h
    "ei_gguf_open", "ei_gguf_close", "ei_gguf_version", "ei_gguf_n_tensors", "ei_gguf_tensor", "ei_gguf_find_tensor",
    "ei_gguf_get_int", "ei_gguf_get_float", "ei_gguf_get_str", "ei_gguf_qwen3_config",
)

_vp, _i, _l, _f, _d, _sz, _u64 = (ctypes.c_void_p, ctypes.c_int, ctypes.c_long, ctypes.c_float, ctypes.c_double,
                                  ctypes.c_size_t, ctypes.c_uint64)

_SIGS = {
    "ei_last_error": ([], ctypes.c_char_p),
    "ei_abi_version": ([], _i),
    "ei_rope_table_fill": ([_vp, _i, _i, _d], _i),
    "ei_headnorm_rope": ([_vp, _vp, _i, _l, _i, _i, _vp, _vp, _vp, _i, _f], _i),
    "ei_kv_append": ([_vp, _vp, _vp, _l, _i, _vp, _vp, _i, _vp], _i),
    "ei_qkv_prepare": ([_vp, _vp, _i, _l, _i, _i, _i, _vp, _vp, _vp, _vp, _i, _f, _vp, _vp], _i),
    "ei_attn_decode_ws_bytes": ([_i, _i, _i, _i], _sz),
    "ei_attn_workspace_init": ([_vp, _vp, _sz], _i),
    "ei_attn_workspace_status": ([_vp, _vp, _sz, ctypes.POINTER(ctypes.c_uint32)], _i),
    "ei_decode_status_check": ([ctypes.c_uint32], _i),
    "ei_read_ceiling": ([_vp, _vp, _sz, _i, _i, _vp], _i),
    "ei_qkv_project_max_rows": ([_i], _i),
    "ei_attn_decode": ([_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _f, _i, _vp, _sz], _i),
    "ei_attn_decode_batched": ([_vp, _vp, _l, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _i, _vp, _sz], _i),
    "ei_decode_step": ([_vp, _vp, _l, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _i, _f, _f, _i,
                        _vp, _sz], _i),
    "ei_decode_step_noalloc": ([_vp, _vp, _l, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _i, _f, _f,
                                _i], _i),
    "ei_attn_decode_paged": ([_vp, _vp, _l, _vp, _vp, _vp, _vp, _i, _i, _vp, _i, _i, _i, _i, _f, _i, _vp, _sz], _i),
    "ei_decode_step_paged": ([_vp, _vp, _l, _vp, _vp, _vp, _vp, _i, _i, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _i, _f,
                              _f, _i, _vp, _sz], _i),
    "ei_attn_prefill": ([_vp, _vp, _l, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f], _i),
    "ei_attn_prefill_ws_bytes": ([_i, _i, _i, _i], _sz),
    "ei_attn_prefill_split": ([_vp, _vp, _l, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _i, _vp, _sz], _i),
    "ei_prefill_step": ([_vp, _vp, _l, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _i, _f, _f, _i, _vp, _sz], _i),
    "ei_prefill_step_paged": ([_vp, _vp, _l, _vp, _vp, _vp, _vp, _i, _i, _vp, _i, _i, _i, _i, _vp, _vp, _vp, _i, _f, _f,
                               _i, _vp, _sz], _i),
    "ei_qkv_project": ([_vp, _vp, _l, _i, _i, _vp, _f, _vp, _i, _i, _vp, _l], _i),
    "ei_gguf_open": ([ctypes.c_char_p], _vp),
    "ei_gguf_close": ([_vp], None),
    "ei_gguf_version": ([_vp], _i),
    "ei_gguf_n_tensors": ([_vp], _l),
    "ei_gguf_tensor": ([_vp, _l, _vp, _vp, _vp, _vp, _vp, _vp], _i),
    "ei_gguf_find_tensor": ([_vp, ctypes.c_char_p], _l),
    "ei_gguf_get_int": ([_vp, ctypes.c_char_p, _vp], _i),
    "ei_gguf_get_float": ([_vp, ctypes.c_char_p, _vp], _i),
    "ei_gguf_get_str": ([_vp, ctypes.c_char_p, _vp], _i),
    "ei_gguf_qwen3_config": ([_vp, _vp], _i),
    "ei_stream_ceiling": ([_vp, _vp, _vp, _i, _i, _vp], _i),
    "ei_synth_fill": ([_vp, _vp, _sz, _u64, _u64, _l, _l, _f], _i),
}

_lib = None


ABI_VERSION = 3  # EI_ABI_VERSION of include/ei_attn.h


class EiError(RuntimeError):
    """A non-zero status from the C ABI (the reference raises std::runtime_error)."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn} failed ({code}): {msg}")
        self.code = code


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run `python -m exactinfer_amd.build` (or "
                               "__graft_entry__.build()) first; there is no non-HIP fallback")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (args, res) in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        if L.ei_abi_version() != ABI_VERSION:  # the signatures above are those of this revision
            raise RuntimeError(f"{LIB_PATH} has ABI version {L.ei_abi_version()}, this binding expects "
                               f"{ABI_VERSION}: rebuild the library")
        _lib = L
    return _lib


def call(name: str, *args) -> None:
    status = getattr(lib(), name)(*args)
    if status != 0:
        raise EiError(name, status, lib().ei_last_error().decode(errors="replace"))


def last_error() -> str:
    return lib().ei_last_error().decode(errors="replace")
