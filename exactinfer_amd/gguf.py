"""Python view of the GGUF reader (include/ei_gguf.h; exactinfer_amd/host/gguf_index.cpp).

The C++ reader maps and validates the file; this module only wraps its C ABI: metadata by key,
the tensor table, tensors as numpy arrays (copied out of the mapping, so they outlive the file),
and the Qwen3 configuration (read_config + read_tensors, src/model.cpp:38-103).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from . import _capi

F32, F16, BF16 = 0, 1, 30


class GgufError(RuntimeError):
    """A file the reader rejects (the reference raises el::GgufError / std::runtime_error)."""


class _Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("n_layer", "n_embd", "n_ff", "n_head", "n_head_kv", "head_dim",
                                            "rope_dim", "n_ctx_train", "n_vocab")] + \
               [("rope_base", ctypes.c_double), ("eps", ctypes.c_float)]


class GgufFile:
    def __init__(self, path: str | Path):
        L = _capi.lib()
        self._h = L.ei_gguf_open(str(path).encode())
        if not self._h:
            raise GgufError(L.ei_last_error().decode(errors="replace"))

    def close(self) -> None:
        if self._h:
            _capi.lib().ei_gguf_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # ------------------------------------------------------------ metadata
    @property
    def version(self) -> int:
        return _capi.lib().ei_gguf_version(self._h)

    def _get(self, fn: str, ctype, key: str):
        out = ctype()
        st = getattr(_capi.lib(), fn)(self._h, key.encode(), ctypes.byref(out))
        if st != 0:
            raise GgufError(_capi.lib().ei_last_error().decode(errors="replace"))
        return out.value

    def get_int(self, key: str) -> int:
        return int(self._get("ei_gguf_get_int", ctypes.c_int64, key))

    def get_float(self, key: str) -> float:
        return float(self._get("ei_gguf_get_float", ctypes.c_double, key))

    def get_str(self, key: str) -> str:
        return self._get("ei_gguf_get_str", ctypes.c_char_p, key).decode()

    # ------------------------------------------------------------ tensors
    def _info(self, i: int):
        name, ty, nd = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_int()
        ne = (ctypes.c_uint64 * 4)()
        data, nbytes = ctypes.c_void_p(), ctypes.c_uint64()
        _capi.call("ei_gguf_tensor", self._h, i, ctypes.byref(name), ctypes.byref(ty), ctypes.byref(nd), ne,
                   ctypes.byref(data), ctypes.byref(nbytes))
        return name.value.decode(), ty.value, [int(ne[k]) for k in range(nd.value)], data.value, nbytes.value

    def tensor_names(self) -> list[str]:
        return [self._info(i)[0] for i in range(_capi.lib().ei_gguf_n_tensors(self._h))]

    def tensor_info(self, name: str):
        """(GGML type id, dims with ne[0] first, byte size) or None."""
        i = _capi.lib().ei_gguf_find_tensor(self._h, name.encode())
        if i < 0:
            return None
        _, ty, ne, _, nb = self._info(i)
        return ty, ne, nb

    def tensor(self, name: str) -> np.ndarray:
        """The tensor as an array of shape ne[::-1] (row-major: ne[0] contiguous): float32 for F32,
        float16 for F16, the raw bytes (uint8, [rows][row bytes]) for other types."""
        i = _capi.lib().ei_gguf_find_tensor(self._h, name.encode())
        if i < 0:
            raise GgufError(f"tensor missing: {name}")
        _, ty, ne, ptr, nb = self._info(i)
        raw = np.frombuffer((ctypes.c_uint8 * nb).from_address(ptr), dtype=np.uint8).copy()
        if ty == F32:
            return raw.view(np.float32).reshape(ne[::-1])
        if ty == F16:
            return raw.view(np.float16).reshape(ne[::-1])
        return raw.reshape(int(np.prod(ne[1:])) if len(ne) > 1 else 1, -1)

    def qwen3_config(self) -> dict:
        c = _Config()
        st = _capi.lib().ei_gguf_qwen3_config(self._h, ctypes.byref(c))
        if st != 0:
            raise GgufError(_capi.lib().ei_last_error().decode(errors="replace"))
        return {n: getattr(c, n) for n, _ in _Config._fields_}
