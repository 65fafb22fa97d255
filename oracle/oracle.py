"""ctypes/numpy front end of the CPU oracle.  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this module,
and only as the checker.  The functions mirror oracle.c one to one; each docstring names
the reference lines the C code restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_LIB_PATH = HERE / "_ref" / "libelref.so"

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i64p = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_c_int, _c_long, _c_float, _c_double = ctypes.c_int, ctypes.c_long, ctypes.c_float, ctypes.c_double
_c_size, _c_u64 = ctypes.c_size_t, ctypes.c_uint64

_lib = None
_ref = None


def build(force: bool = False) -> None:
    """Compile liboracle.so (and _ref/ when the reference tree exists) with the Makefile."""
    if force or not LIB_PATH.exists():
        subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.orc_fill_normal.argtypes = [_f32p, _c_size, _c_u64, _c_u64]
        L.orc_fill_gamma.argtypes = [_f32p, _c_size, _c_u64]
        L.orc_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _c_int, _c_float]
        L.orc_rope_inv_freq.argtypes = [_f64p, _c_int, _c_double]
        L.orc_rope.argtypes = [_f32p, _c_int, _c_int, _f64p]
        L.orc_rope_table.argtypes = [_f32p, _c_int, _c_int, _c_double]
        L.orc_headnorm_rope.argtypes = [_f32p, _c_int, _c_long, _c_int, _c_int, _f32p, _c_int, _c_int, _c_double,
                                        _c_float]
        L.orc_kv_append.argtypes = [_f32p, _f32p, _c_long, _c_int, _f32p, _f32p, _c_int, _c_int]
        L.orc_attn_decode.argtypes = [_f32p, _f32p, _f32p, _f32p, _c_int, _c_int, _c_int, _c_int, _c_float,
                                      ctypes.c_void_p]
        L.orc_attn_prefill.argtypes = [_f32p, _c_long, _f32p, _f32p, _f32p, _c_int, _c_int, _c_int, _c_int, _c_int,
                                       _c_float]
        L.orc_attn_decode_batched.argtypes = [_f32p, _f32p, _f32p, _f32p, _i64p, _i32p, _c_int, _c_int, _c_int,
                                              _c_int, _c_float]
        L.orc_attn_split_combine.argtypes = [_f32p, _f32p, _f32p, _f32p, _c_int, _c_int, _c_int, _c_int, _c_float,
                                             _c_int]
        L.orc_attn_f64.argtypes = [_f32p, _f32p, _f32p, _f64p, _c_int, _c_int, _c_int, _c_int, _c_double]
        L.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f16_to_f32.restype = _c_float
        L.orc_dot_f32.argtypes = [_f32p, _f32p, _c_long]
        L.orc_dot_f32.restype = _c_float
        L.orc_dot_f16.argtypes = [_u16p, _f32p, _c_long]
        L.orc_dot_f16.restype = _c_float
        L.orc_matvec.argtypes = [_c_int, ctypes.c_void_p, _f32p, _f32p, _c_long, _c_long]
        for name in ("orc_dequant_q8_0", "orc_dequant_q4_K", "orc_dequant_q6_K"):
            getattr(L, name).argtypes = [ctypes.c_void_p, _f32p, _c_long]
        L.orc_row_bytes.argtypes = [_c_int, _c_long]
        L.orc_row_bytes.restype = _c_long
        L.orc_threads.restype = _c_int
        L.orc_set_threads.argtypes = [_c_int]
        _lib = L
    return _lib


def ref_lib():
    """The reference's own rmsnorm / rope / rope_inv_freq built from source, or None."""
    global _ref
    if _ref is None and REF_LIB_PATH.exists():
        R = ctypes.CDLL(str(REF_LIB_PATH))
        R.elref_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _c_int, _c_float]
        R.elref_rope_inv_freq.argtypes = [_f64p, _c_int, _c_double]
        R.elref_rope.argtypes = [_f32p, _c_int, _c_int, _f64p]
        if hasattr(R, "elref_dot_f32"):
            R.elref_f16_to_f32.argtypes = [ctypes.c_uint16]
            R.elref_f16_to_f32.restype = _c_float
            R.elref_dot_f32.argtypes = [_f32p, _f32p, _c_long]
            R.elref_dot_f32.restype = _c_float
            R.elref_dot_f16.argtypes = [_u16p, _f32p, _c_long]
            R.elref_dot_f16.restype = _c_float
            for name in ("elref_dequant_q8_0", "elref_dequant_q4_K", "elref_dequant_q6_K"):
                getattr(R, name).argtypes = [ctypes.c_void_p, _f32p, _c_long]
        _ref = R
    return _ref


def _c(a, dt=np.float32):
    return np.ascontiguousarray(a, dtype=dt)


# ---------------------------------------------------------------- synthetic inputs
def normal(shape, seed: int, offset: int = 0) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    lib().orc_fill_normal(out, n, seed, offset)
    return out.reshape(shape)


def gamma(n: int, seed: int) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_fill_gamma(out, n, seed)
    return out


# ---------------------------------------------------------------- QK-norm + RoPE
def rmsnorm(x, w, eps=1e-6):
    """src/ops.cpp:155-160 on one vector."""
    x, w = _c(x), _c(w)
    out = np.empty_like(x)
    lib().orc_rmsnorm(out, x, w, x.size, eps)
    return out


def rope_inv_freq(rope_dim: int, base: float):
    """src/model.cpp:105-109."""
    out = np.empty(rope_dim // 2, np.float64)
    lib().orc_rope_inv_freq(out, rope_dim, base)
    return out


def rope(v, pos: int, inv_freq):
    """src/model.cpp:23-32 on one vector (returns a rotated copy)."""
    v = _c(v).copy()
    lib().orc_rope(v, pos, v.size, _c(inv_freq, np.float64))
    return v


def rope_table(n_ctx: int, rope_dim: int, base: float):
    """src/cuda/model_cuda.cu:1610-1619: [n_ctx][rope_dim/2][2] (cos, sin) float."""
    out = np.empty((n_ctx, rope_dim // 2, 2), np.float32)
    lib().orc_rope_table(out, n_ctx, rope_dim, base)
    return out


def headnorm_rope(buf, n_heads, D, gamma_, pos0, rope_dim, base, eps=1e-6, col0=0):
    """src/model.cpp:176-185 on the rows of `buf` ([rows, row_stride]); heads start at
    column col0.  Returns the modified copy."""
    buf = _c(buf).copy()
    rows, stride = buf.shape
    view = buf.reshape(-1)[col0:]  # contiguous 1-D view sharing buf's memory
    lib().orc_headnorm_rope(view, rows, stride, n_heads, D, _c(gamma_), pos0, rope_dim, base, eps)
    return buf


def kv_append(k_src, v_src, kc, vc, pos0):
    """src/model.cpp:186-189; k_src/v_src [rows, kd]; kc/vc [n_ctx, kd] modified in place."""
    k_src, v_src = _c(k_src), _c(v_src)
    rows, kd = k_src.shape
    assert kc.flags.c_contiguous and vc.flags.c_contiguous
    lib().orc_kv_append(k_src, v_src, kd, rows, kc, vc, kd, pos0)


# ---------------------------------------------------------------- attention
def attn_decode(q, kc, vc, T, H, HKV, D, scale=None):
    """src/model.cpp:191-214: q [H, D]; kc/vc [>=T, HKV, D]; returns [H, D]."""
    scale = np.float32(1.0) / np.sqrt(np.float32(D)) if scale is None else scale
    out = np.empty((H, D), np.float32)
    lib().orc_attn_decode(_c(q), _c(kc), _c(vc), out, T, H, HKV, D, float(scale), None)
    return out


def attn_prefill(q, kc, vc, B, pos0, H, HKV, D, scale=None):
    """Per-token loop of src/model.cpp:138-140 over src/model.cpp:191-214.
    q [B, H*D] (or [B, stride] with heads first); returns [B, H, D]."""
    scale = np.float32(1.0) / np.sqrt(np.float32(D)) if scale is None else scale
    q = _c(q).reshape(B, -1)
    out = np.empty((B, H, D), np.float32)
    lib().orc_attn_prefill(q, q.shape[1], _c(kc), _c(vc), out, B, pos0, H, HKV, D, float(scale))
    return out


def attn_decode_batched(q, kc, vc, kv_offset, kv_len, H, HKV, D, scale=None):
    scale = np.float32(1.0) / np.sqrt(np.float32(D)) if scale is None else scale
    nseq = len(kv_len)
    out = np.empty((nseq, H, D), np.float32)
    lib().orc_attn_decode_batched(_c(q), _c(kc), _c(vc), out, _c(kv_offset, np.int64), _c(kv_len, np.int32), nseq,
                                  H, HKV, D, float(scale))
    return out


def attn_split_combine(q, kc, vc, T, H, HKV, D, nsplit=16, scale=None):
    """src/cuda/model_cuda.cu:1043-1111 semantics."""
    scale = np.float32(1.0) / np.sqrt(np.float32(D)) if scale is None else scale
    out = np.empty((H, D), np.float32)
    lib().orc_attn_split_combine(_c(q), _c(kc), _c(vc), out, T, H, HKV, D, float(scale), nsplit)
    return out


def attn_f64(q, kc, vc, T, H, HKV, D, scale=None):
    scale = 1.0 / np.sqrt(np.float32(D)) if scale is None else scale
    out = np.empty((H, D), np.float64)
    lib().orc_attn_f64(_c(q), _c(kc), _c(vc), out, T, H, HKV, D, float(np.float32(scale)))
    return out


def threads() -> int:
    return int(lib().orc_threads())


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


def env_threads() -> int:
    v = os.environ.get("OMP_NUM_THREADS")
    return int(v) if v and v.isdigit() else (os.cpu_count() or 1)


# ---------------------------------------------------------------- QKV projection
W_F32, W_F16, W_Q8_0, W_Q4_K, W_Q6_K = 0, 1, 8, 12, 14
# values per block and bytes per block of the quantised row formats (src/quant.h:21-39)
QBLOCK = {W_Q8_0: (32, 34), W_Q4_K: (256, 144), W_Q6_K: (256, 210)}


def row_bytes(wtype: int, n: int) -> int:
    return int(lib().orc_row_bytes(wtype, n))


def dequant(wtype: int, blocks, n: int) -> np.ndarray:
    """A quantised row (or rows, as uint8 bytes) of n values each decoded to float32
    (src/quant.cpp:7-60); blocks holds rows * row_bytes bytes."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    out = np.empty(b.size // row_bytes(wtype, n) * n, np.float32)
    name = {W_Q8_0: "orc_dequant_q8_0", W_Q4_K: "orc_dequant_q4_K", W_Q6_K: "orc_dequant_q6_K"}[wtype]
    getattr(lib(), name)(b.ctypes.data, out, out.size)
    return out


def random_blocks(wtype: int, rows: int, n: int, seed: int, d_scale: float = 1.0) -> np.ndarray:
    """Random quantised rows [rows][row_bytes] (uint8): every byte random except the binary16
    block scales, drawn as moderate positive and negative values (d_scale x 2^-7..2^-4) so the
    decoded weights stay finite and O(d_scale)."""
    qk, bb = QBLOCK[wtype]
    rng = np.random.default_rng(seed)
    nb = rows * (n // qk)
    blk = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    def f16(k):
        v = (rng.uniform(2.0 ** -7, 2.0 ** -4, nb) * rng.choice([-1.0, 1.0], nb) * d_scale).astype(np.float16)
        return v.view(np.uint16)
    def put(off, h):
        blk[:, off] = (h & 0xFF).astype(np.uint8)
        blk[:, off + 1] = (h >> 8).astype(np.uint8)
    if wtype == W_Q8_0:
        put(0, f16(0))
    elif wtype == W_Q4_K:
        put(0, f16(0))
        put(2, np.abs(f16(1).view(np.float16)).astype(np.float16).view(np.uint16))
    else:
        put(208, f16(0))
    return blk.reshape(rows, -1)


def f16_to_f32(h) -> np.ndarray:
    """binary16 bit patterns -> float32, exact (src/ops.cpp:22-24)."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    L = lib()
    return np.array([L.orc_f16_to_f32(int(v)) for v in h.reshape(-1)], np.float32).reshape(h.shape)


def dot(w, x, wtype: int) -> float:
    """dot_f32 / dot_f16 of src/ops.cpp:92-118 (w float32, or uint16 binary16 patterns)."""
    x = _c(x)
    if wtype == W_F32:
        return float(lib().orc_dot_f32(_c(w), x, x.size))
    return float(lib().orc_dot_f16(np.ascontiguousarray(w, dtype=np.uint16), x, x.size))


def matvec(w, x, wtype: int) -> np.ndarray:
    """y = W x for W [rows][n] (src/ops.cpp:126-153): float32 weights (W_F32), binary16
    patterns as uint16 (W_F16), or quantised rows as uint8 bytes [rows][row_bytes]."""
    x = _c(x)
    n = x.size
    if wtype in QBLOCK:
        w = np.ascontiguousarray(w, dtype=np.uint8)
        rows = w.size // row_bytes(wtype, n)
    else:
        w = np.ascontiguousarray(w, dtype=np.float32 if wtype == W_F32 else np.uint16)
        rows, n = w.shape
    y = np.empty(rows, np.float32)
    lib().orc_matvec(wtype, w.ctypes.data, x, y, rows, n)
    return y


def rmsnorm_rows(x, w, eps=1e-6):
    """src/ops.cpp:155-160 on every row of x [B][n]."""
    x = np.atleast_2d(_c(x))
    return np.stack([rmsnorm(r, w, eps) for r in x])
