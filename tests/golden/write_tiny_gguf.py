"""Writes a tiny synthetic Qwen3 model as a GGUF file (test infrastructure).

No Qwen3 GGUF exists in this environment, so the reader and the end-to-end harness are exercised
on files this script writes from tests/tiny_qwen3.py's seeded random weights: the tensor names,
shapes and metadata keys a Qwen3 GGUF carries (read_config / read_tensors, src/model.cpp:38-103),
F32 or F16 weights (norm vectors stay F32), or any tensor given as raw GGML blocks (Quantised),
GGUF version 3, the data section aligned to general.alignment.  The writer is independent of the reader under test (plain struct packing).

    python tests/golden/write_tiny_gguf.py OUT.gguf [--f16] [--seed N]
"""
from __future__ import annotations

import argparse
import struct
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

T_U32, T_I32, T_F32, T_STRING, T_ARRAY, T_U64, T_F64 = 4, 5, 6, 8, 9, 10, 12


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _val(t: int, value) -> bytes:
    if t == T_STRING:
        return _s(value)
    if t == T_ARRAY:  # value = (element type, list of elements)
        et, items = value
        return struct.pack("<IQ", et, len(items)) + b"".join(_val(et, x) for x in items)
    fmt = {0: "<B", 1: "<b", 2: "<H", 3: "<h", T_U32: "<I", T_I32: "<i", T_F32: "<f", 7: "<B", T_U64: "<Q",
           11: "<q", T_F64: "<d"}[t]
    return struct.pack(fmt, value)


def _kv(key: str, t: int, value) -> bytes:
    return _s(key) + struct.pack("<I", t) + _val(t, value)


def quantize_q8_0(a: np.ndarray) -> np.ndarray:
    """Rows of a float matrix [rows][n] (n a multiple of 32) as Q8_0 blocks, uint8 [rows][n/32*34]:
    per block of 32, d = max|x| / 127 stored as binary16 and q = round(x / d) in [-127, 127]."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    rows, n = a.shape
    blk = a.reshape(rows, n // 32, 32)
    d16 = (np.abs(blk).max(axis=2) / 127.0).astype(np.float16)
    d = d16.astype(np.float32)
    inv = np.where(d > 0, 1.0 / np.where(d > 0, d, 1.0), 0.0).astype(np.float32)
    q = np.clip(np.rint(blk * inv[..., None]), -127, 127).astype(np.int8)
    out = np.empty((rows, n // 32, 34), np.uint8)
    out[..., :2] = d16.view(np.uint8).reshape(rows, n // 32, 2)
    out[..., 2:] = q.view(np.uint8)
    return out.reshape(rows, -1)


def _f16_bytes(v: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(v, dtype=np.float16).view(np.uint8).reshape(*v.shape, 2)


def quantize_q4_k(a: np.ndarray) -> np.ndarray:
    """Rows [rows][n] (n a multiple of 256) as Q4_K blocks, uint8 [rows][n/256*144].  A plain
    encoder (not llama.cpp's search): sub-block j of 32 values gets y = dl_j q - ml_j with
    ml_j = -min(0, min x) and dl_j = (max x + ml_j) / 15; dl_j and ml_j are 6-bit multiples of
    the block's d and dmin (binary16), q = round((x + ml) / dl) in 0..15.  Layout as the decoder
    reads it (src/quant.cpp:15-33, the scale packing of src/quant.h:43-52): d, dmin, 12 packed
    scale bytes, then 4 chunks of 32 bytes whose low nibbles hold sub-block 2c, high 2c+1."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    rows, n = a.shape
    nb = rows * (n // 256)
    x = a.reshape(nb, 8, 32)
    ml = -np.minimum(x.min(axis=2), 0.0)
    dl = (x.max(axis=2) + ml) / 15.0
    d16 = (dl.max(axis=1) / 63.0).astype(np.float16)
    m16 = (ml.max(axis=1) / 63.0).astype(np.float16)
    d, dm = d16.astype(np.float32), m16.astype(np.float32)
    safe = lambda v: np.where(v > 0, v, 1.0)
    sc = np.where(d[:, None] > 0, np.clip(np.rint(dl / safe(d)[:, None]), 0, 63), 0).astype(np.int32)
    mq = np.where(dm[:, None] > 0, np.clip(np.rint(ml / safe(dm)[:, None]), 0, 63), 0).astype(np.int32)
    dle = d[:, None] * sc.astype(np.float32)
    mle = dm[:, None] * mq.astype(np.float32)
    q = np.where(dle[..., None] > 0, np.rint((x + mle[..., None]) / safe(dle)[..., None]), 0)
    q = np.clip(q, 0, 15).astype(np.uint8)
    out = np.zeros((nb, 144), np.uint8)
    out[:, 0:2] = _f16_bytes(d16)
    out[:, 2:4] = _f16_bytes(m16)
    scb = np.zeros((nb, 12), np.int32)
    for j in range(4):
        scb[:, j] = (sc[:, j] & 63) | ((sc[:, j + 4] >> 4) << 6)
        scb[:, j + 4] = (mq[:, j] & 63) | ((mq[:, j + 4] >> 4) << 6)
        scb[:, j + 8] = (sc[:, j + 4] & 15) | ((mq[:, j + 4] & 15) << 4)
    out[:, 4:16] = scb.astype(np.uint8)
    for c in range(4):
        out[:, 16 + 32 * c:48 + 32 * c] = q[:, 2 * c] | (q[:, 2 * c + 1] << 4)
    return out.reshape(rows, -1)


def quantize_q6_k(a: np.ndarray) -> np.ndarray:
    """Rows [rows][n] (n a multiple of 256) as Q6_K blocks, uint8 [rows][n/256*210].  A plain
    encoder: each group of 16 values gets y = d sc (q - 32) with sc an int8 multiple of the
    block's d (binary16) and q = round(x / (d sc)) + 32 in 0..63.  Layout as the decoder reads
    it (src/quant.cpp:35-60): value v of half h = v / 128, g = (v / 32) % 4, l = v % 32 keeps
    its low 4 bits in ql[64 h + 32 (g % 2) + l] (high nibble when g >= 2), its top 2 bits in
    qh[32 h + l] at bit 2 g, and its scale in scales[8 h + 2 g + l / 16]."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    rows, n = a.shape
    nb = rows * (n // 256)
    x = a.reshape(nb, 256)
    v = np.arange(256)
    h, g, l = v // 128, (v // 32) % 4, v % 32
    sidx = 8 * h + 2 * g + l // 16  # scale index of every value
    amax = np.zeros((nb, 16), np.float32)
    for i in range(16):
        amax[:, i] = np.abs(x[:, sidx == i]).max(axis=1)
    s = amax / 31.0
    d16 = (s.max(axis=1) / 127.0).astype(np.float16)
    d = d16.astype(np.float32)
    safe = lambda t: np.where(t > 0, t, 1.0)
    sc = np.where(d[:, None] > 0, np.clip(np.rint(s / safe(d)[:, None]), 0, 127), 0).astype(np.int32)
    step = (d[:, None] * sc.astype(np.float32))[:, sidx]
    q = np.where(step > 0, np.rint(x / safe(step)), 0)
    q = (np.clip(q, -32, 31) + 32).astype(np.int32)
    out = np.zeros((nb, 210), np.uint8)
    ql = np.zeros((nb, 128), np.int32)
    qh = np.zeros((nb, 64), np.int32)
    for vi in range(256):
        hh, gg, ll = int(h[vi]), int(g[vi]), int(l[vi])
        ql[:, 64 * hh + 32 * (gg & 1) + ll] |= (q[:, vi] & 15) << (4 * (gg >> 1))
        qh[:, 32 * hh + ll] |= (q[:, vi] >> 4) << (2 * gg)
    out[:, 0:128] = ql.astype(np.uint8)
    out[:, 128:192] = qh.astype(np.uint8)
    out[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    out[:, 208:210] = _f16_bytes(d16)
    return out.reshape(rows, -1)


QUANTIZERS = {"q8_0": (8, quantize_q8_0), "q4_k": (12, quantize_q4_k), "q6_k": (14, quantize_q6_k)}


def qwen3_tensors(model, f16: bool, q8_attn: bool = False, attn_type: str | None = None) -> list[tuple[str, np.ndarray]]:
    """(GGUF name, array with ne[0] as its last axis) in file order; matrices F16 when f16; the
    attention projections Wq, Wk, Wv as blocks of attn_type ("q8_0", "q4_k", "q6_k"; q8_attn is
    attn_type "q8_0")."""
    D = 128
    mat = (lambda a: np.ascontiguousarray(a, dtype=np.float16)) if f16 else (
        lambda a: np.ascontiguousarray(a, dtype=np.float32))
    vec = lambda a: np.ascontiguousarray(a, dtype=np.float32)
    if q8_attn:
        attn_type = "q8_0"
    if attn_type:
        tid, quant = QUANTIZERS[attn_type]
        attn = lambda a: Quantised(tid, (a.shape[1], a.shape[0]), quant(a))
    else:
        attn = mat
    QD, KD = model.H * D, model.HKV * D
    out = [("token_embd.weight", mat(model.emb)), ("output_norm.weight", vec(model.out_norm)),
           ("output.weight", mat(model.lm))]
    for l, L in enumerate(model.layers):
        b = f"blk.{l}."
        out += [(b + "attn_norm.weight", vec(L["attn_norm"])),
                (b + "attn_q.weight", attn(L["wqkv"][:QD])),
                (b + "attn_k.weight", attn(L["wqkv"][QD:QD + KD])),
                (b + "attn_v.weight", attn(L["wqkv"][QD + KD:])),
                (b + "attn_q_norm.weight", vec(L["q_norm"])),
                (b + "attn_k_norm.weight", vec(L["k_norm"])),
                (b + "attn_output.weight", mat(L["wo"])),
                (b + "ffn_norm.weight", vec(L["ffn_norm"])),
                (b + "ffn_gate.weight", mat(L["wg"])),
                (b + "ffn_up.weight", mat(L["wu"])),
                (b + "ffn_down.weight", mat(L["wd"]))]
    return out


def qwen3_metadata(model, n_ctx: int = 4096, alignment: int = 32) -> list[tuple[str, int, object]]:
    return [("general.architecture", T_STRING, "qwen3"),
            ("general.name", T_STRING, "tiny synthetic qwen3"),
            ("general.alignment", T_U32, alignment),
            ("qwen3.block_count", T_U32, model.n_layer),
            ("qwen3.context_length", T_U32, n_ctx),
            ("qwen3.embedding_length", T_U32, model.E),
            ("qwen3.feed_forward_length", T_U32, model.layers[0]["wg"].shape[0]),
            ("qwen3.attention.head_count", T_U32, model.H),
            ("qwen3.attention.head_count_kv", T_U32, model.HKV),
            ("qwen3.attention.key_length", T_U32, 128),
            ("qwen3.attention.value_length", T_U32, 128),
            ("qwen3.rope.dimension_count", T_U32, 128),
            ("qwen3.rope.freq_base", T_F32, 1e6),
            ("qwen3.attention.layer_norm_rms_epsilon", T_F32, 1e-6)]


class Quantised:
    """A tensor stored in a GGML block format: its type id, ne (ne[0] contiguous) and raw bytes
    (rows of ne[0] / block_size blocks)."""

    def __init__(self, type_id: int, ne, data: np.ndarray):
        self.type_id, self.ne = type_id, tuple(int(n) for n in ne)
        self.data = np.ascontiguousarray(data, dtype=np.uint8)
        self.nbytes = self.data.nbytes

    def tobytes(self) -> bytes:
        return self.data.tobytes()


def _type_and_ne(a):
    if isinstance(a, Quantised):
        return a.type_id, a.ne
    return (1 if a.dtype == np.float16 else 0), a.shape[::-1]


def write_gguf(path, metadata, tensors, alignment: int = 32, version: int = 3) -> None:
    """metadata: (key, type id, value); tensors: (name, array) with ne = array.shape[::-1], or
    (name, Quantised)."""
    head = struct.pack("<IIQQ", 0x46554747, version, len(tensors), len(metadata))
    head += b"".join(_kv(k, t, v) for k, t, v in metadata)
    offsets, off = [], 0
    for _, a in tensors:
        offsets.append(off)
        off += (a.nbytes + alignment - 1) // alignment * alignment
    for (name, a), o in zip(tensors, offsets):
        ty, ne = _type_and_ne(a)
        head += _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", ty, o)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        for (_, a), o in zip(tensors, offsets):
            b = a.tobytes()
            f.write(b + b"\0" * ((-len(b)) % alignment))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("out")
    ap.add_argument("--f16", action="store_true")
    ap.add_argument("--seed", type=int, default=7)
    a = ap.parse_args()
    from tests.tiny_qwen3 import TinyQwen3
    model = TinyQwen3(seed=a.seed)
    write_gguf(a.out, qwen3_metadata(model), qwen3_tensors(model, a.f16))
    print("wrote", a.out)


if __name__ == "__main__":
    main()
