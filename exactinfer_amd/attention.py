"""Torch-tensor front end of the gfx950 attention path (calls the C ABI, nothing else).

Each function launches on torch's current HIP stream and validates shapes on the host
before any launch (the C ABI validates again).  Tensors are float32, contiguous in the
innermost dimension, on the GPU.

The names follow the reference's per-layer attention steps (src/cuda/model_cuda.cu:
1797-1822): headnorm_rope -> kv_append -> attn_decode (B == 1) or attn_prefill (B > 1).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _capi

HEAD_DIM = 128


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _need_gpu_f32(name: str, t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if t.dtype != torch.float32:
        raise ValueError(f"{name} must be float32, got {t.dtype}")
    if t.stride(-1) != 1:
        raise ValueError(f"{name} must be contiguous in its last dimension")


def default_scale(head_dim: int = HEAD_DIM) -> float:
    """1/sqrt(D) rounded to float as the reference does (src/model.cpp:163, src/cuda/model_cuda.cu:1786)."""
    return float(torch.tensor(1.0, dtype=torch.float32) / torch.sqrt(torch.tensor(float(head_dim),
                                                                                  dtype=torch.float32)))


@dataclass(frozen=True)
class AttnShape:
    """The Config fields the path reads (src/model.h:17-23)."""

    n_head: int
    n_head_kv: int
    head_dim: int = HEAD_DIM
    rope_dim: int = HEAD_DIM
    rope_base: float = 1e6
    eps: float = 1e-6

    @property
    def group(self) -> int:
        return self.n_head // self.n_head_kv

    @property
    def kd(self) -> int:
        return self.n_head_kv * self.head_dim

    @property
    def qkv(self) -> int:
        return (self.n_head + 2 * self.n_head_kv) * self.head_dim


# ---------------------------------------------------------------- RoPE table
def rope_table(n_ctx: int, rope_dim: int = HEAD_DIM, theta: float = 1e6, device="cuda") -> torch.Tensor:
    """[n_ctx, rope_dim/2, 2] (cos, sin) float table, angles in double (src/cuda/model_cuda.cu:1610-1619)."""
    host = torch.empty((n_ctx, rope_dim // 2, 2), dtype=torch.float32)
    _capi.call("ei_rope_table_fill", host.data_ptr(), n_ctx, rope_dim, float(theta))
    return host.to(device) if device != "cpu" else host


# ---------------------------------------------------------------- prologue
def headnorm_rope(buf: torch.Tensor, n_heads: int, gamma: torch.Tensor, cs: torch.Tensor, pos_dev: torch.Tensor,
                  rope_dim: int = HEAD_DIM, eps: float = 1e-6, rows: int | None = None) -> None:
    """In place on buf[rows, row_stride] (heads at column h*128)."""
    _need_gpu_f32("buf", buf)
    rows = buf.shape[0] if rows is None else rows
    _capi.call("ei_headnorm_rope", _stream(), buf.data_ptr(), rows, buf.stride(0), n_heads, HEAD_DIM,
               gamma.data_ptr(), cs.data_ptr(), pos_dev.data_ptr(), rope_dim, float(eps))


def kv_append(k_src: torch.Tensor, v_src: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor,
              pos_dev: torch.Tensor) -> None:
    """Copy rows of k_src/v_src ([rows, >=kd], same row stride) into cache rows *pos_dev + b."""
    for n, t in (("k_src", k_src), ("v_src", v_src), ("kc", kc), ("vc", vc)):
        _need_gpu_f32(n, t)
    if k_src.stride(0) != v_src.stride(0):
        raise ValueError("k_src and v_src must share a row stride")
    kd = kc.shape[-1] * (kc.shape[-2] if kc.dim() == 3 else 1)
    _capi.call("ei_kv_append", _stream(), k_src.data_ptr(), v_src.data_ptr(), k_src.stride(0), k_src.shape[0],
               kc.data_ptr(), vc.data_ptr(), kd, pos_dev.data_ptr())


def qkv_prepare(qkv: torch.Tensor, shape: AttnShape, q_gamma: torch.Tensor, k_gamma: torch.Tensor,
                cs: torch.Tensor, pos_dev: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor) -> None:
    """Fused QK-norm + RoPE (in place) and K/V append for a [rows, (H+2HKV)*128] buffer."""
    _need_gpu_f32("qkv", qkv)
    _capi.call("ei_qkv_prepare", _stream(), qkv.data_ptr(), qkv.shape[0], qkv.stride(0), shape.n_head,
               shape.n_head_kv, shape.head_dim, q_gamma.data_ptr(), k_gamma.data_ptr(), cs.data_ptr(),
               pos_dev.data_ptr(), shape.rope_dim, float(shape.eps), kc.data_ptr(), vc.data_ptr())


# ---------------------------------------------------------------- decode
class DecodeWorkspace:
    """Split-K partials + arrival counters, sized for (n_seq, max_kv); cleared once here."""

    def __init__(self, n_seq: int, n_head: int, n_head_kv: int, max_kv: int, device="cuda"):
        self.n_seq, self.max_kv = n_seq, max_kv
        self.nbytes = int(_capi.lib().ei_attn_decode_ws_bytes(n_seq, n_head, n_head_kv, max_kv))
        if self.nbytes == 0:
            raise ValueError("invalid decode workspace shape")
        self.buf = torch.empty(self.nbytes, dtype=torch.uint8, device=device)
        _capi.call("ei_attn_workspace_init", _stream(), self.buf.data_ptr(), self.nbytes)

    def status(self) -> int:
        """The workspace's sticky status word (uint32 at (nbytes - 256) & ~255; bit 0: the splits of one
        (sequence, KV head) ran on different XCDs, against the placement the in-kernel split
        merge relies on).  Read through ei_attn_workspace_status, which synchronises the stream."""
        import ctypes
        word = ctypes.c_uint32(0)
        _capi.call("ei_attn_workspace_status", _stream(), self.buf.data_ptr(), self.nbytes, ctypes.byref(word))
        return int(word.value)

    def check(self) -> None:
        """Raises EiError (EI_ERR_MERGE) when the status word reports a failed split-merge check."""
        _capi.call("ei_decode_status_check", self.status())


def attn_decode(q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, pos_dev: torch.Tensor, shape: AttnShape,
                ws: DecodeWorkspace, scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """q [H, 128] (normed + roped); keys 0..*pos_dev of the [n_ctx, HKV, 128] cache; returns [H, 128]."""
    _need_gpu_f32("q", q)
    out = torch.empty((shape.n_head, HEAD_DIM), dtype=torch.float32, device=q.device) if out is None else out
    scale = default_scale() if scale is None else scale
    _capi.call("ei_attn_decode", _stream(), q.data_ptr(), out.data_ptr(), kc.data_ptr(), vc.data_ptr(),
               pos_dev.data_ptr(), shape.n_head, shape.n_head_kv, shape.head_dim, float(scale), ws.max_kv,
               ws.buf.data_ptr(), ws.nbytes)
    return out


def attn_decode_batched(q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, kv_offset: torch.Tensor,
                        kv_len: torch.Tensor, shape: AttnShape, ws: DecodeWorkspace, scale: float | None = None,
                        out: torch.Tensor | None = None) -> torch.Tensor:
    """q [n_seq, H*128 (or wider rows)]; kv_offset int64 / kv_len int32 device arrays; returns [n_seq, H, 128]."""
    n_seq = kv_len.shape[0]
    out = torch.empty((n_seq, shape.n_head, HEAD_DIM), dtype=torch.float32, device=q.device) if out is None else out
    scale = default_scale() if scale is None else scale
    if kv_offset.dtype != torch.int64 or kv_len.dtype != torch.int32:
        raise ValueError("kv_offset must be int64 and kv_len int32")
    _capi.call("ei_attn_decode_batched", _stream(), q.data_ptr(), q.stride(0), out.data_ptr(), kc.data_ptr(),
               vc.data_ptr(), kv_offset.data_ptr(), kv_len.data_ptr(), n_seq, shape.n_head, shape.n_head_kv,
               shape.head_dim, float(scale), ws.max_kv, ws.buf.data_ptr(), ws.nbytes)
    return out


def decode_step(qkv: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, shape: AttnShape, q_gamma: torch.Tensor,
                k_gamma: torch.Tensor, cs: torch.Tensor, ws: DecodeWorkspace, pos_dev: torch.Tensor | None = None,
                kv_offset: torch.Tensor | None = None, kv_len: torch.Tensor | None = None,
                scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Fused one-token step: norm+RoPE, KV append, attention.  qkv [n_seq, (H+2HKV)*128]."""
    _need_gpu_f32("qkv", qkv)
    n_seq = qkv.shape[0] if qkv.dim() == 2 else 1
    out = torch.empty((n_seq, shape.n_head, HEAD_DIM), dtype=torch.float32, device=qkv.device) if out is None else out
    scale = default_scale() if scale is None else scale
    _capi.call("ei_decode_step", _stream(), qkv.data_ptr(), qkv.stride(0) if qkv.dim() == 2 else shape.qkv,
               out.data_ptr(), kc.data_ptr(), vc.data_ptr(), _ptr(kv_offset), _ptr(kv_len), _ptr(pos_dev), n_seq,
               shape.n_head, shape.n_head_kv, shape.head_dim, q_gamma.data_ptr(), k_gamma.data_ptr(),
               cs.data_ptr(), shape.rope_dim, float(shape.eps), float(scale), ws.max_kv, ws.buf.data_ptr(),
               ws.nbytes)
    return out


def attn_decode_paged(q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, block_table: torch.Tensor,
                      block_size: int, kv_len: torch.Tensor, shape: AttnShape, ws: DecodeWorkspace,
                      scale: float | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Paged multi-sequence decode: block_table int32 [n_seq, max_blocks] of physical blocks of
    `block_size` rows in the pool kc/vc; q [n_seq, >= H*128]; returns [n_seq, H, 128]."""
    _need_gpu_f32("q", q)
    n_seq, max_blocks = block_table.shape
    out = torch.empty((n_seq, shape.n_head, HEAD_DIM), dtype=torch.float32, device=q.device) if out is None else out
    scale = default_scale() if scale is None else scale
    _capi.call("ei_attn_decode_paged", _stream(), q.data_ptr(), q.stride(0), out.data_ptr(), kc.data_ptr(),
               vc.data_ptr(), block_table.data_ptr(), max_blocks, block_size, kv_len.data_ptr(), n_seq, shape.n_head,
               shape.n_head_kv, shape.head_dim, float(scale), ws.max_kv, ws.buf.data_ptr(), ws.nbytes)
    return out


def decode_step_paged(qkv: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, block_table: torch.Tensor,
                      block_size: int, kv_len: torch.Tensor, shape: AttnShape, q_gamma: torch.Tensor,
                      k_gamma: torch.Tensor, cs: torch.Tensor, ws: DecodeWorkspace, scale: float | None = None,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """Fused paged step: per sequence s, norm+RoPE at position kv_len[s]-1, append to its
    physical row, attention over its kv_len[s] keys.  qkv [n_seq, (H+2HKV)*128]."""
    _need_gpu_f32("qkv", qkv)
    n_seq, max_blocks = block_table.shape
    out = torch.empty((n_seq, shape.n_head, HEAD_DIM), dtype=torch.float32, device=qkv.device) if out is None else out
    scale = default_scale() if scale is None else scale
    _capi.call("ei_decode_step_paged", _stream(), qkv.data_ptr(), qkv.stride(0), out.data_ptr(), kc.data_ptr(),
               vc.data_ptr(), block_table.data_ptr(), max_blocks, block_size, kv_len.data_ptr(), n_seq, shape.n_head,
               shape.n_head_kv, shape.head_dim, q_gamma.data_ptr(), k_gamma.data_ptr(), cs.data_ptr(),
               shape.rope_dim, float(shape.eps), float(scale), ws.max_kv, ws.buf.data_ptr(), ws.nbytes)
    return out


# ---------------------------------------------------------------- prefill
class PrefillWorkspace:
    """Key-split shares for ei_attn_prefill_split / ei_prefill_step: serves chunks of up to max_B
    rows with pos0 + B <= max_kv (max_kv only steers the split plan; larger positions stay correct)."""

    def __init__(self, max_B: int, n_head: int, n_head_kv: int, max_kv: int, device="cuda"):
        self.max_B, self.max_kv = max_B, max_kv
        self.nbytes = int(_capi.lib().ei_attn_prefill_ws_bytes(max_B, n_head, n_head_kv, max_kv))
        self.buf = torch.empty(max(self.nbytes, 256), dtype=torch.uint8, device=device)


def attn_prefill(q: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, pos_dev: torch.Tensor, shape: AttnShape,
                 B: int | None = None, scale: float | None = None, out: torch.Tensor | None = None,
                 ws: PrefillWorkspace | None = None) -> torch.Tensor:
    """q rows [B, >= H*128] (normed + roped, heads first); returns [B, H, 128].
    With `ws` the key range is split over workgroups for short chunks (ei_attn_prefill_split)."""
    _need_gpu_f32("q", q)
    B = q.shape[0] if B is None else B
    out = torch.empty((B, shape.n_head, HEAD_DIM), dtype=torch.float32, device=q.device) if out is None else out
    scale = default_scale() if scale is None else scale
    if ws is None:
        _capi.call("ei_attn_prefill", _stream(), q.data_ptr(), q.stride(0), out.data_ptr(), kc.data_ptr(),
                   vc.data_ptr(), pos_dev.data_ptr(), B, shape.n_head, shape.n_head_kv, shape.head_dim, float(scale))
    else:
        if B > ws.max_B:
            raise ValueError(f"prefill workspace serves chunks of up to {ws.max_B} rows, got B={B}")
        _capi.call("ei_attn_prefill_split", _stream(), q.data_ptr(), q.stride(0), out.data_ptr(), kc.data_ptr(),
                   vc.data_ptr(), pos_dev.data_ptr(), B, shape.n_head, shape.n_head_kv, shape.head_dim, float(scale),
                   ws.max_kv, ws.buf.data_ptr(), ws.nbytes)
    return out


def prefill_step(qkv: torch.Tensor, kc: torch.Tensor, vc: torch.Tensor, shape: AttnShape, q_gamma: torch.Tensor,
                 k_gamma: torch.Tensor, cs: torch.Tensor, pos_dev: torch.Tensor, ws: PrefillWorkspace,
                 B: int | None = None, scale: float | None = None, out: torch.Tensor | None = None,
                 block_table: torch.Tensor | None = None, block_size: int = 0) -> torch.Tensor:
    """Fused chunk step (ei_prefill_step): K heads normed + roped in place and appended with V
    at rows pos..pos+B-1; Q heads left raw in qkv and normed inside the attention kernel.
    qkv [B, >= (H+2HKV)*128]; returns [B, H, 128].  With block_table (int32 [max_blocks]) the
    caches are a paged pool of block_size-row blocks (ei_prefill_step_paged)."""
    _need_gpu_f32("qkv", qkv)
    B = qkv.shape[0] if B is None else B
    if B > ws.max_B:
        raise ValueError(f"prefill workspace serves chunks of up to {ws.max_B} rows, got B={B}")
    out = torch.empty((B, shape.n_head, HEAD_DIM), dtype=torch.float32, device=qkv.device) if out is None else out
    scale = default_scale() if scale is None else scale
    tail = (q_gamma.data_ptr(), k_gamma.data_ptr(), cs.data_ptr(), shape.rope_dim, float(shape.eps), float(scale),
            ws.max_kv, ws.buf.data_ptr(), ws.nbytes)
    if block_table is None:
        _capi.call("ei_prefill_step", _stream(), qkv.data_ptr(), qkv.stride(0), out.data_ptr(), kc.data_ptr(),
                   vc.data_ptr(), pos_dev.data_ptr(), B, shape.n_head, shape.n_head_kv, shape.head_dim, *tail)
    else:
        _capi.call("ei_prefill_step_paged", _stream(), qkv.data_ptr(), qkv.stride(0), out.data_ptr(), kc.data_ptr(),
                   vc.data_ptr(), block_table.data_ptr(), block_table.numel(), block_size, pos_dev.data_ptr(), B,
                   shape.n_head, shape.n_head_kv, shape.head_dim, *tail)
    return out


# ---------------------------------------------------------------- synthetic inputs
def synth_fill(t: torch.Tensor, seed: int, offset: int = 0, row_len: int = 1, spike_every: int = 0,
               spike_mult: float = 1.0) -> torch.Tensor:
    """Fill a contiguous float32 GPU tensor with the counter-based N(0,1) stream (in place)."""
    _need_gpu_f32("t", t)
    if not t.is_contiguous():
        raise ValueError("t must be contiguous")
    _capi.call("ei_synth_fill", _stream(), t.data_ptr(), t.numel(), seed, offset, row_len, spike_every,
               float(spike_mult))
    return t


def flops_causal(T_new: int, pos0: int, n_head: int, head_dim: int = HEAD_DIM) -> float:
    """Algorithmic FLOPs of causal attention: 4*D per visible (query, key) pair, per head."""
    pairs = sum(pos0 + b + 1 for b in range(T_new)) if T_new < 64 else T_new * pos0 + T_new * (T_new + 1) // 2
    return 4.0 * head_dim * pairs * n_head


def decode_bytes(kv_len: int, n_head: int, n_head_kv: int, head_dim: int = HEAD_DIM) -> float:
    """Algorithmic HBM bytes of one decode: the visible K and V rows plus q and out."""
    return 4.0 * (2 * kv_len * n_head_kv * head_dim + 2 * n_head * head_dim)


__all__ = [
    "AttnShape", "DecodeWorkspace", "attn_decode", "attn_decode_batched", "attn_prefill", "decode_step",
    "default_scale", "headnorm_rope", "kv_append", "qkv_prepare", "rope_table", "synth_fill", "flops_causal",
    "decode_bytes",
]
