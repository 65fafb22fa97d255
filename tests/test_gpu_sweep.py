"""Seeded random sweep of the fused entry points against the CPU oracle (GPU).

Each case draws its own shape from its seed, so the sweep covers combinations the hand-picked
tests do not: GQA groups 1..8 (the padded 3, 5, 6, 7 included) over 1, 2, 4 or 8 KV heads;
decode lengths from 1 to ~9000 keys with a workspace planned for up to twice that (so the
split plan, the last split's extra keys and both merge paths all occur); ragged batches with
empty sequences; prefill chunks of 1..300 rows at positions up to ~2000 with key-split plans
from 1 to 8 shares.  Bars as everywhere: cache rows and normed K bit-exact, attention within
the 1e-5 parity gate (tests/parity.py), every case recorded in the evidence table.
"""
import os

import numpy as np
import pytest

from tests.parity import bits_equal, gate

pytestmark = pytest.mark.gpu

D = 128
# EI_SWEEP_EXTRA=n adds seeds 100 .. 100+n-1 to each sweep (ragged: every other one), an extended run on demand
_EXTRA = int(os.environ.get("EI_SWEEP_EXTRA", "0"))


def _seeds(n):
    return list(range(n)) + list(range(100, 100 + _EXTRA))


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def _pos(p):
    import torch
    return torch.tensor([p], dtype=torch.int32, device="cuda")


def _heads(rng):
    HKV = int(rng.choice([1, 2, 4, 8]))
    G = int(rng.integers(1, 9))
    return G * HKV, HKV


@pytest.mark.parametrize("seed", _seeds(24))
def test_sweep_fused_decode(orc, gpu, seed):
    rng = np.random.default_rng(20000 + seed)
    H, HKV = _heads(rng)
    T = int(rng.choice([int(rng.integers(1, 300)), int(rng.integers(300, 9000))]))
    max_kv = int(rng.integers(max(T // 2, 1), 2 * T + 2))  # below T: the last split takes the extra keys
    n_ctx = max(T, max_kv) + 1
    shape = gpu.AttnShape(H, HKV)
    k = orc.normal((n_ctx, HKV * D), 20100 + seed)
    v = orc.normal((n_ctx, HKV * D), 20200 + seed)
    qkv = orc.normal((1, shape.qkv), 20300 + seed) * np.float32(2.0)
    qg, kg = orc.gamma(D, 20400 + seed), orc.gamma(D, 20500 + seed)
    cs = gpu.rope_table(n_ctx)
    kc, vc = _dev(k), _dev(v)
    ws = gpu.DecodeWorkspace(1, H, HKV, max_kv=max_kv)
    pos = T - 1
    out = _host(gpu.decode_step(_dev(qkv), kc, vc, shape, _dev(qg), _dev(kg), cs, ws, pos_dev=_pos(pos)))
    normed = orc.headnorm_rope(qkv, H, D, qg, pos, 128, 1e6, 1e-6)
    normed = orc.headnorm_rope(normed, HKV, D, kg, pos, 128, 1e6, 1e-6, col0=H * D)
    rk, rv = k.copy(), v.copy()
    orc.kv_append(normed[:, H * D:(H + HKV) * D], normed[:, (H + HKV) * D:], rk, rv, pos)
    assert bits_equal(_host(kc), rk) and bits_equal(_host(vc), rv)
    qn = np.ascontiguousarray(normed[0, :H * D].reshape(H, D))
    kk, vv = rk.reshape(n_ctx, HKV, D), rv.reshape(n_ctx, HKV, D)
    ok, msg = gate(f"sweep decode seed {seed} H{H}/HKV{HKV} T={T} max_kv={max_kv}", out.reshape(H, D),
                   orc.attn_decode(qn, kk, vv, T, H, HKV, D), lambda: orc.attn_f64(qn, kk, vv, T, H, HKV, D))
    assert ok, msg
    assert ws.status() == 0


@pytest.mark.parametrize("seed", [s for s in _seeds(12) if s < 100 or s % 2 == 0])
def test_sweep_ragged_decode_step(orc, gpu, seed):
    """ei_decode_step over a contiguous pool: sequence s owns rows off_s .. off_s + len_s - 1 and
    appends its new row at the last of them; sequences of length 0 give zeros and write nothing."""
    rng = np.random.default_rng(21000 + seed)
    H, HKV = _heads(rng)
    n_seq = int(rng.integers(1, 25))
    lens = rng.integers(0, 2500, n_seq).astype(np.int32)
    lens[rng.random(n_seq) < 0.15] = 0
    offs = np.concatenate([[0], np.cumsum(lens.astype(np.int64) + 3)[:-1]]).astype(np.int64)
    rows = int(offs[-1] + lens[-1] + 3)
    shape = gpu.AttnShape(H, HKV)
    k = orc.normal((rows, HKV * D), 21100 + seed)
    v = orc.normal((rows, HKV * D), 21200 + seed)
    qkv = orc.normal((n_seq, shape.qkv), 21300 + seed)
    qg, kg = orc.gamma(D, 21400 + seed), orc.gamma(D, 21500 + seed)
    max_kv = int(max(lens.max(), 1))
    cs = gpu.rope_table(max_kv + 1)
    kc, vc = _dev(k), _dev(v)
    ws = gpu.DecodeWorkspace(n_seq, H, HKV, max_kv=max_kv)
    out = _host(gpu.decode_step(_dev(qkv), kc, vc, shape, _dev(qg), _dev(kg), cs, ws,
                                kv_offset=_dev(offs), kv_len=_dev(lens)))
    rk, rv = k.copy(), v.copy()
    for s in range(n_seq):
        n = int(lens[s])
        if n == 0:
            assert not np.any(out[s]), f"sequence {s} of length 0"
            continue
        normed = orc.headnorm_rope(qkv[s:s + 1], H, D, qg, n - 1, 128, 1e6, 1e-6)
        normed = orc.headnorm_rope(normed, HKV, D, kg, n - 1, 128, 1e6, 1e-6, col0=H * D)
        o = int(offs[s])
        seg_k, seg_v = rk[o:o + n], rv[o:o + n]
        orc.kv_append(normed[:, H * D:(H + HKV) * D], normed[:, (H + HKV) * D:], seg_k, seg_v, n - 1)
        qn = np.ascontiguousarray(normed[0, :H * D].reshape(H, D))
        kk, vv = seg_k.reshape(n, HKV, D), seg_v.reshape(n, HKV, D)
        ok, msg = gate(f"sweep ragged seed {seed} seq {s} H{H}/HKV{HKV} len {n}", out[s],
                       orc.attn_decode(qn, kk, vv, n, H, HKV, D), lambda: orc.attn_f64(qn, kk, vv, n, H, HKV, D))
        assert ok, msg
    assert bits_equal(_host(kc), rk) and bits_equal(_host(vc), rv)
    assert ws.status() == 0


@pytest.mark.parametrize("seed", _seeds(16))
def test_sweep_prefill_step(orc, gpu, seed):
    rng = np.random.default_rng(22000 + seed)
    H, HKV = _heads(rng)
    B = int(rng.integers(1, 301))
    pos0 = int(rng.choice([0, int(rng.integers(1, 2000))]))
    max_kv = pos0 + B + int(rng.integers(0, 2000))
    n_ctx = max_kv
    shape = gpu.AttnShape(H, HKV)
    k = orc.normal((n_ctx, HKV * D), 22100 + seed)
    v = orc.normal((n_ctx, HKV * D), 22200 + seed)
    qkv = orc.normal((B, shape.qkv), 22300 + seed)
    qg, kg = orc.gamma(D, 22400 + seed), orc.gamma(D, 22500 + seed)
    cs = gpu.rope_table(n_ctx)
    kc, vc = _dev(k), _dev(v)
    buf = _dev(qkv)
    ws = gpu.PrefillWorkspace(B, H, HKV, max_kv)
    out = _host(gpu.prefill_step(buf, kc, vc, shape, _dev(qg), _dev(kg), cs, _pos(pos0), ws))
    normed = orc.headnorm_rope(qkv, H, D, qg, pos0, 128, 1e6, 1e-6)
    normed = orc.headnorm_rope(normed, HKV, D, kg, pos0, 128, 1e6, 1e-6, col0=H * D)
    rk, rv = k.copy(), v.copy()
    orc.kv_append(normed[:, H * D:(H + HKV) * D], normed[:, (H + HKV) * D:], rk, rv, pos0)
    assert bits_equal(_host(kc), rk) and bits_equal(_host(vc), rv)
    qn = np.ascontiguousarray(normed[:, :H * D])
    kk, vv = rk.reshape(n_ctx, HKV, D), rv.reshape(n_ctx, HKV, D)
    ref = orc.attn_prefill(qn, kk, vv, B, pos0, H, HKV, D)
    ok, msg = gate(f"sweep prefill step seed {seed} H{H}/HKV{HKV} B={B} pos0={pos0} max_kv={max_kv}", out, ref,
                   lambda: np.stack([orc.attn_f64(qn[b].reshape(H, D), rk, rv, pos0 + b + 1, H, HKV, D)
                                     for b in range(B)]))
    assert ok, msg
