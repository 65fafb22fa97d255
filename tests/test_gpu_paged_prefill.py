"""GPU tests of the paged prefill step (ei_prefill_step_paged) against the contiguous path.

The pool holds the sequence's keys in shuffled blocks, with spare blocks in between that belong
to nobody.  The paged step (full prologue, then the plain attention kernel over the block table)
must give bit for bit what the contiguous path gives on the same keys: ei_qkv_prepare followed by
ei_attn_prefill_split with the same plan (the same kernels, the same tile order, only the row
addresses differ).  The pool's rows of the sequence must equal the contiguous cache rows after
the append, and the spare blocks must be untouched.  Each case is also held to the 1e-5 parity
gate against the CPU oracle.
"""
import numpy as np
import pytest

from tests.parity import bits_equal, gate

pytestmark = pytest.mark.gpu

D = 128


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


def _pool(rng, n_ctx, bs, kd, k, v, spare=3):
    """Blocks of the sequence in shuffled order among `spare` extra blocks; returns the table,
    the pools and the physical row of every logical row."""
    nblk = (n_ctx + bs - 1) // bs
    phys_blocks = rng.permutation(nblk + spare)[:nblk].astype(np.int32)
    rows = (phys_blocks[np.arange(n_ctx) // bs] * bs + np.arange(n_ctx) % bs).astype(np.int64)
    total = (nblk + spare) * bs
    pk = rng.standard_normal((total, kd)).astype(np.float32)  # spare rows: noise that must survive
    pv = rng.standard_normal((total, kd)).astype(np.float32)
    pk[rows], pv[rows] = k, v
    return phys_blocks, pk, pv, rows


@pytest.mark.parametrize("H,HKV,B,pos0,max_kv,bs", [(32, 8, 512, 1536, 2048, 64), (16, 8, 100, 37, 256, 32),
                                                    (32, 8, 77, 3000, 4096, 128), (8, 1, 300, 0, 512, 32),
                                                    (40, 8, 64, 1000, 2048, 256), (16, 8, 1, 500, 1024, 32),
                                                    (12, 4, 200, 64, 300, 64)])
def test_paged_prefill_step_equals_contiguous(orc, gpu, H, HKV, B, pos0, max_kv, bs):
    rng = np.random.default_rng(23000 + B + pos0)
    shape = gpu.AttnShape(H, HKV)
    kd = HKV * D
    n_ctx = max(max_kv, pos0 + B)
    k = orc.normal((n_ctx, kd), 23100 + B)
    v = orc.normal((n_ctx, kd), 23200 + B)
    qkv = orc.normal((B, shape.qkv), 23300 + pos0)
    qg, kg = orc.gamma(D, 23400), orc.gamma(D, 23500)
    cs = gpu.rope_table(n_ctx)
    table, pk, pv, rows = _pool(rng, n_ctx, bs, kd, k, v)
    pos = _pos(pos0)
    # contiguous reference run: full prologue, then the split prefill with the same plan
    kc, vc, buf_c = _dev(k), _dev(v), _dev(qkv)
    ws_c = gpu.PrefillWorkspace(B, H, HKV, max_kv)
    gpu.qkv_prepare(buf_c, shape, _dev(qg), _dev(kg), cs, pos, kc, vc)
    out_c = _host(gpu.attn_prefill(buf_c, kc, vc, pos, shape, ws=ws_c))
    # paged run
    pkd, pvd, buf_p = _dev(pk), _dev(pv), _dev(qkv)
    ws_p = gpu.PrefillWorkspace(B, H, HKV, max_kv)
    out_p = _host(gpu.prefill_step(buf_p, pkd, pvd, shape, _dev(qg), _dev(kg), cs, pos, ws_p,
                                   block_table=_dev(table), block_size=bs))
    assert bits_equal(out_p, out_c)
    assert bits_equal(_host(buf_p), _host(buf_c))
    pk_after, pv_after = _host(pkd), _host(pvd)
    assert bits_equal(pk_after[rows], _host(kc)) and bits_equal(pv_after[rows], _host(vc))
    spare = np.setdiff1d(np.arange(pk.shape[0]), rows)
    assert bits_equal(pk_after[spare], pk[spare]) and bits_equal(pv_after[spare], pv[spare])
    # and the oracle
    normed = orc.headnorm_rope(qkv, H, D, qg, pos0, 128, 1e6, 1e-6)
    normed = orc.headnorm_rope(normed, HKV, D, kg, pos0, 128, 1e6, 1e-6, col0=H * D)
    rk, rv = k.copy(), v.copy()
    orc.kv_append(normed[:, H * D:(H + HKV) * D], normed[:, (H + HKV) * D:], rk, rv, pos0)
    qn = np.ascontiguousarray(normed[:, :H * D])
    ref = orc.attn_prefill(qn, rk.reshape(n_ctx, HKV, D), rv.reshape(n_ctx, HKV, D), B, pos0, H, HKV, D)
    ok, msg = gate(f"paged prefill step H{H}/HKV{HKV} B={B} pos0={pos0} bs={bs}", out_p, ref,
                   lambda: np.stack([orc.attn_f64(qn[b].reshape(H, D), rk, rv, pos0 + b + 1, H, HKV, D)
                                     for b in range(B)]))
    assert ok, msg


def test_paged_prefill_then_paged_decode(orc, gpu):
    """A prompt in two paged chunks, then paged decode steps on the same pool: the serving path
    with every row in blocks, against the contiguous engine path on the same inputs."""
    H, HKV, bs = 16, 8, 64
    shape = gpu.AttnShape(H, HKV)
    kd = HKV * D
    chunks, n_dec = [300, 212], 6
    n_ctx = sum(chunks) + n_dec
    rng = np.random.default_rng(24000)
    qkv_all = orc.normal((n_ctx, shape.qkv), 24100)
    qg, kg = orc.gamma(D, 24200), orc.gamma(D, 24300)
    cs = gpu.rope_table(n_ctx)
    zeros = np.zeros((n_ctx, kd), np.float32)
    table, pk, pv, rows = _pool(rng, n_ctx, bs, kd, zeros, zeros)
    kc, vc = _dev(zeros), _dev(zeros)
    pkd, pvd, tab = _dev(pk), _dev(pv), _dev(table)
    ws_c, ws_p = gpu.PrefillWorkspace(max(chunks), H, HKV, n_ctx), gpu.PrefillWorkspace(max(chunks), H, HKV, n_ctx)
    p = 0
    for n in chunks:
        bc, bp = _dev(qkv_all[p:p + n]), _dev(qkv_all[p:p + n])
        gpu.qkv_prepare(bc, shape, _dev(qg), _dev(kg), cs, _pos(p), kc, vc)
        oc = _host(gpu.attn_prefill(bc, kc, vc, _pos(p), shape, ws=ws_c))
        op = _host(gpu.prefill_step(bp, pkd, pvd, shape, _dev(qg), _dev(kg), cs, _pos(p), ws_p, block_table=tab,
                                    block_size=bs))
        assert bits_equal(op, oc), f"chunk at {p}"
        p += n
    dws_c, dws_p = gpu.DecodeWorkspace(1, H, HKV, n_ctx), gpu.DecodeWorkspace(1, H, HKV, n_ctx)
    lens = _dev(np.array([0], np.int32))
    for _ in range(n_dec):
        row = qkv_all[p:p + 1]
        oc = _host(gpu.decode_step(_dev(row), kc, vc, shape, _dev(qg), _dev(kg), cs, dws_c, pos_dev=_pos(p)))
        lens.fill_(p + 1)
        op = _host(gpu.decode_step_paged(_dev(row), pkd, pvd, tab[None, :], bs, lens, shape, _dev(qg), _dev(kg), cs,
                                         dws_p))
        assert bits_equal(op.reshape(oc.shape), oc), f"decode at {p}"
        p += 1
    assert bits_equal(_host(pkd)[rows], _host(kc)) and bits_equal(_host(pvd)[rows], _host(vc))
