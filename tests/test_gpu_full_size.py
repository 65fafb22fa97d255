"""GPU parity at the benchmarked sizes and for the in-kernel split merge.

- configs[4] at its stated workload: 64 sequences, kv_len ~ U[256, 8192] drawn with the bench's
  seed, H16/HKV8, through the fused step on a contiguous ragged pool (ei_decode_step) and on a
  shuffled paged pool (ei_decode_step_paged); every sequence against the reference attention.
- configs[2]'s timed path: ei_prefill_step at H32/HKV8, 2048 tokens from position 0 (the
  q-norm-in-kernel plan), sampled rows against the reference, the whole cache bit-exact.
- The in-kernel split merge (chunks over 128 keys): consecutive calls and graph replays, where
  every launch advances the split records' epoch.
- A 512-token chunk at position 32256 of a 32768-row context (8 key shares), contiguous and paged.
- Edge contracts: a kv_len beyond the workspace's max_kv, and a fused decode with rope_dim 64.
Calls go through the C ABI; the reference is the oracle's restatement of src/model.cpp:191-214
(oracle/oracle.c), QK-norm + RoPE of src/ops.cpp:155-160 and src/model.cpp:23-32.
"""
import numpy as np
import pytest

from tests.parity import ATTN_RTOL, bits_equal, gate, rel_err

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


def _synth(gpu, shape, seed):
    """Seeded N(0,1) on the GPU (bit-identical to the oracle's generator, tested elsewhere)."""
    import torch
    return gpu.synth_fill(torch.empty(shape, dtype=torch.float32, device="cuda"), seed)


def _normed_row(orc, qkv_row, H, HKV, qg, kg, pos, rope_dim=128):
    row = orc.headnorm_rope(qkv_row[None], H, D, qg, pos, rope_dim, 1e6, 1e-6)
    return orc.headnorm_rope(row, HKV, D, kg, pos, rope_dim, 1e6, 1e-6, col0=H * D)[0]


def _configs4_lengths():
    # the bench's configs[4] draw (bench.py bench_batched, seed 3000)
    rng = np.random.default_rng(3000)
    return rng, rng.integers(256, 8193, 64).astype(np.int32)


@pytest.mark.parametrize("paged", [False, True])
def test_configs4_full_size_fused_step(orc, gpu, paged):
    H, HKV, bs = 16, 8, 64
    shape = gpu.AttnShape(H, HKV)
    rng, lens = _configs4_lengths()
    nseq = len(lens)
    kd = HKV * D
    if paged:  # whole blocks per sequence, every block of every sequence shuffled over the pool
        nblk = [-(-int(n) // bs) for n in lens]
        perm = rng.permutation(sum(nblk)).astype(np.int32)
        table = np.zeros((nseq, max(nblk)), np.int32)
        k0 = 0
        for s, nb in enumerate(nblk):
            table[s, :nb] = perm[k0:k0 + nb]
            k0 += nb
        rows = sum(nblk) * bs
        row_of = lambda s, t: int(table[s, t // bs]) * bs + t % bs
    else:
        offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
        rows = int(lens.sum())
        row_of = lambda s, t: int(offs[s]) + t
    kc, vc = _synth(gpu, (rows, kd), 3100), _synth(gpu, (rows, kd), 3101)
    k_host, v_host = _host(kc), _host(vc)
    qkv = orc.normal((nseq, shape.qkv), 3102)
    qg, kg = orc.gamma(D, 3103), orc.gamma(D, 3104)
    cs = gpu.rope_table(int(lens.max()))
    ws = gpu.DecodeWorkspace(nseq, H, HKV, max_kv=int(lens.max()))
    len_d = _dev(lens)
    if paged:
        out = _host(gpu.decode_step_paged(_dev(qkv), kc, vc, _dev(table), bs, len_d, shape, _dev(qg), _dev(kg), cs,
                                          ws))
    else:
        out = _host(gpu.decode_step(_dev(qkv), kc, vc, shape, _dev(qg), _dev(kg), cs, ws, kv_offset=_dev(offs),
                                    kv_len=len_d))
    kh, vh = _host(kc), _host(vc)
    for s, n in enumerate(lens):
        n = int(n)
        row = _normed_row(orc, qkv[s], H, HKV, qg, kg, n - 1)
        r = row_of(s, n - 1)
        k_host[r] = row[H * D:(H + HKV) * D]
        v_host[r] = row[(H + HKV) * D:]
        idx = np.array([row_of(s, t) for t in range(n)])
        kk, vv = k_host[idx].reshape(n, HKV, D), v_host[idx].reshape(n, HKV, D)
        qn = np.ascontiguousarray(row[:H * D].reshape(H, D))
        ref = orc.attn_decode(qn, kk, vv, n, H, HKV, D)
        ok, msg = gate(f"configs[4] {'paged' if paged else 'contiguous'} seq {s} len {n}", out[s], ref,
                       lambda: orc.attn_f64(qn, kk, vv, n, H, HKV, D))
        assert ok, msg
    # the appended rows are the only change to the pool, bit for bit
    assert bits_equal(kh, k_host) and bits_equal(vh, v_host)
    # the plan splits the long sequences into 1024-key chunks merged inside the launch
    assert ws.status() == 0, "a workgroup ran off the XCD placement the merge relies on"


def test_configs2_prefill_step_full_size(orc, gpu):
    H, HKV, B = 32, 8, 2048
    shape = gpu.AttnShape(H, HKV)
    qkv = orc.normal((B, shape.qkv), 2500)
    qg, kg = orc.gamma(D, 2501), orc.gamma(D, 2502)
    cs = gpu.rope_table(B)
    kc, vc = _dev(np.zeros((B, HKV * D), np.float32)), _dev(np.zeros((B, HKV * D), np.float32))
    buf = _dev(qkv)
    ws = gpu.PrefillWorkspace(B, H, HKV, B)
    out = _host(gpu.prefill_step(buf, kc, vc, shape, _dev(qg), _dev(kg), cs, _pos(0), ws))
    normed = orc.headnorm_rope(qkv, H, D, qg, 0, 128, 1e6, 1e-6)
    normed = orc.headnorm_rope(normed, HKV, D, kg, 0, 128, 1e6, 1e-6, col0=H * D)
    rk, rv = np.zeros((B, HKV * D), np.float32), np.zeros((B, HKV * D), np.float32)
    orc.kv_append(normed[:, H * D:(H + HKV) * D], normed[:, (H + HKV) * D:], rk, rv, 0)
    assert bits_equal(_host(kc), rk) and bits_equal(_host(vc), rv)
    # the timed plan norms q inside the attention kernel: the Q heads stay raw in the buffer
    assert bits_equal(_host(buf)[:, :H * D], qkv[:, :H * D])
    kk, vv = rk.reshape(B, HKV, D), rv.reshape(B, HKV, D)
    for b in (0, 1, 31, 32, 127, 128, 1023, 1024, 1500, 2047):
        q = np.ascontiguousarray(normed[b, :H * D].reshape(H, D))
        ref = orc.attn_decode(q, kk, vv, b + 1, H, HKV, D)
        ok, msg = gate(f"configs[2] prefill step row {b}", out[b], ref, lambda: orc.attn_f64(q, kk, vv, b + 1, H, HKV, D))
        assert ok, msg


@pytest.mark.parametrize("paged", [False, True])
def test_long_position_prefill_chunk(orc, gpu, paged):
    """A 512-token chunk at the end of a 32768-row context (configs[3]'s H16/HKV8): the plan cuts each
    unit pair's ~2000 key tiles into 8 shares (the most it makes), so the step takes the full
    prologue and the share combine reads up to three shares per row.  Contiguous and on a paged
    pool of shuffled 64-row blocks; the appended rows bit-exact, sampled rows (both ends of each
    32-row block among them) against the reference."""
    H, HKV, B, bs = 16, 8, 512, 64
    n_ctx = 32768
    pos0 = n_ctx - B
    shape = gpu.AttnShape(H, HKV)
    kd = HKV * D
    assert gpu._capi.lib().ei_attn_prefill_ws_bytes(B, H, HKV, n_ctx) >= 8 * B * H * D * 4  # 8 shares
    k, v = orc.normal((n_ctx, kd), 2600), orc.normal((n_ctx, kd), 2601)
    qkv = orc.normal((B, shape.qkv), 2602)
    qg, kg = orc.gamma(D, 2603), orc.gamma(D, 2604)
    cs = gpu.rope_table(n_ctx)
    ws = gpu.PrefillWorkspace(B, H, HKV, n_ctx)
    if paged:
        rng = np.random.default_rng(2605)
        nblk = n_ctx // bs
        table = rng.permutation(nblk).astype(np.int32)
        rows = (table[np.arange(n_ctx) // bs].astype(np.int64) * bs + np.arange(n_ctx) % bs)
        pk, pv = np.empty_like(k), np.empty_like(v)
        pk[rows], pv[rows] = k, v
        kc, vc = _dev(pk), _dev(pv)
        out = _host(gpu.prefill_step(_dev(qkv), kc, vc, shape, _dev(qg), _dev(kg), cs, _pos(pos0), ws,
                                     block_table=_dev(table), block_size=bs))
        kc_h, vc_h = _host(kc)[rows], _host(vc)[rows]
    else:
        kc, vc = _dev(k), _dev(v)
        out = _host(gpu.prefill_step(_dev(qkv), kc, vc, shape, _dev(qg), _dev(kg), cs, _pos(pos0), ws))
        kc_h, vc_h = _host(kc), _host(vc)
    normed = orc.headnorm_rope(qkv, H, D, qg, pos0, 128, 1e6, 1e-6)
    normed = orc.headnorm_rope(normed, HKV, D, kg, pos0, 128, 1e6, 1e-6, col0=H * D)
    rk, rv = k.copy(), v.copy()
    orc.kv_append(normed[:, H * D:(H + HKV) * D], normed[:, (H + HKV) * D:], rk, rv, pos0)
    assert bits_equal(kc_h, rk) and bits_equal(vc_h, rv)
    kk, vv = rk.reshape(n_ctx, HKV, D), rv.reshape(n_ctx, HKV, D)
    for b in (0, 1, 31, 32, 255, 256, 480, 511):
        q = np.ascontiguousarray(normed[b, :H * D].reshape(H, D))
        ref = orc.attn_decode(q, kk, vv, pos0 + b + 1, H, HKV, D)
        ok, msg = gate(f"long-position chunk {'paged' if paged else 'contiguous'} row {b}", out[b], ref,
                       lambda: orc.attn_f64(q, kk, vv, pos0 + b + 1, H, HKV, D))
        assert ok, msg


@pytest.mark.parametrize("H,HKV,T", [(32, 8, 8192), (16, 8, 32768), (8, 2, 40000), (40, 8, 9000)])
def test_inkernel_merge_consecutive_calls(orc, gpu, H, HKV, T):
    """Chunks of more than 128 keys merge their splits inside the launch; four calls in a row on
    one workspace (each a new epoch of the split records) with different queries and lengths."""
    shape = gpu.AttnShape(H, HKV)
    k = orc.normal((T, HKV, D), 3300 + T)
    v = orc.normal((T, HKV, D), 3301 + T)
    kd, vd = _dev(k), _dev(v)
    ws = gpu.DecodeWorkspace(1, H, HKV, max_kv=T)
    for i, n in enumerate((T, T - 1, T // 2 + 3, T)):
        q = orc.normal((H, D), 3400 + i)
        out = _host(gpu.attn_decode(_dev(q), kd, vd, _pos(n - 1), shape, ws))
        ref = orc.attn_decode(q, k, v, n, H, HKV, D)
        ok, msg = gate(f"in-kernel merge H{H}/HKV{HKV} call {i} T={n}", out, ref,
                       lambda: orc.attn_f64(q, k, v, n, H, HKV, D))
        assert ok, msg
    assert ws.status() == 0, "a workgroup ran off the XCD placement the merge relies on"


def test_inkernel_merge_graph_replays(orc, gpu):
    """The fused step with an in-kernel merge captured once and replayed at several positions,
    with eager work between replays; every replay equals the eager call bit for bit."""
    import torch
    H, HKV, n_ctx = 32, 8, 8192
    shape = gpu.AttnShape(H, HKV)
    k, v = orc.normal((n_ctx, HKV, D), 3500), orc.normal((n_ctx, HKV, D), 3501)
    qkv = _dev(orc.normal((1, shape.qkv), 3502))
    qg, kg = _dev(orc.gamma(D, 3503)), _dev(orc.gamma(D, 3504))
    cs = gpu.rope_table(n_ctx)
    kc_g, vc_g, kc_e, vc_e = _dev(k), _dev(v), _dev(k), _dev(v)
    ws_g = gpu.DecodeWorkspace(1, H, HKV, max_kv=n_ctx)
    ws_e = gpu.DecodeWorkspace(1, H, HKV, max_kv=n_ctx)
    pos_g = _pos(5000)
    out_g = torch.empty((1, H, D), dtype=torch.float32, device="cuda")
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        gpu.decode_step(qkv, kc_g, vc_g, shape, qg, kg, cs, ws_g, pos_dev=pos_g, out=out_g)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gpu.decode_step(qkv, kc_g, vc_g, shape, qg, kg, cs, ws_g, pos_dev=pos_g, out=out_g)
    gpu.decode_step(qkv, kc_e, vc_e, shape, qg, kg, cs, ws_e, pos_dev=_pos(5000))  # same state as the warm-up
    for p in (5000, 5001, 6000, 8191, 300):
        pos_g.fill_(p)
        graph.replay()
        torch.cuda.synchronize()
        ref = gpu.decode_step(qkv, kc_e, vc_e, shape, qg, kg, cs, ws_e, pos_dev=_pos(p))
        _ = torch.randn(1000, device="cuda").sum()  # unrelated eager work between replays
        assert bits_equal(_host(out_g), _host(ref)), f"replay at pos {p}"
    assert ws_g.status() == 0 and ws_e.status() == 0


@pytest.mark.parametrize("T,max_kv", [(1500, 1000), (5000, 4096), (300, 100)])
def test_kv_len_beyond_max_kv_is_attended_in_full(orc, gpu, T, max_kv):
    """max_kv sizes the split plan; a longer sequence is still attended in full (its last split
    takes the extra keys) and the fused step still appends its new row."""
    H, HKV = 32, 8
    shape = gpu.AttnShape(H, HKV)
    k, v = orc.normal((T, HKV, D), 3600 + T), orc.normal((T, HKV, D), 3601 + T)
    q = orc.normal((H, D), 3602)
    ws = gpu.DecodeWorkspace(1, H, HKV, max_kv=max_kv)
    out = _host(gpu.attn_decode(_dev(q), _dev(k), _dev(v), _pos(T - 1), shape, ws))
    assert rel_err(out, orc.attn_decode(q, k, v, T, H, HKV, D)) <= ATTN_RTOL
    # fused step at position T-1
    qkv = orc.normal((1, shape.qkv), 3603)
    qg, kg = orc.gamma(D, 3604), orc.gamma(D, 3605)
    kc, vc = _dev(k), _dev(v)
    out = _host(gpu.decode_step(_dev(qkv), kc, vc, shape, _dev(qg), _dev(kg), gpu.rope_table(T), ws,
                                pos_dev=_pos(T - 1)))
    row = _normed_row(orc, qkv[0], H, HKV, qg, kg, T - 1)
    rk, rv = k.reshape(T, -1).copy(), v.reshape(T, -1).copy()
    rk[T - 1], rv[T - 1] = row[H * D:(H + HKV) * D], row[(H + HKV) * D:]
    assert bits_equal(_host(kc).reshape(T, -1), rk) and bits_equal(_host(vc).reshape(T, -1), rv)
    ref = orc.attn_decode(np.ascontiguousarray(row[:H * D].reshape(H, D)), rk.reshape(T, HKV, D),
                          rv.reshape(T, HKV, D), T, H, HKV, D)
    assert rel_err(out, ref) <= ATTN_RTOL


@pytest.mark.parametrize("paged", [False, True])
def test_fused_decode_partial_rope_dim(orc, gpu, paged):
    """rope_dim 64 (partial rotary) through the fused decode steps: the RoPE row is 256 bytes."""
    H, HKV, rope_dim, bs = 16, 8, 64, 16
    shape = gpu.AttnShape(H, HKV, rope_dim=rope_dim)
    lens = np.array([700, 33, 1, 129], np.int32)
    nseq = len(lens)
    qkv = orc.normal((nseq, shape.qkv), 3700)
    qg, kg = orc.gamma(D, 3701), orc.gamma(D, 3702)
    n_ctx = int(lens.max())
    cs = gpu.rope_table(n_ctx, rope_dim=rope_dim)
    if paged:
        nblk = [-(-int(n) // bs) for n in lens]
        table = np.arange(sum(nblk), dtype=np.int32)[::-1].copy()
        tab = np.zeros((nseq, max(nblk)), np.int32)
        k0 = 0
        for s, nb in enumerate(nblk):
            tab[s, :nb] = table[k0:k0 + nb]
            k0 += nb
        rows = sum(nblk) * bs
        row_of = lambda s, t: int(tab[s, t // bs]) * bs + t % bs
    else:
        offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
        rows = int(lens.sum())
        row_of = lambda s, t: int(offs[s]) + t
    k, v = orc.normal((rows, HKV * D), 3703), orc.normal((rows, HKV * D), 3704)
    kc, vc = _dev(k), _dev(v)
    ws = gpu.DecodeWorkspace(nseq, H, HKV, max_kv=n_ctx)
    if paged:
        out = _host(gpu.decode_step_paged(_dev(qkv), kc, vc, _dev(tab), bs, _dev(lens), shape, _dev(qg), _dev(kg), cs,
                                          ws))
    else:
        out = _host(gpu.decode_step(_dev(qkv), kc, vc, shape, _dev(qg), _dev(kg), cs, ws, kv_offset=_dev(offs),
                                    kv_len=_dev(lens)))
    for s, n in enumerate(lens):
        n = int(n)
        row = _normed_row(orc, qkv[s], H, HKV, qg, kg, n - 1, rope_dim)
        r = row_of(s, n - 1)
        k[r], v[r] = row[H * D:(H + HKV) * D], row[(H + HKV) * D:]
        idx = np.array([row_of(s, t) for t in range(n)])
        ref = orc.attn_decode(np.ascontiguousarray(row[:H * D].reshape(H, D)), k[idx].reshape(n, HKV, D),
                              v[idx].reshape(n, HKV, D), n, H, HKV, D)
        assert rel_err(out[s], ref) <= ATTN_RTOL, f"sequence {s}"
    assert bits_equal(_host(kc), k) and bits_equal(_host(vc), v)


def test_one_workspace_serves_calls_of_different_plans(orc, gpu):
    """Decode calls of different plans (n_seq, max_kv, contiguous or paged) take turns on one
    workspace, several with the in-kernel split merge: its arrival counters sit where the
    workspace's size puts them, so every call finds them at zero whatever the previous plan wrote."""
    import torch
    from exactinfer_amd import _capi
    H, HKV = 32, 8
    shape = gpu.AttnShape(H, HKV)
    ws = gpu.DecodeWorkspace(4, H, HKV, max_kv=16384)
    rows = 40000
    k, v = orc.normal((rows, HKV * D), 3800), orc.normal((rows, HKV * D), 3801)
    kd, vd = _dev(k), _dev(v)
    scale = gpu.default_scale()
    calls = [("contiguous", [16000], 16384), ("contiguous", [9000, 3000, 16384, 500], 16384),
             ("paged", [12000, 7000], 12288), ("contiguous", [5000], 5000), ("contiguous", [16000], 16384),
             ("paged", [2000, 4000, 9000], 16384), ("contiguous", [300, 8000, 15000, 2], 16000)]
    for i, (kind, lens, max_kv) in enumerate(calls):
        lens = np.array(lens, np.int32)
        n = len(lens)
        q = orc.normal((n, H * D), 3900 + i)
        out = torch.full((n, H, D), float("nan"), device="cuda")
        # (device copies held in names: a temporary's memory could be reused before the launch reads it)
        qd, ld = _dev(q), _dev(lens)
        if kind == "contiguous":
            offs = np.array([(s * 9001) % (rows - int(lens[s])) for s in range(n)], np.int64)
            od = _dev(offs)
            _capi.call("ei_attn_decode_batched", gpu._stream(), qd.data_ptr(), H * D, out.data_ptr(), kd.data_ptr(),
                       vd.data_ptr(), od.data_ptr(), ld.data_ptr(), n, H, HKV, D, float(scale), max_kv,
                       ws.buf.data_ptr(), ws.nbytes)
            row_of = lambda s, t: int(offs[s]) + t
        else:
            bs = 64
            nblk = [-(-int(x) // bs) for x in lens]
            table = np.zeros((n, max(max(nblk), -(-max_kv // bs))), np.int32)  # covers max_kv
            perm = np.random.default_rng(3950 + i).permutation(rows // bs)
            k0 = 0
            for s_, nb in enumerate(nblk):
                table[s_, :nb] = perm[k0:k0 + nb]
                k0 += nb
            td = _dev(table)
            _capi.call("ei_attn_decode_paged", gpu._stream(), qd.data_ptr(), H * D, out.data_ptr(), kd.data_ptr(),
                       vd.data_ptr(), td.data_ptr(), table.shape[1], bs, ld.data_ptr(), n, H, HKV, D,
                       float(scale), max_kv, ws.buf.data_ptr(), ws.nbytes)
            row_of = lambda s, t, table=table, bs=bs: int(table[s, t // bs]) * bs + t % bs
        got = _host(out)
        for s_, T in enumerate(lens):
            idx = np.array([row_of(s_, t) for t in range(int(T))])
            kk, vv = k[idx].reshape(-1, HKV, D), v[idx].reshape(-1, HKV, D)
            qs = np.ascontiguousarray(q[s_].reshape(H, D))
            ok, msg = gate(f"shared workspace call {i} ({kind}) seq {s_} len {T}", got[s_],
                           orc.attn_decode(qs, kk, vv, int(T), H, HKV, D),
                           lambda: orc.attn_f64(qs, kk, vv, int(T), H, HKV, D))
            assert ok, msg
    assert ws.status() == 0
