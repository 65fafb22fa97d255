"""GPU parity of every kernel against the CPU oracle (a restatement of the reference CPU
path, oracle/oracle.c).  Calls go through the C ABI (exactinfer_amd/_capi.py).

Bars: bit-exact for the generator, the RoPE table, KV append and indexing; bit-exact for
QK-norm + RoPE (the kernels use the reference's double-precision sum of squares and the
same float operation order); attention within ATTN_RTOL (tests/parity.py) of the
reference CPU attention, whose near-zero rule is documented there.
"""
import numpy as np
import pytest

from tests.parity import ATTN_RTOL, attn_parity, bits_equal, gate, rel_err

pytestmark = pytest.mark.gpu

D = 128


def _dev(a, dtype=None):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def _pos(p):
    import torch
    return torch.tensor([p], dtype=torch.int32, device="cuda")


def _host(t):
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


# ---------------------------------------------------------------- generator / table
def test_synth_fill_matches_cpu_generator(orc, gpu):
    import torch
    n = 1 << 16
    t = torch.empty(n, dtype=torch.float32, device="cuda")
    gpu.synth_fill(t, seed=1234, offset=77)
    assert bits_equal(_host(t), orc.normal((n,), 1234, 77))
    # spikes: every 4th row of 256 floats times 4
    gpu.synth_fill(t, seed=5, offset=0, row_len=256, spike_every=4, spike_mult=4.0)
    ref = orc.normal((n // 256, 256), 5).copy()
    ref[::4] *= np.float32(4.0)
    assert bits_equal(_host(t), ref.reshape(-1))


# ---------------------------------------------------------------- QK-norm + RoPE
@pytest.mark.parametrize("rows,n_heads,pos0,rope_dim", [(1, 32, 0, 128), (5, 8, 4090, 128), (3, 16, 17, 64)])
def test_headnorm_rope_bit_exact(orc, gpu, rows, n_heads, pos0, rope_dim):
    stride = n_heads * D + 64  # padded rows: columns past the heads must stay untouched
    x = orc.normal((rows, stride), 11 + rows) * np.float32(3.0)
    gam = orc.gamma(D, 99)
    n_ctx = pos0 + rows
    cs = gpu.rope_table(n_ctx, rope_dim, 1e6)
    buf = _dev(x)
    gpu.headnorm_rope(buf, n_heads, _dev(gam), cs, _pos(pos0), rope_dim=rope_dim, eps=1e-6)
    ref = orc.headnorm_rope(x, n_heads, D, gam, pos0, rope_dim, 1e6, 1e-6)
    assert bits_equal(_host(buf), ref)


def test_rope_table_matches_oracle(orc, gpu):
    cs = gpu.rope_table(300, 128, 1e6, device="cpu").numpy()
    assert bits_equal(cs, orc.rope_table(300, 128, 1e6))


# ---------------------------------------------------------------- KV append
@pytest.mark.parametrize("rows,pos0", [(1, 0), (1, 4095), (7, 100), (64, 0)])
def test_kv_append_bit_exact_and_untouched(orc, gpu, rows, pos0):
    HKV, n_ctx = 8, max(4096, pos0 + rows)
    kd = HKV * D
    stride = 3 * kd + 32
    src = orc.normal((rows, stride), 3)
    # NaN payloads and signed zeros must survive the copy bit for bit
    src.view(np.uint32)[0, 5] = 0x7FC12345
    src[0, 6] = -0.0
    sentinel = np.full((n_ctx, kd), 7.25, np.float32)
    kc, vc = _dev(sentinel), _dev(sentinel)
    ksrc = _dev(src)
    gpu.kv_append(ksrc[:, :kd], ksrc[:, kd:2 * kd], kc, vc, _pos(pos0))
    kh, vh = _host(kc), _host(vc)
    ref_k, ref_v = sentinel.copy(), sentinel.copy()
    orc.kv_append(src[:, :kd], src[:, kd:2 * kd], ref_k, ref_v, pos0)
    assert bits_equal(kh, ref_k) and bits_equal(vh, ref_v)


@pytest.mark.parametrize("H,HKV,B,pos0", [(16, 8, 9, 30), (4, 2, 16, 32), (8, 1, 3, 60)])
def test_qkv_prepare_matches_oracle(orc, gpu, H, HKV, B, pos0):
    shape = gpu.AttnShape(H, HKV)
    qkv = orc.normal((B, shape.qkv), 21)
    qg, kg = orc.gamma(D, 1), orc.gamma(D, 2)
    n_ctx = 64
    assert pos0 + B <= n_ctx
    cs = gpu.rope_table(n_ctx)
    kc = _dev(np.zeros((n_ctx, HKV * D), np.float32))
    vc = _dev(np.zeros((n_ctx, HKV * D), np.float32))
    buf = _dev(qkv)
    gpu.qkv_prepare(buf, shape, _dev(qg), _dev(kg), cs, _pos(pos0), kc, vc)
    ref = orc.headnorm_rope(qkv, H, D, qg, pos0, 128, 1e6, 1e-6)
    ref = orc.headnorm_rope(ref, HKV, D, kg, pos0, 128, 1e6, 1e-6, col0=H * D)
    out = _host(buf)
    assert bits_equal(out, ref)
    rk = np.zeros((n_ctx, HKV * D), np.float32)
    rv = np.zeros((n_ctx, HKV * D), np.float32)
    orc.kv_append(ref[:, H * D:(H + HKV) * D], ref[:, (H + HKV) * D:], rk, rv, pos0)
    assert bits_equal(_host(kc), rk) and bits_equal(_host(vc), rv)


# ---------------------------------------------------------------- decode
def _cache(orc, n, HKV, seed, spike_every=0):
    k = orc.normal((n, HKV, D), seed)
    v = orc.normal((n, HKV, D), seed + 1)
    if spike_every:
        k[::spike_every] *= np.float32(4.0)
    return k, v


@pytest.mark.parametrize("H,HKV,T", [(16, 8, 1), (16, 8, 2), (32, 8, 63), (32, 8, 64), (32, 8, 65), (16, 8, 1000),
                                     (32, 8, 4096), (8, 8, 333), (64, 8, 700), (4, 2, 64), (8, 2, 300),
                                     (16, 4, 129), (4, 1, 77), (8, 1, 2048),
                                     (40, 8, 1000), (12, 4, 300), (6, 1, 129), (7, 1, 64), (40, 8, 4096),
                                     (48, 8, 2000)])
def test_decode_matches_reference_attention(orc, gpu, H, HKV, T):
    shape = gpu.AttnShape(H, HKV)
    k, v = _cache(orc, T + 5, HKV, 40 + T)
    q = orc.normal((H, D), 7 + T)
    ws = gpu.DecodeWorkspace(1, H, HKV, max_kv=max(T, 4096))
    out = _host(gpu.attn_decode(_dev(q), _dev(k), _dev(v), _pos(T - 1), shape, ws))
    ref = orc.attn_decode(q, k, v, T, H, HKV, D)
    ok, msg = gate(f"decode H{H}/HKV{HKV} T={T}", out, ref)
    assert ok, msg
    # second call reuses the (re-armed) workspace
    out2 = _host(gpu.attn_decode(_dev(q), _dev(k), _dev(v), _pos(T - 1), shape, ws))
    assert bits_equal(out, out2)


def test_decode_long_context_split_combine(orc, gpu):
    """Config 4 shape: 0.6B heads, 32768 keys, every 512th key x4 (sharp softmax peaks)."""
    H, HKV, T = 16, 8, 32768
    shape = gpu.AttnShape(H, HKV)
    k, v = _cache(orc, T, HKV, 900, spike_every=512)
    q = orc.normal((H, D), 902)
    ws = gpu.DecodeWorkspace(1, H, HKV, max_kv=T)
    out = _host(gpu.attn_decode(_dev(q), _dev(k), _dev(v), _pos(T - 1), shape, ws))
    ref = orc.attn_decode(q, k, v, T, H, HKV, D)
    exact = orc.attn_f64(q, k, v, T, H, HKV, D)
    ok, msg = gate("configs[3] decode T=32768 spiked", out, ref, lambda: exact)
    assert ok, msg
    # the reference's own 16-way split/combine (src/cuda/model_cuda.cu:1043-1111) meets the
    # same gate against its CPU path
    ref16 = orc.attn_split_combine(q, k, v, T, H, HKV, D, nsplit=16)
    ok16, msg16 = attn_parity(ref16, ref, exact)
    assert ok16, msg16


@pytest.mark.parametrize("nseq,empty,H", [(12, (), 16), (12, (3, 7), 16), (40, (0, 39), 16), (12, (5,), 40)])
def test_decode_batched_ragged(orc, gpu, nseq, empty, H):
    """Ragged offsets and lengths; nseq 12 plans a key split per sequence, nseq 40 (320 (seq, KV
    head) units) one workgroup each; H = 40 runs groups of 5 on the 8-head kernel.  Sequences of
    length 0 (`empty`) must come out as zeros."""
    HKV = 8
    rng = np.random.default_rng(5 + nseq)
    lens = rng.integers(1, 3000, nseq).astype(np.int32)
    lens[1], lens[2] = 1, 64
    for i in empty:
        lens[i] = 0
    gaps = rng.integers(0, 50, nseq)
    offs = np.zeros(nseq, np.int64)
    for i in range(1, nseq):
        offs[i] = offs[i - 1] + lens[i - 1] + gaps[i]
    total = int(offs[-1] + lens[-1] + 10)
    k, v = _cache(orc, total, HKV, 77)
    q = orc.normal((nseq, H * D), 78)
    shape = gpu.AttnShape(H, HKV)
    ws = gpu.DecodeWorkspace(nseq, H, HKV, max_kv=int(lens.max()))
    out = _host(gpu.attn_decode_batched(_dev(q), _dev(k), _dev(v), _dev(offs), _dev(lens), shape, ws))
    live = np.array([i for i in range(nseq) if i not in empty])
    ref = orc.attn_decode_batched(q[live], k, v, offs[live], lens[live], H, HKV, D)
    assert rel_err(out[live], ref) <= ATTN_RTOL
    for i in empty:
        assert not np.any(out[i]), f"sequence {i} of length 0 is not zeros"


@pytest.mark.parametrize("H,HKV,T", [(32, 8, 1), (32, 8, 4096), (16, 8, 777), (4, 2, 55), (8, 1, 300), (40, 8, 777),
                                     (12, 4, 55)])
def test_fused_decode_step(orc, gpu, H, HKV, T):
    """ei_decode_step == headnorm_rope(Q,K) + append + reference attention, bit-exact cache."""
    shape = gpu.AttnShape(H, HKV)
    n_ctx = T + 3
    k, v = _cache(orc, n_ctx, HKV, 500 + T)
    qkv = orc.normal((1, shape.qkv), 501)
    qg, kg = orc.gamma(D, 3), orc.gamma(D, 4)
    cs = gpu.rope_table(n_ctx)
    kc, vc = _dev(k), _dev(v)
    ws = gpu.DecodeWorkspace(1, H, HKV, max_kv=n_ctx)
    pos = T - 1
    out = _host(gpu.decode_step(_dev(qkv), kc, vc, shape, _dev(qg), _dev(kg), cs, ws, pos_dev=_pos(pos)))
    normed = orc.headnorm_rope(qkv, H, D, qg, pos, 128, 1e6, 1e-6)
    normed = orc.headnorm_rope(normed, HKV, D, kg, pos, 128, 1e6, 1e-6, col0=H * D)
    rk, rv = k.reshape(n_ctx, -1).copy(), v.reshape(n_ctx, -1).copy()
    orc.kv_append(normed[:, H * D:(H + HKV) * D], normed[:, (H + HKV) * D:], rk, rv, pos)
    assert bits_equal(_host(kc).reshape(n_ctx, -1), rk)
    assert bits_equal(_host(vc).reshape(n_ctx, -1), rv)
    ref = orc.attn_decode(normed[0, :H * D].reshape(H, D), rk, rv, T, H, HKV, D)
    assert rel_err(out.reshape(H, D), ref) <= ATTN_RTOL


# ---------------------------------------------------------------- prefill
@pytest.mark.parametrize("H,HKV,B,pos0", [(16, 8, 1, 0), (16, 8, 31, 0), (32, 8, 33, 0), (16, 8, 100, 37),
                                          (32, 8, 512, 0), (16, 8, 512, 512), (32, 8, 65, 1000), (64, 8, 40, 3),
                                          (4, 2, 16, 32), (8, 2, 48, 0), (16, 4, 70, 5), (4, 4, 20, 3),
                                          (8, 1, 97, 200),
                                          # groups of 5, 3, 7, 1 and 2 heads: units spanning two blocks, idle
                                          # slots after the last block, ragged last blocks
                                          (40, 8, 100, 37), (40, 8, 512, 0), (12, 4, 70, 5), (7, 1, 33, 0),
                                          (8, 8, 200, 0), (8, 8, 129, 64), (16, 8, 70, 0), (16, 8, 97, 300),
                                          (48, 8, 90, 10), (32, 8, 1, 3000)])
def test_prefill_matches_reference_attention(orc, gpu, H, HKV, B, pos0):
    shape = gpu.AttnShape(H, HKV)
    n = pos0 + B
    k, v = _cache(orc, n, HKV, 60 + B)
    q = orc.normal((B, H * D), 61 + pos0)
    out = _host(gpu.attn_prefill(_dev(q), _dev(k), _dev(v), _pos(pos0), shape))
    ref = orc.attn_prefill(q, k, v, B, pos0, H, HKV, D)
    ok, msg = gate(f"prefill H{H}/HKV{HKV} B={B} pos0={pos0}", out, ref)
    assert ok, msg


def test_prefill_row_equals_decode(orc, gpu):
    """Causal prefill row b == single-token decode at position pos0+b (same cache)."""
    H, HKV, B, pos0 = 32, 8, 96, 20
    shape = gpu.AttnShape(H, HKV)
    k, v = _cache(orc, pos0 + B, HKV, 31)
    q = orc.normal((B, H * D), 32)
    kd, vd = _dev(k), _dev(v)
    pre = _host(gpu.attn_prefill(_dev(q), kd, vd, _pos(pos0), shape))
    ws = gpu.DecodeWorkspace(1, H, HKV, max_kv=pos0 + B)
    for b in (0, 31, 32, 95):
        dec = _host(gpu.attn_decode(_dev(q[b].reshape(H, D)), kd, vd, _pos(pos0 + b), shape, ws))
        assert rel_err(pre[b], dec) <= 2 * ATTN_RTOL


def test_prefill_full_size_sampled_rows(orc, gpu):
    """Config 3 shape: 4B heads, 2048-token causal prefill; sampled rows vs the reference."""
    H, HKV, B = 32, 8, 2048
    shape = gpu.AttnShape(H, HKV)
    k, v = _cache(orc, B, HKV, 2048)
    q = orc.normal((B, H * D), 2049)
    out = _host(gpu.attn_prefill(_dev(q), _dev(k), _dev(v), _pos(0), shape))
    for b in (0, 1, 31, 32, 1023, 1024, 2000, 2047):
        ref = orc.attn_decode(q[b].reshape(H, D), k, v, b + 1, H, HKV, D)
        err = rel_err(out[b], ref)
        assert err <= ATTN_RTOL, f"row {b}: {err:.3e}"


# ---------------------------------------------------------------- graph capture
def test_decode_step_graph_replays_track_position(orc, gpu):
    """The fused step captured once in a HIP graph, replayed while the device position
    advances (src/cuda/model_cuda.cu:1848-1859 pattern); every replay equals the eager call
    on the same state, with eager work and syncs between replays."""
    import torch
    H, HKV, n_ctx = 32, 8, 600
    shape = gpu.AttnShape(H, HKV)
    k, v = _cache(orc, n_ctx, HKV, 1200)
    qkv = _dev(orc.normal((1, shape.qkv), 1201))
    qg, kg = _dev(orc.gamma(D, 5)), _dev(orc.gamma(D, 6))
    cs = gpu.rope_table(n_ctx)
    kc_g, vc_g = _dev(k), _dev(v)
    kc_e, vc_e = _dev(k), _dev(v)
    ws_g = gpu.DecodeWorkspace(1, H, HKV, max_kv=n_ctx)
    ws_e = gpu.DecodeWorkspace(1, H, HKV, max_kv=n_ctx)
    pos_g = _pos(100)
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
    for p in (100, 101, 257, 511, 599):
        pos_g.fill_(p)
        graph.replay()
        torch.cuda.synchronize()
        ref = gpu.decode_step(qkv, kc_e, vc_e, shape, qg, kg, cs, ws_e, pos_dev=_pos(p))
        torch.cuda.synchronize()
        _ = torch.randn(1000, device="cuda").sum()  # unrelated eager work between replays
        assert bits_equal(_host(out_g), _host(ref)), f"replay at pos {p}"
        assert bits_equal(_host(kc_g), _host(kc_e)) and bits_equal(_host(vc_g), _host(vc_e))


def test_prefill_graph_replays(orc, gpu):
    import torch
    H, HKV, B = 16, 8, 200
    shape = gpu.AttnShape(H, HKV)
    k, v = _cache(orc, B, HKV, 1300)
    q = _dev(orc.normal((B, H * D), 1301))
    kd, vd = _dev(k), _dev(v)
    pos = _pos(0)
    eager = _host(gpu.attn_prefill(q, kd, vd, pos, shape))
    out = torch.empty((B, H, D), dtype=torch.float32, device="cuda")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gpu.attn_prefill(q, kd, vd, pos, shape, out=out)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert bits_equal(_host(out), eager)


# ---------------------------------------------------------------- key-split prefill (short chunks, long positions)
@pytest.mark.gpu
@pytest.mark.parametrize("H,HKV,B,pos0,max_kv", [(32, 8, 512, 1536, 2048), (16, 8, 100, 3000, 4096),
                                                 (8, 2, 64, 500, 1024), (32, 8, 33, 0, 4096),
                                                 (4, 1, 256, 7000, 8192), (64, 8, 40, 900, 1024),
                                                 (40, 8, 100, 2000, 4096), (8, 8, 64, 1000, 2048),
                                                 (32, 8, 1, 3000, 4096)])
def test_prefill_split_matches_reference_attention(orc, gpu, H, HKV, B, pos0, max_kv):
    """ei_attn_prefill_split == the reference per-token attention; (32, 8, 33, 0, 4096) plans
    more shares than the chunk has tiles, so empty shares are merged too."""
    shape = gpu.AttnShape(H, HKV)
    n = pos0 + B
    k, v = _cache(orc, n, HKV, 90 + B)
    q = orc.normal((B, H * D), 91 + pos0)
    ws = gpu.PrefillWorkspace(B, H, HKV, max_kv)
    assert ws.nbytes > 0, "this shape should plan a key split"
    out = _host(gpu.attn_prefill(_dev(q), _dev(k), _dev(v), _pos(pos0), shape, ws=ws))
    ref = orc.attn_prefill(q, k, v, B, pos0, H, HKV, D)
    kk, vv = k.reshape(n, -1), v.reshape(n, -1)  # long rows: the reference's sequential fp32 sums drift
    ok, msg = gate(f"prefill split H{H}/HKV{HKV} B={B} pos0={pos0}", out, ref, lambda: np.stack(
        [orc.attn_f64(q[b].reshape(H, D), kk, vv, pos0 + b + 1, H, HKV, D) for b in range(B)]))
    assert ok, msg


@pytest.mark.gpu
@pytest.mark.parametrize("ksplit", [2, 3, 5, 8])
@pytest.mark.parametrize("H,HKV,B,pos0", [(12, 4, 77, 1500), (8, 1, 300, 0), (40, 8, 33, 3000), (16, 8, 512, 700)])
def test_prefill_forced_share_counts(orc, gpu, monkeypatch, ksplit, H, HKV, B, pos0):
    """Every share count on shapes that stress the cost-cut shares (a pair's tiles cut into shares
    of equal cost, the unit boundary counting extra): ragged last blocks, GQA groups of 3 and 8, a
    single KV head, a middle unit without a partner, chunks at position 0 (short units, shares
    without tiles) and deep in the context.  The plan's share count is forced (EI_PREFILL_SPLIT,
    read when the workspace is sized and at every call)."""
    monkeypatch.setenv("EI_PREFILL_SPLIT", str(ksplit))
    shape = gpu.AttnShape(H, HKV)
    n = pos0 + B
    k, v = _cache(orc, n, HKV, 190 + B + ksplit)
    q = orc.normal((B, H * D), 191 + pos0)
    ws = gpu.PrefillWorkspace(B, H, HKV, n)
    assert ws.nbytes > 0, "the forced split must be planned"
    out = _host(gpu.attn_prefill(_dev(q), _dev(k), _dev(v), _pos(pos0), shape, ws=ws))
    ref = orc.attn_prefill(q, k, v, B, pos0, H, HKV, D)
    kk, vv = k.reshape(n, -1), v.reshape(n, -1)
    ok, msg = gate(f"prefill forced {ksplit} shares H{H}/HKV{HKV} B={B} pos0={pos0}", out, ref, lambda: np.stack(
        [orc.attn_f64(q[b].reshape(H, D), kk, vv, pos0 + b + 1, H, HKV, D) for b in range(B)]))
    assert ok, msg


@pytest.mark.gpu
def test_prefill_split_graph_replays_track_position(orc, gpu):
    """One captured split prefill replayed at three device positions (the plan is fixed by
    (B, max_kv)); each replay equals the reference at that position."""
    import torch
    H, HKV, B, max_kv = 16, 8, 128, 2048
    shape = gpu.AttnShape(H, HKV)
    k, v = _cache(orc, max_kv, HKV, 1400)
    qh = orc.normal((B, H * D), 1401)
    q, kd, vd = _dev(qh), _dev(k), _dev(v)
    pos = _pos(0)
    ws = gpu.PrefillWorkspace(B, H, HKV, max_kv)
    out = torch.empty((B, H, D), dtype=torch.float32, device="cuda")
    gpu.attn_prefill(q, kd, vd, pos, shape, out=out, ws=ws)  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gpu.attn_prefill(q, kd, vd, pos, shape, out=out, ws=ws)
    for p0 in (0, 700, max_kv - B):
        pos.fill_(p0)
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        ref = orc.attn_prefill(qh, k, v, B, p0, H, HKV, D)
        assert rel_err(_host(out), ref) <= ATTN_RTOL, f"pos0 {p0}"


# ---------------------------------------------------------------- fused prefill step (q normed inside the attention kernel)
@pytest.mark.gpu
@pytest.mark.parametrize("H,HKV,B,pos0,max_kv,rope_dim", [(32, 8, 100, 37, 256, 128), (16, 8, 512, 1536, 2048, 128),
                                                          (40, 8, 64, 1000, 2048, 128), (8, 1, 33, 0, 64, 128),
                                                          (16, 8, 70, 5, 128, 64), (32, 8, 1, 500, 1024, 128),
                                                          (48, 8, 40, 100, 512, 128)])
def test_prefill_step_matches_reference(orc, gpu, H, HKV, B, pos0, max_kv, rope_dim):
    """ei_prefill_step == headnorm_rope(Q), headnorm_rope(K), append, reference attention:
    cache rows and the in-place K heads bit-exact, attention within ATTN_RTOL; the Q heads stay
    raw in qkv when the kernel norms them itself and are normed in place otherwise (rope_dim 64,
    or a plan of more than two key shares, takes the prologue for every head)."""
    shape = gpu.AttnShape(H, HKV, rope_dim=rope_dim)
    n_ctx = max(max_kv, pos0 + B)
    k, v = _cache(orc, n_ctx, HKV, 1500 + B)
    qkv = orc.normal((B, shape.qkv), 1501 + pos0)
    qg, kg = orc.gamma(D, 5), orc.gamma(D, 6)
    cs = gpu.rope_table(n_ctx, rope_dim=rope_dim)
    kc, vc = _dev(k.reshape(n_ctx, -1)), _dev(v.reshape(n_ctx, -1))
    buf = _dev(qkv)
    ws = gpu.PrefillWorkspace(B, H, HKV, max_kv)
    out = _host(gpu.prefill_step(buf, kc, vc, shape, _dev(qg), _dev(kg), cs, _pos(pos0), ws))
    normed = orc.headnorm_rope(qkv, H, D, qg, pos0, rope_dim, 1e6, 1e-6)
    normed = orc.headnorm_rope(normed, HKV, D, kg, pos0, rope_dim, 1e6, 1e-6, col0=H * D)
    rk, rv = k.reshape(n_ctx, -1).copy(), v.reshape(n_ctx, -1).copy()
    orc.kv_append(normed[:, H * D:(H + HKV) * D], normed[:, (H + HKV) * D:], rk, rv, pos0)
    assert bits_equal(_host(kc), rk) and bits_equal(_host(vc), rv)
    got = _host(buf)
    assert bits_equal(got[:, H * D:], normed[:, H * D:])
    # Q heads: raw when the kernel norms them itself, normed in place when the prologue did
    # (partial rope_dim, or a plan of more than two key shares)
    q_raw = bits_equal(got[:, :H * D], qkv[:, :H * D])
    assert q_raw or bits_equal(got[:, :H * D], normed[:, :H * D])
    if rope_dim != D:
        assert not q_raw
    qn = np.ascontiguousarray(normed[:, :H * D])
    ref = orc.attn_prefill(qn, rk.reshape(n_ctx, HKV, D), rv.reshape(n_ctx, HKV, D), B, pos0, H, HKV, D)
    ok, msg = gate(f"prefill step H{H}/HKV{HKV} B={B} pos0={pos0} rope {rope_dim}", out, ref, lambda: np.stack(
        [orc.attn_f64(qn[b].reshape(H, D), rk, rv, pos0 + b + 1, H, HKV, D) for b in range(B)]))
    assert ok, msg


@pytest.mark.gpu
def test_prefill_step_graph_replays(orc, gpu):
    """One captured fused prefill step replayed at three positions, the raw projections restored
    before each replay (the step norms the K heads in place); each replay equals the eager call."""
    import torch
    H, HKV, B, max_kv = 32, 8, 96, 1024
    shape = gpu.AttnShape(H, HKV)
    k, v = _cache(orc, max_kv, HKV, 1600)
    raw = _dev(orc.normal((B, shape.qkv), 1601))
    qg, kg = _dev(orc.gamma(D, 7)), _dev(orc.gamma(D, 8))
    cs = gpu.rope_table(max_kv)
    kc0, vc0 = _dev(k.reshape(max_kv, -1)), _dev(v.reshape(max_kv, -1))
    kc, vc, buf = kc0.clone(), vc0.clone(), raw.clone()
    pos = _pos(0)
    ws = gpu.PrefillWorkspace(B, H, HKV, max_kv)
    out = torch.empty((B, H, D), dtype=torch.float32, device="cuda")
    gpu.prefill_step(buf, kc, vc, shape, qg, kg, cs, pos, ws, out=out)  # warm-up outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gpu.prefill_step(buf, kc, vc, shape, qg, kg, cs, pos, ws, out=out)
    for p0 in (0, 400, max_kv - B):
        pos.fill_(p0)
        buf.copy_(raw), kc.copy_(kc0), vc.copy_(vc0)
        out.zero_()
        graph.replay()
        got, got_k = _host(out), _host(kc)
        buf.copy_(raw), kc.copy_(kc0), vc.copy_(vc0)
        eager = _host(gpu.prefill_step(buf, kc, vc, shape, qg, kg, cs, pos, ws))
        assert bits_equal(got, eager), f"pos0 {p0}"
        assert bits_equal(got_k, _host(kc)), f"pos0 {p0}"


# ---------------------------------------------------------------- paged KV (multi-sequence serving)
def _paged_layout(rng, lens, bs, shared_prefix_blocks, spare=3):
    """Block tables over a shuffled pool: sequences 0 and 1 share their first blocks."""
    nseq = len(lens)
    nblk = [max(1, -(-int(n) // bs)) for n in lens]
    max_blocks = max(nblk)
    total = sum(nblk) + spare
    perm = rng.permutation(total)
    table = np.zeros((nseq, max_blocks), np.int32)
    k = 0
    for s in range(nseq):
        for j in range(nblk[s]):
            if s == 1 and j < shared_prefix_blocks:
                table[s, j] = table[0, j]
            else:
                table[s, j] = perm[k]
                k += 1
    return table, total


def _gather(pool, table, s, n, bs):
    rows = [table[s, t // bs] * bs + t % bs for t in range(n)]
    return pool[rows]


@pytest.mark.parametrize("bs", [16, 64])
def test_decode_paged_matches_reference(orc, gpu, bs):
    H, HKV = (16, 8) if bs == 16 else (40, 8)  # bs 64: groups of 5 on the 8-head kernel
    rng = np.random.default_rng(40 + bs)
    lens = np.array([700, 300, 1, 0, 129, 2048, 64], np.int32)
    shared = 3  # sequences 0 and 1 share their first 3 blocks (a cached common prefix)
    lens[1] = max(lens[1], shared * bs + 5)
    table, nblocks = _paged_layout(rng, lens, bs, shared)
    pool_k, pool_v = _cache(orc, nblocks * bs, HKV, 4000 + bs)
    q = orc.normal((len(lens), H * D), 4001)
    shape = gpu.AttnShape(H, HKV)
    ws = gpu.DecodeWorkspace(len(lens), H, HKV, max_kv=int(lens.max()))
    out = _host(gpu.attn_decode_paged(_dev(q), _dev(pool_k), _dev(pool_v), _dev(table), bs, _dev(lens), shape, ws))
    for s, n in enumerate(lens):
        if n == 0:
            assert not np.any(out[s])
            continue
        kk, vv = _gather(pool_k, table, s, n, bs), _gather(pool_v, table, s, n, bs)
        ref = orc.attn_decode(q[s].reshape(H, D), kk, vv, int(n), H, HKV, D)
        assert rel_err(out[s], ref) <= ATTN_RTOL, f"sequence {s} (len {n})"


@pytest.mark.parametrize("bs", [16, 64])
def test_decode_paged_long_sequences_whole_chunks(orc, gpu, bs):
    """32 sequences x 8 KV heads = 256 units with a workspace planned for 1024 keys: one split
    per unit, which takes every key past the plan (lengths up to 8192), so a wave walks up to
    128 tiles and reads the cache rows of tiles 64..127 from its second row register."""
    H, HKV = 8, 8
    rng = np.random.default_rng(70 + bs)
    lens = np.concatenate([np.array([8192, 6000, 4097, 5000], np.int32), rng.integers(1, 200, 28).astype(np.int32)])
    table, nblocks = _paged_layout(rng, lens, bs, 0)
    pool_k, pool_v = _cache(orc, nblocks * bs, HKV, 5000 + bs)
    q = orc.normal((len(lens), H * D), 5001)
    shape = gpu.AttnShape(H, HKV)
    ws = gpu.DecodeWorkspace(len(lens), H, HKV, max_kv=1024)
    out = _host(gpu.attn_decode_paged(_dev(q), _dev(pool_k), _dev(pool_v), _dev(table), bs, _dev(lens), shape, ws))
    for s_, n in enumerate(lens):
        kk, vv = _gather(pool_k, table, s_, n, bs), _gather(pool_v, table, s_, n, bs)
        ref = orc.attn_decode(q[s_].reshape(H, D), kk, vv, int(n), H, HKV, D)
        assert rel_err(out[s_], ref) <= ATTN_RTOL, f"sequence {s_} (len {n})"


def test_decode_step_paged_appends_to_physical_rows(orc, gpu):
    """Fused paged step: each sequence's new K/V row lands in its physical row (bit-exact),
    the shared prefix blocks and every other row stay untouched, attention sees the append."""
    H, HKV, bs = 32, 8, 32
    rng = np.random.default_rng(41)
    lens = np.array([400, 150, 33, 1], np.int32)  # after the append (the new token included)
    shared = 2
    table, nblocks = _paged_layout(rng, lens, bs, shared)
    n_rows = nblocks * bs
    pool_k, pool_v = _cache(orc, n_rows, HKV, 4100)
    qkv = orc.normal((len(lens), (H + 2 * HKV) * D), 4101)
    qg, kg = orc.gamma(D, 5), orc.gamma(D, 6)
    cs = gpu.rope_table(int(lens.max()))
    shape = gpu.AttnShape(H, HKV)
    ws = gpu.DecodeWorkspace(len(lens), H, HKV, max_kv=int(lens.max()))
    kd, vd = _dev(pool_k), _dev(pool_v)
    out = _host(gpu.decode_step_paged(_dev(qkv), kd, vd, _dev(table), bs, _dev(lens), shape, _dev(qg), _dev(kg), cs,
                                      ws))
    rk, rv = pool_k.reshape(n_rows, -1).copy(), pool_v.reshape(n_rows, -1).copy()
    normed = []
    for s, n in enumerate(lens):
        pos = int(n) - 1
        row = orc.headnorm_rope(qkv[s:s + 1], H, D, qg, pos, 128, 1e6, 1e-6)
        row = orc.headnorm_rope(row, HKV, D, kg, pos, 128, 1e6, 1e-6, col0=H * D)
        phys = table[s, pos // bs] * bs + pos % bs
        rk[phys] = row[0, H * D:(H + HKV) * D]
        rv[phys] = row[0, (H + HKV) * D:]
        normed.append(row)
    assert bits_equal(_host(kd).reshape(n_rows, -1), rk) and bits_equal(_host(vd).reshape(n_rows, -1), rv)
    for s, n in enumerate(lens):
        kk = _gather(rk.reshape(n_rows, HKV, D), table, s, n, bs)
        vv = _gather(rv.reshape(n_rows, HKV, D), table, s, n, bs)
        ref = orc.attn_decode(normed[s][0, :H * D].reshape(H, D), kk, vv, int(n), H, HKV, D)
        assert rel_err(out[s], ref) <= ATTN_RTOL, f"sequence {s}"


def test_decode_step_paged_length_past_table(orc, gpu):
    """A kv_len longer than the table covers (max_blocks x block_size, outside the contract):
    the kernel reads no table entry past max_blocks.  That sequence attends over the keys its
    table holds, with q at the position its length names, and appends nothing; the other
    sequences of the batch are unaffected."""
    H, HKV, bs = 16, 8, 32
    rng = np.random.default_rng(42)
    lens = np.array([96, 200, 45], np.int32)  # in-table lengths; sequence 0 is then made longer
    table, nblocks = _paged_layout(rng, lens, bs, 0)
    cap = table.shape[1] * bs  # 224: sequence 0's 3 blocks are padded to the widest table with block 0
    table[0, 3:] = table[0, 0]
    lens[0] = cap + 9
    n_rows = nblocks * bs
    pool_k, pool_v = _cache(orc, n_rows, HKV, 4200)
    qkv = orc.normal((len(lens), (H + 2 * HKV) * D), 4201)
    qg, kg = orc.gamma(D, 7), orc.gamma(D, 8)
    cs = gpu.rope_table(int(lens.max()))
    shape = gpu.AttnShape(H, HKV)
    ws = gpu.DecodeWorkspace(len(lens), H, HKV, max_kv=cap)  # the host accepts a plan the table covers
    kd, vd = _dev(pool_k), _dev(pool_v)
    out = _host(gpu.decode_step_paged(_dev(qkv), kd, vd, _dev(table), bs, _dev(lens), shape, _dev(qg), _dev(kg), cs,
                                      ws))
    rk, rv = pool_k.reshape(n_rows, -1).copy(), pool_v.reshape(n_rows, -1).copy()
    normed = []
    for s, n in enumerate(lens):
        pos = int(n) - 1
        row = orc.headnorm_rope(qkv[s:s + 1], H, D, qg, pos, 128, 1e6, 1e-6)
        row = orc.headnorm_rope(row, HKV, D, kg, pos, 128, 1e6, 1e-6, col0=H * D)
        if s > 0:
            phys = table[s, pos // bs] * bs + pos % bs
            rk[phys] = row[0, H * D:(H + HKV) * D]
            rv[phys] = row[0, (H + HKV) * D:]
        normed.append(row)
    assert bits_equal(_host(kd).reshape(n_rows, -1), rk) and bits_equal(_host(vd).reshape(n_rows, -1), rv)
    for s, n in enumerate(lens):
        n = min(int(n), cap)
        kk = _gather(rk.reshape(n_rows, HKV, D), table, s, n, bs)
        vv = _gather(rv.reshape(n_rows, HKV, D), table, s, n, bs)
        ref = orc.attn_decode(normed[s][0, :H * D].reshape(H, D), kk, vv, n, H, HKV, D)
        assert rel_err(out[s], ref) <= ATTN_RTOL, f"sequence {s}"
