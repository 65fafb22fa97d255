"""GPU parity of the QKV projection (ei_qkv_project): attention RMSNorm + the fused [Wq|Wk|Wv]
product against the oracle's restatement of the CPU path (rmsnorm, src/ops.cpp:155-160, then
matvec with dot_f32 / dot_f16, src/ops.cpp:92-153; the oracle's dot products are bit-exact with
the reference's own, tests/test_oracle.py).  The sum order differs (a wave tree of per-lane FMA
chains against the reference's 8-lane AVX2 accumulators), so every output must lie within
1e-5 of sum_i |w_i h_i| (float64) of the reference: a dropped or repeated block of 16 terms
moves an output by ~1/160 of that scale.  Then the decode layer from the residual stream:
x -> ei_qkv_project -> ei_decode_step, its cache append bit-exact against the oracle applied to
the projected row and its attention within the 1e-5 attention bar."""
import numpy as np
import pytest

from tests.parity import ATTN_RTOL, bits_equal, gate

pytestmark = pytest.mark.gpu

D = 128
W_F32, W_F16, W_Q8_0, W_Q4_K, W_Q6_K = 0, 1, 8, 12, 14
QTYPES = [W_Q8_0, W_Q4_K, W_Q6_K]


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def _project(gpu, x, gamma, w, wtype, n_out, eps=1e-6):
    import torch
    from exactinfer_amd import _capi
    rows, E = x.shape
    out = torch.full((rows, n_out), float("nan"), dtype=torch.float32, device="cuda")
    xd, gd, wd = _dev(x), _dev(gamma), _dev(w)
    _capi.call("ei_qkv_project", gpu._stream(), xd.data_ptr(), E, rows, E, gd.data_ptr(), float(eps), wd.data_ptr(),
               wtype, n_out, out.data_ptr(), n_out)
    return out


def _weights(orc, n_out, E, wtype, seed):
    w = orc.normal((n_out, E), seed) * np.float32(0.05)
    return w if wtype == W_F32 else w.astype(np.float16).view(np.uint16)


def _wf(w, wtype):
    return (w if wtype == W_F32 else w.view(np.float16)).astype(np.float64)


@pytest.mark.parametrize("wtype,E,H,HKV,rows",
                         [(wt, *c) for wt in (W_F32, W_F16)
                          for c in ((2560, 32, 8, 1), (2560, 32, 8, 4), (1024, 16, 8, 1), (2048, 16, 8, 3),
                                    (4096, 32, 8, 2), (5120, 40, 8, 1))]
                         # the F16-only hidden sizes, at the most rows a launch takes there (3 and 2)
                         + [(W_F16, 8192, 64, 8, 3), (W_F16, 10240, 64, 8, 2)])
def test_qkv_project_matches_oracle(orc, gpu, wtype, E, H, HKV, rows):
    n_out = (H + 2 * HKV) * D
    x = orc.normal((rows, E), 8500 + E) * np.float32(3.0)
    gamma = orc.gamma(E, 8501)
    w = _weights(orc, n_out, E, wtype, 8502 + E)
    got = _host(_project(gpu, x, gamma, w, wtype, n_out))
    for b in range(rows):
        h = orc.rmsnorm(x[b], gamma)
        ref = orc.matvec(w, h, wtype)
        mag = np.abs(_wf(w, wtype)) @ np.abs(h.astype(np.float64))
        err = np.max(np.abs(got[b].astype(np.float64) - ref) / mag)
        assert err <= 1e-5, f"row {b}: max |got - ref| / sum|w h| = {err:.3e}"
        exact = _wf(w, wtype) @ h.astype(np.float64)
        assert np.max(np.abs(got[b] - exact) / mag) <= 1e-5


def _qweights(orc, n_out, E, wtype, seed):
    """Random quantised rows with moderate block scales, and the floats they decode to."""
    blocks = orc.random_blocks(wtype, n_out, E, seed, d_scale=0.05)
    return blocks, orc.dequant(wtype, blocks, E).reshape(n_out, E)


@pytest.mark.parametrize("wtype", QTYPES)
@pytest.mark.parametrize("E,H,HKV,rows", [(2560, 32, 8, 1), (2560, 32, 8, 4), (1024, 16, 8, 2), (2048, 16, 8, 4),
                                         (4096, 32, 8, 1), (5120, 40, 8, 3)])
def test_qkv_project_quantised_matches_oracle(orc, gpu, wtype, E, H, HKV, rows):
    """Q8_0 / Q4_K / Q6_K weights in their GGUF block layout: every output within 1e-5 of
    sum |w h| of the oracle's matvec (decode with the reference's dequant, then dot_f32), and of
    the float64 product of the decoded weights."""
    n_out = (H + 2 * HKV) * D
    x = orc.normal((rows, E), 8700 + E) * np.float32(3.0)
    gamma = orc.gamma(E, 8701)
    blocks, wf = _qweights(orc, n_out, E, wtype, 8702 + E + wtype)
    got = _host(_project(gpu, x, gamma, blocks, wtype, n_out))
    for b in range(rows):
        h = orc.rmsnorm(x[b], gamma)
        ref = orc.matvec(blocks, h, wtype)
        mag = np.abs(wf.astype(np.float64)) @ np.abs(h.astype(np.float64))
        err = np.max(np.abs(got[b].astype(np.float64) - ref) / mag)
        assert err <= 1e-5, f"w_type {wtype} row {b}: max |got - ref| / sum|w h| = {err:.3e}"
        exact = wf.astype(np.float64) @ h.astype(np.float64)
        assert np.max(np.abs(got[b] - exact) / mag) <= 1e-5


@pytest.mark.parametrize("wtype", QTYPES)
def test_qkv_project_quantised_decode_bit_exact(orc, gpu, wtype):
    """One-hot activations isolate single weights: with x = e_i the normed row has one
    non-zero h_i, every other product is an exact zero, so output r is float(w[r][i] * h_i)
    exactly.  Four rows per call, 64 calls cover all 256 positions of every super-block (all
    Q8_0 quarters, Q4_K sub-blocks and nibble halves, Q6_K groups), bit for bit against the
    reference's own decode."""
    E, n_out = 1024, 64
    gamma = orc.gamma(E, 8801)
    blocks, wf = _qweights(orc, n_out, E, wtype, 8802 + wtype)
    for start in range(0, 256, 4):
        cols = [start + i + 256 * (i % (E // 256)) for i in range(4)]  # four super-blocks in turn
        x = np.zeros((4, E), np.float32)
        for b, c in enumerate(cols):
            x[b, c] = np.float32(1.5)
        got = _host(_project(gpu, x, gamma, blocks, wtype, n_out))
        for b, c in enumerate(cols):
            h = orc.rmsnorm(x[b], gamma)
            want = (wf[:, c] * h[c]).astype(np.float32)
            g = got[b].copy()
            g[(g == 0) & (want == 0)] = 0.0  # a zero weight gives a zero of either sign
            want[want == 0] = 0.0
            assert bits_equal(g, want), f"w_type {wtype} column {c}"


@pytest.mark.parametrize("wtype", QTYPES)
def test_qkv_project_quantised_single_row_bit_exact(orc, gpu, wtype):
    """The single-activation-row kernel (a wave takes its rows a pair at a time) on 70 output
    rows, not a multiple of any workgroup's row count, so the last workgroup holds clamped rows:
    one-hot activations at every position of a super-block, each output bit for bit the
    reference's decoded weight times h_i."""
    E, n_out = 1024, 70
    gamma = orc.gamma(E, 8811)
    blocks, wf = _qweights(orc, n_out, E, wtype, 8812 + wtype)
    for c in range(256):
        col = c + 256 * (c % (E // 256))
        x = np.zeros((1, E), np.float32)
        x[0, col] = np.float32(-2.5)
        got = _host(_project(gpu, x, gamma, blocks, wtype, n_out))[0]
        h = orc.rmsnorm(x[0], gamma)
        want = (wf[:, col] * h[col]).astype(np.float32)
        g = got.copy()
        g[(g == 0) & (want == 0)] = 0.0  # a zero weight gives a zero of either sign
        want[want == 0] = 0.0
        assert bits_equal(g, want), f"w_type {wtype} column {col}"


def test_qkv_project_rejects_unbuilt_shapes(gpu):
    import ctypes
    from exactinfer_amd import _capi
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    with pytest.raises(_capi.EiError, match="n_embd 3000"):
        _capi.call("ei_qkv_project", None, p, 3000, 1, 3000, p, 1e-6, p, W_F32, 6144, p, 6144)
    with pytest.raises(_capi.EiError, match="rows 5"):
        _capi.call("ei_qkv_project", None, p, 2560, 5, 2560, p, 1e-6, p, W_F32, 6144, p, 6144)
    with pytest.raises(_capi.EiError, match="w_type"):
        _capi.call("ei_qkv_project", None, p, 2560, 1, 2560, p, 1e-6, p, 7, 6144, p, 6144)
    with pytest.raises(_capi.EiError, match="n_embd 2304"):  # not a multiple of 512
        _capi.call("ei_qkv_project", None, p, 2304, 1, 2304, p, 1e-6, p, W_Q4_K, 6144, p, 6144)


@pytest.mark.parametrize("wtype", [W_F32, W_F16, W_Q8_0])
def test_decode_layer_from_residual(orc, gpu, wtype):
    """Qwen3-4B shapes: residual x -> attention RMSNorm + QKV projection -> fused decode step."""
    E, H, HKV, T = 2560, 32, 8, 1000
    shape = gpu.AttnShape(H, HKV)
    n_out = shape.qkv
    x = orc.normal((1, E), 8600)
    gamma = orc.gamma(E, 8601)
    w = _weights(orc, n_out, E, wtype, 8602) if wtype in (W_F32, W_F16) else _qweights(orc, n_out, E, wtype, 8602)[0]
    qg, kg = orc.gamma(D, 8603), orc.gamma(D, 8604)
    k, v = orc.normal((T, HKV * D), 8605), orc.normal((T, HKV * D), 8606)
    kc, vc = _dev(k), _dev(v)
    cs = gpu.rope_table(T)
    ws = gpu.DecodeWorkspace(1, H, HKV, T)
    qkv = _project(gpu, x, gamma, w, wtype, n_out)
    import torch
    pos = torch.tensor([T - 1], dtype=torch.int32, device="cuda")
    out = _host(gpu.decode_step(qkv, kc, vc, shape, _dev(qg), _dev(kg), cs, ws, pos_dev=pos))
    # stage 2 against the oracle applied to the projected row itself
    row = _host(qkv)
    normed = orc.headnorm_rope(row, H, D, qg, T - 1, 128, 1e6, 1e-6)
    normed = orc.headnorm_rope(normed, HKV, D, kg, T - 1, 128, 1e6, 1e-6, col0=H * D)
    rk, rv = k.copy(), v.copy()
    orc.kv_append(normed[:, H * D:(H + HKV) * D], normed[:, (H + HKV) * D:], rk, rv, T - 1)
    assert bits_equal(_host(kc), rk) and bits_equal(_host(vc), rv)
    qn = np.ascontiguousarray(normed[0, :H * D].reshape(H, D))
    kk, vv = rk.reshape(T, HKV, D), rv.reshape(T, HKV, D)
    ok, msg = gate(f"decode layer from residual w_type {wtype}", out.reshape(H, D),
                   orc.attn_decode(qn, kk, vv, T, H, HKV, D), lambda: orc.attn_f64(qn, kk, vv, T, H, HKV, D))
    assert ok, msg
    # and the whole chain against the oracle chain (rmsnorm -> matvec -> QK-norm/RoPE -> attention):
    # the projection's different sum order moves q and k by ~1e-6, so the bar is looser here
    h = orc.rmsnorm(x[0], gamma)
    qkv_ref = orc.matvec(w, h, wtype)[None]
    nr = orc.headnorm_rope(qkv_ref, H, D, qg, T - 1, 128, 1e6, 1e-6)
    nr = orc.headnorm_rope(nr, HKV, D, kg, T - 1, 128, 1e6, 1e-6, col0=H * D)
    rk2, rv2 = k.copy(), v.copy()
    orc.kv_append(nr[:, H * D:(H + HKV) * D], nr[:, (H + HKV) * D:], rk2, rv2, T - 1)
    ref_chain = orc.attn_decode(np.ascontiguousarray(nr[0, :H * D].reshape(H, D)), rk2.reshape(T, HKV, D),
                                rv2.reshape(T, HKV, D), T, H, HKV, D)
    from tests.parity import rel_err
    assert rel_err(out.reshape(H, D), ref_chain) <= 20 * ATTN_RTOL


def test_projection_from_gguf_mixed_types(orc, gpu, tmp_path):
    """The path a real quantised model takes: a file with Wq Q4_K, Wk Q8_0, Wv Q6_K (the layout
    of a Q4_K_M quantisation) read through the GGUF reader, each segment's mapped bytes uploaded
    as they are and projected into its columns of the QKV row (one call per segment), against the
    oracle's decode + matvec of the same bytes."""
    import torch
    from exactinfer_amd import _capi
    from exactinfer_amd.gguf import GgufFile
    from tests.test_gguf import mixed_type_file
    E, H, HKV = 1024, 8, 2
    p, _, _, _ = mixed_type_file(tmp_path, orc, E, H, HKV)
    x = orc.normal((1, E), 8950) * np.float32(2.0)
    gamma = orc.gamma(E, 8951)
    n_out = (H + 2 * HKV) * D
    qkv = torch.full((1, n_out), float("nan"), dtype=torch.float32, device="cuda")
    xd, gd = _dev(x), _dev(gamma)
    h = orc.rmsnorm(x[0], gamma)
    with GgufFile(p) as g:
        col = 0
        for name, rows in (("blk.0.attn_q.weight", H * D), ("blk.0.attn_k.weight", HKV * D),
                           ("blk.0.attn_v.weight", HKV * D)):
            blocks = g.tensor(name)
            wtype = g.tensor_info(name)[0]
            wd = _dev(blocks)
            _capi.call("ei_qkv_project", gpu._stream(), xd.data_ptr(), E, 1, E, gd.data_ptr(), 1e-6, wd.data_ptr(),
                       wtype, rows, qkv[:, col:].data_ptr(), n_out)
            got = _host(qkv)[0, col:col + rows]
            ref = orc.matvec(blocks, h, wtype)
            wf = orc.dequant(wtype, blocks, E).reshape(rows, E).astype(np.float64)
            mag = np.abs(wf) @ np.abs(h.astype(np.float64))
            assert np.max(np.abs(got.astype(np.float64) - ref) / mag) <= 1e-5, name
            col += rows
