"""The allocation-free fused decode step (ei_decode_step_noalloc) against ei_decode_step with a
workspace: calls in a row through the C ABI (the second with a smaller input than the first, then GQA
groups 8 and 1), each equal bit for bit to the workspace entry point on the same state (both merge their splits with the
second launch for these shapes), cache appends included."""
import ctypes

import numpy as np
import pytest

from tests.parity import bits_equal

pytestmark = pytest.mark.gpu

D = 128


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _host(t):
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def _noalloc(gpu, qkv, kc, vc, shape, qg, kg, cs, max_kv, out, pos_dev=None, kv_offset=None, kv_len=None):
    from exactinfer_amd import _capi
    n_seq = qkv.shape[0]
    p = lambda t: None if t is None else t.data_ptr()
    _capi.call("ei_decode_step_noalloc", gpu._stream(), qkv.data_ptr(), qkv.stride(0), out.data_ptr(), kc.data_ptr(),
               vc.data_ptr(), p(kv_offset), p(kv_len), p(pos_dev), n_seq, shape.n_head, shape.n_head_kv,
               shape.head_dim, qg.data_ptr(), kg.data_ptr(), cs.data_ptr(), shape.rope_dim, float(shape.eps),
               float(gpu.default_scale()), max_kv)


def test_noalloc_decode_step_matches_workspace_step(orc, gpu):
    import torch
    # call 1: configs[1]'s layer (H32/HKV8, ctx 4096, one sequence); call 2: a smaller ragged batch
    # then GQA groups 8 and 1 (H64/HKV8, H8/HKV8) through the same shared array, one sequence on the
    # device position and a ragged batch
    cases = [dict(H=32, HKV=8, lens=[4096], max_kv=4096, seed=7000),
             dict(H=16, HKV=8, lens=[300, 1, 77], max_kv=512, seed=7100),
             dict(H=64, HKV=8, lens=[2500], max_kv=3000, seed=7400),
             dict(H=8, HKV=8, lens=[900, 33], max_kv=1024, seed=7500)]
    for c in cases:
        H, HKV, lens = c["H"], c["HKV"], np.array(c["lens"], np.int32)
        shape = gpu.AttnShape(H, HKV)
        n_seq = len(lens)
        offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
        rows = int(lens.sum())
        k, v = orc.normal((rows, HKV * D), c["seed"]), orc.normal((rows, HKV * D), c["seed"] + 1)
        qkv = _dev(orc.normal((n_seq, shape.qkv), c["seed"] + 2))
        qg, kg = _dev(orc.gamma(D, c["seed"] + 3)), _dev(orc.gamma(D, c["seed"] + 4))
        cs = gpu.rope_table(c["max_kv"])
        kc_a, vc_a, kc_b, vc_b = _dev(k), _dev(v), _dev(k), _dev(v)
        out_a = torch.full((n_seq, H, D), float("nan"), device="cuda")
        if n_seq == 1:
            pos = torch.tensor([int(lens[0]) - 1], dtype=torch.int32, device="cuda")
            _noalloc(gpu, qkv, kc_a, vc_a, shape, qg, kg, cs, c["max_kv"], out_a, pos_dev=pos)
            ws = gpu.DecodeWorkspace(1, H, HKV, c["max_kv"])
            out_b = gpu.decode_step(qkv, kc_b, vc_b, shape, qg, kg, cs, ws, pos_dev=pos)
        else:
            od, ld = _dev(offs), _dev(lens)
            _noalloc(gpu, qkv, kc_a, vc_a, shape, qg, kg, cs, c["max_kv"], out_a, kv_offset=od, kv_len=ld)
            ws = gpu.DecodeWorkspace(n_seq, H, HKV, c["max_kv"])
            out_b = gpu.decode_step(qkv, kc_b, vc_b, shape, qg, kg, cs, ws, kv_offset=od, kv_len=ld)
        assert bits_equal(_host(out_a), _host(out_b)), f"output differs for {c}"
        assert bits_equal(_host(kc_a), _host(kc_b)) and bits_equal(_host(vc_a), _host(vc_b)), f"cache differs for {c}"


def test_noalloc_falls_back_to_the_uncapped_plan(orc, gpu):
    """64 sequences planned for 8192 keys: the workspace plan's 1024-key splits need 4.8 MiB, more
    than the static array; the allocation-free step then runs the plan without the chunk cap (one
    split per sequence and KV head).  Two calls in a row; each output within the parity gate of the
    reference attention, the appended rows bit-identical to the workspace step's."""
    import torch
    from tests.parity import gate
    from exactinfer_amd import _capi
    H, HKV, max_kv, n_seq = 16, 8, 8192, 64
    assert _capi.lib().ei_attn_decode_ws_bytes(n_seq, H, HKV, max_kv) > 4 << 20
    shape = gpu.AttnShape(H, HKV)
    for call, seed in enumerate((7200, 7300)):
        rng = np.random.default_rng(seed)
        lens = rng.integers(1, 600 if call == 0 else 200, n_seq).astype(np.int32)
        offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
        rows = int(lens.sum())
        k, v = orc.normal((rows, HKV * D), seed), orc.normal((rows, HKV * D), seed + 1)
        qkv_h = orc.normal((n_seq, shape.qkv), seed + 2)
        qg_h, kg_h = orc.gamma(D, seed + 3), orc.gamma(D, seed + 4)
        qkv, qg, kg = _dev(qkv_h), _dev(qg_h), _dev(kg_h)
        cs = gpu.rope_table(max_kv)
        kc_a, vc_a, kc_b, vc_b = _dev(k), _dev(v), _dev(k), _dev(v)
        od, ld = _dev(offs), _dev(lens)
        out_a = torch.full((n_seq, H, D), float("nan"), device="cuda")
        _noalloc(gpu, qkv, kc_a, vc_a, shape, qg, kg, cs, max_kv, out_a, kv_offset=od, kv_len=ld)
        ws = gpu.DecodeWorkspace(n_seq, H, HKV, max_kv)
        gpu.decode_step(qkv, kc_b, vc_b, shape, qg, kg, cs, ws, kv_offset=od, kv_len=ld)
        ka, va = _host(kc_a), _host(vc_a)
        assert bits_equal(ka, _host(kc_b)) and bits_equal(va, _host(vc_b)), f"call {call}: appended rows differ"
        got = _host(out_a)
        for s_ in range(n_seq):
            n, o = int(lens[s_]), int(offs[s_])
            normed = orc.headnorm_rope(qkv_h[s_:s_ + 1], H, D, qg_h, n - 1, 128, 1e6, 1e-6)
            qn = np.ascontiguousarray(normed[0, :H * D].reshape(H, D))
            kk, vv = ka[o:o + n].reshape(n, HKV, D), va[o:o + n].reshape(n, HKV, D)
            ok, msg = gate(f"noalloc uncapped call {call} seq {s_} len {n}", got[s_],
                           orc.attn_decode(qn, kk, vv, n, H, HKV, D), lambda: orc.attn_f64(qn, kk, vv, n, H, HKV, D))
            assert ok, msg


def test_noalloc_rejects_shapes_beyond_its_scratch(gpu):
    from exactinfer_amd import _capi
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    with pytest.raises(_capi.EiError, match="allocation-free"):
        _capi.call("ei_decode_step_noalloc", None, p, 6144, p, p, p, p, p, None, 256, 32, 8, 128, p, p, p, 128, 1e-6,
                   0.1, 4096)
