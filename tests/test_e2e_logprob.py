"""End-to-end gate |delta logprob| <= 2.7e-5 on a synthetic tiny Qwen3 (tests/tiny_qwen3.py).

The reference quotes max |delta logprob| <= 2.7e-5 against its numpy forward
(tests/parity_reference.py:35-107, README); that harness needs GGUF weights, which this
environment lacks.  The same gate is applied here to a random-weight model with Qwen3's block
structure: one run with the CPU restatement of the reference's attention (src/model.cpp:174-214),
one with this build's HIP path (prefill chunks through ei_prefill_step, decode steps through
ei_decode_step), all other arithmetic shared.  The CPU tests check the harness
itself: the float32 reference attention sits well inside the gate against a float64 one, and a
plausible mistake (softmax scale 1/sqrt(127)) falls outside it.
"""
import numpy as np
import pytest

from tests.tiny_qwen3 import HEAD_DIM, TinyQwen3, oracle_attention, run_sequence

LOGPROB_TOL = 2.7e-5
CHUNKS = [32, 16]  # prompt of 48 tokens in two prefill chunks (the second at pos0 = 32)
N_DECODE = 8
N_CTX = 64


def _tokens(model, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(0, model.V, size=sum(CHUNKS) + N_DECODE + 1)


def test_harness_reference_vs_f64(orc):
    model = TinyQwen3(seed=7)
    toks = _tokens(model, 8)
    lp32 = run_sequence(model, oracle_attention(model, orc), toks, CHUNKS, N_DECODE, N_CTX)
    lp64 = run_sequence(model, oracle_attention(model, orc, f64=True), toks, CHUNKS, N_DECODE, N_CTX)
    assert np.isfinite(lp32).all()
    d = float(np.max(np.abs(lp32 - lp64)))
    assert d <= LOGPROB_TOL / 4, f"float32 reference attention drifts {d:.2e} from float64"


def test_harness_detects_wrong_scale(orc):
    model = TinyQwen3(seed=7)
    toks = _tokens(model, 8)
    good = run_sequence(model, oracle_attention(model, orc), toks, CHUNKS, N_DECODE, N_CTX)
    bad_scale = float(np.float32(1.0) / np.sqrt(np.float32(HEAD_DIM - 1)))
    bad = run_sequence(model, oracle_attention(model, orc, scale=bad_scale), toks, CHUNKS, N_DECODE, N_CTX)
    assert float(np.max(np.abs(good - bad))) > 10 * LOGPROB_TOL


def _hip_attention(model, A, torch):
    D, H, HKV = HEAD_DIM, model.H, model.HKV
    shape = A.AttnShape(H, HKV)

    def factory(n_ctx):
        dev = "cuda"
        kc = [torch.zeros((n_ctx, HKV * D), device=dev) for _ in range(model.n_layer)]
        vc = [torch.zeros((n_ctx, HKV * D), device=dev) for _ in range(model.n_layer)]
        qg = [torch.from_numpy(L["q_norm"]).to(dev) for L in model.layers]
        kg = [torch.from_numpy(L["k_norm"]).to(dev) for L in model.layers]
        cs = A.rope_table(n_ctx, device=dev)
        ws = A.DecodeWorkspace(1, H, HKV, n_ctx, device=dev)
        pws = A.PrefillWorkspace(n_ctx, H, HKV, n_ctx, device=dev)

        def attn(l, qkv, pos0):
            n = qkv.shape[0]
            t = torch.from_numpy(qkv).to(dev)
            pos = torch.tensor([pos0], dtype=torch.int32, device=dev)
            if n == 1:
                out = A.decode_step(t, kc[l], vc[l], shape, qg[l], kg[l], cs, ws, pos_dev=pos)
            else:
                out = A.prefill_step(t, kc[l], vc[l], shape, qg[l], kg[l], cs, pos, pws)
            torch.cuda.synchronize()
            return out.cpu().numpy().reshape(n, H * D)

        return attn

    return factory


@pytest.mark.gpu
@pytest.mark.parametrize("n_head,n_head_kv", [(4, 2), (8, 2), (10, 2)])
def test_e2e_logprob_hip_vs_reference(orc, gpu, n_head, n_head_kv):
    import torch
    model = TinyQwen3(seed=11, n_head=n_head, n_head_kv=n_head_kv)
    toks = _tokens(model, 12)
    ref = run_sequence(model, oracle_attention(model, orc), toks, CHUNKS, N_DECODE, N_CTX)
    hip = run_sequence(model, _hip_attention(model, gpu, torch), toks, CHUNKS, N_DECODE, N_CTX)
    d = float(np.max(np.abs(hip - ref)))
    print(f"e2e H={n_head} HKV={n_head_kv}: max |d logprob| = {d:.3e} over {len(ref)} positions", flush=True)
    assert d <= LOGPROB_TOL, f"max |delta logprob| {d:.2e} > {LOGPROB_TOL}"


@pytest.mark.gpu
def test_e2e_logprob_longer_prompt(orc, gpu):
    """Four layers, a 320-token prompt in chunks of 128, 128 and 64 (the later chunks at pos0 > 0
    take key-split prefill shares through ei_prefill_step), then 24 decode steps at contexts
    past 320: the same gate."""
    import torch
    model = TinyQwen3(seed=31, n_layer=4, n_head=8, n_head_kv=2)
    chunks, n_decode, n_ctx = [128, 128, 64], 24, 512
    toks = np.random.default_rng(32).integers(0, model.V, size=sum(chunks) + n_decode + 1)
    ref = run_sequence(model, oracle_attention(model, orc), toks, chunks, n_decode, n_ctx)
    hip = run_sequence(model, _hip_attention(model, gpu, torch), toks, chunks, n_decode, n_ctx)
    d = float(np.max(np.abs(hip - ref)))
    print(f"e2e long: max |d logprob| = {d:.3e} over {len(ref)} positions", flush=True)
    assert d <= LOGPROB_TOL, f"max |delta logprob| {d:.2e} > {LOGPROB_TOL}"


@pytest.mark.gpu
def test_serve_prefix_reuse_equals_generate(orc, gpu):
    """The reference's serve invariant (tests/serve_test.py): a persistent server reusing the
    KV rows of a cached common prefix produces the same greedy tokens as a fresh generate, on
    this build's HIP attention; the generated tokens' logprobs agree within the e2e gate."""
    import torch
    from tests.tiny_qwen3 import PrefixServer, greedy_generate

    model = TinyQwen3(seed=21, n_head=8, n_head_kv=2)
    rng = np.random.default_rng(22)
    n, chunk, n_ctx = 12, 32, 160
    p1 = rng.integers(0, model.V, size=40)
    factory = _hip_attention(model, gpu, torch)
    srv = PrefixServer(model, factory, n_ctx, chunk)
    t1, _, s1 = srv.request(p1, n)
    p2 = np.concatenate([p1, np.array(t1[:5]), rng.integers(0, model.V, size=9)])  # continuation turn
    p3 = p1.copy()                                                                 # same prompt again
    p4 = rng.integers(0, model.V, size=23)                                         # unrelated prompt
    cases = [("first", p1, t1, s1)]
    for name, p in (("continuation", p2), ("same prompt", p3), ("unrelated", p4)):
        t, lp, s = srv.request(p, n)
        cases.append((name, p, t, s))
        tf, lpf = greedy_generate(model, factory(n_ctx), p, n, chunk)
        assert t == tf, f"{name}: serve {t} != generate {tf}"
        d = float(np.max(np.abs(lp - lpf)))
        assert d <= LOGPROB_TOL, f"{name}: |d logprob| {d:.2e}"
    starts = {name: s for name, _, _, s in cases}
    assert starts["continuation"] == len(p1) + 5 and starts["same prompt"] == len(p1) - 1 and starts["unrelated"] == 0


@pytest.mark.gpu
@pytest.mark.parametrize("f16", [False, True])
def test_e2e_logprob_model_read_from_gguf(orc, gpu, tmp_path, f16):
    """The gate on a model that reaches the harness through a GGUF file and this build's reader
    (tests/golden/write_tiny_gguf.py writes it; read_config / read_tensors validation,
    src/model.cpp:38-103): F32 and F16 weights, HIP attention against the reference's."""
    import torch
    from tests.golden.write_tiny_gguf import qwen3_metadata, qwen3_tensors, write_gguf
    src = TinyQwen3(seed=41, n_layer=3, n_head=8, n_head_kv=2)
    path = tmp_path / "tiny.gguf"
    write_gguf(path, qwen3_metadata(src), qwen3_tensors(src, f16))
    model = TinyQwen3.from_gguf(path)
    toks = np.random.default_rng(42).integers(0, model.V, size=sum(CHUNKS) + N_DECODE + 1)
    ref = run_sequence(model, oracle_attention(model, orc), toks, CHUNKS, N_DECODE, N_CTX)
    hip = run_sequence(model, _hip_attention(model, gpu, torch), toks, CHUNKS, N_DECODE, N_CTX)
    d = float(np.max(np.abs(hip - ref)))
    print(f"e2e from GGUF ({'F16' if f16 else 'F32'}): max |d logprob| = {d:.3e} over {len(ref)} positions",
          flush=True)
    assert d <= LOGPROB_TOL, f"max |delta logprob| {d:.2e} > {LOGPROB_TOL}"


def _hip_projection(model, torch):
    """project(l, x) on the GPU: ei_qkv_project on the file's own Wq, Wk, Wv bytes (one call per
    segment and per four rows), the rows left raw for the attention step."""
    from exactinfer_amd import _capi
    from exactinfer_amd import attention as A
    dev = "cuda"
    segs = [[(ty, torch.from_numpy(np.ascontiguousarray(w).view(np.uint8)).to(dev), w.shape[0])
             for ty, w in L["qkv_raw"]] for L in model.layers]
    gam = [torch.from_numpy(L["attn_norm"]).to(dev) for L in model.layers]
    width = (model.H + 2 * model.HKV) * HEAD_DIM

    def project(l, x):
        n, E = x.shape
        xd = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(dev)
        out = torch.empty((n, width), dtype=torch.float32, device=dev)
        for r0 in range(0, n, 4):
            rows, col = min(4, n - r0), 0
            for ty, wd, nrows in segs[l]:
                _capi.call("ei_qkv_project", A._stream(), xd[r0].data_ptr(), E, rows, E, gam[l].data_ptr(), 1e-6,
                           wd.data_ptr(), ty, nrows, out[r0, col:].data_ptr(), width)
                col += nrows
        torch.cuda.synchronize()
        return out.cpu().numpy()

    return project


@pytest.mark.gpu
@pytest.mark.parametrize("weights", ["q8_0", "q4_k", "q6_k", "f16"])
def test_e2e_logprob_gpu_projection_from_gguf(orc, gpu, tmp_path, weights):
    """More of the layer on the GPU: the model read from a GGUF file (Wq, Wk, Wv as Q8_0, Q4_K or
    Q6_K blocks, or F16), its attention RMSNorm + QKV projection through ei_qkv_project on the file's bytes, then
    the HIP attention steps; against the reference's CPU chain on the same bytes (rmsnorm, matvec
    of the stored weights, the reference attention).  The same |delta logprob| gate."""
    import torch
    from tests.golden.write_tiny_gguf import qwen3_metadata, qwen3_tensors, write_gguf
    from tests.tiny_qwen3 import oracle_projection
    src = TinyQwen3(seed=51, n_layer=2, n_embd=1024, n_head=8, n_head_kv=2, n_ff=512)
    path = tmp_path / "tiny_proj.gguf"
    write_gguf(path, qwen3_metadata(src), qwen3_tensors(src, weights == "f16",
                                                                 attn_type=None if weights == "f16" else weights))
    model = TinyQwen3.from_gguf(path, dequant=orc.dequant)
    toks = np.random.default_rng(52).integers(0, model.V, size=sum(CHUNKS) + N_DECODE + 1)
    ref = run_sequence(model, oracle_attention(model, orc), toks, CHUNKS, N_DECODE, N_CTX,
                       project=oracle_projection(model, orc))
    hip = run_sequence(model, _hip_attention(model, gpu, torch), toks, CHUNKS, N_DECODE, N_CTX,
                       project=_hip_projection(model, torch))
    d = float(np.max(np.abs(hip - ref)))
    print(f"e2e GPU projection ({weights}): max |d logprob| = {d:.3e} over {len(ref)} positions", flush=True)
    assert d <= LOGPROB_TOL, f"max |delta logprob| {d:.2e} > {LOGPROB_TOL}"
