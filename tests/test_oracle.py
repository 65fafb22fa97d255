"""Pins of the CPU oracle (CPU only).

Each oracle function is checked by something other than a retyping of its own formula:
the reference's own functions compiled from source (oracle/_ref), float64 brute force,
closed forms and invariants chosen so that a dropped term, a swapped operand or a wrong
index fails at least one of them.
"""
import numpy as np
import pytest

from tests.parity import ATTN_RTOL, bits_equal, rel_err

D = 128


# ---------------------------------------------------------------- generator
def test_generator_moments_and_determinism(orc):
    x = orc.normal((200000,), 42)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1.0) < 0.01
    assert np.abs(x).max() <= 8.6
    assert bits_equal(orc.normal((1000,), 42, 500), x[500:1500])  # counter-based: offsets compose
    assert not bits_equal(orc.normal((1000,), 43), x[:1000])


def _mix64(z):
    m = (1 << 64) - 1
    z = (z + 0x9E3779B97F4A7C15) & m
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    return z ^ (z >> 31)


def test_generator_is_box_muller(orc):
    """The generator is N(0,1) itself, not an approximation of it: every element equals
    float32(sqrt(-2 ln u1) cos(2 pi u2)) computed with numpy's float64 log / sqrt / cos from the
    same two 53-bit uniforms, bit for bit; and the sample passes a Kolmogorov-Smirnov test
    against the standard normal (a dropped factor 2 or a swapped sine moves both)."""
    from scipy import stats
    seed, n = 7, 20000
    x = orc.normal((n,), seed, 1000)
    m = (1 << 64) - 1
    ref = np.empty(n, np.float32)
    for i in range(n):
        base = (seed * 0xD1B54A32D192ED03 + 2 * (1000 + i)) & m
        h1, h2 = _mix64(base), _mix64((base + 1) & m)
        u1 = float((h1 >> 11) + 1) * 2.0 ** -53
        u2 = float(h2 >> 11) * 2.0 ** -53
        ref[i] = np.float32(np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2))
    assert bits_equal(x, ref)
    big = orc.normal((400000,), 11).astype(np.float64)
    assert stats.kstest(big, "norm").pvalue > 1e-3


# ---------------------------------------------------------------- QK-norm (src/ops.cpp:155-160)
def test_rmsnorm_bit_exact_vs_reference_source(orc):
    R = orc.ref_lib()
    if R is None:
        pytest.skip("reference tree absent: oracle/_ref not built")
    for s in range(200):
        scale = np.float32(10.0 ** ((s % 9) - 4))
        x = orc.normal((D,), 1000 + s) * scale
        w = orc.gamma(D, 2000 + s)
        ref = np.empty_like(x)
        R.elref_rmsnorm(ref, np.ascontiguousarray(x), w, D, 1e-6)
        assert bits_equal(orc.rmsnorm(x, w), ref)


def test_rmsnorm_closed_forms(orc):
    # constant vector c: rms = |c| (up to eps) -> out = sign(c) * w
    w = orc.gamma(D, 5)
    out = orc.rmsnorm(np.full(D, 3.0, np.float32), w, eps=0.0)
    assert np.allclose(out, w, rtol=1e-6)
    # float64 restatement of the definition on random input
    x = orc.normal((D,), 6) * np.float32(7)
    x64 = x.astype(np.float64)
    exact = x64 / np.sqrt(np.mean(x64 * x64) + 1e-6) * w.astype(np.float64)
    assert np.max(np.abs(orc.rmsnorm(x, w) - exact) / np.abs(exact).max()) < 5e-7
    # eps matters: a tiny vector is not blown up to unit rms
    tiny = np.full(D, 1e-5, np.float32)
    assert np.all(np.abs(orc.rmsnorm(tiny, np.ones(D, np.float32))) < 0.02)


# ---------------------------------------------------------------- RoPE (src/model.cpp:23-32, :105-109)
def test_rope_bit_exact_vs_reference_source(orc):
    R = orc.ref_lib()
    if R is None:
        pytest.skip("reference tree absent: oracle/_ref not built")
    for rope_dim, base in ((128, 1e6), (64, 1e4), (128, 1e4)):
        f = orc.rope_inv_freq(rope_dim, base)
        f_ref = np.empty(rope_dim // 2)
        R.elref_rope_inv_freq(f_ref, rope_dim, base)
        assert np.array_equal(f, f_ref)
        for pos in (0, 1, 7, 511, 4095, 32767, 131071):
            v = orc.normal((rope_dim,), pos + 3)
            r = v.copy()
            R.elref_rope(r, pos, rope_dim, f_ref)
            assert bits_equal(orc.rope(v, pos, f), r)


def test_rope_invariants(orc):
    f = orc.rope_inv_freq(128, 1e6)
    v = orc.normal((128,), 9)
    assert bits_equal(orc.rope(v, 0, f), v)  # position 0 is the identity
    for pos in (1, 100, 30000):
        r = orc.rope(v, pos, f).astype(np.float64)
        # each (i, i+64) pair is rotated: its norm is preserved
        n0 = v[:64].astype(np.float64) ** 2 + v[64:].astype(np.float64) ** 2
        n1 = r[:64] ** 2 + r[64:] ** 2
        assert np.allclose(n0, n1, rtol=1e-6)
        # pair 0 rotates by exactly pos radians (inv_freq[0] = 1)
        ang = np.arctan2(r[64], r[0]) - np.arctan2(v[64], v[0])
        assert abs(np.angle(np.exp(1j * (ang - pos)))) < 1e-5
    # relative-position property of q.k after rotation (the reason RoPE exists)
    q, k = orc.normal((128,), 10), orc.normal((128,), 11)
    d1 = np.dot(orc.rope(q, 50, f).astype(np.float64), orc.rope(k, 40, f).astype(np.float64))
    d2 = np.dot(orc.rope(q, 1010, f).astype(np.float64), orc.rope(k, 1000, f).astype(np.float64))
    assert abs(d1 - d2) < 1e-4 * np.linalg.norm(q) * np.linalg.norm(k)


def test_rope_table_equals_rope_of_unit_vectors(orc):
    """cs[p][i] is what rope() applies: rotating e_i gives (cos, sin) at (i, i+half)."""
    n_ctx = 50
    cs = orc.rope_table(n_ctx, 128, 1e6)
    f = orc.rope_inv_freq(128, 1e6)
    for p in (0, 1, 17, 49):
        for i in (0, 5, 63):
            e = np.zeros(128, np.float32)
            e[i] = 1.0
            r = orc.rope(e, p, f)
            assert r[i] == cs[p, i, 0] and r[i + 64] == cs[p, i, 1]


def test_headnorm_rope_rows_and_heads(orc):
    """Row b uses position pos0+b; heads are independent; columns past the heads untouched."""
    H, rows, pos0 = 3, 4, 10
    buf = orc.normal((rows, H * D + 8), 12)
    g = orc.gamma(D, 13)
    out = orc.headnorm_rope(buf, H, D, g, pos0, 128, 1e6, 1e-6)
    f = orc.rope_inv_freq(128, 1e6)
    for b in range(rows):
        for h in range(H):
            exp = orc.rope(orc.rmsnorm(buf[b, h * D:(h + 1) * D], g), pos0 + b, f)
            assert bits_equal(out[b, h * D:(h + 1) * D], exp)
        assert bits_equal(out[b, H * D:], buf[b, H * D:])


# ---------------------------------------------------------------- KV append (src/model.cpp:186-189)
def test_kv_append_writes_only_target_rows(orc):
    kd, n_ctx = 1024, 32
    kc = np.full((n_ctx, kd), 1.5, np.float32)
    vc = np.full((n_ctx, kd), -2.5, np.float32)
    k = orc.normal((3, kd), 1)
    v = orc.normal((3, kd), 2)
    orc.kv_append(k, v, kc, vc, 20)
    assert bits_equal(kc[20:23], k) and bits_equal(vc[20:23], v)
    assert np.all(kc[:20] == 1.5) and np.all(kc[23:] == 1.5)
    assert np.all(vc[:20] == -2.5) and np.all(vc[23:] == -2.5)


# ---------------------------------------------------------------- attention (src/model.cpp:191-214)
def _kv(orc, T, HKV, seed):
    return orc.normal((T, HKV, D), seed), orc.normal((T, HKV, D), seed + 1)


@pytest.mark.parametrize("H,HKV,T", [(4, 2, 1), (8, 2, 17), (16, 8, 300), (32, 8, 1000)])
def test_attn_decode_vs_float64(orc, H, HKV, T):
    k, v = _kv(orc, T, HKV, T)
    q = orc.normal((H, D), T + 100)
    out = orc.attn_decode(q, k, v, T, H, HKV, D)
    exact = orc.attn_f64(q, k, v, T, H, HKV, D)
    assert rel_err(out, exact) <= ATTN_RTOL


def test_attn_f64_textbook(orc):
    """Independent numpy float64 softmax attention (GQA by np.repeat, as the reference's
    numpy reference does, tests/parity_reference.py:77-82)."""
    H, HKV, T = 8, 2, 40
    k, v = _kv(orc, T, HKV, 3)
    q = orc.normal((H, D), 4)
    kk = np.repeat(k.astype(np.float64), H // HKV, axis=1)
    vv = np.repeat(v.astype(np.float64), H // HKV, axis=1)
    scale = np.float64(np.float32(1.0) / np.sqrt(np.float32(D)))  # the float scale, used in double
    s = np.einsum("hd,thd->ht", q.astype(np.float64), kk) * scale
    s = np.exp(s - s.max(axis=1, keepdims=True))
    s /= s.sum(axis=1, keepdims=True)
    exp = np.einsum("ht,thd->hd", s, vv)
    got = orc.attn_f64(q, k, v, T, H, HKV, D)
    assert np.max(np.abs(got - exp)) < 1e-12


def test_attn_closed_forms(orc):
    H, HKV = 8, 4
    # one key: the output is that key's V row exactly (p = 1)
    k, v = _kv(orc, 1, HKV, 7)
    q = orc.normal((H, D), 8)
    out = orc.attn_decode(q, k, v, 1, H, HKV, D)
    for h in range(H):
        assert bits_equal(out[h], v[0, h // (H // HKV)])
    # identical keys: uniform softmax -> mean of V
    T = 64
    k = np.repeat(orc.normal((1, HKV, D), 9), T, axis=0)
    v = orc.normal((T, HKV, D), 10)
    out = orc.attn_decode(q, k, v, T, H, HKV, D)
    for h in range(H):
        assert np.allclose(out[h], v[:, h // (H // HKV)].astype(np.float64).mean(0), rtol=1e-5, atol=1e-6)
    # a dominant score selects its V row
    T = 50
    k, v = _kv(orc, T, HKV, 11)
    qd = np.zeros((H, D), np.float32)
    qd[:, 0] = 400.0
    k[:, :, 0] = 0.0
    k[23, :, 0] = 1.0
    out = orc.attn_decode(qd, k, v, T, H, HKV, D)
    for h in range(H):
        assert np.allclose(out[h], v[23, h // (H // HKV)], rtol=1e-5, atol=1e-6)


def test_attn_gqa_equals_repeated_kv(orc):
    H, HKV, T = 16, 4, 90
    k, v = _kv(orc, T, HKV, 20)
    q = orc.normal((H, D), 21)
    gqa = orc.attn_decode(q, k, v, T, H, HKV, D)
    kr = np.ascontiguousarray(np.repeat(k, H // HKV, axis=1))
    vr = np.ascontiguousarray(np.repeat(v, H // HKV, axis=1))
    mha = orc.attn_decode(q, kr, vr, T, H, H, D)
    assert bits_equal(gqa, mha)


def test_prefill_is_per_token_decode_and_causal(orc):
    H, HKV, B, pos0 = 8, 2, 20, 5
    k, v = _kv(orc, pos0 + B, HKV, 30)
    q = orc.normal((B, H * D), 31)
    out = orc.attn_prefill(q, k, v, B, pos0, H, HKV, D)
    for b in (0, 7, 19):
        assert bits_equal(out[b], orc.attn_decode(q[b].reshape(H, D), k, v, pos0 + b + 1, H, HKV, D))
    # causality: future keys do not change earlier rows
    k2, v2 = k.copy(), v.copy()
    k2[pos0 + 10:] = 99.0
    v2[pos0 + 10:] = -99.0
    out2 = orc.attn_prefill(q, k2, v2, B, pos0, H, HKV, D)
    assert bits_equal(out[:10], out2[:10]) and not bits_equal(out[10:], out2[10:])


def test_split_combine_equals_single_pass(orc):
    H, HKV, T = 8, 4, 2000
    k, v = _kv(orc, T, HKV, 50)
    k[::512] *= np.float32(4.0)
    q = orc.normal((H, D), 51)
    single = orc.attn_decode(q, k, v, T, H, HKV, D)
    exact = orc.attn_f64(q, k, v, T, H, HKV, D)
    for ns in (1, 16, 37, 2000, 2500):  # includes empty splits (ns > T)
        sc = orc.attn_split_combine(q, k, v, T, H, HKV, D, nsplit=ns)
        assert rel_err(sc, single) <= ATTN_RTOL
        assert rel_err(sc, exact) <= ATTN_RTOL


def test_batched_equals_per_sequence(orc):
    H, HKV = 8, 4
    lens = np.array([1, 5, 300, 64], np.int32)
    offs = np.array([0, 10, 20, 400], np.int64)
    k, v = _kv(orc, 500, HKV, 60)
    q = orc.normal((4, H * D), 61)
    out = orc.attn_decode_batched(q, k, v, offs, lens, H, HKV, D)
    for s in range(4):
        ref = orc.attn_decode(q[s].reshape(H, D), k[offs[s]:], v[offs[s]:], int(lens[s]), H, HKV, D)
        assert bits_equal(out[s], ref)


# ---------------------------------------------------------------- golden fixtures
GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden"


def test_oracle_matches_reference_golden_vectors(orc):
    """Vectors produced by the reference's own rmsnorm / rope_inv_freq / rope (compiled from
    its sources; tests/golden/make_golden.py): the oracle reproduces every one bit for bit."""
    g = np.load(GOLDEN / "ref_qknorm_rope.npz")
    eps = float(g["eps"][0])
    for i in range(g["x"].shape[0]):
        assert bits_equal(orc.rmsnorm(g["x"][i], g["gamma"][i], eps), g["rmsnorm"][i])
    for rd, base in ((128, 1e6), (64, 1e4)):
        f = orc.rope_inv_freq(rd, base)
        assert np.array_equal(f, g[f"inv_freq_{rd}_{int(base)}"])
        for i, p in enumerate(g["pos"]):
            assert bits_equal(orc.rope(g[f"rope_in_{rd}_{int(base)}"][i], int(p), f),
                              g[f"rope_out_{rd}_{int(base)}"][i])


def test_oracle_attention_regression_fixture(orc):
    a = np.load(GOLDEN / "attn_small.npz")
    for name in ("gqa4_t1", "gqa2_t37", "gqa4_t300"):
        H, HKV, T = (int(x) for x in a[f"{name}_shape"])
        sq, sk, sv = (int(x) for x in a[f"{name}_seeds"])
        q, k, v = orc.normal((H, D), sq), orc.normal((T, HKV, D), sk), orc.normal((T, HKV, D), sv)
        out = orc.attn_decode(q, k, v, T, H, HKV, D)
        assert rel_err(out, a[f"{name}_f64"]) <= ATTN_RTOL


# ---------------------------------------------------------------- QKV projection (matvec)
def test_f16_conversion_matches_reference_on_every_pattern(orc):
    """orc_f16_to_f32 == the reference's f16_to_f32 (src/ops.cpp:22-24) on all 65536 binary16
    patterns: directly where oracle/_ref builds, and through the committed bit checksum."""
    allh = np.arange(1 << 16, dtype=np.uint16)
    conv = orc.f16_to_f32(allh)
    # numpy's binary16 -> binary32 conversion is exact too (NaNs compared by bits below)
    ref_np = allh.view(np.float16).astype(np.float32)
    finite = np.isfinite(ref_np)
    assert bits_equal(conv[finite], ref_np[finite])
    assert np.all(np.isnan(conv[~np.isfinite(ref_np) & np.isnan(ref_np)]))
    g = np.load(GOLDEN / "ref_matvec.npz")
    assert int(conv.view(np.uint32).astype(np.uint64).sum()) == int(g["f16_all_bits_sum"][0])
    R = orc.ref_lib()
    if R is not None and hasattr(R, "elref_f16_to_f32"):
        got = np.array([R.elref_f16_to_f32(int(h)) for h in allh[::97]], np.float32)
        assert bits_equal(got, conv[::97])


def test_dot_products_match_reference_golden_vectors(orc):
    """orc_dot_f32 / orc_dot_f16 reproduce the reference's dot_f32 / dot_f16 (src/ops.cpp:92-118,
    AVX2 FMA accumulators and hsum order) bit for bit, with and without scalar tails."""
    g = np.load(GOLDEN / "ref_matvec.npz")
    for n in (7, 8, 16, 31, 32, 37, 128, 2560, 2571):
        x, w32, w16 = g[f"x_{n}"], g[f"w32_{n}"], g[f"w16_{n}"]
        assert bits_equal(np.float32(orc.dot(w32, x, orc.W_F32)), g[f"dot32_{n}"][0]), f"dot_f32 n={n}"
        assert bits_equal(np.float32(orc.dot(w16, x, orc.W_F16)), g[f"dot16_{n}"][0]), f"dot_f16 n={n}"


def test_dot_products_match_reference_built_from_source(orc):
    R = orc.ref_lib()
    if R is None or not hasattr(R, "elref_dot_f32"):
        pytest.skip("oracle/_ref not built (reference tree absent)")
    rng = np.random.default_rng(9)
    for n in (1, 9, 15, 17, 33, 63, 65, 1000, 4096, 4099):
        x = orc.normal((n,), 9100 + n) * np.float32(rng.uniform(0.01, 100))
        w32 = orc.normal((n,), 9200 + n)
        w16 = np.float32(rng.standard_normal(n)).astype(np.float16).view(np.uint16)
        assert bits_equal(np.float32(orc.dot(w32, x, orc.W_F32)), np.float32(R.elref_dot_f32(w32, x, n)))
        assert bits_equal(np.float32(orc.dot(w16, x, orc.W_F16)), np.float32(R.elref_dot_f16(w16, x, n)))


def test_matvec_is_the_float64_product_within_fp32_rounding(orc):
    """Independent of the summation order: |y - W x (float64)| <= 1e-6 * sum |w_i x_i| per row, and a
    dropped or doubled term (an off-by-one in the block loops) would far exceed it."""
    rows, n = 64, 2560
    x = orc.normal((n,), 9300)
    w = orc.normal((rows, n), 9301)
    y = orc.matvec(w, x, orc.W_F32)
    exact = w.astype(np.float64) @ x.astype(np.float64)
    mag = np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64))
    assert np.all(np.abs(y - exact) <= 1e-6 * mag)
    w16 = w.astype(np.float16)
    y16 = orc.matvec(w16.view(np.uint16), x, orc.W_F16)
    exact16 = w16.astype(np.float64) @ x.astype(np.float64)
    assert np.all(np.abs(y16 - exact16) <= 1e-6 * mag)
    # the same bound rejects a matvec missing its last block
    bad = (w[:, :-16].astype(np.float64) @ x[:-16].astype(np.float64))
    assert np.any(np.abs(bad - exact) > 1e-6 * mag)


@pytest.mark.parametrize("wtype", [8, 12, 14])
def test_dequant_matches_reference(orc, wtype):
    """orc_dequant_q8_0 / _q4_K / _q6_K == the reference's dequant_* (src/quant.cpp:7-60) bit for
    bit on random blocks (every byte random, scales included): directly where oracle/_ref builds,
    and through the committed golden vectors."""
    names = {8: "q8_0", 12: "q4_K", 14: "q6_K"}
    g = np.load(GOLDEN / "ref_dequant.npz")
    blocks, want = g[f"{names[wtype]}_blocks"], g[f"{names[wtype]}_out"]
    n = want.size // blocks.shape[0]
    assert bits_equal(orc.dequant(wtype, blocks, n), want)
    R = orc.ref_lib()
    if R is not None:
        for seed in range(4):
            b = np.random.default_rng(9100 + seed).integers(0, 256, size=(3, orc.row_bytes(wtype, 1024)),
                                                            dtype=np.uint8)
            ref = np.empty(3 * 1024, np.float32)
            getattr(R, "elref_dequant_" + names[wtype])(b.ctypes.data, ref, ref.size)
            assert bits_equal(orc.dequant(wtype, b, 1024), ref)


@pytest.mark.parametrize("wtype", [8, 12, 14])
def test_dequant_closed_forms(orc, wtype):
    """Block scales of 1 give the stored integers back: Q8_0 q; Q4_K sub-block scale s and min
    m give s q - m; Q6_K scale s gives s (q - 32).  A transposed nibble, a wrong sub-block or a
    misplaced high bit changes the integers the bytes spell out."""
    rng = np.random.default_rng(9200 + wtype)
    one = np.float16(1.0).view(np.uint16)
    if wtype == 8:
        blk = rng.integers(0, 256, size=(1, 34), dtype=np.uint8)
        blk[0, 0], blk[0, 1] = one & 0xFF, one >> 8
        assert np.array_equal(orc.dequant(8, blk, 32), blk[0, 2:].view(np.int8).astype(np.float32))
    elif wtype == 12:
        blk = rng.integers(0, 256, size=(1, 144), dtype=np.uint8)
        blk[0, 0], blk[0, 1], blk[0, 2], blk[0, 3] = one & 0xFF, one >> 8, one & 0xFF, one >> 8
        p = blk[0, 4:16].astype(int)
        sc = [p[j] & 63 if j < 4 else (p[j + 4] & 15) | ((p[j - 4] >> 6) << 4) for j in range(8)]
        mn = [p[j + 4] & 63 if j < 4 else (p[j + 4] >> 4) | ((p[j] >> 6) << 4) for j in range(8)]
        qs = blk[0, 16:].astype(int)
        want = np.empty(256)
        for c in range(4):
            want[64 * c:64 * c + 32] = sc[2 * c] * (qs[32 * c:32 * c + 32] & 15) - mn[2 * c]
            want[64 * c + 32:64 * c + 64] = sc[2 * c + 1] * (qs[32 * c:32 * c + 32] >> 4) - mn[2 * c + 1]
        assert np.array_equal(orc.dequant(12, blk, 256), want.astype(np.float32))
    else:
        blk = rng.integers(0, 256, size=(1, 210), dtype=np.uint8)
        blk[0, 208], blk[0, 209] = one & 0xFF, one >> 8
        ql, qh, scl = blk[0, :128].astype(int), blk[0, 128:192].astype(int), blk[0, 192:208].view(np.int8).astype(int)
        want = np.empty(256)
        for v in range(256):
            h, r = divmod(v, 128)
            g, l = divmod(r, 32)
            lo = ql[64 * h + l + 32 * (g & 1)]
            q = ((lo & 15) if g < 2 else (lo >> 4)) | (((qh[32 * h + l] >> (2 * g)) & 3) << 4)
            want[v] = scl[8 * h + l // 16 + 2 * g] * (q - 32)
        assert np.array_equal(orc.dequant(14, blk, 256), want.astype(np.float32))


def test_quantised_matvec_is_decode_then_dot_f32(orc):
    """orc_matvec on quantised rows == dot_f32 of each decoded row (the reference's convert_row +
    dot_f32, src/ops.cpp:126-153)."""
    x = orc.normal((2560,), 9300)
    for wtype in (8, 12, 14):
        blocks = orc.random_blocks(wtype, 8, 2560, 9310 + wtype)
        wf = orc.dequant(wtype, blocks, 2560).reshape(8, 2560)
        y = orc.matvec(blocks, x, wtype)
        assert bits_equal(y, np.array([orc.dot(wf[r], x, orc.W_F32) for r in range(8)], np.float32))
