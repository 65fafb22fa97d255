"""The GGUF reader (exactinfer_amd/host/gguf_index.cpp and qwen3_schema.cpp through include/ei_gguf.h), CPU only.

Files come from tests/golden/write_tiny_gguf.py (a tiny synthetic Qwen3; no real Qwen3 GGUF
exists here, so a real file stays unread).  Checked: the tensor table and metadata against the
writer's inputs and against an independent minimal parser; Qwen3 configuration and shape
validation (read_config / read_tensors, src/model.cpp:38-103); and every class of malformed file
the reference reader rejects (src/gguf.cpp:203-254): truncation anywhere, wrong magic or version,
implausible counts, bad dimensions or types, repeated keys or names, bad alignment, tensors
misaligned or past the end.  The forward pass of the model read back equals the in-memory one."""
import shutil
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

from tests.golden.write_tiny_gguf import (T_ARRAY, T_F32, T_I32, T_STRING, T_U32, Quantised, qwen3_metadata,
                                         qwen3_tensors, write_gguf)
from tests.tiny_qwen3 import TinyQwen3, oracle_attention, run_sequence


@pytest.fixture(scope="module")
def model():
    return TinyQwen3(seed=7)


def _write(tmp_path, model, f16=False, name="m.gguf", meta=None, tensors=None, **kw):
    p = tmp_path / name
    write_gguf(p, meta if meta is not None else qwen3_metadata(model),
               tensors if tensors is not None else qwen3_tensors(model, f16), **kw)
    return p


def _parse_independently(path):
    """A minimal parser of the tensor table (a second reading of the format, not the reader)."""
    b = path.read_bytes()
    at = [0]

    def rd(fmt):
        v = struct.unpack_from(fmt, b, at[0])
        at[0] += struct.calcsize(fmt)
        return v[0]

    def rs():
        n = rd("<Q")
        s = b[at[0]:at[0] + n].decode()
        at[0] += n
        return s

    def rv(t):
        if t == T_STRING:
            return rs()
        if t == T_ARRAY:
            et, n = rd("<I"), rd("<Q")
            return [rv(et) for _ in range(n)]
        return rd({4: "<I", 6: "<f", 5: "<i", 10: "<Q", 12: "<d"}[t])

    assert rd("<I") == 0x46554747
    rd("<I")
    nt, nkv = rd("<Q"), rd("<Q")
    meta = {}
    for _ in range(nkv):
        k, t = rs(), rd("<I")
        meta[k] = rv(t)
    tensors = {}
    for _ in range(nt):
        name, nd = rs(), rd("<I")
        ne = [rd("<Q") for _ in range(nd)]
        tensors[name] = (ne, rd("<I"), rd("<Q"))
    align = meta.get("general.alignment", 32)
    return meta, tensors, (at[0] + align - 1) // align * align


@pytest.mark.parametrize("f16", [False, True])
def test_reader_returns_what_was_written(tmp_path, model, f16):
    from exactinfer_amd.gguf import GgufFile
    p = _write(tmp_path, model, f16)
    tens = qwen3_tensors(model, f16)
    meta_i, tab_i, data_start = _parse_independently(p)
    raw = p.read_bytes()
    with GgufFile(p) as g:
        assert g.version == 3
        assert g.tensor_names() == [n for n, _ in tens]
        for name, a in tens:
            got = g.tensor(name)
            assert got.dtype == a.dtype and got.shape == a.shape, name
            assert np.array_equal(got.view(np.uint8), a.view(np.uint8)), name
            ty, ne, nb = g.tensor_info(name)
            assert (ne, ty) == (tab_i[name][0], tab_i[name][1]) and nb == a.nbytes
            off = data_start + tab_i[name][2]
            assert raw[off:off + nb] == a.tobytes()
        assert g.get_str("general.architecture") == "qwen3"
        assert g.get_int("qwen3.block_count") == model.n_layer == meta_i["qwen3.block_count"]
        assert g.get_float("qwen3.rope.freq_base") == np.float32(1e6)
        assert g.get_float("qwen3.block_count") == model.n_layer  # integers read as numbers too
        c = g.qwen3_config()
        assert (c["n_layer"], c["n_embd"], c["n_head"], c["n_head_kv"], c["head_dim"], c["rope_dim"], c["n_vocab"],
                c["n_ff"], c["n_ctx_train"]) == (model.n_layer, model.E, model.H, model.HKV, 128, 128, model.V, 512,
                                                 4096)
        assert np.float32(c["eps"]) == np.float32(1e-6) and c["rope_base"] == np.float32(1e6)
        assert g.tensor_info("no.such.tensor") is None


def test_missing_and_mistyped_metadata(tmp_path, model):
    from exactinfer_amd.gguf import GgufError, GgufFile
    with GgufFile(_write(tmp_path, model)) as g:
        with pytest.raises(GgufError, match="metadata missing"):
            g.get_int("qwen3.nothing")
        with pytest.raises(GgufError, match="not an integer"):
            g.get_int("general.architecture")
        with pytest.raises(GgufError, match="not a string"):
            g.get_str("qwen3.block_count")
        with pytest.raises(GgufError, match="tensor missing"):
            g.tensor("nothing")


def test_model_read_back_runs_the_same_forward(tmp_path, model, orc):
    """The model loaded through the reader gives bit-identical logprobs to the one written."""
    toks = np.random.default_rng(8).integers(0, model.V, 41)
    ref = run_sequence(model, oracle_attention(model, orc), toks, [16, 16], 8, 64)
    m2 = TinyQwen3.from_gguf(_write(tmp_path, model))
    got = run_sequence(m2, oracle_attention(m2, orc), toks, [16, 16], 8, 64)
    assert np.array_equal(got, ref)
    m16 = TinyQwen3.from_gguf(_write(tmp_path, model, f16=True, name="h.gguf"))
    assert np.array_equal(m16.layers[1]["wo"], model.layers[1]["wo"].astype(np.float16).astype(np.float32))


def _expect_rejected(path, match):
    from exactinfer_amd.gguf import GgufError, GgufFile
    with pytest.raises(GgufError, match=match):
        GgufFile(path)


def test_truncated_files_are_rejected_anywhere(tmp_path, model):
    p = _write(tmp_path, model)
    raw = p.read_bytes()
    meta_i, tab_i, data_start = _parse_independently(p)
    last = max(tab_i.values(), key=lambda t: t[2])
    cuts = [0, 3, 7, 20, 40, 100, 300, data_start - 1, data_start + last[2] + 5]
    for k, cut in enumerate(cuts):
        q = tmp_path / f"cut{k}.gguf"
        q.write_bytes(raw[:cut])
        _expect_rejected(q, "empty|ends early|past the end|wrong magic")


def _patched(tmp_path, raw, off, fmt, value, name):
    b = bytearray(raw)
    struct.pack_into(fmt, b, off, value)
    q = tmp_path / name
    q.write_bytes(bytes(b))
    return q


def test_header_errors(tmp_path, model):
    raw = _write(tmp_path, model).read_bytes()
    _expect_rejected(_patched(tmp_path, raw, 0, "<I", 0x46554748, "magic.gguf"), "wrong magic")
    _expect_rejected(_patched(tmp_path, raw, 4, "<I", 1, "v1.gguf"), "version 1")
    _expect_rejected(_patched(tmp_path, raw, 8, "<Q", 200000, "nt.gguf"), "count is not plausible")
    _expect_rejected(_patched(tmp_path, raw, 16, "<Q", 1 << 40, "nkv.gguf"), "count is not plausible")
    # the first key's string length
    _expect_rejected(_patched(tmp_path, raw, 24, "<Q", 1 << 30, "slen.gguf"), "string length")


def test_tensor_table_errors(tmp_path, model):
    from tests.golden.write_tiny_gguf import _s
    tens = qwen3_tensors(model, False)
    meta = qwen3_metadata(model)
    # repeated key / tensor name
    _expect_rejected(_write(tmp_path, model, name="k.gguf", meta=meta + [meta[1]]), "key repeated")
    _expect_rejected(_write(tmp_path, model, name="t.gguf", tensors=tens + [tens[0]]), "name repeated")
    # bad alignment value
    bad = [m if m[0] != "general.alignment" else (m[0], T_U32, 48) for m in meta]
    _expect_rejected(_write(tmp_path, model, name="a.gguf", meta=bad, alignment=32), "alignment 48")
    # patch the first tensor's info: n_dims 0, unknown type, misaligned and out-of-range offsets
    p = _write(tmp_path, model, name="base.gguf")
    raw = p.read_bytes()
    i = raw.index(_s("token_embd.weight")) + len(_s("token_embd.weight"))
    _expect_rejected(_patched(tmp_path, raw, i, "<I", 0, "nd.gguf"), "0 dimensions")
    _expect_rejected(_patched(tmp_path, raw, i, "<I", 5, "nd5.gguf"), "5 dimensions")
    _expect_rejected(_patched(tmp_path, raw, i + 4, "<Q", 0, "dim0.gguf"), "bad shape")
    _expect_rejected(_patched(tmp_path, raw, i + 20, "<I", 99, "ty.gguf"), "unknown type 99")
    q8 = _patched(tmp_path, raw, i + 20, "<I", 8, "q8.gguf").read_bytes()  # Q8_0: blocks of 32 elements
    _expect_rejected(_patched(tmp_path, q8, i + 4, "<Q", 48, "blk.gguf"), "whole number of blocks")
    _expect_rejected(_patched(tmp_path, raw, i + 24, "<Q", 4, "mis.gguf"), "not aligned")
    _expect_rejected(_patched(tmp_path, raw, i + 24, "<Q", 1 << 32, "far.gguf"), "past the end")


def test_qwen3_validation(tmp_path, model):
    from exactinfer_amd.gguf import GgufError, GgufFile
    meta = qwen3_metadata(model)
    tens = qwen3_tensors(model, False)

    def cfg_error(meta_=None, tens_=None, name="x.gguf"):
        with GgufFile(_write(tmp_path, model, name=name, meta=meta_ or meta, tensors=tens_ or tens)) as g:
            with pytest.raises(GgufError) as e:
                g.qwen3_config()
        return str(e.value)

    arch = [m if m[0] != "general.architecture" else (m[0], T_STRING, "llama") for m in meta]
    assert "unsupported architecture" in cfg_error(arch, name="arch.gguf")
    assert "RoPE scaling" in cfg_error(meta + [("qwen3.rope.scaling.type", T_STRING, "linear")], name="rs.gguf")
    odd = [m if m[0] != "qwen3.attention.head_count_kv" else (m[0], T_U32, 3) for m in meta]
    assert "invalid model configuration" in cfg_error(odd, name="kv.gguf")
    no_norm = [t for t in tens if t[0] != "blk.1.attn_k_norm.weight"]
    assert "tensor missing: blk.1.attn_k_norm.weight" in cfg_error(tens_=no_norm, name="nn.gguf")
    bias = tens + [("blk.0.attn_q.bias", np.zeros(512, np.float32))]
    assert "bias" in cfg_error(tens_=bias, name="bias.gguf")
    wrong = [(n, a if n != "blk.0.attn_v.weight" else a[:128]) for n, a in tens]
    assert "blk.0.attn_v.weight has shape [256,128], expected [256,256]" in cfg_error(tens_=wrong, name="sh.gguf")
    # a tied embedding (no output.weight) is accepted
    with GgufFile(_write(tmp_path, model, name="tied.gguf", tensors=[t for t in tens if t[0] != "output.weight"])) as g:
        assert g.qwen3_config()["n_vocab"] == model.V


def mixed_type_file(tmp_path, orc, E=1024, H=8, HKV=2, seed=8900):
    """A one-layer Qwen3 file in the layout of a Q4_K_M quantisation: Wq Q4_K, Wk Q8_0, Wv Q6_K
    (random blocks with moderate scales), the rest F32.  Returns the path and the q/k/v blocks."""
    D, FF, V = 128, 512, 256
    rng = np.random.default_rng(seed)
    f = lambda *shape: rng.standard_normal(shape).astype(np.float32) * np.float32(0.05)
    q = orc.random_blocks(orc.W_Q4_K, H * D, E, seed + 1, d_scale=0.05)
    k = orc.random_blocks(orc.W_Q8_0, HKV * D, E, seed + 2, d_scale=0.05)
    v = orc.random_blocks(orc.W_Q6_K, HKV * D, E, seed + 3, d_scale=0.05)
    tens = [("token_embd.weight", f(V, E)), ("output_norm.weight", np.ones(E, np.float32)),
            ("blk.0.attn_norm.weight", np.ones(E, np.float32)),
            ("blk.0.attn_q.weight", Quantised(orc.W_Q4_K, (E, H * D), q)),
            ("blk.0.attn_k.weight", Quantised(orc.W_Q8_0, (E, HKV * D), k)),
            ("blk.0.attn_v.weight", Quantised(orc.W_Q6_K, (E, HKV * D), v)),
            ("blk.0.attn_q_norm.weight", np.ones(D, np.float32)), ("blk.0.attn_k_norm.weight", np.ones(D, np.float32)),
            ("blk.0.attn_output.weight", f(E, H * D)), ("blk.0.ffn_norm.weight", np.ones(E, np.float32)),
            ("blk.0.ffn_gate.weight", f(FF, E)), ("blk.0.ffn_up.weight", f(FF, E)), ("blk.0.ffn_down.weight", f(E, FF))]

    class M:
        pass
    m = M()
    m.n_layer, m.E, m.H, m.HKV = 1, E, H, HKV
    m.layers = [{"wg": np.zeros((FF, 1))}]
    p = tmp_path / "mixed.gguf"
    write_gguf(p, qwen3_metadata(m), tens)
    return p, q, k, v


def test_quantised_tensors_read_back(tmp_path, orc):
    """Q4_K / Q8_0 / Q6_K tensors: the reader accepts the Qwen3 table with these types and hands
    back each tensor's bytes as written, [rows][row bytes]."""
    from exactinfer_amd.gguf import GgufFile
    p, q, k, v = mixed_type_file(tmp_path, orc)
    with GgufFile(p) as g:
        c = g.qwen3_config()
        assert (c["n_embd"], c["n_head"], c["n_head_kv"]) == (1024, 8, 2)
        for name, want, ty in (("blk.0.attn_q.weight", q, 12), ("blk.0.attn_k.weight", k, 8),
                               ("blk.0.attn_v.weight", v, 14)):
            got = g.tensor(name)
            assert got.dtype == np.uint8 and got.shape == want.shape and np.array_equal(got, want), name
            assert g.tensor_info(name)[0] == ty


def test_q8_0_attention_weights_round_trip(tmp_path, orc):
    """The writer's Q8_0 projections read back as the same blocks, and decode (the reference's
    dequant) to within half a quantisation step of the weights they were made from."""
    from exactinfer_amd.gguf import GgufFile
    m = TinyQwen3(seed=61, n_layer=1, n_embd=256, n_head=4, n_head_kv=2)
    p = _write(tmp_path, m, tensors=qwen3_tensors(m, False, q8_attn=True))
    with GgufFile(p) as g:
        blocks = g.tensor("blk.0.attn_q.weight")
        assert g.tensor_info("blk.0.attn_q.weight")[0] == 8 and blocks.shape == (4 * 128, 256 // 32 * 34)
    w = m.layers[0]["wqkv"][:4 * 128]
    dq = orc.dequant(8, blocks, 256).reshape(w.shape)
    d = np.abs(w).reshape(w.shape[0], -1, 32).max(axis=2) / 127.0
    assert np.all(np.abs(dq - w).reshape(w.shape[0], -1, 32) <= 0.5 * d[..., None] * 1.01 + 1e-6)
    model = TinyQwen3.from_gguf(p, dequant=orc.dequant)
    assert np.array_equal(model.layers[0]["wqkv"][:4 * 128], dq)


@pytest.mark.parametrize("attn_type,tid,rel_bound", [("q4_k", 12, 0.08), ("q6_k", 14, 0.025)])
def test_k_quant_attention_weights_round_trip(tmp_path, orc, attn_type, tid, rel_bound):
    """The writer's Q4_K / Q6_K encoders: the projections read back as the same blocks, and the
    reference's decode of those blocks gives back the weights they were made from, to within the
    format's resolution (16 levels per 32 values for Q4_K, 64 per 16 for Q6_K).  A byte or nibble
    placed where the decoder does not look for it would leave the decoded rows uncorrelated with
    the weights, so this pins the encoders' layout to the reference's decoder."""
    from exactinfer_amd.gguf import GgufFile
    m = TinyQwen3(seed=62, n_layer=1, n_embd=512, n_head=4, n_head_kv=2)
    p = _write(tmp_path, m, tensors=qwen3_tensors(m, False, attn_type=attn_type))
    rb = {12: 144, 14: 210}[tid]
    with GgufFile(p) as g:
        for name, rows in (("blk.0.attn_q.weight", 4 * 128), ("blk.0.attn_v.weight", 2 * 128)):
            assert g.tensor_info(name)[0] == tid and g.tensor(name).shape == (rows, 512 // 256 * rb)
        blocks = g.tensor("blk.0.attn_q.weight")
    w = m.layers[0]["wqkv"][:4 * 128]
    dq = orc.dequant(tid, blocks, 512).reshape(w.shape)
    assert np.abs(dq - w).max() <= rel_bound * np.abs(w).max()
    assert np.corrcoef(dq.ravel(), w.ravel())[0, 1] >= 0.995
    model = TinyQwen3.from_gguf(p, dequant=orc.dequant)
    assert np.array_equal(model.layers[0]["wqkv"][:4 * 128], dq)


def _fuzz_seeds(tmp_path):
    """Small files of each shape the reader meets: F16 matrices with tokenizer arrays in the
    metadata (string, float and integer arrays), F32 with Q8_0 attention projections, and a
    version-2 file aligned to 64 bytes."""
    m = TinyQwen3(seed=11, n_layer=2, n_embd=32, n_head=2, n_head_kv=1, n_ff=32, n_vocab=8)
    toks = [("tokenizer.ggml.model", T_STRING, "gpt2"),
            ("tokenizer.ggml.tokens", T_ARRAY, (T_STRING, [f"t{i}" for i in range(8)])),
            ("tokenizer.ggml.scores", T_ARRAY, (T_F32, [float(-i) for i in range(8)])),
            ("tokenizer.ggml.token_type", T_ARRAY, (T_I32, [1] * 8))]
    seeds = [tmp_path / "f16.gguf", tmp_path / "q8.gguf", tmp_path / "v2.gguf"]
    write_gguf(seeds[0], qwen3_metadata(m) + toks, qwen3_tensors(m, True))
    write_gguf(seeds[1], qwen3_metadata(m), qwen3_tensors(m, False, attn_type="q8_0"))
    write_gguf(seeds[2], qwen3_metadata(m, alignment=64), qwen3_tensors(m, True), alignment=64, version=2)
    return seeds


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ builds the sanitizer-instrumented harness")
def test_mutated_files_under_sanitizers(tmp_path):
    """The reader and the Qwen3 checks built with AddressSanitizer and UndefinedBehaviorSanitizer
    (tests/cpp/gguf_fuzz.cpp) open 24 000 mutated copies of three small files (fixed seeds; three
    mutations in four hit the header, metadata and tensor table): every file is either rejected
    with the reader's error or read whole, every tensor view of an accepted file is read, and no
    sanitizer report, crash, leak or other exception occurs."""
    from exactinfer_amd.gguf import GgufFile
    here = Path(__file__).resolve().parent
    exe = tmp_path / "gguf_fuzz"
    build = subprocess.run(["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined",
                            "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", str(here / "cpp" / "gguf_fuzz.cpp"),
                            str(here.parent / "exactinfer_amd" / "host" / "gguf_index.cpp"),
                            str(here.parent / "exactinfer_amd" / "host" / "qwen3_schema.cpp"), "-o", str(exe)],
                           capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    for i, seed in enumerate(_fuzz_seeds(tmp_path)):
        with GgufFile(seed) as g:  # the seed itself is a valid file
            g.qwen3_config()
        header = _parse_independently(seed)[2]
        r = subprocess.run([str(exe), str(seed), "8000", str(1000 + i), str(tmp_path / "scratch.gguf"), str(header)],
                           capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, f"{seed.name}: {r.stderr[-3000:]}"
        ok, accepted, rejected = r.stdout.split()[-3:]
        assert ok == "ok" and int(accepted) > 0 and int(rejected) > 0, r.stdout[-200:]


def test_metadata_value_types(tmp_path, model):
    """Every GGUF scalar type reads back through the typed accessors: integers (signed ones
    sign-extended, bools as 0/1) through get_int and get_float, reals through get_float only;
    arrays of every element type are accepted and skipped."""
    from exactinfer_amd.gguf import GgufError, GgufFile
    extra = [("t.u8", 0, 250), ("t.i8", 1, -7), ("t.u16", 2, 65000), ("t.i16", 3, -30000), ("t.u32", T_U32, 4000000000),
             ("t.i32", T_I32, -2000000000), ("t.bool", 7, 1), ("t.u64", 10, (1 << 63) - 1), ("t.i64", 11, -(1 << 62)),
             ("t.f32", T_F32, 0.25), ("t.f64", 12, -1.5e300), ("t.str", T_STRING, "x" * 300)]
    arrays = [(f"a.{t}", T_ARRAY, (t, vals)) for t, vals in
              ((0, [1, 2]), (1, [-1]), (2, [3]), (3, [-4]), (T_U32, [5]), (T_I32, [-6]), (T_F32, [0.5]), (7, [0, 1]),
               (T_STRING, ["a", "bc", ""]), (10, [7]), (11, [-8]), (12, [1e-300]))]
    p = _write(tmp_path, model, meta=qwen3_metadata(model) + extra + arrays + [("a.empty", T_ARRAY, (T_U32, []))])
    with GgufFile(p) as g:
        for key, t, v in extra:
            if t in (T_F32, 12):
                assert g.get_float(key) == v
                with pytest.raises(GgufError, match="not an integer"):
                    g.get_int(key)
            elif t == T_STRING:
                assert g.get_str(key) == v
            else:
                assert g.get_int(key) == v and g.get_float(key) == float(v), key
        with pytest.raises(GgufError, match="not an integer"):
            g.get_int("a.0")  # an array is not a scalar
        assert g.qwen3_config()["n_layer"] == model.n_layer


@pytest.mark.parametrize("entry,match", [
    (("t.bool", 7, 2), "bool value 2"),
    (("t.u64", 10, 1 << 63), "does not fit an int64"),
    (("a.bool", T_ARRAY, (7, [0, 1, 3])), "bool value 3"),
    (("a.u64", T_ARRAY, (10, [1, (1 << 64) - 1])), "does not fit an int64"),
    (("a.nested", T_ARRAY, (T_ARRAY, [])), "not supported"),
    (("a.weird", T_ARRAY, (13, [])), "not supported"),
])
def test_metadata_value_errors(tmp_path, model, entry, match):
    """Values no int64 holds, bools other than 0/1 (scalars and array elements) and arrays of arrays
    or of unknown types are rejected when the file is opened."""
    _expect_rejected(_write(tmp_path, model, meta=qwen3_metadata(model) + [entry]), match)


def test_metadata_type_and_count_errors(tmp_path, model):
    raw = _write(tmp_path, model, meta=qwen3_metadata(model) + [("z.last", T_U32, 1)]).read_bytes()
    from tests.golden.write_tiny_gguf import _s
    i = raw.index(_s("z.last")) + len(_s("z.last"))
    _expect_rejected(_patched(tmp_path, raw, i, "<I", 13, "ty13.gguf"), "unknown metadata type 13")
    raw2 = _write(tmp_path, model, name="arr.gguf",
                  meta=qwen3_metadata(model) + [("z.arr", T_ARRAY, (T_U32, [1, 2]))]).read_bytes()
    j = raw2.index(_s("z.arr")) + len(_s("z.arr")) + 8  # value type, element type, then the count
    _expect_rejected(_patched(tmp_path, raw2, j, "<Q", 1 << 27, "cnt.gguf"), "too long")
    _expect_rejected(_patched(tmp_path, raw2, j, "<Q", 1 << 20, "cnt2.gguf"), "ends early|past the end|not plausible")
