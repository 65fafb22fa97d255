"""Writes the golden fixtures under tests/golden/ (run in a container where the reference
tree is present: it needs oracle/_ref/libelref.so, the reference's own QK-norm and RoPE
compiled from its sources by oracle/Makefile).

  ref_qknorm_rope.npz   inputs and outputs of the reference's el::rmsnorm (src/ops.cpp:155-160),
                        el::rope_inv_freq (src/model.cpp:105-109) and el::rope
                        (src/model.cpp:23-32) on seeded inputs: vectors produced by the
                        reference's code, checked against the oracle in tests/test_oracle.py.
  attn_small.npz        seeded small attention cases with the float64 brute-force output
                        (orc_attn_f64): a regression anchor for the oracle's attention.
  ref_matvec.npz        inputs and outputs of the reference's dot_f32 / dot_f16 (src/ops.cpp:92-118,
                        compiled from source) on seeded rows of lengths with and without tails, and
                        of its f16_to_f32 on every binary16 pattern (as a checksum of the bits).
  ref_dequant.npz       random Q8_0 / Q4_K / Q6_K rows (every byte random) and the reference's own
                        dequant_* output for them (src/quant.cpp:7-60, compiled from source).

    python tests/golden/make_golden.py
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from oracle import oracle as O  # noqa: E402


def main():
    O.build()
    R = O.ref_lib()
    if R is None:
        sys.exit("oracle/_ref/libelref.so missing: build it where the reference tree exists (make -C oracle)")
    D = 128
    n = 24
    scales = np.float32(10.0) ** np.arange(-3, 3, dtype=np.float32).repeat(4)
    x = np.stack([O.normal((D,), 5000 + i) * scales[i] for i in range(n)]).astype(np.float32)
    g = np.stack([O.gamma(D, 6000 + i) for i in range(n)]).astype(np.float32)
    eps = np.float32(1e-6)
    norm = np.empty_like(x)
    for i in range(n):
        R.elref_rmsnorm(norm[i], np.ascontiguousarray(x[i]), np.ascontiguousarray(g[i]), D, float(eps))
    rope_cases = [(128, 1e6), (64, 1e4)]
    pos = np.array([0, 1, 2, 17, 511, 4095, 32767, 131071], dtype=np.int32)
    out = {"x": x, "gamma": g, "eps": np.array([eps]), "rmsnorm": norm, "pos": pos}
    for rd, base in rope_cases:
        f = np.empty(rd // 2)
        R.elref_rope_inv_freq(f, rd, base)
        v = np.stack([O.normal((rd,), 7000 + int(p)) for p in pos]).astype(np.float32)
        r = v.copy()
        for i, p in enumerate(pos):
            R.elref_rope(r[i], int(p), rd, f)
        out[f"inv_freq_{rd}_{int(base)}"] = f
        out[f"rope_in_{rd}_{int(base)}"] = v
        out[f"rope_out_{rd}_{int(base)}"] = r
    np.savez_compressed(HERE / "ref_qknorm_rope.npz", **out)

    cases = {}
    for name, (H, HKV, T) in {"gqa4_t1": (8, 2, 1), "gqa2_t37": (8, 4, 37), "gqa4_t300": (16, 4, 300)}.items():
        k = O.normal((T, HKV, D), 100 + T)
        v = O.normal((T, HKV, D), 200 + T)
        q = O.normal((H, D), 300 + T)
        # inputs are regenerated from (shape, seeds) by the counter-based generator
        cases[f"{name}_f64"] = O.attn_f64(q, k, v, T, H, HKV, D)
        cases[f"{name}_shape"] = np.array([H, HKV, T], dtype=np.int32)
        cases[f"{name}_seeds"] = np.array([300 + T, 100 + T, 200 + T], dtype=np.int64)  # q, k, v
    np.savez_compressed(HERE / "attn_small.npz", **cases)

    mv = {}
    rng = np.random.default_rng(8000)
    for n in (7, 8, 16, 31, 32, 37, 128, 2560, 2571):
        x = O.normal((n,), 8100 + n)
        w32 = O.normal((n,), 8200 + n)
        # binary16 weights spanning normals, subnormals and both signs
        w16 = rng.integers(0, 0x7C00, n).astype(np.uint16) | (rng.integers(0, 2, n).astype(np.uint16) << 15)
        mv[f"x_{n}"] = x
        mv[f"w32_{n}"] = w32
        mv[f"w16_{n}"] = w16
        mv[f"dot32_{n}"] = np.array([R.elref_dot_f32(w32, x, n)], np.float32)
        mv[f"dot16_{n}"] = np.array([R.elref_dot_f16(w16, x, n)], np.float32)
    allh = np.arange(1 << 16, dtype=np.uint32)
    conv = np.array([R.elref_f16_to_f32(int(h)) for h in allh], np.float32)
    # NaN payloads compare by bits; the checksum covers every pattern's converted bits
    mv["f16_all_bits_sum"] = np.array([int(conv.view(np.uint32).astype(np.uint64).sum())], np.uint64)
    np.savez_compressed(HERE / "ref_matvec.npz", **mv)
    # dequant_q8_0 / _q4_K / _q6_K (src/quant.cpp:7-60) on random bytes: two rows of 512 values
    dq = {}
    for t, name in ((O.W_Q8_0, "q8_0"), (O.W_Q4_K, "q4_K"), (O.W_Q6_K, "q6_K")):
        blocks = np.random.default_rng(6100 + t).integers(0, 256, size=(2, O.row_bytes(t, 512)), dtype=np.uint8)
        out = np.empty(2 * 512, np.float32)
        getattr(R, "elref_dequant_" + name)(blocks.ctypes.data, out, out.size)
        dq[name + "_blocks"], dq[name + "_out"] = blocks, out
    np.savez_compressed(HERE / "ref_dequant.npz", **dq)
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
