"""Parity metrics shared by the tests.

Relative error per output element, with the near-zero rule: an attention output is a
convex combination of V rows, so single elements can be arbitrarily close to 0 while the
row is O(1).  The denominator is max(|ref_i|, rms(ref row)) (tau = 1 times the row rms,
row = the 128 elements of one head's output); elements larger than the row rms are
judged purely relatively, smaller ones against the row scale.
"""
import numpy as np

ATTN_RTOL = 1e-5  # max relative error per output element vs the reference CPU attention


def rel_err(got, ref) -> float:
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    rms = np.sqrt(np.mean(ref * ref, axis=-1, keepdims=True))
    den = np.maximum(np.abs(ref), rms)
    den = np.where(den == 0, 1.0, den)
    return float(np.max(np.abs(got - ref) / den)) if got.size else 0.0


def bits_equal(a, b) -> bool:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and bool(np.all(a.view(np.uint32) == b.view(np.uint32)))


def ulp_diff(a, b) -> int:
    a = np.ascontiguousarray(a, dtype=np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, dtype=np.float32).view(np.int32).astype(np.int64)
    return int(np.max(np.abs(a - b))) if a.size else 0
