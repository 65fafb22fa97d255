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


# Evidence of every attention gate evaluated in this session: (case, branch, rel err vs the
# reference, rel err vs float64 or None, reference vs float64 or None, plain max |got-ref|/|ref|).
# tests/conftest.py prints it in the terminal summary, so the GPU test log keeps which branch
# each case passed by and how close it came.
EVIDENCE = []


def plain_rel_err(got, ref) -> float:
    """max |got - ref| / |ref| over the elements with ref != 0 (no near-zero rule)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    nz = ref != 0
    return float(np.max(np.abs(got[nz] - ref[nz]) / np.abs(ref[nz]))) if np.any(nz) else 0.0


def gate(case, got, ref, exact_fn=None):
    """attn_parity with evidence: exact_fn() supplies the float64 result, computed only when the
    primary branch fails.  Returns (ok, description) and records the outcome in EVIDENCE."""
    e_ref = rel_err(got, ref)
    exact = exact_fn() if (e_ref > ATTN_RTOL and exact_fn is not None) else None
    ok, msg = attn_parity(got, ref, exact)
    e_gx = rel_err(got, exact) if exact is not None else None
    e_rx = rel_err(ref, exact) if exact is not None else None
    branch = "reference" if e_ref <= ATTN_RTOL else ("float64 fallback" if ok else "FAILED")
    EVIDENCE.append((case, branch, e_ref, e_gx, e_rx, plain_rel_err(got, ref)))
    return ok, f"{case}: {msg}"


def attn_parity(got, ref, exact=None):
    """The attention gate.  Primary: rel_err(got, ref) <= ATTN_RTOL against the reference
    CPU attention (src/model.cpp:191-214 restated).  Fallback, only where the reference's
    own fp32 rounding exceeds the bar (long contexts: its sequential fp32 sums over tens
    of thousands of keys drift by ~sqrt(T) ulps, measured 1.85e-5 at T = 32768 against
    float64): the result must be within ATTN_RTOL of the float64 brute force AND no farther
    from it than the reference itself.  Returns (ok, description)."""
    e_ref = rel_err(got, ref)
    if e_ref <= ATTN_RTOL:
        return True, f"rel err vs reference {e_ref:.3e}"
    if exact is None:
        return False, f"rel err vs reference {e_ref:.3e} (no float64 check supplied)"
    e_gx, e_rx = rel_err(got, exact), rel_err(ref, exact)
    ok = e_gx <= ATTN_RTOL and e_gx <= e_rx
    return ok, f"rel err vs reference {e_ref:.3e}; vs float64 {e_gx:.3e} (reference vs float64 {e_rx:.3e})"
