import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libei_attn.so")
    from exactinfer_amd import build as B
    B.ensure_built()  # builds only when nothing is built


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as O
    O.build()
    return O


@pytest.fixture(scope="session")
def gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from exactinfer_amd import attention as A
    return A


def pytest_terminal_summary(terminalreporter):
    """Which branch of the attention gate each recorded case passed by (tests/parity.py), and per
    group of cases (a test's cases without their sequence / row / call index) the largest error
    against the reference and under the plain |got - ref| / |ref| rule (no near-zero rule)."""
    import re
    from tests.parity import ATTN_RTOL, EVIDENCE
    if not EVIDENCE:
        return
    tr = terminalreporter
    tr.section(f"attention parity evidence (bar {ATTN_RTOL:g})")
    worst = max(e[2] for e in EVIDENCE)
    fb = [e for e in EVIDENCE if e[1] != "reference"]
    tr.write_line(f"{len(EVIDENCE)} cases; worst rel err vs reference {worst:.3e}; "
                  f"{len(fb)} passed by the float64 fallback or failed")
    groups = {}
    for case, branch, e_ref, e_gx, e_rx, plain in EVIDENCE:
        g = re.sub(r" (seq|row|call) .*$", "", case)
        n, r, p, f = groups.get(g, (0, 0.0, 0.0, 0))
        groups[g] = (n + 1, max(r, e_ref), max(p, plain), f + (branch != "reference"))
    for g, (n, r, p, f) in groups.items():
        tr.write_line(f"  group {g}: {n} cases, max vs reference {r:.3e}, max plain |d|/|ref| {p:.3e}"
                      + (f", {f} by the float64 fallback" if f else ""))
    _write_evidence_json(EVIDENCE, ATTN_RTOL)
    for case, branch, e_ref, e_gx, e_rx, plain in EVIDENCE:
        if branch != "reference":
            extra = "" if e_gx is None else f"; vs float64 {e_gx:.3e} (reference vs float64 {e_rx:.3e})"
            tr.write_line(f"  {branch:16s} {case}: vs reference {e_ref:.3e}{extra}; plain |d|/|ref| {plain:.3e}")


def _write_evidence_json(evidence, bar):
    """The session's parity evidence as JSON, per group of cases: count, worst error against the
    reference, worst against float64 and the reference's own distance from float64 (where the
    float64 check ran), cases passed by the float64 fallback, and the plain |d|/|ref| worst.
    Written to gpurun_out/parity_evidence.json (or $EI_PARITY_JSON)."""
    import json
    import os
    import re
    groups = {}
    for case, branch, e_ref, e_gx, e_rx, plain in evidence:
        g = groups.setdefault(re.sub(r" (seq|row|call) .*$", "", case),
                              {"cases": 0, "max_vs_reference": 0.0, "max_vs_float64": None,
                               "reference_vs_float64": None, "float64_fallback": 0, "failed": 0, "max_plain": 0.0})
        g["cases"] += 1
        g["max_vs_reference"] = max(g["max_vs_reference"], e_ref)
        g["max_plain"] = max(g["max_plain"], plain)
        if e_gx is not None:
            g["max_vs_float64"] = max(g["max_vs_float64"] or 0.0, e_gx)
            g["reference_vs_float64"] = max(g["reference_vs_float64"] or 0.0, e_rx)
        g["float64_fallback"] += branch == "float64 fallback"
        g["failed"] += branch == "FAILED"
    out = {"bar": bar, "cases": len(evidence),
           "worst_vs_reference": max(e[2] for e in evidence),
           "worst_vs_float64": max((e[3] for e in evidence if e[3] is not None), default=None),
           "float64_fallback": sum(e[1] == "float64 fallback" for e in evidence),
           "failed": sum(e[1] == "FAILED" for e in evidence), "groups": groups}
    path = os.environ.get("EI_PARITY_JSON") or str(ROOT / "gpurun_out" / "parity_evidence.json")
    try:
        os.makedirs(os.path.dirname(path), exist_ok=True)
        with open(path, "w") as f:
            json.dump(out, f, indent=1, sort_keys=True)
    except OSError:
        pass
