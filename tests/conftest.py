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
    for case, branch, e_ref, e_gx, e_rx, plain in EVIDENCE:
        if branch != "reference":
            extra = "" if e_gx is None else f"; vs float64 {e_gx:.3e} (reference vs float64 {e_rx:.3e})"
            tr.write_line(f"  {branch:16s} {case}: vs reference {e_ref:.3e}{extra}; plain |d|/|ref| {plain:.3e}")
