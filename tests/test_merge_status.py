"""The decode workspace's status word turned into an error, on the CPU (no GPU call).

The in-kernel split merge (exactinfer_amd/csrc/decode.hip, merge path of k_decode) relies on the
splits of one (sequence, kv head) running on one XCD; a merger that finds them on different XCDs
sets bit 0 of the workspace's status word.  These tests stand a host-side word in for one read
back from a workspace and check that the C ABI (ei_decode_status_check) and the engine class
(HipAttention::raise_on_status, the check begin_chunk and check_status run) report it as an
error rather than returning silently."""
import json
import subprocess
from pathlib import Path

import pytest

EXE = Path(__file__).resolve().parent / "cpp" / "engine_test"


def test_status_check_through_the_c_abi():
    from exactinfer_amd import _capi
    L = _capi.lib()
    assert L.ei_decode_status_check(0) == 0
    assert L.ei_decode_status_check(1) == 4  # EI_ERR_MERGE
    assert "different XCDs" in _capi.last_error()
    assert L.ei_decode_status_check(2) == 4
    assert "unknown status bits" in _capi.last_error()


@pytest.mark.parametrize("word,thrown", [("0", False), ("1", True), ("0x3", True), ("0x80000000", True)])
def test_engine_raises_on_a_set_status_word(word, thrown):
    if not EXE.exists():
        pytest.fail(f"{EXE} not built (run __graft_entry__.build())")
    r = subprocess.run([str(EXE), "status", word], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["thrown"] == thrown, res
    if thrown:
        assert "status" in res["what"]
