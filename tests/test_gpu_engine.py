"""Engine-level parity: the C++ HipAttention (exactinfer_amd/host/) driven like the reference
engine drives attention — prompt chunks, then one-token decode steps, every layer — against
the CPU oracle processing the same tokens one at a time.  Runs the compiled driver
tests/cpp/engine_test as a subprocess, as the reference's own tests drive its binary."""
import json
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "cpp" / "engine_test"


def _run(*args):
    if not EXE.exists():
        pytest.fail(f"{EXE} not built (run __graft_entry__.build())")
    r = subprocess.run([str(EXE), *map(str, args)], capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr)
    res = json.loads(r.stdout.strip().splitlines()[-1])
    return r.returncode, res


def test_config0_prefill512_decode128():
    """configs[0] of the benchmark definition: 0.6B heads (16/8), one layer, 512-token prefill then 128 decode
    steps, each appending to the KV cache."""
    rc, res = _run(1, 16, 8, 512, 512, 128, 640)
    assert rc == 0 and res["ok"], res
    assert res["caches_bit_exact"] and res["out_of_range_thrown"]


def test_chunked_prompt_crosses_chunk_boundaries():
    """Prompt evaluated in 128-token chunks (pos0 > 0 for later chunks, the case the
    reference's attn_long test covers), 4B heads, two layers, then decode steps."""
    rc, res = _run(2, 32, 8, 300, 128, 12, 400)
    assert rc == 0 and res["ok"], res


def test_long_prompt_in_512_chunks_then_decode():
    """A 4000-token prompt in 512-token chunks (the reference engine's chunk cap,
    src/cuda/model_cuda.cu:1912): later chunks sit at positions up to 3584, where the engine's
    prefill splits each query block's key range over workgroups; then decode steps at ctx ~4000."""
    rc, res = _run(1, 32, 8, 4000, 512, 8, 4100)
    assert rc == 0 and res["ok"], res


def test_decode_steps_replay_one_captured_graph():
    """The reference replays its decode step as one CUDA graph (src/cuda/model_cuda.cu:1848-1859);
    here every decode step after the first replays one captured hipGraph of all layers'
    HipAttention::layer calls, with only the device-resident position changing (two layers, 4B
    heads, 200-token prompt, 40 steps)."""
    rc, res = _run(2, 32, 8, 200, 128, 40, 300, "graph")
    assert rc == 0 and res["ok"] and res["graph"], res
    assert res["caches_bit_exact"]


def test_projection_then_attention_per_chunk():
    """The engine's QKV projection (HipAttention::project: attention RMSNorm + fused QKV GEMV on the
    GPU, in row groups) on seeded residual rows, prompt chunks of 100 rows then decode steps; each
    chunk's rows within 1e-5 of the CPU path's rmsnorm + matvec, then the attention checks on them."""
    rc, res = _run(2, 32, 8, 260, 100, 6, 300, "project")
    assert rc == 0 and res["ok"] and res["project"], res
    assert res["project_max_rel_err"] <= 1e-5 and res["caches_bit_exact"]
