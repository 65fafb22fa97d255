"""Builds tests/cpp/engine_test (test driver: HipAttention checked against the CPU oracle).
Needs exactinfer_amd/libei_attn.so and oracle/liboracle.so built first."""
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent


def build() -> Path:
    from exactinfer_amd.build import hipcc
    out = HERE / "engine_test"
    cmd = [hipcc(), "--offload-arch=gfx950", "-O2", "-std=c++17", str(HERE / "engine_test.cpp"),
           "-L", str(ROOT / "exactinfer_amd"), "-lei_attn", "-L", str(ROOT / "oracle"), "-loracle",
           "-Wl,-rpath,$ORIGIN/../../exactinfer_amd", "-Wl,-rpath,$ORIGIN/../../oracle", "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"engine_test build failed:\n{r.stderr}")
    return out


if __name__ == "__main__":
    print(build())
