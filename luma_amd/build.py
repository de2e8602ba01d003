"""Build libluma_hip.so in-tree with hipcc for gfx950.

    python -m luma_amd.build

Flags that matter for results, not just speed:
  -ffp-contract=off                      no fused multiply-add in the exact path
  -fhip-fp32-correctly-rounded-divide-sqrt   IEEE float32 division
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed-FP32 instructions
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCES = [os.path.join(HERE, "csrc", "luma_step.hip")]

OUT = os.path.join(HERE, "libluma_hip.so")
ARCH = os.environ.get("LUMA_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "-shared",
    f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", os.path.join(ROOT, "include"),
]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the LUMA HIP library needs ROCm")


def build(verbose: bool = False) -> str:
    """Compile every HIP source into luma_amd/libluma_hip.so; returns its path."""
    tmp = OUT + ".tmp"
    cmd = [hipcc(), *FLAGS, "-o", tmp, *SOURCES]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + res.stdout + res.stderr)
    if verbose and res.stderr:
        sys.stderr.write(res.stderr)
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
