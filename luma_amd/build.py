"""Build the native parts in-tree: libluma_hip.so (hipcc, gfx950) and the
host bookkeeping module _luma_host (g++ against torch's C++ API).

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
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SOURCES = [os.path.join(HERE, "csrc", "luma_step.hip")]

OUT = os.path.join(HERE, "libluma_hip.so")
HOST_SOURCE = os.path.join(HERE, "csrc", "luma_host.cpp")
HOST_OUT = os.path.join(HERE, "_luma_host" + sysconfig.get_config_var("EXT_SUFFIX"))
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


def _run(cmd, what: str, out: str, verbose: bool):
    tmp = out + ".tmp"
    res = subprocess.run([*cmd, "-o", tmp], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{what} failed:\n" + " ".join(cmd) + "\n" + res.stdout + res.stderr)
    if verbose and res.stderr:
        sys.stderr.write(res.stderr)
    os.replace(tmp, out)
    return out


def host_command():
    """g++ line of the host module: torch's headers and libraries, the
    interpreter's headers, torch's C++ ABI setting."""
    import torch

    tdir = os.path.dirname(torch.__file__)
    inc = os.path.join(tdir, "include")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return [shutil.which("g++") or "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
            f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_EXTENSION_NAME=_luma_host",
            f'-DLUMA_TORCH_VERSION="{torch.__version__}"',
            "-I", inc, "-I", os.path.join(inc, "torch", "csrc", "api", "include"),
            "-I", sysconfig.get_paths()["include"], HOST_SOURCE,
            "-L", os.path.join(tdir, "lib"), "-Wl,-rpath," + os.path.join(tdir, "lib"),
            "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python"]


def build(verbose: bool = False) -> str:
    """Compile every HIP source into luma_amd/libluma_hip.so and the host
    module into luma_amd/_luma_host*.so; returns the library's path."""
    _run([hipcc(), *FLAGS, *SOURCES], "hipcc", OUT, verbose)
    _run(host_command(), "g++ (host module)", HOST_OUT, verbose)
    return OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
