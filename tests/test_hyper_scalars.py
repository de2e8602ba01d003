"""The step scalars the kernels derive on the device, checked on the CPU.

Each step's float32 scalars (bias corrections, -eta, decay) are computed by
luma_amd/csrc/luma_hyper.h from the param group's doubles and the device step
count.  This test compiles that header for the host with g++ (the same code
the HIP kernels run, same -ffp-contract=off) and compares every scalar bit for
bit with the reference's Python expressions (functional.py:209-213,
262-264, 278): bc1 = 1 - beta1**t, bc2 = 1 - beta2**t, eta = lr / bc1,
decay = 1 - weight_decay*lr, each rounded once to float32.
"""

import os
import shutil
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)

# (lr, beta1, beta2, eps, weight_decay, [(t0, n), ...])
CASES = [
    (1e-3, 0.9, 0.999, 1e-8, 0.01, [(1, 40000)]),
    (3e-4, 0.95, 0.9999, 1e-6, 0.1, [(1, 40000), (2**31 - 5, 10), (2**40, 3)]),
    (6e-4, 0.9, 0.95, 1e-8, 0.0, [(1, 5000)]),
    (1e-2, 0.8, 0.99999, 1e-10, 0.05, [(1, 40000), (123456789, 50)]),
    (2.5e-5, 0.0, 0.5, 1e-8, 1.0, [(1, 200)]),
    (0.0, 0.5, 0.0, 1e-3, 0.0, [(1, 100)]),
]


@pytest.fixture(scope="module")
def hyper_bin(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    out = str(tmp_path_factory.mktemp("hyper") / "hyper_rows_host")
    cmd = [gxx, "-O2", "-std=c++17", "-ffp-contract=off",
           "-I", os.path.join(ROOT, "luma_amd", "csrc"), "-I", os.path.join(ROOT, "include"),
           "-o", out, os.path.join(HERE, "native", "hyper_rows_host.cpp"), "-lm"]
    subprocess.run(cmd, check=True, capture_output=True)
    return out


def _python_rows(lr, b1, b2, eps, wd, t0, n):
    rows = []
    for t in range(t0, t0 + n):
        bc1 = 1.0 - b1 ** t
        bc2 = 1.0 - b2 ** t
        eta = lr / bc1
        rows.append((b1, 1.0 - b1, b2, 1.0 - b2, 1.0 - wd * lr, -eta, bc2, eps))
    return np.array(rows, dtype=np.float64).astype(np.float32).view(np.uint32)


def _host_rows(binary, lr, b1, b2, eps, wd, t0, n):
    line = " ".join(float(x).hex() for x in (lr, b1, b2, eps, wd)) + f" {t0} {n}\n"
    res = subprocess.run([binary], input=line, capture_output=True, text=True, check=True)
    return np.array([[int(x, 16) for x in ln.split()] for ln in res.stdout.splitlines()],
                    dtype=np.uint32)


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"b1={c[1]},b2={c[2]}")
def test_device_scalars_equal_python(hyper_bin, case):
    lr, b1, b2, eps, wd, spans = case
    for t0, n in spans:
        want = _python_rows(lr, b1, b2, eps, wd, t0, n)
        got = _host_rows(hyper_bin, lr, b1, b2, eps, wd, t0, n)
        assert got.shape == want.shape
        bad = np.nonzero((got != want).any(axis=1))[0]
        assert bad.size == 0, f"t = {t0 + bad[:5]}: {got[bad[:5]]} vs {want[bad[:5]]}"


def test_power_is_correctly_rounded(hyper_bin):
    """A wrong power (say beta**(t-1), or a dropped low word) must show: the
    rows of t and t+1 differ at small t, and t = 1 gives 1 - beta exactly."""
    got = _host_rows(hyper_bin, 1e-3, 0.9, 0.999, 1e-8, 0.01, 1, 3)
    want1 = np.float32([0.9, 0.1, 0.999, 1.0 - 0.999, 1.0 - 1e-5, -(1e-3 / (1.0 - 0.9)),
                        1.0 - 0.999, 1e-8]).view(np.uint32)
    assert (got[0] == want1).all()
    assert (got[1] != got[0]).any() and (got[2] != got[1]).any()
