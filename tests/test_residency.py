"""The resident-weight policy on the CPU: residency.h against a fake device
allocator (tests/residency_test.cpp), and the error-returning drop-in forms
with no device."""
import json
import os
import pathlib
import shutil
import subprocess
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent


def test_residency_policy(tmp_path):
    cxx = shutil.which("g++")
    if not cxx:
        pytest.skip("g++ unavailable")
    exe = tmp_path / "residency_test"
    subprocess.run([cxx, "-std=c++17", "-O1", "-Wall", "-Werror", str(ROOT / "tests" / "residency_test.cpp"),
                    "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0 and r.stdout.strip() == "ok", r.stdout + r.stderr


TRY = r"""
import json, sys, numpy as np
sys.path.insert(0, {root!r})
from demonic_amd import _lib
lib = _lib.load()
k, n = 64, 16
x = np.ones(k, np.float32)
w = np.zeros(k * n, np.uint16)
out = np.full(2 * n, 7.0, np.float32)
codes = [lib.dmc_matmul_bf16_gpu_try(x.ctypes.data, w.ctypes.data, out.ctypes.data, 1, k, n),
         lib.dmc_matmul_bf16_gpu_t_try(x.ctypes.data, w.ctypes.data, out.ctypes.data, 1, k, n),
         lib.dmc_matmul_bf16_gpu_batched_try(x.ctypes.data, w.ctypes.data, out.ctypes.data, 1, k, n, 2, 0, 0),
         lib.dmc_matmul_bf16_gpu_batched_deferred_try(x.ctypes.data, w.ctypes.data, out.ctypes.data, 1, k, n, 2, 0, 0),
         lib.dmc_matmul_bf16_gpu_flush_try()]
print(json.dumps([codes, bool(np.all(out == 7.0)), lib.dmc_hip_last_error().decode()]))
"""


def test_try_forms_report_no_device_and_leave_out_untouched():
    """DMC_HIP_DISABLE=1 (or no GPU): each try form returns DMC_HIP_ENODEV
    (-1) and writes nothing, so a caller falls back to its own CPU kernel; the
    flush form has nothing pending and succeeds.  The void forms abort
    instead (tests/test_abi.py)."""
    env = dict(os.environ, DMC_HIP_DISABLE="1")
    r = subprocess.run([sys.executable, "-c", TRY.format(root=str(ROOT))], capture_output=True, text=True,
                       env=env, timeout=120)
    assert r.returncode == 0, r.stderr
    codes, untouched, msg = json.loads(r.stdout)
    assert codes == [-1, -1, -1, -1, 0], r.stdout
    assert untouched, r.stdout
    assert "DMC_HIP_DISABLE" in msg, r.stdout


def test_try_forms_validate_arguments():
    """Argument errors come back as DMC_HIP_EINVAL (-2) before any device
    work; m == 0 or n == 0 is a successful no-op (gpu.rs:402)."""
    from demonic_amd import _lib
    lib = _lib.load()
    x = np.ones(8, np.float32)
    w = np.zeros(64, np.uint16)
    out = np.full(8, 3.0, np.float32)
    assert lib.dmc_matmul_bf16_gpu_try(x.ctypes.data, w.ctypes.data, out.ctypes.data, -1, 8, 8) == -2
    assert lib.dmc_matmul_bf16_gpu_batched_try(x.ctypes.data, w.ctypes.data, out.ctypes.data, 1, 8, 8, 2, -1, 0) == -2
    assert lib.dmc_matmul_bf16_gpu_t_try(0, 0, out.ctypes.data, 1, 8, 8) == -2  # null l and r with k > 0
    assert lib.dmc_matmul_bf16_gpu_try(x.ctypes.data, w.ctypes.data, out.ctypes.data, 0, 8, 8) == 0
    assert np.all(out == 3.0)
