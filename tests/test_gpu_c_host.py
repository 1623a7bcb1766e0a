"""The C ABI without PyTorch in the process, and the HIP runtime count with it.

The library links the system HIP runtime (libamdhip64.so.7); PyTorch-ROCm wheels carry
their own copy under the same soname.  A C/cgo/JNI host has only the system one; a
Python host must let torch's copy load first so that one runtime serves both
(helios_amd.qmm.load_library imports torch before the library)."""
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _run(code_or_args, timeout):
    return subprocess.run([sys.executable, *code_or_args], cwd=ROOT, capture_output=True, text=True,
                          timeout=timeout)


def test_load_library_maps_one_hip_runtime():
    """Loading the library first (torch not imported yet) still leaves one HIP runtime
    mapped once torch is in the process: load_library brings torch's copy in first."""
    from helios_amd import build

    if not os.path.exists(build.LIB_PATH):
        pytest.skip("library not built")
    code = ("from helios_amd import qmm; qmm.load_library(); import torch; "
            "print(len({l.split()[-1] for l in open('/proc/self/maps') if 'libamdhip64' in l}))")
    r = _run(["-c", code], 300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert r.stdout.strip().splitlines()[-1] == "1", r.stdout


@pytest.mark.gpu
def test_c_abi_without_torch(gpu_lib):
    """create -> forward (decode kernels, then the GEMM) -> free of a 4-bit and an 8-bit
    projection from a process with no torch, against the exact product."""
    from helios_amd import build

    r = _run([os.path.join(ROOT, "tests", "c_abi_host.py"), build.LIB_PATH], 110)
    print(r.stdout, flush=True)
    assert r.returncode == 0, (r.stdout + r.stderr)[-3000:]
    assert r.stdout.strip().endswith("ok")
