"""Builds libgemma4_qmm.so (the gfx950 HIP kernels + the C ABI) in-tree.

    python -m helios_amd.build          # or __graft_entry__.build()

Output: helios_amd/lib/libgemma4_qmm.so.  Every HIP source is compiled for
gfx950 only, with packed-fp32 VALU ops disabled.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB_DIR = os.path.join(PKG, "lib")
LIB_NAME = "libgemma4_qmm.so"
LIB_PATH = os.path.join(LIB_DIR, LIB_NAME)

SOURCES = ["qmm_runtime.cpp", "q4_layout.hip", "q4_decode.hip", "q4_limbs.hip", "q4_gemm.hip", "q4_lora.hip"]
ARCH = "gfx950"
# measurement aid for the benchmark (a read-only HBM streaming kernel), its own library
PROBE_SOURCES = ["hbm_probe.hip"]
PROBE_PATH = os.path.join(LIB_DIR, "libhbm_probe.so")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build libgemma4_qmm")


# device code flags shared by the library build and the assembly checks
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in arch VGPRs: the GEMM's fp32 accumulators are updated by
    # VALU FMAs every group, which cannot read AGPRs
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def device_asm(source: str) -> str:
    """gfx950 assembly of one source file, compiled with the library's flags."""
    import tempfile

    with tempfile.TemporaryDirectory() as d:
        out = os.path.join(d, "out.s")
        cmd = [hipcc()] + DEVICE_FLAGS + ["--offload-device-only", "-S", "-I", os.path.join(ROOT, "include"),
                                          "-o", out, os.path.join(CSRC, source)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc -S failed ({res.returncode}):\n{res.stderr}")
        with open(out) as f:
            return f.read()


def _link(sources, path: str, verbose: bool) -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    tmp = path + ".tmp"
    cmd = [hipcc()] + DEVICE_FLAGS + [
        "-fPIC",
        "-shared",
        "-Wall",
        "-I", os.path.join(ROOT, "include"),
        "-o", tmp,
    ] + [os.path.join(CSRC, s) for s in sources]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    errs = "\n".join(l for l in res.stderr.splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{errs}")
    if errs.strip() and verbose:
        print(errs, file=sys.stderr)
    os.replace(tmp, path)
    return path


def build(verbose: bool = False) -> str:
    """Builds libgemma4_qmm.so and the benchmark's libhbm_probe.so; returns the former."""
    _link(PROBE_SOURCES, PROBE_PATH, verbose)
    return _link(SOURCES, LIB_PATH, verbose)


if __name__ == "__main__":
    print(build(verbose=True))
