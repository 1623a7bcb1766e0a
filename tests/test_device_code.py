"""Checks on the compiled gfx950 code (CPU only: hipcc cross-compiles).

The GEMM issues its LDS DMAs (`buffer_load_dwordx4 ... lds`) from inline asm, which
the compiler's hazard recognizer cannot see into.  A VALU write of an SGPR (for
example a `v_readlane` reloading a spilled resource or offset SGPR) needs 5 wait
states before a vector memory instruction reads that SGPR; the asm supplies them
itself.  Missing wait states made loads use stale offsets (wrong results at
k/q_proj M=512 in an earlier build), so every such pair is checked here, along with
the properties the kernel's manual ordering relies on.
"""

import re

import pytest

from helios_amd import build as hbuild

WAIT_STATES = 5


def _kernels(asm: str):
    for m in re.finditer(r"\n(_ZN\S*gemm_kernel\S*):[^\n]*\n", asm):
        body = asm[m.end():asm.index("s_endpgm", m.end())]
        lines = [l.strip() for l in body.splitlines()
                 if l.strip() and not l.strip().startswith((";", "."))]
        yield m.group(1), lines


def _sgprs(tok: str):
    m = re.match(r"s\[(\d+):(\d+)\]$", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"s(\d+)$", tok)
    if m:
        return {int(m.group(1))}
    return {"m0"} if tok == "m0" else set()


@pytest.fixture(scope="module")
def gemm_asm():
    return hbuild.device_asm("q4_gemm.hip")


def test_lds_dma_sgpr_hazards_covered(gemm_asm):
    kernels = list(_kernels(gemm_asm))
    # bf16 / fp32 outputs, bf16 / fp32 GeGLU pairs, bf16 / fp32 outputs with a LoRA
    # delta; 256, 128 and 64 x 256 tiles, the 256-row tile's fp16 form and the 128-
    # and 256-row tiles' one-pass 8-bit form
    assert len(kernels) == 36
    assert sum("ELi256ELi256ELi1E" in name for name, _ in kernels) == 6
    assert sum("ELi256ELi2E" in name for name, _ in kernels) == 12
    for name, lines in kernels:
        dmas = 0
        for i, line in enumerate(lines):
            if not (line.startswith("buffer_load_dwordx4") and " lds" in line):
                continue
            dmas += 1
            used = set().union(*[_sgprs(t.strip(",")) for t in line.split()[1:]]) | {"m0"}
            waits, j = 0, i - 1
            while j >= 0 and waits < WAIT_STATES:
                op = lines[j].split()[0]
                if op == "s_nop":
                    waits += int(lines[j].split()[1]) + 1
                else:
                    if op.startswith("v_"):
                        dst = lines[j].split()[1].rstrip(",")
                        assert not (_sgprs(dst) & used), f"{name}: {lines[j]!r} feeds {line!r} within {waits} wait states"
                    waits += 1
                j -= 1
        assert dmas > 0, name


def test_no_spills_and_lds_budget(gemm_asm):
    # scratch spills would be VMEM loads counted by the kernel's manual vmcnt waits
    for field in ("vgpr_spill_count", "private_segment_fixed_size"):
        vals = [int(v) for v in re.findall(rf"\.{field}:\s+(\d+)", gemm_asm)]
        assert vals and max(vals) == 0, (field, vals)
    lds = [int(v) for v in re.findall(r"\.group_segment_fixed_size:\s+(\d+)", gemm_asm)]
    assert max(lds) <= 160 * 1024
    # the 64 x 256 tile fits two workgroups per CU (LDS and 4 waves per SIMD)
    small = 0
    for m in re.finditer(r"\.group_segment_fixed_size:\s+(\d+).*?\.name:\s+(\S+).*?\.vgpr_count:\s+(\d+)",
                         gemm_asm, re.S):
        if "gemm_kernelILi" in m.group(2) and "ELi64ELi256E" in m.group(2):
            small += 1
            assert int(m.group(1)) <= 80 * 1024 and int(m.group(3)) <= 128, m.group(2)
    assert small == 6


def _kernel_meta(asm: str):
    """(name, vgpr_count, spill bytes) of every kernel in the metadata block."""
    for m in re.finditer(r"- \.agpr_count:.*?\.name:\s+(\S+).*?\.private_segment_fixed_size:\s+(\d+).*?"
                         r"\.vgpr_count:\s+(\d+)", asm, re.S):
        yield m.group(1), int(m.group(3)), int(m.group(2))


def test_decode_register_budgets():
    asm = hbuild.device_asm("q4_decode.hip")
    meta = list(_kernel_meta(asm))
    assert any("decode_stream_kernel" in n for n, _, _ in meta)
    for name, vgprs, private in meta:
        assert private == 0, f"{name} spills to scratch"
        stream = re.search(r"decode_stream_kernelILi\d+ELi\d+ELi(\d+)E", name)
        if stream:
            # two buffers: two 8-wave workgroups per CU (the launcher's occupancy
            # assumption); four buffers are launched only at one workgroup per CU
            limit = 128 if stream.group(1) == "2" else 256
            assert vgprs <= limit, f"{name}: {vgprs} VGPRs"
        if "decode_rows_kernel" in name:
            # two waves per SIMD (two 4-wave workgroups per CU)
            assert vgprs <= 256, f"{name}: {vgprs} VGPRs"


def test_limb_register_budgets():
    """decode_limb_kernel's launch shapes (q4_limbs.hip limb_config) assume its
    occupancy: three 8-wave workgroups per CU for one chunk in flight (6 waves per
    SIMD: at most 85 VGPRs), one 16-wave workgroup per CU (4 per SIMD: 128)."""
    asm = hbuild.device_asm("q4_limbs.hip")
    meta = [(n, v, p) for n, v, p in _kernel_meta(asm) if "decode_limb_kernel" in n]
    assert len(meta) == 3
    for name, vgprs, private in meta:
        assert private == 0, f"{name} spills to scratch"
        nbuf, waves = map(int, re.search(r"decode_limb_kernelILi(\d+)ELi(\d+)E", name).groups())
        limit = 85 if nbuf == 1 else (128 if waves == 16 else 256)
        assert vgprs <= limit, f"{name}: {vgprs} VGPRs"


def test_limb_rows_register_budgets():
    """decode_limb_rows_kernel: no scratch; the 16-wave instance dealt round the grid at
    4 rows runs two workgroups per CU (8 waves per SIMD: at most 64 VGPRs); the rest
    run one 16-wave workgroup per CU (at most 128; the two phased ones, BATCH > 0,
    among them) or 8-wave ones."""
    asm = hbuild.device_asm("q4_limbs.hip")
    meta = [(n, v, p) for n, v, p in _kernel_meta(asm) if "decode_limb_rows_kernel" in n]
    assert len(meta) == 11
    assert sum(bool(re.search(r"ELb1ELi[1-9]\d*E", n)) for n, _, _ in meta) == 2
    for name, vgprs, private in meta:
        assert private == 0, f"{name} spills to scratch"
        mt, nbuf, waves = map(int, re.search(r"decode_limb_rows_kernelILi(\d+)ELi(\d+)ELi(\d+)E", name).groups())
        limit = 64 if (mt == 4 and nbuf == 1 and waves == 16) else 128 if waves == 16 else 256
        assert vgprs <= limit, f"{name}: {vgprs} VGPRs"

