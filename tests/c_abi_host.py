"""Child program of test_gpu_c_host.py: drives the C ABI from a process without
PyTorch, as a C, cgo or JNI caller would, with the system HIP runtime
(libamdhip64.so.7) the library links and plain ctypes; not collected by pytest.

argv: library path.  Checks a 4-bit and an 8-bit projection on the decode kernels
and on the GEMM against the exact float64 product (max |err| <= 1e-4 * RMS: fp32 accumulation
of exact products) and that the process maps one HIP runtime.  Exit status 0 = pass.
"""
import ctypes
import sys

import numpy as np


class Desc(ctypes.Structure):
    _fields_ = [("out_features", ctypes.c_uint32), ("in_features", ctypes.c_uint32),
                ("bits", ctypes.c_uint32), ("group_size", ctypes.c_uint32)]


def to_bf16(a):
    return (a.astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)  # truncation: exact bf16 values


def from_bf16(u):
    return (u.astype(np.uint32) << 16).view(np.float32)


def check(hip, lib, bits, seed):
    vp, sz = ctypes.c_void_p, ctypes.c_size_t
    rng = np.random.default_rng(seed)
    n, k, m = 320, 1024, 40
    per = 32 // bits
    q = rng.integers(0, 1 << bits, (n, k)).astype(np.uint32)
    w = np.zeros((n, k // per), np.uint32)
    for j in range(per):  # MLX packing: element per*c+j in bits [bits*j, bits*j+bits) of word c
        w |= q[:, j::per] << (bits * j)
    s = to_bf16(rng.uniform(0.001, 0.01, (n, k // 64)))
    b = to_bf16(rng.uniform(-0.05, 0.05, (n, k // 64)))
    x = to_bf16(rng.standard_normal((m, k)))
    wf = from_bf16(s).repeat(64, 1).astype(np.float64) * q + from_bf16(b).repeat(64, 1)
    exact = from_bf16(x).astype(np.float64) @ wf.T
    rms = np.sqrt((exact ** 2).mean())

    h = vp()
    st = lib.gemma4_qlinear_create(ctypes.byref(Desc(n, k, bits, 64)), w.ctypes.data_as(vp),
                                   s.ctypes.data_as(vp), b.ctypes.data_as(vp), ctypes.byref(h))
    msg = ctypes.create_string_buffer(512)
    lib.gemma4_qmm_get_last_error(msg, sz(512))
    assert st == 0, f"create: status {st}: {msg.value.decode()}"
    dx, dy = vp(), vp()
    assert hip.hipMalloc(ctypes.byref(dx), sz(x.nbytes)) == 0
    assert hip.hipMalloc(ctypes.byref(dy), sz(m * n * 4)) == 0
    assert hip.hipMemcpy(dx, x.ctypes.data_as(vp), sz(x.nbytes), 1) == 0  # host to device
    for gemm_from in (0, 32):  # automatic (the decode kernels at 40 rows here), then the GEMM
        lib.gemma4_qmm_set_gemm_min_rows(ctypes.c_uint32(gemm_from))
        st = lib.gemma4_qlinear_forward(h, None, dx, ctypes.c_uint32(m), dy, 1)  # fp32 output
        assert st == 0, f"forward: status {st}"
        assert hip.hipDeviceSynchronize() == 0
        y = np.empty((m, n), np.float32)
        assert hip.hipMemcpy(y.ctypes.data_as(vp), dy, sz(y.nbytes), 2) == 0  # device to host
        err = float(np.abs(y - exact).max() / rms)
        print(f"bits={bits} gemm_min_rows={gemm_from}: max |err| / RMS = {err:.2e}", flush=True)
        assert err <= 1e-4, err
    lib.gemma4_qmm_set_gemm_min_rows(ctypes.c_uint32(0))
    assert lib.gemma4_qlinear_free(h) == 0
    assert hip.hipFree(dx) == 0 and hip.hipFree(dy) == 0


def main(path):
    hip = ctypes.CDLL("libamdhip64.so.7")
    lib = ctypes.CDLL(path)
    count = ctypes.c_int(0)
    assert hip.hipGetDeviceCount(ctypes.byref(count)) == 0 and count.value > 0, "no HIP device"
    check(hip, lib, 4, 5)
    check(hip, lib, 8, 6)
    runtimes = {line.split()[-1] for line in open("/proc/self/maps") if "libamdhip64" in line}
    assert len(runtimes) == 1, runtimes
    print("ok", flush=True)


if __name__ == "__main__":
    main(sys.argv[1])
