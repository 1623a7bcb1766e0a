"""GPU check of gemma4_qlinear_forward_noalloc (the allocation-free forward) through
the C ABI: on a sequence of calls in a row on one stream, each followed by a smaller
one that reuses the same static scratch, its output equals gemma4_qlinear_forward's
bit for bit where both run the same GEMM plan, and otherwise both meet the oracle's
bars (fp32 within 2e-3 * RMS, bf16 within 1e-2 * RMS + ulp/2) and agree to within
the fp32 accumulation error.  The GEMM's one scratch buffer, its split-K partial
sums, is planned to fit what the array has left, so a call of any size runs (18000
rows of an 8-bit K = 15360 projection here).  (This check has no counterpart in the
reference: its MLX ops allocate per call.)"""

import ctypes

import numpy as np
import pytest

from oracle import affine as A
from oracle import c_oracle as C
from test_gpu_parity import assert_close, dev_triple, dev_x, host_bits, random_triple

pytestmark = pytest.mark.gpu


def _both(lin, x, dtype):
    import torch

    ref = lin.forward(x, out_dtype=dtype)
    got = torch.full_like(ref, float("nan"))  # stale contents must not survive
    lin.forward_noalloc(x, got)
    torch.cuda.synchronize()
    return ref, got


def _compare(ref, got, x_bits, tri, rows, what, bits=4):
    import torch

    if torch.equal(ref, got):
        return True
    # a different split of K (less room for partial sums): both within the bars
    rt = torch.from_numpy(rows).cuda()
    want = C.qmm_f64(np.ascontiguousarray(x_bits[rows]), *tri, bits=bits)
    assert_close(got[rt], want, what + " (noalloc)")
    assert_close(ref[rt], want, what + " (forward)")
    if got.dtype == torch.float32:
        rms = float(ref.float().pow(2).mean().sqrt())
        assert float((got - ref).abs().max()) <= 1e-4 * rms, what
    return False


@pytest.mark.parametrize("dtype_name", ["bfloat16", "float32"])
@pytest.mark.parametrize("gemm_min", [32, 0])  # the GEMM from 32 rows on; the automatic choice
def test_noalloc_matches_forward_on_consecutive_calls(gpu_lib, dtype_name, gemm_min):
    import torch

    dtype = getattr(torch, dtype_name)
    cases = [  # (N, K, M), paths as with the GEMM from 32 rows on: each call followed
               # by a smaller one on the same scratch
        (2048, 3840, 512),    # GEMM, K split over workgroups: group sums + partial planes
        (40, 384, 40),        # small GEMM
        (3840, 15360, 2048),  # GEMM, the largest group-sum table of the benchmarked shapes
        (2048, 3840, 1),      # decode: no scratch
        (130, 1088, 300),     # GEMM with a ragged last octet
        (48, 576, 33),
    ]
    with gpu_lib.gemm_min_rows(gemm_min):
        for i, (n, k, m) in enumerate(cases):
            tri = random_triple(n, k, seed=9100 + i)
            x = A.make_activations(m, k, seed=9200 + i, outliers=True)
            lin = gpu_lib.QuantizedLinear(*dev_triple(*tri))
            ref, got = _both(lin, dev_x(x), dtype)
            rows = np.unique(np.linspace(0, m - 1, min(m, 12)).astype(np.int64))
            _compare(ref, got, x, tri, rows, f"n={n} k={k} m={m} {dtype_name} gemm_min={gemm_min}")
            lin.close()


def test_noalloc_eight_bit_and_a_large_call(gpu_lib, gemm_from_32):
    import torch

    # 8-bit: the GEMM's workspace over K' = 2K (x itself is read in place)
    rng = np.random.default_rng(91)
    w = A.round_to_bf16((rng.standard_normal((96, 3840)) * 0.02).astype(np.float32))
    tri = C.quantize(w, bits=8)
    for m in (64, 5):  # GEMM, then decode
        x = A.make_activations(m, 3840, seed=92 + m)
        lin = gpu_lib.QuantizedLinear(*dev_triple(*tri), bits=8)
        ref, got = _both(lin, dev_x(x), torch.float32)
        _compare(ref, got, x, tri, np.arange(m), f"8-bit m={m}", bits=8)
        lin.close()
    # 18000 rows over K' = 30720: the plan splits K only as far as the array's room for
    # partial sums allows (an unsplit plan needs none)
    small = C.quantize(A.round_to_bf16((rng.standard_normal((16, 15360)) * 0.02).astype(np.float32)), bits=8)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*small), bits=8)
    gen = torch.Generator(device="cuda").manual_seed(93)
    x = torch.randn((18000, 15360), generator=gen, device="cuda").to(torch.bfloat16)
    y = torch.full((18000, 16), float("nan"), dtype=torch.bfloat16, device="cuda")
    lin.forward_noalloc(x, y)
    ref = lin.forward(x)
    torch.cuda.synchronize()
    rows = np.array([0, 1, 255, 256, 9000, 17743, 17999])
    xs = x[torch.from_numpy(rows).cuda()].view(torch.int16).cpu().numpy().view(np.uint16)
    want = C.qmm_f64(xs, *small, bits=8)
    rt = torch.from_numpy(rows).cuda()
    assert_close(y[rt], want, "8-bit 18000 rows (noalloc)")
    assert_close(ref[rt], want, "8-bit 18000 rows (forward)")
    assert not torch.isnan(y.float()).any()
    lin.close()


def test_noalloc_through_raw_c_abi(gpu_lib, gemm_from_32):
    """The entry point called with raw pointers and the current stream, as a C caller
    would: status 0 and the forward's bits."""
    import torch

    lib = gpu_lib.load_library()
    tri = random_triple(256, 640, seed=93)
    x = dev_x(A.make_activations(300, 640, seed=94))
    lin = gpu_lib.QuantizedLinear(*dev_triple(*tri))
    y = torch.empty((300, 256), dtype=torch.bfloat16, device="cuda")
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = lib.gemma4_qlinear_forward_noalloc(lin._handle, st, ctypes.c_void_p(x.data_ptr()), 300,
                                            ctypes.c_void_p(y.data_ptr()), gpu_lib.DTYPE_BF16)
    assert rc == 0, gpu_lib.last_error()
    ref = lin.forward(x)
    torch.cuda.synchronize()
    assert torch.equal(ref, y)
    assert np.isfinite(A.bf16_bits_to_f32(host_bits(y))).all()
    lin.close()
