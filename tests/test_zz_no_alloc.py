"""GPU check of gemma4_qlinear_forward_noalloc (the allocation-free forward) through
the C ABI: on a sequence of calls in a row on one stream, each followed by a smaller
one that reuses the same static scratch, its output equals gemma4_qlinear_forward's
bit for bit wherever that call's scratch (gemma4_qlinear_scratch_bytes) fits the
64 MiB array, since both then run the same plan; otherwise both meet the oracle's
bars (fp32 within 2e-3 * RMS, bf16 within 1e-2 * RMS + ulp/2) and agree to within
the fp32 accumulation error.  The GEMM's scratch (the 256-row tile's group sums and
split-K partial sums) is planned to fit what the array has left, so a call of any
size runs (18000 rows of an 8-bit K = 15360 projection here).  It allocates nothing:
captured in global mode on a stream the library never saw, its graph holds kernel
nodes only (no allocation, free or memset node), and eager calls leave the device's
free memory unchanged.  (This check has no counterpart in the reference: its MLX ops
allocate per call.)"""

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


STATIC_SCRATCH = 64 << 20


def _compare(ref, got, x_bits, tri, rows, what, bits=4, lin=None):
    import torch

    if torch.equal(ref, got):
        return True
    if lin is not None:
        need = lin.scratch_bytes(ref.reshape(-1, ref.shape[-1]).shape[0])
        assert need > STATIC_SCRATCH, f"{what}: the forward's plan fits the array ({need} bytes) but the bits differ"
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
            _compare(ref, got, x, tri, rows, f"n={n} k={k} m={m} {dtype_name} gemm_min={gemm_min}", lin=lin)
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
        _compare(ref, got, x, tri, np.arange(m), f"8-bit m={m}", bits=8, lin=lin)
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


def test_noalloc_allocates_nothing(gpu_lib, gemm_from_32):
    """Captured in global mode (where a hipMalloc would fail the capture) on a stream
    the library has never seen, the allocation-free calls leave kernel nodes only;
    the plain forward captured the same way needs allocation nodes for the same split
    plan (the check can see them).  Eager calls on a fresh stream leave the device's
    free memory unchanged."""
    import torch

    import hip_graph_nodes as G

    cases = [(2048, 3840, 512), (3840, 15360, 2048), (2048, 3840, 1), (130, 1088, 300)]
    handles = []
    for i, (n, k, m) in enumerate(cases):
        lin = gpu_lib.QuantizedLinear(*dev_triple(*random_triple(n, k, seed=9300 + i)))
        x = dev_x(A.make_activations(m, k, seed=9400 + i))
        y = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
        handles.append((lin, x, y, m))
    assert handles[0][0].scratch_bytes(512) > 0 and handles[1][0].scratch_bytes(2048) > 0
    torch.cuda.synchronize()

    s = torch.cuda.Stream()
    types = G.capture_node_types(s, lambda: [lin.forward_noalloc(x, y, stream=s) for lin, x, y, _ in handles])
    assert types and all(t == G.KERNEL for t in types), f"node types {types}"

    # the plain forward on another never-seen stream: its split plans take scratch as
    # allocation nodes (so the node check above would have seen an allocation)
    s2 = torch.cuda.Stream()
    lin, x, y, _ = handles[0]
    types2 = G.capture_node_types(s2, lambda: lin.forward(x, out=y, stream=s2))
    assert G.MEM_ALLOC in types2 and G.MEMSET not in types2, f"node types {types2}"

    s3 = torch.cuda.Stream()
    with torch.cuda.stream(s3):
        # first use of the stream and of each kernel (lazily loaded runtime state)
        for lin, x, y, _ in handles:
            lin.forward_noalloc(x, y, stream=s3)
    torch.cuda.synchronize()
    free0 = G.free_device_bytes()
    with torch.cuda.stream(s3):
        for lin, x, y, _ in handles:
            lin.forward_noalloc(x, y, stream=s3)
    torch.cuda.synchronize()
    assert G.free_device_bytes() == free0, "forward_noalloc changed the device's free memory"
    for lin, _, _, _ in handles:
        lin.close()
