"""GPU parity at bits = 8 (the QAT override, model_manifest.cc:148) through the C ABI:
the handle holds two 4-bit planes over 2K and reads x in place as [x | x], so every 4-bit path
(decode, GEMM, GeGLU pair, greedy head, embedding) is checked again at 8 bits against
the oracle's 8-bit dequantize / qmm, with the bars of test_gpu_parity.py (bit-exact
dequantize, bf16 output max|err| <= 1e-2 RMS + ulp/2, fp32 <= 2e-3 RMS)."""

import numpy as np
import pytest

from oracle import affine as A
from oracle import c_oracle as C
from test_gpu_parity import BF16_REL, F32_REL, assert_close, dev_triple, dev_x, host_bits

pytestmark = pytest.mark.gpu


def triple8(n, k, seed, std=0.02):
    rng = np.random.default_rng(seed)
    w = A.round_to_bf16((rng.standard_normal((n, k)) * std).astype(np.float32))
    return C.quantize(w, bits=8)


@pytest.mark.parametrize("n,k", [(16, 64), (40, 192), (33, 640), (4096 + 5, 3840)])
def test_q8_dequantize_bit_exact(gpu_lib, n, k):
    tri = triple8(n, k, n + k)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*tri), bits=8)
    got = lin.dequantize().cpu().numpy()
    assert lin.info()["bits"] == 8 and lin.info()["in_features"] == k
    lin.close()
    assert np.array_equal(got.view(np.uint32), A.dequantize(*tri, bits=8).view(np.uint32))
    # the host-array create path gives the same weights
    lin = gpu_lib.QuantizedLinear(*tri, bits=8)
    assert np.array_equal(lin.dequantize().cpu().numpy().view(np.uint32), got.view(np.uint32))
    lin.close()


@pytest.mark.parametrize("n,k,m", [(4096, 3840, 1), (2048, 3840, 4), (3840, 15360, 8), (300, 640, 17),
                                   (15360, 3840, 1), (15360, 3840, 4), (8192, 3840, 6), (4096, 3840, 3),
                                   (256, 640, 33), (130, 1088, 300), (512, 3840, 512)])
@pytest.mark.parametrize("f32", [False, True])
def test_q8_forward(gpu_lib, gemm_from_32, n, k, m, f32):
    import torch

    tri = triple8(n, k, 7 * n + k)
    x = A.make_activations(m, k, seed=m + n, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*tri), bits=8)
    y = lin.forward(dev_x(x), out_dtype=torch.float32 if f32 else torch.bfloat16)
    torch.cuda.synchronize()
    lin.close()
    rows = np.arange(m) if m <= 64 else np.sort(np.random.default_rng(m).choice(m, 16, replace=False))
    want = C.qmm_f64(np.ascontiguousarray(x[rows]), *tri, bits=8)
    assert_close(y[torch.from_numpy(rows).cuda()], want, f"q8 N={n} K={k} M={m} f32={f32}")


# the automatic path choice at 8 bits: 16-row slabs x N x 2K <= 5.5e7 run on the decode kernels
# past 32 rows (16-row slabs reading x in place as [x | x]; the global-x kernel for
# K = 3840 and 640 x 1088, slabs of one and of several row blocks)
@pytest.mark.parametrize("n,k,m", [(2048, 3840, 48), (512, 3840, 200), (640, 1088, 100), (4096, 3840, 9)])
@pytest.mark.parametrize("f32", [False, True])
def test_q8_decode_slabs_past_32_rows(gpu_lib, n, k, m, f32):
    import torch

    tri = triple8(n, k, 11 * n + k)
    x = A.make_activations(m, k, seed=3 * m + n, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*tri), bits=8)
    y = lin.forward(dev_x(x), out_dtype=torch.float32 if f32 else torch.bfloat16)
    torch.cuda.synchronize()
    lin.close()
    rows = np.unique(np.concatenate([np.linspace(0, m - 1, 20).astype(np.int64), [m - 1]]))
    want = C.qmm_f64(np.ascontiguousarray(x[rows]), *tri, bits=8)
    assert_close(y[torch.from_numpy(rows).cuda()], want, f"q8 slabs N={n} K={k} M={m} f32={f32}")


def test_q8_pair_greedy_and_embed(gpu_lib):
    import torch

    f, k = 520, 384
    gate, up = triple8(f, k, 1), triple8(f, k, 2)
    x = A.make_activations(3, k, seed=3)
    pair = gpu_lib.QuantizedGeGLU(dev_triple(*gate), dev_triple(*up), bits=8)
    h = pair.forward(dev_x(x), out_dtype=torch.float32)
    w = pair.dequantize().cpu().numpy()
    torch.cuda.synchronize()
    pair.close()
    assert np.array_equal(w[0].view(np.uint32), A.dequantize(*gate, bits=8).view(np.uint32))
    assert np.array_equal(w[1].view(np.uint32), A.dequantize(*up, bits=8).view(np.uint32))
    g = C.qmm_f64(x, *gate, bits=8).astype(np.float32)
    u = C.qmm_f64(x, *up, bits=8).astype(np.float32)
    ok, worst = A.check_f32_output(host_bits(h), A.geglu_ops(g, u, bf16=False), F32_REL)
    assert ok, f"q8 GeGLU f32: worst error / RMS = {worst:.3e}"

    n = 5000
    tri = triple8(n, k, 4)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*tri), bits=8)
    tok, val, logits = lin.forward_greedy(dev_x(x), softcap=30.0, return_logits=True)
    ids = np.array([0, 17, n - 1, n + 3], np.int32)
    emb = lin.embed(torch.from_numpy(ids).cuda(), out_dtype=torch.float32).cpu().numpy()
    torch.cuda.synchronize()
    lin.close()
    sc = A.softcap_ops(C.qmm_f64(x, *tri, bits=8).astype(np.float32), 30.0, bf16=True)
    ok, worst = A.check_bf16_output(host_bits(logits), sc, BF16_REL)
    assert ok, f"q8 greedy logits: worst error / RMS = {worst:.3e}"
    lg = A.bf16_bits_to_f32(host_bits(logits))
    tok = tok.cpu().numpy()
    assert np.array_equal(val.cpu().numpy(), lg[np.arange(3), tok]) and np.all(lg <= val.cpu().numpy()[:, None])
    deq = A.dequantize(*tri, bits=8)
    assert np.array_equal(emb[:3].view(np.uint32), deq[ids[:3]].view(np.uint32))
    assert not np.any(emb[3])
