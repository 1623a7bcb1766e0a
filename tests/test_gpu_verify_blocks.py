"""GPU parity at the verify-block sizes: every Gemma projection at full size with
M = 16 (the block cap) and a ragged M = 12, against the float64 oracle.

The reference's block decode runs all seven projections on a block of at most 16
rows (native_model.cc:1954-2026, :1158-1171, :1366-1369; the cap at
gemma4_mlx.h:77-79).  Cases: q, k, v, o, gate, up, down (bf16 and fp32 output on
every element), the q|k|v projections concatenated along N (one handle, y split
into column views, as a caller that fuses them would), and the gate|up GeGLU pair.
Bars as in test_gpu_parity.py and test_gpu_geglu.py."""

import numpy as np
import pytest

from oracle import affine as A
from oracle import c_oracle as C

from test_gpu_geglu import _check, _exact_gu
from test_gpu_parity import ACC_REL, PROJ, assert_close, assert_rounded, dev_triple, dev_x

pytestmark = pytest.mark.gpu

BLOCK_M = [12, 16]


@pytest.mark.parametrize("m", BLOCK_M)
@pytest.mark.parametrize("proj", sorted(PROJ))
def test_verify_block_projection(gpu_lib, proj, m):
    import torch

    n, k = PROJ[proj]
    wq, s, b = A.make_weights(n, k, seed=6100 + sorted(PROJ).index(proj))
    x = A.make_activations(m, k, seed=6200 + m, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    xd = dev_x(x)
    y_bf = lin.forward(xd)
    y_f = lin.forward(xd, out_dtype=torch.float32)
    torch.cuda.synchronize()
    y_exact = C.qmm_f64(x, wq, s, b)
    assert_close(y_bf, y_exact, f"{proj} m={m} bf16")
    assert_rounded(y_bf, y_exact, f"{proj} m={m} bf16")
    assert assert_close(y_f, y_exact, f"{proj} m={m} f32") < ACC_REL
    lin.close()


@pytest.mark.parametrize("m", BLOCK_M)
def test_verify_block_fused_qkv(gpu_lib, m):
    """q, k and v concatenated along N at load (8192 x 3840); the output's column
    views [0, 4096), [4096, 6144), [6144, 8192) are q, k and v, each checked
    against its own oracle product."""
    import torch

    names = ("q_proj", "k_proj", "v_proj")
    parts = [A.make_weights(*PROJ[p], seed=6300 + i) for i, p in enumerate(names)]
    wq, s, b = (np.concatenate([p[j] for p in parts]) for j in range(3))
    x = A.make_activations(m, 3840, seed=6400 + m, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    xd = dev_x(x)
    y_bf = lin.forward(xd)
    y_f = lin.forward(xd, out_dtype=torch.float32)
    torch.cuda.synchronize()
    col = 0
    for name, (pw, ps, pb) in zip(names, parts):
        n = PROJ[name][0]
        y_exact = C.qmm_f64(x, pw, ps, pb)
        assert_rounded(y_bf[:, col:col + n].contiguous(), y_exact, f"qkv:{name} m={m} bf16")
        assert assert_close(y_f[:, col:col + n].contiguous(), y_exact, f"qkv:{name} m={m} f32") < ACC_REL
        col += n
    lin.close()


@pytest.mark.parametrize("m", BLOCK_M)
def test_verify_block_gate_up_pair(gpu_lib, m):
    import torch

    gate = A.make_weights(15360, 3840, seed=6500)
    up = A.make_weights(15360, 3840, seed=6501)
    x = A.make_activations(m, 3840, seed=6600 + m, outliers=True)
    pair = gpu_lib.QuantizedGeGLU(dev_triple(*gate), dev_triple(*up))
    xd = dev_x(x)
    h = pair.forward(xd)
    hf = pair.forward(xd, out_dtype=torch.float32)
    torch.cuda.synchronize()
    g_exact, u_exact = _exact_gu(x, gate, up)
    _check(h, g_exact, u_exact, f"pair m={m} bf16")
    _check(hf, g_exact, u_exact, f"pair m={m} f32")
    pair.close()
