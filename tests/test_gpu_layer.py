"""One decoder layer's quantized matmuls chained as the model runs them, on the GPU
through the C ABI, against the oracle at every stage.

The reference runs the projections layer by layer, prefill at
native_model.cc:899-974 and decode at :1284-1328: q|k|v from the normed hidden
state, o from the attention output, gate and up (then geglu) from the normed
residual, down from the GeGLU output, and after the last layer the lm_head with the
softcap and argmax (:1782-1795, :3734).  Attention, norms and residuals are out of
scope, so each stage's input here is the previous stage's GPU output (identical
bf16 bytes go to the kernel and to the oracle): x -> qkv (q, k, v fused along N,
N = 8192) -> o (fed the q columns, 4096 wide) -> the gate|up GeGLU pair -> down ->
the greedy lm_head on the last row.  Run at decode M = 1 and at the prefill chunk
M = 2048 (sampled rows against the oracle there).

Bars: the plain outputs as in test_gpu_parity (bf16 max |err| <= 1e-2 * RMS +
ulp/2, plus one rounding of a value within 1e-4 * RMS of the exact one), the
GeGLU output as in test_gpu_geglu, the greedy token as in test_gpu_greedy.
"""

import numpy as np
import pytest

from oracle import affine as A
from oracle import c_oracle as C
from test_gpu_geglu import _check as check_geglu
from test_gpu_greedy import _check_token, _oracle as greedy_oracle
from test_gpu_parity import assert_close, assert_rounded, dev_triple, dev_x, host_bits, lm_head_triple

pytestmark = pytest.mark.gpu

HIDDEN = 3840
SEED = 20260630 + 5000


def _layer():
    q = A.make_weights(4096, HIDDEN, seed=SEED + 0)
    k = A.make_weights(2048, HIDDEN, seed=SEED + 1)
    v = A.make_weights(2048, HIDDEN, seed=SEED + 2)
    qkv = tuple(np.ascontiguousarray(np.concatenate([t[j] for t in (q, k, v)], axis=0)) for j in range(3))
    return {
        "qkv": qkv,
        "o": A.make_weights(HIDDEN, 4096, seed=SEED + 3),
        "gate": A.make_weights(15360, HIDDEN, seed=SEED + 4),
        "up": A.make_weights(15360, HIDDEN, seed=SEED + 5),
        "down": A.make_weights(HIDDEN, 15360, seed=SEED + 6),
    }


@pytest.mark.parametrize("m", [1, 2048])
def test_decoder_layer_chain(gpu_lib, m):
    import torch

    tri = _layer()
    qkv = gpu_lib.QuantizedLinear(*dev_triple(*tri["qkv"]))
    o = gpu_lib.QuantizedLinear(*dev_triple(*tri["o"]))
    mlp = gpu_lib.QuantizedGeGLU(dev_triple(*tri["gate"]), dev_triple(*tri["up"]))
    down = gpu_lib.QuantizedLinear(*dev_triple(*tri["down"]))
    head = gpu_lib.QuantizedLinear(*dev_triple(*lm_head_triple()))

    x = A.make_activations(m, HIDDEN, seed=SEED + 10 + m, outliers=m > 1)
    xd = dev_x(x)
    y_qkv = qkv.forward(xd)
    a = y_qkv[:, :4096].contiguous()          # the q columns stand in for the attention output
    y_o = o.forward(a)
    h = mlp.forward(y_o)
    y_d = down.forward(h)
    tok, val, logits = head.forward_greedy(y_d[-1:], softcap=30.0, return_logits=True)
    torch.cuda.synchronize()

    rows = np.arange(m) if m == 1 else np.sort(np.random.default_rng(m).choice(m, 8, replace=False))
    rt = torch.from_numpy(rows).cuda()
    sub = lambda t: np.ascontiguousarray(host_bits(t[rt]))  # noqa: E731

    want = C.qmm_f64(np.ascontiguousarray(x[rows]), *tri["qkv"])
    assert_close(y_qkv[rt], want, f"qkv m={m}")
    assert_rounded(y_qkv[rt], want, f"qkv m={m}")

    want = C.qmm_f64(sub(a), *tri["o"])
    assert_close(y_o[rt], want, f"o m={m}")
    assert_rounded(y_o[rt], want, f"o m={m}")

    g = C.qmm_f64(sub(y_o), *tri["gate"]).astype(np.float32)
    u = C.qmm_f64(sub(y_o), *tri["up"]).astype(np.float32)
    check_geglu(h[rt], g, u, f"gate|up GeGLU m={m}")

    want = C.qmm_f64(sub(h), *tri["down"])
    assert_close(y_d[rt], want, f"down m={m}")
    assert_rounded(y_d[rt], want, f"down m={m}")

    last = np.ascontiguousarray(host_bits(y_d[-1:]))
    sc = greedy_oracle(last, lm_head_triple(), 30.0, True)
    ok, worst = A.check_bf16_output(host_bits(logits), sc)
    assert ok, f"lm_head logits m={m}: worst error / RMS = {worst:.3e}"
    _check_token(tok.cpu().numpy(), sc, bf16=True)
    assert float(val.cpu()[0]) == float(A.bf16_bits_to_f32(host_bits(logits))[0, int(tok.cpu()[0])])

    for hnd in (qkv, o, mlp, down, head):
        hnd.close()
