"""GPU parity of the greedy lm_head (gemma4_qlinear_forward_greedy) against the oracle:
softcap_ops on the correctly rounded exact products, then the first maximum.

Bars:
  * logits (when returned): the output bars of the plain forward (bf16: max |err| <=
    1e-2 * RMS + ulp/2; fp32: <= 2e-3 * RMS) against softcap_ops of the exact products;
  * value: equals the returned logits at the returned token (one reduction);
  * token: the oracle's argmax whenever the oracle's best value leads the runner-up
    by more than 2 bf16 ulps (fp32: 1e-5 relative); otherwise the token's oracle
    value is within that margin of the best (the kernel's fp32 accumulation may
    order near-ties differently) — and ties of identical rows always go to the
    lower index.
"""

import numpy as np
import pytest

from oracle import affine as A
from oracle import c_oracle as C
from test_gpu_parity import BF16_REL, F32_REL, dev_triple, dev_x, host_bits, lm_head_triple, random_triple

pytestmark = pytest.mark.gpu


def _oracle(x, tri, cap, bf16):
    return A.softcap_ops(C.qmm_f64(x, *tri).astype(np.float32), cap, bf16=bf16)


def _check_token(tokens, sc, bf16):
    for r in range(sc.shape[0]):
        row = sc[r].astype(np.float64)
        best = int(np.argmax(row))
        top = row[best]
        margin = 2 * A.bf16_ulp(top) if bf16 else 1e-5 * abs(top) + 1e-30
        runner = np.max(np.delete(row, best)) if row.size > 1 else -np.inf
        t = int(tokens[r])
        if top - runner > margin:
            assert t == best, f"row {r}: token {t} != {best}"
        else:
            assert 0 <= t < row.size and row[t] >= top - margin, f"row {r}: token {t} value {row[t]} vs best {top}"


@pytest.mark.parametrize("n,k,m", [(4096 + 13, 256, 1), (4096 + 13, 256, 5), (20000, 3840, 16), (1000, 128, 3)])
@pytest.mark.parametrize("f32", [False, True])
@pytest.mark.parametrize("cap", [30.0, 0.0])
def test_greedy_head(gpu_lib, n, k, m, f32, cap):
    import torch

    tri = random_triple(n, k, 700 + n + k)
    x = A.make_activations(m, k, seed=800 + m, outliers=True)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*tri))
    dt = torch.float32 if f32 else torch.bfloat16
    tok, val, logits = lin.forward_greedy(dev_x(x), softcap=cap, out_dtype=dt, return_logits=True)
    tok2, val2, none = lin.forward_greedy(dev_x(x), softcap=cap, out_dtype=dt)
    torch.cuda.synchronize()
    assert none is None
    tok, val, tok2, val2 = (t.cpu().numpy() for t in (tok, val, tok2, val2))
    assert np.array_equal(tok, tok2) and np.array_equal(val.view(np.uint32), val2.view(np.uint32))
    sc = _oracle(x, tri, cap, bf16=not f32)
    lg = host_bits(logits)
    lgf = A.bf16_bits_to_f32(lg) if not f32 else lg
    if f32:
        ok, worst = A.check_f32_output(lg, sc, F32_REL)
    else:
        ok, worst = A.check_bf16_output(lg, sc, BF16_REL)
    assert ok, f"logits: worst error / RMS = {worst:.3e}"
    assert np.array_equal(val, lgf[np.arange(m), tok])  # value is the logit at the token
    assert np.all(lgf <= val[:, None])                   # and the row maximum
    assert all(int(tok[r]) == int(np.nonzero(lgf[r] == val[r])[0][0]) for r in range(m))  # the first one
    _check_token(tok, sc, bf16=not f32)
    lin.close()


def test_greedy_ties_go_to_the_lowest_index(gpu_lib):
    import torch

    n, k, m = 3000, 192, 4
    wq, s, b = random_triple(n, k, 91)
    x = A.make_activations(m, k, seed=92)
    best = A.greedy(_oracle(x, (wq, s, b), 30.0, True))[0]
    # copy the winning row of row 0's maximum into a lower and a higher index
    a = int(best[0])
    lo, hi = (a // 3, min(n - 1, a + 777)) if a > 0 else (0, n - 1)
    for arr in (wq, s, b):
        arr[lo] = arr[a]
        arr[hi] = arr[a]
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    tok, val, _ = lin.forward_greedy(dev_x(x), softcap=30.0)
    torch.cuda.synchronize()
    assert int(tok.cpu()[0]) == min(lo, a)
    lin.close()


@pytest.mark.parametrize("m", [1, 8, 16])
@pytest.mark.parametrize("f32", [False, True])
def test_greedy_lm_head_full_vocab(gpu_lib, m, f32):
    """The full 262144-token head at decode (M = 1) and verify blocks (M = 8, 16; the
    four-chunks-in-flight decode kernel): logits, values and tokens against the
    oracle, with and without returning the logits."""
    import torch

    wq, s, b = lm_head_triple()
    x = A.make_activations(m, 3840, seed=33 + m)
    lin = gpu_lib.QuantizedLinear(*dev_triple(wq, s, b))
    dt = torch.float32 if f32 else torch.bfloat16
    tok, val, logits = lin.forward_greedy(dev_x(x), softcap=30.0, out_dtype=dt, return_logits=True)
    tok2, val2, _ = lin.forward_greedy(dev_x(x), softcap=30.0, out_dtype=dt)
    torch.cuda.synchronize()
    sc = _oracle(x, (wq, s, b), 30.0, bf16=not f32)
    lg = host_bits(logits)
    ok, worst = (A.check_f32_output(lg, sc, F32_REL) if f32 else A.check_bf16_output(lg, sc, BF16_REL))
    assert ok, f"lm_head m={m} logits: worst error / RMS = {worst:.3e}"
    tok, val = tok.cpu().numpy(), val.cpu().numpy()
    assert np.array_equal(tok, tok2.cpu().numpy()) and np.array_equal(val.view(np.uint32),
                                                                      val2.cpu().numpy().view(np.uint32))
    lgf = lg if f32 else A.bf16_bits_to_f32(lg)
    assert np.array_equal(val, lgf[np.arange(m), tok])
    _check_token(tok, sc, bf16=not f32)
    lin.close()


def test_greedy_rejects_large_blocks_and_pairs(gpu_lib):
    import torch

    tri = random_triple(64, 64, 5)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*tri))
    with pytest.raises(gpu_lib.Gemma4Error) as e:
        lin.forward_greedy(dev_x(A.make_activations(17, 64, seed=1)))
    assert e.value.status == gpu_lib.Status.UNSUPPORTED_CONFIG
    with pytest.raises(gpu_lib.Gemma4Error):
        lin.forward_greedy(dev_x(A.make_activations(1, 64, seed=1)), softcap=-1.0)
    lin.close()
