"""GPU parity of the quantized embedding gather (gemma4_qlinear_embed) — the take +
dequantize of native_model.cc:364-376 — against the oracle's dequantize:

  * fp32 rows are bit-exact (w = s*q + b is exact in fp32);
  * bf16 rows are those fp32 values rounded once to nearest even, bit-exact;
  * ids outside [0, N) give zero rows; duplicates and the ragged last row block work.
"""

import numpy as np
import pytest

from oracle import affine as A
from test_gpu_parity import dev_triple, host_bits, random_triple

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n,k", [(1003, 192), (4096 + 7, 3840), (262144, 3840)])
def test_embed_rows_bit_exact(gpu_lib, n, k):
    import torch

    tri = random_triple(n, k, 300 + n + k) if n < 262144 else A.make_weights(n, k, seed=20260630 + 3000)
    rng = np.random.default_rng(n)
    ids = np.concatenate([rng.integers(0, n, 37), [0, n - 1, n - 1, 5, -1, n, n + 100]]).astype(np.int32)
    lin = gpu_lib.QuantizedLinear(*dev_triple(*tri))
    idt = torch.from_numpy(ids).cuda()
    f = lin.embed(idt, out_dtype=torch.float32).cpu().numpy()
    b = host_bits(lin.embed(idt))
    lin.close()
    valid = (ids >= 0) & (ids < n)
    want = np.zeros((ids.size, k), np.float32)
    rows = ids[valid]
    want[valid] = A.dequantize(tri[0][rows], tri[1][rows], tri[2][rows])
    assert np.array_equal(f.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(b, A.f32_to_bf16_bits(want))
    assert not np.any(f[~valid])
