"""The 48-layer decoder pass (hidden 3840, 16 query / 8 KV heads of 256, FFN 15360,
every projection 4-bit group-64 on the library) at one decode token, chained: each
projection's input is the previous op's output (RMSNorm, attention over the token's
own position, residual adds in torch between them; bench.decoder_forward_m1).

The reference's forward (native_model.cc:1843-1911, the decode layer at
:993-1321) is what this chain follows; its attention and norms are plain torch ops
here, as in the benchmark's description of this workload.  Checks:
  * every residual state and the greedy token are finite / valid;
  * a HIP graph of the whole token, replayed three times with eager work between
    the replays, equals the eager run bit for bit (every residual state, the token);
  * layer 0's four launches, fed the chain's own intermediate values, against the
    float64 product of the handles' bit-exact dequantized weights (bars of
    test_gpu_parity.py), so the chain computes the projections it claims to."""

import numpy as np
import pytest

from oracle import affine as A

from test_gpu_geglu import _check
from test_gpu_parity import ACC_REL, assert_close, assert_rounded, host_bits

pytestmark = pytest.mark.gpu


def _exact(x_dev, lin):
    """float64 x . W^T from the handle's dequantized fp32 W (bit-exact)."""
    import torch

    w = lin.dequantize().double().cpu().numpy()
    x = x_dev.float().cpu().numpy().astype(np.float64)
    torch.cuda.synchronize()
    return x @ (w.reshape(-1, w.shape[-1]).T)


def test_decoder_48_layers_chained_m1(gpu_lib):
    import torch

    import bench

    net, lm = bench.build_decoder(torch, gpu_lib, layers=48)
    try:
        chk = bench.decoder_check(torch, net, lm, replays=3)
        print(f"48-layer chained forward: {chk}", flush=True)
        assert chk["finite"], "a residual state holds inf or NaN"
        assert chk["graph_equals_eager"], "graph replays differ from the eager forward"
        assert chk["token_stable"], f"token changed across replays: {chk}"
        assert 0 <= chk["token"] < 262144
        assert 0.1 < chk["final_rms"] < 1e6

        # layer 0 fed its own chain values, against float64 products
        L = net[0]
        x0 = torch.randn((1, bench.HIDDEN), device="cuda", generator=torch.Generator(device="cuda").manual_seed(5)) \
            .bfloat16()
        h = bench.rms_norm(torch, x0, L["norm"][0])
        qkv = L["qkv"].forward(h)
        qkv_f = L["qkv"].forward(h, out_dtype=torch.float32)
        want = _exact(h, L["qkv"])
        assert_rounded(qkv, want, "layer 0 qkv bf16")
        assert assert_close(qkv_f, want, "layer 0 qkv f32") < ACC_REL
        attn = qkv[:, 6144:8192].reshape(1, 8, 256).repeat_interleave(2, dim=1).reshape(1, 4096)
        o = L["o"].forward(attn)
        assert_rounded(o, _exact(attn, L["o"]), "layer 0 o bf16")
        x1 = (x0.float() + o.float()).bfloat16()
        h2 = bench.rms_norm(torch, x1, L["norm"][1])
        hh = L["mlp"].forward(h2)
        gu = _exact(h2, L["mlp"])  # [gate; up] rows of the pair's dequantize
        f = hh.shape[-1]
        _check(hh, gu[:, :f].astype(np.float32), gu[:, f:].astype(np.float32), "layer 0 gate|up GeGLU bf16")
        d = L["down"].forward(hh)
        assert_rounded(d, _exact(hh, L["down"]), "layer 0 down bf16")
        assert host_bits(d).shape == (1, bench.HIDDEN) and np.isfinite(A.bf16_bits_to_f32(host_bits(d))).all()
    finally:
        bench.free_decoder(net, lm)
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
