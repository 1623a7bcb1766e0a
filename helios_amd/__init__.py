"""helios_amd — MI355X-native affine 4-bit quantized matmul (MLX format).

The hot path of the reference (every q/k/v/o, gate/up/down and lm_head
projection of Gemma 4 12B, native/gemma4_mlx/src/native_model.cc:349-362 and
:1782-1795) as hand-written gfx950 HIP kernels behind a C ABI
(include/gemma4_qmm.h, libgemma4_qmm.so), plus the gate|up pair with the GeGLU
epilogue (native_model.cc:934-949, :378-386).  ``helios_amd.qmm`` is the Python
binding of that ABI.
"""

from .quantize import quantize  # noqa: F401
from .qmm import (  # noqa: F401
    Gemma4Error,
    QuantizedGeGLU,
    QuantizedLinear,
    Status,
    dequantize,
    load_library,
    quantized_matmul,
    runtime_version,
)
