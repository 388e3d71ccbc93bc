"""aestrix_amd -- MI355X-native (gfx950) MLX-format affine 4-bit quantized linear.

The hot path of the reference's FLUX.2 klein runtime: quantized Linear layers
with uint32 words of eight low-nibble-first 4-bit codes, one bf16 (scale, bias)
per 64 K elements, w = scale * q + bias.  Three hand-written HIP kernels behind
the C ABI of ``include/imq.h`` (``aestrix_amd/libimq.so``):

* ``dequantize``        -- standalone, bit-exact, HBM-bound
* ``qgemv``             -- M <= 16, register dequant, no MFMA, HBM-bound
* ``qgemm``             -- dense M, dequant fused into bf16 MFMA tiles

``quantized_matmul`` dispatches between the two matmul regimes;
``qmm_postscale`` / ``qmm_gate_add`` / ``qmm_swiglu`` fold the reference's
post-qmm glue kernels into the MFMA kernel's epilogue; ``cast_prescale`` and
``apply_linear`` are the f16 sandwich around them (x / 16 to f16, qmm, x 16).
"""

from ._lib import ImqError, ImqInvalid, ImqLibraryMissing, ImqUnsupported  # noqa: F401
from .ops import (  # noqa: F401
    BITS,
    GROUP_SIZE,
    Q,
    QuantizedLinear,
    apply_linear,
    cast_prescale,
    context,
    dequantize,
    dequantize_rows,
    dynamic_scale,
    qgemm,
    qgemv,
    qmm,
    qmm_add,
    qmm_gate_add,
    qmm_plan,
    qmm_postscale,
    qmm_swiglu,
    quantized_matmul,
    rmsnorm,
)
