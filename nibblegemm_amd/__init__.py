"""nibblegemm_amd -- W4A16 (INT4 weight, fp16 activation) kernels for AMD
Instinct MI355X (gfx950).

Drop-in for the Python surface of arvindcr4/nibblegemm
(python/nibblegemm/__init__.py:19-38): the packed format and its helpers, the
kernel entry points, the batch-size dispatch and ``QuantLinear``.  The kernels
are hand-written HIP behind the C ABI in ``include/nibblegemm_amd.h``.

The reference's GPTQ quantiser is here too (``gptq_quantize``,
``quantize_model_gptq``, ``HessianAccumulator``, ``find_decoder_blocks``, in
:mod:`nibblegemm_amd.gptq`, its column loop a kernel of this library);
symmetric GPTQ / AWQ 4-bit checkpoints are converted by
:mod:`nibblegemm_amd.convert`.  The reference's Triton baseline is not.
"""

from . import convert, gptq
from .gptq import HessianAccumulator, find_decoder_blocks, gptq_quantize, quantize_model_gptq
from .ops import (DECODE_MAX_M, QuantLinear, dequant, extension, gemm, gemv, matmul, matmul_bias,
                  matmul_swiglu, rmsnorm_matmul, strip_major_cols, to_strip_major)
from .quant import (
    QuantizedWeight,
    StripMajorWeight,
    concat_columns,
    dequantize,
    interleave_swiglu,
    pack_nibbles,
    quantize,
    quantize_device,
    reference_matmul,
    unpack_nibbles,
)

__all__ = [
    "DECODE_MAX_M",
    "HessianAccumulator",
    "QuantLinear",
    "QuantizedWeight",
    "concat_columns",
    "convert",
    "gptq",
    "gptq_quantize",
    "dequant",
    "dequantize",
    "extension",
    "find_decoder_blocks",
    "gemm",
    "gemv",
    "interleave_swiglu",
    "matmul",
    "matmul_bias",
    "matmul_swiglu",
    "pack_nibbles",
    "quantize",
    "quantize_device",
    "quantize_model_gptq",
    "reference_matmul",
    "rmsnorm_matmul",
    "StripMajorWeight",
    "strip_major_cols",
    "to_strip_major",
    "unpack_nibbles",
]
__version__ = "0.1.0"
