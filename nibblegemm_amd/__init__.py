"""nibblegemm_amd -- W4A16 (INT4 weight, fp16 activation) kernels for AMD
Instinct MI355X (gfx950).

Drop-in for the Python surface of arvindcr4/nibblegemm
(python/nibblegemm/__init__.py:19-38): the packed format and its helpers, the
kernel entry points, the batch-size dispatch and ``QuantLinear``.  The kernels
are hand-written HIP behind the C ABI in ``include/nibblegemm_amd.h``.

Symmetric GPTQ / AWQ 4-bit checkpoints are converted into the packed format
by :mod:`nibblegemm_amd.convert`.  The reference's offline GPTQ quantiser
(python/nibblegemm/gptq.py) is not part of this library: its names are kept
as stubs that raise ``NotImplementedError``, so ``from nibblegemm_amd import
*`` keeps the reference package's namespace.  Its Triton baseline is absent.
"""

from . import convert
from .ops import (DECODE_MAX_M, QuantLinear, dequant, extension, gemm, gemv, matmul, matmul_bias,
                  matmul_swiglu, rmsnorm_matmul, strip_major_cols, to_strip_major)
from .quant import (
    QuantizedWeight,
    StripMajorWeight,
    concat_columns,
    dequantize,
    from_strip_major,
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
    "gptq_quantize",
    "dequant",
    "dequantize",
    "extension",
    "find_decoder_blocks",
    "from_strip_major",
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


def _not_built(name: str):
    msg = (f"{name} is the reference's offline GPTQ quantiser (python/nibblegemm/gptq.py), "
           "which nibblegemm_amd does not provide; quantise with nibblegemm_amd.quantize "
           "(RTN) or convert a GPTQ checkpoint with nibblegemm_amd.convert.from_gptq")

    def stub(*_args, **_kwargs):
        raise NotImplementedError(msg)

    stub.__name__ = stub.__qualname__ = name
    stub.__doc__ = msg
    return stub


gptq_quantize = _not_built("gptq_quantize")
quantize_model_gptq = _not_built("quantize_model_gptq")
find_decoder_blocks = _not_built("find_decoder_blocks")
HessianAccumulator = _not_built("HessianAccumulator")
