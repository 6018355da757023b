"""higgs_amd: MI355X (gfx950) MLX-format affine group-quantized linear path.

quantized_matmul (qmv for decode, MFMA qmm for prefill), gather_qmm (MoE
experts) and dequantize, implemented as hand-written HIP kernels in
libhiggs_qmm.so behind the C ABI in include/higgs_qmm.h. This package is the
torch-facing host facade over that ABI.
"""
from ._lib import HiggsQmmError, version  # noqa: F401
from .ops import (  # noqa: F401
    dequantize,
    embedding,
    gather_qmm,
    quantized_matmul,
    result_dtype,
)
