"""MI355X (gfx950) IQ2_XXS quantised matmul — Python side of the package.

The compute path is libcmk_iq2.so (HIP kernels behind the C ABI in
include/cmk_iq2.h).  This package gives Python callers the same surface as the
reference crate's public API (iq2_matmul, iq2_matmul_with_activation_quant,
iq2_dequantize_to_f16, Iq2MatmulVariant, ActivationQuantMode/Config) over
PyTorch device tensors, plus the GGUF block split (iq2_split_gguf_blocks), the MLP's
silu(gate) * up step (swiglu, and iq2_matmul_swiglu: the step folded into the
up projection's epilogue) and seeded input generators.
"""

from . import cabi, inputs  # noqa: F401
from .activation_quant import ActivationQuantConfig, ActivationQuantMode  # noqa: F401
from .iq2_matmul import (  # noqa: F401
    Iq2MatmulError,
    Iq2MatmulVariant,
    iq2_dequantize_to_f16,
    iq2_matmul,
    iq2_matmul_with_activation_quant,
    iq2_s_matmul,
    iq2_split_gguf_blocks,
    iq2_matmul_swiglu,
    iq2_xs_matmul,
    iq2_xxs_matmul,
    iq3_s_matmul,
    swiglu,
)

__all__ = [
    "ActivationQuantConfig",
    "ActivationQuantMode",
    "Iq2MatmulError",
    "Iq2MatmulVariant",
    "iq2_dequantize_to_f16",
    "iq2_matmul",
    "iq2_matmul_with_activation_quant",
    "iq2_xxs_matmul",
    "iq2_xs_matmul",
    "iq2_s_matmul",
    "iq3_s_matmul",
    "iq2_split_gguf_blocks",
    "iq2_matmul_swiglu",
    "swiglu",
]
