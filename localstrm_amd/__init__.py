"""localstrm_amd: MI355X-native quantized linear layers (INT8 / INT4 x bf16, W8A8).

Drop-in for LocalStrm's src/kernels/quantization.py hot path; the compute runs in the
gfx950 HIP kernels of liblsq.so (built by `python -m localstrm_amd.build`).
"""

from .checkpoint import load_packed, save_packed  # noqa: F401
from .paged_attention import paged_attention_decode  # noqa: F401
from .quantization import (  # noqa: F401
    VALID_MODES,
    CachedQuantizedLinear,
    FusedQuantizedLinear,
    Int8GEMMLinear,
    QuantizedLinear,
    apply_optional_quantization,
    can_use_int8_gemm,
    format_bytes,
    fuse_linears,
    load_and_quantize_model,
    pack_int4,
)

__all__ = [
    "VALID_MODES",
    "CachedQuantizedLinear",
    "FusedQuantizedLinear",
    "Int8GEMMLinear",
    "QuantizedLinear",
    "apply_optional_quantization",
    "can_use_int8_gemm",
    "format_bytes",
    "fuse_linears",
    "load_and_quantize_model",
    "load_packed",
    "pack_int4",
    "paged_attention_decode",
    "save_packed",
]
