"""localstrm_amd: MI355X-native weight-only quantized linear layer (INT8 / INT4 x bf16).

Drop-in for LocalStrm's src/kernels/quantization.py hot path; the compute runs in the
gfx950 HIP kernels of liblsq.so (built by `python -m localstrm_amd.build`).
"""

from .quantization import (  # noqa: F401
    VALID_MODES,
    FusedQuantizedLinear,
    QuantizedLinear,
    apply_optional_quantization,
    format_bytes,
    fuse_linears,
    load_and_quantize_model,
    pack_int4,
)

__all__ = [
    "VALID_MODES",
    "FusedQuantizedLinear",
    "QuantizedLinear",
    "apply_optional_quantization",
    "format_bytes",
    "fuse_linears",
    "load_and_quantize_model",
    "pack_int4",
]
