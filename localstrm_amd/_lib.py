"""ctypes binding of liblsq.so (declared in include/localstrm_amd.h).

torch is imported before the library is opened: liblsq.so needs libamdhip64.so.7, and
when torch's copy (same SONAME) is already loaded the dynamic linker binds to it, so
torch and the kernels share one HIP runtime, one device context and one stream space.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "liblsq.so")

F32, F16, BF16, I8 = 0, 1, 2, 3
ACT_NONE, ACT_SILU_MUL = 0, 1
DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int

# name -> (restype, argtypes); must match include/localstrm_amd.h
SIGNATURES = {
    "lsq_version": (_int, []),
    "lsq_status_string": (ctypes.c_char_p, [_int]),
    "lsq_dequant_w8": (_int, [_vp, _vp, _int, _vp, _int, _i64, _i64, _vp]),
    "lsq_dequant_w4": (_int, [_vp, _vp, _int, _i64, _vp, _int, _i64, _i64, _vp]),
    "lsq_unpack_w4": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "lsq_w4_tiled_bytes": (_i64, [_i64, _i64]),
    "lsq_w4_retile": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "lsq_w4_untile": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "lsq_w8_tiled_bytes": (_i64, [_i64, _i64]),
    "lsq_w8_retile": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "lsq_w8_untile": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "lsq_w8_linear": (
        _int,
        [_vp, _i64, _vp, _vp, _vp, _int, _vp, _int, _vp, _i64, _int, _i64, _i64, _i64, _vp],
    ),
    "lsq_w4_linear": (
        _int,
        [_vp, _i64, _vp, _vp, _vp, _int, _i64, _vp, _int, _vp, _i64, _int, _i64, _i64, _i64, _vp],
    ),
    "lsq_linear_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "lsq_w8_linear_ws": (
        _int,
        [_vp, _i64, _vp, _vp, _vp, _int, _vp, _int, _vp, _i64, _int, _i64, _i64, _i64, _vp, _i64,
         _vp],
    ),
    "lsq_w4_linear_ws": (
        _int,
        [_vp, _i64, _vp, _vp, _vp, _int, _i64, _vp, _int, _vp, _i64, _int, _i64, _i64, _i64, _vp,
         _i64, _vp],
    ),
    "lsq_w8_linear_act": (
        _int,
        [_vp, _i64, _vp, _vp, _vp, _int, _vp, _int, _vp, _i64, _int, _i64, _i64, _i64, _int, _vp],
    ),
    "lsq_w4_linear_act": (
        _int,
        [_vp, _i64, _vp, _vp, _vp, _int, _i64, _vp, _int, _vp, _i64, _int, _i64, _i64, _i64, _int,
         _vp],
    ),
    "lsq_silu_mul": (_int, [_vp, _i64, _vp, _i64, _int, _i64, _i64, _vp]),
    "lsq_paged_attention_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "lsq_paged_attention_decode": (
        _int,
        [_vp, _vp, _vp, _int, _vp, _vp, _int, _vp, _i64, _vp, _vp, _i64, _i64, _vp, _int, _i64,
         _i64, _i64, _i64, _i64, _i64, _i64, _int, _vp, _i64, _vp],
    ),
    "lsq_w8a8_tiled_bytes": (_i64, [_i64, _i64]),
    "lsq_w8a8_retile": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "lsq_w8a8_untile": (_int, [_vp, _vp, _i64, _i64, _vp]),
    "lsq_act_quant_i8": (_int, [_vp, _i64, _int, _i64, _i64, _vp, _i64, _vp, _vp]),
    "lsq_w8a8_linear": (
        _int,
        [_vp, _i64, _vp, _vp, _int, _vp, _int, _vp, _i64, _int, _i64, _i64, _i64, _vp, _vp, _vp],
    ),
    "lsq_w8a8_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "lsq_w8a8_linear_ws": (
        _int,
        [_vp, _i64, _vp, _vp, _int, _vp, _int, _vp, _i64, _int, _i64, _i64, _i64, _vp, _vp, _vp, _i64,
         _vp],
    ),
    "lsq_quantize_w8": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "lsq_quantize_w4": (_int, [_vp, _int, _i64, _i64, _i64, _i64, _vp, _int, _vp, _vp, _vp]),
    "lsq_probe_empty": (_int, [_vp]),
    "lsq_probe_read": (_int, [_vp, _i64, _vp, _int, _int, _vp]),
    "lsq_w8a8_linear_noalloc": (
        _int,
        [_vp, _i64, _vp, _vp, _int, _vp, _int, _vp, _i64, _int, _i64, _i64, _i64, _vp],
    ),
}

_lib = None
_lock = threading.Lock()


class LsqError(RuntimeError):
    """A liblsq entry point returned a non-zero status."""


def load() -> ctypes.CDLL:
    """Open liblsq.so once. Raises if it has not been built: there is no CPU fallback."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build the HIP kernels with "
                    "`python -m localstrm_amd.build` (needs hipcc for gfx950)"
                )
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().lsq_status_string(status).decode()
        raise LsqError(f"{what}: {msg} (status {status})")


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODE[dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, float16 or bfloat16") from None


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()
