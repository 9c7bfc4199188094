"""Weight-only quantized linear layer for MI355X: drop-in for LocalStrm's QuantizedLinear.

Mirrors the public surface of the reference module src/kernels/quantization.py:
`QuantizedLinear` (:34-149) with the same constructor, buffers (`weight_q`,
`weight_packed`, `scale`), `bias` parameter, `from_float`, `dequantize`, `forward` and
`memory_footprint_bytes`; `apply_optional_quantization` (:462-532) and
`load_and_quantize_model` (:535-630). What changes is where the arithmetic runs:
`forward` and `dequantize` of a quantized layer call the hand-written gfx950 kernels in
liblsq.so through its C ABI on the caller's current HIP stream. They never fall back to
a CPU or library implementation; on a CPU tensor, or without the built library, they
raise.

Extensions beyond the reference (all opt-in, defaults reproduce the reference):
  * `group_size` for INT4: scales `[N, ceil(K/group_size)]`, default `None` = the
    reference's per-output-channel scale `[N, 1]`.
  * `from_quantized` to install pre-quantized weights (pattern of
    CachedQuantizedLinear.from_quantized, quantization.py:241-256).
  * `weight_tiled`: a derived, non-persistent copy of `weight_q` / `weight_packed`
    re-tiled on the GPU for the decode kernels (16x128 tiles, each 1 KB wavefront load
    contiguous in HBM). It is rebuilt whenever the module moves to a GPU or the canonical
    buffer changes; `weight_q` / `weight_packed` keep the reference's layouts.
    LSQ_WEIGHT_LAYOUT=canonical makes forward() read the canonical buffers instead.
"""

from __future__ import annotations

import logging
import os
from typing import Any, List, Optional, Tuple, Union

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib

_log = logging.getLogger("mini_vllm.quantization")

VALID_MODES = ("none", "int8", "int4", "hybrid_int8")
TILE_K = 128  # column width of one tile of the tiled INT4 layout


def format_bytes(num_bytes: int) -> str:
    """Human-readable byte count (quantization.py:26-31)."""
    for unit in ["B", "KB", "MB", "GB"]:
        if abs(num_bytes) < 1024.0:
            return f"{num_bytes:3.2f} {unit}"
        num_bytes /= 1024.0
    return f"{num_bytes:.2f} TB"


def _use_tiled_layout() -> bool:
    return os.environ.get("LSQ_WEIGHT_LAYOUT", "tiled").lower() != "canonical"


def _require_gpu(t: torch.Tensor, what: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(
            f"QuantizedLinear.{what}: the quantized kernels run on the GPU only; "
            f"got a tensor on {t.device}. Move the module and its inputs to a HIP device "
            "(module.to('cuda'))."
        )


class _QuantizedLinearFn(torch.autograd.Function):
    """Forward through liblsq; backward gives grad w.r.t. x (and bias) only, since the
    quantized weights are buffers. Inference callers run under torch.no_grad() and never
    reach backward."""

    @staticmethod
    def forward(ctx, x, bias, module):  # type: ignore[override]
        ctx.module = module
        ctx.has_bias = bias is not None
        return module._hip_forward(x)

    @staticmethod
    def backward(ctx, gy):  # type: ignore[override]
        module = ctx.module
        w = module.dequantize(dtype=gy.dtype)
        gx = gy.matmul(w)
        gb = gy.reshape(-1, gy.shape[-1]).sum(0) if ctx.has_bias else None
        return gx, gb, None


class QuantizedLinear(nn.Module):
    """Drop-in replacement for nn.Linear with INT8 per-channel or INT4 packed weights.

    Reference: src/kernels/quantization.py:34-59 (constructor and buffers).
    """

    def __init__(
        self,
        in_features: int,
        out_features: int,
        bias: bool = False,
        quant_type: str = "none",
        group_size: Optional[int] = None,
        scale_dtype: Optional[torch.dtype] = None,
    ):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.quant_type = quant_type.lower()
        self.group_size = None
        if self.quant_type == "int8":
            self.register_buffer("weight_q", torch.zeros((out_features, in_features), dtype=torch.int8))
            self.register_buffer(
                "scale", torch.zeros((out_features, 1), dtype=scale_dtype or torch.float32)
            )
            self.register_buffer("weight_tiled", torch.zeros(0, dtype=torch.int8), persistent=False)
            self._tiled_key = None
        elif self.quant_type == "int4":
            if group_size is not None and group_size < 1:
                raise ValueError(f"group_size must be >= 1, got {group_size}")
            if group_size is not None and group_size < in_features:
                self.group_size = int(group_size)
            n_groups = 1 if self.group_size is None else -(-in_features // self.group_size)
            default_sdt = torch.float32 if self.group_size is None else torch.bfloat16
            self.register_buffer(
                "weight_packed",
                torch.zeros((out_features, (in_features + 1) // 2), dtype=torch.uint8),
            )
            self.register_buffer(
                "scale", torch.zeros((out_features, n_groups), dtype=scale_dtype or default_sdt)
            )
            self.register_buffer("weight_tiled", torch.zeros(0, dtype=torch.uint8), persistent=False)
            self._tiled_key = None
        else:
            self.weight = nn.Parameter(torch.zeros((out_features, in_features)))

        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features))
        else:
            self.register_parameter("bias", None)

    # ------------------------------------------------------------------ construction

    @classmethod
    def from_float(
        cls,
        float_linear: nn.Linear,
        quant_type: str = "none",
        group_size: Optional[int] = None,
        scale_dtype: Optional[torch.dtype] = None,
    ) -> "QuantizedLinear":
        """Quantize an nn.Linear (quantization.py:61-102).

        INT8 / per-channel INT4 follow the reference exactly: fp32 scale
        max|w|/127 (resp. /7) clamped to 1e-8, q = clamp(round_half_even(w / s)).
        Group-wise INT4 (group_size < in_features) takes the same steps per group of
        `group_size` columns and quantizes against the stored (dtype-rounded) scale.
        """
        qlayer = cls(
            in_features=float_linear.in_features,
            out_features=float_linear.out_features,
            bias=float_linear.bias is not None,
            quant_type=quant_type,
            group_size=group_size,
            scale_dtype=scale_dtype,
        )
        w = float_linear.weight.data.float()
        qt = quant_type.lower()
        if qt == "int8":
            max_val = torch.max(torch.abs(w), dim=-1, keepdim=True)[0]
            scale = torch.clamp(max_val / 127.0, min=1e-8)
            w_q = torch.clamp(torch.round(w / scale), -128, 127).to(torch.int8)
            qlayer.weight_q.copy_(w_q)
            qlayer.scale.copy_(scale)
        elif qt == "int4":
            if qlayer.group_size is None:
                max_val = torch.max(torch.abs(w), dim=-1, keepdim=True)[0]
                scale = torch.clamp(max_val / 7.0, min=1e-8)
                w_q = torch.clamp(torch.round(w / scale), -8, 7).to(torch.int8)
                qlayer.scale.copy_(scale)
            else:
                scale_q = _group_scales(w, qlayer.group_size, 7.0).to(qlayer.scale.dtype)
                s_full = scale_q.float().repeat_interleave(qlayer.group_size, dim=1)[:, : w.shape[1]]
                w_q = torch.clamp(torch.round(w / s_full), -8, 7).to(torch.int8)
                qlayer.scale.copy_(scale_q)
            qlayer.weight_packed.copy_(pack_int4(w_q))
        else:
            qlayer.weight.data.copy_(float_linear.weight.data)

        if float_linear.bias is not None:
            qlayer.bias.data.copy_(float_linear.bias.data)
        qlayer._refresh_tiled()
        return qlayer

    @classmethod
    def from_quantized(
        cls,
        weight: torch.Tensor,
        scale: torch.Tensor,
        bias: Optional[torch.Tensor] = None,
        quant_type: str = "int8",
        in_features: Optional[int] = None,
        group_size: Optional[int] = None,
    ) -> "QuantizedLinear":
        """Install pre-quantized weights (pattern of quantization.py:241-256).

        int8: `weight` int8 [N, K], `scale` [N] or [N, 1].
        int4: `weight` uint8 [N, ceil(K/2)] in the reference nibble layout, `scale`
        [N, ceil(K/group_size)] (or [N, 1] per-channel); `in_features` defaults to
        2 * weight.shape[1].
        The module is created on `weight`'s device.
        """
        qt = quant_type.lower()
        if qt == "int8":
            if weight.dtype != torch.int8 or weight.dim() != 2:
                raise ValueError("int8 weight must be a 2-D torch.int8 tensor")
            n, k = weight.shape
            layer = cls(k, n, bias=bias is not None, quant_type="int8", scale_dtype=scale.dtype)
            layer.weight_q = weight.detach().clone()
            layer.scale = scale.detach().reshape(n, 1).clone()
        elif qt == "int4":
            if weight.dtype != torch.uint8 or weight.dim() != 2:
                raise ValueError("int4 weight must be a 2-D torch.uint8 tensor of packed nibbles")
            n = weight.shape[0]
            k = int(in_features) if in_features is not None else 2 * weight.shape[1]
            if (k + 1) // 2 != weight.shape[1]:
                raise ValueError(f"packed weight has {weight.shape[1]} columns; in_features={k} needs {(k + 1) // 2}")
            layer = cls(k, n, bias=bias is not None, quant_type="int4", group_size=group_size,
                        scale_dtype=scale.dtype)
            g = 1 if layer.group_size is None else -(-k // layer.group_size)
            if scale.numel() != n * g:
                raise ValueError(f"scale has {scale.numel()} elements; expected [{n}, {g}]")
            layer.weight_packed = weight.detach().clone()
            layer.scale = scale.detach().reshape(n, g).clone()
        else:
            raise ValueError(f"from_quantized supports 'int8' and 'int4', got '{quant_type}'")
        if bias is not None:
            layer.bias = nn.Parameter(bias.detach().clone().to(weight.device), requires_grad=bias.requires_grad)
        layer.to(weight.device)
        layer._refresh_tiled()
        return layer

    # ------------------------------------------------------------------ tiled layout

    def _canonical(self) -> torch.Tensor:
        return self.weight_q if self.quant_type == "int8" else self.weight_packed

    def _tiled_wanted(self) -> bool:
        return (
            self.quant_type in ("int8", "int4")
            and self._canonical().device.type == "cuda"
            and self.in_features % TILE_K == 0
            and self.in_features > 0
            and self.out_features > 0
        )

    def _refresh_tiled(self) -> None:
        """(Re)build weight_tiled from the canonical buffer on the GPU; empty elsewhere."""
        if self.quant_type not in ("int8", "int4"):
            return
        src = self._canonical()
        tdt = torch.int8 if self.quant_type == "int8" else torch.uint8
        if not self._tiled_wanted():
            if self.weight_tiled.numel() != 0 or self.weight_tiled.device != src.device:
                self.weight_tiled = torch.zeros(0, dtype=tdt, device=src.device)
            self._tiled_key = None
            return
        if not src.is_contiguous():
            src = src.contiguous()
            if self.quant_type == "int8":
                self.weight_q = src
            else:
                self.weight_packed = src
        lib = _lib.load()
        w8 = self.quant_type == "int8"
        nbytes = (lib.lsq_w8_tiled_bytes if w8 else lib.lsq_w4_tiled_bytes)(
            self.out_features, self.in_features)
        if self.weight_tiled.numel() != nbytes or self.weight_tiled.device != src.device:
            self.weight_tiled = torch.empty(nbytes, dtype=tdt, device=src.device)
        with torch.cuda.device(src.device):
            _lib.check(
                (lib.lsq_w8_retile if w8 else lib.lsq_w4_retile)(
                    src.data_ptr(), self.weight_tiled.data_ptr(), self.out_features,
                    self.in_features, _lib.stream_handle(src.device)),
                "lsq_w8_retile" if w8 else "lsq_w4_retile",
            )
        self._tiled_key = (src.data_ptr(), src._version, src.device)

    def _apply(self, fn, recurse=True):
        super()._apply(fn, recurse)
        if self.quant_type in ("int8", "int4"):
            self._refresh_tiled()
        return self

    def _tiled_for_forward(self) -> Optional[torch.Tensor]:
        if not self._tiled_wanted() or not _use_tiled_layout():
            return None
        src = self._canonical()
        if self._tiled_key != (src.data_ptr(), src._version, src.device):
            self._refresh_tiled()
        return self.weight_tiled

    # ------------------------------------------------------------------ compute

    def dequantize(self, dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """Dequantized weight [N, K] in `dtype` (default fp32), bit-exact with
        quantization.py:104-127: round_T(T(q) * round_T(scale))."""
        if self.quant_type not in ("int8", "int4"):
            w = self.weight
            if dtype is not None and w.dtype != dtype:
                w = w.to(dtype)
            return w
        target = dtype if dtype is not None else torch.float32
        code = _lib.dtype_code(target)
        src = self.weight_q if self.quant_type == "int8" else self.weight_packed
        _require_gpu(src, "dequantize")
        lib = _lib.load()
        out = torch.empty((self.out_features, self.in_features), dtype=target, device=src.device)
        scale = self.scale.contiguous()
        with torch.cuda.device(src.device):
            stream = _lib.stream_handle(src.device)
            if self.quant_type == "int8":
                rc = lib.lsq_dequant_w8(src.contiguous().data_ptr(), scale.data_ptr(),
                                        _lib.dtype_code(scale.dtype), out.data_ptr(), code,
                                        self.out_features, self.in_features, stream)
            else:
                rc = lib.lsq_dequant_w4(src.contiguous().data_ptr(), scale.data_ptr(),
                                        _lib.dtype_code(scale.dtype), self._group_for_kernel(),
                                        out.data_ptr(), code, self.out_features,
                                        self.in_features, stream)
        _lib.check(rc, "lsq_dequant")
        return out

    def unpack_int4(self) -> torch.Tensor:
        """INT4 nibbles as int8 q in [-8, 7], [N, K] (the `unpacked` tensor of
        quantization.py:113-121), computed on the GPU."""
        if self.quant_type != "int4":
            raise ValueError("unpack_int4 needs quant_type 'int4'")
        _require_gpu(self.weight_packed, "unpack_int4")
        out = torch.empty((self.out_features, self.in_features), dtype=torch.int8,
                          device=self.weight_packed.device)
        with torch.cuda.device(out.device):
            _lib.check(
                _lib.load().lsq_unpack_w4(self.weight_packed.contiguous().data_ptr(), out.data_ptr(),
                                          self.out_features, self.in_features,
                                          _lib.stream_handle(out.device)),
                "lsq_unpack_w4",
            )
        return out

    def _group_for_kernel(self) -> int:
        return self.group_size if self.group_size is not None else max(self.in_features, 1)

    def _hip_forward(self, x: torch.Tensor) -> torch.Tensor:
        _require_gpu(x, "forward")
        code = _lib.dtype_code(x.dtype)
        src = self.weight_q if self.quant_type == "int8" else self.weight_packed
        if src.device != x.device:
            raise RuntimeError(
                f"QuantizedLinear.forward: input on {x.device} but weights on {src.device}"
            )
        if x.shape[-1] != self.in_features:
            raise RuntimeError(
                f"mat1 and mat2 shapes cannot be multiplied ({x.reshape(-1, x.shape[-1]).shape[0]}"
                f"x{x.shape[-1]} and {self.in_features}x{self.out_features})"
            )
        x2 = x.reshape(-1, self.in_features)
        if x2.stride(-1) != 1 or (x2.shape[0] > 1 and x2.stride(0) < self.in_features):
            x2 = x2.contiguous()
        m = x2.shape[0]
        y = torch.empty((m, self.out_features), dtype=x.dtype, device=x.device)
        bias = self.bias
        bias_ptr, bias_code = None, 0
        if bias is not None:
            bias = bias.detach()
            if bias.device != x.device:
                bias = bias.to(x.device)
            bias = bias.contiguous()
            bias_ptr, bias_code = bias.data_ptr(), _lib.dtype_code(bias.dtype)
        scale = self.scale if self.scale.is_contiguous() else self.scale.contiguous()
        lib = _lib.load()
        ldx = x2.stride(0) if m > 1 else self.in_features
        stream = _lib.stream_handle(x.device)
        tiled = self._tiled_for_forward()
        if self.quant_type == "int8":
            rc = lib.lsq_w8_linear(x2.data_ptr(), ldx, src.data_ptr(), _lib.ptr(tiled),
                                   scale.data_ptr(), _lib.dtype_code(scale.dtype), bias_ptr,
                                   bias_code, y.data_ptr(), self.out_features, code, m,
                                   self.out_features, self.in_features, stream)
        else:
            rc = lib.lsq_w4_linear(x2.data_ptr(), ldx, src.data_ptr(), _lib.ptr(tiled),
                                   scale.data_ptr(), _lib.dtype_code(scale.dtype),
                                   self._group_for_kernel(), bias_ptr, bias_code, y.data_ptr(),
                                   self.out_features, code, m, self.out_features,
                                   self.in_features, stream)
        _lib.check(rc, f"lsq_{'w8' if self.quant_type == 'int8' else 'w4'}_linear")
        return y.reshape(*x.shape[:-1], self.out_features)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """y = x @ dequantize(x.dtype).T + bias.to(x.dtype) (quantization.py:129-141)."""
        if self.quant_type not in ("int8", "int4"):
            w_float = self.dequantize(dtype=x.dtype)
            if w_float.device != x.device:
                w_float = w_float.to(x.device)
            bias = self.bias
            if bias is not None:
                bias = bias.to(device=x.device, dtype=x.dtype)
            return F.linear(x, w_float, bias)
        needs_grad = torch.is_grad_enabled() and (
            x.requires_grad or (self.bias is not None and self.bias.requires_grad)
        )
        if needs_grad:
            return _QuantizedLinearFn.apply(x, self.bias, self)
        return self._hip_forward(x)

    def memory_footprint_bytes(self) -> int:
        """Bytes of all buffers and parameters (quantization.py:143-149), including the
        derived tiled copy when it exists."""
        total = 0
        for b in self.buffers():
            total += b.numel() * b.element_size()
        for p in self.parameters():
            total += p.numel() * p.element_size()
        return total

    def extra_repr(self) -> str:
        g = f", group_size={self.group_size}" if self.group_size else ""
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, quant_type={self.quant_type}{g}")


class FusedQuantizedLinear(nn.Module):
    """Several quantized layers that read the same input, run as one launch.

    The concatenated-N form of a decoder layer's q/k/v projections and of its gate/up
    projections (modeling_qwen2.py:46-48 and :206-208 call them one after the other on
    the same hidden state). The layers' weights, scales and biases are concatenated along
    the output dimension into one QuantizedLinear (`fused`); forward runs it once and
    returns one output per layer, as views of the single output (last dimension split
    into `splits`). Every output element is computed exactly as its own layer would
    compute it; only the launch count changes.
    """

    def __init__(self, fused: QuantizedLinear, splits: List[int]):
        super().__init__()
        self.fused = fused
        self.splits = [int(v) for v in splits]
        self.in_features = fused.in_features
        self.out_features = fused.out_features

    def forward(self, x: torch.Tensor) -> Tuple[torch.Tensor, ...]:
        return tuple(torch.split(self.fused(x), self.splits, dim=-1))

    def memory_footprint_bytes(self) -> int:
        return self.fused.memory_footprint_bytes()

    def extra_repr(self) -> str:
        return f"splits={self.splits}"


def fuse_linears(layers: List[QuantizedLinear]) -> FusedQuantizedLinear:
    """Fuse quantized layers with the same input into one launch (see
    FusedQuantizedLinear). All layers must share quant_type (int8 / int4), in_features,
    group size, scale dtype and device; a layer without bias contributes zeros when
    others have one."""
    if not layers:
        raise ValueError("fuse_linears needs at least one layer")
    first = layers[0]
    qt = first.quant_type
    if qt not in ("int8", "int4"):
        raise ValueError(f"fuse_linears supports int8 / int4 layers, got '{qt}'")
    for l in layers[1:]:
        if l.quant_type != qt:
            raise ValueError(f"fuse_linears: quant_type {l.quant_type} differs from {qt}")
        if l.in_features != first.in_features:
            raise ValueError(f"fuse_linears: in_features {l.in_features} differs from {first.in_features}")
        if l.group_size != first.group_size:
            raise ValueError(f"fuse_linears: group_size {l.group_size} differs from {first.group_size}")
        if l.scale.dtype != first.scale.dtype:
            raise ValueError(f"fuse_linears: scale dtype {l.scale.dtype} differs from {first.scale.dtype}")
        if l._canonical().device != first._canonical().device:
            raise ValueError("fuse_linears: layers are on different devices")
    weight = torch.cat([l._canonical() for l in layers], dim=0)
    scale = torch.cat([l.scale for l in layers], dim=0)
    bias = None
    if any(l.bias is not None for l in layers):
        bdt = next(l.bias.dtype for l in layers if l.bias is not None)
        bias = torch.cat([
            l.bias.detach().to(bdt) if l.bias is not None
            else torch.zeros(l.out_features, dtype=bdt, device=weight.device)
            for l in layers
        ])
    fused = QuantizedLinear.from_quantized(weight, scale, bias, quant_type=qt,
                                           in_features=first.in_features,
                                           group_size=first.group_size)
    return FusedQuantizedLinear(fused, [l.out_features for l in layers])


# ---------------------------------------------------------------------------- helpers


def pack_int4(q: torch.Tensor) -> torch.Tensor:
    """int8 q in [-8, 7] [N, K] -> uint8 [N, ceil(K/2)]; byte j = (q[2j]+8) | (q[2j+1]+8) << 4.
    Odd K pads the high nibble with 0 (quantization.py:86-91)."""
    u = (q + 8).to(torch.uint8)
    low = u[:, 0::2]
    high = u[:, 1::2] if u.shape[1] % 2 == 0 else F.pad(u[:, 1::2], (0, 1))
    return low | (high << 4)


def _group_scales(w: torch.Tensor, group_size: int, qmax: float) -> torch.Tensor:
    """fp32 scales [N, ceil(K/g)] = clamp(max|w| over each group / qmax, 1e-8)."""
    n, k = w.shape
    g = -(-k // group_size)
    pad = g * group_size - k
    wa = torch.abs(w)
    if pad:
        wa = F.pad(wa, (0, pad))
    max_val = wa.reshape(n, g, group_size).amax(dim=-1)
    return torch.clamp(max_val / qmax, min=1e-8)


def apply_optional_quantization(
    model: nn.Module, quant_type: str = "none", group_size: Optional[int] = None
) -> Tuple[int, int]:
    """Replace the 7 transformer projections with QuantizedLinear (quantization.py:462-532).

    Returns (orig_weight_bytes, quantized_weight_bytes). `group_size` applies to int4.
    The 'hybrid_int8' mode (W8A8 + cached fp16 layers) is not part of this library.
    """
    quant_type = quant_type.lower()
    if quant_type not in VALID_MODES:
        raise ValueError(f"Invalid quantization type '{quant_type}'. Must be one of {VALID_MODES}.")

    orig_bytes = sum(p.numel() * p.element_size() for p in model.parameters())
    if quant_type == "none":
        return orig_bytes, orig_bytes

    layers = None
    if hasattr(model, "model") and hasattr(model.model, "layers"):
        layers = model.model.layers
    elif hasattr(model, "layers"):
        layers = model.layers

    targets = []
    if layers is not None:
        for layer in layers:
            if hasattr(layer, "self_attn"):
                for proj in ("q_proj", "k_proj", "v_proj", "o_proj"):
                    mod = getattr(layer.self_attn, proj, None)
                    if isinstance(mod, nn.Linear):
                        targets.append((layer.self_attn, proj, mod))
            if hasattr(layer, "mlp"):
                for proj in ("gate_proj", "up_proj", "down_proj"):
                    mod = getattr(layer.mlp, proj, None)
                    if isinstance(mod, nn.Linear):
                        targets.append((layer.mlp, proj, mod))

    if not targets:
        raise ValueError(
            f"Quantization '{quant_type}' failed: no compatible linear layers found in model "
            f"architecture ({model.__class__.__name__}). Supported architectures require transformer "
            f"blocks with standard self_attn (q, k, v, o) and mlp (gate, up, down) projections "
            f"(e.g., LLaMA, Qwen2, Mistral)."
        )
    if quant_type == "hybrid_int8":
        raise NotImplementedError(
            "quantization 'hybrid_int8' (W8A8 Int8GEMMLinear + cached fp16 attention) is not "
            "provided by localstrm_amd; use 'int8' or 'int4'"
        )

    for parent, proj, mod in targets:
        setattr(parent, proj, QuantizedLinear.from_float(mod, quant_type, group_size=group_size))

    quant_bytes = 0
    for m in model.modules():
        if isinstance(m, QuantizedLinear):
            quant_bytes += m.memory_footprint_bytes()
        elif len(list(m.children())) == 0:
            for p in m.parameters(recurse=False):
                quant_bytes += p.numel() * p.element_size()
    return orig_bytes, quant_bytes


def load_and_quantize_model(
    model_name_or_path: Union[str, nn.Module],
    device: Union[torch.device, str],
    quantization: str = "none",
    dtype: Optional[torch.dtype] = None,
    logger: Optional[Any] = None,
    trust_remote_code: bool = False,
    group_size: Optional[int] = None,
) -> Tuple[nn.Module, int, int]:
    """Load a CausalLM (or take an nn.Module), quantize on CPU, then move to `device`
    (quantization.py:535-630). Moving a quantized model to a GPU builds the tiled INT4
    layout there (QuantizedLinear._apply)."""
    quantization = quantization.lower()
    if quantization not in VALID_MODES:
        raise ValueError(f"Invalid quantization mode '{quantization}'. Must be one of {VALID_MODES}.")
    if isinstance(device, str):
        device = torch.device(device)
    if dtype is None:
        dtype = torch.float32 if device.type == "cpu" else torch.float16
    log_fn = logger.info if logger is not None else None

    try:
        if isinstance(model_name_or_path, nn.Module):
            model = model_name_or_path
            if quantization != "none" and device.type == "cuda":
                if log_fn:
                    log_fn("Staging model on CPU before applying %s quantization...", quantization.upper())
                model = model.to("cpu")
                model.eval()
                orig_bytes, quant_bytes = apply_optional_quantization(model, quantization, group_size)
                if log_fn:
                    log_fn("Transferring quantized model to %s...", device)
                model = model.to(device)
            else:
                model = model.to(device)
                model.eval()
                if quantization != "none":
                    if log_fn:
                        log_fn("Applying %s weight quantization on %s...", quantization.upper(), device)
                    orig_bytes, quant_bytes = apply_optional_quantization(model, quantization, group_size)
                else:
                    orig_bytes = sum(p.numel() * p.element_size() for p in model.parameters())
                    quant_bytes = orig_bytes
            return model, orig_bytes, quant_bytes

        from transformers import AutoModelForCausalLM

        def _from_pretrained(dev):
            try:
                return AutoModelForCausalLM.from_pretrained(
                    model_name_or_path, dtype=dtype, trust_remote_code=trust_remote_code
                ).to(dev)
            except TypeError:
                return AutoModelForCausalLM.from_pretrained(
                    model_name_or_path, torch_dtype=dtype, trust_remote_code=trust_remote_code
                ).to(dev)

        if quantization != "none" and device.type == "cuda":
            if log_fn:
                log_fn("Staging uncompressed model on CPU before applying %s quantization...", quantization.upper())
            model = _from_pretrained("cpu")
            model.eval()
            if log_fn:
                log_fn("Applying %s weight quantization on CPU...", quantization.upper())
            orig_bytes, quant_bytes = apply_optional_quantization(model, quantization, group_size)
            if log_fn:
                savings = (1.0 - (quant_bytes / orig_bytes)) * 100 if orig_bytes > 0 else 0.0
                log_fn("Transferring quantized model to %s (%.1f%% VRAM reduction, compressed from %.2f GB to %.2f GB)...",
                       device, savings, orig_bytes / (1024**3), quant_bytes / (1024**3))
            model = model.to(device)
        else:
            model = _from_pretrained(device)
            model.eval()
            if quantization != "none":
                if log_fn:
                    log_fn("Applying %s weight quantization on %s...", quantization.upper(), device)
                orig_bytes, quant_bytes = apply_optional_quantization(model, quantization, group_size)
            else:
                orig_bytes = sum(p.numel() * p.element_size() for p in model.parameters())
                quant_bytes = orig_bytes
        return model, orig_bytes, quant_bytes
    except Exception:
        if torch.cuda.is_available():
            torch.cuda.empty_cache()
        raise
