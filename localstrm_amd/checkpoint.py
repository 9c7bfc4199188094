"""Pre-packed quantized checkpoints: save a quantized model's layers once, load them onto a
GPU later without re-quantizing on the CPU or re-tiling on the GPU.

The reference keeps no quantized checkpoint: every load stages the float model on the CPU,
quantizes it there and moves it (src/kernels/quantization.py:593-610). `save_packed`
writes every QuantizedLinear, Int8GEMMLinear and CachedQuantizedLinear of a model to one
safetensors file: their state_dict tensors (the reference's buffers) plus, for layers on a
GPU, the derived tiled weight copy the kernels stream. `load_packed` installs them into a
model of the same architecture (float or quantized) on any device; on a GPU the saved
tiled copy is used as is. safetensors stores raw tensors and JSON metadata only (nothing in
the file is executed on load).
"""

from __future__ import annotations

import json
from typing import Dict, Tuple, Union

import torch
import torch.nn as nn

from .quantization import CachedQuantizedLinear, Int8GEMMLinear, QuantizedLinear

FORMAT = "localstrm_amd.packed"
VERSION = 1
# Version of the tiled weight layouts (16 x 128 tiles; INT4 nibble order; W8A8 K padding).
# A file whose tiled copies were written with another version is loaded from the canonical
# buffers and re-tiled.
TILED_LAYOUT = 1

_DTYPES = {"float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16}


def _dt_name(dt: torch.dtype) -> str:
    return str(dt).replace("torch.", "")


def _entry(mod: nn.Module) -> Tuple[dict, Dict[str, torch.Tensor]]:
    tensors = {k: v.detach() for k, v in mod.state_dict().items()}
    if isinstance(mod, QuantizedLinear):
        e = {"cls": "QuantizedLinear", "quant_type": mod.quant_type, "in_features": mod.in_features,
             "out_features": mod.out_features, "group_size": mod.group_size,
             "bias": mod.bias is not None}
        if mod.quant_type in ("int8", "int4"):
            e["scale_dtype"] = _dt_name(mod.scale.dtype)
            if mod.weight_tiled.numel():
                tensors["weight_tiled"] = mod.weight_tiled.detach()
    elif isinstance(mod, Int8GEMMLinear):
        e = {"cls": "Int8GEMMLinear", "in_features": mod.in_features, "out_features": mod.out_features,
             "bias": mod.bias is not None, "dtype": _dt_name(mod.output_dtype)}
        if mod.weight_tiled.numel():
            tensors["weight_tiled"] = mod.weight_tiled.detach()
    else:
        e = {"cls": "CachedQuantizedLinear", "in_features": mod.in_features,
             "out_features": mod.out_features, "bias": mod.bias is not None,
             "dtype": _dt_name(mod.dtype)}
    return e, tensors


def save_packed(model: nn.Module, path: str) -> int:
    """Write every quantized layer of `model` to the safetensors file `path`; returns the
    number of layers written. Layers on a GPU also write their tiled weight copy."""
    from safetensors.torch import save_file

    layers, out = {}, {}
    for name, mod in model.named_modules():
        if not isinstance(mod, (QuantizedLinear, Int8GEMMLinear, CachedQuantizedLinear)):
            continue
        e, tensors = _entry(mod)
        e["tensors"] = sorted(tensors)
        layers[name] = e
        for k, t in tensors.items():
            out[f"{name}.{k}" if name else k] = t.to("cpu").contiguous()
    if not layers:
        raise ValueError("save_packed: the model has no quantized layers")
    meta = {"format": FORMAT, "version": str(VERSION), "tiled_layout": str(TILED_LAYOUT),
            "layers": json.dumps(layers)}
    save_file(out, path, metadata=meta)
    return len(layers)


def _build(e: dict, get, device: torch.device, tiled_ok: bool) -> nn.Module:
    cls = e["cls"]
    if cls == "QuantizedLinear":
        sdt = _DTYPES.get(e.get("scale_dtype", ""), None)
        mod = QuantizedLinear(e["in_features"], e["out_features"], bias=e["bias"],
                              quant_type=e["quant_type"], group_size=e["group_size"], scale_dtype=sdt)
    elif cls == "Int8GEMMLinear":
        mod = Int8GEMMLinear(e["in_features"], e["out_features"], bias=e["bias"],
                             dtype=_DTYPES[e["dtype"]])
    elif cls == "CachedQuantizedLinear":
        mod = CachedQuantizedLinear(e["in_features"], e["out_features"], bias=e["bias"],
                                    dtype=_DTYPES[e["dtype"]])
    else:
        raise ValueError(f"load_packed: unknown layer class {cls!r}")
    # install the saved tensors as they are (no copy into the constructor's zeros)
    for k in e["tensors"]:
        if k == "weight_tiled":
            continue
        t = get(k).to(device)
        if k == "bias":
            mod.bias = nn.Parameter(t, requires_grad=False)
        elif k == "weight" and isinstance(mod, QuantizedLinear):
            mod.weight = nn.Parameter(t, requires_grad=False)
        else:
            setattr(mod, k, t)
    if isinstance(mod, (QuantizedLinear, Int8GEMMLinear)) and (
            not isinstance(mod, QuantizedLinear) or mod.quant_type in ("int8", "int4")):
        src = mod.weight_q_t if isinstance(mod, Int8GEMMLinear) else mod._canonical()
        if tiled_ok and "weight_tiled" in e["tensors"] and device.type == "cuda":
            mod.weight_tiled = get("weight_tiled").to(device)
            mod._tiled_key = (src.data_ptr(), src._version, src.device)
        else:
            mod._refresh_tiled()
    return mod


def load_packed(model: nn.Module, path: str, device: Union[str, torch.device, None] = None) -> int:
    """Install the layers saved in `path` into `model` (same module names; the layers it
    holds there, float or quantized, are replaced) on `device` (default: where the file's
    tensors are loaded, the CPU). Returns the number of layers installed. On a GPU the saved
    tiled copies are installed directly, skipping the re-tile kernels."""
    from safetensors import safe_open

    dev = torch.device(device) if device is not None else torch.device("cpu")
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT:
            raise ValueError(f"load_packed: {path} is not a {FORMAT} file")
        if int(meta.get("version", "0")) > VERSION:
            raise ValueError(f"load_packed: file version {meta.get('version')} is newer than {VERSION}")
        tiled_ok = meta.get("tiled_layout") == str(TILED_LAYOUT)
        layers = json.loads(meta["layers"])
        modules = dict(model.named_modules())
        for name, e in layers.items():
            if name not in modules:
                raise ValueError(f"load_packed: the model has no module named {name!r}")
            mod = _build(e, lambda k, n=name: f.get_tensor(f"{n}.{k}" if n else k), dev, tiled_ok)
            parent_name, _, attr = name.rpartition(".")
            setattr(modules[parent_name] if parent_name else model, attr, mod)
    return len(layers)
