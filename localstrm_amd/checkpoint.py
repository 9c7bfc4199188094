"""Pre-packed quantized checkpoints: save a quantized model's layers once, load them onto a
GPU later without re-quantizing on the CPU or re-tiling on the GPU.

The reference keeps no quantized checkpoint: every load stages the float model on the CPU,
quantizes it there and moves it (src/kernels/quantization.py:593-610). `save_packed`
writes every QuantizedLinear, Int8GEMMLinear and CachedQuantizedLinear of a model to one
safetensors file: their state_dict tensors (the reference's buffers, in the reference's
layouts) plus, for layers on a GPU, the tiled weight copy the kernels stream. `load_packed`
installs them into a model of the same architecture (float or quantized) on any device; on
a GPU the saved tiled copy is installed as the layer's only weight copy (the canonical
tensor is not moved to the GPU at all). Every tensor is checked against the layer's
metadata (shape, dtype, tiled byte count) before it is installed, so a truncated or
mismatched file raises ValueError instead of reaching a kernel. safetensors stores raw
tensors and JSON metadata only (nothing in the file is executed on load).
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
             "bias": mod.bias is not None, "dtype": _dt_name(mod.output_dtype),
             "scale_dtype": _dt_name(mod.scale_w_t.dtype)}  # fp32, or what .half() made it
        if mod.weight_tiled.numel():
            tensors["weight_tiled"] = mod.weight_tiled.detach()
    else:
        # (the weight's own dtype: a .half() / .to(dtype) of the model converts it)
        e = {"cls": "CachedQuantizedLinear", "in_features": mod.in_features,
             "out_features": mod.out_features, "bias": mod.bias is not None,
             "dtype": _dt_name(mod.weight.dtype)}
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


_ST_DTYPES = {torch.int8: "I8", torch.uint8: "U8", torch.float32: "F32", torch.float16: "F16",
              torch.bfloat16: "BF16"}
_FLOAT_ST = ("F32", "F16", "BF16")


def _spec(e: dict, mod: nn.Module) -> Dict[str, Tuple[tuple, object]]:
    """Tensors a saved layer must hold: name -> (shape, safetensors dtype or the tuple of
    float dtypes allowed). Shapes follow from the layer's metadata, so a truncated or
    mismatched tensor is rejected before any kernel reads it."""
    n, k = int(e["out_features"]), int(e["in_features"])
    spec: Dict[str, Tuple[tuple, object]] = {}
    if isinstance(mod, QuantizedLinear):
        if mod.quant_type == "int8":
            spec["weight_q"] = ((n, k), "I8")
            spec["scale"] = ((n, 1), _ST_DTYPES[mod.scale.dtype])
        elif mod.quant_type == "int4":
            ng = 1 if mod.group_size is None else -(-k // mod.group_size)
            spec["weight_packed"] = ((n, (k + 1) // 2), "U8")
            spec["scale"] = ((n, ng), _ST_DTYPES[mod.scale.dtype])
        else:
            spec["weight"] = ((n, k), _FLOAT_ST)
        if e["bias"]:
            spec["bias"] = ((n,), _FLOAT_ST)
    elif isinstance(mod, Int8GEMMLinear):
        spec["weight_q_t"] = ((k, n), "I8")
        sdt = _DTYPES.get(e.get("scale_dtype", "float32"))
        if sdt not in _ST_DTYPES or not sdt.is_floating_point:
            raise ValueError(f"load_packed: Int8GEMMLinear scale dtype {e.get('scale_dtype')!r} is not a float type")
        spec["scale_w_t"] = ((1, n), _ST_DTYPES[sdt])
        if e["bias"]:
            spec["bias"] = ((n,), _FLOAT_ST)
    else:
        spec["weight"] = ((n, k), _ST_DTYPES[mod.dtype])
        if e["bias"]:
            spec["bias"] = ((n,), _FLOAT_ST)
    return spec


def _tiled_spec(mod: nn.Module) -> Tuple[int, str]:
    """(bytes, safetensors dtype) of the layer's tiled copy."""
    from . import _lib

    lib = _lib.load()
    n, k = mod.out_features, mod.in_features
    if isinstance(mod, Int8GEMMLinear):
        return lib.lsq_w8a8_tiled_bytes(n, k), "I8"
    if mod.quant_type == "int8":
        return lib.lsq_w8_tiled_bytes(n, k), "I8"
    return lib.lsq_w4_tiled_bytes(n, k), "U8"


def _build(e: dict, get, info, device: torch.device, tiled_ok: bool, lname: str) -> nn.Module:
    cls = e["cls"]
    try:
        if cls == "QuantizedLinear":
            sdt = _DTYPES.get(e.get("scale_dtype", ""), None)
            mod = QuantizedLinear(int(e["in_features"]), int(e["out_features"]), bias=bool(e["bias"]),
                                  quant_type=e["quant_type"], group_size=e["group_size"], scale_dtype=sdt)
        elif cls == "Int8GEMMLinear":
            mod = Int8GEMMLinear(int(e["in_features"]), int(e["out_features"]), bias=bool(e["bias"]),
                                 dtype=_DTYPES[e["dtype"]])
        elif cls == "CachedQuantizedLinear":
            mod = CachedQuantizedLinear(int(e["in_features"]), int(e["out_features"]), bias=bool(e["bias"]),
                                        dtype=_DTYPES[e["dtype"]])
        else:
            raise ValueError(f"load_packed: unknown layer class {cls!r}")
    except (KeyError, TypeError) as exc:
        raise ValueError(f"load_packed: layer {lname!r} has incomplete metadata ({exc})") from exc
    # check every tensor against the metadata before installing anything
    spec = _spec(e, mod)
    names = set(e["tensors"])
    quantized = isinstance(mod, Int8GEMMLinear) or (
        isinstance(mod, QuantizedLinear) and mod.quant_type in ("int8", "int4"))
    allowed = set(spec) | ({"weight_tiled"} if quantized else set())
    if names - allowed:
        raise ValueError(f"load_packed: layer {lname!r} holds unexpected tensors {sorted(names - allowed)}")
    if set(spec) - names:
        raise ValueError(f"load_packed: layer {lname!r} lacks tensors {sorted(set(spec) - names)}")
    for k_, (shape, dts) in spec.items():
        got_shape, got_dt = info(k_)
        ok_dt = got_dt in dts if isinstance(dts, tuple) else got_dt == dts
        if tuple(got_shape) != tuple(shape) or not ok_dt:
            raise ValueError(f"load_packed: {lname}.{k_} is {tuple(got_shape)} {got_dt}; the layer's "
                             f"metadata needs {tuple(shape)} {dts}")
    use_tiled = False
    if "weight_tiled" in names:
        nbytes, tdt = _tiled_spec(mod)
        got_shape, got_dt = info("weight_tiled")
        if tuple(got_shape) != (nbytes,) or got_dt != tdt:
            raise ValueError(f"load_packed: {lname}.weight_tiled is {tuple(got_shape)} {got_dt}; the "
                             f"layer's metadata needs ({nbytes},) {tdt}")
        use_tiled = tiled_ok and device.type == "cuda" and (
            isinstance(mod, Int8GEMMLinear) or mod._tiled_wanted(device))
    canon = "weight_q_t" if isinstance(mod, Int8GEMMLinear) else (
        mod._cname() if isinstance(mod, QuantizedLinear) and quantized else None)
    # install the saved tensors as they are (no copy into the constructor's zeros)
    for k_ in spec:
        if use_tiled and k_ == canon:
            continue
        t = get(k_).to(device)
        if k_ == "bias":
            mod.bias = nn.Parameter(t, requires_grad=False)
        elif k_ == "weight" and isinstance(mod, QuantizedLinear):
            mod.weight = nn.Parameter(t, requires_grad=False)
        else:
            setattr(mod, k_, t)
    if quantized:
        if use_tiled:
            t = get("weight_tiled").to(device)
            mod._buffers["weight_tiled"] = t
            mod._buffers[canon] = torch.empty(0, dtype=t.dtype, device=device)
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
        present = set(f.keys())
        modules = dict(model.named_modules())
        for name, e in layers.items():
            if name not in modules:
                raise ValueError(f"load_packed: the model has no module named {name!r}")
            if not isinstance(e, dict) or not isinstance(e.get("tensors"), list):
                raise ValueError(f"load_packed: layer {name!r} has malformed metadata")
            def key(k, n=name):
                return f"{n}.{k}" if n else k

            def info(k, key=key):
                if key(k) not in present:
                    raise ValueError(f"load_packed: {key(k)} is listed in the header but not in the file")
                sl = f.get_slice(key(k))
                return tuple(sl.get_shape()), sl.get_dtype()

            mod = _build(e, lambda k, key=key: f.get_tensor(key(k)), info, dev, tiled_ok, name)
            parent_name, _, attr = name.rpartition(".")
            setattr(modules[parent_name] if parent_name else model, attr, mod)
    return len(layers)
