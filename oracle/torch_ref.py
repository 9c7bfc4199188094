"""Torch-CPU restatement of the reference forward. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import this
module. It re-expresses LocalStrm's QuantizedLinear.dequantize + forward
(src/kernels/quantization.py:104-141) as the same sequence of ATen ops on CPU tensors:
materialize the dequantized weight in the activation dtype, then F.linear. It is the
"reference CPU path" that bench.py times next to the GPU kernels, and a second,
independently written formulation that tests cross-check against the numpy oracle.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def dequant_int8(weight_q: torch.Tensor, scale: torch.Tensor, dtype=torch.float32) -> torch.Tensor:
    """quantization.py:106-108: weight_q.to(T) * scale.to(T)."""
    return weight_q.to(dtype) * scale.reshape(-1, 1).to(dtype)


def unpack_int4(weight_packed: torch.Tensor, k: int) -> torch.Tensor:
    """quantization.py:113-121: interleave the low/high nibbles minus 8 into int8 [N, K]."""
    n = weight_packed.shape[0]
    out = torch.empty((n, k), dtype=torch.int8, device=weight_packed.device)
    even = out[:, 0::2].shape[1]
    odd = out[:, 1::2].shape[1]
    out[:, 0::2] = (weight_packed[:, :even] & 0x0F).to(torch.int8) - 8
    out[:, 1::2] = ((weight_packed[:, :odd] >> 4) & 0x0F).to(torch.int8) - 8
    return out


def dequant_int4(weight_packed, scale, k: int, group_size=None, dtype=torch.float32):
    """quantization.py:122 with the group-wise extension: scale[n, k // group_size]."""
    q = unpack_int4(weight_packed, k)
    s = scale.reshape(scale.shape[0], -1)
    if group_size is not None and group_size < k and s.shape[1] > 1:
        s = s.repeat_interleave(group_size, dim=1)[:, :k]
    return q.to(dtype) * s.to(dtype)


def forward(x: torch.Tensor, w_deq: torch.Tensor, bias=None) -> torch.Tensor:
    """quantization.py:129-141: F.linear(x, W.to(x.dtype), bias.to(x.dtype))."""
    if w_deq.dtype != x.dtype:
        w_deq = w_deq.to(x.dtype)
    if bias is not None and bias.dtype != x.dtype:
        bias = bias.to(x.dtype)
    return F.linear(x, w_deq, bias)


def forward_int8(x, weight_q, scale, bias=None):
    return forward(x, dequant_int8(weight_q, scale, x.dtype), bias)


def forward_int4(x, weight_packed, scale, k, group_size=None, bias=None):
    return forward(x, dequant_int4(weight_packed, scale, k, group_size, x.dtype), bias)
