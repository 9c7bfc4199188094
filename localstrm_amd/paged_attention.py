"""Paged attention for the decode step, on liblsq's gfx950 kernel.

Drop-in for paged_attention_decode (src/kernels/paged_attention.py:33-173): same
arguments, shapes and ValueErrors. The reference gathers every cached block into
contiguous tensors, dequantizes an INT8 cache (keys.to(T) * k_scales), expands the GQA
heads and calls F.scaled_dot_product_attention; here lsq_paged_attention_decode reads the
pool through the block table directly (no gather, no dequantized copy). Decode only: one
query token per sequence (query [B, H, 1, D]), head_dim 64 or 128, at most 16 query heads
per KV head; on a CPU tensor it raises (no CPU path). Block-table entries: a negative one
counts from the end of the pool (Python indexing, as the reference's gather does); one
outside [-num_blocks, num_blocks) masks its token (it contributes nothing) where the
reference's gather would raise IndexError, which a kernel cannot do without a host sync.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib

def paged_attention_decode(
    query: torch.Tensor,
    k_cache_pool: torch.Tensor,
    v_cache_pool: torch.Tensor,
    block_tables: torch.Tensor,
    seq_lens: torch.Tensor,
    block_size: int = 16,
    k_scales: Optional[torch.Tensor] = None,
    v_scales: Optional[torch.Tensor] = None,
    sub_tables: Optional[torch.Tensor] = None,
    max_sl: Optional[int] = None,
    attn_mask: Optional[torch.Tensor] = None,
    head_mapping: str = "contiguous",
) -> torch.Tensor:
    """Attention of one new token per sequence over its paged KV cache
    (paged_attention.py:33-173). Returns [batch, num_heads, 1, head_dim] in query's dtype."""
    # argument checks in the reference's order and wording (:66-95)
    if query.ndim != 4:
        raise ValueError(f"Expected query to be a 4D tensor [batch_size, num_heads, seq_len, head_dim], got shape {list(query.shape)}")
    if k_cache_pool.ndim != 4 or v_cache_pool.ndim != 4:
        raise ValueError("k_cache_pool and v_cache_pool must be 4D tensors [blocks, block_size, kv_heads, head_dim]")
    if k_cache_pool.shape[2] != v_cache_pool.shape[2]:
        raise ValueError(f"Mismatch in KV heads: k has {k_cache_pool.shape[2]}, v has {v_cache_pool.shape[2]}")
    if k_cache_pool.shape[3] != query.shape[3] or v_cache_pool.shape[3] != query.shape[3]:
        raise ValueError(f"head_dim mismatch: query={query.shape[3]}, k={k_cache_pool.shape[3]}, v={v_cache_pool.shape[3]}")
    batch_size, num_heads, q_len, head_dim = query.shape
    num_kv_heads = k_cache_pool.shape[2]
    if num_heads < num_kv_heads:
        raise ValueError(f"num_heads ({num_heads}) cannot be less than num_kv_heads ({num_kv_heads})")
    if num_heads % num_kv_heads != 0:
        raise ValueError(
            f"num_heads ({num_heads}) must be divisible by num_kv_heads ({num_kv_heads}) for GQA/MHA."
        )
    if head_mapping not in ("contiguous", "interleaved"):
        raise ValueError(
            f"Unsupported head_mapping: {head_mapping!r}. Supported options are 'contiguous' and 'interleaved'."
        )
    if k_cache_pool.dtype == torch.int8 and (k_scales is None or v_scales is None):
        raise ValueError("INT8 quantized KV cache requires both k_scales and v_scales for dequantization.")

    # what this kernel covers
    if query.device.type != "cuda":
        raise RuntimeError("paged_attention_decode: the kernel runs on the GPU only; got a CPU query")
    if q_len != 1:
        raise NotImplementedError(f"paged_attention_decode: one query token per sequence (got {q_len})")
    if head_dim not in (64, 128):
        raise NotImplementedError(f"paged_attention_decode: head_dim 64 or 128 (got {head_dim})")
    if num_heads // num_kv_heads > 16:
        raise NotImplementedError("paged_attention_decode: at most 16 query heads per KV head")
    if k_cache_pool.shape[0] * k_cache_pool.shape[1] * num_kv_heads >= 2 ** 31:
        raise NotImplementedError("paged_attention_decode: pools of 2^31 or more rows")
    int8_kv = k_cache_pool.dtype == torch.int8
    if not int8_kv and query.dtype == torch.float32 and head_dim == 128:
        raise NotImplementedError("paged_attention_decode: an fp32 KV cache with head_dim 128")
    if not int8_kv and (k_cache_pool.dtype != query.dtype or v_cache_pool.dtype != query.dtype):
        raise ValueError("paged_attention_decode: a non-INT8 KV cache must have the query's dtype")

    if seq_lens.numel() < batch_size:
        raise ValueError(f"paged_attention_decode: seq_lens has {seq_lens.numel()} entries for "
                         f"{batch_size} sequences")
    if max_sl is None:
        max_sl = int(seq_lens.max().item())  # the reference's host read (:97-98)
    tables = sub_tables if sub_tables is not None else block_tables
    if tables.ndim != 2 or tables.shape[0] < batch_size or tables.shape[1] * block_size < max_sl:
        # the reference gathers ceil(max_sl / block_size) table entries per sequence
        raise ValueError(
            f"paged_attention_decode: block tables of shape {list(tables.shape)} do not cover "
            f"{batch_size} sequences of max_sl={max_sl} tokens in blocks of {block_size}")
    if tables.dtype != torch.int64:
        tables = tables.to(torch.int64)
    if tables.stride(-1) != 1:
        tables = tables.contiguous()
    lens = seq_lens if seq_lens.dtype == torch.int64 else seq_lens.to(torch.int64)
    lens = lens.contiguous()
    q = query.reshape(batch_size, num_heads, head_dim)
    if not q.is_contiguous():
        q = q.contiguous()
    kp, vp = k_cache_pool.contiguous(), v_cache_pool.contiguous()
    ks = k_scales.contiguous() if int8_kv else None
    vs = v_scales.contiguous() if int8_kv else None
    mask, mask_ld, mask_rows = None, 0, 1
    if attn_mask is not None:
        rows = attn_mask.shape[0]
        m2 = attn_mask.reshape(rows, -1)[:, :max_sl]
        mask = m2.to(torch.uint8).contiguous() if m2.dtype != torch.uint8 else m2.contiguous()
        mask_ld = mask.shape[1]
        mask_rows = rows // batch_size if batch_size else 1
    out = torch.empty((batch_size, num_heads, 1, head_dim), dtype=query.dtype, device=query.device)
    lib = _lib.load()
    wbytes = lib.lsq_paged_attention_workspace_bytes(batch_size, num_heads, head_dim, max_sl)
    ws = torch.empty(max(wbytes // 4, 1), dtype=torch.float32, device=query.device) if wbytes else None
    with torch.cuda.device(query.device):
        rc = lib.lsq_paged_attention_decode(
            q.data_ptr(), kp.data_ptr(), vp.data_ptr(),
            _lib.I8 if int8_kv else _lib.dtype_code(query.dtype), _lib.ptr(ks), _lib.ptr(vs),
            _lib.dtype_code(ks.dtype) if int8_kv else 0, tables.data_ptr(), tables.stride(0),
            lens.data_ptr(), _lib.ptr(mask), mask_ld, mask_rows, out.data_ptr(),
            _lib.dtype_code(query.dtype), batch_size, num_heads, num_kv_heads, head_dim, block_size,
            k_cache_pool.shape[0], max_sl, 0 if head_mapping == "contiguous" else 1, _lib.ptr(ws), wbytes,
            _lib.stream_handle(query.device))
    _lib.check(rc, "lsq_paged_attention_decode")
    return out
