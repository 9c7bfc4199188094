"""CPU oracle for the weight-only quantized linear layer. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import this
module, and only as the checker. The product (localstrm_amd) never imports it.

A numpy restatement of LocalStrm's src/kernels/quantization.py, written from the
reference's behaviour (no code copied):

  quantize_int8       quantization.py:72-78   per-row symmetric INT8
  quantize_int4       quantization.py:80-94   per-row symmetric INT4 + nibble pack;
                      group_size < K is the group-wise extension (same steps per group,
                      quantized against the stored, dtype-rounded scale)
  pack_int4           quantization.py:86-91   byte j = (q[2j]+8) | (q[2j+1]+8) << 4
  unpack_int4         quantization.py:113-121 the int8 `unpacked` tensor
  dequant_int8        quantization.py:106-108 round_T(T(q) * round_T(s))
  dequant_int4        quantization.py:109-122 same closed form, s[n, k // group_size]
  linear              quantization.py:129-141 F.linear(x, W_T, bias_T), evaluated in
                      float64 then rounded once to T
  act_scale_i8        quantization.py:412-413 per-token activation scale of
                      Int8GEMMLinear, in the GPU's evaluation order (below)
  act_quant_i8        quantization.py:411-414 per-token int8 activations
  w8a8_linear         quantization.py:404-447 Int8GEMMLinear's native path: int32 GEMM,
                      fp32 rescale, bias, one rounding to T (bit-exact target)
  silu_mul            modeling_qwen2.py:48 F.silu(gate) * up on T-valued layer outputs
  paged_attention     paged_attention.py:33-173 decode attention over a paged (INT8) KV
                      cache: gather by block table, keys.to(T) * scales, GQA mapping,
                      SDPA (float64 here), one rounding to T

How each part is pinned (tests/test_oracle.py):
  * round_bf16 / round_f16 against torch's dtype casts on every bf16 boundary case,
    plus hand-computed ties;
  * quantizers against hand-computed known answers, round-half-even tie cases built
    so that w / s is exactly .5, and torch's own op sequence on random data;
  * pack/unpack against a hand-written byte vector, all 256 byte values, round trip;
  * dequant exhaustively over all q values x random scales against torch casts;
  * linear against float64 closed forms (one-hot x, identity W) and torch's CPU GEMM;
  * group-wise dequant reduces to the per-channel form when group_size = K;
  * act_quant_i8 / w8a8_linear against hand-computed answers (scale 1 rows, round-half-
    even ties, zero rows per dtype), torch's CPU ops for the quantization given the scale,
    torch._int_mm plus torch's elementwise epilogue for the GEMM and rescale; the scale's
    device evaluation order (product with fp32 1/127) against torch on the GPU over every
    bf16 / fp16 value and random fp32 (tests/test_gpu_w8a8.py);
  * silu_mul against torch's CPU F.silu and product, and closed forms (silu(0) = 0,
    large |g|);
  * paged_attention against torch's CPU scaled_dot_product_attention on the gathered,
    dequantized tensors (the reference's own ground truth, paged_attention.py:23-30,
    :196-225), closed forms (equal keys -> mean of the values; one dominant key -> its
    value) and the interleaved / contiguous head mappings.
"""

from __future__ import annotations

import numpy as np

F32, F16, BF16 = "f32", "f16", "bf16"


# ----------------------------------------------------------------------------- rounding


def round_bf16(a) -> np.ndarray:
    """fp32 -> nearest bf16 (ties to even), returned as fp32. NaN stays NaN.

    IEEE-754 round-to-nearest-even on the upper 16 bits: add 0x7FFF plus the lowest kept
    bit, then truncate. Infinities and overflow to infinity fall out of the same carry.
    """
    f = np.ascontiguousarray(a, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(f)
    out[nan] = np.float32("nan")
    return out


def round_f16(a) -> np.ndarray:
    """fp32 -> nearest fp16 (numpy's correctly rounded conversion), back to fp32."""
    return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(a, dt: str) -> np.ndarray:
    if dt == F32:
        return np.asarray(a, dtype=np.float32)
    if dt == F16:
        return round_f16(a)
    if dt == BF16:
        return round_bf16(a)
    raise ValueError(dt)


def bf16_bits(a) -> np.ndarray:
    """uint16 bit patterns of already-bf16-representable fp32 values."""
    return (np.ascontiguousarray(round_bf16(a)).view(np.uint32) >> 16).astype(np.uint16)


def from_bf16_bits(b) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------------------- quantizers


def _row_scale(w32: np.ndarray, qmax: float) -> np.ndarray:
    """clamp(max|w| / qmax, min=1e-8) in fp32, [N, 1] (quantization.py:74-75, :82-83)."""
    max_val = np.max(np.abs(w32), axis=-1, keepdims=True).astype(np.float32)
    return np.maximum(max_val / np.float32(qmax), np.float32(1e-8)).astype(np.float32)


def quantize_int8(w) -> tuple[np.ndarray, np.ndarray]:
    """(q int8 [N,K], scale fp32 [N,1]) per quantization.py:72-78; np.rint is half-to-even
    like torch.round."""
    w32 = np.asarray(w, dtype=np.float32)
    s = _row_scale(w32, 127.0)
    q = np.clip(np.rint(w32 / s), -128, 127).astype(np.int8)
    return q, s


def quantize_int4(w, group_size: int | None = None, scale_dt: str = F32):
    """(packed uint8 [N, ceil(K/2)], scale [N, G] as fp32 values of dtype scale_dt).

    group_size None (or >= K): quantization.py:80-94 exactly, fp32 scale.
    group_size < K: per group of columns, scale = clamp(max|w|/7, 1e-8) rounded to
    scale_dt, q = clamp(round(w / scale_stored), -8, 7).
    """
    w32 = np.asarray(w, dtype=np.float32)
    n, k = w32.shape
    if group_size is None or group_size >= k:
        s = _row_scale(w32, 7.0)
        q = np.clip(np.rint(w32 / s), -8, 7).astype(np.int8)
        return pack_int4(q), s
    g = -(-k // group_size)
    pad = g * group_size - k
    wa = np.abs(w32)
    if pad:
        wa = np.pad(wa, ((0, 0), (0, pad)))
    max_val = wa.reshape(n, g, group_size).max(axis=-1).astype(np.float32)
    s = round_to(np.maximum(max_val / np.float32(7.0), np.float32(1e-8)), scale_dt)
    s_full = np.repeat(s, group_size, axis=1)[:, :k]
    q = np.clip(np.rint(w32 / s_full), -8, 7).astype(np.int8)
    return pack_int4(q), s


def pack_int4(q) -> np.ndarray:
    """int8 q in [-8,7] [N,K] -> uint8 [N, ceil(K/2)], low nibble = even column,
    odd K pads the last high nibble with 0 (quantization.py:86-91)."""
    q = np.asarray(q)
    n, k = q.shape
    u = (q.astype(np.int16) + 8).astype(np.uint8)
    if k % 2:
        u = np.concatenate([u, np.zeros((n, 1), np.uint8)], axis=1)
    return (u[:, 0::2] | (u[:, 1::2] << 4)).astype(np.uint8)


def unpack_int4(packed, k: int) -> np.ndarray:
    """uint8 [N, ceil(K/2)] -> int8 q [N, K] (quantization.py:113-121)."""
    p = np.asarray(packed, dtype=np.uint8)
    n = p.shape[0]
    out = np.empty((n, k), dtype=np.int8)
    out[:, 0::2] = ((p & 0x0F).astype(np.int16) - 8)[:, : (k + 1) // 2]
    out[:, 1::2] = ((p >> 4).astype(np.int16) - 8)[:, : k // 2]
    return out


# ----------------------------------------------------------------------------- dequant


def dequant_int8(q, scale, dt: str) -> np.ndarray:
    """round_T(T(q) * round_T(scale)) as fp32 values (quantization.py:106-108).
    T(q) is exact for |q| <= 128 in all three types; the fp32 product is exact for bf16
    and fp16 scales, and is the single fp32 rounding for T = fp32."""
    qf = np.asarray(q, dtype=np.float32)
    s = round_to(np.asarray(scale, dtype=np.float32).reshape(-1, 1), dt)
    return round_to(qf * s, dt)


def dequant_int4(packed, scale, k: int, group_size: int | None, dt: str) -> np.ndarray:
    """round_T(T(q) * round_T(scale[n, k // g])) (quantization.py:109-122 + groups)."""
    q = unpack_int4(packed, k).astype(np.float32)
    s = np.asarray(scale, dtype=np.float32)
    s = s.reshape(s.shape[0], -1)
    if group_size is None or group_size >= k or s.shape[1] == 1:
        s_full = np.broadcast_to(s[:, :1], q.shape)
    else:
        s_full = np.repeat(s, group_size, axis=1)[:, :k]
    return round_to(q * round_to(s_full, dt), dt)


# ----------------------------------------------------------------------------- linear


def linear(x, w_deq, bias=None, dt: str = BF16) -> np.ndarray:
    """y = round_T(x @ W^T + round_T(bias)) with the sum in float64 (quantization.py:141).

    x and w_deq hold the T-valued inputs as fp32/float64. The reference's own GEMM
    accumulates in fp32 in an unspecified order; float64 is the order-free target the
    1e-2 relative bound is measured against.
    """
    x64 = np.asarray(x, dtype=np.float64)
    acc = x64 @ np.asarray(w_deq, dtype=np.float64).T
    if bias is not None:
        acc = acc + round_to(np.asarray(bias, dtype=np.float32), dt).astype(np.float64)
    return round_to(acc.astype(np.float32), dt)


def linear_f64(x, w_deq, bias=None, dt: str = BF16) -> np.ndarray:
    """Same as linear() but without the final rounding (for error budgets)."""
    acc = np.asarray(x, dtype=np.float64) @ np.asarray(w_deq, dtype=np.float64).T
    if bias is not None:
        acc = acc + round_to(np.asarray(bias, dtype=np.float32), dt).astype(np.float64)
    return acc


def rel_err(a, b) -> float:
    """max|a - b| / max(max|b|, 1e-6), the reference's convention
    (tests/test_int8_multi_step.py:184-188)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b)) / max(float(np.max(np.abs(b))), 1e-6))


# ----------------------------------------------------------------------------- W8A8

INV127_F32 = np.float32(1.0) / np.float32(127.0)


def act_scale_i8(x, dt: str) -> np.ndarray:
    """Per-token scale of Int8GEMMLinear.forward (quantization.py:412-413) as fp32 [M, 1]:
    clamp(max|x| / 127.0, min=1e-8) in the activation type T.

    max|x| is exact in T. torch evaluates `tensor / 127.0` (a Python scalar) on the GPU as
    tensor * fp32(1/127) in fp32, then rounds to T; the reference only quantizes
    activations on the GPU (its CPU path is the dequantizing fallback), so that is the
    order restated here. The clamp bound is 1e-8 converted to T: bf16 1.0012e-8, fp16 0
    (below the smallest subnormal), fp32 1e-8. NaN propagates.
    """
    x32 = np.asarray(x, dtype=np.float32)
    mx = np.max(np.abs(x32), axis=-1, keepdims=True).astype(np.float32)
    s = round_to((mx * INV127_F32).astype(np.float32), dt)
    smin = round_to(np.float32(1e-8), dt)
    return np.where(s < smin, smin, s).astype(np.float32)


def act_quant_i8(x, dt: str) -> tuple[np.ndarray, np.ndarray]:
    """(x_q int8 [M, K], scale_x fp32 [M, 1]): clamp(round_half_even(fp32(x) / s),
    -128, 127) (quantization.py:414), fp32 division. A 0 / 0 (fp16 rows whose scale
    rounds to 0) gives NaN, which converts to 0; with a zero scale the row's outputs are
    0 * acc whatever x_q holds."""
    x32 = np.asarray(x, dtype=np.float32)
    s = act_scale_i8(x32, dt)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.rint(x32 / s)
    r = np.clip(r, -128, 127)
    r = np.where(np.isnan(r), 0, r)
    return r.astype(np.int8), s


def w8a8_linear(x, w_q, scale_w, bias=None, dt: str = BF16) -> np.ndarray:
    """Int8GEMMLinear's native output (quantization.py:404-447) as fp32 values of T.

    w_q int8 [N, K] (= weight_q_t transposed), scale_w [N] (scale_w_t), bias [N] as the
    fp32 values of its stored dtype or None. acc = x_q @ w_q^T is exact (int32 range; it
    is formed in float64, exact for these integer sums); then
    y = round_T(fp32(acc) * fp32(scale_x * scale_w) [+ bias]), every step one fp32
    rounding (:432-440, :446).
    """
    xq, sx = act_quant_i8(x, dt)
    acc = xq.astype(np.float64) @ np.asarray(w_q, dtype=np.float64).T
    if acc.size and np.abs(acc).max() >= 2.0 ** 31:
        raise OverflowError("int32 accumulator range exceeded")
    comb = (sx.reshape(-1, 1) * np.asarray(scale_w, dtype=np.float32).reshape(1, -1)).astype(np.float32)
    out = (acc.astype(np.float32) * comb).astype(np.float32)
    if bias is not None:
        out = (out + np.asarray(bias, dtype=np.float32).reshape(1, -1)).astype(np.float32)
    return round_to(out, dt)


# ----------------------------------------------------------------------------- SiLU.mul


def silu_mul(g, u, dt: str) -> np.ndarray:
    """round_T(round_T(silu(g)) * u) for T-valued g, u (fp32 arrays): F.silu evaluates
    g / (1 + exp(-g)) in fp32 and rounds to T, the product is one more fp32 product
    rounded to T (modeling_qwen2.py:48)."""
    g32 = np.asarray(g, dtype=np.float32)
    with np.errstate(over="ignore"):
        sg = round_to((g32 / (np.float32(1.0) + np.exp(-g32))).astype(np.float32), dt)
    return round_to((sg * np.asarray(u, dtype=np.float32)).astype(np.float32), dt)


# ----------------------------------------------------------------------------- paged attention


def paged_attention(q, k_pool, v_pool, block_tables, seq_lens, block_size, dt: str,
                    k_scales=None, v_scales=None, head_mapping: str = "contiguous",
                    mask=None, max_sl=None) -> np.ndarray:
    """Decode attention of paged_attention_decode (paged_attention.py:33-173) as fp32
    values of T, [B, H, D]. q [B, H, D] (T values); pools [NB, BS, Hkv, D] (int8 with
    scales [NB, BS, Hkv] as fp32 values of their dtype, or T values); block_tables
    [B, nblk]; token t of sequence b attends when t < max_sl and (mask[b or b*Hkv+kvh, t]
    if a mask [rows, max_sl] is given, else t < seq_lens[b]). Keys / values are
    round_T(k * s) for an INT8 cache; scores (q . k) / sqrt(D), softmax and the value
    sum in float64, then one rounding to T."""
    q = np.asarray(q, dtype=np.float64)
    b_, h_, d_ = q.shape
    hkv = k_pool.shape[2]
    g_ = h_ // hkv
    if max_sl is None:
        max_sl = int(np.max(seq_lens))
    out = np.zeros((b_, h_, d_), dtype=np.float64)
    for b in range(b_):
        ts = np.arange(max_sl)
        rows = (np.asarray(block_tables[b])[ts // block_size], ts % block_size)
        for kvh in range(hkv):
            k = np.asarray(k_pool[rows[0], rows[1], kvh, :], dtype=np.float32)
            v = np.asarray(v_pool[rows[0], rows[1], kvh, :], dtype=np.float32)
            if k_scales is not None:
                k = round_to(k * np.asarray(k_scales[rows[0], rows[1], kvh], np.float32)[:, None], dt)
                v = round_to(v * np.asarray(v_scales[rows[0], rows[1], kvh], np.float32)[:, None], dt)
            if mask is not None:
                mrow = b * hkv + kvh if mask.shape[0] == b_ * hkv and hkv > 1 else b
                valid = np.asarray(mask[mrow][:max_sl], dtype=bool)
            else:
                valid = ts < int(seq_lens[b])
            for g in range(g_):
                h = kvh * g_ + g if head_mapping == "contiguous" else g * hkv + kvh
                sc = (k.astype(np.float64) @ q[b, h]) / np.sqrt(d_)
                sc = np.where(valid, sc, -np.inf)
                with np.errstate(invalid="ignore"):
                    p = np.exp(sc - np.max(sc))
                    out[b, h] = (p @ v.astype(np.float64)) / np.sum(p)
    return round_to(out.astype(np.float32), dt)
