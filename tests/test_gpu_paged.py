"""GPU parity of the paged attention decode kernel (paged_attention_decode,
src/kernels/paged_attention.py:33-173) against the oracle (float64 attention on the same
T-valued, dequantized keys and values), to the 1e-2 relative bar; plus the reference's
own ground truth (gather + SDPA in torch) on one case."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from localstrm_amd import paged_attention_decode
from oracle import quant_oracle as qo

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TDT = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}


def _case(seed, b, h, hkv, d, bs, seqs, int8, dt, spare=5):
    rng = np.random.default_rng(seed)
    nblk = max(-(-max(seqs) // bs), 1)
    nb = b * nblk + spare
    bt = rng.permutation(nb)[: b * nblk].reshape(b, nblk).astype(np.int64)
    if int8:
        kp = rng.integers(-128, 128, size=(nb, bs, hkv, d)).astype(np.int8)
        vp = rng.integers(-128, 128, size=(nb, bs, hkv, d)).astype(np.int8)
        ks = qo.round_f16(rng.uniform(0.002, 0.03, size=(nb, bs, hkv)).astype(np.float32))
        vs = qo.round_f16(rng.uniform(0.002, 0.03, size=(nb, bs, hkv)).astype(np.float32))
    else:
        kp = qo.round_to(rng.standard_normal((nb, bs, hkv, d)).astype(np.float32), dt)
        vp = qo.round_to(rng.standard_normal((nb, bs, hkv, d)).astype(np.float32), dt)
        ks = vs = None
    q = qo.round_to(rng.standard_normal((b, h, d)).astype(np.float32), dt)
    return q, kp, vp, ks, vs, bt, np.array(seqs, dtype=np.int64)


def _run(q, kp, vp, ks, vs, bt, seqs, bs, dt, mapping="contiguous", mask=None, max_sl=None,
         scale_dtype=torch.float16):
    t = TDT[dt]
    kv_t = torch.int8 if kp.dtype == np.int8 else t
    args = dict(
        query=torch.from_numpy(q).to(t).unsqueeze(2).to(DEV),
        k_cache_pool=torch.from_numpy(kp).to(kv_t).to(DEV),
        v_cache_pool=torch.from_numpy(vp).to(kv_t).to(DEV),
        block_tables=torch.from_numpy(bt).to(DEV), seq_lens=torch.from_numpy(seqs).to(DEV),
        block_size=bs, head_mapping=mapping, max_sl=max_sl,
        attn_mask=None if mask is None else torch.from_numpy(mask).to(DEV),
    )
    if ks is not None:
        args["k_scales"] = torch.from_numpy(ks).to(scale_dtype).unsqueeze(-1).to(DEV)
        args["v_scales"] = torch.from_numpy(vs).to(scale_dtype).unsqueeze(-1).to(DEV)
    out = paged_attention_decode(**args)
    torch.cuda.synchronize()
    return out[:, :, 0, :].float().cpu().numpy()


CASES = [
    # (b, h, hkv, d, bs, seqs, int8, dt, mapping)
    (4, 14, 2, 64, 16, [1, 17, 300, 1000], True, "f16", "contiguous"),
    (3, 28, 4, 128, 16, [256, 257, 2048], True, "bf16", "contiguous"),
    (2, 4, 4, 64, 16, [5, 513], False, "f16", "contiguous"),
    (3, 8, 2, 64, 32, [100, 64, 700], True, "f16", "interleaved"),
    (2, 16, 1, 128, 8, [33, 260], False, "bf16", "contiguous"),
    (2, 6, 2, 64, 16, [40, 9], False, "f32", "contiguous"),
]


# kernels: "default" (an INT8 cache with fp16 / bf16 queries: the wave-wise kernel, 4 waves
# at these sizes; a T cache: the block-wide MFMA kernel; fp32: the VALU kernel), "waves8"
# (the wave-wise kernel with 8 waves and 512-token chunks, LSQ_PAGED_WAVES=8), "block"
# (LSQ_PAGED_KERNEL=mfma: the block-wide MFMA kernel for an INT8 cache too), "valu" (the
# VALU kernel throughout)
KERNEL_ENV = {"default": None, "waves8": None, "block": "mfma", "valu": "valu"}


def _kernel(monkeypatch, kernel):
    if KERNEL_ENV[kernel]:
        monkeypatch.setenv("LSQ_PAGED_KERNEL", KERNEL_ENV[kernel])
    if kernel == "waves8":
        monkeypatch.setenv("LSQ_PAGED_WAVES", "8")


@pytest.mark.parametrize("kernel", ["default", "waves8", "block", "valu"])
@pytest.mark.parametrize("b,h,hkv,d,bs,seqs,int8,dt,mapping", CASES)
def test_paged_attention_matches_oracle(monkeypatch, kernel, b, h, hkv, d, bs, seqs, int8, dt, mapping):
    _kernel(monkeypatch, kernel)
    print(f"paged {kernel} B={b} H={h} Hkv={hkv} D={d} BS={bs} seqs={seqs} int8={int8} {dt} {mapping}", flush=True)
    q, kp, vp, ks, vs, bt, sl = _case(b + h + d, b, h, hkv, d, bs, seqs, int8, dt)
    got = _run(q, kp, vp, ks, vs, bt, sl, bs, dt, mapping)
    ref = qo.paged_attention(q, kp, vp, bt, sl, bs, dt, ks, vs, mapping)
    err = qo.rel_err(got, ref)
    print(f"  rel_err={err:.2e}", flush=True)
    assert err <= 1e-2


@pytest.mark.parametrize("kernel", ["default", "waves8", "block"])
@pytest.mark.parametrize("chunks", ["2", "3", "8"])
@pytest.mark.parametrize("b,h,hkv,d,bs,seqs,int8,dt,mapping", [c for c in CASES if c[7] != "f32"])
def test_paged_attention_multi_chunk_splits(monkeypatch, kernel, chunks, b, h, hkv, d, bs, seqs, int8, dt, mapping):
    # workgroups that loop over several 256-token chunks (online softmax across chunks,
    # next chunk's loads in flight), forced for every MFMA case; a split count that does not
    # divide the chunks leaves a short last split, and 8 chunks puts whole sequences in one
    if kernel in ("block", "waves8") and not int8:
        pytest.skip("a T cache runs the block-wide kernel")
    _kernel(monkeypatch, kernel)
    print(f"paged {kernel} chunks={chunks} B={b} H={h} Hkv={hkv} D={d} seqs={seqs} int8={int8} {dt} {mapping}",
          flush=True)
    monkeypatch.setenv("LSQ_PAGED_CHUNKS", chunks)
    q, kp, vp, ks, vs, bt, sl = _case(b + h + d + 1, b, h, hkv, d, bs, seqs, int8, dt)
    got = _run(q, kp, vp, ks, vs, bt, sl, bs, dt, mapping)
    ref = qo.paged_attention(q, kp, vp, bt, sl, bs, dt, ks, vs, mapping)
    err = qo.rel_err(got, ref)
    print(f"  rel_err={err:.2e}", flush=True)
    assert err <= 1e-2


def test_paged_attention_multi_chunk_mask(monkeypatch):
    # the engine's mask with two chunks per workgroup: a sequence whose second chunk is
    # fully masked, and one masked from the start of a chunk
    monkeypatch.setenv("LSQ_PAGED_CHUNKS", "2")
    b, h, hkv, d, bs = 3, 14, 2, 64, 16
    seqs = [300, 256, 1100]
    q, kp, vp, ks, vs, bt, sl = _case(12, b, h, hkv, d, bs, seqs, True, "bf16")
    max_sl = max(seqs)
    m = (np.arange(max_sl)[None, :] < sl[:, None]).reshape(b, 1, 1, max_sl)
    mask = np.repeat(m, hkv, axis=0)
    got = _run(q, kp, vp, ks, vs, bt, sl, bs, "bf16", mask=mask, max_sl=max_sl)
    ref = qo.paged_attention(q, kp, vp, bt, sl, bs, "bf16", ks, vs, "contiguous")
    assert qo.rel_err(got, ref) <= 1e-2
    plain = _run(q, kp, vp, ks, vs, bt, sl, bs, "bf16")
    assert np.array_equal(got, plain)


def test_paged_attention_engine_mask_and_reference_ground_truth():
    # the engine passes a repeat_interleave'd [B * Hkv, 1, 1, max_sl] mask
    # (model_runner.py:138-143); and the reference's ground truth (gather, dequantize,
    # SDPA) on the GPU with torch
    b, h, hkv, d, bs = 3, 14, 2, 64, 16
    seqs = [70, 5, 200]
    q, kp, vp, ks, vs, bt, sl = _case(11, b, h, hkv, d, bs, seqs, True, "f16")
    max_sl = max(seqs)
    m = (np.arange(max_sl)[None, :] < sl[:, None]).reshape(b, 1, 1, max_sl)
    mask = np.repeat(m, hkv, axis=0)
    got = _run(q, kp, vp, ks, vs, bt, sl, bs, "f16", mask=mask, max_sl=max_sl)
    plain = _run(q, kp, vp, ks, vs, bt, sl, bs, "f16")
    assert np.array_equal(got, plain)
    kt = torch.from_numpy(kp).to(DEV)
    vt = torch.from_numpy(vp).to(DEV)
    kst = torch.from_numpy(ks).half().to(DEV)
    vst = torch.from_numpy(vs).half().to(DEV)
    g = h // hkv
    for bb in range(b):
        n = seqs[bb]
        tok = torch.arange(n, device=DEV)
        blk = torch.from_numpy(bt[bb]).to(DEV)[tok // bs]
        off = tok % bs
        k = kt[blk, off].half() * kst[blk, off][..., None]
        v = vt[blk, off].half() * vst[blk, off][..., None]
        qq = torch.from_numpy(q[bb]).half().to(DEV).view(hkv, g, 1, d)
        kk = k.permute(1, 0, 2).float().contiguous().view(hkv, 1, n, d).expand(hkv, g, n, d)
        vv = v.permute(1, 0, 2).float().contiguous().view(hkv, 1, n, d).expand(hkv, g, n, d)
        ref = F.scaled_dot_product_attention(qq.float(), kk, vv).half().float().view(h, d).cpu().numpy()
        assert qo.rel_err(got[bb], ref) <= 1e-2


def test_paged_attention_validation():
    q = torch.zeros(2, 4, 1, 64, device=DEV, dtype=torch.float16)
    kp = torch.zeros(4, 16, 2, 64, device=DEV, dtype=torch.int8)
    bt = torch.zeros(2, 2, dtype=torch.int64, device=DEV)
    sl = torch.ones(2, dtype=torch.int64, device=DEV)
    with pytest.raises(ValueError, match="requires both k_scales and v_scales"):
        paged_attention_decode(q, kp, kp, bt, sl)
    with pytest.raises(ValueError, match="Unsupported head_mapping"):
        paged_attention_decode(q, kp, kp, bt, sl, head_mapping="strided")
    with pytest.raises(ValueError, match="must be divisible"):
        paged_attention_decode(torch.zeros(2, 3, 1, 64, device=DEV), kp, kp, bt, sl)
    with pytest.raises(NotImplementedError):
        paged_attention_decode(torch.zeros(2, 4, 2, 64, device=DEV, dtype=torch.float16),
                               kp.half(), kp.half(), bt, sl)
    with pytest.raises(ValueError, match="do not cover"):  # 2 blocks of 16 < 40 tokens
        paged_attention_decode(q, kp.half(), kp.half(), bt, sl, max_sl=40)


@pytest.mark.parametrize("kernel", ["default", "block", "valu"])
def test_paged_attention_out_of_range_block_ids(monkeypatch, kernel):
    """Block-table entries past each sequence's length may hold anything: -1 pads, ids at
    or above the pool size, huge values. They are read (the table is read up to max_sl)
    but must neither fault nor change the result; an in-range negative entry counts from
    the end of the pool. Inside a sequence, an out-of-range entry masks its tokens."""
    _kernel(monkeypatch, kernel)
    b, h, hkv, d, bs = 3, 14, 2, 64, 16
    seqs = [40, 300, 513]
    q, kp, vp, ks, vs, bt, sl = _case(77, b, h, hkv, d, bs, seqs, True, "f16")
    nb = kp.shape[0]
    ref = qo.paged_attention(q, kp, vp, bt, sl, bs, "f16", ks, vs, "contiguous")
    bad = bt.copy()
    junk = [-1, nb, nb + 7, 2 ** 40, -(2 ** 40)]
    for i, n in enumerate(seqs):
        used = -(-n // bs)
        for j in range(used, bad.shape[1]):
            bad[i, j] = junk[(i + j) % len(junk)]
    got = _run(q, kp, vp, ks, vs, bad, sl, bs, "f16", max_sl=int(max(seqs)))
    assert qo.rel_err(got, ref) <= 1e-2
    # an in-range negative entry names the same block as its positive form
    neg = bt.copy()
    neg[1, 2] -= nb
    got_neg = _run(q, kp, vp, ks, vs, neg, sl, bs, "f16")
    assert qo.rel_err(got_neg, ref) <= 1e-2
    # an out-of-range entry inside sequence 2: its 16 tokens are masked
    hole = bt.copy()
    hole[2, 3] = nb + 1
    mask = np.zeros((b, int(max(seqs))), dtype=np.uint8)
    for i, n in enumerate(seqs):
        mask[i, :n] = 1
    mask[2, 3 * bs:4 * bs] = 0
    ref_hole = qo.paged_attention(q, kp, vp, bt, sl, bs, "f16", ks, vs, "contiguous", mask=mask)
    got_hole = _run(q, kp, vp, ks, vs, hole, sl, bs, "f16")
    assert qo.rel_err(got_hole, ref_hole) <= 1e-2


def test_paged_attention_rejects_short_seq_lens():
    q, kp, vp, ks, vs, bt, sl = _case(5, 3, 4, 2, 64, 16, [20, 30, 40], True, "f16")
    with pytest.raises(ValueError, match="seq_lens"):
        _run(q, kp, vp, ks, vs, bt, sl[:2], 16, "f16", max_sl=40)


@pytest.mark.parametrize("bs", [1, 5, 24, 64, 80, 256])
def test_paged_attention_block_sizes(bs):
    """The wave-wise kernel's block / slot arithmetic (a multiply-high below 64 tokens per
    block, one wrap from 64 on) on block sizes that are and are not powers of two, with
    sequences that end inside a block and cross chunk boundaries; INT8 cache, fp16 queries."""
    seqs = [3, bs + 1, 257, 700]
    print(f"paged block size {bs} seqs={seqs}", flush=True)
    q, kp, vp, ks, vs, bt, sl = _case(bs + 3, 4, 14, 2, 64, bs, seqs, True, "f16")
    got = _run(q, kp, vp, ks, vs, bt, sl, bs, "f16")
    ref = qo.paged_attention(q, kp, vp, bt, sl, bs, "f16", ks, vs, "contiguous")
    assert qo.rel_err(got, ref) <= 1e-2


@pytest.mark.parametrize("kernel", ["default", "block"])
@pytest.mark.parametrize("d,dt", [(64, "f16"), (128, "f16"), (64, "bf16")])
def test_paged_attention_fp32_scales(monkeypatch, kernel, d, dt):
    """fp32 per-token scales (the same values as the fp16 ones of the other tests): the
    dequantization through fp32 instead of the packed fp16 product for fp16 queries."""
    _kernel(monkeypatch, kernel)
    seqs = [100, 600, 2048]
    q, kp, vp, ks, vs, bt, sl = _case(d + 9, 3, 8, 2, d, 16, seqs, True, dt)
    got = _run(q, kp, vp, ks, vs, bt, sl, 16, dt, scale_dtype=torch.float32)
    ref = qo.paged_attention(q, kp, vp, bt, sl, 16, dt, ks, vs, "contiguous")
    assert qo.rel_err(got, ref) <= 1e-2
    half = _run(q, kp, vp, ks, vs, bt, sl, 16, dt)
    assert qo.rel_err(got, half) <= 1e-2


def test_paged_attention_eight_wave_choice(monkeypatch):
    """Batch 64 x 2048 tokens, 2 KV heads: 256 workgroups of 8 waves and 1024 tokens, no
    combine (the default there); the 4-wave kernel with its split and combine forced for
    comparison; both against the oracle. Ragged lengths inside the chunks."""
    b, h, hkv, d, bs = 64, 14, 2, 64, 16
    seqs = [2048 - 23 * i for i in range(b)]
    q, kp, vp, ks, vs, bt, sl = _case(77, b, h, hkv, d, bs, seqs, True, "f16")
    got8 = _run(q, kp, vp, ks, vs, bt, sl, bs, "f16")
    monkeypatch.setenv("LSQ_PAGED_WAVES", "4")
    got4 = _run(q, kp, vp, ks, vs, bt, sl, bs, "f16")
    ref = qo.paged_attention(q, kp, vp, bt, sl, bs, "f16", ks, vs, "contiguous")
    e8, e4 = qo.rel_err(got8, ref), qo.rel_err(got4, ref)
    print(f"  8 waves {e8:.2e} 4 waves {e4:.2e}", flush=True)
    assert e8 <= 1e-2 and e4 <= 1e-2


def test_paged_attention_wave_kernel_matches_block_kernel(monkeypatch):
    """The two MFMA kernels on the benchmark's attention shapes (14 / 2 heads, head 64,
    INT8 cache with fp16 scales, blocks of 16), 2048 tokens: within the contract of each
    other and of the oracle."""
    seqs = [2048, 1999, 1024, 17]
    q, kp, vp, ks, vs, bt, sl = _case(41, 4, 14, 2, 64, 16, seqs, True, "f16")
    wave = _run(q, kp, vp, ks, vs, bt, sl, 16, "f16")
    monkeypatch.setenv("LSQ_PAGED_KERNEL", "mfma")
    block = _run(q, kp, vp, ks, vs, bt, sl, 16, "f16")
    ref = qo.paged_attention(q, kp, vp, bt, sl, 16, "f16", ks, vs, "contiguous")
    print(f"  wave {qo.rel_err(wave, ref):.2e} block {qo.rel_err(block, ref):.2e} "
          f"wave-block {qo.rel_err(wave, block.astype(np.float64)):.2e}", flush=True)
    assert qo.rel_err(wave, ref) <= 1e-2 and qo.rel_err(block, ref) <= 1e-2
