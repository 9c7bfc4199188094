"""GPU checks of lsq_w8a8_linear_noalloc, the allocation-free W8A8 entry point: its output
must equal lsq_w8a8_linear's (same kernels, caller workspace) bit for bit, on two calls in
a row with the second one smaller, over the decode (fused and unfused activation
quantization) and GEMM paths, and one case against the oracle (qo.w8a8_linear, the CPU
restatement of src/kernels/quantization.py:404-447). The fixed scratch array keeps the
previous call's contents, so a smaller second call with K not a multiple of 128 reads
K-padding columns that the previous call filled with data: they must be rewritten.
"""

import numpy as np
import pytest
import torch

from localstrm_amd import _lib
from oracle import quant_oracle as qo

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
TDT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}
SCRATCH = 8 * 1024 * 1024  # LSQ_NOALLOC_SCRATCH_BYTES
E_SCRATCH = -7


def _say(msg):
    print(msg, flush=True)


def _pad_k(k):
    return -(-k // 128) * 128


def _layer(n, k, dt, seed, bias=True):
    """Tiled int8 weights, fp32 scales and an optional bias on the GPU."""
    g = torch.Generator().manual_seed(seed)
    wq = torch.randint(-128, 128, (n, k), generator=g, dtype=torch.int8)
    sw = torch.rand(n, generator=g) * 0.02 + 1e-3
    b = torch.randn(n, generator=g).to(TDT[dt]) if bias else None
    lib = _lib.load()
    wt = wq.t().contiguous().to(DEV)
    tiled = torch.empty(lib.lsq_w8a8_tiled_bytes(n, k), dtype=torch.int8, device=DEV)
    _lib.check(lib.lsq_w8a8_retile(wt.data_ptr(), tiled.data_ptr(), n, k, _lib.stream_handle(DEV)), "retile")
    return wq, sw, b, tiled, sw.to(DEV), None if b is None else b.to(DEV)


def _x(m, k, dt, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(m, k, generator=g) * 2).to(TDT[dt])
    if m >= 2:
        x[1] = 0  # a zero row: the scale takes its clamp bound
    return x


def _call(noalloc, x, tiled, swd, bd, n):
    m, k = x.shape
    lib = _lib.load()
    y = torch.full((m, n), float("nan"), dtype=x.dtype, device=DEV)
    args = (x.data_ptr(), x.stride(0), tiled.data_ptr(), swd.data_ptr(), _lib.dtype_code(swd.dtype),
            _lib.ptr(bd), _lib.dtype_code(bd.dtype) if bd is not None else 0, y.data_ptr(), n,
            _lib.dtype_code(x.dtype), m, n, k)
    if noalloc:
        rc = lib.lsq_w8a8_linear_noalloc(*args, _lib.stream_handle(DEV))
        _lib.check(rc, "lsq_w8a8_linear_noalloc")
    else:
        xq = torch.empty((m, _pad_k(k)), dtype=torch.int8, device=DEV)
        sx = torch.empty(m, dtype=torch.float32, device=DEV)
        rc = lib.lsq_w8a8_linear(*args, xq.data_ptr(), sx.data_ptr(), _lib.stream_handle(DEV))
        _lib.check(rc, "lsq_w8a8_linear")
    torch.cuda.synchronize()
    return y


# (M, N, K) pairs: the first call, then a smaller second one
PAIRS = [
    ((1024, 1040, 4096), (300, 1040, 1000)),   # GEMM then GEMM with K padding to rewrite
    ((64, 4864, 4096), (8, 4864, 4096)),       # decode on the quantized scratch, both calls
    ((2046, 272, 4096), (1, 4864, 896)),       # the largest M that fits, then fused decode
    ((48, 896, 4864), (33, 272, 1000)),        # decode, then decode with K padding
]


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_workspace_entry_point(first, second, dt):
    for i, (m, n, k) in enumerate((first, second)):
        _say(f"noalloc {dt} call {i + 1}: M={m} N={n} K={k}")
        _, _, _, tiled, swd, bd = _layer(n, k, dt, seed=m + n + k, bias=(i == 0))
        x = _x(m, k, dt, seed=7 * m + k).to(DEV)
        got = _call(True, x, tiled, swd, bd, n)
        ref = _call(False, x, tiled, swd, bd, n)
        assert torch.equal(got.view(torch.uint8 if dt != "f32" else torch.int32).view(-1).cpu(),
                           ref.view(torch.uint8 if dt != "f32" else torch.int32).view(-1).cpu()), \
            f"call {i + 1}: outputs differ from lsq_w8a8_linear"


def test_noalloc_matches_oracle_and_repeats():
    """Against the oracle bit for bit, twice on the same inputs (the second call reuses the
    scratch as the first left it)."""
    m, n, k = 300, 1040, 1000
    wq, sw, b, tiled, swd, bd = _layer(n, k, "bf16", seed=3)
    x = _x(m, k, "bf16", seed=4)
    ref = qo.w8a8_linear(x.float().numpy(), wq.numpy(), sw.numpy(), b.float().numpy(), "bf16")
    for _ in range(2):
        got = _call(True, x.to(DEV), tiled, swd, bd, n).float().cpu().numpy()
        assert np.array_equal(got.view(np.uint32), np.asarray(ref, dtype=np.float32).view(np.uint32))


def test_noalloc_rejects_sizes_beyond_the_scratch():
    """One row past the limit is refused with LSQ_E_SCRATCH before any HIP call (NULL
    pointers: nothing is touched); the limit itself is exercised by the pairs above."""
    lib = _lib.load()
    k = 4096
    need = lambda m: -(-m * k // 256) * 256 + 4 * m
    assert need(2046) <= SCRATCH < need(2047)
    assert lib.lsq_w8a8_linear_noalloc(None, k, None, None, 0, None, 0, None, 64, 2, 2047, 64, k,
                                       None) == E_SCRATCH
    msg = lib.lsq_status_string(E_SCRATCH).decode()
    assert "scratch" in msg
