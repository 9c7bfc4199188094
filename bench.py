"""Benchmark of the weight-only quantized linear layer on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-sweep] [--no-cpu]
python bench.py --calibrate-copy   # one 64 MiB device-to-device copy, for PMC calibration
python bench.py --case int4,14336,4096,2048 --steps 20   # one layer shape only

Headline workload (one JSON line, `value`): INT4 group-128 decode GEMV at the
Qwen2.5-7B MLP shape, W int4 [18944, 3584] (two nibbles per byte, bf16 scales
[18944, 28]), x bf16 [1, 3584] -> y bf16 [1, 18944]. A step is one forward of the layer.
`value` is algorithmic GB/s = (W + scales + x + y bytes) / time per step, with inputs
resident in HBM. The timed region is a HIP graph of K back-to-back launches bracketed by
events on the launch stream, replayed 7 times; every figure is the median replay.
Successive launches cycle through enough distinct weight copies (> 256 MB) that every
launch streams its weights from HBM rather than from the 256 MB Infinity Cache.

`floors` times, the same way in the same run, an empty kernel (the cost of one launch)
and a bare streaming read of the headline's bytes (lsq_probe_read): the time no kernel
that must stream those bytes in one launch can beat on this device.

`roofline.traffic` is the HBM bytes one launch of the headline kernel moves, as measured
by rocprofv3 FETCH_SIZE + WRITE_SIZE (each scaled by what the counter reads for a 64 MiB
copy, see --calibrate-copy) and recorded in profiles/decode_int4_g128_m1_18944x3584.txt.

`sweep` reports the other shapes of the same metric (INT8 per-channel decode M in
{1,8,32,64} at 18944x3584, INT4 group-128 decode M in {16,64}, INT4 group-128 prefill M in
{256,2048,8192} at 14336x4096 in TFLOP/s, the single INT8 layer 4864x896 at M=1 (bf16 and
fp32 activations), INT4 group-128 decode M=1 at 18944x3584 with fp32 activations, INT4
decode M in {1,16} at the transposed 3584x18944 shape, W8A8 layers, the batch-32 decode
step through the 168 INT4 projections of a Qwen2.5-0.5B-architecture stack, its MLPs, and
paged attention). `cpu_baseline` times the reference's CPU path (dequantize, then
F.linear, on the host cores) on the headline shape; `cpu_baselines_more` on INT8 M=1 and
on INT4 prefill M=2048.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import platform
import statistics
import sys
import time

import torch
import torch.nn.functional as F

METRIC = "W-only INT4/INT8 GEMM: decode GB/s (% HBM peak); prefill TFLOP/s (% MFMA)"
HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, vendor spec
MFMA_BF16_PEAK_TF = 2500.0  # MI355X dense bf16, vendor spec
MFMA_INT8_PEAK_TOPS = 5000.0  # MI355X dense int8, vendor spec
MALL_BYTES = 256 << 20


# ----------------------------------------------------------------------------- inputs


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()[:16]


def make_int8(n: int, k: int, m: int, x_dtype=torch.bfloat16, seed: int = 0,
              s_lo: float = 0.001, s_hi: float = 0.02):
    """INT8 per-channel inputs on the CPU, draw order W -> scale -> x:
    W uniform int in [-127, 127], fp32 scale U[s_lo, s_hi] [N, 1], x ~ N(0, 1)."""
    g = _gen(seed)
    w = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
    s = torch.rand((n, 1), generator=g) * (s_hi - s_lo) + s_lo
    x = torch.randn((m, k), generator=g).to(x_dtype)
    return w, s, x


def make_int4(n: int, k: int, m: int, group: int = 128, x_dtype=torch.bfloat16, seed: int = 0,
              s_lo: float = 0.001, s_hi: float = 0.05):
    """INT4 group-wise inputs on the CPU, draw order W -> scale -> x:
    q uniform int in [-8, 7] packed two per byte (low nibble = even column), bf16 scales
    U[s_lo, s_hi] [N, K/group], x ~ N(0, 1)."""
    from localstrm_amd.quantization import pack_int4

    g = _gen(seed)
    q = torch.randint(-8, 8, (n, k), generator=g, dtype=torch.int8)
    s = (torch.rand((n, -(-k // group)), generator=g) * (s_hi - s_lo) + s_lo).to(torch.bfloat16)
    x = torch.randn((m, k), generator=g).to(x_dtype)
    return pack_int4(q), s, x


def decode_bytes(kind: str, n: int, k: int, m: int, group: int = 128, xb: int = 2) -> int:
    """Algorithmic bytes per call: W + scales + x + y (xb bytes per activation / output:
    2 for bf16, 4 for fp32). W8A8 counts the layer's own inputs and outputs the same way as
    INT8 (its int8 activation copy is an intermediate)."""
    if kind in ("int8", "w8a8"):
        return n * k + n * 4 + m * k * xb + m * n * xb
    return n * k // 2 + n * (-(-k // group)) * 2 + m * k * xb + m * n * xb


# ----------------------------------------------------------------------------- timing


def _layers(kind, w, s, group, copies, device):
    from localstrm_amd import Int8GEMMLinear, QuantizedLinear

    out = []
    for i in range(copies):
        wc = w.to(device)
        if i:
            wc = wc.clone()
        if kind == "w8a8":
            out.append(Int8GEMMLinear.from_quantized(wc, s.to(device), dtype=torch.bfloat16))
        elif kind == "int8":
            out.append(QuantizedLinear.from_quantized(wc, s.to(device), quant_type="int8"))
        else:
            out.append(QuantizedLinear.from_quantized(wc, s.to(device), quant_type="int4",
                                                      in_features=w.shape[1] * 2, group_size=group))
    return out


REPLAYS = 7  # timed replays of each graph; figures are their median


def graph_time(step, steps: int, warmup: int, replays: int = REPLAYS):
    """(median, min, max) ms per step: `step(i)` launches step i's work; `steps` of them are
    captured in one HIP graph on a side stream, replayed once untimed, then `replays` times,
    each bracketed by events recorded on that stream (the stream the kernels run on)."""
    stream = torch.cuda.Stream()
    with torch.no_grad():
        for i in range(max(warmup, 1)):
            step(i)
        torch.cuda.synchronize()
        stream.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                for i in range(steps):
                    step(i)
        graph.replay()  # warm replay
        torch.cuda.synchronize()
        per = []
        for _ in range(replays):
            start = torch.cuda.Event(enable_timing=True)
            stop = torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(stream):
                start.record(stream)
                graph.replay()
                stop.record(stream)
            stop.synchronize()
            per.append(start.elapsed_time(stop) / steps)
        del graph
    return statistics.median(per), min(per), max(per)


def time_layers(layers, x, steps: int, warmup: int):
    """graph_time of one forward per step, cycling the weight copies."""
    return graph_time(lambda i: layers[i % len(layers)](x), steps, warmup)


PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                       "decode_int4_g128_m1_18944x3584.txt")


def measured_traffic():
    """HBM bytes per launch of the headline kernel from its committed rocprofv3 summary
    (line 'traffic_bytes_per_launch: N'), or None."""
    try:
        with open(PROFILE) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except (OSError, ValueError):
        pass
    return None


def calibrate_copy(device) -> None:
    """A plain device-to-device copy of 64 MiB, 5 times: run under rocprofv3 --pmc to get
    what FETCH_SIZE / WRITE_SIZE read for 64 MiB moved."""
    a = torch.empty(64 << 20, dtype=torch.uint8, device=device)
    b = torch.empty_like(a)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(f"copied {a.numel()} bytes x 5", flush=True)


def copies_for(nbytes: int) -> int:
    return max(2, min(32, -(-2 * MALL_BYTES // max(nbytes, 1)) + 1))


READ_SHAPES = ((256, 1024), (256, 512), (512, 512), (512, 1024), (1024, 256))


def bench_floors(nbytes: int, steps: int, warmup: int, device) -> dict:
    """Floors for one launch of the headline, timed the same way in the same run: an empty
    kernel (what one graph node costs with no work) and a bare streaming read of `nbytes`
    (lsq_probe_read: the same bytes, nothing computed), cycling enough buffers to exceed
    the Infinity Cache; the read floor is the fastest of READ_SHAPES (grid, threads)."""
    from localstrm_amd import _lib

    lib = _lib.load()
    copies = copies_for(nbytes)
    bufs = [torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=device) for _ in range(copies)]
    sink = torch.empty(max(g for g, _ in READ_SHAPES) * 64, dtype=torch.float32, device=device)

    def empty(i):
        _lib.check(lib.lsq_probe_empty(_lib.stream_handle(device)), "lsq_probe_empty")

    launch = graph_time(empty, steps, warmup)[0]
    per_shape = {}
    for grid, block in READ_SHAPES:
        def read(i, grid=grid, block=block):
            _lib.check(lib.lsq_probe_read(bufs[i % copies].data_ptr(), nbytes, sink.data_ptr(), grid, block,
                                          _lib.stream_handle(device)), "lsq_probe_read")
        per_shape[f"{grid}x{block}"] = graph_time(read, steps, warmup)[0] * 1e3
    best = min(per_shape, key=per_shape.get)
    del bufs
    torch.cuda.empty_cache()
    return {
        "launch_us": launch * 1e3, "bare_read_bytes": nbytes, "bare_read_us": per_shape[best],
        "bare_read_shape": best, "bare_read_GB_s": nbytes / (per_shape[best] * 1e-6) / 1e9,
        "bare_read_us_by_shape": per_shape, "buffers": copies,
    }


def bench_decode(kind: str, n: int, k: int, m: int, steps: int, warmup: int, device, group=128,
                 copies=None, x_dtype=torch.bfloat16):
    """One layer shape timed over `steps` back-to-back launches; by default the launches
    rotate over enough weight copies to exceed the 256 MB Infinity Cache (every launch reads
    HBM); copies=1 times the hot-cache case (one copy, resident in the Infinity Cache).
    x_dtype: the activation (and output) type."""
    if kind in ("int8", "w8a8"):
        w, s, x = make_int8(n, k, m, x_dtype=x_dtype)
    else:
        w, s, x = make_int4(n, k, m, group, x_dtype=x_dtype)
    wbytes = w.numel()
    copies = copies or copies_for(wbytes)
    layers = _layers(kind, w, s, group, copies, device)
    ms, lo, hi = time_layers(layers, x.to(device), steps, warmup)
    nbytes = decode_bytes(kind, n, k, m, group, xb=4 if x_dtype == torch.float32 else 2)
    flops = 2.0 * m * n * k
    del layers
    torch.cuda.empty_cache()
    peak = MFMA_INT8_PEAK_TOPS if kind == "w8a8" else MFMA_BF16_PEAK_TF
    return {
        "kind": kind, "M": m, "N": n, "K": k, "group": None if kind in ("int8", "w8a8") else group,
        "x_dtype": str(x_dtype).replace("torch.", ""), "us_per_call": ms * 1e3, "us_range": [lo * 1e3, hi * 1e3], "GB_s": nbytes / (ms * 1e-3) / 1e9,
        "TFLOP_s": flops / (ms * 1e-3) / 1e12, "bytes": nbytes, "weight_copies": copies,
        "frac_hbm": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "frac_mfma": flops / (ms * 1e-3) / 1e12 / peak,
    }


# Qwen2.5-0.5B attention and MLP projections (name, out_features N, in_features K, bias):
# modeling_qwen2.py q/k/v carry a bias, o/gate/up/down do not.
QWEN05_LINEARS = [("q", 896, 896, True), ("k", 128, 896, True), ("v", 128, 896, True),
                  ("o", 896, 896, False), ("gate", 4864, 896, False), ("up", 4864, 896, False),
                  ("down", 896, 4864, False)]


def stack_bytes(m: int, group: int = 128) -> int:
    """Algorithmic bytes of one decode step through the 7 projections of one layer."""
    tot = 0
    for _, n, k, bias in QWEN05_LINEARS:
        tot += decode_bytes("int4", n, k, m, group) + (2 * n if bias else 0)
    return tot


def bench_stack(steps: int, warmup: int, device, m: int = 32, n_layers: int = 24, group: int = 128,
                fused: bool = False):
    """One decode step of a random-init Qwen2.5-0.5B-architecture stack: the 168 INT4
    group-128 forwards (24 layers x q, k, v, o, gate, up, down) in layer order, batch m,
    bf16 activations. Every layer holds its own copy of the weights, and steps alternate
    between enough copies of the whole stack to exceed the 256 MB Infinity Cache.
    fused=True runs q/k/v and gate/up as one launch each (fuse_linears): 96 launches."""
    from localstrm_amd import QuantizedLinear, fuse_linears

    protos = []
    for _, n, k, bias in QWEN05_LINEARS:
        p, s, _ = make_int4(n, k, 1, group, seed=n * 7 + k)
        b = torch.randn(n, generator=_gen(n + k)).to(torch.bfloat16) if bias else None
        protos.append((p.to(device), s.to(device), None if b is None else b.to(device), k))
    per_step = n_layers * stack_bytes(m, group)
    copies = max(2, -(-2 * MALL_BYTES // per_step))
    def one_layer():
        lins = [QuantizedLinear.from_quantized(p.clone(), s, bias=b, quant_type="int4", in_features=k,
                                               group_size=group) for (p, s, b, k) in protos]
        if not fused:
            return lins
        return [fuse_linears(lins[0:3]), lins[3], fuse_linears(lins[4:6]), lins[6]]

    stacks = [[lin for _ in range(n_layers) for lin in one_layer()] for _ in range(copies)]
    xs = {k: torch.randn(m, k, generator=_gen(k)).to(torch.bfloat16).to(device) for k in (896, 4864)}

    def run(i):
        for lin in stacks[i % copies]:
            lin(xs[lin.in_features])

    ms, lo, hi = graph_time(run, steps, warmup)
    del stacks
    torch.cuda.empty_cache()
    flops = 2.0 * m * n_layers * sum(n * k for _, n, k, _ in QWEN05_LINEARS)
    return {
        "kind": "int4 stack" + (" fused" if fused else ""), "M": m, "layers": n_layers,
        "forwards": n_layers * len(QWEN05_LINEARS), "launches": n_layers * (4 if fused else 7),
        "group": group, "us_per_call": ms * 1e3, "us_range": [lo * 1e3, hi * 1e3],
        "GB_s": per_step / (ms * 1e-3) / 1e9,
        "TFLOP_s": flops / (ms * 1e-3) / 1e12, "bytes": per_step, "stack_copies": copies,
        "frac_hbm": per_step / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "frac_mfma": flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TF,
    }


def bench_mlp(steps: int, warmup: int, device, m: int = 32, n_layers: int = 24, group: int = 128,
              fused: bool = False):
    """The MLP blocks of one decode step of the same stack: down(silu(gate(x)) * up(x))
    (modeling_qwen2.py:46-48) for 24 layers, INT4 group-128, batch m. Unfused: gate, up,
    down launches plus torch's silu and mul (5 launches per layer). fused=True:
    fuse_linears([gate, up], act="silu_mul") (one launch with the SiLU.mul epilogue) and
    down (2 launches per layer)."""
    from localstrm_amd import QuantizedLinear, fuse_linears

    shapes = [l for l in QWEN05_LINEARS if l[0] in ("gate", "up", "down")]
    protos = []
    for _, n, k, _ in shapes:
        p, s, _ = make_int4(n, k, 1, group, seed=n * 7 + k)
        protos.append((p.to(device), s.to(device), k))
    per_step = n_layers * sum(n * k // 2 + n * (-(-k // group)) * 2 + m * k * 2 + m * n * 2
                              for _, n, k, _ in shapes)
    copies = max(2, -(-2 * MALL_BYTES // per_step))

    def one_layer():
        g, u, d = [QuantizedLinear.from_quantized(p.clone(), s, quant_type="int4", in_features=k,
                                                  group_size=group) for (p, s, k) in protos]
        if fused:
            gu = fuse_linears([g, u], act="silu_mul")
            return lambda x: d(gu(x))
        return lambda x: d(F.silu(g(x)) * u(x))

    stacks = [[one_layer() for _ in range(n_layers)] for _ in range(copies)]
    x = torch.randn(m, 896, generator=_gen(5)).to(torch.bfloat16).to(device)
    def run(i):
        for mlp in stacks[i % copies]:
            mlp(x)

    ms, lo, hi = graph_time(run, steps, warmup)
    del stacks
    torch.cuda.empty_cache()
    return {
        "kind": "int4 mlp" + (" fused silu_mul" if fused else ""), "M": m, "layers": n_layers,
        "launches": n_layers * (2 if fused else 5), "group": group, "us_per_call": ms * 1e3,
        "us_range": [lo * 1e3, hi * 1e3], "GB_s": per_step / (ms * 1e-3) / 1e9, "bytes": per_step, "stack_copies": copies,
        "frac_hbm": per_step / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
    }


def bench_paged(steps: int, warmup: int, device, b: int = 32, h: int = 14, hkv: int = 2, d: int = 64,
                seq: int = 2048, bs: int = 16, n_layers: int = 24, int8: bool = True):
    """Paged attention of one decode step over n_layers layers (each with its own KV pool),
    batch b at context seq: Qwen2.5-0.5B attention shapes (14 query / 2 KV heads, head 64),
    INT8 KV with fp16 per-token scales (the reference's kv_cache_dtype 'int8'), scattered
    blocks of 16 tokens. Bytes = K + V + scales + q + out."""
    from localstrm_amd import paged_attention_decode

    g = _gen(3)
    nblk = -(-seq // bs)
    nb = b * nblk
    pools = []
    for _ in range(n_layers):
        if int8:
            kp = torch.randint(-128, 128, (nb, bs, hkv, d), generator=g, dtype=torch.int8).to(device)
            vp = torch.randint(-128, 128, (nb, bs, hkv, d), generator=g, dtype=torch.int8).to(device)
            ks = (torch.rand(nb, bs, hkv, 1, generator=g) * 0.02 + 0.002).half().to(device)
            vs = (torch.rand(nb, bs, hkv, 1, generator=g) * 0.02 + 0.002).half().to(device)
        else:
            kp = torch.randn(nb, bs, hkv, d, generator=g).half().to(device)
            vp = torch.randn(nb, bs, hkv, d, generator=g).half().to(device)
            ks = vs = None
        pools.append((kp, vp, ks, vs))
    bt = torch.randperm(nb, generator=g).reshape(b, nblk).to(device)
    sl = torch.full((b,), seq, dtype=torch.int64, device=device)
    q = torch.randn(b, h, 1, d, generator=g).half().to(device)
    esz = 1 if int8 else 2
    per_step = n_layers * (2 * b * seq * hkv * d * esz + (2 * b * seq * hkv * 2 if int8 else 0)
                           + 2 * b * h * d * 2)
    def run(i):
        for kp, vp, ks, vs in pools:
            paged_attention_decode(q, kp, vp, bt, sl, bs, ks, vs, max_sl=seq)

    ms, lo, hi = graph_time(run, steps, warmup)
    del pools
    torch.cuda.empty_cache()
    return {
        "kind": "paged attention" + (" int8 kv" if int8 else " fp16 kv"), "B": b, "H": h, "Hkv": hkv,
        "D": d, "seq": seq, "layers": n_layers, "us_per_call": ms * 1e3,
        "us_range": [lo * 1e3, hi * 1e3],
        "us_per_layer": ms * 1e3 / n_layers, "GB_s": per_step / (ms * 1e-3) / 1e9,
        "bytes": per_step, "frac_hbm": per_step / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
    }


# ----------------------------------------------------------------------------- CPU baseline


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(kind: str, n: int, k: int, m: int, budget_s: float = 10.0, min_runs: int = 3,
                 group: int = 128):
    """The reference's CPU path (quantization.py:104-141: dequantize in the activation dtype,
    then F.linear) on the host cores, on the same seeded inputs as the GPU case, repeated for
    about `budget_s` seconds (at least `min_runs` timed runs after one warm-up). Decode
    shapes report GB/s of the same algorithmic bytes as the GPU; M >= 256 reports TFLOP/s."""
    from oracle import torch_ref

    torch.set_num_threads(os.cpu_count() or 1)
    if kind == "int8":
        w, s, x = make_int8(n, k, m)
        fwd = lambda: torch_ref.forward_int8(x, w, s)
    else:
        w, s, x = make_int4(n, k, m, group)
        fwd = lambda: torch_ref.forward_int4(x, w, s, k, group)
    times = []
    with torch.no_grad():
        fwd()
        t_end = time.perf_counter() + budget_s
        while (time.perf_counter() < t_end or len(times) < min_runs) and len(times) < 2000:
            t0 = time.perf_counter()
            fwd()
            times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    prefill = m >= 256
    value = 2.0 * m * n * k / med / 1e12 if prefill else decode_bytes(kind, n, k, m, group) / med / 1e9
    what = f"{kind}" + ("" if kind == "int8" else f" group-{group}") + (" prefill" if prefill else " decode")
    return {
        "value": value, "unit": "TFLOP/s" if prefill else "GB/s", "ms_per_call": med * 1e3,
        "cores": torch.get_num_threads(), "kind": "port",
        "sample": (f"{what} {n}x{k} M={m}, bf16: torch CPU dequantize + F.linear on the same "
                   f"seeded inputs, median of {len(times)} runs ({med * 1e3:.1f} ms/call), cpu "
                   f"'{_cpu_model()}', os.cpu_count()={os.cpu_count()}"),
    }


# ----------------------------------------------------------------------------- main


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--calibrate-copy", action="store_true")
    ap.add_argument("--case", default=None,
                    help="kind,N,K,M (kind int8 | int4 | w8a8; e.g. int4,14336,4096,2048), or "
                         "'stack' for the batch-32 "
                         "decode step through the Qwen2.5-0.5B-architecture stack: time only "
                         "that case and print its line (used for the rocprofv3 summaries in "
                         "profiles/)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this layer's multi-GPU sharding is not built "
              "(run with --gpus 1)", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.calibrate_copy:
        calibrate_copy(device)
        return 0

    if args.case in ("stack", "stack-fused"):
        print(json.dumps(bench_stack(max(2, args.steps), args.warmup, device,
                                     fused=args.case == "stack-fused")), flush=True)
        return 0
    if args.case and args.case.startswith("paged"):
        # paged[,B,seq[,fp16]]: Qwen2.5-0.5B attention shapes, 24 layers
        parts = args.case.split(",")
        bsz = int(parts[1]) if len(parts) > 1 else 32
        seq = int(parts[2]) if len(parts) > 2 else 2048
        int8 = not (len(parts) > 3 and parts[3] == "fp16")
        print(json.dumps(bench_paged(max(2, args.steps), args.warmup, device, b=bsz, seq=seq,
                                     int8=int8)), flush=True)
        return 0
    if args.case in ("mlp", "mlp-fused"):
        print(json.dumps(bench_mlp(max(2, args.steps), args.warmup, device,
                                   fused=args.case == "mlp-fused")), flush=True)
        return 0
    if args.case:
        # kind,N,K,M[,f32]: one layer shape; a fifth field f32 times fp32 activations
        parts = args.case.split(",")
        kind, n, k, m = parts[:4]
        xdt = torch.float32 if len(parts) > 4 and parts[4] == "f32" else torch.bfloat16
        r = bench_decode(kind, int(n), int(k), int(m), args.steps, args.warmup, device, x_dtype=xdt)
        print(json.dumps(r), flush=True)
        return 0

    N, K, M, G = 18944, 3584, 1, 128
    head = bench_decode("int4", N, K, M, args.steps, args.warmup, device, group=G)
    hot = bench_decode("int4", N, K, M, args.steps, args.warmup, device, group=G, copies=1)
    floors = bench_floors(decode_bytes("int4", N, K, M, G), args.steps, args.warmup, device)
    sweep = []
    if not args.no_sweep:
        for m in (1, 8, 32, 64):
            sweep.append(bench_decode("int8", N, K, m, args.steps, args.warmup, device))
        for m in (16, 64):
            sweep.append(bench_decode("int4", N, K, m, args.steps, args.warmup, device))
        for m in (256, 2048, 8192):
            sweep.append(bench_decode("int4", 14336, 4096, m, max(10, args.steps // 20),
                                      max(2, args.warmup // 4), device))
        sweep.append(bench_decode("int8", 4864, 896, 1, args.steps, args.warmup, device))
        # fp32 activations (the reference's CPU type, allowed for the single INT8 layer): that
        # layer (4864x896) and the headline shape
        sweep.append(bench_decode("int8", 4864, 896, 1, args.steps, args.warmup, device, x_dtype=torch.float32))
        sweep.append(bench_decode("int4", N, K, 1, args.steps, args.warmup, device, group=G, x_dtype=torch.float32))
        # the transposed (down-projection) shape, whose activations exceed LDS from 4 tokens
        for m in (1, 16):
            sweep.append(bench_decode("int4", K, N, m, args.steps, args.warmup, device))
        for m in (1, 64):
            sweep.append(bench_decode("w8a8", N, K, m, args.steps, args.warmup, device))
        # W8A8 on the down-projection shape (split-K GEMM with the module's workspace)
        sweep.append(bench_decode("w8a8", K, N, 64, args.steps, args.warmup, device))
        sweep.append(bench_decode("w8a8", 14336, 4096, 2048, max(10, args.steps // 20),
                                  max(2, args.warmup // 4), device))
        sweep.append(bench_stack(max(5, args.steps // 20), 2, device))
        sweep.append(bench_stack(max(5, args.steps // 20), 2, device, fused=True))
        sweep.append(bench_mlp(max(5, args.steps // 20), 2, device))
        sweep.append(bench_mlp(max(5, args.steps // 20), 2, device, fused=True))
        sweep.append(bench_paged(max(5, args.steps // 20), 2, device))
    cpu, cpu_more = None, []
    if not args.no_cpu:
        cpu = cpu_baseline("int4", N, K, M, group=G)
        cpu_more = [cpu_baseline("int8", N, K, M), cpu_baseline("int4", 14336, 4096, 2048, group=G)]

    ms = head["us_per_call"] / 1e3
    line = {
        "metric": METRIC,
        "value": round(head["GB_s"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded torch.Generator(0) inputs of the stated shapes",
        "config": {
            "workload": ("int4 group-128 decode GEMV, W int4 18944x3584 (packed 2 per byte, bf16 "
                         "scales [18944, 28]), x bf16 [1, 3584]"),
            "M": M, "N": N, "K": K, "group": G, "weight_copies": head["weight_copies"],
            "timing": (f"median of {REPLAYS} replays of a HIP graph of `steps` launches, events "
                       "on the launch stream"),
            "us_range": head["us_range"],
        },
        "roofline": {
            "bound": "hbm", "achieved": round(head["GB_s"], 2), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(head["frac_hbm"], 4), "traffic": measured_traffic(),
        },
        "floors": dict(floors, kernel_vs_bare_read=head["us_per_call"] / floors["bare_read_us"]),
        "hot_cache": {
            "what": ("the headline with one weight copy resident in the 256 MB Infinity Cache "
                     "(not HBM-bound; value above rotates copies so every launch reads HBM)"),
            "us_per_call": hot["us_per_call"], "GB_s": round(hot["GB_s"], 2),
        },
        "cpu_baseline": cpu,
        "cpu_baselines_more": cpu_more,
        "sweep": sweep,
        "host": platform.node(),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
