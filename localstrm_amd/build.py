"""Build liblsq.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

Usage: python -m localstrm_amd.build [--verbose]

Each .hip source under csrc/ is compiled to an object in parallel, then linked into
localstrm_amd/liblsq.so. Always rebuilds: this is the "does it build" check.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_PATH = os.path.join(PKG_DIR, "liblsq.so")
ARCH = "gfx950"

# Packed-fp32 VALU ops are disabled for every HIP translation unit; -O3 would otherwise
# emit them from plain float code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: install ROCm or set HIPCC")


def sources() -> list[str]:
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        ln for ln in proc.stdout.splitlines() if "packed-fp32-ops" not in ln and ln.strip()
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out:
        print(out, flush=True)


def build(verbose: bool = False) -> str:
    hipcc = _hipcc()
    srcs = sources()
    with tempfile.TemporaryDirectory(prefix="lsq_build_") as tmp:
        objs = [os.path.join(tmp, os.path.basename(s) + ".o") for s in srcs]
        jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
        with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
            futs = [
                ex.submit(_run, [hipcc, *HIP_FLAGS, "-c", s, "-o", o], verbose)
                for s, o in zip(srcs, objs)
            ]
            for f in futs:
                f.result()
        tmp_lib = LIB_PATH + ".tmp"
        _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp_lib], verbose)
        os.replace(tmp_lib, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="--verbose" in sys.argv)
    print(path)
