"""Build libunifur_nf4.so (gfx950) from unifur_amd/csrc with hipcc.

Each .hip source compiles to an object under unifur_amd/_build/ (in
parallel), then one shared library is linked in-tree next to this file, so
it travels with the repository snapshot.  No GPU is needed to build.

    python -m unifur_amd.build            # or: python unifur_amd/build.py
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libunifur_nf4.so")
PROBE_DIR = os.path.join(HERE, "bench_probe")
PROBE_LIB = os.path.join(PROBE_DIR, "libunifur_bench_probe.so")
ARCH = os.environ.get("UNIFUR_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (the host pass warns
# that it does not know the feature; that is harmless).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# -amdgpu-kernarg-preload-count: a kernel's leading scalar parameters are
# preloaded into SGPRs before a wave starts, so the prologue needs no load
# through the scalar cache for them (the code object keeps the loads as a
# fallback for firmware without preloading).  The striped GEMV and skinny
# kernels pass what their prologues read that way.
HIPCC_FLAGS += ["-mllvm", "-amdgpu-kernarg-preload-count=16"]

# hipBLASLt: the plain bf16 GEMM of the prefill path (nf4_blas.hip).
LINK_LIBS = ["-L/opt/rocm/lib", "-lhipblaslt", "-Wl,-rpath,/opt/rocm/lib"]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the HIP toolchain is required to build libunifur_nf4.so")
    return path


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def _link(objs, out: str, libs) -> None:
    tmp = out + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp, *libs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, out)


def build(verbose: bool = False) -> str:
    """libunifur_nf4.so (the product) and, beside it, the bench's streaming
    probes (bench_probe/libunifur_bench_probe.so: measurement kernels that are
    not part of the product's ABI)."""
    os.makedirs(BUILD, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    probe_src = os.path.join(PROBE_DIR, "stream_probe.hip")
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources) + 1)) as ex:
        objs = list(ex.map(_compile, sources + [probe_src]))
    _link(objs[:-1], LIB, LINK_LIBS)
    _link(objs[-1:], PROBE_LIB, [])
    if verbose:
        print(f"built {LIB} and {PROBE_LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
