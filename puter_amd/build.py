"""Build the gfx950 HIP library puter_amd/libputer_hip.so from puter_amd/csrc,
and the C++ host library puter_amd/libputer_host.so from puter_amd/host.

Each .hip file is compiled ahead of time for gfx950 only (no JIT, no CUDA
headers) into an object under puter_amd/_build/, then linked into one shared
library whose exported symbols are exactly the extern "C" entry points of
include/puter_hip.h.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIBRARY = os.path.join(HERE, "libputer_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["runtime.hip", "cast.hip", "norm.hip", "rope.hip", "gated.hip", "page.hip",
           "attention.hip", "prefill.hip", "decode.hip", "flash.hip", "matmul.hip", "quant.hip", "probe.hip"]

HIPFLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-fvisibility=hidden",
    # no implicit FMA contraction: every float expression rounds per operation
    # as the reference's Go code does on amd64 (explicit fmaf stays fused)
    "-ffp-contract=off",
    # packed-FP32 VALU ops stay disabled (known-bad on this pool)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result", "-Wno-unused-variable",
]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, src.replace(".hip", ".o"))
    cmd = [HIPCC, *HIPFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    if r.stderr.strip():
        # hipcc's host pass warns about the unknown packed-fp32 feature: harmless
        lines = [l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l and l.strip()]
        if lines:
            sys.stderr.write("\n".join(lines) + "\n")
    return obj


HOST_SOURCES = ["host/backend.cpp", "host/kernels.cpp"]
HOST_LIBRARY = os.path.join(HERE, "libputer_host.so")
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra", "-Wno-unused-parameter",
              "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(HERE, "host")]


def build_host(verbose: bool = False) -> str:
    """The C++ host side (puter_amd/host: the device.Backend methods, hooks,
    workspace slots and kernel registry over the C ABI) into
    puter_amd/libputer_host.so, linked against libputer_hip.so."""
    tmp = HOST_LIBRARY + ".tmp"
    cmd = ["g++", *HOST_FLAGS, *[os.path.join(HERE, s) for s in HOST_SOURCES], "-o", tmp,
           "-L" + HERE, "-lputer_hip", "-Wl,-rpath,$ORIGIN", "-Wl,-rpath-link,/opt/rocm/lib"]
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"g++ failed for the host library:\n{r.stdout}\n{r.stderr}")
    if r.stderr.strip():
        sys.stderr.write(r.stderr)
    os.replace(tmp, HOST_LIBRARY)
    return HOST_LIBRARY


def build(jobs: int = 8, verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    sources = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIBRARY + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIBRARY)
    build_host(verbose)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
