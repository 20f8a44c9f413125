"""Build recipe for the C++ host tests (test infrastructure).

Compiles tests/cpp/*_test.cpp with g++ into tests/cpp/bin/, linked against the
host library puter_amd/libputer_host.so (and libputer_hip.so); the GPU parity
program also links the CPU oracle oracle/liboracle.so as its checker.  The
binaries find those libraries through an rpath relative to themselves, so the
tree can move (the GPU box runs them from its own copy).
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
BIN = os.path.join(HERE, "bin")
PROGRAMS = {"host_registry_test": False, "host_parity_test": True}   # name -> links the oracle

FLAGS = ["-O2", "-std=c++17", "-Wall", "-Wextra", "-Wno-unused-parameter",
         "-I" + os.path.join(ROOT, "include"), "-I" + os.path.join(ROOT, "puter_amd", "host"),
         "-I" + os.path.join(ROOT, "oracle"), "-I" + HERE]


def program(name: str) -> str:
    return os.path.join(BIN, name)


def build(verbose: bool = False) -> list:
    """Build every test program (the host and oracle libraries must be built)."""
    os.makedirs(BIN, exist_ok=True)
    out = []
    for name, oracle in PROGRAMS.items():
        libs = ["-pthread", "-L" + os.path.join(ROOT, "puter_amd"), "-lputer_host", "-lputer_hip",
                "-Wl,-rpath,$ORIGIN/../../../puter_amd", "-Wl,-rpath-link,/opt/rocm/lib"]
        if oracle:
            libs += ["-L" + os.path.join(ROOT, "oracle"), "-loracle", "-Wl,-rpath,$ORIGIN/../../../oracle",
                     "-fopenmp"]
        target = program(name)
        cmd = ["g++", *FLAGS, os.path.join(HERE, name + ".cpp"), "-o", target + ".tmp", *libs]
        if verbose:
            print(" ".join(cmd), flush=True)
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"g++ failed for {name}:\n{r.stdout}\n{r.stderr}")
        os.replace(target + ".tmp", target)
        out.append(target)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
