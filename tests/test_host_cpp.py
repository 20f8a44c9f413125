"""The C++ host side (puter_amd/host: the device.Backend methods, hooks,
workspace slots and kernel registry over the C ABI) through its own C++ test
programs under tests/cpp: the registry's semantics and the Go contract's error
behaviour on the CPU, parity against the CPU oracle on the GPU.  build() builds
the programs; they are built here only when missing."""
import importlib.util
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _program(name):
    spec = importlib.util.spec_from_file_location("cpp_tests_build", os.path.join(ROOT, "tests", "cpp", "build.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    path = mod.program(name)
    if not os.path.exists(path):
        from puter_amd import build as hip_build
        if not os.path.exists(hip_build.HOST_LIBRARY):
            hip_build.build_host()
        import oracle
        if not os.path.exists(oracle.LIBRARY):
            oracle.build()
        mod.build()
    return path


def _run(name, timeout):
    r = subprocess.run([_program(name)], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-2000:]
    assert ", 0 failed" in r.stdout


def test_host_registry_and_error_behaviour():
    _run("host_registry_test", 120)


@pytest.mark.gpu
def test_host_parity_against_the_oracle():
    _run("host_parity_test", 300)
