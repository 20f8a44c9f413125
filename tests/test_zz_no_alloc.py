"""GPU tier (collected last): the allocation-free Matmul entry point (puter_hip_matmul_noalloc)
against puter_hip_matmul, both through the C ABI.  The two share every kernel
and split-K chunking, so the results must be bit-identical.  Two calls in a row
on the shared static scratch, the second smaller, and a call at the scratch's
full 16 MiB capacity."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from helpers import empty_dev, seeded, to_dev, to_host

pytestmark = pytest.mark.gpu


def _call(lib, name, out, a, b, m, k, n, dt):
    import torch
    rc = getattr(lib, name)(C.c_void_p(out.data_ptr()), C.c_void_p(a.data_ptr()), C.c_void_p(b.data_ptr()),
                            m, k, n, dt, C.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, (name, rc, lib.puter_hip_last_error())


def _operands(dt, m, k, n, seed):
    a, b = seeded(seed, (m, k)), seeded(seed + 1, (k, n))
    if dt == O.F32:
        return to_dev(a), to_dev(b), np.float32
    return to_dev(O.from_f32(a, dt)), to_dev(O.from_f32(b, dt)), np.uint16


@pytest.mark.parametrize("dt,shapes", [
    # 16-bit skinny split-K path: 128 x 4096 x 4096 (8 chunks x 64 tiles: the full
    # 16 MiB of partials), then a smaller split-K shape and a ragged one
    (O.BF16, [(128, 4096, 4096), (16, 1024, 512), (5, 256, 136)]),
    (O.F16, [(64, 2048, 1024), (33, 512, 264)]),
    # f32: K split inside each block (128x512x512, no scratch), then K split
    # across blocks on the f32 MFMA kernel with partials in the scratch (256x4096x512,
    # 16 chunks: 8 MiB; 1024x8192x1024, chunks capped at 4 to fit the 16 MiB), the
    # VALU kernel's split (32x256x130: N not a multiple of 4), then a tiny one
    (O.F32, [(128, 512, 512), (256, 4096, 512), (1024, 8192, 1024), (32, 256, 130), (7, 13, 5)]),
])
def test_noalloc_matmul_matches_matmul(backend, dt, shapes):
    import torch
    lib = backend.lib
    for i, (m, k, n) in enumerate(shapes):
        a, b, npt = _operands(dt, m, k, n, 900 + 7 * i + dt)
        ref = empty_dev((m, n), npt)
        got = empty_dev((m, n), npt)
        got.fill_(0x7FC0 if npt == np.uint16 else float("nan"))   # poison: every output must be written
        _call(lib, "puter_hip_matmul", ref, a, b, m, k, n, dt)
        _call(lib, "puter_hip_matmul_noalloc", got, a, b, m, k, n, dt)
        torch.cuda.synchronize()
        r, g = to_host(ref, npt), to_host(got, npt)
        assert np.array_equal(r.view(np.uint8), g.view(np.uint8)), (dt, m, k, n)


def test_noalloc_matmul_validation(backend):
    lib = backend.lib
    assert lib.puter_hip_matmul_noalloc(C.c_void_p(0x1000), C.c_void_p(0x1000), C.c_void_p(0x1000),
                                        4, 4, 4, 3, None) == -6          # fp8: unsupported, as Matmul
    assert lib.puter_hip_matmul_noalloc(None, None, None, 0, 4, 4, 2, None) == 0   # empty output
