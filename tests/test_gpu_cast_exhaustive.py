"""GPU: every one of the 2^32 f32 bit patterns narrowed by puter_hip_cast to bf16,
f16, fp8-E4M3 and fp8-E5M2, bit-exact against the oracle.

Reference: convert/bf16_f32.go:21-38 (Float32ToBFloat16), convert/f16_f32.go:10-42
(Float32ToFloat16), convert/fp8_f32.go:8-65 (Float32ToFloat8E4M3 / E5M2), whose
narrowing lives in manifesto/dtype; the oracle states the rule (RNE, saturating fp8,
the NaN encodings) and tests/test_oracle_pins.py pins it against torch and numpy for
every finite in-range input.  The patterns are walked in 16 chunks of 2^28: the
device builds each chunk's inputs (an iota plus the chunk base), the four narrowings
run on the GPU, and the host compares them with the oracle run on the same patterns
over all host cores."""
import os

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

CHUNK = 1 << 28
FORMATS = ((O.BF16, np.uint16), (O.F16, np.uint16), (O.F8E4M3, np.uint8), (O.F8E5M2, np.uint8))


@pytest.mark.timeout(900)
def test_narrow_every_f32_pattern(backend):
    import torch

    O.set_threads(min(16, os.cpu_count() or 1))
    iota = torch.arange(CHUNK, dtype=torch.int32, device="cuda")
    src = torch.empty(CHUNK, dtype=torch.int32, device="cuda")
    tdt = {np.uint16: torch.int16, np.uint8: torch.uint8}
    dst = {dt: torch.empty(CHUNK, dtype=tdt[npt], device="cuda") for dt, npt in FORMATS}
    host_iota = np.arange(CHUNK, dtype=np.uint32)
    checked = 0
    for c in range((1 << 32) // CHUNK):
        start = c * CHUNK
        # the chunk's patterns start..start+CHUNK-1 as int32 (no overflow either side of 2^31)
        src.copy_(iota).add_(start if start < (1 << 31) else start - (1 << 32))
        bits = host_iota + np.uint32(start)
        x = bits.view(np.float32)
        for dt, npt in FORMATS:
            backend.Cast(dst[dt], dt, src.view(torch.float32), O.F32, CHUNK)
        torch.cuda.synchronize()
        for dt, npt in FORMATS:
            got = dst[dt].cpu().numpy().view(npt)
            ref = O.from_f32(x, dt)
            bad = np.flatnonzero(got != ref)
            assert bad.size == 0, (f"format {dt}: {bad.size} mismatches in patterns {start:#x}.., e.g. "
                                   f"f32 {bits[bad[:4]]} -> {got[bad[:4]]} vs {ref[bad[:4]]}")
            del got, ref
        checked += CHUNK
        print(f"patterns {start:#010x}..{start + CHUNK - 1:#010x}: 4 formats bit-exact", flush=True)
    assert checked == 1 << 32
