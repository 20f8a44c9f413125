"""Shared test helpers: seeded inputs, host<->device moves, parity metrics.

Parity bars (north star): bit-exact for casts, page gathers and the gated
residual's 16-bit output; otherwise the relative error
  normwise    ||gpu - ref||_inf / ||ref||_inf  <= tol
with tol = 1e-5 for f32 and 1e-2 for bf16 / fp8 (1e-3 for f16), and, as a
guard against errors confined to a few elements,
  elementwise |gpu - ref| / max(|ref|, 1e-3 * ||ref||_inf) <= elem_tol.
elem_tol = tol for element-wise kernels (RoPE, activations: no reductions, so
per-element errors are rounding-level).  Kernels that reduce (norms, matmul,
attention) sum in another order than the reference's sequential loop, so an
output that cancels to near zero carries the sum's absolute rounding error;
there elem_tol is 1e-3 for f32 and the normwise bar is the contract (bf16
attention: normwise only, its outputs are softmax-weighted sums over
thousands of keys).
"""
import numpy as np

import oracle as O

TOL = {O.F32: 1e-5, O.F16: 1e-3, O.BF16: 1e-2, O.F8E4M3: 1e-2}


def seeded(seed, shape, mean=0.0, std=1.0):
    n = int(np.prod(shape))
    return O.normal(seed, n, mean, std).reshape(shape)


def encode(x32, dtype):
    """f32 numpy -> storage numpy (bits for 16/8-bit formats)."""
    return x32.astype(np.float32) if dtype == O.F32 else O.from_f32(x32, dtype)


def decode(bits, dtype):
    return bits.astype(np.float32) if dtype == O.F32 else O.to_f32(bits, dtype)


def to_dev(arr):
    import torch
    arr = np.ascontiguousarray(arr)
    if arr.dtype == np.uint16:
        t = torch.from_numpy(arr.view(np.int16))
    elif arr.dtype == np.uint64:
        t = torch.from_numpy(arr.view(np.int64))
    elif arr.dtype == np.uint8:
        t = torch.from_numpy(arr)
    else:
        t = torch.from_numpy(arr)
    return t.cuda()


def empty_dev(shape, np_dtype):
    import torch
    table = {np.float32: torch.float32, np.uint16: torch.int16, np.uint8: torch.uint8,
             np.int32: torch.int32, np.int8: torch.int8, np.float64: torch.float64,
             np.uint64: torch.int64}
    return torch.empty(tuple(shape), dtype=table[np.dtype(np_dtype).type], device="cuda")


def to_host(t, np_dtype):
    import torch
    torch.cuda.synchronize()
    a = t.cpu().numpy()
    return a.view(np_dtype) if a.dtype != np_dtype else a


def errors(got, ref, floor=1e-3):
    got = np.asarray(got, np.float64).ravel()
    ref = np.asarray(ref, np.float64).ravel()
    scale = np.max(np.abs(ref)) if ref.size else 0.0
    if scale == 0:
        return float(np.max(np.abs(got - ref), initial=0.0)), 0.0
    norm = float(np.max(np.abs(got - ref)) / scale)
    elem = float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), floor * scale)))
    return norm, elem


REDUCE_ELEM_TOL = {O.F32: 1e-3, O.F16: 1e-2, O.BF16: 1e-2, O.F8E4M3: 1e-2}


def assert_close(got, ref, tol, elem_tol="same", floor=1e-3, what=""):
    """elem_tol: "same" -> tol; None -> normwise only; else a number."""
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    norm, elem = errors(got, ref, floor)
    et = tol if elem_tol == "same" else elem_tol
    ok = norm <= tol and (et is None or elem <= et)
    assert ok, f"{what}: normwise {norm:.3e} (tol {tol}), elementwise {elem:.3e} (tol {et})"
    return norm, elem
