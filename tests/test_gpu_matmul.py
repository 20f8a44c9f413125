"""GPU tier: Matmul in BF16 / F16 (MFMA kernel and its generic fallback), F64 and
the empty-inner case, against the oracle restatement of
device/cpu/matmul/compute.go:46-92 through the C ABI."""
import numpy as np
import pytest

import oracle as O
from helpers import TOL, assert_close, empty_dev, seeded, to_dev, to_host

pytestmark = pytest.mark.gpu

# (rows, inner, cols): MFMA path (cols % 8 == 0, inner % 8 == 0) with ragged
# tile edges and a K tail, then shapes that take the generic kernel
SHAPES = [(256, 256, 128), (300, 200, 136), (1, 8, 8), (513, 1032, 264), (128, 512, 512),
          (1024, 4096, 1024), (7, 13, 5), (65, 64, 130), (33, 12, 40)]


@pytest.mark.parametrize("dt", [O.BF16, O.F16])
@pytest.mark.parametrize("rows,inner,cols", SHAPES)
def test_matmul_16bit(backend, dt, rows, inner, cols):
    a = O.from_f32(seeded(rows * 7 + inner, (rows, inner)), dt)
    b = O.from_f32(seeded(cols * 5 + inner, (inner, cols), 0.0, 0.05), dt)
    ref = O.to_f32(O.matmul(a, b, dt), dt)
    out = empty_dev((rows, cols), np.uint16)
    backend.Matmul(out, to_dev(a), to_dev(b), rows, inner, cols, dt)
    got = O.to_f32(to_host(out, np.uint16), dt)
    # sums over `inner` in another order than the reference's index order: normwise bar
    assert_close(got, ref, TOL[dt], elem_tol=None, what="matmul %dx%dx%d" % (rows, inner, cols))


@pytest.mark.parametrize("dt", [O.BF16, O.F16])
@pytest.mark.parametrize("rows,inner,cols", [(4000, 200, 4000), (4096, 1024, 4096), (4000, 200, 4104)])
def test_matmul_16bit_wide_tiles(backend, dt, rows, inner, cols):
    """Shapes of 256 output tiles of 256 x 256 (one round over the 256 CUs) take
    the 8-wave kernel, the first with ragged rows, columns and a K tail; 4000 x
    4104 (272 such tiles, two rounds, against three of 128 x 128 tiles) the 4-wave
    128 x 128 kernel.  The
    oracle checks one row in every 256-row band (all columns, so every tile) and
    the last row; the whole product is checked against numpy's f64 product of
    the same 16-bit inputs."""
    a = O.from_f32(seeded(rows + 11 * inner, (rows, inner)), dt)
    b = O.from_f32(seeded(cols + 13 * inner, (inner, cols), 0.0, 0.05), dt)
    out = empty_dev((rows, cols), np.uint16)
    backend.Matmul(out, to_dev(a), to_dev(b), rows, inner, cols, dt)
    got = O.to_f32(to_host(out, np.uint16), dt)
    sample = sorted({t * 256 + (t * 37) % 256 for t in range((rows + 255) // 256) if t * 256 + (t * 37) % 256 < rows}
                    | {rows - 1})
    ref = O.to_f32(O.matmul(np.ascontiguousarray(a[sample]), b, dt), dt)
    assert_close(got[sample], ref, TOL[dt], elem_tol=None, what="wide matmul rows %s" % sample[:4])
    full = O.to_f32(a, dt).astype(np.float64) @ O.to_f32(b, dt).astype(np.float64)
    assert_close(got, full, TOL[dt], elem_tol=None, what="wide matmul %dx%dx%d" % (rows, inner, cols))


@pytest.mark.parametrize("dt", [O.BF16, O.F16])
@pytest.mark.parametrize("rows,inner,cols", [(4000, 264, 4000), (4000, 264, 4104), (1000, 520, 1032), (513, 64, 2056),
                                             (1000, 2048, 520)])
def test_matmul_16bit_exact_integer_products(backend, dt, rows, inner, cols):
    """Every output element, bit for bit: operands are small integers (|a| <= 3,
    |b| <= 2), so each partial sum is an integer below 2^24 and exact in f32 in any
    summation order; the result must be the f32 sum of compute.go:74-92 rounded
    once to the 16-bit format, i.e. the oracle's narrowing of numpy's exact integer
    product.  The first shape takes the 8-wave 256 x 256 kernel, the second the
    4-wave 128 x 128 one, the others (under one round of 128 x 128 tiles) the
    split-K kernel, unsplit, then in two chunks (1000 x 2048 x 520); all have
    ragged row and column tiles (the epilogue's bounds) and K tails.  A misplaced, missing or duplicated element fails here,
    where a normwise bar could hide it."""
    rng = np.random.default_rng(rows + 7 * inner + 3 * cols)
    ai = rng.integers(-3, 4, (rows, inner))
    bi = rng.integers(-2, 3, (inner, cols))
    a = O.from_f32(ai.astype(np.float32), dt)
    b = O.from_f32(bi.astype(np.float32), dt)
    assert np.array_equal(O.to_f32(a, dt), ai) and np.array_equal(O.to_f32(b, dt), bi)
    exact = (ai @ bi).astype(np.float32)   # |sum| <= 6 * inner < 2^24: exact
    out = empty_dev((rows, cols), np.uint16)
    out.fill_(0x7FC0)   # a NaN pattern in both formats' sign/exponent field: unwritten cells show
    backend.Matmul(out, to_dev(a), to_dev(b), rows, inner, cols, dt)
    got = to_host(out, np.uint16)
    want = O.from_f32(exact, dt)
    bad = np.argwhere(got != want)
    assert bad.size == 0, f"{bad.shape[0]} cells differ, e.g. {bad[:4].tolist()}: {got[tuple(bad[:4].T)]} vs {want[tuple(bad[:4].T)]}"


def _random_matmul_shapes(n, seed):
    """Seeded random shapes across the Matmul routing rules: the small in-block
    split-K kernels, the 16-bit skinny split-K kernel (few rows or few tiles), the f32
    MFMA kernel split or not, the 128 x 128 and 256 x 256 16-bit tiles, and K / N
    that are not multiples of 4 or 8 (the generic kernels)."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        rows = int(rng.choice([int(rng.integers(1, 64)), int(rng.integers(64, 600)), int(rng.integers(600, 2500))]))
        inner = int(rng.choice([int(rng.integers(1, 128)), int(rng.integers(128, 1200)), int(rng.integers(1200, 4200))]))
        cols = int(rng.choice([int(rng.integers(1, 256)), int(rng.integers(256, 2600))]))
        if rng.integers(0, 2):   # aligned half the time
            inner, cols = max(8, inner // 8 * 8), max(8, cols // 8 * 8)
        out.append((rows, inner, cols))
    return out


@pytest.mark.parametrize("dt", [O.F32, O.BF16])
@pytest.mark.parametrize("rows,inner,cols", _random_matmul_shapes(12, 777))
def test_matmul_random_exact_integer_products(backend, dt, rows, inner, cols):
    """Small integer operands keep every partial sum exact in f32 whatever the kernel,
    tiling or split, so every output equals the exact product narrowed once to the
    output format, bit for bit; NaN-poisoned output catches a missing or misplaced
    element."""
    rng = np.random.default_rng(rows + 7 * inner + 3 * cols + dt)
    ai = rng.integers(-3, 4, (rows, inner)).astype(np.float32)
    bi = rng.integers(-2, 3, (inner, cols)).astype(np.float32)
    exact = (ai.astype(np.float64) @ bi.astype(np.float64)).astype(np.float32)
    if dt == O.F32:
        a, b, want, npt = ai, bi, exact, np.float32
    else:
        a, b, want, npt = O.from_f32(ai, dt), O.from_f32(bi, dt), O.from_f32(exact, dt), np.uint16
    out = empty_dev((rows, cols), npt)
    out.fill_(float("nan") if npt == np.float32 else 0x7FC0)
    backend.Matmul(out, to_dev(a), to_dev(b), rows, inner, cols, dt)
    got = to_host(out, npt)
    bad = np.argwhere(got.view(np.uint8).reshape(rows, -1) != want.view(np.uint8).reshape(rows, -1))
    assert bad.size == 0, f"{bad.shape[0]} bytes differ at {rows}x{inner}x{cols}, e.g. {bad[:4].tolist()}"


@pytest.mark.parametrize("rows,inner,cols", [(4000, 264, 4104), (2048, 100, 2052), (2100, 64, 2048)])
def test_matmul_f32_exact_integer_products(backend, rows, inner, cols):
    """F32 outputs of at least 256 tiles of 128 x 128 take the f32 MFMA kernel: small
    integer operands keep every partial sum exact in f32 whatever the summation
    order, so every output must equal numpy's exact integer product bit for bit
    (ragged row and column tiles, K tails of 8 and 4, K of exactly two slices).
    NaN-poisoned output: a missing, misplaced or duplicated element fails."""
    rng = np.random.default_rng(rows + 7 * inner + 3 * cols)
    ai = rng.integers(-3, 4, (rows, inner)).astype(np.float32)
    bi = rng.integers(-2, 3, (inner, cols)).astype(np.float32)
    want = (ai.astype(np.int64) @ bi.astype(np.int64)).astype(np.float32)
    out = empty_dev((rows, cols), np.float32)
    out.fill_(float("nan"))
    backend.Matmul(out, to_dev(ai), to_dev(bi), rows, inner, cols, O.F32)
    got = to_host(out, np.float32)
    bad = np.argwhere(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{bad.shape[0]} cells differ, e.g. {bad[:4].tolist()}: {got[tuple(bad[:4].T)]} vs {want[tuple(bad[:4].T)]}"


def test_matmul_f32_mfma_k_tail_never_reads_the_next_row(backend):
    """The f32 MFMA kernel's last 32-deep slice holds 4 valid columns (inner = 68);
    the chunks past inner must arrive as zeros, not as the next row's first values.
    Row 1 of `left` starts with NaN: only output row 1 may be NaN, and the rest
    matches the oracle."""
    rows, inner, cols = 2048, 68, 2048
    a = seeded(907, (rows, inner))
    a[1, 0] = np.nan
    b = seeded(908, (inner, cols), 0.0, 0.05)
    out = empty_dev((rows, cols), np.float32)
    backend.Matmul(out, to_dev(a), to_dev(b), rows, inner, cols, O.F32)
    got = to_host(out, np.float32)
    assert np.isnan(got[1]).all()
    keep = np.ones(rows, bool)
    keep[1] = False
    assert np.isfinite(got[keep]).all()
    sample = [0, 2, 127, 128, 1023, 2047]
    ref = O.matmul(np.ascontiguousarray(a[sample]), b, O.F32)
    assert_close(got[sample], ref, TOL[O.F32], elem_tol=None, what="f32 mfma k tail")


@pytest.mark.parametrize("dt", [O.BF16, O.F16])
@pytest.mark.parametrize("rows,inner,cols", [(64, 4096, 4096), (1, 4104, 2056), (200, 1000, 1024),
                                             (256, 512, 14336), (3, 64, 8), (500, 1032, 4104), (256, 512, 1024),
                                             (1000, 4096, 1000)])
def test_matmul_16bit_skinny_split_k(backend, dt, rows, inner, cols):
    """rows <= 512 take the split-K kernel (64 x 128 tiles over chunks of K, f32
    partials summed in chunk order), as do outputs under one round of 128 x 128
    tiles (1000 x 4096 x 1000: four chunks of 1024): ragged rows / columns, K
    tails, one-chunk and many-chunk splits; 200 x 1000 x 1024 (128 to 256 rows, a right operand of at
    most 2^22 elements) takes the small kernel instead, K split over the 8 waves of
    each block, on 16 x 16 tiles (as do 256x256x128 and 128x512x512 above), and
    256 x 512 x 1024 (256 tiles of 32 x 32) on 32 x 32 tiles.  Oracle rows sampled across the tile bands (all columns),
    numpy's f64 product for the whole output, and two calls bit-identical."""
    a = O.from_f32(seeded(rows * 3 + inner, (rows, inner)), dt)
    b = O.from_f32(seeded(cols * 7 + inner, (inner, cols), 0.0, 0.05), dt)
    ad, bd = to_dev(a), to_dev(b)
    out = empty_dev((rows, cols), np.uint16)
    backend.Matmul(out, ad, bd, rows, inner, cols, dt)
    got_bits = to_host(out, np.uint16)
    got = O.to_f32(got_bits, dt)
    sample = sorted({0, rows - 1, rows // 2, min(rows - 1, 63), min(rows - 1, 64), min(rows - 1, 131)})
    ref = O.to_f32(O.matmul(np.ascontiguousarray(a[sample]), b, dt), dt)
    assert_close(got[sample], ref, TOL[dt], elem_tol=None, what="skinny matmul rows %s" % sample)
    full = O.to_f32(a, dt).astype(np.float64) @ O.to_f32(b, dt).astype(np.float64)
    assert_close(got, full, TOL[dt], elem_tol=None, what="skinny matmul %dx%dx%d" % (rows, inner, cols))
    out2 = empty_dev((rows, cols), np.uint16)
    backend.Matmul(out2, ad, bd, rows, inner, cols, dt)
    assert np.array_equal(to_host(out2, np.uint16), got_bits)


def test_matmul_skinny_two_streams_share_the_scratch_safely(backend):
    """Split-K calls alternate between two streams (the second shape needs a larger
    scratch than the first, so the buffer grows while the first stream's work may
    still be queued); every result must match the same call made alone."""
    import torch
    shapes = [(64, 4096, 1024), (128, 8192, 2048), (64, 4096, 1024), (32, 2048, 512)]
    ins = []
    for i, (m, k, n) in enumerate(shapes):
        a = O.from_f32(seeded(950 + i, (m, k)), O.BF16)
        b = O.from_f32(seeded(960 + i, (k, n), 0.0, 0.05), O.BF16)
        ins.append((to_dev(a), to_dev(b)))
    alone = []
    for (m, k, n), (ad, bd) in zip(shapes, ins):
        out = empty_dev((m, n), np.uint16)
        backend.Matmul(out, ad, bd, m, k, n, O.BF16)
        alone.append(to_host(out, np.uint16))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [empty_dev((m, n), np.uint16) for m, k, n in shapes]
    torch.cuda.synchronize()
    for rep in range(3):
        for i, ((m, k, n), (ad, bd)) in enumerate(zip(shapes, ins)):
            with torch.cuda.stream(streams[i % 2]):
                backend.Matmul(outs[i], ad, bd, m, k, n, O.BF16)
        torch.cuda.synchronize()
        for i in range(len(shapes)):
            assert np.array_equal(to_host(outs[i], np.uint16), alone[i]), (rep, i)


def test_matmul_unaligned_16bit_falls_back(backend):
    """A left operand at an odd element offset is not 16-byte aligned: the MFMA and
    split-K paths are skipped for the generic kernel, whose result still meets the
    bar."""
    import torch
    rows, inner, cols = 64, 256, 512
    a = O.from_f32(seeded(971, (rows, inner)), O.BF16)
    b = O.from_f32(seeded(972, (inner, cols), 0.0, 0.05), O.BF16)
    abuf = torch.zeros(rows * inner + 1, dtype=torch.int16, device="cuda")
    abuf[1:] = to_dev(a).view(-1)
    out = empty_dev((rows, cols), np.uint16)
    backend.Matmul(out, abuf[1:], to_dev(b), rows, inner, cols, O.BF16)
    ref = O.to_f32(O.matmul(a, b, O.BF16), O.BF16)
    assert_close(O.to_f32(to_host(out, np.uint16), O.BF16), ref, TOL[O.BF16], elem_tol=None, what="unaligned")


def test_matmul_skinny_k_tail_never_reads_the_next_row(backend):
    """Split-K path: inner = 72 is two chunks of one 64-deep slice each, the second
    holding 8 valid columns; only output row 1 may be NaN."""
    rows, inner, cols = 64, 72, 4096
    a32 = seeded(905, (rows, inner))
    a32[1, 0] = np.nan
    a = O.from_f32(a32, O.BF16)
    b = O.from_f32(seeded(906, (inner, cols), 0.0, 0.05), O.BF16)
    out = empty_dev((rows, cols), np.uint16)
    backend.Matmul(out, to_dev(a), to_dev(b), rows, inner, cols, O.BF16)
    got = O.to_f32(to_host(out, np.uint16), O.BF16)
    assert np.isnan(got[1]).all()
    keep = np.ones(rows, bool)
    keep[1] = False
    assert np.isfinite(got[keep]).all()
    ref = O.to_f32(O.matmul(a, b, O.BF16), O.BF16)
    assert_close(got[keep], ref[keep], TOL[O.BF16], elem_tol=None, what="skinny k tail")


def test_matmul_k_tail_never_reads_the_next_row(backend):
    """64 rows (the split-K kernel), inner = 40: the one 64-deep K slice holds 40
    valid columns; the chunks past inner must arrive as zeros, not as the next
    row's first elements.  Row 1 of
    `left` starts with NaN: only output row 1 may be NaN."""
    rows, inner, cols = 64, 40, 128
    a32 = seeded(901, (rows, inner))
    a32[1, 0] = np.nan
    a = O.from_f32(a32, O.BF16)
    b = O.from_f32(seeded(902, (inner, cols), 0.0, 0.05), O.BF16)
    out = empty_dev((rows, cols), np.uint16)
    backend.Matmul(out, to_dev(a), to_dev(b), rows, inner, cols, O.BF16)
    got = O.to_f32(to_host(out, np.uint16), O.BF16)
    ref = O.to_f32(O.matmul(a, b, O.BF16), O.BF16)
    assert np.isnan(got[1]).all() and np.isnan(ref[1]).all()
    keep = np.ones(rows, bool)
    keep[1] = False
    assert np.isfinite(got[keep]).all()
    assert_close(got[keep], ref[keep], TOL[O.BF16], elem_tol=None, what="k tail")


@pytest.mark.parametrize("rows,inner,cols,sample", [(4096, 72, 4096, [0, 2, 255, 256, 2047, 4095]),
                                                    (4000, 72, 4104, [0, 2, 127, 128, 2047, 3999])])
def test_matmul_wide_k_tail_never_reads_the_next_row(backend, rows, inner, cols, sample):
    """The same isolation on the MFMA GEMM, 256 x 256 tiles (4096 x 4096) and
    128 x 128 tiles (4000 x 4104, ragged): inner = 72 leaves 8 valid columns in the
    last 64-wide slice; only output row 1 may be NaN."""
    a32 = seeded(903, (rows, inner))
    a32[1, 0] = np.nan
    a = O.from_f32(a32, O.BF16)
    b = O.from_f32(seeded(904, (inner, cols), 0.0, 0.05), O.BF16)
    out = empty_dev((rows, cols), np.uint16)
    backend.Matmul(out, to_dev(a), to_dev(b), rows, inner, cols, O.BF16)
    got = O.to_f32(to_host(out, np.uint16), O.BF16)
    assert np.isnan(got[1]).all()
    keep = np.ones(rows, bool)
    keep[1] = False
    assert np.isfinite(got[keep]).all()
    ref = O.to_f32(O.matmul(np.ascontiguousarray(a[sample]), b, O.BF16), O.BF16)
    assert_close(got[sample], ref, TOL[O.BF16], elem_tol=None, what="wide k tail")


def test_matmul_f64_and_f32(backend):
    for rows, inner, cols in [(64, 96, 48), (7, 13, 5)]:
        a = seeded(rows, (rows, inner)).astype(np.float64)
        b = seeded(cols + 3, (inner, cols)).astype(np.float64)
        ref = O.matmul(a, b, O.F64)
        out = empty_dev((rows, cols), np.float64)
        backend.Matmul(out, to_dev(a), to_dev(b), rows, inner, cols, O.F64)
        assert np.allclose(to_host(out, np.float64), ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("rows,inner,cols", [(128, 512, 512), (100, 1000, 300), (64, 96, 48), (7, 13, 5),
                                             (300, 40, 1100), (200, 333, 250), (32, 8192, 1024),
                                             (256, 1024, 1024), (33, 4100, 1030)])
def test_matmul_f32_split_k(backend, rows, inner, cols):
    """F32 (config 1's Matmul): small outputs of moderate depth (at least 32 32x32
    tiles and few 64-deep steps per wave: 128x512x512, 100x1000x300, 200x333x250
    with unaligned A rows on 16 x 16 tiles, 256x1024x1024 on 32 x 32 tiles) split
    K across the 8 waves of a block on the f32 MFMA; other aligned shapes take the
    128 x 128 f32 MFMA kernel, 64x96x48 in one block, 32x8192x1024 (8 tiles) with K
    split into 16 chunks summed in order; unaligned ones the VALU kernel, 33x4100x1030
    (cols not a multiple of 4) with K split across blocks into 16-deep-step chunks;
    ragged shapes and K tails, against the oracle's index-order f32 sum at the f32
    bar, and two calls bit-identical."""
    a = seeded(rows * 5 + inner, (rows, inner))
    b = seeded(cols * 3 + inner, (inner, cols), 0.0, 0.05)
    ref = O.matmul_f32(a, b)
    ad, bd = to_dev(a), to_dev(b)
    out = empty_dev((rows, cols), np.float32)
    backend.Matmul(out, ad, bd, rows, inner, cols, O.F32)
    got = to_host(out, np.float32)
    assert_close(got, ref, TOL[O.F32], elem_tol=1e-3, what="f32 matmul %dx%dx%d" % (rows, inner, cols))
    out2 = empty_dev((rows, cols), np.float32)
    backend.Matmul(out2, ad, bd, rows, inner, cols, O.F32)
    assert np.array_equal(to_host(out2, np.float32), got)


def test_matmul_f32_small_unaligned_left(backend):
    """The small f32 kernel with A rows that are a whole number of 16-byte vectors
    but an A base off by one float (the scalar-load variant): equal bit for bit to
    the aligned call on the same values, and to the oracle at the f32 bar."""
    import torch
    rows, inner, cols = 128, 512, 512
    a = seeded(77, (rows, inner))
    b = seeded(78, (inner, cols), 0.0, 0.05)
    ad, bd = to_dev(a), to_dev(b)
    shifted = torch.empty(rows * inner + 1, dtype=torch.float32, device="cuda")
    shifted[1:].copy_(ad.reshape(-1))
    au = shifted[1:]                      # 4 bytes past a 16-byte boundary
    assert au.data_ptr() % 16 == 4
    out, out_u = empty_dev((rows, cols), np.float32), empty_dev((rows, cols), np.float32)
    backend.Matmul(out, ad, bd, rows, inner, cols, O.F32)
    backend.Matmul(out_u, au, bd, rows, inner, cols, O.F32)
    got, got_u = to_host(out, np.float32), to_host(out_u, np.float32)
    assert np.array_equal(got, got_u)
    assert_close(got_u, O.matmul_f32(a, b), TOL[O.F32], elem_tol=1e-3, what="f32 matmul, unaligned A")


@pytest.mark.parametrize("dt,np_dt", [(O.BF16, np.uint16), (O.F32, np.float32), (O.F64, np.float64)])
def test_matmul_empty_inner_is_zero(backend, dt, np_dt):
    rows, cols = 5, 7   # odd element count
    out = to_dev(np.full((rows, cols), 7, np_dt))
    dummy = to_dev(np.zeros(8, np_dt))
    backend.Matmul(out, dummy, dummy, rows, 0, cols, dt)
    assert not to_host(out, np_dt).any()
