"""GPU parity: paged KV write/gather (bit-exact), multi-head attention, paged
decode and the f32 matmul against the CPU oracle.

Reference: device/cpu/shape/page_generic.go, execution/page_intrinsic.go,
device/cpu/attention/{compute,typed_compute,softmax}.go, device/cpu/matmul."""
import numpy as np
import pytest

import oracle as O
from helpers import TOL, assert_close, decode, empty_dev, encode, seeded, to_dev, to_host

pytestmark = pytest.mark.gpu
NP = {O.F32: np.float32, O.F16: np.uint16, O.BF16: np.uint16, O.F8E4M3: np.uint8}


# -------------------------------------------------------------- paged KV --
def test_page_write_reference_kat(backend):
    """execution/page_intrinsic_test.go:15-71: storage [2,3,2,1,1] f32, layer 1
    (storageOffset 6), rows 7, 8 -> page 1 slots 0, 1 -> storage[8]=7, [9]=8."""
    storage = to_dev(np.zeros(12, np.float32))
    values = to_dev(np.array([7, 8], np.float32))
    ids = to_dev(np.array([1, 1], np.int32))
    offs = to_dev(np.array([0, 1], np.int32))
    backend.KVPageWrite(storage, values, ids, offs, storage, 3, 2, 1, 2, 6, O.F32)
    got = to_host(storage, np.float32)
    expect = np.zeros(12, np.float32)
    expect[8], expect[9] = 7, 8
    assert np.array_equal(got, expect)


@pytest.mark.parametrize("dt,inner", [(O.BF16, 1024), (O.F32, 24), (O.F16, 3), (O.F8E4M3, 1024), (O.BF16, 7)])
def test_page_write_gather_roundtrip(backend, dt, inner):
    rng = np.random.default_rng(inner + dt)
    pages, ps = 40, 16
    es = np.dtype(NP[dt]).itemsize
    storage = rng.integers(0, 2**(8 * es) if es < 4 else 2**31, size=pages * ps * inner).astype(
        np.uint32 if es == 4 else NP[dt])
    if es == 4:
        storage = storage.view(np.float32)
    rows = 37
    ids = rng.integers(0, pages, rows).astype(np.int32)
    offs = rng.integers(0, ps, rows).astype(np.int32)
    vals = rng.integers(0, 200, size=ids.size * inner).astype(NP[dt] if es < 4 else np.float32)
    ref_store = O.page_write(storage, vals, ids, offs, ps, inner)
    d_store = to_dev(storage)
    backend.KVPageWrite(d_store, to_dev(vals), to_dev(ids), to_dev(offs), d_store, pages, ps, inner,
                        ids.size, 0, dt)
    got_store = to_host(d_store, storage.dtype)
    assert np.array_equal(got_store.view(np.uint8), ref_store.view(np.uint8))
    table = rng.permutation(pages)[:9].astype(np.int32)
    out_rows = 9 * ps - 5
    ref = O.page_gather(ref_store, table, ps, inner, out_rows)
    out = empty_dev((out_rows, inner), storage.dtype)
    backend.KVPageGather(d_store, to_dev(table), out, pages, ps, inner, out_rows, 0, dt)
    got = to_host(out, storage.dtype)
    assert np.array_equal(got.view(np.uint8), ref.view(np.uint8))


def test_page_write_gather_beyond_4gib(backend):
    """A bf16 pool of more than 4 GiB (2 KiB rows): rows written to and gathered
    from pages past the 4 GiB mark, bit-exact against the oracle on a compact
    copy of those pages (the kernels index with 64-bit offsets)."""
    import torch
    ps, inner = 16, 1024
    pages = (1 << 32) // (ps * inner * 2) + 64
    far0 = pages - 8                                   # the last 8 pages
    rng = np.random.default_rng(19)
    vals = rng.integers(0, 1 << 16, (40, inner)).astype(np.uint16)
    ids = rng.integers(0, 8, 40).astype(np.int32)
    offs = rng.integers(0, ps, 40).astype(np.int32)
    compact = rng.integers(0, 1 << 16, (8, ps, inner)).astype(np.uint16)
    pool = torch.zeros((pages, ps, inner), dtype=torch.int16, device="cuda")
    pool[far0:] = torch.from_numpy(compact.view(np.int16)).cuda()
    backend.KVPageWrite(pool, to_dev(vals), to_dev(ids + far0), to_dev(offs), pool, pages, ps, inner, 40, 0, O.BF16)
    want = O.page_write(compact.ravel(), vals, ids, offs, ps, inner).reshape(8, ps, inner)
    assert np.array_equal(pool[far0:].cpu().numpy().view(np.uint16), want)
    table = rng.permutation(8).astype(np.int32)
    out = empty_dev((8 * ps, inner), np.uint16)
    backend.KVPageGather(pool, to_dev(table + far0), out, pages, ps, inner, 8 * ps, 0, O.BF16)
    assert np.array_equal(to_host(out, np.uint16), O.page_gather(want.ravel(), table, ps, inner, 8 * ps))
    backend.CheckStatus()
    del pool
    torch.cuda.empty_cache()


def test_page_gather_identity_table_is_contiguous_copy(backend):
    pages, ps, inner = 8, 4, 32
    storage = seeded(3, (pages * ps * inner,))
    out = empty_dev((pages * ps, inner), np.float32)
    backend.KVPageGather(to_dev(storage), to_dev(np.arange(pages, dtype=np.int32)), out, pages, ps,
                         inner, pages * ps, 0, O.F32)
    assert np.array_equal(to_host(out, np.float32).ravel(), storage)


@pytest.mark.parametrize("dt", [O.BF16, O.F16, O.F32])
def test_page_write_fp8_matches_oracle(backend, dt):
    """Extension hook: quantising write into an fp8-E4M3 pool [pages, 16, 4, 128],
    bit-exact against the oracle (IEEE division, saturating RNE narrowing),
    including values beyond the E4M3 range (saturation) and a layer offset."""
    rng = np.random.default_rng(31 + dt)
    pages, ps, kvh, hd = 24, 16, 4, 128
    inner = kvh * hd
    layer_off = pages * ps * inner                # second layer of a rank-5 storage
    storage = rng.integers(0, 256, size=2 * pages * ps * inner).astype(np.uint8)
    rows = 100
    slots = rng.choice(pages * ps, size=rows, replace=False)      # unique (page, slot)
    ids = (slots // ps).astype(np.int32)
    offs = (slots % ps).astype(np.int32)
    scales = rng.uniform(0.01, 1.0, kvh).astype(np.float32)
    x = rng.normal(0, 1, (rows, inner)).astype(np.float32) * 200.0   # |x / s| up to ~1e5: saturates
    vals = encode(x, dt)
    ref = O.page_write_fp8(storage, vals, ids, offs, ps, kvh, hd, scales, dt, storage_offset=layer_off)
    d = to_dev(storage)
    backend.KVPageWriteFP8(d, to_dev(vals), to_dev(ids), to_dev(offs), pages, ps, kvh, hd, rows,
                           layer_off, to_dev(scales), dt)
    got = to_host(d, np.uint8)
    assert np.array_equal(got, ref)


def test_page_write_fp8_roundtrip_and_bounds(backend):
    import puter_amd
    """Dequantised pool rows equal the values within E4M3's half-ulp (2^-4 relative
    for normal codes); rows with a bad page id or slot leave the pool untouched."""
    rng = np.random.default_rng(7)
    pages, ps, kvh, hd = 8, 16, 2, 64
    inner = kvh * hd
    storage = np.zeros(pages * ps * inner, np.uint8)
    scales = np.array([0.5, 0.03125], np.float32)
    x = rng.normal(0, 1, (4, inner)).astype(np.float32)
    vals = encode(x, O.BF16)
    ids = np.array([3, 99, 5, -1], np.int32)      # rows 1 and 3 are out of range
    offs = np.array([2, 0, 15, 4], np.int32)
    d = to_dev(storage)
    backend.KVPageWriteFP8(d, to_dev(vals), to_dev(ids), to_dev(offs), pages, ps, kvh, hd, 4, 0,
                           to_dev(scales), O.BF16)
    got = to_host(d, np.uint8).reshape(pages, ps, inner)
    touched = np.zeros((pages, ps), bool)
    touched[3, 2] = touched[5, 15] = True
    assert not got[~touched].any(), "an out-of-range row was written"
    with pytest.raises(puter_amd.PuterError):      # the status word reports the rejected rows
        backend.CheckStatus()
    xs = decode(vals, O.BF16)
    for r, (pg, sl) in ((0, (3, 2)), (2, (5, 15))):
        deq = O.to_f32(got[pg, sl], O.F8E4M3).reshape(kvh, hd) * scales[:, None]
        want = xs[r].reshape(kvh, hd)
        assert np.all(np.abs(deq - want) <= np.abs(want) * 2.0 ** -4 + scales[:, None] * 2.0 ** -9)


def test_page_out_of_range_ids_never_touch_memory(backend):
    """Where the reference rejects the call (device/cpu/shape/page.go:139-146,191-203)
    the device path skips (write) or zero-fills (gather) the bad rows, never
    touches memory outside the storage, and reports through the status word."""
    import puter_amd
    backend.CheckStatus()
    pages, ps, inner = 4, 2, 8
    storage = seeded(4, (pages * ps * inner,))
    d = to_dev(storage)
    vals = seeded(5, (4, inner))
    ids, offs = np.array([9, 1, -1, 2], np.int32), np.array([0, 1, 0, 2], np.int32)   # rows 0, 2, 3 bad
    backend.KVPageWrite(d, to_dev(vals), to_dev(ids), to_dev(offs), d, pages, ps, inner, 4, 0, O.F32)
    with pytest.raises(puter_amd.PuterError) as e:
        backend.CheckStatus()
    assert e.value.status == -6
    want = O.page_write(storage, vals[1:2], ids[1:2], offs[1:2], ps, inner)   # only the valid row landed
    assert np.array_equal(to_host(d, np.float32), want)
    backend.CheckStatus()                                     # cleared by the read
    out = empty_dev((2 * ps, inner), np.float32)
    backend.KVPageGather(d, to_dev(np.array([1, 77], np.int32)), out, pages, ps, inner, 2 * ps, 0, O.F32)
    got = to_host(out, np.float32)
    assert np.array_equal(got[:ps].ravel(), want[ps * inner:2 * ps * inner])
    assert np.all(got[ps:] == 0)
    with pytest.raises(puter_amd.PuterError):
        backend.CheckStatus()
    # a valid call leaves the word clear
    backend.KVPageGather(d, to_dev(np.array([1, 3], np.int32)), out, pages, ps, inner, 2 * ps, 0, O.F32)
    backend.CheckStatus()
    # the batching hooks (execution/dispatch.go:120-123): EndBatch returns the
    # batch's page error instead of raising, and clears it
    assert backend.BeginBatch() is None
    backend.KVPageGather(d, to_dev(np.array([5], np.int32)), out, pages, ps, inner, ps, 0, O.F32)
    err = backend.EndBatch()
    assert isinstance(err, puter_amd.PuterError) and err.status == -6
    assert backend.EndBatch() is None


@pytest.mark.parametrize("dt,inner,rows", [(O.BF16, 1024, 300), (O.F32, 3, 77), (O.F8E4M3, 1024, 200),
                                           (O.F16, 5, 1000)])
def test_page_write_duplicate_slots_last_row_wins(backend, dt, inner, rows):
    """Rows aimed at the same (page, slot): the reference copies rows in order,
    so the last one wins (device/cpu/shape/page_generic.go:23-27).  Ids and slots
    drawn from a small range so most slots are hit several times; every value
    row distinct, so the pool shows which row landed."""
    backend.CheckStatus()
    rng = np.random.default_rng(rows + inner)
    pages, ps = 6, 4
    es = np.dtype(NP[dt]).itemsize
    storage = np.zeros(pages * ps * inner, NP[dt])
    ids = rng.integers(0, 3, rows).astype(np.int32)
    offs = rng.integers(0, ps, rows).astype(np.int32)
    assert np.unique(ids * ps + offs).size < rows // 4
    vals = (np.arange(rows * inner) % (2**(8 * min(es, 2)) - 3) + 1).astype(NP[dt]) if es < 4 else \
        np.arange(rows * inner, dtype=np.float32)
    ref = O.page_write(storage, vals, ids, offs, ps, inner)
    d = to_dev(storage)
    backend.KVPageWrite(d, to_dev(vals), to_dev(ids), to_dev(offs), d, pages, ps, inner, rows, 0, dt)
    assert np.array_equal(to_host(d, storage.dtype).view(np.uint8), ref.view(np.uint8))
    backend.CheckStatus()


def test_page_write_fp8_duplicate_slots_last_row_wins(backend):
    backend.CheckStatus()
    rng = np.random.default_rng(11)
    pages, ps, kvh, hd, rows = 4, 16, 2, 128, 500
    inner = kvh * hd
    ids = rng.integers(0, 2, rows).astype(np.int32)
    offs = rng.integers(0, ps, rows).astype(np.int32)
    scales = np.array([0.25, 2.0], np.float32)
    vals = encode(rng.normal(0, 1, (rows, inner)).astype(np.float32), O.BF16)
    storage = np.zeros(pages * ps * inner, np.uint8)
    ref = O.page_write_fp8(storage, vals, ids, offs, ps, kvh, hd, scales, O.BF16)
    d = to_dev(storage)
    backend.KVPageWriteFP8(d, to_dev(vals), to_dev(ids), to_dev(offs), pages, ps, kvh, hd, rows, 0,
                           to_dev(scales), O.BF16)
    assert np.array_equal(to_host(d, np.uint8), ref)
    backend.CheckStatus()


@pytest.mark.parametrize("dt,inner,rows", [(O.BF16, 1024, 20000), (O.F32, 6, 70001), (O.F8E4M3, 1024, 16384)])
def test_page_write_prefill_sized_duplicates_far_apart(backend, dt, inner, rows):
    """A prefill-sized KVPageWrite (16K to 70K rows: 16 to 128 rows per block,
    2 KiB rows on the 16-byte path, 24-byte rows on the 4-byte path with a unit
    count that is not a power of two, and the fp8 quantising write) whose
    repeated (page, slot) pairs sit far apart: a tenth of the rows reuse the slot
    of a random earlier row, the first and last rows share a slot, two adjacent
    rows share one, and one slot is hit in three distant blocks.  The reference
    copies the rows in order, so the last row of each slot wins
    (device/cpu/shape/page_generic.go:23-27); the pool must equal the oracle's
    bit for bit."""
    backend.CheckStatus()
    rng = np.random.default_rng(rows + inner + dt)
    ps = 16
    pages = rows // ps + 8
    slot = rng.permutation(pages * ps)[:rows].astype(np.int64)
    reuse = rng.choice(np.arange(1000, rows), rows // 10, replace=False)
    for r in np.sort(reuse):
        slot[r] = slot[rng.integers(0, r)]
    slot[rows - 1] = slot[0]
    slot[101] = slot[100]
    slot[rows // 3] = slot[rows // 2] = slot[7]
    ids, offs = (slot // ps).astype(np.int32), (slot % ps).astype(np.int32)
    assert np.unique(slot).size < rows - rows // 20
    if dt == O.F8E4M3:
        kvh, hd = 8, 128
        scales = (rng.random(kvh).astype(np.float32) + 0.5) / 64
        vals = encode(rng.normal(0, 1, (rows, inner)).astype(np.float32), O.BF16)
        storage = rng.integers(0, 256, pages * ps * inner).astype(np.uint8)
        ref = O.page_write_fp8(storage, vals, ids, offs, ps, kvh, hd, scales, O.BF16)
        d = to_dev(storage)
        backend.KVPageWriteFP8(d, to_dev(vals), to_dev(ids), to_dev(offs), pages, ps, kvh, hd, rows, 0,
                               to_dev(scales), O.BF16)
        assert np.array_equal(to_host(d, np.uint8), ref)
    else:
        es = np.dtype(NP[dt]).itemsize
        bits = np.uint32 if es == 4 else np.uint16
        storage = rng.integers(0, 1 << (8 * es), pages * ps * inner, dtype=np.uint64).astype(bits)
        vals = rng.integers(0, 1 << (8 * es), rows * inner, dtype=np.uint64).astype(bits)
        if es == 4:
            storage, vals = storage.view(np.float32), vals.view(np.float32)
        ref = O.page_write(storage, vals, ids, offs, ps, inner)
        d = to_dev(storage)
        backend.KVPageWrite(d, to_dev(vals), to_dev(ids), to_dev(offs), d, pages, ps, inner, rows, 0, dt)
        assert np.array_equal(to_host(d, storage.dtype).view(np.uint8), ref.view(np.uint8))
    backend.CheckStatus()


# -------------------------------------------------------------- attention --
@pytest.mark.parametrize("dt", [O.F32, O.BF16, O.F16])
@pytest.mark.parametrize("sq,sk,h,kvh,d,causal", [
    (128, 128, 8, 8, 64, True),     # config 1
    (77, 77, 4, 2, 64, True),
    (5, 300, 4, 1, 128, True),       # bottom-right aligned causal
    (64, 64, 8, 2, 128, False),
    (1, 513, 8, 2, 128, True),       # decode shape
    (300, 300, 8, 2, 128, True),     # ragged query and key tiles (f32: the f32 MFMA prefill kernel, 24 blocks)
    (200, 520, 16, 4, 64, True),     # causal shift 320, head dim 64 (32 blocks)
    (150, 150, 16, 4, 128, False),   # not causal, ragged tiles (32 blocks)
])
def test_mha(backend, dt, sq, sk, h, kvh, d, causal):
    import puter_amd
    std = 1.0 / np.sqrt(d) if dt != O.F32 else 1.0
    q = encode(seeded(90 + sq, (sq, h * d), 0.0, std), dt)
    k = encode(seeded(91 + sk, (sk, kvh * d), 0.0, std), dt)
    v = encode(seeded(92 + sk, (sk, kvh * d)), dt)
    ref = decode(O.mha(q, k, v, h, d, causal=causal, kv_heads=kvh, dtype=dt), dt)
    out = empty_dev((sq, h * d), NP[dt])
    cfg = puter_amd.MultiHeadAttentionConfig(h, d, causal, 0, 0.0, kvh)
    backend.MultiHeadAttention(cfg, to_dev(q), to_dev(k), to_dev(v), out, sq, sk, dt)
    assert_close(decode(to_host(out, NP[dt]), dt), ref, TOL[dt],
                 elem_tol=1e-3 if dt == O.F32 else None, what="mha")


@pytest.mark.parametrize("sq,sk,h,kvh,d,causal", [
    (1024, 1024, 4, 1, 64, True),    # 32 blocks, 4 runs of 8 key tiles; the first query tile's last 3 are empty
    (200, 2100, 12, 4, 64, False),   # 24 blocks, 4 runs of 17 tiles, the last ragged
    (300, 1300, 8, 2, 128, True),    # head dim 128, causal shift 1000, 5 runs of 9 tiles, the last ragged
    (256, 256, 8, 2, 128, True),     # 16 blocks (under 24: split in runs of 2 tiles, 4 runs)
    (640, 640, 4, 4, 64, True),      # 20 blocks, 10 runs of 2 tiles
])
def test_mha_f32_key_split(backend, sq, sk, h, kvh, d, causal):
    """f32 grids under one block per CU split each block's key range over blockIdx.y
    and merge the runs' (max, sum, output) partials in a second kernel."""
    import puter_amd
    dt = O.F32
    q = encode(seeded(190 + sq, (sq, h * d)), dt)
    k = encode(seeded(191 + sk, (sk, kvh * d)), dt)
    v = encode(seeded(192 + sk, (sk, kvh * d)), dt)
    ref = decode(O.mha(q, k, v, h, d, causal=causal, kv_heads=kvh, dtype=dt), dt)
    out = empty_dev((sq, h * d), NP[dt])
    cfg = puter_amd.MultiHeadAttentionConfig(h, d, causal, 0, 0.0, kvh)
    backend.MultiHeadAttention(cfg, to_dev(q), to_dev(k), to_dev(v), out, sq, sk, dt)
    assert_close(decode(to_host(out, NP[dt]), dt), ref, TOL[dt], elem_tol=1e-3, what="mha split")


def _random_mha_cases(n, seed):
    """Seeded random MultiHeadAttention shapes across the routing rules: grid sizes
    on both sides of the f32 kernel's 24-block and split thresholds, ragged tiles,
    seqK above and below seqQ, GQA groups, windows and ALiBi slopes."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        d = int(rng.choice([64, 128]))
        kvh = int(rng.choice([1, 2, 4]))
        h = kvh * int(rng.choice([1, 2, 4]))
        sq = int(rng.integers(16, 700))
        sk = int(max(1, sq + rng.integers(-sq // 2, 600)))
        b = int(rng.choice([1, 2]))
        causal = bool(rng.integers(0, 2))
        window = int(rng.choice([0, 0, int(rng.integers(1, 300))]))
        alibi = float(rng.choice([0.0, 0.0, 0.0625, -0.125]))
        cases.append((b, sq, sk, h, kvh, d, causal, window, alibi))
    return cases


@pytest.mark.parametrize("dt", [O.F32, O.BF16])
@pytest.mark.parametrize("case", _random_mha_cases(10, 4242))
def test_mha_random_shapes(backend, dt, case):
    """MultiHeadAttentionBatched on seeded random shapes against the oracle, each
    batch element separately (the reference's per-call layout)."""
    import puter_amd
    b, sq, sk, h, kvh, d, causal, window, alibi = case
    std = 1.0 / np.sqrt(d)
    q = encode(seeded(400 + sq, (b, sq, h * d), 0.0, std), dt)
    k = encode(seeded(401 + sk, (b, sk, kvh * d), 0.0, std), dt)
    v = encode(seeded(402 + sk, (b, sk, kvh * d)), dt)
    out = empty_dev((b, sq, h * d), NP[dt])
    cfg = puter_amd.MultiHeadAttentionConfig(h, d, causal, window, alibi, kvh)
    backend.MultiHeadAttentionBatched(cfg, to_dev(q), to_dev(k), to_dev(v), out, b, sq, sk, dt)
    got = decode(to_host(out, NP[dt]), dt)
    O.set_threads(8)
    for i in range(b):
        ref = decode(O.mha(q[i], k[i], v[i], h, d, causal=causal, kv_heads=kvh, window=window, alibi=alibi,
                           dtype=dt), dt)
        assert_close(got[i], ref, TOL[dt], elem_tol=None, what=f"random mha {case} batch {i}")


@pytest.mark.parametrize("dt", [O.BF16, O.F16])
@pytest.mark.parametrize("b,sk,h,kvh,causal,window", [
    (1, 4096, 32, 8, True, 0),     # configs[4]'s heads at one sequence's full context
    (1, 100, 8, 8, False, 0),      # group size 1, part of one split
    (1, 300, 16, 2, True, 0),      # group size 8
    (3, 700, 8, 4, True, 0),       # batched, partial last split
    (64, 2000, 32, 8, True, 0),    # 256-token splits (enough waves)
    (2, 900, 16, 4, True, 128),    # sliding_window_attention's window: hides no key of row 0
    (2, 1000, 28, 4, True, 0),     # group size 7 (read at run time)
])
def test_mha_one_query_row(backend, dt, b, sk, h, kvh, causal, window):
    """seqQ = 1 (the reference's decode step after KVPageGather) runs on the paged
    decode kernels over contiguous K/V: against the oracle's MHA per sequence.  The
    window compares keys with the query's row index (typed_compute.go:172), 0
    for one row, so it masks nothing."""
    import puter_amd
    d = 128
    std = 1.0 / np.sqrt(d)
    q = encode(seeded(700 + sk, (b, 1, h * d), 0.0, std), dt)
    k = encode(seeded(701 + sk, (b, sk, kvh * d), 0.0, std), dt)
    v = encode(seeded(702 + sk, (b, sk, kvh * d)), dt)
    out = empty_dev((b, 1, h * d), np.uint16)
    cfg = puter_amd.MultiHeadAttentionConfig(h, d, causal, window, 0.0, kvh)
    if b == 1:
        backend.MultiHeadAttention(cfg, to_dev(q[0]), to_dev(k[0]), to_dev(v[0]), out, 1, sk, dt)
    else:
        backend.MultiHeadAttentionBatched(cfg, to_dev(q), to_dev(k), to_dev(v), out, b, 1, sk, dt)
    got = decode(to_host(out, np.uint16), dt)
    for i in range(b):
        ref = decode(O.mha(q[i], k[i], v[i], h, d, causal=causal, kv_heads=kvh, window=window, dtype=dt), dt)
        assert_close(got[i], ref, TOL[dt], elem_tol=None, what=f"one-row mha sequence {i}")


@pytest.mark.parametrize("dt,d,b,sk,h,kvh,causal,window,alibi", [
    (O.BF16, 64, 1, 4096, 8, 2, True, 0, 0.0),      # the registered 8 x 64 heads at a decode step
    (O.BF16, 64, 3, 769, 8, 8, True, 128, 0.0),     # four chunks, the last of one key; window
    (O.F16, 48, 2, 1000, 4, 2, False, 0, 0.0),      # odd head dim, f16 dots
    (O.F32, 64, 1, 800, 8, 8, True, 0, 0.0),        # f32 (config 1's format)
    (O.BF16, 128, 2, 900, 8, 2, True, 0, 0.25),     # head dim 128 with ALiBi (not the decode kernels)
    (O.F32, 256, 1, 1100, 2, 1, True, 0, -0.5),     # widest head dim
    (O.BF16, 64, 2, 512, 8, 2, True, 0, 0.0),       # two chunks: the unsplit kernel
])
def test_mha_one_query_row_split(backend, dt, d, b, sk, h, kvh, causal, window, alibi):
    """seqQ = 1 outside the decode kernels' shapes, over more than 768 keys: the
    general kernel split over 256-key chunks, merged in order, against the oracle
    per sequence (the last case stays unsplit)."""
    import puter_amd
    std = 1.0 / np.sqrt(d)
    q = encode(seeded(710 + sk, (b, 1, h * d), 0.0, std), dt)
    k = encode(seeded(711 + sk, (b, sk, kvh * d), 0.0, std), dt)
    v = encode(seeded(712 + sk, (b, sk, kvh * d)), dt)
    out = empty_dev((b, 1, h * d), NP[dt])
    cfg = puter_amd.MultiHeadAttentionConfig(h, d, causal, window, alibi, kvh)
    backend.MultiHeadAttentionBatched(cfg, to_dev(q), to_dev(k), to_dev(v), out, b, 1, sk, dt)
    got = decode(to_host(out, NP[dt]), dt)
    for i in range(b):
        ref = decode(O.mha(q[i], k[i], v[i], h, d, causal=causal, kv_heads=kvh, window=window, alibi=alibi,
                           dtype=dt), dt)
        assert_close(got[i], ref, TOL[dt], elem_tol=1e-3 if dt == O.F32 else None,
                     what=f"split one-row mha sequence {i}")


def test_mha_one_query_row_unaligned_falls_back(backend):
    """A query not 16-byte aligned (an odd element offset) cannot take the decode
    kernels' 16-byte loads: the call falls back to the general kernel and the
    result still matches the oracle."""
    import puter_amd
    import torch
    dt, h, kvh, d, sk = O.BF16, 8, 2, 128, 300
    std = 1.0 / np.sqrt(d)
    q = encode(seeded(801, (1, h * d), 0.0, std), dt)
    k = encode(seeded(802, (sk, kvh * d), 0.0, std), dt)
    v = encode(seeded(803, (sk, kvh * d)), dt)
    qbuf = torch.zeros(h * d + 1, dtype=torch.int16, device="cuda")
    qbuf[1:] = to_dev(q).view(-1)
    out = empty_dev((1, h * d), np.uint16)
    cfg = puter_amd.MultiHeadAttentionConfig(h, d, True, 0, 0.0, kvh)
    backend.MultiHeadAttention(cfg, qbuf[1:], to_dev(k), to_dev(v), out, 1, sk, dt)
    ref = decode(O.mha(q, k, v, h, d, causal=True, kv_heads=kvh, dtype=dt), dt)
    assert_close(decode(to_host(out, np.uint16), dt), ref, TOL[dt], elem_tol=None, what="unaligned one-row mha")


def test_mha_window_alibi(backend):
    import puter_amd
    dt, sq, h, d = O.F32, 40, 2, 32
    q, k, v = (seeded(s, (sq, h * d)) for s in (1, 2, 3))
    ref = O.mha(q, k, v, h, d, causal=True, kv_heads=0, window=7, alibi=0.25, dtype=dt)
    out = empty_dev((sq, h * d), np.float32)
    cfg = puter_amd.MultiHeadAttentionConfig(h, d, True, 7, 0.25, 0)
    backend.MultiHeadAttention(cfg, to_dev(q), to_dev(k), to_dev(v), out, sq, sq, dt)
    assert_close(to_host(out, np.float32), ref, TOL[dt], elem_tol=None, what="window+alibi")


def test_mha_batched_prefill_bf16(backend):
    import puter_amd
    dt, b, s, h, kvh, d = O.BF16, 2, 256, 8, 2, 128
    std = 1.0 / np.sqrt(d)
    q = encode(seeded(7, (b, s, h * d), 0.0, std), dt)
    k = encode(seeded(8, (b, s, kvh * d), 0.0, std), dt)
    v = encode(seeded(9, (b, s, kvh * d), 0.0, std), dt)
    out = empty_dev((b, s, h * d), np.uint16)
    cfg = puter_amd.MultiHeadAttentionConfig(h, d, True, 0, 0.0, kvh)
    backend.MultiHeadAttentionBatched(cfg, to_dev(q), to_dev(k), to_dev(v), out, b, s, s, dt)
    got = decode(to_host(out, np.uint16), dt)
    for i in range(b):
        ref = decode(O.mha(q[i], k[i], v[i], h, d, causal=True, kv_heads=kvh, dtype=dt), dt)
        assert_close(got[i], ref, TOL[dt], elem_tol=None, what=f"batch {i}")


def test_prefill_rows_agree_with_one_row_path_bf16(backend):
    """The MFMA prefill keeps each bf16 score dot in f32, where the reference
    (typed_compute.go:16-20, dot/bf16_generic.go:9-21) and the one-row kernel
    round it to bf16.  Row i of a causal prefill sees keys 0..i, exactly what a
    one-row call over the first i+1 keys sees: the two paths agree to the bf16
    bar elementwise on every element above a tenth of the row's largest."""
    import puter_amd
    dt, s, h, kvh, d = O.BF16, 512, 8, 2, 128
    std = 1.0 / np.sqrt(d)
    q = encode(seeded(41, (s, h * d), 0.0, 4 * std), dt)
    k = encode(seeded(42, (s, kvh * d), 0.0, 4 * std), dt)
    v = encode(seeded(43, (s, kvh * d)), dt)
    cfg = puter_amd.MultiHeadAttentionConfig(h, d, True, 0, 0.0, kvh)
    out = empty_dev((s, h * d), np.uint16)
    backend.MultiHeadAttention(cfg, to_dev(q), to_dev(k), to_dev(v), out, s, s, dt)
    rows = decode(to_host(out, np.uint16), dt)
    for i in (0, 63, 64, 300, s - 1):
        one = empty_dev((1, h * d), np.uint16)
        backend.MultiHeadAttention(cfg, to_dev(q[i:i + 1]), to_dev(k[:i + 1].copy()), to_dev(v[:i + 1].copy()),
                                   one, 1, i + 1, dt)
        ref1 = decode(to_host(one, np.uint16), dt)[0]
        assert_close(rows[i], ref1, TOL[dt], elem_tol=2e-2, floor=0.1, what=f"row {i}")
        oracle_row = decode(O.mha(q[i:i + 1], k[:i + 1], v[:i + 1], h, d, causal=True, kv_heads=kvh, dtype=dt), dt)
        assert_close(ref1, oracle_row[0], TOL[dt], elem_tol=2e-2, floor=0.1, what=f"one-row {i} vs oracle")


@pytest.mark.parametrize("b,sq,sk,h,kvh,causal", [
    (1, 1024, 1024, 8, 2, True),    # several diagonal and full tiles per block
    (2, 333, 333, 4, 1, True),      # ragged: partial query and key tiles
    (1, 200, 520, 4, 4, True),      # seqK > seqQ: bottom-right aligned causal window
    (1, 130, 77, 8, 8, False),      # non-causal, seqK < 64-key tile
    (1, 96, 40, 4, 2, True),        # seqQ > seqK: leading queries see no key -> zeros
])
@pytest.mark.parametrize("dt", [O.BF16, O.F16])
@pytest.mark.parametrize("d", [128, 64])
def test_prefill_mfma_shapes(backend, dt, d, b, sq, sk, h, kvh, causal):
    import puter_amd
    std = 1.0 / np.sqrt(d)
    q = encode(seeded(300 + sq, (b, sq, h * d), 0.0, std), dt)
    k = encode(seeded(301 + sk, (b, sk, kvh * d), 0.0, std), dt)
    v = encode(seeded(302 + sk, (b, sk, kvh * d)), dt)
    out = empty_dev((b, sq, h * d), np.uint16)
    cfg = puter_amd.MultiHeadAttentionConfig(h, d, causal, 0, 0.0, kvh)
    backend.MultiHeadAttentionBatched(cfg, to_dev(q), to_dev(k), to_dev(v), out, b, sq, sk, dt)
    got = decode(to_host(out, np.uint16), dt)
    O.set_threads(8)
    for i in range(b):
        ref = decode(O.mha(q[i], k[i], v[i], h, d, causal=causal, kv_heads=kvh, dtype=dt), dt)
        assert_close(got[i], ref, TOL[dt], elem_tol=None, what=f"prefill batch {i}")
        if causal and sq > sk:   # rows with no visible key are exactly zero, as softmax.go:50-56
            assert np.all(got[i][:sq - sk] == 0)


@pytest.mark.parametrize("b,sq,sk,h,kvh,causal,window", [
    (1, 1024, 1024, 8, 2, True, 128),   # sliding_window_attention's window: tile-aligned edge
    (2, 333, 333, 4, 1, True, 37),      # ragged edge inside tiles, partial tiles
    (1, 300, 300, 4, 4, True, 1),       # each query sees only itself
    (1, 200, 520, 4, 2, True, 200),     # seqK > seqQ: the edge trails the shifted diagonal
    (1, 96, 40, 4, 2, True, 20),        # seqQ > seqK: leading queries see no key -> zeros
    (1, 300, 77, 8, 8, False, 50),      # non-causal: queries past key 76 + 50 see no key
    (1, 700, 700, 4, 2, False, 300),    # non-causal, edge crosses several tiles per block
])
@pytest.mark.parametrize("dt", [O.BF16, O.F16, O.F32])
@pytest.mark.parametrize("d", [128, 64])
def test_prefill_mfma_window(backend, dt, d, b, sq, sk, h, kvh, causal, window):
    """Sliding-window prefill on the MFMA kernels (query q sees key k only if
    q - k < window, typed_compute.go:172) against the oracle; rows with no
    visible key are exactly zero.  f32 runs on the f32 MFMA kernel where the grid
    takes it (at least 24 blocks, or causal over at least 8 key tiles) and on the
    general kernel otherwise."""
    import puter_amd
    std = 1.0 / np.sqrt(d)
    q = encode(seeded(310 + sq, (b, sq, h * d), 0.0, std), dt)
    k = encode(seeded(311 + sk, (b, sk, kvh * d), 0.0, std), dt)
    v = encode(seeded(312 + sk, (b, sk, kvh * d)), dt)
    out = empty_dev((b, sq, h * d), NP[dt])
    cfg = puter_amd.MultiHeadAttentionConfig(h, d, causal, window, 0.0, kvh)
    backend.MultiHeadAttentionBatched(cfg, to_dev(q), to_dev(k), to_dev(v), out, b, sq, sk, dt)
    got = decode(to_host(out, NP[dt]), dt)
    O.set_threads(8)
    shift = sk - sq
    for i in range(b):
        ref = decode(O.mha(q[i], k[i], v[i], h, d, causal=causal, kv_heads=kvh, window=window, dtype=dt), dt)
        assert_close(got[i], ref, TOL[dt], elem_tol=None, what=f"window prefill batch {i}")
        for r in range(sq):
            hi = min(sk - 1, r + shift) if causal else sk - 1
            if max(0, r - window + 1) > hi:
                assert np.all(got[i][r] == 0), f"row {r} sees no key"


@pytest.mark.parametrize("b,sq,sk,h,kvh,causal,window,alibi", [
    (1, 512, 512, 8, 2, True, 0, 0.25),      # causal ALiBi, distant keys fade out
    (2, 333, 333, 4, 1, False, 0, 0.0625),   # non-causal: later keys gain, ragged tiles
    (1, 200, 520, 4, 2, True, 100, 0.5),     # seqK > seqQ with a window and ALiBi
    (1, 96, 40, 4, 4, True, 0, -0.125),      # negative slope; leading queries see no key
])
@pytest.mark.parametrize("dt", [O.BF16, O.F16, O.F32])
@pytest.mark.parametrize("d", [128, 64])
def test_prefill_mfma_alibi(backend, dt, d, b, sq, sk, h, kvh, causal, window, alibi):
    """ALiBi prefill on the MFMA kernels (score += slope * (k - q) on the scaled
    score, typed_compute.go:176-178; with or without a window) against the oracle."""
    import puter_amd
    std = 1.0 / np.sqrt(d)
    q = encode(seeded(330 + sq, (b, sq, h * d), 0.0, std), dt)
    k = encode(seeded(331 + sk, (b, sk, kvh * d), 0.0, std), dt)
    v = encode(seeded(332 + sk, (b, sk, kvh * d)), dt)
    out = empty_dev((b, sq, h * d), NP[dt])
    cfg = puter_amd.MultiHeadAttentionConfig(h, d, causal, window, alibi, kvh)
    backend.MultiHeadAttentionBatched(cfg, to_dev(q), to_dev(k), to_dev(v), out, b, sq, sk, dt)
    got = decode(to_host(out, NP[dt]), dt)
    O.set_threads(8)
    for i in range(b):
        ref = decode(O.mha(q[i], k[i], v[i], h, d, causal=causal, kv_heads=kvh, window=window, alibi=alibi,
                           dtype=dt), dt)
        assert_close(got[i], ref, TOL[dt], elem_tol=None, what=f"alibi prefill batch {i}")


@pytest.mark.parametrize("d", [128, 64])
def test_prefill_mfma_wide_window_is_no_window(backend, d):
    """A window wider than every query-key distance (seqQ or more) hides no key:
    the output equals the windowless call bit for bit."""
    import puter_amd
    dt, s, h, kvh = O.BF16, 777, 8, 2
    std = 1.0 / np.sqrt(d)
    q = to_dev(encode(seeded(320, (s, h * d), 0.0, std), dt))
    k = to_dev(encode(seeded(321, (s, kvh * d), 0.0, std), dt))
    v = to_dev(encode(seeded(322, (s, kvh * d)), dt))
    outs = []
    for causal in (True, False):
        for window in (0, s, 1 << 20):
            out = empty_dev((s, h * d), np.uint16)
            backend.MultiHeadAttention(puter_amd.MultiHeadAttentionConfig(h, d, causal, window, 0.0, kvh),
                                       q, k, v, out, s, s, dt)
            outs.append(to_host(out, np.uint16))
        assert np.array_equal(outs[-3], outs[-2]) and np.array_equal(outs[-3], outs[-1])


@pytest.mark.parametrize("dt", [O.F32, O.F16, O.BF16])
@pytest.mark.parametrize("sq,sk,d,vd,causal", [
    (37, 37, 64, 64, True),
    (20, 300, 48, 24, True),        # top-left causal with seqK > seqQ
    (300, 20, 32, 80, True),        # later rows see every key
    (65, 513, 128, 128, False),     # bf16 / f16 here take the MFMA kernel
    (200, 700, 128, 128, True),     # bf16 / f16 MFMA path, top-left causal
    (3, 5, 1000, 1000, False),      # wide rows, four output dims per thread
])
def test_scaled_dot_product_attention(backend, dt, sq, sk, d, vd, causal):
    import puter_amd
    std = 1.0 / np.sqrt(d) if dt != O.F32 else 0.25
    q = encode(seeded(500 + sq, (sq, d), 0.0, std), dt)
    k = encode(seeded(501 + sk, (sk, d), 0.0, std), dt)
    v = encode(seeded(502 + sk, (sk, vd)), dt)
    ref = decode(O.flash_attention(q, k, v, causal=causal, dtype=dt), dt)
    cfg = puter_amd.FlashAttentionConfig(64, causal)
    for fn in (backend.ScaledDotProductAttention, backend.FlashAttention):
        out = empty_dev((sq, vd), NP[dt])
        fn(cfg, to_dev(q), to_dev(k), to_dev(v), out, sq, sk, d, vd, dt)
        assert_close(decode(to_host(out, NP[dt]), dt), ref, TOL[dt],
                     elem_tol=1e-3 if dt == O.F32 else None, what="sdpa")


def out_dtype(kv_dt):
    """Query and output format of a paged decode: the pool's for f16 / bf16
    pools, bf16 for fp8 pools."""
    return O.F16 if kv_dt == O.F16 else O.BF16


def paged_case(seed, batch, ctx_lo, ctx_hi, ps, h, kvh, d, kv_dt):
    rng = np.random.default_rng(seed)
    ctx = rng.integers(ctx_lo, ctx_hi + 1, batch).astype(np.int32)
    npages = (ctx + ps - 1) // ps
    total = int(npages.sum())
    perm = rng.permutation(total).astype(np.int32)
    max_pages = int(npages.max())
    table = np.zeros((batch, max_pages), np.int32)
    at = 0
    for i in range(batch):
        table[i, :npages[i]] = perm[at:at + npages[i]]
        at += npages[i]
    q = O.from_f32(seeded(seed + 1, (batch, h * d)), out_dtype(kv_dt))
    kf = seeded(seed + 2, (total, ps, kvh, d))
    vf = seeded(seed + 3, (total, ps, kvh, d))
    if kv_dt in (O.BF16, O.F16):
        kp, vp, ks, vs = O.from_f32(kf, kv_dt), O.from_f32(vf, kv_dt), None, None
    else:
        ks = (np.abs(kf).reshape(-1, kvh, d).max(axis=(0, 2)) / 448.0).astype(np.float32)
        vs = (np.abs(vf).reshape(-1, kvh, d).max(axis=(0, 2)) / 448.0).astype(np.float32)
        kp = O.from_f32((kf / ks[None, None, :, None]).astype(np.float32), O.F8E4M3)
        vp = O.from_f32((vf / vs[None, None, :, None]).astype(np.float32), O.F8E4M3)
    return ctx, table, total, q, kp, vp, ks, vs


def run_paged_decode(backend, q, kp, vp, table, ctx, ps, total, h, kvh, d, kv_dt, ks, vs):
    """kp / vp: host arrays, or pools already on the device (torch tensors)."""
    batch = len(ctx)
    max_ctx = int(ctx.max())
    ws_bytes = backend.PagedDecodeWorkspaceBytes(batch, h, d, max_ctx)
    ws = empty_dev((ws_bytes // 4,), np.float32)
    out = empty_dev((batch, h * d), np.uint16)
    dev = lambda x: x if hasattr(x, "data_ptr") else to_dev(x)  # noqa: E731
    backend.PagedDecodeAttention(to_dev(q), dev(kp), dev(vp), to_dev(table), to_dev(ctx), batch,
                                 table.shape[1], ps, total, h, kvh, d, max_ctx,
                                 None if ks is None else to_dev(ks), None if vs is None else to_dev(vs),
                                 kv_dt, out, ws, ws_bytes)
    return to_host(out, np.uint16)


@pytest.mark.parametrize("kv_dt", [O.BF16, O.F16, O.F8E4M3])
@pytest.mark.parametrize("batch,lo,hi,ps", [(3, 1, 40, 16), (4, 500, 1300, 16), (2, 256, 256, 16)])
def test_paged_decode(backend, kv_dt, batch, lo, hi, ps):
    h, kvh, d = 32, 8, 128
    ctx, table, total, q, kp, vp, ks, vs = paged_case(batch * 100 + lo, batch, lo, hi, ps, h, kvh, d, kv_dt)
    ref = O.paged_decode(q, kp, vp, table, ctx, ps, h, kvh, d, kv_dt, ks, vs)
    out = run_paged_decode(backend, q, kp, vp, table, ctx, ps, total, h, kvh, d, kv_dt, ks, vs)
    od = out_dtype(kv_dt)
    assert_close(O.to_f32(out, od), O.to_f32(ref, od), TOL[od], elem_tol=None, what="paged decode")


@pytest.mark.parametrize("kv_dt", [O.BF16, O.F16, O.F8E4M3])
def test_paged_decode_pool_beyond_4gib(backend, kv_dt):
    """Pools of more than 4 GiB take 64-bit row offsets (smaller ones 32-bit):
    sequences whose pages lie past the 4 GiB mark of both pools, checked
    against the oracle on a compact copy of those pages."""
    import torch
    h, kvh, d, ps = 32, 8, 128, 16
    es = 1 if kv_dt == O.F8E4M3 else 2
    row_bytes = kvh * d * es
    pages = (1 << 32) // (ps * row_bytes) + 2048           # just past 4 GiB per pool
    ctx, table, total, q, kp, vp, ks, vs = paged_case(77, 2, 150, 400, ps, h, kvh, d, kv_dt)
    far = (pages - total + np.arange(total)).astype(np.int32)   # compact page i -> pool page far[i]
    big_table = far[table]
    tdt = torch.uint8 if kv_dt == O.F8E4M3 else torch.int16
    npd = np.uint8 if kv_dt == O.F8E4M3 else np.int16
    kpool = torch.zeros((pages, ps, kvh, d), dtype=tdt, device="cuda")
    vpool = torch.zeros((pages, ps, kvh, d), dtype=tdt, device="cuda")
    idx = torch.from_numpy(far.astype(np.int64)).cuda()
    kpool[idx] = torch.from_numpy(kp.view(npd)).cuda()
    vpool[idx] = torch.from_numpy(vp.view(npd)).cuda()
    ref = O.paged_decode(q, kp, vp, table, ctx, ps, h, kvh, d, kv_dt, ks, vs)
    out = run_paged_decode(backend, q, kpool, vpool, big_table, ctx, ps, pages, h, kvh, d, kv_dt, ks, vs)
    del kpool, vpool
    torch.cuda.empty_cache()
    od = out_dtype(kv_dt)
    assert_close(O.to_f32(out, od), O.to_f32(ref, od), TOL[O.BF16], elem_tol=None, what="paged decode > 4 GiB")


@pytest.mark.parametrize("kvh", [1, 2])
def test_paged_decode_fp8_value_codes_exact(backend, kvh):
    """One live token per sequence: its softmax weight is exactly 1, so the output
    is the token's V row widened from fp8 and narrowed to bf16, bit for bit.  Two
    sequences hold all 256 E4M3 codes in their V rows (NaN codes give NaN), which
    pins the kernel's fp8 -> bf16 widening code by code (convert/fp8_f32.go).
    With two kv heads (the kernel that takes a pair of heads per block) head 1
    holds the codes in reverse order, so a head or dim placed wrongly fails."""
    h = kvh
    d, ps = 128, 16
    ctx = np.array([1, 1], np.int32)
    table = np.array([[0], [1]], np.int32)
    q = O.from_f32(seeded(5, (2, h * d)), O.BF16)
    kp = np.zeros((2, ps, kvh, d), np.uint8)
    vp = np.zeros((2, ps, kvh, d), np.uint8)
    codes = np.arange(256, dtype=np.uint8)
    per_head = [codes, codes[::-1]]
    for hh in range(kvh):
        vp[0, 0, hh] = per_head[hh][:128]
        vp[1, 0, hh] = per_head[hh][128:]
    ks = vs = np.ones(kvh, np.float32)
    out = run_paged_decode(backend, q, kp, vp, table, ctx, ps, 2, h, kvh, d, O.F8E4M3, ks, vs)
    got = O.to_f32(out.reshape(2, h, d), O.BF16)
    for hh in range(kvh):
        want = O.to_f32(per_head[hh], O.F8E4M3).reshape(2, d)
        g = got[:, hh]
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(g), nan), hh
        assert np.array_equal(g[~nan], want[~nan]), hh   # -0 sums to +0, as the reference's 0 + 1 * v does


# group sizes 1, 2, 4, 8 (compiled in) and 3, 5, 7, 16 (read at run time); kv head
# counts 1, 2, 3, 4, 8 (the XCD grouping of kv heads falls back to smaller groups,
# down to one, when it does not divide them); page sizes that do not divide a
# wave's 64 tokens
@pytest.mark.parametrize("kv_dt", [O.BF16, O.F16, O.F8E4M3])
@pytest.mark.parametrize("h,kvh", [(8, 8), (8, 4), (16, 2), (4, 1), (6, 3), (32, 2), (7, 1), (15, 3),
                                   (12, 4)])
@pytest.mark.parametrize("ps,lo,hi", [(1, 1, 70), (5, 30, 300), (32, 200, 700)])
def test_paged_decode_groups_pages(backend, kv_dt, h, kvh, ps, lo, hi):
    d, batch = 128, 3
    ctx, table, total, q, kp, vp, ks, vs = paged_case(7000 + 31 * h + kvh + ps, batch, lo, hi, ps, h, kvh, d, kv_dt)
    ref = O.paged_decode(q, kp, vp, table, ctx, ps, h, kvh, d, kv_dt, ks, vs)
    out = run_paged_decode(backend, q, kp, vp, table, ctx, ps, total, h, kvh, d, kv_dt, ks, vs)
    od = out_dtype(kv_dt)
    assert_close(O.to_f32(out, od), O.to_f32(ref, od), TOL[od],
                 elem_tol=None, what="paged decode G=%d ps=%d" % (h // kvh, ps))


@pytest.mark.parametrize("kv_dt", [O.BF16, O.F16, O.F8E4M3])
def test_paged_decode_bad_page_ids_are_masked(backend, kv_dt):
    """A token whose page id is outside [0, num_pages) is masked: the result
    equals attention over the same sequence with that page removed."""
    h, kvh, d, ps, batch = 16, 4, 128, 16, 2
    ctx, table, total, q, kp, vp, ks, vs = paged_case(8101, batch, 300, 600, ps, h, kvh, d, kv_dt)
    bad = table.copy()
    ref_table = np.zeros_like(table)
    ref_ctx = ctx.copy()
    for i in range(batch):
        npg = (int(ctx[i]) + ps - 1) // ps
        j = 3 + i                               # a full page inside the context
        bad[i, j] = -1 if i == 0 else total + 5
        keep = [table[i, c] for c in range(npg) if c != j]
        ref_table[i, :len(keep)] = keep
        ref_ctx[i] = ctx[i] - ps
    ref = O.paged_decode(q, kp, vp, ref_table, ref_ctx, ps, h, kvh, d, kv_dt, ks, vs)
    out = run_paged_decode(backend, q, kp, vp, bad, ctx, ps, total, h, kvh, d, kv_dt, ks, vs)
    od = out_dtype(kv_dt)
    assert_close(O.to_f32(out, od), O.to_f32(ref, od), TOL[od],
                 elem_tol=None, what="paged decode, bad page ids")


@pytest.mark.parametrize("kv_dt", [O.BF16, O.F8E4M3])
@pytest.mark.parametrize("batch,lo,hi", [(70, 1, 600), (256, 1, 40), (300, 1, 40)])
def test_paged_decode_empty_sequences_and_batches(backend, kv_dt, batch, lo, hi):
    """Sequences of zero context among live ones in batches of 70 (fp8 pools number
    the live (sequence, split) pairs with a prefix sum over 64 sequences at a time:
    two passes), 256 (four passes, the largest batch numbered so) and 300 (past 256
    sequences the plain block order).  A sequence with
    no key has no reference output (the reference's gather yields no rows and its
    zero-size attention call returns early); this extension writes zeros for it.  The
    live sequences match the oracle run on them alone."""
    h, kvh, d, ps = 8, 2, 128, 16
    ctx, table, total, q, kp, vp, ks, vs = paged_case(8300 + batch, batch, lo, hi, ps, h, kvh, d, kv_dt)
    empty = [0, 5, 63, 64, batch - 1]
    ctx[empty] = 0
    live = ctx > 0
    ref = O.paged_decode(q[live], kp, vp, table[live], ctx[live], ps, h, kvh, d, kv_dt, ks, vs)
    out = run_paged_decode(backend, q, kp, vp, table, ctx, ps, total, h, kvh, d, kv_dt, ks, vs)
    od = out_dtype(kv_dt)
    got = O.to_f32(out, od).reshape(batch, h * d)
    assert not got[~live].any()
    assert_close(got[live], O.to_f32(ref, od).reshape(-1, h * d), TOL[od], elem_tol=None,
                 what="paged decode, empty sequences")


def test_paged_decode_empty_pool(backend):
    """num_pages = 0: every page id is out of range, every token masked, output 0."""
    h, kvh, d, ps, batch = 8, 2, 128, 16, 2
    ctx = np.array([17, 40], np.int32)
    table = np.zeros((batch, 3), np.int32)
    q = O.from_f32(seeded(8201, (batch, h * d)), O.BF16)
    pool = np.zeros((1, ps, kvh, d), np.uint16)   # a valid buffer the kernel must not depend on
    out = run_paged_decode(backend, q, pool, pool, table, ctx, ps, 0, h, kvh, d, O.BF16, None, None)
    assert not out.any()


def test_paged_decode_rejects_misaligned_workspace(backend):
    """The split partials are stored as 16-byte vectors: a workspace view that is
    not 16-byte aligned is rejected before any launch."""
    import puter_amd
    h, kvh, d, ps = 8, 2, 128, 16
    ctx, table, total, q, kp, vp, _, _ = paged_case(8301, 2, 20, 40, ps, h, kvh, d, O.BF16)
    ws_bytes = backend.PagedDecodeWorkspaceBytes(2, h, d, int(ctx.max()))
    ws = empty_dev((ws_bytes // 4 + 4,), np.float32)
    out = empty_dev((2, h * d), np.uint16)
    with pytest.raises(puter_amd.PuterError):
        backend.PagedDecodeAttention(to_dev(q), to_dev(kp), to_dev(vp), to_dev(table), to_dev(ctx), 2,
                                     table.shape[1], ps, total, h, kvh, d, int(ctx.max()), None, None,
                                     O.BF16, out, ws[1:], ws_bytes)


def test_matmul_f32(backend):
    for rows, inner, cols in [(128, 512, 512), (7, 13, 5), (65, 64, 130)]:
        a = seeded(rows, (rows, inner))
        b = seeded(cols + 1, (inner, cols), 0.0, 0.02)
        ref = O.matmul_f32(a, b)
        out = empty_dev((rows, cols), np.float32)
        backend.Matmul(out, to_dev(a), to_dev(b), rows, inner, cols, O.F32)
        assert_close(to_host(out, np.float32), ref, TOL[O.F32], elem_tol=1e-3, what="matmul")
