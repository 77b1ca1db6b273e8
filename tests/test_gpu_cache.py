"""GPU tests of the latent KV cache (replacement of KVCache,
src/model.rs:86-105): append == concatenation, ragged appends, capacity
errors, Clone, bf16 round-to-nearest-even on the device."""
import numpy as np
import pytest

import oracle as O
from helpers import bf16_bits, bf16_to_f32

pytestmark = pytest.mark.gpu


def test_append_is_concatenation_f32(qmla_gpu):
    q = qmla_gpu
    cache = q.KVCache([10, 10, 10], 16, 8, q.F32)
    a = O.normal((3, 4, 24), 1)
    b = O.normal((3, 2, 24), 2)
    cache.append(q.DeviceBuffer.from_numpy(a), 3, 4)
    cache.append(q.DeviceBuffer.from_numpy(b), 3, 2)
    assert list(cache.lengths()) == [6, 6, 6]
    got = np.stack([cache.read_seq(i) for i in range(3)])
    np.testing.assert_array_equal(got, np.concatenate([a, b], 1))


def test_append_bf16_rounds_to_nearest_even(qmla_gpu):
    q = qmla_gpu
    cache = q.KVCache([8], 576 - 64, 64, q.BF16)
    x = O.normal((1, 8, 576), 3)
    x[0, 0, :4] = [1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 1.0 + 2 ** -8 + 2 ** -20]
    cache.append(q.DeviceBuffer.from_numpy(x), 1, 8)
    np.testing.assert_array_equal(cache.read_seq(0), bf16_bits(x[0]))
    np.testing.assert_array_equal(cache.read_seq(0)[0, :4], [0x3F80, 0x3F82, 0xC020, 0x3F81])


def test_ragged_append_and_set_lengths(qmla_gpu):
    q = qmla_gpu
    cache = q.KVCache([5, 3, 7], 8, 8, q.F32)
    r0 = O.normal((1, 5, 16), 4)
    r2 = O.normal((1, 2, 16), 5)
    cache.append_seq(0, q.DeviceBuffer.from_numpy(r0), 5)
    cache.append_seq(2, q.DeviceBuffer.from_numpy(r2), 2)
    assert list(cache.lengths()) == [5, 0, 2]
    pool = cache.read_rows()
    offs = cache.offsets()
    assert list(offs) == [0, 256, 512]     # one 256-row page each, in order
    np.testing.assert_array_equal(pool[0:5], r0[0])
    np.testing.assert_array_equal(pool[512:514], r2[0])
    np.testing.assert_array_equal(cache.read_seq(2), r2[0])
    cache.set_lengths([1, 3, 7])
    assert list(cache.lengths()) == [1, 3, 7]


def test_capacity_and_shape_errors(qmla_gpu):
    q = qmla_gpu
    cache = q.KVCache([4, 4], 8, 8, q.F32)
    rows = q.DeviceBuffer.from_numpy(np.zeros((2, 5, 16), np.float32))
    with pytest.raises(q.QmlaError) as e:
        cache.append(rows, 2, 5)
    assert e.value.status == 6 and "capacity" in str(e.value)
    with pytest.raises(q.QmlaError) as e:
        cache.append(rows, 3, 1)
    assert e.value.status == 2
    with pytest.raises(q.QmlaError):
        cache.set_lengths([5, 0])
    assert list(cache.lengths()) == [0, 0]   # failed calls changed nothing


def test_clone_is_deep(qmla_gpu):
    q = qmla_gpu
    cache = q.KVCache([6], 8, 8, q.BF16)
    a = O.normal((1, 3, 16), 6)
    cache.append(q.DeviceBuffer.from_numpy(a), 1, 3)
    c2 = cache.clone()
    b = O.normal((1, 2, 16), 7)
    cache.append(q.DeviceBuffer.from_numpy(b), 1, 2)
    assert list(c2.lengths()) == [3] and list(cache.lengths()) == [5]
    np.testing.assert_array_equal(c2.read_rows()[:3], bf16_bits(a[0]))
    np.testing.assert_array_equal(cache.read_rows()[:5], bf16_bits(np.concatenate([a[0], b[0]])))


def _seq_rows(cache, i):
    """Live rows of sequence i (host copy), wherever its pages are."""
    return cache.read_seq(i)


def test_reserve_keeps_rows_in_place(qmla_gpu):
    q = qmla_gpu
    cache = q.KVCache([3, 4, 2], 8, 8, q.BF16)
    a = [O.normal((1, n, 16), 40 + i) for i, n in enumerate((3, 1, 2))]
    for i, x in enumerate(a):
        cache.append_seq(i, q.DeviceBuffer.from_numpy(x), x.shape[1])
    offs = list(cache.offsets())
    cache.reserve([10, 2, 5])            # sequence 1 keeps its capacity of 4
    assert list(cache.capacity()) == [10, 4, 5]
    assert list(cache.offsets()) == offs  # no row moved
    assert list(cache.lengths()) == [3, 1, 2]
    for i, x in enumerate(a):
        np.testing.assert_array_equal(_seq_rows(cache, i), bf16_bits(x[0]))
    more = O.normal((1, 7, 16), 50)
    cache.append_seq(0, q.DeviceBuffer.from_numpy(more), 7)   # fits only after the reserve
    np.testing.assert_array_equal(_seq_rows(cache, 0), bf16_bits(np.concatenate([a[0][0], more[0]])))
    with pytest.raises(q.QmlaError) as e:
        cache.reserve([-1, 0, 0])
    assert e.value.status == 2
    assert list(cache.capacity()) == [10, 4, 5]


def test_growth_mode_append_never_runs_out(qmla_gpu):
    """With growth on, appends behave like Tensor::cat (src/model.rs:99-104):
    any number of rows fit, and decode over the grown cache matches the
    oracle on the concatenated rows."""
    q = qmla_gpu
    cache = q.KVCache([2, 2], 64, 16, q.F32, grow=True)
    chunks = [O.normal((2, n, 80), 60 + k) for k, n in enumerate((2, 5, 1, 30, 3))]
    for x in chunks:
        cache.append(q.DeviceBuffer.from_numpy(x), 2, x.shape[1])
    full = np.concatenate(chunks, 1)
    assert list(cache.lengths()) == [41, 41]
    assert all(c >= 41 for c in cache.capacity())
    for i in range(2):
        np.testing.assert_array_equal(_seq_rows(cache, i), full[i])
    c2 = cache.clone()                   # clones keep the growth mode
    c2.append(q.DeviceBuffer.from_numpy(O.normal((2, 40, 80), 70)), 2, 40)
    assert list(c2.lengths()) == [81, 81]
    ql, qr = O.normal((2, 4, 64), 71), O.normal((2, 4, 16), 72)
    out = q.DeviceBuffer(2 * 4 * 64 * 4)
    ws_n = q.decode_workspace_bytes(cache, 2, 4)
    ws = q.DeviceBuffer(ws_n)
    q.decode_absorbed(cache, 2, 4, q.DeviceBuffer.from_numpy(ql), q.DeviceBuffer.from_numpy(qr), 0.2,
                      out, workspace=ws, workspace_bytes=ws_n)
    got = out.to_numpy(np.float32, (2, 4, 64))
    ref, _ = O.decode_absorbed(ql, qr, full.reshape(-1, 80), np.array([0, 41], np.int64),
                               np.array([41, 41], np.int32), 0.2)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-4


def _scattered_cache(q, dtype, r, dr, chunks, seqs, page_rows=32, seed=300):
    """Growth-mode cache created empty; sequences append ragged chunks in
    turn, so each sequence's pages come from several chunks of the pool and
    are interleaved with the other sequences' pages.  Returns the cache and
    the rows each sequence holds (as stored: bf16 bits for a bf16 cache)."""
    cache = q.KVCache([0] * seqs, r, dr, dtype, grow=True, page_rows=page_rows)
    held = [[] for _ in range(seqs)]
    for k, n in enumerate(chunks):
        for i in range(seqs):
            m = n + 3 * i
            x = O.normal((1, m, r + dr), seed + 17 * k + i)
            cache.append_seq(i, q.DeviceBuffer.from_numpy(x), m)
            held[i].append(bf16_bits(x[0]) if dtype == q.BF16 else x[0])
    return cache, [np.concatenate(h) for h in held]


@pytest.mark.parametrize("dtype_name", ["f32", "bf16"])
def test_growth_takes_pages_without_moving_rows(qmla_gpu, dtype_name):
    """Growth never copies: every sequence's rows stay where they were
    written while the pool grows by chunks and pages interleave."""
    q = qmla_gpu
    dtype = q.F32 if dtype_name == "f32" else q.BF16
    cache, held = _scattered_cache(q, dtype, 64, 16, (5, 40, 1, 70, 33), 3)
    lens = [h.shape[0] for h in held]
    assert list(cache.lengths()) == lens
    d = cache.describe()
    assert d.contiguous == 0 and d.page_rows == 32
    with pytest.raises(q.QmlaError):
        cache.read_rows()                # no single chunk describes the rows any more
    table = cache.page_table()
    used = []
    for i, n in enumerate(lens):
        npages = -(-n // 32)
        used += list(table[i, :npages])
        assert cache.capacity()[i] >= n
        np.testing.assert_array_equal(cache.read_seq(i), held[i])
    assert len(set(used)) == len(used) and 0 not in used      # no page shared or missing
    pool_rows, free_rows = cache.pool_info()
    assert pool_rows >= sum(-(-n // 32) * 32 for n in lens) and free_rows % 32 == 0


def test_trim_returns_pages_and_growth_reuses_them(qmla_gpu):
    q = qmla_gpu
    cache = q.KVCache([0, 0], 64, 16, q.F32, grow=True, page_rows=32, pool_rows=256)
    pool0, free0 = cache.pool_info()
    assert (pool0, free0) == (256, 256)
    a = O.normal((1, 100, 80), 1)
    cache.append_seq(0, q.DeviceBuffer.from_numpy(a), 100)          # 4 pages from the free list
    assert cache.pool_info() == (256, 128)
    cache.set_lengths([10, 0])
    cache.trim()                                                     # keeps 1 page
    assert cache.pool_info() == (256, 224) and list(cache.capacity()) == [32, 0]
    b = O.normal((1, 200, 80), 2)
    cache.append_seq(1, q.DeviceBuffer.from_numpy(b), 200)          # 7 pages, no new chunk
    assert cache.pool_info() == (256, 0)
    np.testing.assert_array_equal(cache.read_seq(0), a[0, :10])
    np.testing.assert_array_equal(cache.read_seq(1), b[0])
    cache.set_growth(False)
    with pytest.raises(q.QmlaError) as e:                            # capacity is 224 rows
        cache.append_seq(1, q.DeviceBuffer.from_numpy(O.normal((1, 25, 80), 3)), 25)
    assert e.value.status == 6
    cache.reserve_pool(64)                                           # allocates outside the loop
    assert cache.pool_info()[1] >= 64


def test_growth_stops_at_max_len_and_changes_nothing(qmla_gpu):
    q = qmla_gpu
    cache = q.KVCache([0], 64, 16, q.F32, grow=True, page_rows=32, max_len=64)
    cache.append_seq(0, q.DeviceBuffer.from_numpy(O.normal((1, 60, 80), 4)), 60)
    before = (cache.pool_info(), list(cache.capacity()), list(cache.lengths()))
    with pytest.raises(q.QmlaError) as e:
        cache.append_seq(0, q.DeviceBuffer.from_numpy(O.normal((1, 5, 80), 5)), 5)
    assert e.value.status == 6 and "maximum length" in str(e.value)
    assert (cache.pool_info(), list(cache.capacity()), list(cache.lengths())) == before


@pytest.mark.parametrize("case", [
    # dtype, r, dr, rows, splits
    ("f32", 64, 16, 4, 0),
    ("f32", 512, 64, 16, 5),
    ("bf16", 64, 16, 16, 0),
    ("bf16", 64, 16, 40, 3),
    ("bf16", 512, 64, 16, 0),     # narrow MFMA path
    ("bf16", 512, 64, 16, 64),
    ("bf16", 512, 64, 128, 0),    # wide MFMA path
    ("bf16", 512, 64, 128, 1),
    ("bf16", 512, 64, 128, 11),
])
def test_decode_over_scattered_pages(qmla_gpu, case):
    """Absorbed decode over 32-row pages scattered across the pool equals the
    oracle on the concatenated rows: every 32-token tile reads its own page,
    and pieces cut sequences only at tile boundaries, for any split count."""
    q = qmla_gpu
    dt, r, dr, rows_m, splits = case
    dtype = q.F32 if dt == "f32" else q.BF16
    cache, held = _scattered_cache(q, dtype, r, dr, (33, 2, 64, 31, 97), 4, seed=500 + r)
    lens = np.array([h.shape[0] for h in held], np.int32)
    flat = np.concatenate(held)
    flat = bf16_to_f32(flat) if dtype == q.BF16 else flat
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    ql, qr = O.normal((4, rows_m, r), 61), O.normal((4, rows_m, dr), 62)
    s = (r // 4 + dr) ** -0.5
    q_dtype = q.BF16 if dtype == q.BF16 else q.F32
    qa, qb = (bf16_bits(ql), bf16_bits(qr)) if dtype == q.BF16 else (ql, qr)
    out, lse = q.decode_numpy(cache, qa, qb, s, splits=splits, q_dtype=q_dtype)
    ref, rlse = O.decode_absorbed(bf16_to_f32(qa) if dtype == q.BF16 else ql,
                                  bf16_to_f32(qb) if dtype == q.BF16 else qr, flat, offs, lens, s)
    tol = 1e-4 if dtype == q.F32 else 2e-2
    err = np.abs(out - ref).max() / np.abs(ref).max()
    print(f"{case} lens={list(lens)} rel_err={err:.2e}")
    assert err < tol
    np.testing.assert_allclose(lse, rlse, atol=tol)


def test_clone_of_scattered_cache_is_deep_and_packed(qmla_gpu):
    """A clone of a cache whose pages are scattered holds the same rows per
    sequence, packed in order into one chunk, and is independent of it."""
    q = qmla_gpu
    cache, held = _scattered_cache(q, q.BF16, 64, 16, (5, 40, 1, 70, 33), 3)
    c2 = cache.clone()
    assert c2.describe().contiguous == 1
    assert list(c2.lengths()) == list(cache.lengths())
    assert list(c2.capacity()) == list(cache.capacity())
    for i in range(3):
        np.testing.assert_array_equal(c2.read_seq(i), held[i])
    more = O.normal((1, 50, 80), 9)
    cache.append_seq(0, q.DeviceBuffer.from_numpy(more), 50)
    np.testing.assert_array_equal(c2.read_seq(0), held[0])
    np.testing.assert_array_equal(cache.read_seq(0), np.concatenate([held[0], bf16_bits(more[0])]))


@pytest.mark.parametrize("page_rows", [64, 1024])
def test_decode_over_other_page_sizes(qmla_gpu, page_rows):
    """The same scattered-pages decode with 64- and 1024-row pages (the tile
    and its page share a 32-row alignment for every power-of-two page)."""
    q = qmla_gpu
    cache, held = _scattered_cache(q, q.BF16, 512, 64, (33, 300, 64, 1111), 4, page_rows=page_rows,
                                   seed=900 + page_rows)
    lens = np.array([h.shape[0] for h in held], np.int32)
    flat = bf16_to_f32(np.concatenate(held))
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    for rows_m in (16, 128):
        ql, qr = O.normal((4, rows_m, 512), 63), O.normal((4, rows_m, 64), 64)
        out, lse = q.decode_numpy(cache, bf16_bits(ql), bf16_bits(qr), 192 ** -0.5, q_dtype=q.BF16)
        ref, rlse = O.decode_absorbed(bf16_to_f32(bf16_bits(ql)), bf16_to_f32(bf16_bits(qr)), flat,
                                      offs, lens, 192 ** -0.5)
        err = np.abs(out - ref).max() / np.abs(ref).max()
        print(f"page_rows={page_rows} rows={rows_m} lens={list(lens)} rel_err={err:.2e}")
        assert err < 2e-2
        np.testing.assert_allclose(lse, rlse, atol=2e-2)


def test_trim_then_regrow_and_decode(qmla_gpu):
    """Truncate every sequence, return the spare pages, regrow with new rows:
    pages freed by one sequence are reused by another, and the decode sees
    exactly the rows each sequence now holds."""
    q = qmla_gpu
    cache, held = _scattered_cache(q, q.F32, 64, 16, (40, 70), 3)
    keep = [10, 33, 0]
    cache.set_lengths(keep)
    cache.trim()
    pool, free = cache.pool_info()
    assert free > 0
    new = [O.normal((1, n, 80), 70 + i) for i, n in enumerate((90, 3, 150))]
    for i, x in enumerate(new):
        cache.append_seq(i, q.DeviceBuffer.from_numpy(x), x.shape[1])
    assert cache.pool_info()[0] == pool            # no new chunk: freed pages reused
    rows = [np.concatenate([held[i][:keep[i]], new[i][0]]) for i in range(3)]
    for i in range(3):
        np.testing.assert_array_equal(cache.read_seq(i), rows[i])
    lens = np.array([r.shape[0] for r in rows], np.int32)
    offs = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    ql, qr = O.normal((3, 4, 64), 81), O.normal((3, 4, 16), 82)
    out, lse = q.decode_numpy(cache, ql, qr, 0.15)
    ref, rlse = O.decode_absorbed(ql, qr, np.concatenate(rows), offs, lens, 0.15)
    assert np.abs(out - ref).max() / np.abs(ref).max() < 1e-4
