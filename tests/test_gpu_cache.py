"""GPU tests of the latent KV cache (replacement of KVCache,
src/model.rs:86-105): append == concatenation, ragged appends, capacity
errors, Clone, bf16 round-to-nearest-even on the device."""
import numpy as np
import pytest

import oracle as O
from helpers import bf16_bits

pytestmark = pytest.mark.gpu


def test_append_is_concatenation_f32(qmla_gpu):
    q = qmla_gpu
    cache = q.KVCache([10, 10, 10], 16, 8, q.F32)
    a = O.normal((3, 4, 24), 1)
    b = O.normal((3, 2, 24), 2)
    cache.append(q.DeviceBuffer.from_numpy(a), 3, 4)
    cache.append(q.DeviceBuffer.from_numpy(b), 3, 2)
    assert list(cache.lengths()) == [6, 6, 6]
    pool = cache.read_rows().reshape(3, 10, 24)
    np.testing.assert_array_equal(pool[:, :6], np.concatenate([a, b], 1))


def test_append_bf16_rounds_to_nearest_even(qmla_gpu):
    q = qmla_gpu
    cache = q.KVCache([8], 576 - 64, 64, q.BF16)
    x = O.normal((1, 8, 576), 3)
    x[0, 0, :4] = [1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 1.0 + 2 ** -8 + 2 ** -20]
    cache.append(q.DeviceBuffer.from_numpy(x), 1, 8)
    np.testing.assert_array_equal(cache.read_rows().reshape(1, 8, 576), bf16_bits(x))
    np.testing.assert_array_equal(cache.read_rows()[0, :4], [0x3F80, 0x3F82, 0xC020, 0x3F81])


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
    assert list(offs) == [0, 5, 8]
    np.testing.assert_array_equal(pool[0:5], r0[0])
    np.testing.assert_array_equal(pool[8:10], r2[0])
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
    """Live rows of sequence i (host copy), wherever the pool holds them."""
    pool, offs, lens = cache.read_rows(), cache.offsets(), cache.lengths()
    return pool[offs[i]:offs[i] + lens[i]]


def test_reserve_keeps_rows_and_moves_offsets(qmla_gpu):
    q = qmla_gpu
    cache = q.KVCache([3, 4, 2], 8, 8, q.BF16)
    a = [O.normal((1, n, 16), 40 + i) for i, n in enumerate((3, 1, 2))]
    for i, x in enumerate(a):
        cache.append_seq(i, q.DeviceBuffer.from_numpy(x), x.shape[1])
    cache.reserve([10, 2, 5])            # sequence 1 keeps its capacity of 4
    assert list(cache.capacity()) == [10, 4, 5]
    assert list(cache.offsets()) == [0, 10, 14]
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
