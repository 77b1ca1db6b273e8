"""GPU test of qmla_decode_absorbed_noalloc, the allocation-free form of
qmla_decode_absorbed: its split partials live in a static per-device array
instead of a caller workspace.  Both entry points run the same kernels and
plan, so their outputs must be bit-identical; two calls in a row (the
second smaller) check that nothing stale from the first leaks into it."""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from helpers import rel_err

pytestmark = pytest.mark.gpu


def _cache(q, lens, dtype, seed):
    lens = np.asarray(lens, np.int32)
    cache = q.KVCache(lens, 512, 64, dtype)
    rows = O.normal((int(lens.sum()), 576), seed)
    cache.write_pool(O.to_bf16_bits(rows) if dtype == q.BF16 else rows)
    cache.set_lengths(lens)
    return cache


def _both(q, cache, batch, rows, seed):
    ql = q.DeviceBuffer.from_numpy(O.normal((batch, rows, 512), seed))
    qr = q.DeviceBuffer.from_numpy(O.normal((batch, rows, 64), seed + 1))
    dd = q.DecodeDims(batch, rows, 512, 64)
    scale = 192 ** -0.5
    outs = []
    for noalloc in (False, True):
        out = q.DeviceBuffer(batch * rows * 512 * 4)
        lse = q.DeviceBuffer(batch * rows * 4)
        if noalloc:
            st = q.lib().qmla_decode_absorbed_noalloc(C.byref(dd), cache.handle, q.F32, ql.ptr, qr.ptr, scale,
                                                      out.ptr, lse.ptr, None)
        else:
            wsb = q.decode_workspace_bytes(cache, batch, rows)
            ws = q.DeviceBuffer(wsb)
            st = q.lib().qmla_decode_absorbed(C.byref(dd), cache.handle, q.F32, ql.ptr, qr.ptr, scale, out.ptr,
                                              lse.ptr, ws.ptr, wsb, None)
        assert st == 0, q.lib().qmla_last_error()
        q.check(q.lib().qmla_stream_synchronize(None))
        outs.append((out.to_numpy(np.float32, (batch, rows, 512)), lse.to_numpy(np.float32, (batch, rows))))
    return outs


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_noalloc_decode_equals_the_workspace_entry_point(qmla_gpu, dt):
    q = qmla_gpu
    dtype = q.BF16 if dt == "bf16" else q.F32
    # call 1: 8 ragged sequences, 128 query rows (4-wave core, several splits each)
    lens1 = [4097, 1, 9000, 0, 2500, 777, 6000, 33]
    c1 = _cache(q, lens1, dtype, 40)
    (a_o, a_l), (b_o, b_l) = _both(q, c1, len(lens1), 128, 41)
    print(f"[{dt}] call 1: batch 8, 128 rows", flush=True)
    assert np.array_equal(a_o, b_o) and np.array_equal(a_l, b_l)
    # the result is the decode itself, not just self-consistent
    pool = c1.read_rows()
    pool = O.bf16_bits_to_f32(pool) if dtype == q.BF16 else pool
    offs, lens = c1.offsets(), np.asarray(lens1, np.int32)
    ql = O.normal((8, 128, 512), 41)
    qr = O.normal((8, 128, 64), 42)
    if dtype == q.BF16:
        ql, qr = O.round_bf16(ql), O.round_bf16(qr)
    ref, _ = O.decode_absorbed(ql[:3], qr[:3], pool, offs[:3], lens[:3], 192 ** -0.5)
    assert rel_err(b_o[:3], ref) < (2e-2 if dtype == q.BF16 else 1e-4)
    # call 2, smaller: 3 sequences, 16 query rows (narrow core for bf16)
    lens2 = [300, 2049, 5]
    c2 = _cache(q, lens2, dtype, 50)
    (a_o, a_l), (b_o, b_l) = _both(q, c2, len(lens2), 16, 51)
    print(f"[{dt}] call 2: batch 3, 16 rows", flush=True)
    assert np.array_equal(a_o, b_o) and np.array_equal(a_l, b_l)


def test_noalloc_decode_rejects_a_workspace_beyond_its_scratch(qmla_gpu):
    """400 sequences x 128 rows need more than the 48 MiB scratch: the call
    fails before launching anything and leaves the output untouched."""
    q = qmla_gpu
    c = _cache(q, [1] * 400, q.BF16, 60)
    assert q.decode_workspace_bytes(c, 400, 128) > (48 << 20)
    dd = q.DecodeDims(400, 128, 512, 64)
    ql = q.DeviceBuffer(400 * 128 * 512 * 4)
    qr = q.DeviceBuffer(400 * 128 * 64 * 4)
    out = q.DeviceBuffer.from_numpy(np.full((400, 128, 512), 7.0, np.float32))
    st = q.lib().qmla_decode_absorbed_noalloc(C.byref(dd), c.handle, q.F32, ql.ptr, qr.ptr, 0.1, out.ptr, None,
                                              None)
    assert st == 3 and b"allocation-free" in q.lib().qmla_last_error()
    assert (out.to_numpy(np.float32, (400, 128, 512)) == 7.0).all()
