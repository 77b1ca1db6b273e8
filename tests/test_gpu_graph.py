"""HIP graph capture of the entry points a serving loop replays: the
absorbed decode (with a workspace and allocation-free), the 2-bit MoE layer,
the zero fill and a prefill call without keys.  A captured call records kernel nodes only (no
memset or copy nodes), and every replay reproduces the eager result bit for
bit, with eager work and synchronisations between the replays.

The graph calls go to the HIP runtime libqmla.so itself loaded (RTLD_NOLOAD),
so the library and the test share one runtime and one stream handle."""
import ctypes as C
import os

import numpy as np
import pytest

import oracle as O
from helpers import rel_err

pytestmark = pytest.mark.gpu

_CAPTURE_RELAXED = 2  # hipStreamCaptureModeRelaxed
_NODE_KERNEL = 0      # hipGraphNodeTypeKernel
_REPLAYS = 3


def _hip(q):
    q.lib()  # loads libamdhip64.so.7 as a dependency of libqmla.so
    h = C.CDLL("libamdhip64.so.7", mode=os.RTLD_NOLOAD | os.RTLD_GLOBAL)
    for f in ("hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiate", "hipGraphLaunch",
              "hipGraphGetNodes", "hipGraphNodeGetType", "hipGraphExecDestroy", "hipGraphDestroy",
              "hipStreamSynchronize"):
        getattr(h, f).restype = C.c_int
    return h


class _Graph:
    """Captures fn() on `stream` and instantiates it; .kinds lists the node types."""

    def __init__(self, hip, stream, fn):
        self.hip, self.stream = hip, C.c_void_p(stream)
        assert hip.hipStreamBeginCapture(self.stream, _CAPTURE_RELAXED) == 0
        self.graph = C.c_void_p()
        try:
            fn()
        finally:
            rc = hip.hipStreamEndCapture(self.stream, C.byref(self.graph))
        assert rc == 0
        n = C.c_size_t(0)
        assert hip.hipGraphGetNodes(self.graph, None, C.byref(n)) == 0
        nodes = (C.c_void_p * n.value)()
        assert hip.hipGraphGetNodes(self.graph, nodes, C.byref(n)) == 0
        self.kinds = []
        for nd in nodes:
            t = C.c_int(-1)
            assert hip.hipGraphNodeGetType(C.c_void_p(nd), C.byref(t)) == 0
            self.kinds.append(t.value)
        self.exe = C.c_void_p()
        assert hip.hipGraphInstantiate(C.byref(self.exe), self.graph, None, None, C.c_size_t(0)) == 0

    def replay(self):
        assert self.hip.hipGraphLaunch(self.exe, self.stream) == 0
        assert self.hip.hipStreamSynchronize(self.stream) == 0

    def close(self):
        self.hip.hipGraphExecDestroy(self.exe)
        self.hip.hipGraphDestroy(self.graph)


def _cache(q, lens, seed):
    lens = np.asarray(lens, np.int32)
    cache = q.KVCache(lens, 512, 64, q.BF16)
    cache.write_pool(O.to_bf16_bits(O.normal((int(lens.sum()), 576), seed)))
    cache.set_lengths(lens)
    return cache


def _garbage(buf, seed):
    buf.upload(np.random.default_rng(seed).integers(0, 256, buf.nbytes, dtype=np.uint8))


@pytest.mark.parametrize("noalloc", [False, True])
def test_captured_decode_replays_the_eager_result(qmla_gpu, noalloc):
    """bf16 cache, 128 query rows, ragged lengths with an empty sequence."""
    q = qmla_gpu
    hip = _hip(q)
    lens = [0, 70, 1000, 33, 513, 4097]
    batch, rows = len(lens), 128
    cache = _cache(q, lens, 1800)
    ql_f = O.round_bf16(O.normal((batch, rows, 512), 1801))
    qr_f = O.round_bf16(O.normal((batch, rows, 64), 1802))
    ql = q.DeviceBuffer.from_numpy(O.to_bf16_bits(ql_f))
    qr = q.DeviceBuffer.from_numpy(O.to_bf16_bits(qr_f))
    dd = q.DecodeDims(batch, rows, 512, 64)
    out = q.DeviceBuffer(batch * rows * 512 * 4)
    lse = q.DeviceBuffer(batch * rows * 4)
    wsb = q.decode_workspace_bytes(cache, batch, rows)
    ws = q.DeviceBuffer(wsb)
    s = q.Stream()

    def call():
        if noalloc:
            st = q.lib().qmla_decode_absorbed_noalloc(C.byref(dd), cache.handle, q.BF16, ql.ptr, qr.ptr, 0.07,
                                                      out.ptr, lse.ptr, s.handle)
        else:
            st = q.lib().qmla_decode_absorbed(C.byref(dd), cache.handle, q.BF16, ql.ptr, qr.ptr, 0.07, out.ptr,
                                              lse.ptr, ws.ptr, wsb, s.handle)
        assert st == 0, q.lib().qmla_last_error()

    call()
    s.sync()
    want_o = out.to_numpy(np.float32, (batch, rows, 512))
    want_l = lse.to_numpy(np.float32, (batch, rows))
    g = _Graph(hip, s.handle, call)
    print(f"noalloc={noalloc}: {len(g.kinds)} nodes, kinds {sorted(set(g.kinds))}", flush=True)
    assert g.kinds and set(g.kinds) == {_NODE_KERNEL}
    for i in range(_REPLAYS):
        _garbage(out, 10 + i)
        _garbage(lse, 20 + i)
        call()  # eager work on the same stream between the replays
        s.sync()
        _garbage(out, 30 + i)
        g.replay()
        assert np.array_equal(out.to_numpy(np.float32, (batch, rows, 512)), want_o), f"replay {i}"
        assert np.array_equal(lse.to_numpy(np.float32, (batch, rows)), want_l), f"replay {i}"
    g.close()
    assert np.all(want_o[0] == 0) and np.all(np.isneginf(want_l[0]))
    # and the replayed result is the decode itself
    pool = O.bf16_bits_to_f32(cache.read_rows())
    ref, _ = O.decode_absorbed(ql_f[1:4], qr_f[1:4], pool, cache.offsets()[1:4],
                               np.asarray(lens[1:4], np.int32), 0.07)
    assert rel_err(want_o[1:4], ref) < 2e-2


def test_captured_zero_fill_and_keyless_prefill(qmla_gpu):
    """qmla_memset_zero over unaligned ranges and a prefill with seq_k = 0
    (every output row empty) record kernels, and each replay zeroes exactly
    the ranges again after the buffers were overwritten."""
    q = qmla_gpu
    hip = _hip(q)
    buf = q.DeviceBuffer(4096 + 64)
    ranges = [(3, 1), (5, 11), (16, 16), (7, 1000), (1031, 3000)]  # (offset, bytes)
    dims = q.PrefillDims(2, 3, 5, 0, 16, 8, 16, 1, 0)
    pre = q.DeviceBuffer(2 * 3 * 5 * 16 * 2)
    s = q.Stream()

    def call():
        for off, n in ranges:
            q.check(q.lib().qmla_memset_zero(C.c_void_p(buf.ptr + off), n, s.handle))
        q.check(q.lib().qmla_fused_prefill_attn(C.byref(dims), q.BF16, 1, 1, 1, 1, 1, 0.25, 1, pre.ptr,
                                                s.handle))

    def expect(seed):
        b = np.random.default_rng(seed).integers(0, 256, buf.nbytes, dtype=np.uint8)
        for off, n in ranges:
            b[off:off + n] = 0
        return b

    _garbage(buf, 1)
    call()
    s.sync()
    assert np.array_equal(buf.to_numpy(np.uint8, (buf.nbytes,)), expect(1))
    g = _Graph(hip, s.handle, call)
    print(f"{len(g.kinds)} nodes, kinds {sorted(set(g.kinds))}", flush=True)
    assert len(g.kinds) == len(ranges) + 1 and set(g.kinds) == {_NODE_KERNEL}
    for i in range(_REPLAYS):
        _garbage(buf, 40 + i)
        _garbage(pre, 50 + i)
        g.replay()
        assert np.array_equal(buf.to_numpy(np.uint8, (buf.nbytes,)), expect(40 + i)), f"replay {i}"
        assert not pre.to_numpy(np.uint16, (2 * 3 * 5 * 16,)).any(), f"replay {i}"
    g.close()


def test_captured_moe_layer_replays_the_eager_result(qmla_gpu):
    """qmla_moe_forward (routing, the two expert GEMVs, the combine) for 16
    tokens: kernel nodes only, and each replay reproduces the eager output
    and routing after they were overwritten."""
    q = qmla_gpu
    hip = _hip(q)
    W = O.random_moe_weights(16, 4, 256, 384, seed=1900)
    cfg = q.MoEConfig(W.num_experts, W.top_k, W.hidden_dim, W.intermediate_dim)
    layer = q.QMoELayer(cfg, W.gate_weight, [((W.gate_packed[e], W.gate_scales[e]), (W.up_packed[e], W.up_scales[e]),
                                              (W.down_packed[e], W.down_scales[e]))
                                             for e in range(W.num_experts)])
    T = 16
    xs = O.normal((T, 256), 1901)
    bx = q.DeviceBuffer.from_numpy(xs)
    out = q.DeviceBuffer(T * 256 * 4)
    ti, tw = q.DeviceBuffer(T * 4 * 4), q.DeviceBuffer(T * 4 * 4)
    n = layer.workspace_bytes(T)
    ws = q.DeviceBuffer(n)
    s = q.Stream()

    def call():
        layer.forward_device(bx, T, out, ws, n, ti, tw, stream=s.handle)

    def read():
        return (out.to_numpy(np.float32, (T, 256)), ti.to_numpy(np.int32, (T, 4)), tw.to_numpy(np.float32, (T, 4)))

    call()
    s.sync()
    want = read()
    g = _Graph(hip, s.handle, call)
    print(f"{len(g.kinds)} nodes, kinds {sorted(set(g.kinds))}", flush=True)
    assert g.kinds and set(g.kinds) == {_NODE_KERNEL}
    for i in range(_REPLAYS):
        for j, b in enumerate((out, ti, tw)):
            _garbage(b, 60 + 3 * i + j)
        g.replay()
        got = read()
        for a, b in zip(got, want):
            assert np.array_equal(a, b), f"replay {i}"
    g.close()
    ref, ridx, _ = O.moe_forward(W, xs, return_routing=True)
    np.testing.assert_array_equal(want[1], ridx)
    assert rel_err(want[0], ref) < 1e-4
