"""GPU parity tests of the MLA layer entry points (MlaAttention,
src/model.rs:107-307) over the latent cache, in f32 mode (1e-4).

C1 is the tiny single decode step of the reference's CPU path: batch 1,
8 heads, hidden 512, kv_lora_rank 64, qk_nope 32, qk_rope 16, v_head 32,
256 cached tokens; weights N(0, 0.02^2), activations and cache N(0, 1).
Its expected output is the golden vector written by the independent
float64 restatement (tests/golden/make_golden.py)."""
import numpy as np
import pytest

import oracle as O
from helpers import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-4


def c1_layer(q):
    w = O.MlaWeights.random(512, 8, 32, 16, 32, 64, seed=100)
    return w, q.MlaLayer(w)


def test_c1_decode_step_matches_golden(qmla_gpu, golden):
    q = qmla_gpu
    w, layer = c1_layer(q)
    lat = O.normal((1, 256, 80), 5)
    cache = q.KVCache([257], 64, 16, q.F32)
    cache.append(q.DeviceBuffer.from_numpy(lat), 1, 256)
    xs = O.normal((1, 1, 512), 7)
    out = layer.forward_with_cache(xs, cache)
    err = rel_err(out, golden["c1_out"])
    print(f"C1 rel_err={err:.2e}")
    assert err < TOL
    assert list(cache.lengths()) == [257]
    new_row = cache.read_rows()[256]
    assert rel_err(new_row, golden["c1_new_row"][0, 0]) < TOL


def test_multi_token_decode_two_sequences(qmla_gpu, golden):
    q = qmla_gpu
    w, layer = c1_layer(q)
    lat = O.normal((2, 256, 80), 6)
    cache = q.KVCache([259, 259], 64, 16, q.F32)
    cache.append(q.DeviceBuffer.from_numpy(lat), 2, 256)
    out = layer.forward_with_cache(O.normal((2, 3, 512), 9), cache)
    assert rel_err(out, golden["c1b_out"]) < TOL
    rows = np.stack([cache.read_seq(i) for i in range(2)])
    assert rel_err(rows[:, 256:], golden["c1b_new_rows"]) < TOL


def test_prefill_then_decode_matches_reference(qmla_gpu):
    """forward_prefill (src/model.rs:193-253) then three forward_with_cache
    steps, against the reference's decompressed path in the oracle."""
    q = qmla_gpu
    w = O.MlaWeights.random(256, 4, 32, 16, 32, 64, seed=700)
    layer = q.MlaLayer(w)
    b, s = 2, 37
    xs = O.normal((b, s, 256), 701)
    cache = q.KVCache([s + 3] * b, 64, 16, q.F32)
    out = layer.forward_prefill(xs, cache)
    ref, (k, v, kr) = O.mla_forward_prefill(w, xs)
    assert rel_err(out, ref) < TOL
    for step in range(3):
        x1 = O.normal((b, 1, 256), 710 + step)
        out1 = layer.forward_with_cache(x1, cache)
        ref1, (k, v, kr) = O.mla_forward_with_cache(w, x1, k, v, kr, return_cache=True)
        err = rel_err(out1, ref1)
        print(f"step {step} rel_err={err:.2e}")
        assert err < TOL
    assert list(cache.lengths()) == [s + 3] * b


def test_layer_argument_errors(qmla_gpu):
    q = qmla_gpu
    w, layer = c1_layer(q)
    cache = q.KVCache([4, 4], 64, 16, q.F32)
    cache.set_lengths([3, 4])
    with pytest.raises(q.QmlaError) as e:   # sequence 1 has no room for the new token
        layer.forward_with_cache(O.normal((2, 1, 512), 1), cache)
    assert e.value.status == 6
    assert list(cache.lengths()) == [3, 4]
    cache.set_lengths([4, 4])
    with pytest.raises(q.QmlaError) as e:   # no room for the new token
        layer.forward_with_cache(O.normal((2, 1, 512), 1), cache)
    assert e.value.status == 6
    wrong = q.KVCache([4], 128, 16, q.F32)
    with pytest.raises(q.QmlaError) as e:
        layer.forward_with_cache(O.normal((1, 1, 512), 1), wrong)
    assert e.value.status == 2
    # rows and workspace must be aligned (16 and 256 bytes); the rejected
    # calls leave the cache as it was
    cache.set_lengths([3, 3])
    x = q.DeviceBuffer.from_numpy(O.normal((2, 1, 512), 2))
    out = q.DeviceBuffer(2 * 512 * 4 + 64)
    need = layer.workspace_bytes(cache, 2, 1)
    ws = q.DeviceBuffer(need + 512)
    f = q.lib().qmla_layer_forward_with_cache
    assert f(layer.handle, x.ptr, 2, 1, cache.handle, out.ptr + 4, ws.ptr, need, None) == 1
    assert f(layer.handle, x.ptr, 2, 1, cache.handle, out.ptr, ws.ptr + 16, need, None) == 7
    assert list(cache.lengths()) == [3, 3]
    assert f(layer.handle, x.ptr, 2, 1, cache.handle, out.ptr + 16, ws.ptr + 256, need, None) == 0
    q.check(q.lib().qmla_stream_synchronize(None))
    assert list(cache.lengths()) == [4, 4]


@pytest.mark.parametrize("dims", [
    # hidden, heads, qk_nope, qk_rope, v_dim, kv_lora_rank
    (512, 8, 32, 16, 32, 64),      # the tiny CPU-path shape
    (512, 16, 128, 64, 128, 512),  # V2-Lite head shape (hidden reduced)
    (256, 4, 48, 16, 32, 64),      # head dims the bf16 prefill does not take: f32 attention
])
def test_bf16_cache_prefill_then_decode(qmla_gpu, dims):
    """forward_prefill then forward_with_cache steps over a bf16 latent
    cache: the prefill attention and the decode core are the bf16 MFMA
    kernels (the prefill attention stays f32 for head dims the bf16 prefill
    does not take); the reference is the oracle's f32 decompressed path on
    the same weights and inputs (tolerance 2e-2)."""
    q = qmla_gpu
    hidden, H, dn, dr, dv, r = dims
    w = O.MlaWeights.random(hidden, H, dn, dr, dv, r, seed=900 + r)
    layer = q.MlaLayer(w)
    b, s = 2, 45
    xs = O.normal((b, s, hidden), 901)
    cache = q.KVCache([s + 3] * b, r, dr, q.BF16)
    out = layer.forward_prefill(xs, cache)
    ref, (k, v, kr) = O.mla_forward_prefill(w, xs)
    assert rel_err(out, ref) < 2e-2
    for step in range(3):
        x1 = O.normal((b, 1, hidden), 910 + step)
        out1 = layer.forward_with_cache(x1, cache)
        ref1, (k, v, kr) = O.mla_forward_with_cache(w, x1, k, v, kr, return_cache=True)
        err = rel_err(out1, ref1)
        print(f"dims={dims} step {step} rel_err={err:.2e}")
        assert err < 2e-2
    assert list(cache.lengths()) == [s + 3] * b


def test_bf16_cache_prefill_spans_query_tiles(qmla_gpu):
    """forward_prefill over a bf16 cache at V2-Lite head shapes with 300
    tokens per sequence: the attention runs on the bf16 MFMA prefill (q, k, v
    rounded to bf16) across two 256-row query tiles, the second one partial;
    the reference is the oracle's f32 path (tolerance 2e-2)."""
    q = qmla_gpu
    hidden, H, dn, dr, dv, r = 512, 16, 128, 64, 128, 512
    w = O.MlaWeights.random(hidden, H, dn, dr, dv, r, seed=1600)
    layer = q.MlaLayer(w)
    b, s = 2, 300
    xs = O.normal((b, s, hidden), 1601)
    cache = q.KVCache([s] * b, r, dr, q.BF16)
    out = layer.forward_prefill(xs, cache)
    ref, _ = O.mla_forward_prefill(w, xs)
    err = rel_err(out, ref)
    print(f"prefill b={b} s={s} bf16 cache rel_err={err:.2e}")
    assert err < 2e-2
    assert list(cache.lengths()) == [s] * b


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("b,s", [(2, 96), (1, 160)])
def test_prefill_split_gemms_at_small_latent_dims(qmla_gpu, dt, b, s):
    """forward_prefill through the hand-written split GEMMs at the tiny
    CPU-path head shapes (hidden 512, 8 heads, kv_lora_rank 64, dn 32, dr 16,
    dv 32): K = 64 for kv_b_proj (two chunks), the latent rows kernel with
    eight lanes per row, and with a bf16 cache the context written as
    records (s % 32 == 0).  Against the oracle's decompressed path, then two
    decode steps."""
    q = qmla_gpu
    hidden, H, dn, dr, dv, r = 512, 8, 32, 16, 32, 64
    w = O.MlaWeights.random(hidden, H, dn, dr, dv, r, seed=2100 + s)
    layer = q.MlaLayer(w)
    xs = O.normal((b, s, hidden), 2101)
    cache = q.KVCache([s + 2] * b, r, dr, q.F32 if dt == "f32" else q.BF16)
    out = layer.forward_prefill(xs, cache)
    ref, (k, v, kr) = O.mla_forward_prefill(w, xs)
    tol = TOL if dt == "f32" else 2e-2
    err = rel_err(out, ref)
    print(f"small-dims prefill {b}x{s} {dt} rel_err={err:.2e}", flush=True)
    assert err < tol
    for step in range(2):
        x1 = O.normal((b, 1, hidden), 2110 + step)
        out1 = layer.forward_with_cache(x1, cache)
        ref1, (k, v, kr) = O.mla_forward_with_cache(w, x1, k, v, kr, return_cache=True)
        assert rel_err(out1, ref1) < tol
    assert list(cache.lengths()) == [s + 2] * b


def _ragged_cache(q, lens, r, dr, dtype, seed, spare=2):
    """A cache whose sequences hold `lens` random latent rows (N(0,1); bf16
    rounded for a bf16 cache) with `spare` free rows each; returns the cache
    and the per-sequence f32 rows the oracle sees."""
    lens = np.asarray(lens, np.int32)
    cache = q.KVCache(lens + spare, r, dr, dtype)
    total = int((lens + spare).sum())
    pool = O.normal((total, r + dr), seed)
    if dtype == q.BF16:
        bits = O.to_bf16_bits(pool)
        cache.write_pool(bits)
        pool = O.bf16_bits_to_f32(bits)
    else:
        cache.write_pool(pool)
    cache.set_lengths(lens)
    offs = np.concatenate([[0], np.cumsum(lens + spare)[:-1]])  # rows of `pool` per sequence
    per_seq = [pool[offs[i]:offs[i] + lens[i]] for i in range(lens.size)]
    return cache, per_seq


@pytest.mark.parametrize("case", [
    # (hidden, heads, dn, dr, dv, r, cache dtype, lengths, new tokens, tolerance,
    #  bf16-operand projections)
    ((512, 8, 32, 16, 32, 64), "f32", [4096, 32768, 300], 1, 1e-4, False),
    ((512, 8, 32, 16, 32, 64), "f32", [1, 17000, 0], 2, 1e-4, False),
    ((512, 16, 128, 64, 128, 512), "bf16", [300, 4097, 1], 1, 2e-2, False),
    ((512, 16, 128, 64, 128, 512), "bf16", [300, 4097, 1], 1, 2e-2, True),
], ids=["c1-dims-f32-4096-32768-300", "c1-dims-f32-two-tokens", "v2lite-dims-bf16-300-4097-1",
        "v2lite-dims-bf16-projections"])
def test_ragged_layer_decode_at_real_positions(qmla_gpu, case):
    """forward_with_cache over a ragged batch whose contexts reach 32768:
    each sequence's new tokens take RoPE positions from its own length, and
    every sequence's output and new cache rows equal a batch-1 run of the
    reference's absorbed-latent step in the oracle at that position (with
    bf16-operand projections: at the bf16 tolerance, rows included)."""
    q = qmla_gpu
    dims, dt, lens, s, tol, proj16 = case
    hidden, H, dn, dr, dv, r = dims
    w = O.MlaWeights.random(hidden, H, dn, dr, dv, r, seed=1200 + r)
    layer = q.MlaLayer(w)
    if proj16:
        layer.set_projection_dtype(q.BF16)
    dtype = q.BF16 if dt == "bf16" else q.F32
    cache, per_seq = _ragged_cache(q, lens, r, dr, dtype, 1201, spare=s)
    xs = O.normal((len(lens), s, hidden), 1202)
    out = layer.forward_with_cache(xs, cache)
    assert list(cache.lengths()) == [n + s for n in lens]
    pool = cache.read_rows()
    if dtype == q.BF16:
        pool = O.bf16_bits_to_f32(pool)
    offs = cache.offsets()
    for b, n in enumerate(lens):
        lat = per_seq[b].reshape(1, n, r + dr)
        ref, rows = O.mla_forward_with_latent(w, xs[b:b + 1], lat)
        err = rel_err(out[b], ref[0])
        row_err = rel_err(pool[offs[b] + n: offs[b] + n + s], rows[0])
        print(f"{dt} seq {b} len {n}: out rel_err={err:.2e} new-row rel_err={row_err:.2e}")
        assert err < tol
        assert row_err < (1e-5 if dtype == q.F32 else 2e-2 if proj16 else 4e-3)


def test_rejected_layer_call_leaves_the_cache_unchanged(qmla_gpu):
    """A layer call that fails validation (unsupported bf16 decode shape,
    short workspace) neither grows the cache nor appends rows."""
    q = qmla_gpu
    import ctypes as C
    w = O.MlaWeights.random(256, 4, 32, 32, 32, 256, seed=1300)   # bf16 r 256 / dr 32: no MFMA core
    layer = q.MlaLayer(w)
    cache = q.KVCache([2, 2], 256, 32, q.BF16, grow=True)
    cache.set_lengths([2, 2])
    with pytest.raises(q.QmlaError) as e:
        layer.forward_with_cache(O.normal((2, 1, 256), 1), cache)
    assert e.value.status == 3
    assert list(cache.lengths()) == [2, 2] and list(cache.capacity()) == [2, 2]
    w2, layer2 = c1_layer(q)
    cache2 = q.KVCache([2, 2], 64, 16, q.F32, grow=True)
    cache2.set_lengths([2, 2])
    x = q.DeviceBuffer.from_numpy(O.normal((2, 1, 512), 2))
    out = q.DeviceBuffer(2 * 512 * 4)
    need = layer2.workspace_bytes(cache2, 2, 1)
    ws = q.DeviceBuffer(need)
    st = q.lib().qmla_layer_forward_with_cache(layer2.handle, x.ptr, 2, 1, cache2.handle, out.ptr, ws.ptr,
                                               need - 256, None)
    assert st == 7
    assert list(cache2.lengths()) == [2, 2] and list(cache2.capacity()) == [2, 2]
    # with the full workspace the same call grows the cache and appends
    st = q.lib().qmla_layer_forward_with_cache(layer2.handle, x.ptr, 2, 1, cache2.handle, out.ptr, ws.ptr,
                                               need, None)
    assert st == 0, q.lib().qmla_last_error()
    q.check(q.lib().qmla_stream_synchronize(None))
    assert list(cache2.lengths()) == [3, 3] and min(cache2.capacity()) >= 3
    del C


def test_split_projections_keep_f32_parity(qmla_gpu):
    """Products of at least 256 token rows run as split bf16 hi/lo GEMMs
    (x w = x_hi w_hi + x_lo w_hi + x_hi w_lo, f32 accumulation): with an f32
    cache, forward_prefill over 2 x 160 tokens and a 130-token
    forward_with_cache step (260 rows, the GEMM path) stay within the f32
    tolerance of the oracle's decompressed path."""
    q = qmla_gpu
    hidden, H, dn, dr, dv, r = 512, 16, 128, 64, 128, 512
    w = O.MlaWeights.random(hidden, H, dn, dr, dv, r, seed=1750)
    layer = q.MlaLayer(w)
    b, s, s2 = 2, 160, 130
    cache = q.KVCache([s + s2] * b, r, dr, q.F32)
    xs = O.normal((b, s, hidden), 1751)
    out = layer.forward_prefill(xs, cache)
    ref, (k, v, kr) = O.mla_forward_prefill(w, xs)
    err = rel_err(out, ref)
    print(f"prefill {b}x{s} f32 cache rel_err={err:.2e}")
    assert err < TOL
    x2 = O.normal((b, s2, hidden), 1752)
    out2 = layer.forward_with_cache(x2, cache)
    ref2 = O.mla_forward_with_cache(w, x2, k, v, kr)
    err2 = rel_err(out2, ref2)
    print(f"decode step {b}x{s2} f32 cache rel_err={err2:.2e}")
    assert err2 < TOL
    assert list(cache.lengths()) == [s + s2] * b


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_materialise_long_sequences_split_gemm(qmla_gpu, dt):
    """qmla_cache_materialise over sequences of at least 256 tokens runs
    compute_kv as split bf16 GEMMs batched over heads: k and v equal the
    oracle's decompression of the same latent rows within the f32
    tolerance, k_rope is the rows' k_pe broadcast to every head."""
    q = qmla_gpu
    hidden, H, dn, dr, dv, r = 256, 8, 64, 32, 48, 128
    w = O.MlaWeights.random(hidden, H, dn, dr, dv, r, seed=1760)
    layer = q.MlaLayer(w)
    b, T = 2, 300
    dtype = q.F32 if dt == "f32" else q.BF16
    cache = q.KVCache([T] * b, r, dr, dtype)
    rows = O.normal((b * T, r + dr), 1761)
    if dtype == q.BF16:
        bits = O.to_bf16_bits(rows)
        cache.write_pool(bits)
        rows = O.bf16_bits_to_f32(bits)
    else:
        cache.write_pool(rows)
    cache.set_lengths([T] * b)
    gk, gv, gkr = layer.materialise(cache)
    ek, ev, ekr = O.decompress_cache(w, rows.reshape(b, T, r + dr))
    for name, got, ref in (("k", gk, ek), ("v", gv, ev), ("k_rope", gkr, ekr)):
        err = rel_err(got, ref)
        print(f"{dt} {name} rel_err={err:.2e}")
        assert err < TOL


def test_prefill_workspace_is_its_own_and_is_enforced(qmla_gpu):
    """qmla_layer_prefill_workspace_bytes sizes forward_prefill alone: at
    most the size that serves both calls, and far below it where the decode
    core's partials (seq x heads rows per piece) dominate.  A workspace one
    alignment step short is rejected with the cache untouched; the exact
    size runs and matches the oracle."""
    q = qmla_gpu
    hidden, H, dn, dr, dv, r = 512, 16, 128, 64, 128, 512
    w = O.MlaWeights.random(hidden, H, dn, dr, dv, r, seed=1700)
    layer = q.MlaLayer(w)
    big = q.KVCache([2048] * 4, r, dr, q.BF16)
    pre, both = layer.prefill_workspace_bytes(big, 4, 2048), layer.workspace_bytes(big, 4, 2048)
    print(f"B4 S2048 workspace: prefill {pre >> 20} MiB, either call {both >> 20} MiB")
    assert pre < (1 << 30) and pre * 4 < both
    del big
    # 80 rows run the rocBLAS projections, 128 rows the hand-written split
    # GEMMs (whose workspace leaves out the regions only rocBLAS uses)
    for dt, (b, s) in [(q.F32, (2, 40)), (q.BF16, (2, 40)), (q.F32, (2, 64)), (q.BF16, (2, 64))]:
        cache = q.KVCache([s] * b, r, dr, dt)
        need = layer.prefill_workspace_bytes(cache, b, s)
        assert need <= layer.workspace_bytes(cache, b, s)
        xs = O.normal((b, s, hidden), 1701)
        x = q.DeviceBuffer.from_numpy(xs)
        out = q.DeviceBuffer(b * s * hidden * 4)
        ws = q.DeviceBuffer(need)
        st = q.lib().qmla_layer_forward_prefill(layer.handle, x.ptr, b, s, cache.handle, out.ptr, ws.ptr,
                                                need - 256, None)
        assert st == 7
        assert list(cache.lengths()) == [0] * b
        st = q.lib().qmla_layer_forward_prefill(layer.handle, x.ptr, b, s, cache.handle, out.ptr, ws.ptr,
                                                need, None)
        assert st == 0, q.lib().qmla_last_error()
        q.check(q.lib().qmla_stream_synchronize(None))
        ref, _ = O.mla_forward_prefill(w, xs)
        err = rel_err(out.to_numpy(np.float32, (b, s, hidden)), ref)
        print(f"dtype {dt} {b}x{s} prefill rel_err={err:.2e}")
        assert err < (TOL if dt == q.F32 else 2e-2)
        assert list(cache.lengths()) == [s] * b


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_materialised_cache_equals_the_reference_kvcache(qmla_gpu, dt):
    """qmla_cache_materialise rebuilds KVCache {k, v, k_rope}
    (src/model.rs:88-92): after forward_prefill and two decode steps, the
    tensors equal the cache the reference's decompressed path returns."""
    q = qmla_gpu
    hidden, H, dn, dr, dv, r = (256, 4, 32, 16, 32, 64) if dt == "f32" else (512, 16, 128, 64, 128, 512)
    w = O.MlaWeights.random(hidden, H, dn, dr, dv, r, seed=1400 + r)
    layer = q.MlaLayer(w)
    b, s = 2, 29
    dtype = q.F32 if dt == "f32" else q.BF16
    cache = q.KVCache([s + 2] * b, r, dr, dtype)
    xs = O.normal((b, s, hidden), 1401)
    layer.forward_prefill(xs, cache)
    _, (k, v, kr) = O.mla_forward_prefill(w, xs)
    for step in range(2):
        x1 = O.normal((b, 1, hidden), 1410 + step)
        layer.forward_with_cache(x1, cache)
        _, (k, v, kr) = O.mla_forward_with_cache(w, x1, k, v, kr, return_cache=True)
    gk, gv, gkr = layer.materialise(cache)
    assert gk.shape == k.shape and gv.shape == v.shape and gkr.shape == kr.shape
    if dtype == q.F32:
        tol = 1e-4
    else:
        # the bf16 cache stores the latent rounded to bf16: compare with the
        # oracle's decompression of exactly those rows (1e-4), and with the
        # reference's f32 cache within the bf16 tolerance
        pool = O.bf16_bits_to_f32(cache.read_rows())
        offs = cache.offsets()
        lat = np.stack([pool[offs[i]:offs[i] + s + 2] for i in range(b)])
        ek, ev, ekr = O.decompress_cache(w, lat)
        for got, ref in ((gk, ek), (gv, ev), (gkr, ekr)):
            assert rel_err(got, ref) < 1e-4
        tol = 2e-2
    for name, got, ref in (("k", gk, k), ("v", gv, v), ("k_rope", gkr, kr)):
        err = rel_err(got, ref)
        print(f"{dt} {name} rel_err={err:.2e}")
        assert err < tol
    # one sequence of a ragged cache at a time; unequal lengths are refused
    cache.set_lengths([s + 2, s])
    k1, v1, kr1 = layer.materialise(cache, 1, 1)
    assert k1.shape == (1, H, s, dn)
    assert rel_err(k1[0], gk[1][:, :s]) < 1e-6
    with pytest.raises(q.QmlaError) as e:
        layer.materialise(cache, 0, 2)
    assert e.value.status == 2


@pytest.mark.parametrize("batch,seq,dt", [(40, 1, "f32"), (1, 1, "f32"), (3, 12, "bf16")],
                         ids=["40x1-f32-two-chunks", "1x1-f32", "3x12-bf16"])
def test_decode_step_projections_at_v2lite_width(qmla_gpu, batch, seq, dt):
    """forward_with_cache at V2-Lite widths (hidden 2048, 16 heads, dn 128,
    dr 64, dv 128, r 512).  With at most 64 new tokens the projections run
    on the skinny bf16 hi/lo MFMA kernel, 32 token rows per launch (40 rows:
    two launches); the result equals the oracle's absorbed-latent step (f32
    throughout) within 1e-4 for an f32 cache, 2e-2 for a bf16 cache."""
    q = qmla_gpu
    hidden, H, dn, dr, dv, r = 2048, 16, 128, 64, 128, 512
    w = O.MlaWeights.random(hidden, H, dn, dr, dv, r, seed=1500)
    layer = q.MlaLayer(w)
    dtype = q.F32 if dt == "f32" else q.BF16
    lens = [97 + 13 * (i % 5) for i in range(batch)]
    cache, per_seq = _ragged_cache(q, lens, r, dr, dtype, 1501, spare=seq)
    xs = O.normal((batch, seq, hidden), 1502)
    out = layer.forward_with_cache(xs, cache)
    tol = 1e-4 if dtype == q.F32 else 2e-2
    worst = 0.0
    for b, n in enumerate(lens):
        ref, _ = O.mla_forward_with_latent(w, xs[b:b + 1], per_seq[b].reshape(1, n, r + dr))
        worst = max(worst, rel_err(out[b], ref[0]))
    print(f"batch {batch} seq {seq} {dt}: worst rel_err={worst:.2e}")
    assert worst < tol


@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_growth_mode_layer_loop_over_pages(qmla_gpu, dt):
    """forward_prefill then decode steps of 1-3 tokens on a cache created
    empty in growth mode with 32-row pages: the steps take new pages as the
    sequences cross page boundaries, and every output and new cache row
    matches the reference's decompressed path."""
    q = qmla_gpu
    w = O.MlaWeights.random(256, 4, 32, 16, 32, 64, seed=720)
    layer = q.MlaLayer(w)
    b, s = 3, 29
    dtype = q.F32 if dt == "f32" else q.BF16
    tol = TOL if dt == "f32" else 2e-2
    cache = q.KVCache([0] * b, 64, 16, dtype, grow=True, page_rows=32)
    xs = O.normal((b, s, 256), 721)
    out = layer.forward_prefill(xs, cache)
    ref, (k, v, kr) = O.mla_forward_prefill(w, xs)
    assert rel_err(out, ref) < tol
    n = s
    for step, m in enumerate((1, 1, 2, 1, 3, 1, 29, 1)):
        x1 = O.normal((b, m, 256), 730 + step)
        out1 = layer.forward_with_cache(x1, cache)
        ref1, (k, v, kr) = O.mla_forward_with_cache(w, x1, k, v, kr, return_cache=True)
        n += m
        err = rel_err(out1, ref1)
        print(f"{dt} step {step} (+{m} -> {n}) rel_err={err:.2e}")
        assert err < tol
    assert list(cache.lengths()) == [n] * b
    assert cache.describe().contiguous == 0
    assert all(c >= n for c in cache.capacity())


def test_layer_calls_from_several_threads(qmla_gpu):
    """forward_prefill (the rocBLAS GEMM path) on one layer from four
    threads at once, each with its own stream and cache, gives exactly the
    results of the same calls made one after another."""
    import threading
    q = qmla_gpu
    w = O.MlaWeights.random(256, 4, 32, 16, 32, 64, seed=800)
    layer = q.MlaLayer(w)
    xs = [O.normal((2, 37, 256), 801 + i) for i in range(4)]
    want = [layer.forward_prefill(x, q.KVCache([40, 40], 64, 16, q.F32)) for x in xs]
    got, errs = [None] * 4, []

    def run(i):
        try:
            st = q.Stream()
            for _ in range(3):
                got[i] = layer.forward_prefill(xs[i], q.KVCache([40, 40], 64, 16, q.F32), stream=st)
            st.close()
        except Exception as e:  # reported below
            errs.append(e)

    ts = [threading.Thread(target=run, args=(i,)) for i in range(4)]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    assert not errs, errs
    for i in range(4):
        np.testing.assert_array_equal(got[i], want[i])


@pytest.mark.parametrize("b,s", [(1, 128), (1, 512), (1, 2048), (2, 2048)])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_layer_prefill_at_bench_widths(qmla_gpu, dt, b, s):
    """forward_prefill at the widths the layer-prefill bench line runs:
    hidden 2048, 16 heads, kv_lora_rank 512, dn 128 / dr 64 / dv 128, b
    sequences of s tokens, through the hand-written split GEMMs: 128 and
    512 rows split K over several blocks (partial sums added by a second
    launch), 2048 rows run the 64 x 128 tiles whole, 4096 rows the 256 x
    256 tiles.  Against the oracle's decompressed path: 1e-4 with an f32
    cache, 2e-2 with a bf16 cache.  Then one decode step on the filled
    cache."""
    q = qmla_gpu
    hidden, H, dn, dr, dv, r = 2048, 16, 128, 64, 128, 512
    w = O.MlaWeights.random(hidden, H, dn, dr, dv, r, seed=1900)
    layer = q.MlaLayer(w)
    xs = O.normal((b, s, hidden), 1901)
    cache = q.KVCache([s + 1] * b, r, dr, q.F32 if dt == "f32" else q.BF16)
    out = layer.forward_prefill(xs, cache)
    ref, (k, v, kr) = O.mla_forward_prefill(w, xs)
    tol = TOL if dt == "f32" else 2e-2
    err = rel_err(out, ref)
    print(f"layer prefill {b}x{s} hidden {hidden} {dt} cache rel_err={err:.2e}", flush=True)
    assert err < tol
    x1 = O.normal((b, 1, hidden), 1902)
    out1 = layer.forward_with_cache(x1, cache)
    ref1 = O.mla_forward_with_cache(w, x1, k, v, kr)
    err1 = rel_err(out1, ref1)
    print(f"decode step after it, {dt} cache rel_err={err1:.2e}", flush=True)
    assert err1 < tol
    assert list(cache.lengths()) == [s + 1] * b


@pytest.mark.parametrize("b,s", [(1, 128), (1, 512), (2, 2048)])
@pytest.mark.parametrize("dt", ["f32", "bf16"])
def test_layer_bf16_projections(qmla_gpu, dt, b, s):
    """qmla_layer_set_projection_dtype(BF16): the projection kernels take
    bf16 operands (one MFMA per step; 128 rows split K, 512 rows the 64 x
    128 tiles, 4096 rows the 256 x 256 tiles), then a decode step on the
    skinny kernels.  Against the oracle's f32 path at the bf16 tolerance,
    with either cache dtype; the results must differ from the f32-exact
    projections (the mode took effect), and switching back to F32 gives the
    f32-exact results bit for bit."""
    q = qmla_gpu
    hidden, H, dn, dr, dv, r = 2048, 16, 128, 64, 128, 512
    w = O.MlaWeights.random(hidden, H, dn, dr, dv, r, seed=1950)
    xs = O.normal((b, s, hidden), 1951)
    x1 = O.normal((b, 1, hidden), 1952)
    cdt = q.F32 if dt == "f32" else q.BF16
    ref, (k, v, kr) = O.mla_forward_prefill(w, xs)
    ref1 = O.mla_forward_with_cache(w, x1, k, v, kr)

    def run(layer):
        cache = q.KVCache([s + 1] * b, r, dr, cdt)
        return layer.forward_prefill(xs, cache), layer.forward_with_cache(x1, cache)

    layer = q.MlaLayer(w)
    exact, exact1 = run(layer)
    layer.set_projection_dtype(q.BF16)
    out, out1 = run(layer)
    err, err1 = rel_err(out, ref), rel_err(out1, ref1)
    print(f"bf16 projections, {dt} cache, prefill {b}x{s} rel_err={err:.2e}, "
          f"decode step rel_err={err1:.2e}", flush=True)
    assert err < 2e-2 and err1 < 2e-2
    assert rel_err(out, exact) > 1e-5 and rel_err(out1, exact1) > 1e-5
    layer.set_projection_dtype(q.F32)
    again, again1 = run(layer)
    np.testing.assert_array_equal(again, exact)
    np.testing.assert_array_equal(again1, exact1)


def test_layer_bf16_projections_leave_the_rocblas_paths_exact(qmla_gpu):
    """Calls below the hand-written kernels' range stay f32-exact in the
    bf16-operand mode: a 64-token prefill (rocBLAS projections) and a decode
    step of 65 new tokens per sequence (more rows than the skinny kernel
    takes) give the f32-exact results bit for bit."""
    q = qmla_gpu
    w = O.MlaWeights.random(512, 8, 32, 16, 32, 64, seed=1970)
    xs = O.normal((1, 64, 512), 1971)
    x1 = O.normal((1, 65, 512), 1972)

    def run(dtype):
        layer = q.MlaLayer(w)
        layer.set_projection_dtype(dtype)
        cache = q.KVCache([200], 64, 16, q.BF16)
        return layer.forward_prefill(xs, cache), layer.forward_with_cache(x1, cache)

    exact, exact1 = run(q.F32)
    got, got1 = run(q.BF16)
    np.testing.assert_array_equal(got, exact)
    np.testing.assert_array_equal(got1, exact1)


@pytest.mark.parametrize("b,s", [(2, 96), (1, 160)])
def test_layer_bf16_projections_at_small_latent_dims(qmla_gpu, b, s):
    """bf16 operands at the tiny head shapes (hidden 512, 8 heads, dn 32 /
    dr 16 / dv 32, kv_lora_rank 64: kv_b_proj's K = 64 is two chunks of the
    64 x 128 tiling), bf16 cache, prefill then a decode step: 2e-2."""
    q = qmla_gpu
    w = O.MlaWeights.random(512, 8, 32, 16, 32, 64, seed=1960)
    layer = q.MlaLayer(w)
    layer.set_projection_dtype(q.BF16)
    xs = O.normal((b, s, 512), 1961)
    cache = q.KVCache([s + 1] * b, 64, 16, q.BF16)
    out = layer.forward_prefill(xs, cache)
    ref, (k, v, kr) = O.mla_forward_prefill(w, xs)
    err = rel_err(out, ref)
    x1 = O.normal((b, 1, 512), 1962)
    err1 = rel_err(layer.forward_with_cache(x1, cache), O.mla_forward_with_cache(w, x1, k, v, kr))
    print(f"bf16 projections small dims {b}x{s}: prefill {err:.2e}, step {err1:.2e}", flush=True)
    assert err < 2e-2 and err1 < 2e-2
    with pytest.raises(q.QmlaError):
        layer.set_projection_dtype(7)
