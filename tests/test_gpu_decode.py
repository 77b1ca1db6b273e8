"""GPU parity tests of the absorbed-latent decode core (qmla_decode_absorbed),
the attention core of MlaAttention::forward_with_cache (src/model.rs:294-303)
rewritten over the latent cache.

Tolerances (max |gpu - ref| / max |ref|): 1e-4 for the f32 cache, 2e-2 for
the bf16 cache (bf16 MFMA, f32 accumulate), as the north-star contract
states.  The reference side is the CPU oracle (oracle/mla_oracle.c) on the
same inputs (the bf16 cache values exactly, q unrounded)."""
import numpy as np
import pytest

import oracle as O
from helpers import bf16_bits, bf16_to_f32, rel_err

pytestmark = pytest.mark.gpu

TOL_F32, TOL_BF16 = 1e-4, 2e-2


def make_cache(q, lens, r, dr, dtype, seed, cap_extra=0):
    """Cache whose sequence i holds lens[i] N(0,1) rows (host generated)."""
    lens = np.asarray(lens, np.int32)
    cache = q.KVCache(lens + cap_extra, r, dr, dtype)
    total = int((lens + cap_extra).sum())
    rows = O.normal((total, r + dr), seed)
    if dtype == q.BF16:
        bits = bf16_bits(rows)
        cache.write_pool(bits)
        rows = bf16_to_f32(bits)
    else:
        cache.write_pool(rows)
    cache.set_lengths(lens)
    offs = np.concatenate([[0], np.cumsum(lens + cap_extra)[:-1]]).astype(np.int64)
    return cache, rows, offs


def run(q, cache, ql, qr, scale, splits=0, q_dtype=None):
    q_dtype = q.F32 if q_dtype is None else q_dtype
    if q_dtype == q.BF16:
        ql, qr = bf16_bits(ql), bf16_bits(qr)
    return q.decode_numpy(cache, ql, qr, scale, splits=splits, q_dtype=q_dtype)


def test_decode_f32_ragged_golden(qmla_gpu, golden):
    q = qmla_gpu
    cache, rows, offs = make_cache(q, [5, 17, 40], 64, 16, q.F32, 31)
    ql, qr = O.normal((3, 4, 64), 32), O.normal((3, 4, 16), 33)
    out, lse = run(q, cache, ql, qr, 0.1)
    assert rel_err(out, golden["ragged_out"]) < TOL_F32
    np.testing.assert_allclose(lse, golden["ragged_lse"], rtol=1e-5)


@pytest.mark.parametrize("rows_m", [4, 16, 40, 96, 128])
def test_decode_bf16_small_latent(qmla_gpu, rows_m):
    q = qmla_gpu
    lens = [5, 17, 40, 1, 100]
    cache, rows, offs = make_cache(q, lens, 64, 16, q.BF16, 41)
    ql, qr = O.normal((5, rows_m, 64), 42), O.normal((5, rows_m, 16), 43)
    out, lse = run(q, cache, ql, qr, 0.125)
    ref, rlse = O.decode_absorbed(ql, qr, rows, offs, lens, 0.125)
    err = rel_err(out, ref)
    print(f"rows={rows_m} rel_err={err:.2e}")
    assert err < TOL_BF16
    np.testing.assert_allclose(lse, rlse, atol=2e-2)


def test_decode_f32_v2lite_subset(qmla_gpu):
    """C2 shapes (H16, r512, rope64, T=4096+1) with an f32 cache: 1e-4."""
    q = qmla_gpu
    lens = [4097] * 4
    cache, rows, offs = make_cache(q, lens, 512, 64, q.F32, 51)
    ql, qr = O.normal((4, 16, 512), 52), O.normal((4, 16, 64), 53)
    s = 192 ** -0.5
    out, lse = run(q, cache, ql, qr, s)
    ref, rlse = O.decode_absorbed(ql, qr, rows, offs, lens, s)
    assert rel_err(out, ref) < TOL_F32
    np.testing.assert_allclose(lse, rlse, rtol=1e-5)


@pytest.mark.parametrize("rows_m", [70, 96])
def test_decode_bf16_rows_not_multiple_of_pass(qmla_gpu, rows_m):
    """Row counts that leave the last wave of a 128-row pass without rows:
    its partial results must not be stored (they would land in the next
    split slot).  Several sequences and two split counts, so neighbouring
    slots belong to different sequences."""
    q = qmla_gpu
    lens = [300, 1, 2048, 77, 515, 4096]
    cache, rows, offs = make_cache(q, lens, 512, 64, q.BF16, 131)
    ql, qr = O.normal((6, rows_m, 512), 132), O.normal((6, rows_m, 64), 133)
    ref, rlse = O.decode_absorbed(ql, qr, rows, offs, lens, 0.08)
    for splits in (0, 37):
        out, lse = run(q, cache, ql, qr, 0.08, splits=splits)
        err = rel_err(out, ref)
        print(f"rows={rows_m} splits={splits} rel_err={err:.2e}")
        assert err < TOL_BF16
        np.testing.assert_allclose(lse, rlse, atol=2e-2)


@pytest.mark.parametrize("rows_m", [1, 7, 32])
def test_decode_bf16_narrow_rows(qmla_gpu, rows_m):
    """At most 32 query rows over kv_lora_rank 512 take the four-wave narrow
    path (S^T split over the latent dims, P.V over the columns): partial
    tiles, a one-token sequence, two split counts and a negative scale."""
    q = qmla_gpu
    lens = [1, 31, 33, 300, 1025, 64]
    cache, rows, offs = make_cache(q, lens, 512, 64, q.BF16, 141)
    ql, qr = O.normal((6, rows_m, 512), 142), O.normal((6, rows_m, 64), 143)
    for scale in (0.09, -0.05):
        ref, rlse = O.decode_absorbed(ql, qr, rows, offs, lens, scale)
        for splits in (0, 9):
            out, lse = run(q, cache, ql, qr, scale, splits=splits)
            err = rel_err(out, ref)
            print(f"rows={rows_m} scale={scale} splits={splits} rel_err={err:.2e}")
            assert err < TOL_BF16
            np.testing.assert_allclose(lse, rlse, atol=2e-2)


def test_decode_bf16_v2lite_full(qmla_gpu):
    """C2: batch 32, 16 heads, 4096 cached + 1, bf16 cache, scale 1/sqrt(192)."""
    q = qmla_gpu
    lens = [4097] * 32
    cache, rows, offs = make_cache(q, lens, 512, 64, q.BF16, 61)
    ql, qr = O.normal((32, 16, 512), 62), O.normal((32, 16, 64), 63)
    s = 192 ** -0.5
    out, lse = run(q, cache, ql, qr, s)
    ref, rlse = O.decode_absorbed(ql, qr, rows, offs, lens, s)
    err = rel_err(out, ref)
    print(f"C2 bf16 rel_err={err:.2e}")
    assert err < TOL_BF16
    np.testing.assert_allclose(lse, rlse, atol=2e-2)
    # q given as bf16 or as f32 (rounded on the device) must agree exactly
    out_b, _ = run(q, cache, ql, qr, s, q_dtype=q.BF16)
    np.testing.assert_array_equal(out_b, out)


def test_decode_bf16_v3_ragged_full_size(qmla_gpu):
    """C4: batch 64, 128 heads, contexts U[1024, 32768] + 1 (seeded), bf16.
    Full-size run, every sequence checked against the oracle (~330 GFLOP of
    host work, a few seconds on the oracle's OpenMP loops), then again with
    another split count."""
    q = qmla_gpu
    lens = (O.uniform_int(64, 4, 1024, 32768) + 1).astype(np.int32)
    print(f"C4 tokens={int(lens.sum())} min={lens.min()} max={lens.max()}", flush=True)
    cache = q.KVCache(lens, 512, 64, q.BF16)
    d = cache.describe()
    total = int(d.total_rows)  # every page, padding included
    tmp = q.DeviceBuffer(total * 576 * 4)
    q.check(q.lib().qmla_fill_normal_f32(tmp.ptr, total * 576, 77, 0.0, 1.0, None))
    q.check(q.lib().qmla_f32_to_bf16(tmp.ptr, d.rows, total * 576, None))
    tmp.free()
    cache.set_lengths(lens)
    ql, qr = O.normal((64, 128, 512), 72), O.normal((64, 128, 64), 73)
    s = 192 ** -0.5
    out, lse = run(q, cache, ql, qr, s)
    assert np.isfinite(out).all() and np.isfinite(lse).all()
    pool = cache.read_rows()
    offs = cache.offsets()
    pick = list(range(64))
    rows = np.concatenate([bf16_to_f32(pool[offs[b]:offs[b] + lens[b]]) for b in pick])
    del pool
    sel_lens = lens[pick]
    sel_offs = np.concatenate([[0], np.cumsum(sel_lens)[:-1]]).astype(np.int64)
    ref, rlse = O.decode_absorbed(ql[pick], qr[pick], rows, sel_offs, sel_lens, s)
    for i, b in enumerate(pick):
        err = rel_err(out[b], ref[i])
        print(f"C4 seq {b} T={lens[b]} rel_err={err:.2e}", flush=True)
        assert err < TOL_BF16
        np.testing.assert_allclose(lse[b], rlse[i], atol=2e-2)
    # Another split count cuts the sequences elsewhere, so P and the bf16
    # partials round differently: each run stays within ~5e-3 of the oracle
    # (above), two runs within the sum, on every sequence.
    out2, lse2 = run(q, cache, ql, qr, s, splits=97)
    for i, b in enumerate(pick):
        assert rel_err(out2[b], ref[i]) < TOL_BF16
        np.testing.assert_allclose(lse2[b], rlse[i], atol=2e-2)
    per_seq = [rel_err(out2[b], out[b]) for b in range(64)]
    print(f"C4 splits=97 vs default: max per-sequence rel_err={max(per_seq):.2e}", flush=True)
    assert max(per_seq) < 1e-2
    np.testing.assert_allclose(lse2, lse, atol=5e-3)


def test_decode_rows_beyond_one_pass(qmla_gpu):
    """256 query rows (128 heads x 2 new tokens) run as two row passes."""
    q = qmla_gpu
    lens = [300, 65]
    cache, rows, offs = make_cache(q, lens, 512, 64, q.BF16, 81)
    ql, qr = O.normal((2, 256, 512), 82), O.normal((2, 256, 64), 83)
    out, _ = run(q, cache, ql, qr, 0.07)
    ref, _ = O.decode_absorbed(ql, qr, rows, offs, lens, 0.07)
    assert rel_err(out, ref) < TOL_BF16


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_decode_empty_sequence_and_splits(qmla_gpu, dtype):
    q = qmla_gpu
    dt = q.F32 if dtype == "f32" else q.BF16
    lens = [0, 33, 1, 700]
    cache, rows, offs = make_cache(q, lens, 512, 64, dt, 91, cap_extra=3)
    ql, qr = O.normal((4, 32, 512), 92), O.normal((4, 32, 64), 93)
    ref, rlse = O.decode_absorbed(ql, qr, rows, offs, lens, 0.09)
    tol = TOL_F32 if dtype == "f32" else TOL_BF16
    for splits in (0, 1, 5, 64):
        out, lse = run(q, cache, ql, qr, 0.09, splits=splits)
        np.testing.assert_array_equal(out[0], 0.0)
        assert np.all(np.isneginf(lse[0]))
        assert rel_err(out[1:], ref[1:]) < tol
        np.testing.assert_allclose(lse[1:], rlse[1:], atol=tol)


def test_decode_argument_errors(qmla_gpu):
    q = qmla_gpu
    cache, _, _ = make_cache(q, [10, 10], 512, 64, q.BF16, 5)
    ql = q.DeviceBuffer(2 * 16 * 512 * 4)
    qr = q.DeviceBuffer(2 * 16 * 64 * 4)
    out = q.DeviceBuffer(2 * 16 * 512 * 4)
    need = q.decode_workspace_bytes(cache, 2, 16)
    ws = q.DeviceBuffer(need)
    with pytest.raises(q.QmlaError) as e:
        q.decode_absorbed(cache, 2, 16, ql, qr, 0.1, out, workspace=ws, workspace_bytes=need - 1)
    assert e.value.status == 7
    with pytest.raises(q.QmlaError) as e:
        q.decode_absorbed(cache, 3, 16, ql, qr, 0.1, out, workspace=ws, workspace_bytes=need)
    assert e.value.status == 2
    with pytest.raises(q.QmlaError) as e:
        q.decode_absorbed(cache, 2, 16, ql, qr, float("inf"), out, workspace=ws, workspace_bytes=need)
    assert e.value.status == 1


@pytest.mark.parametrize("rows_m", [16, 128])
def test_decode_bf16_growing_scores_restart(qmla_gpu, rows_m):
    """Scores that grow along the context by far more than the kernel's
    reference slack force the segment-restart path; the result must still
    match the oracle."""
    q = qmla_gpu
    lens = np.array([2000, 700], np.int32)
    ql, qr = O.normal((2, rows_m, 512), 120), O.normal((2, rows_m, 64), 121)
    rows = O.normal((int(lens.sum()), 576), 122) * 0.1
    # c_t drifts along the mean query direction of each sequence: s_t grows ~ t
    off = 0
    for b, T in enumerate(lens):
        d = ql[b].mean(0)
        d /= np.linalg.norm(d)
        ramp = np.linspace(0.0, 200.0, T, dtype=np.float32)[:, None]
        rows[off:off + T, :512] += ramp * d[None, :]
        off += T
    cache = q.KVCache(lens, 512, 64, q.BF16)
    bits = bf16_bits(rows)
    cache.write_pool(bits)
    cache.set_lengths(lens)
    out, lse = run(q, cache, ql, qr, 0.05)
    ref, rlse = O.decode_absorbed(ql, qr, bf16_to_f32(bits), np.array([0, 2000], np.int64), lens, 0.05)
    err = rel_err(out, ref)
    print(f"growing scores rows={rows_m} rel_err={err:.2e} lse range {rlse.min():.1f}..{rlse.max():.1f}")
    assert np.isfinite(out).all()
    assert err < TOL_BF16
    # |s| reaches tens of nats here, so bf16 rounding of q moves lse by ~0.1
    np.testing.assert_allclose(lse, rlse, atol=0.5)


@pytest.mark.parametrize("rows_m,q_bf16", [(48, False), (64, True), (33, True), (128, False)])
def test_decode_bf16_mixed_lengths_sweep(qmla_gpu, rows_m, q_bf16):
    """Latent 512/64 with 33..128 query rows (the 2- and 4-wave kernels),
    f32 and bf16 queries, lengths from 1 to a few tiles past a piece,
    empty sequences in between, and several split counts."""
    q = qmla_gpu
    lens = [1, 0, 31, 32, 33, 700, 5000, 0, 64, 2049]
    cache, rows, offs = make_cache(q, lens, 512, 64, q.BF16, 900 + rows_m, cap_extra=3)
    b = len(lens)
    ql, qr = O.normal((b, rows_m, 512), 901), O.normal((b, rows_m, 64), 902)
    if q_bf16:
        ql, qr = bf16_to_f32(bf16_bits(ql)), bf16_to_f32(bf16_bits(qr))
    ref, rlse = O.decode_absorbed(ql, qr, rows, offs, np.asarray(lens, np.int32), 0.06)
    for splits in (0, 7, 300):
        out, lse = run(q, cache, ql, qr, 0.06, splits=splits, q_dtype=q.BF16 if q_bf16 else q.F32)
        err = rel_err(out, ref)
        print(f"rows={rows_m} q_bf16={q_bf16} splits={splits} rel_err={err:.2e}", flush=True)
        assert np.isfinite(out).all()
        assert err < TOL_BF16
        empty = np.asarray(lens) == 0
        assert np.all(out[empty] == 0) and np.all(np.isneginf(lse[empty]))
        np.testing.assert_allclose(lse[~empty], rlse[~empty], atol=2e-2)


@pytest.mark.parametrize("rows_m", [16, 128])
def test_decode_bf16_large_batch_lds_plan(qmla_gpu, rows_m):
    """More than 64 sequences: the blocks plan their segments through LDS
    (up to 64 they plan in registers).  150 ragged sequences with empty ones,
    the narrow (16 rows) and the 4-wave (128 rows) kernels, two split counts."""
    q = qmla_gpu
    lens = O.uniform_int(150, 77, 0, 400).astype(np.int32)
    lens[::17] = 0
    cache, rows, offs = make_cache(q, lens, 512, 64, q.BF16, 1300 + rows_m)
    b = len(lens)
    ql, qr = O.normal((b, rows_m, 512), 1301), O.normal((b, rows_m, 64), 1302)
    ref, rlse = O.decode_absorbed(ql, qr, rows, offs, lens, 0.07)
    empty = lens == 0
    for splits in (0, 300):
        out, lse = run(q, cache, ql, qr, 0.07, splits=splits)
        err = rel_err(out, ref)
        print(f"batch={b} rows={rows_m} splits={splits} rel_err={err:.2e}", flush=True)
        assert err < TOL_BF16
        assert np.all(out[empty] == 0) and np.all(np.isneginf(lse[empty]))
        np.testing.assert_allclose(lse[~empty], rlse[~empty], atol=2e-2)
