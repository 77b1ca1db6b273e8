"""GPU parity tests of prefill attention (qmla_fused_prefill_attn and the
eager entry points), i.e. fused_prefill_attn / reference_eager_attn of
src/attention_kernel.rs:64-134, including the chunk offset of
make_causal_mask (:14-31).

Tolerances: f32 inputs 1e-4 (max-abs / max |ref|); bf16 inputs with f32
accumulation 2e-2.  The reference side is the oracle on the same inputs
(bf16 values exactly)."""
import numpy as np
import pytest

import oracle as O
from helpers import bf16_bits, bf16_to_f32, rel_err

pytestmark = pytest.mark.gpu

TOL_F32, TOL_BF16 = 1e-4, 2e-2


def _ref_make_tensor(b, h, s, d, seed):
    i = np.arange(b * h * s * d, dtype=np.float32)
    return (np.sin(i * np.float32(seed)) + np.float32(0.5)).astype(np.float32).reshape(b, h, s, d)


def inputs(b, h, sq, sk, dn, dr, dv, krh, seed):
    return [O.normal(sh, seed + i) for i, sh in enumerate(
        [(b, h, sq, dn), (b, h, sq, dr), (b, h, sk, dn), (b, krh, sk, dr), (b, h, sk, dv)])]


class _Lazy:
    """bf16 bit arrays that convert to f32 only for the slices a test reads."""

    def __init__(self, bits):
        self.bits = bits

    def __getitem__(self, idx):
        return bf16_to_f32(self.bits[idx])

    def __array__(self, dtype=None, copy=None):
        return bf16_to_f32(self.bits)


def gpu_prefill(q, arrs, scale, causal, q_offset=0, bf16=False):
    if bf16:
        bits = [O.to_bf16_bits(a) for a in arrs]
        out = q.prefill_numpy(*bits, scale, causal, q_offset=q_offset, dtype=q.BF16)
        return bf16_to_f32(out), [_Lazy(x) for x in bits]
    return q.prefill_numpy(*arrs, scale, causal, q_offset=q_offset, dtype=q.F32), arrs


@pytest.mark.parametrize("name,b,h,s,d,causal", [
    ("ref_no_causal_small", 1, 4, 64, 32, False),
    ("ref_causal_small", 1, 4, 64, 32, True),
    ("ref_causal_medium", 1, 2, 256, 32, True)])
@pytest.mark.parametrize("bf16", [False, True])
def test_reference_tiling_cases(qmla_gpu, golden, name, b, h, s, d, causal, bf16):
    """The reference's own cases (src/attention_kernel.rs:169-197): fused
    with nope/rope halves vs eager, max-abs < 1e-3 in f32."""
    q = qmla_gpu
    qq, kk, vv = (_ref_make_tensor(b, h, s, d, sd) for sd in (0.1, 0.2, 0.3))
    half = d // 2
    arrs = [qq[..., :half], qq[..., half:], kk[..., :half], kk[..., half:], vv]
    fused, used = gpu_prefill(q, arrs, d ** -0.5, causal, bf16=bf16)
    if bf16:
        ref = O.fused_prefill_attn(*[np.asarray(u) for u in used], d ** -0.5, causal)
        assert rel_err(fused, ref) < TOL_BF16
        return
    eager = q.reference_eager_attn_numpy(qq, kk, vv, d ** -0.5, causal)
    assert np.abs(fused - eager).max() < 1e-3
    assert rel_err(fused, golden[name]) < TOL_F32
    assert rel_err(eager, golden[name]) < TOL_F32


@pytest.mark.parametrize("bf16", [False, True])
def test_chunked_prefill_golden(qmla_gpu, golden, bf16):
    q = qmla_gpu
    arrs = inputs(1, 2, 16, 64, 32, 16, 32, 1, 21)
    # the golden uses seeds 21..25 in this order
    out, used = gpu_prefill(q, arrs, 0.125, True, q_offset=48, bf16=bf16)
    if bf16:
        ref = O.fused_prefill_attn(*[np.asarray(u) for u in used], 0.125, True, q_offset=48)
        assert rel_err(out, ref) < TOL_BF16
    else:
        assert rel_err(out, golden["chunk_out"]) < TOL_F32


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("sq,sk,causal,krh", [(300, 300, True, 1), (257, 257, True, 3), (100, 333, False, 1),
                                              (1, 1, True, 1), (65, 65, True, 1), (200, 200, True, 1)])
def test_prefill_shapes_mla_dims(qmla_gpu, bf16, sq, sk, causal, krh):
    q = qmla_gpu
    arrs = inputs(2, 3, sq, sk, 128, 64, 128, krh, 100 + sq)
    out, used = gpu_prefill(q, arrs, 192 ** -0.5, causal, bf16=bf16)
    ref = O.fused_prefill_attn(*[np.asarray(u) for u in used], 192 ** -0.5, causal)
    err = rel_err(out, ref)
    print(f"sq={sq} sk={sk} causal={causal} krh={krh} bf16={bf16} rel_err={err:.2e}")
    assert err < (TOL_BF16 if bf16 else TOL_F32)


def test_prefill_bf16_shape_sweep(qmla_gpu):
    """Shapes that leave waves of a 256-row block without query rows (and
    some DMA waves idle), partial last key tiles, one query row, chunks with
    an offset and keys beyond the queries, non-causal and causal."""
    q = qmla_gpu
    cases = [  # b, h, sq, sk, q_offset, causal
        (1, 2, 33, 33, 0, True), (1, 1, 97, 97, 0, True), (2, 1, 129, 129, 0, True),
        (1, 3, 225, 225, 0, True), (1, 2, 1, 500, 0, False), (1, 2, 5, 300, 295, True),
        (2, 2, 40, 1000, 960, True), (1, 9, 70, 70, 0, False), (3, 1, 256, 256, 0, True),
        (1, 1, 300, 700, 400, True)]
    for i, (b, h, sq, sk, off, causal) in enumerate(cases):
        arrs = inputs(b, h, sq, sk, 128, 64, 128, 1, 800 + 10 * i)
        out, used = gpu_prefill(q, arrs, 192 ** -0.5, causal, q_offset=off, bf16=True)
        ref = O.fused_prefill_attn(*[np.asarray(u) for u in used], 192 ** -0.5, causal, q_offset=off)
        err = rel_err(out, ref)
        print(f"b={b} h={h} sq={sq} sk={sk} off={off} causal={causal} rel_err={err:.2e}", flush=True)
        assert np.isfinite(out).all()
        assert err < TOL_BF16, (b, h, sq, sk, off, causal, err)


@pytest.mark.parametrize("causal", [True, False])
def test_prefill_bf16_growing_scores_restart(qmla_gpu, causal):
    """Keys drift along a direction every query shares, so the scores grow
    along the keys by up to ~60 bits beyond the first key tile's maximum --
    far past the kernel's reference slack.  The block-restart path runs and
    the result must still match the oracle."""
    q = qmla_gpu
    s = 600
    arrs = inputs(1, 2, s, s, 128, 64, 128, 1, 400)
    u = O.normal((128,), 450)
    u /= np.linalg.norm(u)
    arrs[0] += 2.0 * u
    arrs[2] += np.linspace(0.0, 150.0, s, dtype=np.float32)[:, None] * u
    out, used = gpu_prefill(q, arrs, 192 ** -0.5, causal, bf16=True)
    ref = O.fused_prefill_attn(*[np.asarray(x) for x in used], 192 ** -0.5, causal)
    err = rel_err(out, ref)
    print(f"growing scores causal={causal} rel_err={err:.2e}")
    assert np.isfinite(out).all()
    assert err < TOL_BF16


def test_rope_key_shared_equals_broadcast(qmla_gpu):
    """k_rope_heads = 1 (latent layout) == the reference's head-broadcast copy."""
    q = qmla_gpu
    qn, qr, k, kr1, v = inputs(1, 4, 96, 96, 128, 64, 128, 1, 7)
    krh = np.ascontiguousarray(np.broadcast_to(kr1, (1, 4, 96, 64)))
    a = q.prefill_numpy(qn, qr, k, kr1, v, 0.1, True)
    b = q.prefill_numpy(qn, qr, k, krh, v, 0.1, True)
    np.testing.assert_array_equal(a, b)


def test_prefill_v2lite_causal_full_size_bf16(qmla_gpu):
    """C3: batch 4, seq 2048, 16 heads, dn 128, dr 64, dv 128, bf16 in, f32
    accumulate.  The oracle checks every one of the 64 (b, h) pairs."""
    q = qmla_gpu
    b, h, s = 4, 16, 2048
    arrs = inputs(b, h, s, s, 128, 64, 128, 1, 300)
    out, used = gpu_prefill(q, arrs, 192 ** -0.5, True, bf16=True)
    assert np.isfinite(out).all()
    ref = O.fused_prefill_attn(*used, 192 ** -0.5, True)
    worst = 0.0
    for bi in range(b):
        for hi in range(h):
            err = rel_err(out[bi, hi], ref[bi, hi])
            worst = max(worst, err)
            assert err < TOL_BF16, (bi, hi, err)
    print(f"C3 all 64 (b, h) pairs: worst rel_err={worst:.2e}", flush=True)


def _c5_pairs(heads: int):
    """16 (b, h) pairs of the chunked case whose flat index b * heads + h
    takes every residue mod 8 twice.  Blocks are dealt to the 8 XCDs
    round-robin and, with the query tiles paired per (b, h), a pair's two
    tiles sit at block indices 8 apart on XCD (b * heads + h) mod 8; the
    oracle compares both tiles (all 512 rows) of each pair."""
    flat = [i * 64 + (i % 8) for i in range(16)]
    return [(f // heads, f % heads) for f in flat]


def test_chunked_prefill_v3_full_size_bf16(qmla_gpu):
    """C5: 8 sequences x (8192 cached + 512 new), 128 heads, causal within
    the chunk and full to the cache.  Oracle on 16 (b, h) pairs covering
    every XCD position of the paired block order."""
    q = qmla_gpu
    b, h, P, C = 8, 128, 8192, 512
    arrs = inputs(b, h, C, P + C, 128, 64, 128, 1, 500)
    out, used = gpu_prefill(q, arrs, 192 ** -0.5, True, q_offset=P, bf16=True)
    assert np.isfinite(out).all()
    pairs = _c5_pairs(h)
    assert sorted({(bi * h + hi) % 8 for bi, hi in pairs}) == list(range(8))
    sub = [np.stack([used[i][bi, hi] for bi, hi in pairs])[:, None] for i in (0, 1, 2)]
    sub.insert(3, np.stack([used[3][bi, 0] for bi, _ in pairs])[:, None])
    sub.append(np.stack([used[4][bi, hi] for bi, hi in pairs])[:, None])
    ref = O.fused_prefill_attn(*sub, 192 ** -0.5, True, q_offset=P)
    for i, (bi, hi) in enumerate(pairs):
        for tile in range(2):
            rows = slice(256 * tile, 256 * (tile + 1))
            err = rel_err(out[bi, hi, rows], ref[i, 0, rows])
            print(f"C5 (b={bi}, h={hi}, xcd {(bi * h + hi) % 8}, tile {tile}) rel_err={err:.2e}", flush=True)
            assert err < TOL_BF16


def test_eager_entry_points(qmla_gpu):
    q = qmla_gpu
    qq, kk, vv = (O.normal((2, 2, 70, 32), 600 + i) for i in range(3))
    ref = O.reference_eager_attn(qq, kk, vv, 0.2, True)
    assert rel_err(q.reference_eager_attn_numpy(qq, kk, vv, 0.2, True), ref) < TOL_F32
    out = bf16_to_f32(q.reference_eager_attn_numpy(bf16_bits(qq), bf16_bits(kk), bf16_bits(vv), 0.2, True,
                                                   dtype=q.BF16))
    ref_b = O.reference_eager_attn(*(bf16_to_f32(bf16_bits(x)) for x in (qq, kk, vv)), 0.2, True)
    assert rel_err(out, ref_b) < TOL_BF16


def test_prefill_unsupported_bf16_dims_raise(qmla_gpu):
    q = qmla_gpu
    arrs = [bf16_bits(x) for x in inputs(1, 1, 8, 8, 40, 8, 40, 1, 9)]
    with pytest.raises(q.QmlaError) as e:
        q.prefill_numpy(*arrs, 0.1, True, dtype=q.BF16)
    assert e.value.status == 3
