"""GPU parity tests of the 2-bit packed path: PackedQMoETensor::forward_simd
(src/tensor.rs:64-95) through qmla_packed_forward and QMoELayer::forward
(src/moe.rs:40-130) through qmla_moe_forward, against the oracle on the
same inputs.

Tolerance 1e-4 (max-abs / max |ref|, f32).  The int8-MFMA path (in_features
a multiple of 128) sums an exact integer form of the activations, so it
lands ~1e-7 from the oracle; the fallback path for other widths repeats the
reference's f32 lane sums in order and must match bit for bit.  Routing
(expert indices) must match exactly."""
import numpy as np
import pytest

import oracle as O
from helpers import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-4


def rand_packed(out_f, in_f, seed):
    p = O.uniform_int(out_f * (in_f // 4), seed, 0, 255).astype(np.uint8).reshape(out_f, in_f // 4)
    s = O.normal((out_f,), seed + 1, 0.1)
    return p, s


@pytest.mark.parametrize("out_f,in_f,batch", [
    (64, 128, 1), (33, 2048, 3), (2048, 1408, 2), (1, 2048, 16), (1408, 2048, 11), (7, 128, 25),
    (40, 8192, 5), (130, 4224, 10)])
def test_packed_forward_mfma_matches_oracle(qmla_gpu, out_f, in_f, batch):
    q = qmla_gpu
    p, s = rand_packed(out_f, in_f, out_f + in_f)
    x = O.normal((batch, in_f), batch)
    got = q.PackedQMoETensor.from_bytes(p, (out_f, in_f), s).forward_simd(x)
    ref = O.packed_forward(p, s, out_f, in_f, x)
    err = rel_err(got, ref)
    print(f"out={out_f} in={in_f} batch={batch} rel_err={err:.2e}", flush=True)
    assert err < 1e-6


@pytest.mark.parametrize("out_f,in_f,batch", [(5, 12, 4), (64, 64, 3), (130, 1000, 2), (3, 2, 2)])
def test_packed_forward_fallback_is_bit_exact(qmla_gpu, out_f, in_f, batch):
    q = qmla_gpu
    p, s = rand_packed(out_f, in_f, 3 * out_f + in_f)
    x = O.normal((batch, in_f), 17)
    got = q.PackedQMoETensor.from_bytes(p, (out_f, in_f), s).forward_simd(x)
    np.testing.assert_array_equal(got, O.packed_forward(p, s, out_f, in_f, x))


def test_packed_forward_unaligned_input_uses_fallback(qmla_gpu):
    """x not 16-byte aligned: the fallback kernel runs (bit-exact with the
    oracle) instead of the MFMA kernel's 16-byte loads."""
    q = qmla_gpu
    p, s = rand_packed(64, 256, 31)
    x = O.normal((3, 256), 32)
    t = q.PackedQMoETensor.from_bytes(p, (64, 256), s)
    buf = q.DeviceBuffer.from_numpy(np.concatenate([np.zeros(1, np.float32), x.reshape(-1)]))
    out = q.DeviceBuffer(3 * 64 * 4)
    t.forward(buf.ptr + 4, 3, out)
    q.check(q.lib().qmla_stream_synchronize(None))
    np.testing.assert_array_equal(out.to_numpy(np.float32, (3, 64)), O.packed_forward(p, s, 64, 256, x))


def test_packed_forward_simd_kat(qmla_gpu):
    """src/simd.rs:51-65 through the device path."""
    t = qmla_gpu.PackedQMoETensor.from_bytes(np.array([[0x58]], np.uint8), (1, 4), np.array([1.5], np.float32))
    got = t.forward_simd(np.array([[2, 3, 4, 5]], np.float32))
    assert abs(float(got[0, 0]) - 1.5) < 1e-5


@pytest.mark.parametrize("byte,factor", [(0x55, 0.0), (0xAA, 1.0), (0x00, -1.0), (0xFF, 2.0)])
def test_packed_forward_closed_forms(qmla_gpu, byte, factor):
    out_f, in_f = 48, 1024
    x = O.normal((3, in_f), 5)
    s = O.normal((out_f,), 6, 0.5)
    got = qmla_gpu.PackedQMoETensor.from_bytes(np.full((out_f, in_f // 4), byte, np.uint8), (out_f, in_f),
                                               s).forward_simd(x)
    want = factor * x.astype(np.float64).sum(1)[:, None] * s[None, :]
    assert np.abs(got - want).max() <= 1e-6 * max(1.0, np.abs(x).sum(1).max())


def test_packed_forward_reference_bench_pattern(qmla_gpu):
    """The reference bench's tensor (benches/packed_tensor.rs:10-35):
    1408 x 2048, bytes 0x58 0xA7 0x2E 0xE4 repeating, 16 input rows."""
    p, s = O.bench_packed_data(1408, 2048)
    x = O.bench_moe_input(16, 2048)
    got = qmla_gpu.PackedQMoETensor.from_bytes(p, (1408, 2048), s).forward_simd(x)
    assert rel_err(got, O.packed_forward(p, s, 1408, 2048, x)) < 1e-6


def test_packed_forward_nonfinite_row_is_nan_alone(qmla_gpu):
    p, s = rand_packed(32, 256, 9)
    x = O.normal((3, 256), 10)
    x[1, 7] = np.inf
    got = qmla_gpu.PackedQMoETensor.from_bytes(p, (32, 256), s).forward_simd(x)
    assert np.isnan(got[1]).all()
    ref = O.packed_forward(p, s, 32, 256, x)
    assert rel_err(got[[0, 2]], ref[[0, 2]]) < 1e-6


def test_packed_forward_zero_rows_and_errors(qmla_gpu):
    q = qmla_gpu
    p, s = rand_packed(16, 128, 11)
    t = q.PackedQMoETensor.from_bytes(p, (16, 128), s)
    np.testing.assert_array_equal(t.forward_simd(np.zeros((2, 128), np.float32)), 0.0)
    assert q.packed_workspace_bytes(16, 128, 4) == 0   # no workspace: registers and LDS only
    with pytest.raises(q.QmlaError) as e:
        q.packed_workspace_bytes(16, -1, 4)
    assert e.value.status == 2


def test_moe_workspace_too_small(qmla_gpu):
    q = qmla_gpu
    W = O.random_moe_weights(4, 2, 128, 128, 21)
    layer = moe_layer(q, W)
    need = layer.workspace_bytes(3)
    xs = q.DeviceBuffer.from_numpy(O.normal((3, 128), 22))
    out = q.DeviceBuffer(3 * 128 * 4)
    ws = q.DeviceBuffer(need)
    with pytest.raises(q.QmlaError) as e:
        layer.forward_device(xs, 3, out, ws, need - 1)
    assert e.value.status == 7


def moe_layer(q, W: O.MoEWeights):
    cfg = q.MoEConfig(W.num_experts, W.top_k, W.hidden_dim, W.intermediate_dim)
    experts = [((W.gate_packed[e], W.gate_scales[e]), (W.up_packed[e], W.up_scales[e]),
                (W.down_packed[e], W.down_scales[e])) for e in range(W.num_experts)]
    return q.QMoELayer(cfg, W.gate_weight, experts)


def check_moe(q, W, xs, label):
    out, idx, wts = moe_layer(q, W).forward(xs, return_routing=True)
    ref, ridx, rw = O.moe_forward(W, xs, return_routing=True)
    np.testing.assert_array_equal(idx, ridx)
    # The gate logits are f32 dot products over the hidden size summed in
    # different orders; a weight exp(l - max) / sum inherits the logits'
    # absolute error (~1e-5 for logits of ~100 in the bench layer).
    np.testing.assert_allclose(wts, rw, rtol=1e-4, atol=1e-7)
    err = rel_err(out, ref)
    print(f"{label}: rel_err={err:.2e}", flush=True)
    assert np.isfinite(out).all()
    assert err < TOL


@pytest.mark.parametrize("E,k,H,I,T", [
    (8, 2, 128, 256, 5),      # both GEMVs on the MFMA path
    (32, 4, 64, 256, 16),     # reference toy dims: gate/up fallback, down MFMA
    (16, 2, 256, 128, 300),   # many tokens per expert: several tiles a bin
    (6, 6, 128, 100, 4),      # top_k = num_experts; down on the fallback
    (64, 8, 512, 384, 33),    # 2112 logits: ranked by the routing kernel
    (128, 8, 256, 128, 16),   # 2048 logits, 128 experts: ranked in the GEMV blocks
    (8, 2, 128, 128, 256)])   # 256 tokens, the most the GEMV blocks rank
def test_moe_forward_matches_oracle(qmla_gpu, E, k, H, I, T):
    W = O.random_moe_weights(E, k, H, I, 1000 + E + H)
    xs = O.normal((T, H), 2000 + T)
    check_moe(qmla_gpu, W, xs, f"E={E} k={k} H={H} I={I} T={T}")


def test_moe_forward_default_bench_shape_random(qmla_gpu):
    """benches/moe_layer.rs:465-469 sizes: 16 tokens, 32 experts, top-4,
    hidden 2048, intermediate 1408 (random packed experts)."""
    W = O.random_moe_weights(32, 4, 2048, 1408, 77)
    check_moe(qmla_gpu, W, O.normal((16, 2048), 78), "default bench shape")


def test_moe_forward_reference_bench_layer(qmla_gpu):
    """make_moe_layer / generate_input of benches/moe_layer.rs:68-90."""
    W = O.bench_moe_weights(32, 4, 2048, 1408)
    check_moe(qmla_gpu, W, O.bench_moe_input(16, 2048), "reference bench layer")


@pytest.mark.parametrize("E,k,H,I,T", [
    (4, 2, 4352, 256, 3),     # hidden past one 4096-code LDS slab: ring path, two slabs
    (1, 1, 128, 128, 1),      # one expert, one token
    (3, 1, 512, 1152, 2)])    # intermediate 1152: ring path for the down GEMV
def test_moe_forward_other_paths(qmla_gpu, E, k, H, I, T):
    W = O.random_moe_weights(E, k, H, I, 3000 + H)
    check_moe(qmla_gpu, W, O.normal((T, H), 3100 + T), f"E={E} k={k} H={H} I={I} T={T}")


def test_moe_nonfinite_token_stays_in_its_row(qmla_gpu):
    """A NaN activation poisons its own token's output only."""
    q = qmla_gpu
    W = O.random_moe_weights(8, 2, 256, 256, 41)
    xs = O.normal((4, 256), 42)
    xs[2, 5] = np.nan
    out = moe_layer(q, W).forward(xs)
    assert np.isnan(out[2]).all()
    ref = O.moe_forward(W, xs)
    keep = [0, 1, 3]
    assert rel_err(out[keep], ref[keep]) < TOL


def test_moe_ties_pick_lowest_indices(qmla_gpu):
    W = O.random_moe_weights(6, 2, 128, 128, 5)
    W.gate_weight[:] = 0.0
    out, idx, wts = moe_layer(qmla_gpu, W).forward(O.normal((3, 128), 6), return_routing=True)
    np.testing.assert_array_equal(idx, np.tile([0, 1], (3, 1)))
    np.testing.assert_allclose(wts, 1 / 6, rtol=1e-6)


def test_moe_no_experts_and_bad_top_k(qmla_gpu):
    q = qmla_gpu
    layer = q.QMoELayer(q.MoEConfig(0, 0, 64, 64), np.zeros((0, 64), np.float32), [])
    np.testing.assert_array_equal(layer.forward(O.normal((2, 64), 1)), 0.0)
    W = O.random_moe_weights(2, 2, 64, 64, 3)
    W.top_k = 3
    with pytest.raises(q.QmlaError) as e:
        moe_layer(q, W).workspace_bytes(4)
    assert e.value.status == 2


@pytest.mark.parametrize("E,k,H,I,T", [
    (64, 6, 256, 384, 1024),  # prefill-sized: ~10 tiles a bin, bins split over 10 blocks
    (4, 2, 100, 256, 64),     # gate/up on the fallback, down on MFMA with its own pass 1, ~3 tiles a bin
])
def test_moe_forward_prefill_sized_bins(qmla_gpu, E, k, H, I, T):
    """Many (token, expert) pairs per expert: each bin spans several tiles
    of 10 pairs, which the blocks of the expert's slices share (tiles s,
    s + slices, ...)."""
    W = O.random_moe_weights(E, k, H, I, 5000 + E + T)
    check_moe(qmla_gpu, W, O.normal((T, H), 5100 + T), f"E={E} k={k} H={H} I={I} T={T}")


@pytest.mark.parametrize("H,I", [(256, 256), (100, 384)])
def test_moe_forward_skewed_routing(qmla_gpu, H, I):
    """Every token ranks expert 0 first: its bin holds all 200 tokens (20
    tiles) while the other experts share the second choices, so the hot
    bin is split over the expert's slices."""
    E, k, T = 8, 2, 200
    W = O.random_moe_weights(E, k, H, I, 6000 + H)
    W.gate_weight[0] = 0.5  # with x ~ N(1, 1), expert 0's logit is ~0.5 H
    xs = (O.normal((T, H), 6001) + 1.0).astype(np.float32)
    out, idx, _ = moe_layer(qmla_gpu, W).forward(xs, return_routing=True)
    assert (idx[:, 0] == 0).all()
    check_moe(qmla_gpu, W, xs, f"skewed H={H} I={I}")
