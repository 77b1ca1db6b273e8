"""CPU tests that pin the 2-bit packed MoE oracle (oracle/moe_oracle.c)
before it is trusted: the reference's known-answer test (src/simd.rs:51-65),
closed forms over all four codes, a dense float64 matmul of the unpacked
weights, and a float64 numpy restatement of QMoELayer::forward
(src/moe.rs:40-130) written from the mathematics (stable arg-sort, softmax
over every expert, SwiGLU, weighted sum)."""
import numpy as np
import pytest

import oracle as O
from helpers import rel_err


def unpack_dense(packed: np.ndarray) -> np.ndarray:
    """[rows, n] bytes -> [rows, 4n] weights in {-1, 0, 1, 2}: weight 4j + q
    of a row is bits 2q..2q+1 of byte j, minus one."""
    p = packed.astype(np.int64)
    w = np.stack([(p >> (2 * q)) & 3 for q in range(4)], axis=-1) - 1
    return w.reshape(p.shape[0], -1).astype(np.float64)


def test_simd_kat():
    """src/simd.rs:51-65: byte 0x58 = codes (0, 2, 1, 1) = weights
    (-1, 1, 0, 0); activations (2, 3, 4, 5), scale 1.5 -> 1.5."""
    got = O.fused_dequantize_and_dot(np.array([0x58], np.uint8), np.array([2, 3, 4, 5], np.float32), 1.5)
    assert abs(got - 1.5) < 1e-5


@pytest.mark.parametrize("byte,factor", [(0x55, 0.0), (0xAA, 1.0), (0x00, -1.0), (0xFF, 2.0)])
def test_dot_closed_forms(byte, factor):
    """All codes equal c: the dot is (c - 1) * sum(a) * scale."""
    a = O.normal((256,), 3)
    got = O.fused_dequantize_and_dot(np.full(64, byte, np.uint8), a, 0.75)
    want = factor * float(a.astype(np.float64).sum()) * 0.75
    assert abs(got - want) <= 1e-5 * float(np.abs(a).sum())


def test_dot_bit_order_single_codes():
    """Code q of a byte multiplies activation 4j + q: a one-hot activation
    reads back each 2-bit field separately."""
    rng_bytes = O.uniform_int(16, 5, 0, 255).astype(np.uint8)
    for k in range(64):
        a = np.zeros(64, np.float32)
        a[k] = 1.0
        want = ((int(rng_bytes[k // 4]) >> (2 * (k % 4))) & 3) - 1
        assert O.fused_dequantize_and_dot(rng_bytes, a, 1.0) == want


def test_dot_ignores_trailing_activations_and_bytes():
    """num_bytes = min(len(packed), len(act) / 4) (src/simd.rs:15)."""
    p = np.full(10, 0xAA, np.uint8)
    a = np.arange(1, 23, dtype=np.float32)  # 22 activations -> 5 bytes used
    assert O.fused_dequantize_and_dot(p, a, 1.0) == float(a[:20].sum())
    assert O.fused_dequantize_and_dot(p[:3], a, 1.0) == float(a[:12].sum())


@pytest.mark.parametrize("out_f,in_f,batch", [(64, 128, 1), (33, 2048, 3), (2048, 1408, 2), (5, 12, 4)])
def test_packed_forward_is_dense_matmul(out_f, in_f, batch):
    packed = O.uniform_int(out_f * (in_f // 4), out_f + in_f, 0, 255).astype(np.uint8).reshape(out_f, -1)
    scales = O.normal((out_f,), 7, 0.1)
    x = O.normal((batch, in_f), 8)
    got = O.packed_forward(packed, scales, out_f, in_f, x)
    want = (x.astype(np.float64) @ unpack_dense(packed).T) * scales.astype(np.float64)
    assert rel_err(got, want) < 1e-5


def test_packed_forward_reference_bench_pattern():
    """The bench's repeating bytes 0x58 0xA7 0x2E 0xE4 decode to the weight
    cycle (-1,1,0,0, 2,0,1,1, 1,2,1,-1, -1,0,1,2)."""
    packed, scales = O.bench_packed_data(3, 16)
    np.testing.assert_array_equal(unpack_dense(packed)[0],
                                  [-1, 1, 0, 0, 2, 0, 1, 1, 1, 2, 1, -1, -1, 0, 1, 2])
    x = O.bench_moe_input(1, 16)
    got = O.packed_forward(packed, scales, 3, 16, x)
    want = (x.astype(np.float64) @ unpack_dense(packed).T) * scales
    assert rel_err(got, want) < 1e-6


def moe_f64(W: O.MoEWeights, xs: np.ndarray):
    """float64 restatement: logits, stable descending arg-sort, softmax over
    all experts, top-k weights, SwiGLU experts, sum over the chosen experts."""
    x = xs.astype(np.float64)
    logits = x @ W.gate_weight.astype(np.float64).T
    order = np.argsort(-logits, axis=1, kind="stable")[:, :W.top_k]
    p = np.exp(logits - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    out = np.zeros_like(x)
    for t in range(x.shape[0]):
        for e in order[t]:
            g = (unpack_dense(W.gate_packed[e]) @ x[t]) * W.gate_scales[e]
            u = (unpack_dense(W.up_packed[e]) @ x[t]) * W.up_scales[e]
            h = g / (1.0 + np.exp(-g)) * u
            out[t] += (unpack_dense(W.down_packed[e]) @ h) * W.down_scales[e] * p[t, e]
    return out, order, np.take_along_axis(p, order, 1)


@pytest.mark.parametrize("E,k,H,I,T", [(8, 2, 64, 128, 5), (6, 3, 128, 64, 3), (4, 4, 32, 48, 2)])
def test_moe_forward_matches_f64(E, k, H, I, T):
    W = O.random_moe_weights(E, k, H, I, 100 + E)
    xs = O.normal((T, H), 9)
    out, idx, wts = O.moe_forward(W, xs, return_routing=True)
    ref, ridx, rw = moe_f64(W, xs)
    np.testing.assert_array_equal(idx, ridx)
    np.testing.assert_allclose(wts, rw, rtol=1e-5)
    assert rel_err(out, ref) < 1e-5


def test_moe_ties_keep_lowest_expert_index():
    """Equal logits: the stable sort keeps ascending expert order, so the
    lowest indices win (src/moe.rs:71)."""
    W = O.random_moe_weights(6, 2, 32, 32, 7)
    W.gate_weight[:] = 0.0  # every logit 0 -> all tied
    xs = O.normal((2, 32), 1)
    out, idx, wts = O.moe_forward(W, xs, return_routing=True)
    np.testing.assert_array_equal(idx, [[0, 1], [0, 1]])
    np.testing.assert_allclose(wts, np.full((2, 2), 1 / 6), rtol=1e-6)
    assert rel_err(out, moe_f64(W, xs)[0]) < 1e-5


def test_moe_identical_experts_all_selected():
    """top_k = num_experts with identical experts: the weights sum to one,
    so the output is the single expert's SwiGLU output."""
    W = O.random_moe_weights(4, 4, 64, 32, 11)
    for a in (W.gate_packed, W.up_packed, W.down_packed, W.gate_scales, W.up_scales, W.down_scales):
        a[:] = a[0]
    xs = O.normal((3, 64), 2)
    out, _, wts = O.moe_forward(W, xs, return_routing=True)
    np.testing.assert_allclose(wts.sum(1), 1.0, rtol=1e-6)
    x = xs.astype(np.float64)
    g = (x @ unpack_dense(W.gate_packed[0]).T) * W.gate_scales[0]
    u = (x @ unpack_dense(W.up_packed[0]).T) * W.up_scales[0]
    y = ((g / (1 + np.exp(-g)) * u) @ unpack_dense(W.down_packed[0]).T) * W.down_scales[0]
    assert rel_err(out, y) < 1e-5


def test_moe_no_experts_gives_zeros():
    """src/moe.rs:46-48."""
    W = O.random_moe_weights(1, 1, 16, 16, 3)
    W.num_experts, W.top_k = 0, 0
    out = O.moe_forward(W, O.normal((2, 16), 4))
    np.testing.assert_array_equal(out, 0.0)
