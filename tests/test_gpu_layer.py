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
    pool = cache.read_rows().reshape(2, 259, 80)
    assert rel_err(pool[:, 256:], golden["c1b_new_rows"]) < TOL


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
    cache.set_lengths([1, 2])
    with pytest.raises(q.QmlaError) as e:   # lengths differ across the batch
        layer.forward_with_cache(O.normal((2, 1, 512), 1), cache)
    assert e.value.status == 2
    cache.set_lengths([4, 4])
    with pytest.raises(q.QmlaError) as e:   # no room for the new token
        layer.forward_with_cache(O.normal((2, 1, 512), 1), cache)
    assert e.value.status == 6
    wrong = q.KVCache([4], 128, 16, q.F32)
    with pytest.raises(q.QmlaError) as e:
        layer.forward_with_cache(O.normal((1, 1, 512), 1), wrong)
    assert e.value.status == 2


@pytest.mark.parametrize("dims", [
    # hidden, heads, qk_nope, qk_rope, v_dim, kv_lora_rank
    (512, 8, 32, 16, 32, 64),      # the tiny CPU-path shape
    (512, 16, 128, 64, 128, 512),  # V2-Lite head shape (hidden reduced)
])
def test_bf16_cache_prefill_then_decode(qmla_gpu, dims):
    """forward_prefill then forward_with_cache steps over a bf16 latent
    cache: the decode core is the bf16 MFMA kernel; the reference is the
    oracle's f32 decompressed path on the same weights and inputs
    (tolerance 2e-2)."""
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
