"""Writes tests/golden/golden.npz: golden vectors for the MLA path.

The reference (Rust + candle, a git-fetched fork) cannot be built in this
image, so these vectors come from an independent float64 numpy restatement of
the reference's math, written separately from oracle/mla_oracle.c:

  * SplitMix64 -> Box-Muller input generator (same definition as the oracle)
  * RoPE table / interleaved RoPE            src/model.rs:55-84
  * YaRN scales                              src/model.rs:46-52, :160-173
  * LayerNorm, Linear, softmax               src/model.rs:126-146 (candle ops)
  * MlaAttention::forward_with_cache         src/model.rs:256-307
  * fused_prefill_attn / causal mask          src/attention_kernel.rs:14-31, :64-107
  * the reference's own tiling-invariance cases, src/attention_kernel.rs:140-197
    (generator sin(i * seed) + 0.5; the expected value is the eager form)

Run:  python tests/golden/make_golden.py   (takes a few seconds)
"""
from __future__ import annotations

import os

import numpy as np

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden.npz")
GOLD = np.uint64(0x9E3779B97F4A7C15)


def splitmix64_at(seed: int, idx: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + (idx.astype(np.uint64) + np.uint64(1)) * GOLD
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def normal(shape, seed: int, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    i = np.arange(n, dtype=np.uint64)
    a = splitmix64_at(seed, 2 * i)
    b = splitmix64_at(seed, 2 * i + np.uint64(1))
    u1 = ((a >> np.uint64(11)).astype(np.float64) + 1.0) / 9007199254740992.0
    u2 = (b >> np.uint64(11)).astype(np.float64) / 9007199254740992.0
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (std * z).astype(np.float32).reshape(shape)


def yarn_mscale(scale, m):
    return 1.0 if scale <= 1.0 else 0.1 * m * np.log(scale) + 1.0


def scales(dn, dr):
    rope_mscale = yarn_mscale(40.0, 1.0) / yarn_mscale(40.0, 0.707)
    softmax_scale = (dn + dr) ** -0.5 * yarn_mscale(40.0, 0.707) ** 2
    return rope_mscale, softmax_scale


def rope_table(pos0, n, d, mscale):
    inv = 1.0 / 10000.0 ** (2.0 * np.arange(d // 2) / d)
    ang = (pos0 + np.arange(n))[:, None] * inv[None, :]
    return np.cos(ang) * mscale, np.sin(ang) * mscale


def apply_rope(x, cos, sin):
    """x [..., s, d] with interleaved pairs; cos/sin [s, d/2]."""
    e, o = x[..., 0::2], x[..., 1::2]
    y = np.empty_like(x)
    y[..., 0::2] = e * cos - o * sin
    y[..., 1::2] = o * cos + e * sin
    return y


def layer_norm(x, w, b, eps=1e-6):
    mu = x.mean(-1, keepdims=True)
    var = ((x - mu) ** 2).mean(-1, keepdims=True)
    return (x - mu) / np.sqrt(var + eps) * w + b


def softmax(x):
    m = x.max(-1, keepdims=True)
    e = np.exp(x - m)
    return e / e.sum(-1, keepdims=True)


def attention(qn, qr, k, kr, v, scale, causal, q_offset=0):
    s = (qn @ np.swapaxes(k, -1, -2) + qr @ np.swapaxes(kr, -1, -2)) * scale
    if causal:
        rows = q_offset + np.arange(s.shape[-2])[:, None]
        cols = np.arange(s.shape[-1])[None, :]
        s = np.where(rows < cols, -np.inf, s)
    return softmax(s) @ v


def weights(hidden, H, dn, dr, dv, r, seed):
    shapes = [("wq", (H * (dn + dr), hidden)), ("bq", (H * (dn + dr),)), ("wkva", (r + dr, hidden)),
              ("bkva", (r + dr,)), ("ln_w", (r,)), ("ln_b", (r,)), ("wkvb", (H * (dn + dv), r)),
              ("bkvb", (H * (dn + dv),)), ("wo", (hidden, H * dv)), ("bo", (hidden,))]
    w = {k: normal(s, seed + i, 0.02).astype(np.float64) for i, (k, s) in enumerate(shapes)}
    w["ln_w"] = (w["ln_w"].astype(np.float32) + np.float32(1.0)).astype(np.float64)
    return w


def forward_with_cache(w, xs, latent, H, dn, dr, dv, r):
    """src/model.rs:256-307 with the cache decompressed from latent rows."""
    b, s, hidden = xs.shape
    Tc = latent.shape[1]
    rm, sc = scales(dn, dr)
    q = (xs @ w["wq"].T + w["bq"]).reshape(b, s, H, dn + dr).transpose(0, 2, 1, 3)
    cos, sin = rope_table(Tc, s, dr, rm)
    qn, qr = q[..., :dn], apply_rope(q[..., dn:], cos, sin)
    kva = xs @ w["wkva"].T + w["bkva"]
    c_new = layer_norm(kva[..., :r], w["ln_w"], w["ln_b"])
    kpe_new = apply_rope(kva[..., r:], cos, sin)
    c_all = np.concatenate([latent[..., :r], c_new], 1)
    kpe_all = np.concatenate([latent[..., r:], kpe_new], 1)
    kvb = (c_all @ w["wkvb"].T + w["bkvb"]).reshape(b, Tc + s, H, dn + dv).transpose(0, 2, 1, 3)
    k, v = kvb[..., :dn], kvb[..., dn:]
    kr = kpe_all[:, None]
    ctx = attention(qn, qr, k, kr, v, sc, causal=False)
    ctx = ctx.transpose(0, 2, 1, 3).reshape(b, s, H * dv)
    return ctx @ w["wo"].T + w["bo"], np.concatenate([c_new, kpe_new], -1)


def ref_make_tensor(b, h, s, d, seed):
    """src/attention_kernel.rs:140-145, evaluated in f32 as the reference does."""
    i = np.arange(b * h * s * d, dtype=np.float32)
    return (np.sin(i * np.float32(seed)) + np.float32(0.5)).astype(np.float32).reshape(b, h, s, d)


def main():
    g = {}
    # 1. generator head (pins the oracle's RNG)
    g["rng_seed1_head"] = normal((64,), 1)
    g["splitmix_1234567_head"] = splitmix64_at(1234567, np.arange(5, dtype=np.uint64))

    # 2. C1: tiny MLA decode step (fp32, B1, H8, hidden 512, r64, dn32, dr16, dv32, 256 cached)
    H, hidden, dn, dr, dv, r, Tc = 8, 512, 32, 16, 32, 64, 256
    w = weights(hidden, H, dn, dr, dv, r, seed=100)
    xs = normal((1, 1, hidden), 7).astype(np.float64)
    latent = normal((1, Tc, r + dr), 5).astype(np.float64)
    out, new_row = forward_with_cache(w, xs, latent, H, dn, dr, dv, r)
    g["c1_out"] = out
    g["c1_new_row"] = new_row
    # same layer, 3 new tokens for 2 sequences (multi-token decode, no mask)
    xs3 = normal((2, 3, hidden), 9).astype(np.float64)
    lat2 = normal((2, Tc, r + dr), 6).astype(np.float64)
    out3, rows3 = forward_with_cache(w, xs3, lat2, H, dn, dr, dv, r)
    g["c1b_out"] = out3
    g["c1b_new_rows"] = rows3

    # 3. the reference's tiling-invariance cases (src/attention_kernel.rs:169-197)
    for name, (b, h, s, d, causal) in {"ref_no_causal_small": (1, 4, 64, 32, False),
                                       "ref_causal_small": (1, 4, 64, 32, True),
                                       "ref_causal_medium": (1, 2, 256, 32, True)}.items():
        q = ref_make_tensor(b, h, s, d, 0.1).astype(np.float64)
        k = ref_make_tensor(b, h, s, d, 0.2).astype(np.float64)
        v = ref_make_tensor(b, h, s, d, 0.3).astype(np.float64)
        half = d // 2
        g[name] = attention(q[..., :half], q[..., half:], k[..., :half], k[..., half:], v, d ** -0.5,
                            causal).astype(np.float32)

    # 4. chunked prefill: 16 new queries after 48 cached keys (rope key shared)
    b, h, P, Cn, dn2, dr2, dv2 = 1, 2, 48, 16, 32, 16, 32
    qn = normal((b, h, Cn, dn2), 21).astype(np.float64)
    qr = normal((b, h, Cn, dr2), 22).astype(np.float64)
    k = normal((b, h, P + Cn, dn2), 23).astype(np.float64)
    kr = normal((b, 1, P + Cn, dr2), 24).astype(np.float64)
    v = normal((b, h, P + Cn, dv2), 25).astype(np.float64)
    g["chunk_out"] = attention(qn, qr, k, kr, v, 0.125, True, q_offset=P)

    # 5. absorbed latent decode over a ragged batch
    lens = np.array([5, 17, 40], np.int64)
    M, r5, dr5 = 4, 64, 16
    cache = normal((int(lens.sum()), r5 + dr5), 31).astype(np.float64)
    ql = normal((3, M, r5), 32).astype(np.float64)
    qrr = normal((3, M, dr5), 33).astype(np.float64)
    outs, lses = [], []
    off = 0
    for i, T in enumerate(lens):
        C = cache[off:off + T]
        s = (ql[i] @ C[:, :r5].T + qrr[i] @ C[:, r5:].T) * 0.1
        m = s.max(-1, keepdims=True)
        e = np.exp(s - m)
        outs.append((e / e.sum(-1, keepdims=True)) @ C[:, :r5])
        lses.append((m + np.log(e.sum(-1, keepdims=True)))[:, 0])
        off += T
    g["ragged_out"] = np.stack(outs)
    g["ragged_lse"] = np.stack(lses)
    np.savez_compressed(OUT, **g)
    print("wrote", OUT, {k: v.shape for k, v in g.items()})


if __name__ == "__main__":
    main()
