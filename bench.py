#!/usr/bin/env python3
"""bench.py -- MI355X benchmark of the MLA attention hot path.

Headline workload (one step = one absorbed-latent decode over the batch's
latent cache, i.e. one attention layer's decode: the decode kernel and its
split-KV merge):
  128 heads, kv_lora_rank 512, rope 64, batch 64, ragged contexts
  U[1024, 32768] + 1 (seeded), bf16 latent cache, scale 1/sqrt(192).
value = decode tokens/s (batch / step time), the step time from one HIP event
pair on the launch stream around exactly --steps back-to-back steps (after
--warmup untimed ones).  roofline: latent-cache bytes (sum_b T_b * 1152 B)
per step against 8 TB/s; traffic: HBM bytes per step from the committed
rocprofv3 counter summary (profiles/decode_v3_pmc.md).

Secondary lines (same JSON object, "secondary"): 16-head decode (batch 32,
4096 + 1 tokens), causal prefill (batch 4, 2048 tokens, 16 heads) and chunked
prefill (batch 8, 8192 cached + 512 new, 128 heads), the prefills in TFLOP/s
of unmasked attention work (MHA form, dqk 192 + dv 128) against the
2.5 PFLOP/s bf16 dense peak; and one full MLA layer decode step
(forward_with_cache: projections, latent append, decode core, W_UV, o_proj)
at V2-Lite head shapes, in tokens/s and weight + cache bytes per step; and the
2-bit packed MoE layer forward at the reference bench's default sizes, in
tokens/s and the active experts' packed bytes per step against 8 TB/s.

Inputs are generated on the device (seeded) before the timed region.  The
decode caches rotate over replicas totalling >= 2 GB so consecutive steps
never re-read a cache that could still sit in the 256 MB Infinity Cache.
cpu_baseline: the oracle's C restatement of the decode on the host cores,
on a bounded sample (>= 10 s), scaled to the full batch.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
       python bench.py --calibrate   (copy kernel for scaling PMC counters)
       python bench.py --moe-only    (the MoE layer line alone, for profiling)
       python bench.py --layer-only  (the MLA layer decode step alone, for profiling)
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import math
import os
import sys
import time
import types

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "qmoe-rs_amd"))

import numpy as np  # noqa: E402

import qmla  # noqa: E402
from qmla import synth  # noqa: E402

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
F32_PEAK_TFLOPS = 157.3    # dense f32 MFMA
ROW_ELEMS = 576            # kv_lora_rank 512 + rope 64
ROW_BYTES = ROW_ELEMS * 2  # bf16
SCALE = 192 ** -0.5
METRIC = "MLA decode tok/s + HBM GB/s (% of peak); prefill TFLOP/s (% MFMA peak)"
# Warm-up time of every secondary line (beyond its --warmup steps): the
# clock settles ~20 ms into sustained load after a start from idle.
WARM_MS = 25.0


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def fill_bf16(dst_ptr: int, n: int, seed: int, tmp: qmla.DeviceBuffer, stream):
    """dst (bf16, n elements) <- N(0,1) via an f32 staging buffer."""
    done = 0
    cap = tmp.nbytes // 4
    while done < n:
        m = min(cap, n - done)
        qmla.check(qmla.lib().qmla_fill_normal_f32(tmp.ptr, m, seed + done, 0.0, 1.0, qmla._sh(stream)))
        qmla.check(qmla.lib().qmla_f32_to_bf16(tmp.ptr, dst_ptr + 2 * done, m, qmla._sh(stream)))
        done += m


STATS = {}  # per-step event statistics of the last time_steps call


def time_steps(step, steps: int, warmup: int, stream, min_warm_ms: float = 0.0, max_extra: int = 1 << 30):
    """Runs warmup steps, then times exactly `steps` back-to-back steps on
    the launch stream twice, synchronised on both sides of each pass.  Pass
    1 is bracketed by one HIP event pair and gives the mean: nothing is
    enqueued between its steps.  Pass 2 records an event after every step
    for the per-step distribution (median, p10, p90 in STATS); each such
    event leaves the GPU idle for ~3 us before the next step, which pass 1
    excludes.  Returns (wall ms per step, event ms per step) of pass 1.

    With min_warm_ms the warmup continues past `warmup` steps until that
    much GPU time has run (the secondary lines: the power controller's
    transient after a start from idle lasts ~20 ms of sustained load, and a
    fixed step count covers very different times for 40 us and 1 ms
    steps).  The headline uses exactly `warmup` steps."""
    for i in range(warmup):
        step(i)
    stream.sync()
    done = warmup
    if min_warm_ms > 0:
        e0, e1 = qmla.Event(), qmla.Event()
        e0.record(stream)
        step(done)
        done += 1
        e1.record(stream)
        stream.sync()
        per = max(e0.elapsed_ms(e1), 1e-3)
        extra = max(0, min(int(math.ceil(min_warm_ms / per)), max_extra - 1))
        for i in range(extra):
            step(done + i)
        done += extra
        stream.sync()
    warmup = done
    e0, e1 = qmla.Event(), qmla.Event()
    t0 = time.perf_counter()
    e0.record(stream)
    for i in range(steps):
        step(warmup + i)
    e1.record(stream)
    stream.sync()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    mean = e0.elapsed_ms(e1) / steps
    ev = [qmla.Event() for _ in range(steps + 1)]
    ev[0].record(stream)
    for i in range(steps):
        step(warmup + steps + i)
        ev[i + 1].record(stream)
    stream.sync()
    per = np.array([ev[i].elapsed_ms(ev[i + 1]) for i in range(steps)])
    STATS.clear()
    STATS.update({"warmup_steps": warmup, "p10_ms": float(np.percentile(per, 10)), "median_ms": float(np.median(per)),
                  "p90_ms": float(np.percentile(per, 90)), "min_ms": float(per.min()), "max_ms": float(per.max()),
                  "per_step_events": True,
                  "pass": "a second pass of the same K steps with an event after every step; each event leaves "
                          "the GPU idle ~3 us before the next step, and the clock runs a little higher across "
                          "those gaps, so this distribution differs from ms_per_step (the first pass, no events "
                          "between steps)"})
    return wall, mean


class DecodeBench:
    """Absorbed decode over a bf16 latent cache, rotating cache replicas."""

    def __init__(self, lens, heads, stream, seed, min_rotation_bytes=2 << 30):
        self.lens = np.asarray(lens, np.int32)
        self.batch, self.heads, self.stream = len(self.lens), heads, stream
        self.tokens = int(self.lens.sum())
        self.cache_bytes = self.tokens * ROW_BYTES
        self.replicas = max(2, math.ceil(min_rotation_bytes / self.cache_bytes))
        tmp = qmla.DeviceBuffer(min(self.tokens * ROW_ELEMS, 256 << 20) * 4)
        self.caches = []
        for r in range(self.replicas):
            c = qmla.KVCache(self.lens, 512, 64, qmla.BF16)
            d = c.describe()  # fill every page, padding included
            fill_bf16(d.rows, d.total_rows * ROW_ELEMS, seed + 1000003 * r, tmp, stream)
            c.set_lengths(self.lens, stream)
            self.caches.append(c)
        nq = self.batch * heads
        self.q_lat = qmla.DeviceBuffer(nq * 512 * 2)
        self.q_rope = qmla.DeviceBuffer(nq * 64 * 2)
        fill_bf16(self.q_lat.ptr, nq * 512, seed + 7, tmp, stream)
        fill_bf16(self.q_rope.ptr, nq * 64, seed + 8, tmp, stream)
        self.out = qmla.DeviceBuffer(nq * 512 * 4)
        self.lse = qmla.DeviceBuffer(nq * 4)
        self.ws_bytes = qmla.decode_workspace_bytes(self.caches[0], self.batch, heads)
        self.ws = qmla.DeviceBuffer(self.ws_bytes)
        stream.sync()
        tmp.free()

    def step(self, i):
        qmla.decode_absorbed(self.caches[i % self.replicas], self.batch, self.heads, self.q_lat, self.q_rope,
                             SCALE, self.out, self.lse, qmla.BF16, self.ws, self.ws_bytes, stream=self.stream)

    def run(self, steps, warmup, min_warm_ms=0.0):
        wall, ev = time_steps(self.step, steps, warmup, self.stream, min_warm_ms)
        t = ev * 1e-3
        gbs = self.cache_bytes / t / 1e9
        flops = self.tokens * self.heads * (2 * ROW_ELEMS + 2 * 512)
        return {
            "tok_s": self.batch / t,
            "ms_per_step": ev,
            "wall_ms_per_step": wall,
            "hbm_gbs": gbs,
            "hbm_frac": gbs / HBM_PEAK_GBS,
            "mfma_tflops": flops / t / 1e12,
            "bytes_per_step": self.cache_bytes,
            "tokens": self.tokens,
            "replicas": self.replicas,
            "step_ms": dict(STATS),
        }


class PrefillBench:
    """bf16 causal prefill (optionally after a cached prefix)."""

    def __init__(self, b, h, sq, sk, q_offset, stream, seed):
        self.dims = qmla.PrefillDims(b, h, sq, sk, 128, 64, 128, 1, q_offset)
        self.stream = stream
        shapes = [b * h * sq * 128, b * h * sq * 64, b * h * sk * 128, b * sk * 64, b * h * sk * 128]
        tmp = qmla.DeviceBuffer(min(max(shapes), 256 << 20) * 4)
        self.bufs = []
        for i, n in enumerate(shapes):
            buf = qmla.DeviceBuffer(n * 2)
            fill_bf16(buf.ptr, n, seed + 31 * i, tmp, stream)
            self.bufs.append(buf)
        self.out = qmla.DeviceBuffer(b * h * sq * 128 * 2)
        stream.sync()
        tmp.free()
        C, P = sq, q_offset
        pairs = C * P + C * (C + 1) // 2  # unmasked (query, key) pairs per (b, h)
        self.flops = b * h * pairs * 2 * (192 + 128)

    def step(self, i):
        qmla.fused_prefill_attn(*self.bufs, SCALE, True, dims=self.dims, dtype=qmla.BF16, out=self.out,
                                stream=self.stream)

    def run(self, steps, warmup, min_warm_ms=0.0):
        wall, ev = time_steps(self.step, steps, warmup, self.stream, min_warm_ms)
        tf = self.flops / (ev * 1e-3) / 1e12
        return {"tflops": tf, "mfma_frac": tf / BF16_PEAK_TFLOPS, "ms_per_step": ev,
                "wall_ms_per_step": wall, "gflop_per_step": self.flops / 1e9,
                "tflops_at_median": self.flops / (STATS["median_ms"] * 1e-3) / 1e12, "step_ms": dict(STATS)}


def v2lite_weights(seed, hidden=2048, heads=16):
    """Host f32 weights of one MlaAttention at V2-Lite head shapes (dn 128,
    dr 64, dv 128, r 512): N(0, 0.02^2), LayerNorm weight 1 + N(0, 0.02^2)."""
    rng = np.random.default_rng(seed)
    H, dn, dr, dv, r = heads, 128, 64, 128, 512

    def nrm(*shape):
        return (rng.standard_normal(shape, dtype=np.float32) * np.float32(0.02)).astype(np.float32)

    w = types.SimpleNamespace(hidden=hidden, heads=H, dn=dn, dr=dr, dv=dv, r=r, softmax_scale=None)
    w.wq, w.bq = nrm(H * (dn + dr), hidden), nrm(H * (dn + dr))
    w.wkva, w.bkva = nrm(r + dr, hidden), nrm(r + dr)
    w.ln_w, w.ln_b = (1.0 + nrm(r)).astype(np.float32), nrm(r)
    w.wkvb, w.bkvb = nrm(H * (dn + dv), r), nrm(H * (dn + dv))
    w.wo, w.bo = nrm(hidden, H * dv), nrm(hidden)
    return w


def weight_bytes_of(w, proj_dtype=qmla.F32):
    """Weight bytes a step streams: 4 per weight (f32, held as bf16 hi + lo
    halves), 2 with bf16 operands (the hi halves)."""
    return (4 if proj_dtype == qmla.F32 else 2) * (w.wq.size + w.wkva.size + w.wkvb.size + w.wo.size)


class LayerDecodeBench:
    """MlaAttention::forward_with_cache (src/model.rs:256-307), one new token
    per sequence: f32 projections, LayerNorm + RoPE of the new latent rows
    into a bf16 latent cache, the absorbed decode core, W_UV and o_proj.
    V2-Lite head shapes (hidden 2048, 16 heads, dn 128, dr 64, dv 128,
    r 512), batch 32, 4096 cached tokens per sequence; weights N(0, 0.02^2),
    activations N(0, 1), seeded.  Steps rotate over `layers` layer copies
    and `caches` caches (caches >= 512 MB in all, with the weights
    ~0.7 GB), so no step re-reads weights or rows the 256 MB Infinity Cache
    could still hold.  Each cache grows by one token per use in growth mode:
    each sequence holds exactly its 4096 rows (16 pages of 256) and takes a
    page from the pool's free list (sized for 512 more tokens per sequence
    at creation) when it crosses a page boundary.  proj_dtype BF16 runs the
    projections with bf16 operands (qmla_layer_set_projection_dtype)."""

    def __init__(self, stream, seed, batch=32, ctx=4096, hidden=2048, heads=16, layers=2,
                 min_cache_bytes=512 << 20, proj_dtype=qmla.F32):
        r, dr = 512, 64
        ws = [v2lite_weights(seed + 7 * i, hidden, heads) for i in range(layers)]
        self.layers = [qmla.MlaLayer(w) for w in ws]
        for layer in self.layers:
            layer.set_projection_dtype(proj_dtype)
        self.weight_bytes = weight_bytes_of(ws[0], proj_dtype)
        self.batch, self.ctx, self.stream = batch, ctx, stream
        ncache = max(2, math.ceil(min_cache_bytes / (batch * ctx * ROW_BYTES)))
        tmp = qmla.DeviceBuffer(64 << 20)
        self.caches = []
        for i in range(ncache):
            c = qmla.KVCache([ctx] * batch, r, dr, qmla.BF16, grow=True, pool_rows=batch * (ctx + 512))
            d = c.describe()
            fill_bf16(d.rows, d.total_rows * ROW_ELEMS, seed + 1 + 1000003 * i, tmp, stream)
            c.set_lengths([ctx] * batch, stream)
            self.caches.append(c)
        stream.sync()
        tmp.free()
        self.xs = qmla.DeviceBuffer(batch * hidden * 4)
        qmla.check(qmla.lib().qmla_fill_normal_f32(self.xs.ptr, batch * hidden, seed + 2, 0.0, 1.0,
                                                   qmla._sh(stream)))
        self.out = qmla.DeviceBuffer(batch * hidden * 4)
        self.ws_bytes = self.layers[0].workspace_bytes(self.caches[0], batch, 1)
        self.ws = qmla.DeviceBuffer(self.ws_bytes)
        stream.sync()

    def step(self, i):
        layer, cache = self.layers[i % len(self.layers)], self.caches[i % len(self.caches)]
        qmla.check(qmla.lib().qmla_layer_forward_with_cache(
            layer.handle, self.xs.ptr, self.batch, 1, cache.handle, self.out.ptr, self.ws.ptr,
            self.ws_bytes, qmla._sh(self.stream)))

    def run(self, steps, warmup, min_warm_ms=0.0):
        nc = len(self.caches)
        assert (warmup + 2 * steps) / nc <= 512, "each page pool has room for 512 new tokens per sequence"
        pools0 = [c.pool_info() for c in self.caches]
        # extra warmup steps only while every pool keeps room for the timed steps
        wall, ev = time_steps(self.step, steps, warmup, self.stream, min_warm_ms,
                              max_extra=512 * nc - warmup - 2 * steps - nc)
        warmup = STATS["warmup_steps"]
        assert all(c.pool_info()[0] == p[0] for c, p in zip(self.caches, pools0)), "a pool grew: a step allocated"
        t = ev * 1e-3
        mean_ctx = self.ctx + (warmup + (steps + 1) / 2.0) / nc
        hbm = self.weight_bytes + self.batch * mean_ctx * ROW_BYTES
        pages = sum((p[1] - c.pool_info()[1]) // 256 for c, p in zip(self.caches, pools0))
        return {"tok_s": self.batch / t, "ms_per_step": ev, "wall_ms_per_step": wall,
                "weight_bytes": self.weight_bytes, "bytes_per_step": hbm, "tb_s": hbm / t / 1e12,
                "hbm_frac": hbm / t / 1e12 / (HBM_PEAK_GBS / 1e3), "pages_taken": int(pages),
                "rotation": {"layers": len(self.layers), "caches": nc,
                             "bytes": nc * self.batch * self.ctx * ROW_BYTES + len(self.layers) * self.weight_bytes},
                "step_ms": dict(STATS)}


class LayerPrefillBench:
    """MlaAttention::forward_prefill (src/model.rs:193-253) at the causal
    prefill workload's shapes: batch 4 x 2048 tokens, hidden 2048, V2-Lite
    heads (16, dn 128, dr 64, dv 128, r 512), bf16 latent cache; weights
    N(0, 0.02^2), activations N(0, 1), seeded.  One call runs the
    projections and the kv_b decompression (compute_kv, :178-190) as split
    bf16 GEMMs with f32 accumulation, the bf16 MFMA causal attention and
    o_proj, and fills the cache.  The decompression is also timed on its
    own, through qmla_cache_materialise over the same 4 x 2048 cached latent
    rows (the kv_b_proj product batched over heads, plus the gather of the
    rows and the head-broadcast k_rope copy).  proj_dtype BF16 runs the
    projections with bf16 operands (qmla_layer_set_projection_dtype); the
    decompression is then not timed."""

    def __init__(self, stream, seed, batch=4, seq=2048, hidden=2048, heads=16, proj_dtype=qmla.F32):
        H, dr, r = heads, 64, 512
        self.layer = qmla.MlaLayer(v2lite_weights(seed, hidden, heads))
        self.layer.set_projection_dtype(proj_dtype)
        self.proj_dtype = proj_dtype
        self.batch, self.seq, self.heads, self.hidden, self.stream = batch, seq, H, hidden, stream
        self.caches = [qmla.KVCache([seq] * batch, r, dr, qmla.BF16) for _ in range(2)]
        self.xs = qmla.DeviceBuffer(batch * seq * hidden * 4)
        qmla.check(qmla.lib().qmla_fill_normal_f32(self.xs.ptr, batch * seq * hidden, seed + 2, 0.0, 1.0,
                                                   qmla._sh(stream)))
        self.out = qmla.DeviceBuffer(batch * seq * hidden * 4)
        self.ws_bytes = self.layer.prefill_workspace_bytes(self.caches[0], batch, seq)
        self.ws = qmla.DeviceBuffer(self.ws_bytes)
        stream.sync()

    def step(self, i):
        c = self.caches[i % 2]
        c.set_lengths([0] * self.batch, self.stream)
        qmla.check(qmla.lib().qmla_layer_forward_prefill(
            self.layer.handle, self.xs.ptr, self.batch, self.seq, c.handle, self.out.ptr, self.ws.ptr,
            self.ws_bytes, qmla._sh(self.stream)))

    def run(self, steps, warmup, min_warm_ms=0.0):
        b, s, H = self.batch, self.seq, self.heads
        wall, ev = time_steps(self.step, steps, warmup, self.stream, min_warm_ms)
        step_ms = dict(STATS)
        att = b * H * (s * (s + 1) // 2) * 2 * (192 + 128)
        kvb = 2 * b * s * 512 * H * (128 + 128)
        proj = 2 * b * s * self.hidden * (H * 192 + 576 + H * 128)
        gflop = {"attention": att / 1e9, "kv_b_decompress": kvb / 1e9, "projections": proj / 1e9}
        if self.proj_dtype != qmla.F32:
            return {"tok_s": b * s / (ev * 1e-3), "ms_per_step": ev, "wall_ms_per_step": wall,
                    "gflop": gflop, "step_ms": step_ms}
        # the decompression alone, over a cache the steps above filled
        c = self.caches[0]
        n = C.c_size_t()
        qmla.check(qmla.lib().qmla_cache_materialise_workspace_bytes(self.layer.handle, c.handle, 0, b,
                                                                     C.byref(n)))
        k, v = qmla.DeviceBuffer(b * H * s * 128 * 4), qmla.DeviceBuffer(b * H * s * 128 * 4)
        kr = qmla.DeviceBuffer(b * H * s * 64 * 4)
        mws = qmla.DeviceBuffer(max(n.value, 1))

        def mstep(i):
            qmla.check(qmla.lib().qmla_cache_materialise(self.layer.handle, c.handle, 0, b, k.ptr, v.ptr, kr.ptr,
                                                         mws.ptr, n.value, qmla._sh(self.stream)))

        _, evm = time_steps(mstep, steps, 2, self.stream)
        # the split form runs x w = x_hi w_hi + x_lo w_hi + x_hi w_lo (+ the
        # bias columns) as one bf16 GEMM over K' = 3 K + 2 columns padded to
        # a multiple of 64: the bf16 flops the MFMAs execute
        kp = -(-(3 * 512 + 2) // 64) * 64
        kvb_bf16 = kvb * kp / 512
        return {"tok_s": b * s / (ev * 1e-3), "ms_per_step": ev, "wall_ms_per_step": wall,
                "gflop": gflop, "step_ms": step_ms,
                "decompress": {"ms": evm, "gflop": kvb / 1e9,
                               "f32_equivalent_tflops": kvb / (evm * 1e-3) / 1e12,
                               "bf16_gflop_executed": kvb_bf16 / 1e9,
                               "bf16_tflops": kvb_bf16 / (evm * 1e-3) / 1e12,
                               "bf16_mfma_frac": kvb_bf16 / (evm * 1e-3) / 1e12 / BF16_PEAK_TFLOPS,
                               "what": "qmla_cache_materialise over the 4 x 2048 cached rows: the kv_b_proj "
                                       "product as split bf16 GEMMs (x w = x_hi w_hi + x_lo w_hi + x_hi w_lo, "
                                       "f32 accumulation, K' = 3K + 2 padded to 64, batched over heads) plus "
                                       "the gather of the rows into split form and the head-broadcast k_rope "
                                       "copy; bf16_mfma_frac counts the executed bf16 flops against 2.5 PF"}}


class Batch1Sweeps:
    """The reference's batch-1 sweeps (benches/attention.rs:375-429), the
    product's own call shape (src/main.rs:120-135 decodes one token at
    batch 1): MlaAttention::forward_with_cache of one token over a cache of
    `cache_len` tokens, and forward_prefill of `seq_len` tokens, at the
    bench's widths (hidden 2048, 16 heads, kv_lora_rank 512, dn 128, dr 64,
    dv 128), bf16 latent cache, f32 weights and activations.

    Every timed call gets a cache of its own, filled to exactly the point's
    length (the reference times cache.clone() + forward_with_cache, so each
    iteration decodes against the same length), and the calls rotate over
    `layers` layer copies (~1 GB of weights in all), so each call streams
    its weights from HBM as a multi-layer model's step does rather than from
    the 256 MB Infinity Cache."""

    DECODE_LENS = (0, 64, 256, 1024, 4096)   # benches/attention.rs:406
    PREFILL_LENS = (32, 64, 128, 256, 512, 1024, 2048)  # benches/attention.rs:380

    def __init__(self, stream, seed, layers=6, hidden=2048):
        self.stream, self.hidden = stream, hidden
        ws = [v2lite_weights(seed + 11 * i, hidden) for i in range(layers)]
        self.layers = [qmla.MlaLayer(w) for w in ws]
        self.weight_bytes = weight_bytes_of(ws[0])
        self.x = qmla.DeviceBuffer(2048 * hidden * 4)
        qmla.check(qmla.lib().qmla_fill_normal_f32(self.x.ptr, 2048 * hidden, seed + 3, 0.0, 1.0,
                                                   qmla._sh(stream)))
        self.out = qmla.DeviceBuffer(2048 * hidden * 4)

    def _caches(self, n, cap, fill_len):
        tmp = qmla.DeviceBuffer(8 << 20)
        cs = []
        for i in range(n):
            c = qmla.KVCache([cap], 512, 64, qmla.BF16)
            if fill_len:
                d = c.describe()
                fill_bf16(d.rows, d.total_rows * ROW_ELEMS, 9000 + i, tmp, self.stream)
                c.set_lengths([fill_len], self.stream)
            cs.append(c)
        self.stream.sync()
        tmp.free()
        return cs

    def _point(self, fn, steps, warmup):
        wall, ev = time_steps(fn, steps, warmup, self.stream)
        return wall, ev, dict(STATS)

    def decode(self, steps, warmup):
        n = warmup + 2 * steps
        pts = []
        for L in self.DECODE_LENS:
            caches = self._caches(n, L + 1, L)
            wsb = self.layers[0].workspace_bytes(caches[0], 1, 1)
            ws = qmla.DeviceBuffer(wsb)

            def step(i, caches=caches, ws=ws, wsb=wsb):
                qmla.check(qmla.lib().qmla_layer_forward_with_cache(
                    self.layers[i % len(self.layers)].handle, self.x.ptr, 1, 1, caches[i].handle, self.out.ptr,
                    ws.ptr, wsb, qmla._sh(self.stream)))

            wall, ev, st = self._point(step, steps, warmup)
            assert all(list(c.lengths()) == [L + 1] for c in caches)
            pts.append({"cache_len": L, "us_per_token": ev * 1e3, "tok_s": 1e3 / ev,
                        "median_us": st["median_ms"] * 1e3, "p10_us": st["p10_ms"] * 1e3,
                        "p90_us": st["p90_ms"] * 1e3, "wall_us": wall * 1e3,
                        "hbm_bytes": self.weight_bytes + (L + 1) * ROW_BYTES})
            del caches, ws
        return pts

    def prefill(self, steps, warmup):
        n = warmup + 2 * steps
        pts = []
        for S in self.PREFILL_LENS:
            caches = self._caches(n, S, 0)
            wsb = self.layers[0].prefill_workspace_bytes(caches[0], 1, S)
            ws = qmla.DeviceBuffer(wsb)

            def step(i, caches=caches, ws=ws, wsb=wsb, S=S):
                qmla.check(qmla.lib().qmla_layer_forward_prefill(
                    self.layers[i % len(self.layers)].handle, self.x.ptr, 1, S, caches[i].handle, self.out.ptr,
                    ws.ptr, wsb, qmla._sh(self.stream)))

            wall, ev, st = self._point(step, steps, warmup)
            assert all(list(c.lengths()) == [S] for c in caches)
            flops = (2 * S * self.hidden * (16 * 192 + 576 + 16 * 128) + 2 * S * 512 * 16 * 256
                     + 16 * (S * (S + 1) // 2) * 2 * 320)
            pts.append({"seq_len": S, "us_per_call": ev * 1e3, "tok_s": S / (ev * 1e-3),
                        "median_us": st["median_ms"] * 1e3, "p10_us": st["p10_ms"] * 1e3,
                        "p90_us": st["p90_ms"] * 1e3, "wall_us": wall * 1e3,
                        "f32_equivalent_tflops": flops / (ev * 1e-3) / 1e12})
            del caches, ws
        return pts


def cpu_baseline_batch1(min_seconds=1.0):
    """The batch-1 sweeps on the host in the reference's own form (numpy
    with BLAS matmuls: oracle.blas_layer_decode_step over the decompressed
    per-head cache with KVCache::append's cat, oracle.blas_layer_prefill),
    each point repeated for at least `min_seconds`."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O  # checker library, used here only as the CPU baseline

    w = O.MlaWeights.random(2048, 16, 128, 64, 128, 512, seed=98)
    th = blas_threads()
    dec, pre = {}, {}
    x1 = O.normal((1, 1, 2048), 99)
    for L in Batch1Sweeps.DECODE_LENS:
        k, v, kr = O.normal((1, 16, L, 128), 100), O.normal((1, 16, L, 128), 101), O.normal((1, 16, L, 64), 102)
        per, reps = _repeat(lambda: O.blas_layer_decode_step(w, x1, k, v, kr), min_seconds)
        dec[L] = {"us_per_token": per * 1e6, "runs": reps}
    for S in Batch1Sweeps.PREFILL_LENS:
        xs = O.normal((1, S, 2048), 103)
        per, reps = _repeat(lambda: O.blas_layer_prefill(w, xs), min_seconds)
        pre[S] = {"us_per_call": per * 1e6, "tok_s": S / per, "runs": reps}
    return {"cores": th, "kind": "port", "cpu_model": cpu_model(),
            "what": f"the reference's form in numpy on {th} BLAS threads: forward_with_cache with the "
                    f"per-head f32 cache and its cat (oracle.blas_layer_decode_step), forward_prefill with "
                    f"compute_kv and the tiled causal attention (oracle.blas_layer_prefill); each point "
                    f"repeated for >= {min_seconds:.0f} s",
            "decode": dec, "prefill": pre}


def cpu_baseline_layer_prefill(min_seconds=5.0):
    """MlaAttention::forward_prefill (src/model.rs:193-253) in the
    reference's own form on the host (numpy with BLAS matmuls,
    oracle.blas_layer_prefill, checked against the C oracle's layer): one of
    the 4 sequences of 2048 tokens, scaled by 4."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O  # checker library, used here only as the CPU baseline

    w = O.MlaWeights.random(2048, 16, 128, 64, 128, 512, seed=96)
    xs = O.normal((1, 2048, 2048), 97)
    per, reps = _repeat(lambda: O.blas_layer_prefill(w, xs), min_seconds)
    full = per * 4
    th = blas_threads()
    return {"value": 4 * 2048 / full, "unit": "tok/s", "cores": th, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"1 of 4 sequences (2048 tokens) x {reps} runs = {per * reps:.1f} s; scaled by 4 "
                      f"({full * 1e3:.0f} ms per call); the reference's form (f32 projections, compute_kv, "
                      f"tiled causal attention over per-head K/V, o_proj; src/model.rs:193-253) in numpy on "
                      f"{th} BLAS threads (oracle.blas_layer_prefill)"}


def ref_bench_packed(out_f: int, in_f: int):
    """The reference benches' packed tensor (benches/moe_layer.rs:11-29):
    bytes cycling 0x58, 0xA7, 0x2E, 0xE4; scale i = sin(0.05 i) + 1."""
    packed = np.resize(np.array([0x58, 0xA7, 0x2E, 0xE4], np.uint8), out_f * (in_f // 4))
    i = np.arange(out_f, dtype=np.float32)
    return packed.reshape(out_f, in_f // 4), (np.sin(i * np.float32(0.05)) + np.float32(1.0)).astype(np.float32)


def ref_bench_moe(tokens=16, experts=32, top_k=4, hidden=2048, inter=1408):
    """make_moe_layer + generate_input of benches/moe_layer.rs:31-90: every
    expert holds the deterministic pattern above, gate_weight[i] =
    cos(0.07 i), input[i] = sin(0.1 i) + 0.5."""
    gp, gs = ref_bench_packed(inter, hidden)
    dp, ds = ref_bench_packed(hidden, inter)
    gw = np.cos(np.arange(experts * hidden, dtype=np.float32) * np.float32(0.07)).astype(np.float32)
    xs = (np.sin(np.arange(tokens * hidden, dtype=np.float32) * np.float32(0.1)) + np.float32(0.5)).astype(np.float32)
    return (gw.reshape(experts, hidden), [((gp, gs), (gp, gs), (dp, ds))] * experts,
            xs.reshape(tokens, hidden))


class MoEBench:
    """QMoELayer::forward (src/moe.rs:40-130) at the reference bench's default
    sizes (benches/moe_layer.rs:465-469): 16 tokens, 32 experts, top-4,
    hidden 2048, intermediate 1408, 2-bit packed experts, f32 activations.
    The layer is replicated (8 copies, 553 MB of packed weights) and the
    steps rotate over the copies, so no step reads weights the 256 MB
    Infinity Cache could still hold."""

    def __init__(self, stream, replicas=8, tokens=16, experts=32, top_k=4, hidden=2048, inter=1408):
        gw, ex, xs = ref_bench_moe(tokens, experts, top_k, hidden, inter)
        cfg = qmla.MoEConfig(experts, top_k, hidden, inter)
        self.layers = [qmla.QMoELayer(cfg, gw, ex) for _ in range(replicas)]
        self.cfg, self.tokens, self.stream = cfg, tokens, stream
        self.xs = qmla.DeviceBuffer.from_numpy(xs)
        self.out = qmla.DeviceBuffer(tokens * hidden * 4)
        self.idx = qmla.DeviceBuffer(tokens * top_k * 4)
        self.ws_bytes = self.layers[0].workspace_bytes(tokens)
        self.ws = qmla.DeviceBuffer(self.ws_bytes)
        self.expert_bytes = 3 * inter * (hidden // 4) + 4 * (2 * inter + hidden)

    def step(self, i):
        self.layers[i % len(self.layers)].forward_device(self.xs, self.tokens, self.out, self.ws, self.ws_bytes,
                                                         self.idx, None, self.stream)

    def run(self, steps, warmup, min_warm_ms=0.0):
        wall, ev = time_steps(self.step, steps, warmup, self.stream, min_warm_ms)
        active = len(np.unique(self.idx.to_numpy(np.int32, (self.tokens, self.cfg.top_k), self.stream)))
        c = self.cfg
        hbm = active * self.expert_bytes + 4 * (c.num_experts * c.hidden_dim + 2 * self.tokens * c.hidden_dim)
        t = ev * 1e-3
        return {"tok_s": self.tokens / t, "ms_per_step": ev, "wall_ms_per_step": wall,
                "active_experts": active, "bytes_per_step": hbm, "tb_s": hbm / t / 1e12,
                "hbm_frac": hbm / t / 1e12 / (HBM_PEAK_GBS / 1e3), "replicas": len(self.layers),
                "step_ms": dict(STATS)}


def moe_cpu_baseline(min_seconds=5.0):
    """The oracle's QMoELayer::forward restatement (single thread, like the
    reference's loops in src/moe.rs:60-127) on the same 16-token input,
    repeated for at least `min_seconds`."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O  # checker library, used here only as the CPU baseline

    gw, ex, xs = ref_bench_moe()
    (gp, gs), _, (dp, ds) = ex[0]
    E = gw.shape[0]
    rep = lambda a: np.ascontiguousarray(np.broadcast_to(a, (E,) + a.shape))
    W = O.MoEWeights(E, 4, 2048, 1408, gw, rep(gp), rep(gs), rep(gp), rep(gs), rep(dp), rep(ds))
    reps, t0 = 0, time.perf_counter()
    while True:
        O.moe_forward(W, xs)
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds:
            break
    per = dt / reps
    return {"value": xs.shape[0] / per, "unit": "tok/s", "cores": 1, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"the full 16-token step x {reps} runs = {dt:.1f} s on 1 thread "
                      f"({per * 1e3:.0f} ms per step); f32 C restatement (oracle/moe_oracle.c)"}


def cpu_baseline(lens, heads, sample_seqs, min_seconds=10.0):
    """The oracle's absorbed-latent decode (the CPU restatement of the
    reference path), timed on the host cores on a bounded sample of the same
    workload: the first `sample_seqs` sequences, repeated until at least
    `min_seconds` have elapsed, scaled by token count to the full batch.  A
    single-thread figure on a smaller sample is reported beside it."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O  # checker library, used here only as the CPU baseline

    def timed(sample, threads, min_s):
        O.set_num_threads(threads)
        rows = O.normal((int(sample.sum()), ROW_ELEMS), 4242)
        ql = O.normal((len(sample), heads, 512), 4243)
        qr = O.normal((len(sample), heads, 64), 4244)
        offs = np.concatenate([[0], np.cumsum(sample)[:-1]]).astype(np.int64)
        reps, t0 = 0, time.perf_counter()
        while True:
            O.decode_absorbed(ql, qr, rows, offs, sample, SCALE)
            reps += 1
            dt = time.perf_counter() - t0
            if dt >= min_s:
                return dt / reps, reps

    total = float(np.sum(lens))
    threads = O.num_threads()
    sample = np.asarray(lens[:sample_seqs], np.int32)
    per, reps = timed(sample, threads, min_seconds)
    full = per * total / float(sample.sum())
    one = np.asarray(lens[:1], np.int32)
    per1, reps1 = timed(one, 1, min_seconds / 4)
    full1 = per1 * total / float(one.sum())
    O.set_num_threads(threads)
    return {"value": len(lens) / full, "unit": "tok/s", "cores": threads, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"first {len(sample)} of {len(lens)} sequences ({int(sample.sum())} of {int(total)} tokens, "
                      f"{heads} heads) x {reps} runs = {per * reps:.1f} s on {threads} threads; scaled by token "
                      f"count to the full batch ({full * 1e3:.0f} ms per step); absorbed-latent f32 C restatement "
                      f"(oracle/mla_oracle.c), OpenMP over (sequence, row block)",
            "single_thread": {"value": len(lens) / full1, "unit": "tok/s", "cores": 1,
                              "sample": f"sequence 0 ({int(one.sum())} tokens) x {reps1} runs = "
                                        f"{per1 * reps1:.1f} s; {full1:.1f} s per full step"}}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def blas_threads() -> int:
    try:
        import threadpoolctl
        return max([int(i.get("num_threads", 1)) for i in threadpoolctl.threadpool_info()
                    if i.get("user_api") == "blas"] or [1])
    except Exception:
        return 1


def _repeat(fn, min_seconds):
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds:
            return dt / reps, reps


def cpu_baseline_v2lite(sample_seqs=4, batch=32, heads=16, ctx=4096, min_seconds=5.0):
    """The reference's decode attention in its own (decompressed) form on
    the host: for each step, KVCache::append's cat of the cache along T and
    scores / softmax / @ v over the per-head f32 K, V, k_rope
    (src/model.rs:291-303), numpy with the matmuls on BLAS.  Bounded sample:
    `sample_seqs` of the `batch` sequences, scaled by sequence count."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O  # checker library, used here only as the CPU baseline

    b = sample_seqs
    k, v = O.normal((b, heads, ctx, 128), 61), O.normal((b, heads, ctx, 128), 62)
    kr = O.normal((b, heads, ctx, 64), 63)
    kn, vn, krn = O.normal((b, heads, 1, 128), 64), O.normal((b, heads, 1, 128), 65), O.normal((b, heads, 1, 64), 66)
    qn, qr = O.normal((b, heads, 1, 128), 67), O.normal((b, heads, 1, 64), 68)
    per, reps = _repeat(lambda: O.blas_decode_step(qn, qr, k, v, kr, kn, vn, krn, SCALE), min_seconds)
    full = per * batch / b
    th = blas_threads()
    return {"value": batch / full, "unit": "tok/s", "cores": th, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"{b} of {batch} sequences x {reps} steps = {per * reps:.1f} s; scaled by sequence count "
                      f"({full * 1e3:.0f} ms per step); the reference's decompressed form (f32 per-head K/V/k_rope "
                      f"[b,16,4097,d], cache cat + scores + softmax + @v, src/model.rs:291-303) in numpy on "
                      f"{th} BLAS threads (oracle.blas_decode_step)"}


def cpu_baseline_prefill(min_seconds=5.0):
    """The reference's tiled fused_prefill_attn (src/attention_kernel.rs:64-107)
    on the host at the causal workload's shapes (f32, numpy with BLAS
    matmuls): one of the 4 sequences (16 heads x 2048 tokens), scaled by 4."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O  # checker library, used here only as the CPU baseline

    s = 2048
    qn, qr = O.normal((1, 16, s, 128), 71), O.normal((1, 16, s, 64), 72)
    k, kr, v = O.normal((1, 16, s, 128), 73), O.normal((1, 16, s, 64), 74), O.normal((1, 16, s, 128), 75)
    per, reps = _repeat(lambda: O.blas_fused_prefill_attn(qn, qr, k, kr, v, SCALE, True), min_seconds)
    full = per * 4
    flops = 4 * 16 * (s * (s + 1) // 2) * 2 * (192 + 128)
    th = blas_threads()
    return {"value": flops / full / 1e12, "unit": "TFLOP/s", "cores": th, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"1 of 4 sequences (16 heads x 2048 tokens) x {reps} runs = {per * reps:.1f} s; scaled by 4 "
                      f"({full * 1e3:.0f} ms per call); the reference's tiled form (query tiles of "
                      f"{O.tile_size(s)}, full-row softmax, per-head k_rope) in numpy on {th} BLAS threads "
                      f"(oracle.blas_fused_prefill_attn); unmasked-pair flops as the GPU line"}


def cpu_baseline_chunked(heads_sample=8, min_seconds=5.0):
    """The reference's fused_prefill_attn with the chunk's causal offset
    (src/attention_kernel.rs:64-107, make_causal_mask :14-31) on the host at
    the chunked workload's shapes (f32, numpy with BLAS matmuls, per-head
    decompressed K/V): `heads_sample` heads of one of the 8 sequences,
    scaled to the 8 x 128 (sequence, head) pairs."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O  # checker library, used here only as the CPU baseline

    h, sq, off = heads_sample, 512, 8192
    sk = off + sq
    qn, qr = O.normal((1, h, sq, 128), 81), O.normal((1, h, sq, 64), 82)
    k, kr, v = O.normal((1, h, sk, 128), 83), O.normal((1, h, sk, 64), 84), O.normal((1, h, sk, 128), 85)
    per, reps = _repeat(lambda: O.blas_fused_prefill_attn(qn, qr, k, kr, v, SCALE, True, q_offset=off),
                        min_seconds)
    pairs = 8 * 128
    full = per * pairs / h
    flops = pairs * (sq * off + sq * (sq + 1) // 2) * 2 * (192 + 128)
    th = blas_threads()
    return {"value": flops / full / 1e12, "unit": "TFLOP/s", "cores": th, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"{h} of 1024 (sequence, head) pairs x {reps} runs = {per * reps:.1f} s; scaled by "
                      f"{pairs // h} ({full:.1f} s per call); the reference's tiled form with the chunk's causal "
                      f"offset (query tiles of {O.tile_size(sq)}, per-head K/V/k_rope) in numpy on {th} BLAS "
                      f"threads (oracle.blas_fused_prefill_attn); unmasked-pair flops as the GPU line"}


def cpu_baseline_layer(sample_seqs=4, batch=32, ctx=4096, min_seconds=5.0):
    """MlaAttention::forward_with_cache (src/model.rs:256-307) in the
    reference's own form on the host: f32 projections, the decompressed
    per-head cache with KVCache::append's cat, attention and o_proj, numpy
    with BLAS matmuls (oracle.blas_layer_decode_step, checked against the C
    oracle's layer).  V2-Lite widths; `sample_seqs` of the `batch` sequences,
    scaled by sequence count."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O  # checker library, used here only as the CPU baseline

    b = sample_seqs
    w = O.MlaWeights.random(2048, 16, 128, 64, 128, 512, seed=91)
    k, v = O.normal((b, 16, ctx, 128), 92), O.normal((b, 16, ctx, 128), 93)
    kr = O.normal((b, 16, ctx, 64), 94)
    xs = O.normal((b, 1, 2048), 95)
    per, reps = _repeat(lambda: O.blas_layer_decode_step(w, xs, k, v, kr), min_seconds)
    full = per * batch / b
    th = blas_threads()
    return {"value": batch / full, "unit": "tok/s", "cores": th, "kind": "port", "cpu_model": cpu_model(),
            "sample": f"{b} of {batch} sequences x {reps} steps = {per * reps:.1f} s; scaled by sequence count "
                      f"({full * 1e3:.0f} ms per step); the reference's decompressed form (f32 projections, "
                      f"per-head K/V/k_rope [b,16,{ctx + 1},d] with the cache cat, attention, o_proj; "
                      f"src/model.rs:256-307) in numpy on {th} BLAS threads (oracle.blas_layer_decode_step)"}


def copy_calibration(stream, n=256 << 20, reps=4):
    """A plain streaming kernel of known traffic for scaling the rocprofv3
    FETCH_SIZE / WRITE_SIZE counters: qmla_f32_to_bf16 over n elements reads
    4n bytes and writes 2n bytes."""
    src = qmla.DeviceBuffer(n * 4)
    dst = qmla.DeviceBuffer(n * 2)
    qmla.check(qmla.lib().qmla_fill_normal_f32(src.ptr, n, 5, 0.0, 1.0, qmla._sh(stream)))
    for _ in range(reps):
        qmla.check(qmla.lib().qmla_f32_to_bf16(src.ptr, dst.ptr, n, qmla._sh(stream)))
    stream.sync()
    log(f"copy calibration: {reps} x qmla_f32_to_bf16 over {n} elements "
        f"({4 * n} bytes read, {2 * n} bytes written per launch)")


def measured_traffic(name="decode_v3_pmc.md"):
    """HBM bytes per step from a committed rocprofv3 PMC summary (counter
    reads scaled by the copy calibration), or None."""
    path = os.path.join(ROOT, "profiles", name)
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_step:"):
                    return float(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # the first ~1 ms of sustained load runs at the boost clock; 20 warmup
    # steps put the timed steps in the sustained regime
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-sample-seqs", type=int, default=32)
    ap.add_argument("--calibrate", action="store_true",
                    help="only run the copy kernel used to scale the PMC byte counters")
    ap.add_argument("--moe-only", action="store_true",
                    help="only run the 2-bit packed MoE layer line (for profiling)")
    ap.add_argument("--layer-only", action="store_true",
                    help="only run the MLA layer decode step line (for profiling)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only run the two prefill lines (for profiling)")
    ap.add_argument("--layer-prefill-only", action="store_true",
                    help="only run the MLA layer prefill line (for profiling)")
    ap.add_argument("--sweeps-only", action="store_true",
                    help="only run the batch-1 decode and prefill sweeps (for profiling)")
    ap.add_argument("--bf16-projections", action="store_true",
                    help="with --layer-only / --layer-prefill-only: bf16-operand projections")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the decode path shards by batch "
              f"with no exchange, so N GPUs scale the one-GPU number.", file=sys.stderr)
        sys.exit(2)

    dev, cus, arch = qmla.device_info()
    log(f"device {dev} {arch} with {cus} CUs")
    stream = qmla.Stream()
    if args.calibrate:
        copy_calibration(stream)
        return
    if args.moe_only:
        mb = MoEBench(stream)
        print(json.dumps({"moe_layer": mb.run(args.steps, args.warmup, WARM_MS)}), flush=True)
        return
    pdt = qmla.BF16 if args.bf16_projections else qmla.F32
    if args.layer_only:
        lb = LayerDecodeBench(stream, seed=51, proj_dtype=pdt)
        print(json.dumps({"layer_decode_step": lb.run(args.steps, args.warmup, WARM_MS)}), flush=True)
        return
    if args.layer_prefill_only:
        lp = LayerPrefillBench(stream, seed=61, proj_dtype=pdt)
        print(json.dumps({"layer_prefill": lp.run(max(3, args.steps // 5), 3, WARM_MS)}), flush=True)
        return
    if args.sweeps_only:
        sw = Batch1Sweeps(stream, seed=71)
        print(json.dumps({"batch1_decode_sweep": sw.decode(args.steps, args.warmup),
                          "batch1_prefill_sweep": sw.prefill(max(3, args.steps // 2), 3)}), flush=True)
        return
    if args.prefill_only:
        res = {}
        for name, dims in (("causal_prefill", (4, 16, 2048, 2048, 0)), ("chunked_prefill", (8, 128, 512, 8704, 8192))):
            pb = PrefillBench(*dims, stream, seed=31 if name == "causal_prefill" else 41)
            res[name] = pb.run(args.steps, args.warmup, WARM_MS)
            del pb
        print(json.dumps(res), flush=True)
        return

    lens = synth.v3_decode_lengths()
    log(f"v3 decode: batch {len(lens)}, {int(lens.sum())} tokens, {int(lens.sum()) * ROW_BYTES / 1e9:.3f} GB latent")
    dec = DecodeBench(lens, 128, stream, seed=11)
    log(f"replicas {dec.replicas}, workspace {dec.ws_bytes / 1e6:.1f} MB")
    main_res = dec.run(args.steps, args.warmup)
    log("v3 decode", json.dumps(main_res))
    del dec

    secondary = {}
    if not args.no_secondary:
        d2 = DecodeBench(np.full(32, 4097, np.int32), 16, stream, seed=21)
        secondary["v2lite_decode"] = {"workload": "16 heads, batch 32, 4096 cached + 1, bf16 latent", **d2.run(args.steps, args.warmup, WARM_MS)}
        if not args.no_cpu_baseline:
            secondary["v2lite_decode"]["cpu_baseline"] = cpu_baseline_v2lite()
        log("v2lite decode", json.dumps(secondary["v2lite_decode"]))
        del d2
        p3 = PrefillBench(4, 16, 2048, 2048, 0, stream, seed=31)
        secondary["causal_prefill"] = {"workload": "batch 4, 2048 tokens, 16 heads, dn 128 dr 64 dv 128, bf16, causal",
                                       **p3.run(args.steps, args.warmup, WARM_MS)}
        if not args.no_cpu_baseline:
            secondary["causal_prefill"]["cpu_baseline"] = cpu_baseline_prefill()
        log("causal prefill", json.dumps(secondary["causal_prefill"]))
        del p3
        p5 = PrefillBench(8, 128, 512, 8704, 8192, stream, seed=41)
        secondary["chunked_prefill"] = {"workload": "batch 8, 8192 cached + 512 new, 128 heads, bf16, causal in chunk",
                                        **p5.run(args.steps, max(1, args.warmup // 2), WARM_MS)}
        if not args.no_cpu_baseline:
            secondary["chunked_prefill"]["cpu_baseline"] = cpu_baseline_chunked()
        log("chunked prefill", json.dumps(secondary["chunked_prefill"]))
        del p5
        lb = LayerDecodeBench(stream, seed=51)
        secondary["layer_decode_step"] = {
            "workload": "MlaAttention forward_with_cache, hidden 2048, 16 heads, r 512, batch 32, "
                        "4096 cached + 1, f32 weights, bf16 latent cache in growth mode (256-row pages "
                        "taken from a pre-sized pool)",
            **lb.run(args.steps, args.warmup, WARM_MS)}
        if not args.no_cpu_baseline:
            secondary["layer_decode_step"]["cpu_baseline"] = cpu_baseline_layer()
        log("layer decode step", json.dumps(secondary["layer_decode_step"]))
        del lb
        lp = LayerPrefillBench(stream, seed=61)
        secondary["layer_prefill"] = {
            "workload": "MlaAttention forward_prefill, batch 4 x 2048 tokens, hidden 2048, 16 heads, r 512, "
                        "f32 weights (projections as split bf16 GEMMs, f32 accumulation), bf16 latent cache "
                        "(attention on the bf16 MFMA prefill)",
            **lp.run(max(3, args.steps // 5), 3, WARM_MS)}
        if not args.no_cpu_baseline:
            secondary["layer_prefill"]["cpu_baseline"] = cpu_baseline_layer_prefill()
        log("layer prefill", json.dumps(secondary["layer_prefill"]))
        del lp
        # the same two calls with bf16-operand projections (the bf16 tolerance)
        bf16_note = ("projections with bf16 operands (qmla_layer_set_projection_dtype BF16: the weights' bf16 "
                     "halves, activations rounded to bf16, f32 accumulation; the bf16 tolerance, 2e-2), "
                     "bf16 latent cache")
        lb = LayerDecodeBench(stream, seed=51, proj_dtype=qmla.BF16)
        secondary["layer_decode_step_bf16_projections"] = {
            "workload": "MlaAttention forward_with_cache, hidden 2048, 16 heads, r 512, batch 32, 4096 cached "
                        "+ 1, " + bf16_note + "; CPU baseline: layer_decode_step's",
            **lb.run(args.steps, args.warmup, WARM_MS)}
        log("layer decode step, bf16 projections", json.dumps(secondary["layer_decode_step_bf16_projections"]))
        del lb
        lp = LayerPrefillBench(stream, seed=61, proj_dtype=qmla.BF16)
        secondary["layer_prefill_bf16_projections"] = {
            "workload": "MlaAttention forward_prefill, batch 4 x 2048 tokens, hidden 2048, 16 heads, r 512, "
                        + bf16_note + "; CPU baseline: layer_prefill's",
            **lp.run(max(3, args.steps // 5), 3, WARM_MS)}
        log("layer prefill, bf16 projections", json.dumps(secondary["layer_prefill_bf16_projections"]))
        del lp
        sw = Batch1Sweeps(stream, seed=71)
        dsw = sw.decode(args.steps, args.warmup)
        psw = sw.prefill(max(3, args.steps // 2), 3)
        del sw
        cb1 = None if args.no_cpu_baseline else cpu_baseline_batch1()
        if cb1:
            for p in dsw:
                p["cpu_baseline_us_per_token"] = cb1["decode"][p["cache_len"]]["us_per_token"]
            for p in psw:
                p["cpu_baseline_us_per_call"] = cb1["prefill"][p["seq_len"]]["us_per_call"]
        secondary["batch1_decode_sweep"] = {
            "workload": "batch 1, one new token, forward_with_cache at cache_len tokens (benches/attention.rs "
                        "decode_throughput), hidden 2048, 16 heads, r 512, bf16 latent cache, f32 weights "
                        "rotating over 6 layer copies; every call on its own cache of exactly cache_len tokens",
            "points": dsw,
            "cpu_baseline": None if cb1 is None else {k: cb1[k] for k in ("cores", "kind", "cpu_model", "what")}}
        secondary["batch1_prefill_sweep"] = {
            "workload": "batch 1, forward_prefill of seq_len tokens (benches/attention.rs prefill_throughput), "
                        "hidden 2048, 16 heads, r 512, bf16 latent cache, f32 weights rotating over 6 layer "
                        "copies",
            "points": psw,
            "cpu_baseline": None if cb1 is None else {k: cb1[k] for k in ("cores", "kind", "cpu_model", "what")}}
        log("batch-1 sweeps", json.dumps({"decode": dsw, "prefill": psw}))
        mb = MoEBench(stream)
        moe = mb.run(args.steps, args.warmup, WARM_MS)
        del mb
        secondary["moe_layer"] = {
            "workload": "QMoELayer forward, 16 tokens, 32 experts, top-4, hidden 2048, intermediate 1408, "
                        "2-bit packed experts (reference bench pattern), f32 activations, int8 MFMA",
            **moe,
            "roofline": {"bound": "hbm", "achieved": moe["tb_s"] * 1e3, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": moe["hbm_frac"], "traffic": measured_traffic("moe_layer_kernel_trace.md"),
                         "kernel": "whole qmla_moe_forward call (k_moe_logits, k_packed_mfma gate/up and down, "
                                   "k_moe_combine), HIP events on the launch stream",
                         "bytes_per_launch": moe["bytes_per_step"]},
            "cpu_baseline": None if args.no_cpu_baseline else moe_cpu_baseline()}
        log("moe layer", json.dumps(secondary["moe_layer"]))

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(lens, 128, args.cpu_sample_seqs)
        log("cpu baseline", json.dumps(cpu))

    line = {
        "metric": METRIC,
        "value": main_res["tok_s"],
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": main_res["ms_per_step"],
        "wall_ms_per_step": main_res["wall_ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,1) latent cache and absorbed queries generated on device; no checkpoint",
        "config": {
            "workload": "v3 absorbed MLA decode: 128 heads, kv_lora_rank 512, rope 64, batch 64, ragged contexts "
                        "U[1024,32768]+1 (seed 4), bf16 latent cache, f32 accumulate, one step = one layer's "
                        "decode attention over the batch",
            "batch": int(len(lens)), "heads": 128, "kv_lora_rank": 512, "rope_dim": 64,
            "tokens": main_res["tokens"], "cache_replicas": main_res["replicas"],
        },
        "step_ms": main_res["step_ms"],
        "hbm_gbs": main_res["hbm_gbs"],
        "hbm_frac": main_res["hbm_frac"],
        "roofline": {
            "bound": "hbm",
            "achieved": main_res["hbm_gbs"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": main_res["hbm_frac"],
            "traffic": measured_traffic(),
            "kernel": "decode step = k_decode_mfma + k_decode_merge_frag (one qmla_decode_absorbed call), "
                      "HIP events on the launch stream around the timed steps",
            "bytes_per_launch": main_res["bytes_per_step"],
        },
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
