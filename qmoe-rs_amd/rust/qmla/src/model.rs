//! Drop-ins for the MLA part of qmoe-rs src/model.rs (feature `candle`):
//! `KVCache` (:86-105) stores the latent cache on the device, and
//! `MlaAttention` (:107-307) keeps its constructor `new(vb, config)`, its
//! public fields and `forward_prefill` / `forward_with_cache` with their
//! signatures.  The decoder layer and model (:350-489) call them unchanged:
//! `DecoderLayer::new` builds the layer with `MlaAttention::new(vb.pp(..),
//! config)` (:357), `Vec<KVCache>` holds one cache per layer, one sequence
//! per cache.
//!
//! The one API change: the reference's `KVCache::new(k, v, k_rope)` and
//! `append(k, v, k_rope)` take decompressed per-head tensors, and a latent
//! cache cannot be built from those.  Here a cache comes from
//! `MlaAttention::forward_prefill` (as every engine call site gets it) or
//! from [`KVCache::empty`]; the decompressed `k`, `v`, `k_rope` are read
//! through [`KVCache::k`], [`KVCache::v`], [`KVCache::k_rope`].
use std::sync::Mutex;

use anyhow::{anyhow, bail, Result};
use candle_core::{Device, Tensor};
use candle_nn::VarBuilder;

use crate::{DType, DeviceBuffer, Stream};

fn gpu<T>(r: crate::Result<T>) -> Result<T> {
    r.map_err(|e| anyhow!("{e}"))
}

/// The fields of the engine's `ModelConfig` (src/model.rs:8-20) that
/// `MlaAttention::new` reads.  `impl_mla_config!(ModelConfig)` next to the
/// engine's struct implements it from those fields, so that
/// `MlaAttention::new(vb, config)` takes the engine's `&ModelConfig` as the
/// reference constructor does.
pub trait MlaConfig {
    fn hidden_size(&self) -> usize;
    fn num_attention_heads(&self) -> usize;
    fn num_key_value_heads(&self) -> usize;
    fn qk_nope_head_dim(&self) -> usize;
    fn qk_rope_head_dim(&self) -> usize;
    fn v_head_dim(&self) -> usize;
    fn kv_lora_rank(&self) -> usize;
}

/// Implements [`MlaConfig`] for a struct with the reference ModelConfig's
/// field names (src/model.rs:8-20).
#[macro_export]
macro_rules! impl_mla_config {
    ($t:ty) => {
        impl $crate::model::MlaConfig for $t {
            fn hidden_size(&self) -> usize { self.hidden_size }
            fn num_attention_heads(&self) -> usize { self.num_attention_heads }
            fn num_key_value_heads(&self) -> usize { self.num_key_value_heads }
            fn qk_nope_head_dim(&self) -> usize { self.qk_nope_head_dim }
            fn qk_rope_head_dim(&self) -> usize { self.qk_rope_head_dim }
            fn v_head_dim(&self) -> usize { self.v_head_dim }
            fn kv_lora_rank(&self) -> usize { self.kv_lora_rank }
        }
    };
}

/// `yarn_get_mscale`, src/model.rs:46-52.
fn yarn_get_mscale(scale: f64, mscale: f64) -> f64 {
    if scale <= 1.0 { 1.0 } else { 0.1 * mscale * scale.ln() + 1.0 }
}

/// The latent KV cache of one layer: one `[c_kv | k_pe]` row per token on
/// the device (bf16, or f32 for the 1e-4 parity mode), for `batch`
/// sequences.  The reference's public tensors `k`, `v`, `k_rope` are
/// available through [`KVCache::k`], [`KVCache::v`] and [`KVCache::k_rope`],
/// which decompress through the layer's kv_b_proj (the benches read them;
/// the decode path never does).  `Clone` deep-copies the rows, as the
/// reference's derived Clone (:87) gives a cache that later appends do not
/// share.
pub struct KVCache {
    pub inner: crate::KVCache,
    pub batch: usize,
}

impl Clone for KVCache {
    fn clone(&self) -> Self {
        KVCache { inner: self.inner.clone(), batch: self.batch }
    }
}

impl KVCache {
    /// An empty latent cache for `batch` sequences whose capacity grows on
    /// demand, as Tensor::cat does.  Replaces `KVCache::new(k, v, k_rope)`
    /// with empty tensors (benches/attention.rs:50-55).
    pub fn empty(batch: usize, kv_lora_rank: usize, rope_dim: usize, dtype: DType) -> Result<Self> {
        let caps = vec![256i32; batch];
        Ok(KVCache { inner: gpu(crate::KVCache::new(&caps, kv_lora_rank, rope_dim, dtype, true))?, batch })
    }

    /// Cached tokens per sequence (`cache.k.dim(2)`, src/model.rs:259; the
    /// batch is uniform when filled through MlaAttention).
    pub fn seq_len(&self) -> Result<usize> {
        Ok(gpu(self.inner.lengths())?[0] as usize)
    }

    fn materialise(&self, layer: &MlaAttention, which: usize) -> Result<Tensor> {
        let stream = Stream::default_stream();
        let (k, v, kr, t) = gpu(layer.device.materialise(&self.inner, 0, self.batch, &stream))?;
        let h = layer.num_heads;
        let (d, buf) = match which {
            0 => (layer.qk_nope_head_dim, k),
            1 => (layer.v_head_dim, v),
            _ => (layer.qk_rope_head_dim, kr),
        };
        let n = self.batch * h * t * d;
        Ok(Tensor::from_vec(gpu(buf.to_vec_f32(n, &stream))?, (self.batch, h, t, d), &Device::Cpu)?)
    }

    /// `KVCache.k` [b, H, T, dn] (src/model.rs:89).
    pub fn k(&self, layer: &MlaAttention) -> Result<Tensor> {
        self.materialise(layer, 0)
    }
    /// `KVCache.v` [b, H, T, dv] (src/model.rs:90).
    pub fn v(&self, layer: &MlaAttention) -> Result<Tensor> {
        self.materialise(layer, 1)
    }
    /// `KVCache.k_rope` [b, H, T, dr] (src/model.rs:91).
    pub fn k_rope(&self, layer: &MlaAttention) -> Result<Tensor> {
        self.materialise(layer, 2)
    }
}

/// Device buffers one layer reuses from call to call: the input rows, the
/// output rows and the workspace, each grown (never shrunk) when a call
/// needs more, so a decode step of an unchanged shape allocates nothing.
#[derive(Default)]
struct Scratch {
    x: Option<DeviceBuffer>,
    out: Option<DeviceBuffer>,
    ws: Option<DeviceBuffer>,
}

fn at_least(slot: &mut Option<DeviceBuffer>, bytes: usize) -> Result<&mut DeviceBuffer> {
    if slot.as_ref().map_or(true, |b| b.bytes() < bytes) {
        *slot = None; // free the smaller buffer first
        *slot = Some(gpu(DeviceBuffer::new(bytes))?);
    }
    Ok(slot.as_mut().expect("buffer"))
}

/// MlaAttention (src/model.rs:107-175) with its weights copied to HBM.  The
/// public fields are the reference's; the candle modules stay on the host
/// as loaded, and `device` holds the copy the GPU path runs on.
pub struct MlaAttention {
    pub q_proj: candle_nn::Linear,
    pub kv_a_proj_with_mqa: candle_nn::Linear,
    pub kv_a_layernorm: candle_nn::LayerNorm,
    pub kv_b_proj: candle_nn::Linear,
    pub o_proj: candle_nn::Linear,
    pub num_heads: usize,
    pub num_kv_heads: usize,
    pub qk_nope_head_dim: usize,
    pub qk_rope_head_dim: usize,
    pub v_head_dim: usize,
    pub kv_lora_rank: usize,
    pub rope_mscale: f64,
    pub softmax_scale: f64,
    /// Element type of the caches `forward_prefill` creates: bf16 (the
    /// default; within 2e-2 of the reference) or f32 (within 1e-4).
    pub cache_dtype: DType,
    pub device: crate::MlaAttention,
    hidden: usize,
    scratch: Mutex<Scratch>,
}

fn host(t: &Tensor) -> Result<Vec<f32>> {
    Ok(t.flatten_all()?.to_vec1::<f32>()?)
}

fn host_opt(t: Option<&Tensor>) -> Result<Option<Vec<f32>>> {
    t.map(host).transpose()
}

impl MlaAttention {
    /// MlaAttention::new, src/model.rs:125-175: the five modules from the
    /// reference's VarBuilder paths, the YaRN scales of :160-173.  The
    /// latent path shares one c_kv among all heads, which the reference's
    /// per-head products also require (num_key_value_heads ==
    /// num_attention_heads, else its matmuls fail on the head dimension).
    pub fn new<C: MlaConfig + ?Sized>(vb: VarBuilder, config: &C) -> Result<Self> {
        let (hid, h, hkv) = (config.hidden_size(), config.num_attention_heads(), config.num_key_value_heads());
        let (dn, dr, dv, r) =
            (config.qk_nope_head_dim(), config.qk_rope_head_dim(), config.v_head_dim(), config.kv_lora_rank());
        if hkv != h {
            bail!("num_key_value_heads ({hkv}) must equal num_attention_heads ({h})");
        }
        let q_proj = candle_nn::linear(hid, h * (dn + dr), vb.pp("q_proj"))?;
        let kv_a_proj_with_mqa = candle_nn::linear(hid, r + dr, vb.pp("kv_a_proj_with_mqa"))?;
        let kv_a_layernorm = candle_nn::layer_norm(r, 1e-6, vb.pp("kv_a_layernorm"))?;
        let kv_b_proj = candle_nn::linear(r, hkv * (dn + dv), vb.pp("kv_b_proj"))?;
        let o_proj = candle_nn::linear(h * dv, hid, vb.pp("o_proj"))?;
        Self::from_modules(q_proj, kv_a_proj_with_mqa, kv_a_layernorm, kv_b_proj, o_proj, h, dn, dr, dv, r)
    }

    /// The same from already built modules (hidden size from q_proj).
    #[allow(clippy::too_many_arguments)]
    pub fn from_modules(q_proj: candle_nn::Linear, kv_a_proj_with_mqa: candle_nn::Linear,
                        kv_a_layernorm: candle_nn::LayerNorm, kv_b_proj: candle_nn::Linear,
                        o_proj: candle_nn::Linear, heads: usize, qk_nope: usize, qk_rope: usize, v_dim: usize,
                        kv_lora_rank: usize) -> Result<Self> {
        let hidden = q_proj.weight().dim(1)?;
        // src/model.rs:160-173
        let rope_mscale = yarn_get_mscale(40.0, 1.0) / yarn_get_mscale(40.0, 0.707);
        let m = yarn_get_mscale(40.0, 0.707);
        let softmax_scale = ((qk_nope + qk_rope) as f64).powf(-0.5) * m * m;
        let cfg = crate::sys::qmla_layer_config {
            hidden: hidden as i32,
            heads: heads as i32,
            qk_nope: qk_nope as i32,
            qk_rope: qk_rope as i32,
            v_dim: v_dim as i32,
            kv_lora_rank: kv_lora_rank as i32,
            rope_mscale,
            softmax_scale,
            ln_eps: 1e-6,
        };
        let (wq, bq) = (host(q_proj.weight())?, host_opt(q_proj.bias())?);
        let (wkva, bkva) = (host(kv_a_proj_with_mqa.weight())?, host_opt(kv_a_proj_with_mqa.bias())?);
        let (ln_w, ln_b) = (host(kv_a_layernorm.weight())?, host_opt(kv_a_layernorm.bias())?);
        let (wkvb, bkvb) = (host(kv_b_proj.weight())?, host_opt(kv_b_proj.bias())?);
        let (wo, bo) = (host(o_proj.weight())?, host_opt(o_proj.bias())?);
        let w = crate::MlaWeights {
            wq: &wq,
            bq: bq.as_deref(),
            wkva: &wkva,
            bkva: bkva.as_deref(),
            ln_w: &ln_w,
            ln_b: ln_b.as_deref(),
            wkvb: &wkvb,
            bkvb: bkvb.as_deref(),
            wo: &wo,
            bo: bo.as_deref(),
        };
        let device = gpu(crate::MlaAttention::new(cfg, &w))?;
        Ok(MlaAttention {
            q_proj,
            kv_a_proj_with_mqa,
            kv_a_layernorm,
            kv_b_proj,
            o_proj,
            num_heads: heads,
            num_kv_heads: heads,
            qk_nope_head_dim: qk_nope,
            qk_rope_head_dim: qk_rope,
            v_head_dim: v_dim,
            kv_lora_rank,
            rope_mscale,
            softmax_scale,
            cache_dtype: DType::BF16,
            device,
            hidden,
            scratch: Mutex::new(Scratch::default()),
        })
    }

    /// The same layer making caches of `dtype` (DType::F32 for the 1e-4
    /// parity mode).
    pub fn with_cache_dtype(mut self, dtype: DType) -> Self {
        self.cache_dtype = dtype;
        self
    }

    /// The same layer with its projection kernels on bf16 operands and f32
    /// accumulation (DType::BF16: the bf16 tolerance, whatever the cache
    /// dtype) or f32-exact (DType::F32, the default).  No counterpart in the
    /// reference, whose Linear layers compute in the weights' dtype.
    pub fn with_projection_dtype(mut self, dtype: DType) -> Result<Self> {
        gpu(self.device.set_projection_dtype(dtype))?;
        Ok(self)
    }

    fn run(&self, xs: &Tensor, cache: &mut KVCache, prefill: bool) -> Result<Tensor> {
        let (b, s, hid) = xs.dims3()?;
        if hid != self.hidden {
            bail!("xs has hidden size {hid}, the layer {}", self.hidden);
        }
        if b > cache.batch {
            bail!("batch {b} exceeds the cache's {} sequences", cache.batch);
        }
        let stream = Stream::default_stream();
        let n = b * s * self.hidden;
        let ws_bytes = if prefill {
            gpu(self.device.prefill_workspace_bytes(&cache.inner, b, s))?
        } else {
            gpu(self.device.workspace_bytes(&cache.inner, b, s))?
        };
        let mut guard = self.scratch.lock().map_err(|_| anyhow!("layer scratch poisoned"))?;
        let sc = &mut *guard;
        gpu(at_least(&mut sc.x, 4 * n)?.copy_from_slice(&host(xs)?, &stream))?;
        at_least(&mut sc.out, 4 * n)?;
        at_least(&mut sc.ws, ws_bytes)?;
        let (x, out, ws) = (sc.x.as_ref().expect("x"), sc.out.as_mut().expect("out"), sc.ws.as_mut().expect("ws"));
        if prefill {
            gpu(self.device.forward_prefill(x, b, s, &mut cache.inner, out, ws, &stream))?;
        } else {
            gpu(self.device.forward_with_cache(x, b, s, &mut cache.inner, out, ws, &stream))?;
        }
        let v = gpu(out.to_vec_f32(n, &stream))?;
        Ok(Tensor::from_vec(v, (b, s, self.hidden), xs.device())?)
    }

    /// forward_prefill, src/model.rs:193-253: the output and a new cache of
    /// the layer's `cache_dtype` holding the prompt's latent rows.
    pub fn forward_prefill(&self, xs: &Tensor) -> Result<(Tensor, KVCache)> {
        let (b, _, _) = xs.dims3()?;
        let mut cache = KVCache::empty(b, self.kv_lora_rank, self.qk_rope_head_dim, self.cache_dtype)?;
        let out = self.run(xs, &mut cache, true)?;
        Ok((out, cache))
    }

    /// forward_with_cache, src/model.rs:256-307.
    pub fn forward_with_cache(&self, xs: &Tensor, cache: &mut KVCache) -> Result<Tensor> {
        self.run(xs, cache, false)
    }
}
