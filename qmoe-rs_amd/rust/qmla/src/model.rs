//! Drop-ins for the MLA part of qmoe-rs src/model.rs (feature `candle`):
//! `KVCache` (:86-105) stores the latent cache on the device, and
//! `MlaAttention` (:107-307) keeps `forward_prefill` / `forward_with_cache`
//! with their signatures.  The decoder layer and model (:372-489) call them
//! unchanged: `Vec<KVCache>` one per layer, one sequence per cache.
use anyhow::{anyhow, Result};
use candle_core::{Device, Tensor};

use crate::{DType, DeviceBuffer, Stream};

fn gpu<T>(r: crate::Result<T>) -> Result<T> {
    r.map_err(|e| anyhow!("{e}"))
}

/// The latent KV cache of one layer: one `[c_kv | k_pe]` bf16 row per
/// token on the device, for `batch` sequences.  The reference's public
/// tensors `k`, `v`, `k_rope` are available through [`KVCache::k`],
/// [`KVCache::v`] and [`KVCache::k_rope`], which decompress through the
/// layer's kv_b_proj (the benches read them; the decode path never does).
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
    /// An empty cache for `batch` sequences (capacity grows on demand, as
    /// Tensor::cat does).
    pub fn new(batch: usize, kv_lora_rank: usize, rope_dim: usize) -> Result<Self> {
        let caps = vec![256i32; batch];
        Ok(KVCache { inner: gpu(crate::KVCache::new(&caps, kv_lora_rank, rope_dim, DType::BF16, true))?, batch })
    }

    /// Cached tokens per sequence (`cache.k.dim(2)`, src/model.rs:259; the
    /// batch is uniform when filled through MlaAttention).
    pub fn seq_len(&self) -> Result<usize> {
        Ok(gpu(self.inner.lengths())?[0] as usize)
    }

    fn materialise(&self, layer: &MlaAttention, which: usize) -> Result<Tensor> {
        let stream = Stream::default_stream();
        let (k, v, kr, t) = gpu(layer.inner.materialise(&self.inner, 0, self.batch, &stream))?;
        let c = &layer.inner.config;
        let (h, d, buf) = match which {
            0 => (c.heads as usize, c.qk_nope as usize, k),
            1 => (c.heads as usize, c.v_dim as usize, v),
            _ => (c.heads as usize, c.qk_rope as usize, kr),
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

/// MlaAttention with its weights in HBM, built from the candle layer's
/// Linear / LayerNorm weights.
pub struct MlaAttention {
    pub inner: crate::MlaAttention,
    pub hidden: usize,
}

fn host(t: &Tensor) -> Result<Vec<f32>> {
    Ok(t.flatten_all()?.to_vec1::<f32>()?)
}

fn host_opt(t: Option<&Tensor>) -> Result<Option<Vec<f32>>> {
    t.map(host).transpose()
}

impl MlaAttention {
    /// From the reference layer's modules (src/model.rs:126-146); the scales
    /// are the reference constructor's (:160-173).
    pub fn from_linear(q_proj: &candle_nn::Linear, kv_a_proj_with_mqa: &candle_nn::Linear,
                       kv_a_layernorm: &candle_nn::LayerNorm, kv_b_proj: &candle_nn::Linear,
                       o_proj: &candle_nn::Linear, heads: usize, qk_nope: usize, qk_rope: usize, v_dim: usize,
                       kv_lora_rank: usize) -> Result<Self> {
        let hidden = q_proj.weight().dim(1)?;
        let cfg = gpu(crate::MlaAttention::default_config(hidden, heads, qk_nope, qk_rope, v_dim, kv_lora_rank))?;
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
        Ok(MlaAttention { inner: gpu(crate::MlaAttention::new(cfg, &w))?, hidden })
    }

    fn run(&self, xs: &Tensor, cache: &mut KVCache, prefill: bool) -> Result<Tensor> {
        let (b, s, _) = xs.dims3()?;
        let stream = Stream::default_stream();
        let x = gpu(DeviceBuffer::from_slice(&host(xs)?, &stream))?;
        let mut out = gpu(DeviceBuffer::new(4 * b * s * self.hidden))?;
        let mut ws = gpu(DeviceBuffer::new(gpu(self.inner.workspace_bytes(&cache.inner, b, s))?))?;
        if prefill {
            gpu(self.inner.forward_prefill(&x, b, s, &mut cache.inner, &mut out, &mut ws, &stream))?;
        } else {
            gpu(self.inner.forward_with_cache(&x, b, s, &mut cache.inner, &mut out, &mut ws, &stream))?;
        }
        let v = gpu(out.to_vec_f32(b * s * self.hidden, &stream))?;
        Ok(Tensor::from_vec(v, (b, s, self.hidden), xs.device())?)
    }

    /// forward_prefill, src/model.rs:193-253.
    pub fn forward_prefill(&self, xs: &Tensor) -> Result<(Tensor, KVCache)> {
        let (b, _, _) = xs.dims3()?;
        let c = &self.inner.config;
        let mut cache = KVCache::new(b, c.kv_lora_rank as usize, c.qk_rope as usize)?;
        let out = self.run(xs, &mut cache, true)?;
        Ok((out, cache))
    }

    /// forward_with_cache, src/model.rs:256-307.
    pub fn forward_with_cache(&self, xs: &Tensor, cache: &mut KVCache) -> Result<Tensor> {
        self.run(xs, cache, false)
    }
}
