//! Drop-in for qmoe-rs src/attention_kernel.rs (feature `candle`): the same
//! three public functions with the same signatures, computed by libqmla on
//! the GPU.  Inputs are candle f32 tensors on the host; they are staged to
//! HBM, the kernel runs, and the result comes back as a new Tensor.
use candle_core::{Device, Result, Tensor};
use qmla_sys::qmla_prefill_dims;

use crate::{DType, DeviceBuffer, Stream};

fn to_device(t: &Tensor, stream: &Stream) -> Result<DeviceBuffer> {
    let host: Vec<f32> = t.flatten_all()?.to_vec1::<f32>()?;
    DeviceBuffer::from_slice(&host, stream).map_err(|e| candle_core::Error::Msg(e.to_string()))
}

fn from_device(b: &DeviceBuffer, shape: (usize, usize, usize, usize), stream: &Stream,
               device: &Device) -> Result<Tensor> {
    let n = shape.0 * shape.1 * shape.2 * shape.3;
    let v = b.to_vec_f32(n, stream).map_err(|e| candle_core::Error::Msg(e.to_string()))?;
    Tensor::from_vec(v, shape, device)
}

fn gpu<T>(r: crate::Result<T>) -> Result<T> {
    r.map_err(|e| candle_core::Error::Msg(e.to_string()))
}

/// fused_prefill_attn, src/attention_kernel.rs:64-107: causal (or full)
/// attention with scores `(q_nope k^T + q_rope k_rope^T) * scale`.  k_rope
/// may have one head (the latent layout) or as many as q (the reference's
/// broadcast).  f32 in, f32 out, f32 arithmetic on the device.
pub fn fused_prefill_attn(q_nope: &Tensor, q_rope: &Tensor, k: &Tensor, k_rope: &Tensor, v: &Tensor,
                          scale: f64, causal: bool) -> Result<Tensor> {
    let (b, h, s, dn) = q_nope.dims4()?;
    let (_, _, sk, _) = k.dims4()?;
    let dr = q_rope.dim(3)?;
    let dv = v.dim(3)?;
    let dims = qmla_prefill_dims {
        batch: b as i32,
        heads: h as i32,
        seq_q: s as i32,
        seq_k: sk as i32,
        qk_nope: dn as i32,
        qk_rope: dr as i32,
        v_dim: dv as i32,
        k_rope_heads: k_rope.dim(1)? as i32,
        q_offset: 0,
    };
    let stream = Stream::default_stream();
    let bufs = [q_nope, q_rope, k, k_rope, v].map(|t| to_device(t, &stream));
    let [qn, qr, kk, kr, vv] = bufs;
    let (qn, qr, kk, kr, vv) = (qn?, qr?, kk?, kr?, vv?);
    let mut out = gpu(DeviceBuffer::new(4 * b * h * s * dv))?;
    gpu(crate::fused_prefill_attn(&dims, DType::F32, &qn, &qr, &kk, &kr, &vv, scale, causal, &mut out,
                                  &stream))?;
    from_device(&out, (b, h, s, dv), &stream, q_nope.device())
}

fn single_part(q: &Tensor, k: &Tensor, v: &Tensor, scale: f64, causal: bool, eager: bool) -> Result<Tensor> {
    let (b, h, s, d) = q.dims4()?;
    let dv = v.dim(3)?;
    let stream = Stream::default_stream();
    let (qb, kb, vb) = (to_device(q, &stream)?, to_device(k, &stream)?, to_device(v, &stream)?);
    let mut out = gpu(DeviceBuffer::new(4 * b * h * s * dv))?;
    let (bi, hi, si, di, dvi) = (b as i32, h as i32, s as i32, d as i32, dv as i32);
    let o = out.ptr_mut();
    let st = unsafe {
        if eager {
            qmla_sys::qmla_eager_prefill_attn(bi, hi, si, di, dvi, qmla_sys::QMLA_F32, qb.ptr(), kb.ptr(),
                                              vb.ptr(), scale, causal as i32, o, stream.raw())
        } else {
            qmla_sys::qmla_reference_eager_attn(bi, hi, si, di, dvi, qmla_sys::QMLA_F32, qb.ptr(), kb.ptr(),
                                                vb.ptr(), scale, causal as i32, o, stream.raw())
        }
    };
    qmla_sys::check(st).map_err(candle_core::Error::Msg)?;
    from_device(&out, (b, h, s, dv), &stream, q.device())
}

/// eager_prefill_attn, src/attention_kernel.rs:34-57 (its intended math:
/// the causal mask broadcast over batch and heads).
pub fn eager_prefill_attn(q: &Tensor, k: &Tensor, v: &Tensor, scale: f64, causal: bool) -> Result<Tensor> {
    single_part(q, k, v, scale, causal, true)
}

/// reference_eager_attn, src/attention_kernel.rs:110-134.
pub fn reference_eager_attn(q: &Tensor, k: &Tensor, v: &Tensor, scale: f64, causal: bool) -> Result<Tensor> {
    single_part(q, k, v, scale, causal, false)
}
