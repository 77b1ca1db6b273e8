//! Safe wrappers of libqmla (raw bindings in `qmla-sys`).
//!
//! * [`DeviceBuffer`]: the HBM-resident buffers src/tensor.rs gains.
//! * [`KVCache`]: the device latent cache that replaces KVCache
//!   (src/model.rs:86-105), one `[c_kv | k_pe]` row per token with a ragged
//!   length table.
//! * [`MlaAttention`]: MlaAttention (src/model.rs:107-307) with device
//!   weights; `forward_with_cache` / `forward_prefill` on device buffers.
//! * [`fused_prefill_attn`], [`decode_absorbed`]: the attention cores.
//! * [`PackedQMoETensor`], [`QMoELayer`]: src/tensor.rs:64-95 and
//!   src/moe.rs:40-130 on the device.
//!
//! With the `candle` feature, [`attention_kernel`] and [`model`] keep the
//! reference's candle signatures on top of these.
use std::os::raw::c_void;
use std::ptr;

pub use qmla_sys as sys;
use qmla_sys::*;

#[cfg(feature = "candle")]
pub mod attention_kernel;
#[cfg(feature = "candle")]
pub mod model;

/// A failed library call: its status and message.
#[derive(Debug, Clone)]
pub struct Error {
    pub status: qmla_status,
    pub message: String,
}

impl std::fmt::Display for Error {
    fn fmt(&self, f: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        write!(f, "qmla status {}: {}", self.status, self.message)
    }
}

impl std::error::Error for Error {}

pub type Result<T> = std::result::Result<T, Error>;

fn ok(st: qmla_status) -> Result<()> {
    if st == QMLA_OK {
        Ok(())
    } else {
        Err(Error { status: st, message: last_error() })
    }
}

/// A size the caller got wrong, caught before the call reaches C (which
/// would read or write past the end of the slice or buffer).
fn shape_err(message: String) -> Error {
    Error { status: QMLA_ERR_SHAPE, message }
}

/// Host slice `what` must hold exactly `want` elements.
fn check_len(what: &str, got: usize, want: usize) -> Result<()> {
    if got == want { Ok(()) } else { Err(shape_err(format!("{what}: {got} elements, expected {want}"))) }
}

/// Optional host slice: absent, or exactly `want` elements.
fn check_opt_len(what: &str, got: Option<&[f32]>, want: usize) -> Result<()> {
    got.map_or(Ok(()), |s| check_len(what, s.len(), want))
}

/// Device buffer `what` must hold at least `want` bytes.
fn check_bytes(what: &str, b: &DeviceBuffer, want: usize) -> Result<()> {
    if b.bytes() >= want {
        Ok(())
    } else {
        Err(shape_err(format!("{what}: {}-byte buffer, need {want} bytes", b.bytes())))
    }
}

/// A dimension as usize: negative values are a shape error.
fn dim(what: &str, v: i32) -> Result<usize> {
    usize::try_from(v).map_err(|_| shape_err(format!("{what} = {v} is negative")))
}

/// Element types of device tensors (bf16 as u16 bit patterns).
#[derive(Clone, Copy, Debug, PartialEq, Eq)]
pub enum DType {
    F32,
    BF16,
}

impl DType {
    pub fn raw(self) -> qmla_dtype {
        match self {
            DType::F32 => QMLA_F32,
            DType::BF16 => QMLA_BF16,
        }
    }
    pub fn size(self) -> usize {
        match self {
            DType::F32 => 4,
            DType::BF16 => 2,
        }
    }
}

/// A HIP stream (null = the default stream).
pub struct Stream {
    raw: qmla_stream,
    owned: bool,
}

impl Stream {
    pub fn new() -> Result<Self> {
        let mut raw: qmla_stream = ptr::null_mut();
        ok(unsafe { qmla_stream_create(&mut raw) })?;
        Ok(Stream { raw, owned: true })
    }
    pub fn default_stream() -> Self {
        Stream { raw: ptr::null_mut(), owned: false }
    }
    pub fn raw(&self) -> qmla_stream {
        self.raw
    }
    pub fn synchronize(&self) -> Result<()> {
        ok(unsafe { qmla_stream_synchronize(self.raw) })
    }
}

impl Drop for Stream {
    fn drop(&mut self) {
        if self.owned && !self.raw.is_null() {
            unsafe {
                qmla_stream_destroy(self.raw);
            }
        }
    }
}

/// An HBM allocation (qmla_buffer_alloc / qmla_buffer_free).
pub struct DeviceBuffer {
    ptr: *mut c_void,
    bytes: usize,
}

impl DeviceBuffer {
    pub fn new(bytes: usize) -> Result<Self> {
        let mut ptr: *mut c_void = ptr::null_mut();
        ok(unsafe { qmla_buffer_alloc(bytes.max(1), &mut ptr) })?;
        Ok(DeviceBuffer { ptr, bytes })
    }
    /// Zero-filled buffer.
    pub fn zeros(bytes: usize, stream: &Stream) -> Result<Self> {
        let b = DeviceBuffer::new(bytes)?;
        ok(unsafe { qmla_memset_zero(b.ptr, b.bytes.max(1), stream.raw()) })?;
        Ok(b)
    }
    /// Copy of a host slice (synchronous).
    pub fn from_slice<T: Copy>(data: &[T], stream: &Stream) -> Result<Self> {
        let bytes = std::mem::size_of_val(data);
        let b = DeviceBuffer::new(bytes)?;
        if bytes > 0 {
            ok(unsafe { qmla_memcpy_h2d(b.ptr, data.as_ptr() as *const c_void, bytes, stream.raw()) })?;
            stream.synchronize()?;
        }
        Ok(b)
    }
    /// Overwrites the start of the buffer with a host slice (synchronous);
    /// allocates nothing.
    pub fn copy_from_slice<T: Copy>(&mut self, data: &[T], stream: &Stream) -> Result<()> {
        let bytes = std::mem::size_of_val(data);
        check_bytes("copy destination", self, bytes)?;
        if bytes > 0 {
            ok(unsafe { qmla_memcpy_h2d(self.ptr, data.as_ptr() as *const c_void, bytes, stream.raw()) })?;
            stream.synchronize()?;
        }
        Ok(())
    }
    /// Copies the first `out.len()` elements back to the host (synchronous).
    pub fn copy_to<T: Copy>(&self, out: &mut [T], stream: &Stream) -> Result<()> {
        let bytes = std::mem::size_of_val(out);
        check_bytes("copy source", self, bytes)?;
        if bytes > 0 {
            ok(unsafe { qmla_memcpy_d2h(out.as_mut_ptr() as *mut c_void, self.ptr, bytes, stream.raw()) })?;
            stream.synchronize()?;
        }
        Ok(())
    }
    pub fn to_vec_f32(&self, n: usize, stream: &Stream) -> Result<Vec<f32>> {
        let mut v = vec![0f32; n];
        self.copy_to(&mut v, stream)?;
        Ok(v)
    }
    pub fn ptr(&self) -> *const c_void {
        self.ptr
    }
    pub fn ptr_mut(&mut self) -> *mut c_void {
        self.ptr
    }
    pub fn bytes(&self) -> usize {
        self.bytes
    }
}

impl Drop for DeviceBuffer {
    fn drop(&mut self) {
        if !self.ptr.is_null() {
            unsafe {
                qmla_buffer_free(self.ptr);
            }
        }
    }
}

/// The latent KV cache: one `[c_kv | k_pe]` row per token, held in HBM
/// pages that a device block table lists per sequence (token t of sequence
/// i is row t % page_rows of its page t / page_rows), with a device length
/// table.  Growth adds pages and never moves a row.
pub struct KVCache {
    raw: *mut qmla_kv_cache,
    num_seqs: usize,
    kv_lora_rank: usize,
    rope_dim: usize,
    dtype: DType,
}

impl KVCache {
    /// KVCache::new (src/model.rs:95-97): empty sequences with the given
    /// capacities.  `grow` lets appends past a capacity grow it, as
    /// Tensor::cat never runs out of room.
    pub fn new(capacity: &[i32], kv_lora_rank: usize, rope_dim: usize, dtype: DType, grow: bool) -> Result<Self> {
        let mut raw: *mut qmla_kv_cache = ptr::null_mut();
        ok(unsafe {
            qmla_cache_create(capacity.len() as i32, capacity.as_ptr(), kv_lora_rank as i32, rope_dim as i32,
                              dtype.raw(), &mut raw)
        })?;
        let c = KVCache { raw, num_seqs: capacity.len(), kv_lora_rank, rope_dim, dtype };
        if grow {
            ok(unsafe { qmla_cache_set_growth(c.raw, 1) })?;
        }
        Ok(c)
    }
    /// KVCache::new with the page pool laid out by the caller: `pool_rows`
    /// rows of HBM now (growth draws on the spare ones without allocating),
    /// `max_len` the longest a sequence may grow (0: default), `page_rows`
    /// a power of two >= 32 (0: 256).
    pub fn paged(capacity: &[i32], kv_lora_rank: usize, rope_dim: usize, dtype: DType, max_len: i64,
                 pool_rows: i64, page_rows: i32, grow: bool) -> Result<Self> {
        let mut raw: *mut qmla_kv_cache = ptr::null_mut();
        ok(unsafe {
            qmla_cache_create_paged(capacity.len() as i32, capacity.as_ptr(), max_len, pool_rows, page_rows,
                                    kv_lora_rank as i32, rope_dim as i32, dtype.raw(), &mut raw)
        })?;
        let c = KVCache { raw, num_seqs: capacity.len(), kv_lora_rank, rope_dim, dtype };
        if grow {
            ok(unsafe { qmla_cache_set_growth(c.raw, 1) })?;
        }
        Ok(c)
    }
    /// Rows [t0, t0 + n) of sequence `seq` into `out` ([n, r + dr] in the
    /// cache dtype), wherever its pages are.
    pub fn gather(&self, seq: usize, t0: usize, n: usize, out: &mut DeviceBuffer, stream: &Stream) -> Result<()> {
        check_bytes("gather out", out, n * (self.kv_lora_rank + self.rope_dim) * self.dtype.size())?;
        ok(unsafe { qmla_cache_gather(self.raw, seq as i32, t0 as i32, n as i32, out.ptr_mut(), stream.raw()) })
    }
    /// Returns the pages of sequences seq0..seq0 + n beyond their lengths to
    /// the free list.
    pub fn trim(&mut self, seq0: usize, n: usize, stream: &Stream) -> Result<()> {
        ok(unsafe { qmla_cache_trim(self.raw, seq0 as i32, n as i32, stream.raw()) })
    }
    /// Tops the free list up to at least `free_rows` rows (allocates now).
    pub fn reserve_pool(&mut self, free_rows: i64) -> Result<()> {
        ok(unsafe { qmla_cache_reserve_pool(self.raw, free_rows) })
    }
    /// (pool rows, free rows).
    pub fn pool_info(&self) -> Result<(i64, i64)> {
        let (mut a, mut b) = (0i64, 0i64);
        ok(unsafe { qmla_cache_pool_info(self.raw, &mut a, &mut b) })?;
        Ok((a, b))
    }
    pub fn raw(&self) -> *mut qmla_kv_cache {
        self.raw
    }
    pub fn num_seqs(&self) -> usize {
        self.num_seqs
    }
    pub fn dtype(&self) -> DType {
        self.dtype
    }
    /// KVCache::append (src/model.rs:99-104): `n_new` rows for each of
    /// sequences 0..n_seqs, `rows` [n_seqs, n_new, r + dr] on the device.
    pub fn append(&mut self, rows: &DeviceBuffer, rows_dtype: DType, n_seqs: usize, n_new: usize,
                  stream: &Stream) -> Result<()> {
        let need = n_seqs * n_new * (self.kv_lora_rank + self.rope_dim) * rows_dtype.size();
        check_bytes("rows", rows, need)?;
        ok(unsafe {
            qmla_cache_append(self.raw, rows.ptr(), rows_dtype.raw(), n_seqs as i32, n_new as i32, stream.raw())
        })
    }
    /// Current lengths (`cache.k.dim(2)` per sequence, src/model.rs:259).
    pub fn lengths(&self) -> Result<Vec<i32>> {
        let mut v = vec![0i32; self.num_seqs];
        ok(unsafe { qmla_cache_lengths(self.raw, v.as_mut_ptr()) })?;
        Ok(v)
    }
    pub fn set_lengths(&mut self, lengths: &[i32], stream: &Stream) -> Result<()> {
        check_len("lengths", lengths.len(), self.num_seqs)?;
        ok(unsafe { qmla_cache_set_lengths(self.raw, lengths.as_ptr(), stream.raw()) })
    }
    pub fn reserve(&mut self, min_capacity: &[i32], stream: &Stream) -> Result<()> {
        check_len("min_capacity", min_capacity.len(), self.num_seqs)?;
        ok(unsafe { qmla_cache_reserve(self.raw, min_capacity.as_ptr(), stream.raw()) })
    }
    /// `#[derive(Clone)]` (src/model.rs:87) on a stream.
    pub fn try_clone(&self, stream: &Stream) -> Result<Self> {
        let mut raw: *mut qmla_kv_cache = ptr::null_mut();
        ok(unsafe { qmla_cache_clone(self.raw, &mut raw, stream.raw()) })?;
        Ok(KVCache {
            raw,
            num_seqs: self.num_seqs,
            kv_lora_rank: self.kv_lora_rank,
            rope_dim: self.rope_dim,
            dtype: self.dtype,
        })
    }
}

impl Clone for KVCache {
    fn clone(&self) -> Self {
        self.try_clone(&Stream::default_stream()).expect("qmla_cache_clone")
    }
}

impl Drop for KVCache {
    fn drop(&mut self) {
        if !self.raw.is_null() {
            unsafe {
                qmla_cache_destroy(self.raw);
            }
        }
    }
}

/// Host f32 weights of one MlaAttention in the Linear layout ([out, in]
/// weight, [out] bias): q_proj, kv_a_proj_with_mqa, kv_a_layernorm,
/// kv_b_proj, o_proj (src/model.rs:107-146).
pub struct MlaWeights<'a> {
    pub wq: &'a [f32],
    pub bq: Option<&'a [f32]>,
    pub wkva: &'a [f32],
    pub bkva: Option<&'a [f32]>,
    pub ln_w: &'a [f32],
    pub ln_b: Option<&'a [f32]>,
    pub wkvb: &'a [f32],
    pub bkvb: Option<&'a [f32]>,
    pub wo: &'a [f32],
    pub bo: Option<&'a [f32]>,
}

fn opt_ptr(b: Option<&[f32]>) -> *const f32 {
    b.map_or(ptr::null(), |s| s.as_ptr())
}

/// MlaAttention with device-resident weights.
pub struct MlaAttention {
    raw: *mut qmla_layer,
    pub config: qmla_layer_config,
}

impl MlaAttention {
    /// The reference constructor's scales (src/model.rs:160-173) for these
    /// dimensions.
    pub fn default_config(hidden: usize, heads: usize, qk_nope: usize, qk_rope: usize, v_dim: usize,
                          kv_lora_rank: usize) -> Result<qmla_layer_config> {
        let mut cfg = qmla_layer_config {
            hidden: hidden as i32,
            heads: heads as i32,
            qk_nope: qk_nope as i32,
            qk_rope: qk_rope as i32,
            v_dim: v_dim as i32,
            kv_lora_rank: kv_lora_rank as i32,
            ..Default::default()
        };
        ok(unsafe { qmla_layer_default_scales(&mut cfg) })?;
        Ok(cfg)
    }

    pub fn new(config: qmla_layer_config, w: &MlaWeights) -> Result<Self> {
        let c = &config;
        let hid = dim("hidden", c.hidden)?;
        let h = dim("heads", c.heads)?;
        let (dn, dr, dv) = (dim("qk_nope", c.qk_nope)?, dim("qk_rope", c.qk_rope)?, dim("v_dim", c.v_dim)?);
        let r = dim("kv_lora_rank", c.kv_lora_rank)?;
        check_len("q_proj weight", w.wq.len(), h * (dn + dr) * hid)?;
        check_opt_len("q_proj bias", w.bq, h * (dn + dr))?;
        check_len("kv_a_proj_with_mqa weight", w.wkva.len(), (r + dr) * hid)?;
        check_opt_len("kv_a_proj_with_mqa bias", w.bkva, r + dr)?;
        check_len("kv_a_layernorm weight", w.ln_w.len(), r)?;
        check_opt_len("kv_a_layernorm bias", w.ln_b, r)?;
        check_len("kv_b_proj weight", w.wkvb.len(), h * (dn + dv) * r)?;
        check_opt_len("kv_b_proj bias", w.bkvb, h * (dn + dv))?;
        check_len("o_proj weight", w.wo.len(), hid * h * dv)?;
        check_opt_len("o_proj bias", w.bo, hid)?;
        let mut raw: *mut qmla_layer = ptr::null_mut();
        ok(unsafe {
            qmla_layer_create(&config, w.wq.as_ptr(), opt_ptr(w.bq), w.wkva.as_ptr(), opt_ptr(w.bkva),
                              w.ln_w.as_ptr(), opt_ptr(w.ln_b), w.wkvb.as_ptr(), opt_ptr(w.bkvb),
                              w.wo.as_ptr(), opt_ptr(w.bo), &mut raw)
        })?;
        Ok(MlaAttention { raw, config })
    }

    /// Operand precision of the projection kernels: DType::F32 (default,
    /// f32-exact) or DType::BF16 (bf16 operands, f32 accumulation).
    pub fn set_projection_dtype(&mut self, dtype: DType) -> Result<()> {
        ok(unsafe { qmla_layer_set_projection_dtype(self.raw, dtype.raw()) })
    }

    /// Scratch that serves either forward call for (batch, seq) tokens.
    pub fn workspace_bytes(&self, cache: &KVCache, batch: usize, seq: usize) -> Result<usize> {
        let mut n = 0usize;
        ok(unsafe { qmla_layer_workspace_bytes(self.raw, cache.raw, batch as i32, seq as i32, &mut n) })?;
        Ok(n)
    }

    /// Scratch that forward_prefill alone needs for (batch, seq) tokens.
    pub fn prefill_workspace_bytes(&self, cache: &KVCache, batch: usize, seq: usize) -> Result<usize> {
        let mut n = 0usize;
        ok(unsafe {
            qmla_layer_prefill_workspace_bytes(self.raw, cache.raw, batch as i32, seq as i32, &mut n)
        })?;
        Ok(n)
    }

    /// xs and out hold [batch, seq, hidden] f32 each.
    fn check_io(&self, xs: &DeviceBuffer, out: &DeviceBuffer, batch: usize, seq: usize) -> Result<()> {
        let n = 4 * batch * seq * self.config.hidden.max(0) as usize;
        check_bytes("xs", xs, n)?;
        check_bytes("out", out, n)
    }

    /// forward_with_cache (src/model.rs:256-307): xs [batch, seq, hidden]
    /// -> out, appending the new tokens to sequences 0..batch of `cache`.
    pub fn forward_with_cache(&self, xs: &DeviceBuffer, batch: usize, seq: usize, cache: &mut KVCache,
                              out: &mut DeviceBuffer, workspace: &mut DeviceBuffer, stream: &Stream) -> Result<()> {
        self.check_io(xs, out, batch, seq)?;
        ok(unsafe {
            qmla_layer_forward_with_cache(self.raw, xs.ptr() as *const f32, batch as i32, seq as i32, cache.raw,
                                          out.ptr_mut() as *mut f32, workspace.ptr_mut(), workspace.bytes(),
                                          stream.raw())
        })
    }

    /// forward_prefill (src/model.rs:193-253) into empty sequences.
    pub fn forward_prefill(&self, xs: &DeviceBuffer, batch: usize, seq: usize, cache: &mut KVCache,
                           out: &mut DeviceBuffer, workspace: &mut DeviceBuffer, stream: &Stream) -> Result<()> {
        self.check_io(xs, out, batch, seq)?;
        ok(unsafe {
            qmla_layer_forward_prefill(self.raw, xs.ptr() as *const f32, batch as i32, seq as i32, cache.raw,
                                       out.ptr_mut() as *mut f32, workspace.ptr_mut(), workspace.bytes(),
                                       stream.raw())
        })
    }

    /// The public tensors of the reference KVCache (src/model.rs:88-92),
    /// rebuilt through kv_b_proj for sequences seq0..seq0 + n of one length
    /// T: (k [n, H, T, dn], v [n, H, T, dv], k_rope [n, H, T, dr]) in f32.
    pub fn materialise(&self, cache: &KVCache, seq0: usize, n: usize, stream: &Stream)
                       -> Result<(DeviceBuffer, DeviceBuffer, DeviceBuffer, usize)> {
        let lens = cache.lengths()?;
        if seq0 + n > lens.len() || n == 0 {
            return Err(shape_err(format!("sequences {seq0}..{} of a {}-sequence cache", seq0 + n, lens.len())));
        }
        let t = lens[seq0] as usize;
        let mut ws_bytes = 0usize;
        ok(unsafe {
            qmla_cache_materialise_workspace_bytes(self.raw, cache.raw, seq0 as i32, n as i32, &mut ws_bytes)
        })?;
        let c = &self.config;
        let (h, dn, dv, dr) = (c.heads as usize, c.qk_nope as usize, c.v_dim as usize, c.qk_rope as usize);
        let mut k = DeviceBuffer::new(4 * n * h * t * dn)?;
        let mut v = DeviceBuffer::new(4 * n * h * t * dv)?;
        let mut kr = DeviceBuffer::new(4 * n * h * t * dr)?;
        let mut ws = DeviceBuffer::new(ws_bytes)?;
        ok(unsafe {
            qmla_cache_materialise(self.raw, cache.raw, seq0 as i32, n as i32, k.ptr_mut() as *mut f32,
                                   v.ptr_mut() as *mut f32, kr.ptr_mut() as *mut f32, ws.ptr_mut(), ws_bytes,
                                   stream.raw())
        })?;
        stream.synchronize()?;
        Ok((k, v, kr, t))
    }
}

impl Drop for MlaAttention {
    fn drop(&mut self) {
        if !self.raw.is_null() {
            unsafe {
                qmla_layer_destroy(self.raw);
            }
        }
    }
}

/// fused_prefill_attn (src/attention_kernel.rs:64-107) on device tensors
/// q_nope [b,h,sq,dn], q_rope [b,h,sq,dr], k [b,h,sk,dn],
/// k_rope [b,krh,sk,dr], v [b,h,sk,dv] -> out [b,h,sq,dv].
pub fn fused_prefill_attn(dims: &qmla_prefill_dims, dtype: DType, q_nope: &DeviceBuffer, q_rope: &DeviceBuffer,
                          k: &DeviceBuffer, k_rope: &DeviceBuffer, v: &DeviceBuffer, scale: f64, causal: bool,
                          out: &mut DeviceBuffer, stream: &Stream) -> Result<()> {
    let (b, h, sq, sk) = (dim("batch", dims.batch)?, dim("heads", dims.heads)?, dim("seq_q", dims.seq_q)?,
                          dim("seq_k", dims.seq_k)?);
    let (dn, dr, dv) = (dim("qk_nope", dims.qk_nope)?, dim("qk_rope", dims.qk_rope)?, dim("v_dim", dims.v_dim)?);
    let krh = dim("k_rope_heads", dims.k_rope_heads)?;
    let es = dtype.size();
    check_bytes("q_nope", q_nope, b * h * sq * dn * es)?;
    check_bytes("q_rope", q_rope, b * h * sq * dr * es)?;
    check_bytes("k", k, b * h * sk * dn * es)?;
    check_bytes("k_rope", k_rope, b * krh * sk * dr * es)?;
    check_bytes("v", v, b * h * sk * dv * es)?;
    check_bytes("out", out, b * h * sq * dv * es)?;
    ok(unsafe {
        qmla_fused_prefill_attn(dims, dtype.raw(), q_nope.ptr(), q_rope.ptr(), k.ptr(), k_rope.ptr(), v.ptr(),
                                scale, causal as i32, out.ptr_mut(), stream.raw())
    })
}

/// Absorbed-latent decode over sequences 0..dims.batch of `cache`
/// (attention core of forward_with_cache, src/model.rs:294-303).
pub fn decode_absorbed(dims: &qmla_decode_dims, cache: &KVCache, q_dtype: DType, q_latent: &DeviceBuffer,
                       q_rope: &DeviceBuffer, scale: f64, out_latent: &mut DeviceBuffer,
                       out_lse: Option<&mut DeviceBuffer>, workspace: &mut DeviceBuffer,
                       stream: &Stream) -> Result<()> {
    let (b, rows) = (dim("batch", dims.batch)?, dim("rows", dims.rows)?);
    let (r, dr) = (dim("kv_lora_rank", dims.kv_lora_rank)?, dim("rope_dim", dims.rope_dim)?);
    check_bytes("q_latent", q_latent, b * rows * r * q_dtype.size())?;
    check_bytes("q_rope", q_rope, b * rows * dr * q_dtype.size())?;
    check_bytes("out_latent", out_latent, b * rows * r * 4)?;
    if let Some(l) = out_lse.as_deref() {
        check_bytes("out_lse", l, b * rows * 4)?;
    }
    let lse = out_lse.map_or(ptr::null_mut(), |b| b.ptr_mut() as *mut f32);
    ok(unsafe {
        qmla_decode_absorbed(dims, cache.raw, q_dtype.raw(), q_latent.ptr(), q_rope.ptr(), scale,
                             out_latent.ptr_mut() as *mut f32, lse, workspace.ptr_mut(), workspace.bytes(),
                             stream.raw())
    })
}

pub fn decode_workspace_bytes(dims: &qmla_decode_dims, cache: &KVCache) -> Result<usize> {
    let mut n = 0usize;
    ok(unsafe { qmla_decode_workspace_bytes(dims, cache.raw, &mut n) })?;
    Ok(n)
}

/// PackedQMoETensor (src/tensor.rs:16-122) with its bytes and scales in HBM.
pub struct PackedQMoETensor {
    data: DeviceBuffer,
    scales: DeviceBuffer,
    pub out_features: usize,
    pub in_features: usize,
}

impl PackedQMoETensor {
    pub fn from_bytes(packed: &[u8], out_features: usize, in_features: usize, scales: &[f32],
                      stream: &Stream) -> Result<Self> {
        check_len("packed bytes", packed.len(), out_features * (in_features / 4))?;
        check_len("scales", scales.len(), out_features)?;
        Ok(PackedQMoETensor {
            data: DeviceBuffer::from_slice(packed, stream)?,
            scales: DeviceBuffer::from_slice(scales, stream)?,
            out_features,
            in_features,
        })
    }
    /// forward_simd (src/tensor.rs:64-95): x [batch, in] -> out [batch, out].
    pub fn forward(&self, x: &DeviceBuffer, batch: usize, out: &mut DeviceBuffer, stream: &Stream) -> Result<()> {
        check_bytes("x", x, 4 * batch * self.in_features)?;
        check_bytes("out", out, 4 * batch * self.out_features)?;
        let mut n = 0usize;
        ok(unsafe {
            qmla_packed_forward_workspace_bytes(self.out_features as i32, self.in_features as i32, batch as i32,
                                                &mut n)
        })?;
        let mut ws = DeviceBuffer::new(n)?;
        ok(unsafe {
            qmla_packed_forward(self.data.ptr() as *const u8, self.scales.ptr() as *const f32,
                                self.out_features as i32, self.in_features as i32, x.ptr() as *const f32,
                                batch as i32, out.ptr_mut() as *mut f32, ws.ptr_mut(), n, stream.raw())
        })
    }
}

/// QMoELayer (src/moe.rs:23-131): gate weight and every expert's packed
/// gate/up/down stacked per kind in HBM.
pub struct QMoELayer {
    pub config: qmla_moe_config,
    gate_weight: DeviceBuffer,
    packed: [DeviceBuffer; 3],
    scales: [DeviceBuffer; 3],
}

impl QMoELayer {
    /// `packed[k]` / `scales[k]` for k = gate, up, down: [E, I, H/4] /
    /// [E, I], [E, I, H/4] / [E, I], [E, H, I/4] / [E, H].
    pub fn new(config: qmla_moe_config, gate_weight: &[f32], packed: [&[u8]; 3], scales: [&[f32]; 3],
               stream: &Stream) -> Result<Self> {
        let e = dim("num_experts", config.num_experts)?;
        let (hd, id) = (dim("hidden_dim", config.hidden_dim)?, dim("intermediate_dim", config.intermediate_dim)?);
        check_len("gate weight", gate_weight.len(), e * hd)?;
        check_len("gate packed", packed[0].len(), e * id * (hd / 4))?;
        check_len("up packed", packed[1].len(), e * id * (hd / 4))?;
        check_len("down packed", packed[2].len(), e * hd * (id / 4))?;
        check_len("gate scales", scales[0].len(), e * id)?;
        check_len("up scales", scales[1].len(), e * id)?;
        check_len("down scales", scales[2].len(), e * hd)?;
        Ok(QMoELayer {
            config,
            gate_weight: DeviceBuffer::from_slice(gate_weight, stream)?,
            packed: [DeviceBuffer::from_slice(packed[0], stream)?, DeviceBuffer::from_slice(packed[1], stream)?,
                     DeviceBuffer::from_slice(packed[2], stream)?],
            scales: [DeviceBuffer::from_slice(scales[0], stream)?, DeviceBuffer::from_slice(scales[1], stream)?,
                     DeviceBuffer::from_slice(scales[2], stream)?],
        })
    }
    pub fn workspace_bytes(&self, seq_len: usize) -> Result<usize> {
        let mut n = 0usize;
        ok(unsafe { qmla_moe_workspace_bytes(&self.config, seq_len as i32, &mut n) })?;
        Ok(n)
    }
    /// forward (src/moe.rs:40-130): xs [seq_len, hidden] -> out.
    pub fn forward(&self, xs: &DeviceBuffer, seq_len: usize, out: &mut DeviceBuffer, workspace: &mut DeviceBuffer,
                   stream: &Stream) -> Result<()> {
        let n = 4 * seq_len * self.config.hidden_dim.max(0) as usize;
        check_bytes("xs", xs, n)?;
        check_bytes("out", out, n)?;
        ok(unsafe {
            qmla_moe_forward(&self.config, xs.ptr() as *const f32, seq_len as i32,
                             self.gate_weight.ptr() as *const f32, self.packed[0].ptr() as *const u8,
                             self.scales[0].ptr() as *const f32, self.packed[1].ptr() as *const u8,
                             self.scales[1].ptr() as *const f32, self.packed[2].ptr() as *const u8,
                             self.scales[2].ptr() as *const f32, out.ptr_mut() as *mut f32, ptr::null_mut(),
                             ptr::null_mut(), workspace.ptr_mut(), workspace.bytes(), stream.raw())
        })
    }
}
