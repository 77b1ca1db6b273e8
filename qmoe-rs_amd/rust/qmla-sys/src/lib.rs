//! Raw bindings of `include/qmla.h`, the C ABI of libqmla.so (the MI355X
//! MLA attention hot path of qmoe-rs and its 2-bit packed MoE GEMV).
//!
//! One declaration per header entry point, with the header's names,
//! argument names and argument order; `#[repr(C)]` structs with the
//! header's field order.  `tests/test_rust_binding.py` in the repository
//! checks this file against the header.  Safe wrappers live in the `qmla`
//! crate beside this one.
#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_int, c_void};

pub const QMLA_VERSION: c_int = 100;

/// `qmla_status`: every call returns one; the message of a failure is in
/// `qmla_last_error()` (thread-local).
pub type qmla_status = c_int;
pub const QMLA_OK: qmla_status = 0;
pub const QMLA_ERR_INVALID_ARG: qmla_status = 1;
pub const QMLA_ERR_SHAPE: qmla_status = 2;
pub const QMLA_ERR_UNSUPPORTED: qmla_status = 3;
pub const QMLA_ERR_HIP: qmla_status = 4;
pub const QMLA_ERR_OOM: qmla_status = 5;
pub const QMLA_ERR_CAPACITY: qmla_status = 6;
pub const QMLA_ERR_WORKSPACE: qmla_status = 7;

/// `qmla_dtype`: element type of a tensor (bf16 as u16 bit patterns).
pub type qmla_dtype = c_int;
pub const QMLA_F32: qmla_dtype = 0;
pub const QMLA_BF16: qmla_dtype = 1;

/// `hipStream_t`; null is the default stream.
pub type qmla_stream = *mut c_void;

/// Scratch of `qmla_decode_absorbed_noalloc` per GPU, in bytes.
pub const QMLA_DECODE_NOALLOC_SCRATCH_BYTES: usize = 48 << 20;

/// Opaque latent KV cache (replaces KVCache, src/model.rs:86-105).
#[repr(C)]
pub struct qmla_kv_cache {
    _private: [u8; 0],
}

/// Opaque MlaAttention with device weights (src/model.rs:107-307).
#[repr(C)]
pub struct qmla_layer {
    _private: [u8; 0],
}

/// Shapes of a prefill call (fused_prefill_attn, src/attention_kernel.rs:64-107).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct qmla_prefill_dims {
    pub batch: i32,
    pub heads: i32,
    pub seq_q: i32,
    pub seq_k: i32,
    pub qk_nope: i32,
    pub qk_rope: i32,
    pub v_dim: i32,
    pub k_rope_heads: i32,
    pub q_offset: i32,
}

/// Device layout of a latent cache (qmla_cache_describe).
#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct qmla_cache_desc {
    pub num_seqs: i32,
    pub kv_lora_rank: i32,
    pub rope_dim: i32,
    pub dtype: qmla_dtype,
    pub row_elems: i64,
    pub total_rows: i64,
    pub rows: *mut c_void,
    pub offsets: *mut i64,
    pub lengths: *mut i32,
    pub capacity: *mut i32,
    pub pages: *mut u64,
    pub page_rows: i32,
    pub table_width: i32,
    pub contiguous: i32,
    pub reserved: i32,
}

/// Shapes of an absorbed decode call.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct qmla_decode_dims {
    pub batch: i32,
    pub rows: i32,
    pub kv_lora_rank: i32,
    pub rope_dim: i32,
}

/// MlaAttention's dimensions and scales (src/model.rs:107-173).
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct qmla_layer_config {
    pub hidden: i32,
    pub heads: i32,
    pub qk_nope: i32,
    pub qk_rope: i32,
    pub v_dim: i32,
    pub kv_lora_rank: i32,
    pub rope_mscale: f64,
    pub softmax_scale: f64,
    pub ln_eps: f64,
}

/// MoEConfig, src/moe.rs:5-11.
#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct qmla_moe_config {
    pub num_experts: i32,
    pub top_k: i32,
    pub hidden_dim: i32,
    pub intermediate_dim: i32,
}

extern "C" {
    pub fn qmla_version() -> c_int;
    pub fn qmla_last_error() -> *const c_char;
    pub fn qmla_status_string(s: qmla_status) -> *const c_char;
    pub fn qmla_device_info(
        device: *mut c_int, cu_count: *mut c_int, arch_name: *mut c_char, arch_len: usize
    ) -> qmla_status;
    // src/tensor.rs: HBM-resident buffers
    pub fn qmla_buffer_alloc(bytes: usize, out: *mut *mut c_void) -> qmla_status;
    pub fn qmla_buffer_free(ptr: *mut c_void) -> qmla_status;
    pub fn qmla_memcpy_h2d(
        dst: *mut c_void, src: *const c_void, bytes: usize, stream: qmla_stream
    ) -> qmla_status;
    pub fn qmla_memcpy_d2h(
        dst: *mut c_void, src: *const c_void, bytes: usize, stream: qmla_stream
    ) -> qmla_status;
    pub fn qmla_memcpy_d2d(
        dst: *mut c_void, src: *const c_void, bytes: usize, stream: qmla_stream
    ) -> qmla_status;
    pub fn qmla_memset_zero(dst: *mut c_void, bytes: usize, stream: qmla_stream) -> qmla_status;
    pub fn qmla_stream_create(out: *mut qmla_stream) -> qmla_status;
    pub fn qmla_stream_destroy(stream: qmla_stream) -> qmla_status;
    pub fn qmla_stream_synchronize(stream: qmla_stream) -> qmla_status;
    pub fn qmla_f32_to_bf16(
        src: *const f32, dst: *mut u16, n: usize, stream: qmla_stream
    ) -> qmla_status;
    pub fn qmla_fill_normal_f32(
        dst: *mut f32, n: usize, seed: u64, mean: f32, std_: f32, stream: qmla_stream
    ) -> qmla_status;
    // fused_prefill_attn, src/attention_kernel.rs:64-107
    pub fn qmla_fused_prefill_attn(
        dims: *const qmla_prefill_dims, dtype: qmla_dtype, q_nope: *const c_void,
        q_rope: *const c_void, k: *const c_void, k_rope: *const c_void, v: *const c_void,
        scale: f64, causal: c_int, out: *mut c_void, stream: qmla_stream
    ) -> qmla_status;
    // reference_eager_attn, src/attention_kernel.rs:110-134
    pub fn qmla_reference_eager_attn(
        b: i32, h: i32, s: i32, d: i32, dv: i32, dtype: qmla_dtype, q: *const c_void,
        k: *const c_void, v: *const c_void, scale: f64, causal: c_int, out: *mut c_void,
        stream: qmla_stream
    ) -> qmla_status;
    // eager_prefill_attn, src/attention_kernel.rs:34-57
    pub fn qmla_eager_prefill_attn(
        b: i32, h: i32, s: i32, d: i32, dv: i32, dtype: qmla_dtype, q: *const c_void,
        k: *const c_void, v: *const c_void, scale: f64, causal: c_int, out: *mut c_void,
        stream: qmla_stream
    ) -> qmla_status;
    // KVCache::new, src/model.rs:95-97
    pub fn qmla_cache_create(
        num_seqs: i32, capacity: *const i32, kv_lora_rank: i32, rope_dim: i32, dtype: qmla_dtype,
        out: *mut *mut qmla_kv_cache
    ) -> qmla_status;
    pub fn qmla_cache_create_paged(
        num_seqs: i32, capacity: *const i32, max_len: i64, pool_rows: i64, page_rows: i32,
        kv_lora_rank: i32, rope_dim: i32, dtype: qmla_dtype, out: *mut *mut qmla_kv_cache
    ) -> qmla_status;
    pub fn qmla_cache_destroy(cache: *mut qmla_kv_cache) -> qmla_status;
    // #[derive(Clone)] KVCache, src/model.rs:87
    pub fn qmla_cache_clone(
        cache: *const qmla_kv_cache, out: *mut *mut qmla_kv_cache, stream: qmla_stream
    ) -> qmla_status;
    // KVCache::append, src/model.rs:99-104
    pub fn qmla_cache_append(
        cache: *mut qmla_kv_cache, rows: *const c_void, rows_dtype: qmla_dtype, n_seqs: i32,
        n_new: i32, stream: qmla_stream
    ) -> qmla_status;
    pub fn qmla_cache_append_seq(
        cache: *mut qmla_kv_cache, seq: i32, rows: *const c_void, rows_dtype: qmla_dtype,
        n_new: i32, stream: qmla_stream
    ) -> qmla_status;
    pub fn qmla_cache_set_lengths(
        cache: *mut qmla_kv_cache, lengths: *const i32, stream: qmla_stream
    ) -> qmla_status;
    // cache.k.dim(2), src/model.rs:259
    pub fn qmla_cache_lengths(cache: *const qmla_kv_cache, lengths_out: *mut i32) -> qmla_status;
    pub fn qmla_cache_describe(
        cache: *const qmla_kv_cache, out: *mut qmla_cache_desc
    ) -> qmla_status;
    pub fn qmla_cache_gather(
        cache: *const qmla_kv_cache, seq: i32, t0: i32, n: i32, out: *mut c_void,
        stream: qmla_stream
    ) -> qmla_status;
    pub fn qmla_cache_reserve(
        cache: *mut qmla_kv_cache, min_capacity: *const i32, stream: qmla_stream
    ) -> qmla_status;
    pub fn qmla_cache_reserve_pool(cache: *mut qmla_kv_cache, free_rows: i64) -> qmla_status;
    pub fn qmla_cache_set_growth(cache: *mut qmla_kv_cache, enable: i32) -> qmla_status;
    pub fn qmla_cache_capacity(cache: *const qmla_kv_cache, capacity_out: *mut i32) -> qmla_status;
    pub fn qmla_cache_trim(
        cache: *mut qmla_kv_cache, seq0: i32, n_seqs: i32, stream: qmla_stream
    ) -> qmla_status;
    pub fn qmla_cache_pool_info(
        cache: *const qmla_kv_cache, pool_rows: *mut i64, free_rows: *mut i64
    ) -> qmla_status;
    // attention core of forward_with_cache, src/model.rs:294-303
    pub fn qmla_decode_workspace_bytes(
        dims: *const qmla_decode_dims, cache: *const qmla_kv_cache, bytes: *mut usize
    ) -> qmla_status;
    pub fn qmla_decode_absorbed(
        dims: *const qmla_decode_dims, cache: *const qmla_kv_cache, q_dtype: qmla_dtype,
        q_latent: *const c_void, q_rope: *const c_void, scale: f64, out_latent: *mut f32,
        out_lse: *mut f32, workspace: *mut c_void, workspace_bytes: usize, stream: qmla_stream
    ) -> qmla_status;
    pub fn qmla_decode_absorbed_splits(
        dims: *const qmla_decode_dims, cache: *const qmla_kv_cache, q_dtype: qmla_dtype,
        q_latent: *const c_void, q_rope: *const c_void, scale: f64, out_latent: *mut f32,
        out_lse: *mut f32, num_splits: i32, workspace: *mut c_void, workspace_bytes: usize,
        stream: qmla_stream
    ) -> qmla_status;
    pub fn qmla_decode_workspace_bytes_splits(
        dims: *const qmla_decode_dims, cache: *const qmla_kv_cache, num_splits: i32,
        bytes: *mut usize
    ) -> qmla_status;
    // no counterpart in the reference: for callers that cannot allocate
    pub fn qmla_decode_absorbed_noalloc(
        dims: *const qmla_decode_dims, cache: *const qmla_kv_cache, q_dtype: qmla_dtype,
        q_latent: *const c_void, q_rope: *const c_void, scale: f64, out_latent: *mut f32,
        out_lse: *mut f32, stream: qmla_stream
    ) -> qmla_status;
    // MlaAttention::new, src/model.rs:160-173
    pub fn qmla_layer_default_scales(cfg: *mut qmla_layer_config) -> qmla_status;
    // MlaAttention fields, src/model.rs:107-146
    pub fn qmla_layer_create(
        cfg: *const qmla_layer_config, wq: *const f32, bq: *const f32, wkva: *const f32,
        bkva: *const f32, ln_w: *const f32, ln_b: *const f32, wkvb: *const f32, bkvb: *const f32,
        wo: *const f32, bo: *const f32, out: *mut *mut qmla_layer
    ) -> qmla_status;
    pub fn qmla_layer_destroy(layer: *mut qmla_layer) -> qmla_status;
    // no counterpart in the reference: bf16 operands in the projection kernels
    pub fn qmla_layer_set_projection_dtype(layer: *mut qmla_layer, dtype: qmla_dtype) -> qmla_status;
    pub fn qmla_layer_workspace_bytes(
        layer: *const qmla_layer, cache: *const qmla_kv_cache, batch: i32, seq: i32,
        bytes: *mut usize
    ) -> qmla_status;
    pub fn qmla_layer_prefill_workspace_bytes(
        layer: *const qmla_layer, cache: *const qmla_kv_cache, batch: i32, seq: i32,
        bytes: *mut usize
    ) -> qmla_status;
    // MlaAttention::forward_with_cache, src/model.rs:256-307
    pub fn qmla_layer_forward_with_cache(
        layer: *const qmla_layer, xs: *const f32, batch: i32, seq: i32,
        cache: *mut qmla_kv_cache, out: *mut f32, workspace: *mut c_void, workspace_bytes: usize,
        stream: qmla_stream
    ) -> qmla_status;
    // MlaAttention::forward_prefill, src/model.rs:193-253
    pub fn qmla_layer_forward_prefill(
        layer: *const qmla_layer, xs: *const f32, batch: i32, seq: i32,
        cache: *mut qmla_kv_cache, out: *mut f32, workspace: *mut c_void, workspace_bytes: usize,
        stream: qmla_stream
    ) -> qmla_status;
    // KVCache {k, v, k_rope}, src/model.rs:88-92, via compute_kv :178-190
    pub fn qmla_cache_materialise_workspace_bytes(
        layer: *const qmla_layer, cache: *const qmla_kv_cache, seq0: i32, n_seqs: i32,
        bytes: *mut usize
    ) -> qmla_status;
    pub fn qmla_cache_materialise(
        layer: *const qmla_layer, cache: *const qmla_kv_cache, seq0: i32, n_seqs: i32,
        k: *mut f32, v: *mut f32, k_rope: *mut f32, workspace: *mut c_void,
        workspace_bytes: usize, stream: qmla_stream
    ) -> qmla_status;
    // PackedQMoETensor::forward_simd, src/tensor.rs:64-95
    pub fn qmla_packed_forward_workspace_bytes(
        out_features: i32, in_features: i32, batch: i32, bytes: *mut usize
    ) -> qmla_status;
    pub fn qmla_packed_forward(
        packed: *const u8, scales: *const f32, out_features: i32, in_features: i32,
        x: *const f32, batch: i32, out: *mut f32, workspace: *mut c_void, workspace_bytes: usize,
        stream: qmla_stream
    ) -> qmla_status;
    // QMoELayer::forward, src/moe.rs:40-130
    pub fn qmla_moe_workspace_bytes(
        cfg: *const qmla_moe_config, seq_len: i32, bytes: *mut usize
    ) -> qmla_status;
    pub fn qmla_moe_forward(
        cfg: *const qmla_moe_config, xs: *const f32, seq_len: i32, gate_weight: *const f32,
        gate_packed: *const u8, gate_scales: *const f32, up_packed: *const u8,
        up_scales: *const f32, down_packed: *const u8, down_scales: *const f32, out: *mut f32,
        top_experts: *mut i32, top_weights: *mut f32, workspace: *mut c_void,
        workspace_bytes: usize, stream: qmla_stream
    ) -> qmla_status;
}

/// The library's message for a failed call on this thread.
pub fn last_error() -> String {
    // SAFETY: qmla_last_error returns a NUL-terminated thread-local string.
    unsafe { std::ffi::CStr::from_ptr(qmla_last_error()) }
        .to_string_lossy()
        .into_owned()
}

/// Maps a status to `Err(message)`.
pub fn check(st: qmla_status) -> Result<(), String> {
    if st == QMLA_OK {
        Ok(())
    } else {
        Err(last_error())
    }
}
