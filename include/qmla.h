/*
 * qmla.h -- C ABI of the MI355X (gfx950) MLA attention library (libqmla.so).
 *
 * This is the drop-in boundary for qmoe-rs's MLA attention hot path.  Each
 * entry point names the reference interface it replaces (paths relative to
 * the qmoe-rs source tree).  Plain C: no C++ types, no exceptions, no torch
 * types.  Device pointers are HIP device addresses (e.g. from
 * qmla_buffer_alloc); streams are hipStream_t passed as void* (NULL = the
 * default stream).
 *
 * Conventions
 *  - Every call returns a qmla_status.  On failure qmla_last_error() holds a
 *    message for the calling thread.  Shapes and pointers are validated
 *    before anything is launched; nothing aborts the process.
 *  - Compute calls are asynchronous on the given stream and allocate no
 *    device memory; scratch comes from a caller-provided workspace whose
 *    size is returned by the matching *_workspace_bytes query.  The one
 *    exception is cache growth past an exhausted page pool (see
 *    qmla_cache_set_growth; qmla_cache_reserve_pool avoids it).
 *  - Tensors are row-major and contiguous, in the layouts documented at
 *    each call.  bf16 values are stored as uint16 bit patterns.
 *  - Global mutable state: the per-thread error string, a per-device cached
 *    CU count, and the allocation-free decode's scratch array (one per GPU,
 *    with its device address cached per device; see
 *    qmla_decode_absorbed_noalloc: calls of that entry point that overlap on
 *    one GPU race and must be serialised by the caller).  Every other call
 *    on different streams may run from different threads.  A cache object
 *    must not be mutated concurrently.
 *    A layer object may be used from several threads at once: its GEMM path
 *    (prefill, and decode shapes the skinny kernel does not take) takes one
 *    of 4 rocBLAS handles created with the layer, so up to 4 such calls run
 *    without waiting for each other.
 */
#ifndef QMLA_H
#define QMLA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QMLA_VERSION 100 /* 0.1.0 */

#if defined(__GNUC__)
#define QMLA_API __attribute__((visibility("default")))
#else
#define QMLA_API
#endif

typedef enum {
  QMLA_OK = 0,
  QMLA_ERR_INVALID_ARG = 1, /* null pointer, bad enum, non-positive size      */
  QMLA_ERR_SHAPE = 2,       /* dimensions inconsistent or out of range        */
  QMLA_ERR_UNSUPPORTED = 3, /* valid request this build does not implement    */
  QMLA_ERR_HIP = 4,         /* a HIP runtime call failed                      */
  QMLA_ERR_OOM = 5,         /* device allocation failed                       */
  QMLA_ERR_CAPACITY = 6,    /* cache append beyond a sequence's capacity      */
  QMLA_ERR_WORKSPACE = 7    /* workspace missing or smaller than required     */
} qmla_status;

typedef enum { QMLA_F32 = 0, QMLA_BF16 = 1 } qmla_dtype;

typedef void *qmla_stream; /* hipStream_t */

/* ------------------------------------------------------------ library ---- */
QMLA_API int qmla_version(void);
/* Message of the last failed call on this thread ("" if none). */
QMLA_API const char *qmla_last_error(void);
QMLA_API const char *qmla_status_string(qmla_status s);
/* Current device ordinal, its compute-unit count and gfx name (>= 16 bytes). */
QMLA_API qmla_status qmla_device_info(int *device, int *cu_count, char *arch_name, size_t arch_len);

/* ------------------------------------------------ HBM-resident buffers ---
 * Replaces the host-only storage of src/tensor.rs:1-122 (PackedQMoETensor
 * owns mmap'd or Vec storage) with device buffers the engine owns.        */
QMLA_API qmla_status qmla_buffer_alloc(size_t bytes, void **out);
QMLA_API qmla_status qmla_buffer_free(void *ptr);
QMLA_API qmla_status qmla_memcpy_h2d(void *dst, const void *src, size_t bytes, qmla_stream stream);
QMLA_API qmla_status qmla_memcpy_d2h(void *dst, const void *src, size_t bytes, qmla_stream stream);
QMLA_API qmla_status qmla_memcpy_d2d(void *dst, const void *src, size_t bytes, qmla_stream stream);
QMLA_API qmla_status qmla_memset_zero(void *dst, size_t bytes, qmla_stream stream);
QMLA_API qmla_status qmla_stream_create(qmla_stream *out);
QMLA_API qmla_status qmla_stream_destroy(qmla_stream stream);
QMLA_API qmla_status qmla_stream_synchronize(qmla_stream stream);
/* Convert n f32 values to bf16 (round to nearest even) on the device. */
QMLA_API qmla_status qmla_f32_to_bf16(const float *src, uint16_t *dst, size_t n, qmla_stream stream);
/* Fill n f32 values with N(mean, std^2) from a counter-based generator
 * (a deterministic function of (seed, index); not bit-identical to any host
 * generator).  For synthetic benchmark inputs. */
QMLA_API qmla_status qmla_fill_normal_f32(float *dst, size_t n, uint64_t seed, float mean, float std_,
                                 qmla_stream stream);

/* ------------------------------------------- attention_kernel.rs -------- */
typedef struct {
  int32_t batch;        /* b                                              */
  int32_t heads;        /* h                                              */
  int32_t seq_q;        /* query rows per (b, h)                          */
  int32_t seq_k;        /* key rows per (b, h)                            */
  int32_t qk_nope;      /* dn (q_nope / k width)                          */
  int32_t qk_rope;      /* dr (q_rope / k_rope width, may be 0)           */
  int32_t v_dim;        /* dv                                             */
  int32_t k_rope_heads; /* 1: one rope key shared by all heads (latent
                           layout); heads: per-head copy (reference layout) */
  int32_t q_offset;     /* absolute position of query row 0 in the causal
                           mask (0 for plain prefill; cached length for a
                           chunk appended after a cache)                   */
} qmla_prefill_dims;

/* fused_prefill_attn, src/attention_kernel.rs:64-107:
 *   out = softmax((q_nope k^T + q_rope k_rope^T) * scale + mask) v
 * with the causal mask of make_causal_mask (:14-31): key j is masked for
 * query row i when q_offset + i < j.
 *   q_nope [b,h,seq_q,dn]  q_rope [b,h,seq_q,dr]  k [b,h,seq_k,dn]
 *   k_rope [b,k_rope_heads,seq_k,dr]  v [b,h,seq_k,dv]  out [b,h,seq_q,dv]
 * dtype QMLA_F32: f32 in/out, f32 math (parity mode).
 * dtype QMLA_BF16: bf16 in/out, bf16 MFMA with f32 accumulation.
 * q_offset >= 0, so every query row sees key 0; with causal = 0, q_offset
 * must be 0 and seq_q and seq_k may differ.  seq_k == 0 yields zeros. */
QMLA_API qmla_status qmla_fused_prefill_attn(const qmla_prefill_dims *dims, qmla_dtype dtype,
                                    const void *q_nope, const void *q_rope, const void *k,
                                    const void *k_rope, const void *v, double scale, int causal,
                                    void *out, qmla_stream stream);

/* reference_eager_attn, src/attention_kernel.rs:110-134 (and the intended
 * math of eager_prefill_attn, :34-57): single-part scores q k^T.
 *   q, k [b,h,s,d]  v [b,h,s,dv]  out [b,h,s,dv]                          */
QMLA_API qmla_status qmla_reference_eager_attn(int32_t b, int32_t h, int32_t s, int32_t d, int32_t dv,
                                      qmla_dtype dtype, const void *q, const void *k,
                                      const void *v, double scale, int causal, void *out,
                                      qmla_stream stream);
QMLA_API qmla_status qmla_eager_prefill_attn(int32_t b, int32_t h, int32_t s, int32_t d, int32_t dv,
                                    qmla_dtype dtype, const void *q, const void *k,
                                    const void *v, double scale, int causal, void *out,
                                    qmla_stream stream);

/* --------------------------------------- latent KV cache (model.rs) -----
 * Replaces KVCache, src/model.rs:86-105 ({k, v, k_rope} decompressed
 * per-head tensors grown by Tensor::cat on every append) with one latent row
 * per token, [c_kv (kv_lora_rank) | k_pe (rope_dim)], stored once for all
 * heads.  Rows live in pages of page_rows rows (a power of two >= 32); a
 * device block table lists each sequence's pages, so token t of sequence i
 * is row t % page_rows of page pages[i * table_width + t / page_rows].
 * Lengths live in a device int32 table, mirrored on the host together with
 * the block table, so no call needs a device sync to validate or to grow.
 * A sequence's capacity is the number of rows it may hold without growing
 * (at most its pages x page_rows). */
typedef struct qmla_kv_cache qmla_kv_cache;

typedef struct {
  int32_t num_seqs;
  int32_t kv_lora_rank;
  int32_t rope_dim;
  qmla_dtype dtype;  /* element type of the rows                    */
  int64_t row_elems; /* kv_lora_rank + rope_dim                      */
  /* Layout at creation: one chunk holding every sequence's pages in order,
   * sequence i from row offsets[i].  Valid while `contiguous` is 1 (no page
   * has been taken from the free list since); otherwise rows and offsets
   * are NULL and total_rows is 0. */
  int64_t total_rows;
  void *rows;        /* device: [total_rows, row_elems]               */
  int64_t *offsets;  /* device: [num_seqs] first row of each sequence */
  int32_t *lengths;  /* device: [num_seqs] current lengths            */
  int32_t *capacity; /* device: [num_seqs]                            */
  uint64_t *pages;   /* device: [num_seqs, table_width] page addresses */
  int32_t page_rows;
  int32_t table_width; /* pages one sequence can hold                 */
  int32_t contiguous;
  int32_t reserved;
} qmla_cache_desc;

/* KVCache::new, src/model.rs:95-97.  capacity[num_seqs] is a host array of
 * per-sequence token capacities; all lengths start at 0.  Same as
 * qmla_cache_create_paged(num_seqs, capacity, 0, 0, 0, ...). */
QMLA_API qmla_status qmla_cache_create(int32_t num_seqs, const int32_t *capacity, int32_t kv_lora_rank,
                              int32_t rope_dim, qmla_dtype dtype, qmla_kv_cache **out);
/* KVCache::new with the pool laid out by the caller.  max_len: the longest
 * a sequence may grow (0: 163840, DeepSeek-V2's max_position_embeddings, or
 * the largest capacity if larger); it sizes the block table.  pool_rows:
 * rows of HBM to allocate now (0: just the capacities); rows beyond the
 * capacities start on the free list that growth draws from.  page_rows: 0
 * for 256. */
QMLA_API qmla_status qmla_cache_create_paged(int32_t num_seqs, const int32_t *capacity, int64_t max_len,
                                    int64_t pool_rows, int32_t page_rows, int32_t kv_lora_rank,
                                    int32_t rope_dim, qmla_dtype dtype, qmla_kv_cache **out);
QMLA_API qmla_status qmla_cache_destroy(qmla_kv_cache *cache);
/* #[derive(Clone)] on KVCache, src/model.rs:87: deep copy of rows and
 * lengths (capacities kept; the clone's pages are packed into one chunk). */
QMLA_API qmla_status qmla_cache_clone(const qmla_kv_cache *cache, qmla_kv_cache **out, qmla_stream stream);
/* KVCache::append, src/model.rs:99-104: appends n_new tokens to each of
 * sequences 0..n_seqs-1.  rows [n_seqs, n_new, kv_lora_rank + rope_dim] on
 * the device, f32 (converted to the cache dtype, bf16 by round-to-nearest-
 * even) or already in the cache dtype (rows_dtype == cache dtype).  O(new
 * rows) work, never a copy of the existing cache. */
QMLA_API qmla_status qmla_cache_append(qmla_kv_cache *cache, const void *rows, qmla_dtype rows_dtype,
                              int32_t n_seqs, int32_t n_new, qmla_stream stream);
/* Ragged form: appends n_new rows to sequence `seq` only. */
QMLA_API qmla_status qmla_cache_append_seq(qmla_kv_cache *cache, int32_t seq, const void *rows,
                                  qmla_dtype rows_dtype, int32_t n_new, qmla_stream stream);
/* Sets every sequence's length (host array [num_seqs], each <= its
 * capacity) without writing rows: rows past the old length keep whatever
 * the pages hold.  Used to truncate, or after filling the pool directly
 * through qmla_cache_describe.  Stream-ordered; `lengths` may be reused as
 * soon as the call returns and the host does not wait for the device. */
QMLA_API qmla_status qmla_cache_set_lengths(qmla_kv_cache *cache, const int32_t *lengths,
                                   qmla_stream stream);
/* Length read (`cache.k.dim(2)`, src/model.rs:259) from the host mirror. */
QMLA_API qmla_status qmla_cache_lengths(const qmla_kv_cache *cache, int32_t *lengths_out);
QMLA_API qmla_status qmla_cache_describe(const qmla_kv_cache *cache, qmla_cache_desc *out);
/* Rows [t0, t0 + n) of sequence `seq` (t0 + n <= its capacity) copied into
 * `out` (device, [n, row_elems] in the cache dtype): the reference's
 * `cache.k` read of one sequence, in latent form, whatever pages hold it. */
QMLA_API qmla_status qmla_cache_gather(const qmla_kv_cache *cache, int32_t seq, int32_t t0, int32_t n,
                              void *out, qmla_stream stream);
/* Capacity growth.  KVCache::append (src/model.rs:99-104) grows its tensors
 * without bound by copying them; here a sequence grows by taking pages from
 * the cache's free list and writing their addresses into its block table
 * (one small kernel on `stream`).  No row moves, no pointer from
 * qmla_cache_describe changes meaning except rows/offsets (see above), and
 * the host does not wait.  Device memory is allocated only when the free
 * list is short: then a chunk of max(missing pages, min(half the pool,
 * 1 GiB)) is added with hipMalloc.  qmla_cache_reserve_pool tops the free list up ahead
 * of time, so that appends and layer calls allocate nothing.
 * qmla_cache_reserve raises sequence i's capacity to at least
 * min_capacity[i] (host array [num_seqs]; smaller entries change nothing).
 * qmla_cache_set_growth(cache, 1): appends and the layer calls that would
 * pass a sequence's capacity first take the pages they need (the capacity
 * becomes every row of the sequence's pages) instead of failing with
 * QMLA_ERR_CAPACITY; past max_len they still fail.  Off by default; clones
 * inherit it.  qmla_cache_capacity reads the host mirror of the capacities.
 * qmla_cache_trim returns each listed sequence's pages beyond its current
 * length to the free list (capacities shrink to match); pages freed here
 * may be handed out by the next growth, so work on other streams that still
 * reads those rows must be ordered before it.  qmla_cache_pool_info reports
 * the pool's rows and the free list's rows (either pointer may be NULL).
 * On failure (QMLA_ERR_CAPACITY past max_len, QMLA_ERR_OOM) the cache is
 * unchanged. */
QMLA_API qmla_status qmla_cache_reserve(qmla_kv_cache *cache, const int32_t *min_capacity,
                               qmla_stream stream);
QMLA_API qmla_status qmla_cache_reserve_pool(qmla_kv_cache *cache, int64_t free_rows);
QMLA_API qmla_status qmla_cache_set_growth(qmla_kv_cache *cache, int32_t enable);
QMLA_API qmla_status qmla_cache_capacity(const qmla_kv_cache *cache, int32_t *capacity_out);
QMLA_API qmla_status qmla_cache_trim(qmla_kv_cache *cache, int32_t seq0, int32_t n_seqs,
                            qmla_stream stream);
QMLA_API qmla_status qmla_cache_pool_info(const qmla_kv_cache *cache, int64_t *pool_rows,
                                 int64_t *free_rows);

/* ------------------------------------------- absorbed latent decode ------
 * The attention core of MlaAttention::forward_with_cache,
 * src/model.rs:294-303, in absorbed form over the latent cache.  For query
 * row m of sequence i (rows are heads x new tokens; every row attends every
 * cached token, as :297-302 applies no mask):
 *   s_t = scale * (q_latent[i,m] . c_t + q_rope[i,m] . kpe_t)
 *   out_latent[i,m] = sum_t softmax(s)_t c_t,  out_lse[i,m] = logsumexp(s)
 * q_latent [batch, rows, kv_lora_rank], q_rope [batch, rows, rope_dim] are
 * f32 (QMLA_F32) or bf16 (QMLA_BF16); out_latent is f32 [batch, rows, r];
 * out_lse f32 [batch, rows] or NULL.  Sequences 0..batch-1 of the cache are
 * used with their current device lengths (a zero-length sequence yields 0
 * and lse = -inf).  f32 cache: f32 math.  bf16 cache: bf16 MFMA, f32
 * accumulation; q is rounded to bf16.
 * The token range of all sequences is split evenly over the device's
 * compute units; partial results are merged by log-sum-exp.               */
typedef struct {
  int32_t batch;
  int32_t rows;         /* query rows per sequence (heads x new tokens) */
  int32_t kv_lora_rank; /* must equal the cache's                       */
  int32_t rope_dim;     /* must equal the cache's                       */
} qmla_decode_dims;

QMLA_API qmla_status qmla_decode_workspace_bytes(const qmla_decode_dims *dims, const qmla_kv_cache *cache,
                                        size_t *bytes);
QMLA_API qmla_status qmla_decode_absorbed(const qmla_decode_dims *dims, const qmla_kv_cache *cache,
                                 qmla_dtype q_dtype, const void *q_latent, const void *q_rope,
                                 double scale, float *out_latent, float *out_lse,
                                 void *workspace, size_t workspace_bytes, qmla_stream stream);
/* Same, with the number of token splits fixed by the caller (>= 1): used by
 * the split-invariance tests and for tuning.  0 means automatic. */
QMLA_API qmla_status qmla_decode_absorbed_splits(const qmla_decode_dims *dims, const qmla_kv_cache *cache,
                                        qmla_dtype q_dtype, const void *q_latent,
                                        const void *q_rope, double scale, float *out_latent,
                                        float *out_lse, int32_t num_splits, void *workspace,
                                        size_t workspace_bytes, qmla_stream stream);
QMLA_API qmla_status qmla_decode_workspace_bytes_splits(const qmla_decode_dims *dims,
                                               const qmla_kv_cache *cache, int32_t num_splits,
                                               size_t *bytes);

/* Allocation-free form of qmla_decode_absorbed.  It has no counterpart in
 * the reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, results and errors as qmla_decode_absorbed,
 * without the workspace: the split partials live in a static device array
 * of QMLA_DECODE_NOALLOC_SCRATCH_BYTES per GPU, held from the library's
 * first use of that GPU until the process ends.  A call whose workspace
 * (qmla_decode_workspace_bytes) would exceed that size returns
 * QMLA_ERR_UNSUPPORTED before anything is launched; the 128-head,
 * batch-64 decode over 256 compute units needs 40 MiB.  The call allocates
 * nothing.  Every call on one GPU shares that GPU's array: calls that
 * overlap on one GPU (other streams, other threads) race and must be
 * serialised by the caller. */
#define QMLA_DECODE_NOALLOC_SCRATCH_BYTES ((size_t)48 << 20)
QMLA_API qmla_status qmla_decode_absorbed_noalloc(const qmla_decode_dims *dims,
                                         const qmla_kv_cache *cache, qmla_dtype q_dtype,
                                         const void *q_latent, const void *q_rope, double scale,
                                         float *out_latent, float *out_lse, qmla_stream stream);

/* --------------------------------------------- MLA layer (model.rs) -----
 * MlaAttention, src/model.rs:107-307, with device-resident weights.
 * Weights are given as host f32 arrays in the reference's Linear layout
 * ([out, in] weight, [out] bias), copied to the device at creation:
 *   wq [H(dn+dr), hidden]   bq    q_proj              src/model.rs:126-130
 *   wkva [r+dr, hidden]     bkva  kv_a_proj_with_mqa  src/model.rs:131-135
 *   ln_w, ln_b [r]                kv_a_layernorm      src/model.rs:136
 *   wkvb [H(dn+dv), r]      bkvb  kv_b_proj           src/model.rs:137-141
 *   wo [hidden, H dv]       bo    o_proj              src/model.rs:142-146
 * Any bias pointer may be NULL (treated as zero).                        */
typedef struct {
  int32_t hidden, heads, qk_nope, qk_rope, v_dim, kv_lora_rank;
  double rope_mscale;   /* src/model.rs:160-165 (1.0857263992...)   */
  double softmax_scale; /* src/model.rs:166-173 (0.1147213868 at 192) */
  double ln_eps;        /* 1e-6, src/model.rs:136                     */
} qmla_layer_config;

typedef struct qmla_layer qmla_layer;

/* Fills rope_mscale / softmax_scale / ln_eps from the reference's
 * constructor (YaRN factor 40, mscale 1.0, mscale_all_dim 0.707). */
QMLA_API qmla_status qmla_layer_default_scales(qmla_layer_config *cfg);
QMLA_API qmla_status qmla_layer_create(const qmla_layer_config *cfg, const float *wq, const float *bq,
                              const float *wkva, const float *bkva, const float *ln_w,
                              const float *ln_b, const float *wkvb, const float *bkvb,
                              const float *wo, const float *bo, qmla_layer **out);
QMLA_API qmla_status qmla_layer_destroy(qmla_layer *layer);
/* Operand precision of the layer's hand-written projection kernels: q_proj
 * with kv_a_proj_with_mqa, the W_UK / W_UV absorption products and o_proj of
 * a decode step, and q_proj, kv_a_proj_with_mqa, kv_b_proj and o_proj of a
 * prefill.  No counterpart in the reference, whose Linear layers compute in
 * the weights' dtype (f32 there).
 *   QMLA_F32 (the default): f32-exact products (each operand as bf16 hi + lo
 *     halves, three bf16 MFMAs per step, f32 accumulation; ~2^-16 relative).
 *   QMLA_BF16: bf16 operands with f32 accumulation -- the weights rounded to
 *     bf16 (their hi halves), the activations rounded to nearest even; one
 *     MFMA per step and half the weight bytes.  Results then hold the bf16
 *     tolerance (2e-2), whatever the cache dtype.
 * The rocBLAS paths (prefill below 128 tokens, decode shapes the skinny
 * kernel does not take) and qmla_cache_materialise stay f32-exact.  Applies
 * to calls issued after it returns: set it before the layer is shared with
 * other threads.  QMLA_ERR_INVALID_ARG for a NULL layer or another dtype. */
QMLA_API qmla_status qmla_layer_set_projection_dtype(qmla_layer *layer, qmla_dtype dtype);
/* Device scratch that serves either forward call below for (batch, seq)
 * new tokens: the larger of the two calls' needs (their call-specific
 * regions overlay one another).  No counterpart in the reference, which
 * allocates per call; the size does not depend on the cached lengths. */
QMLA_API qmla_status qmla_layer_workspace_bytes(const qmla_layer *layer, const qmla_kv_cache *cache,
                                       int32_t batch, int32_t seq, size_t *bytes);
/* Device scratch that qmla_layer_forward_prefill alone needs for (batch,
 * seq) tokens (at most qmla_layer_workspace_bytes; the decode core's
 * partials, which grow with seq x heads, are not part of it).  No
 * counterpart in the reference. */
QMLA_API qmla_status qmla_layer_prefill_workspace_bytes(const qmla_layer *layer,
                                               const qmla_kv_cache *cache, int32_t batch,
                                               int32_t seq, size_t *bytes);
/* MlaAttention::forward_with_cache, src/model.rs:256-307, over the latent
 * cache: xs [batch, seq, hidden] f32 device, out [batch, seq, hidden] f32
 * (both 16-byte aligned, the workspace 256-byte aligned, as device
 * allocations are; otherwise QMLA_ERR_INVALID_ARG / QMLA_ERR_WORKSPACE).
 * Appends the seq new latent rows of sequences 0..batch-1 to the cache and
 * attends all cached + new tokens without a mask (as :297-302).  Lengths
 * may differ across the batch (a ragged batch; the reference's KVCache is
 * uniform, :259): sequence b's new tokens take RoPE positions len_b + i,
 * read from the cache's device length table, so the call needs no host
 * copy of the lengths.  Every argument, shape and workspace check runs
 * before the cache is modified: a rejected call leaves it unchanged.
 * f32 cache: f32 throughout.  bf16 cache: the new rows are stored rounded
 * to bf16 and the attention core is the bf16 MFMA decode (kv_lora_rank /
 * rope 512/64, 128/32 or 64/16; other shapes return QMLA_ERR_UNSUPPORTED);
 * the projections stay f32 unless qmla_layer_set_projection_dtype chose
 * bf16 operands. */
QMLA_API qmla_status qmla_layer_forward_with_cache(const qmla_layer *layer, const float *xs, int32_t batch,
                                          int32_t seq, qmla_kv_cache *cache, float *out,
                                          void *workspace, size_t workspace_bytes,
                                          qmla_stream stream);
/* MlaAttention::forward_prefill, src/model.rs:193-253: causal attention
 * over the seq tokens, which are appended to the (empty) cache sequences
 * 0..batch-1 -- the latent replacement of the KVCache it returns (:250).
 * Same pointer alignment as qmla_layer_forward_with_cache. */
QMLA_API qmla_status qmla_layer_forward_prefill(const qmla_layer *layer, const float *xs, int32_t batch,
                                       int32_t seq, qmla_kv_cache *cache, float *out,
                                       void *workspace, size_t workspace_bytes,
                                       qmla_stream stream);

/* The public tensors of KVCache, src/model.rs:88-92 ({k, v, k_rope}, read
 * and written directly by benches/attention.rs:68-70,256), rebuilt from the
 * latent rows through the layer's kv_b_proj (compute_kv, :178-190):
 *   k      [n_seqs, H, T, qk_nope]  = c W_UK^h^T + b_K^h
 *   v      [n_seqs, H, T, v_dim]    = c W_UV^h^T + b_V^h
 *   k_rope [n_seqs, H, T, qk_rope]  = the stored roped k_pe, broadcast to
 *                                     every head (:217-219)
 * for sequences seq0 .. seq0 + n_seqs - 1, which must share one length T
 * (a KVCache tensor has one T; materialise a ragged cache one sequence at a
 * time).  f32 device outputs; any of k, v, k_rope may be NULL to skip it.
 * The latent rows are gathered into a workspace whose size the query
 * gives: n_seqs * T * kv_lora_rank floats, or, for T >= 256, the rows in
 * the split form of the bf16 GEMMs that then compute k and v (about
 * 3 kv_lora_rank bf16 per row; x w as x_hi w_hi + x_lo w_hi + x_hi w_lo with
 * f32 accumulation, within the f32 tolerance).
 * The writes are O(T * H * (dn + dv + dr)) per sequence: this is the
 * legacy path for callers that read the decompressed tensors, not the
 * decode path. */
QMLA_API qmla_status qmla_cache_materialise_workspace_bytes(const qmla_layer *layer,
                                                   const qmla_kv_cache *cache, int32_t seq0,
                                                   int32_t n_seqs, size_t *bytes);
QMLA_API qmla_status qmla_cache_materialise(const qmla_layer *layer, const qmla_kv_cache *cache,
                                   int32_t seq0, int32_t n_seqs, float *k, float *v,
                                   float *k_rope, void *workspace, size_t workspace_bytes,
                                   qmla_stream stream);

/* ------------------------------------ 2-bit packed MoE (tensor.rs, moe.rs)
 * Packed format (src/simd.rs:20-31): an [out_features, in_features] tensor
 * is out_features rows of in_features / 4 bytes; weight 4j + q of a row is
 * bits 2q..2q+1 of byte j, a code c in 0..3 standing for the weight c - 1.
 * All buffers are device memory.
 *
 * PackedQMoETensor::forward_simd (src/tensor.rs:64-95, forward_simd_raw
 * :99-121): out[b][i] = (sum_k w_ik x[b][k]) * scales[i] for x
 * [batch, in_features] f32, out [batch, out_features] f32.  Activations past
 * 4 * (in_features / 4) are ignored, as in src/simd.rs:15.
 * in_features a multiple of 128: int8 MFMA over an exact integer form of x
 * (x rounded to 23 bits relative to each row's largest element, sums exact);
 * other widths: f32 lane sums in the reference's order.  A row of x holding
 * inf or NaN yields NaN outputs on the MFMA path.                          */
QMLA_API qmla_status qmla_packed_forward_workspace_bytes(int32_t out_features, int32_t in_features,
                                                int32_t batch, size_t *bytes);
QMLA_API qmla_status qmla_packed_forward(const uint8_t *packed, const float *scales,
                                int32_t out_features, int32_t in_features, const float *x,
                                int32_t batch, float *out, void *workspace,
                                size_t workspace_bytes, qmla_stream stream);

/* MoEConfig (src/moe.rs:5-11). */
typedef struct {
  int32_t num_experts;
  int32_t top_k;
  int32_t hidden_dim;
  int32_t intermediate_dim;
} qmla_moe_config;

/* QMoELayer::forward (src/moe.rs:40-130) for xs [seq_len, hidden] f32:
 * gate logits xs . gate_weight^T (gate_weight [E, hidden] f32), the top_k
 * experts by (logit descending, expert index ascending) -- the order of the
 * reference's stable sort --, weights softmax-over-all-experts of their
 * logits, SwiGLU experts
 *   y_e(x) = down_e(swish(gate_e(x)) * up_e(x)),  swish(g) = g / (1 + e^-g)
 * with packed gate/up [E, I, hidden/4], down [E, hidden, I/4] (expert e's
 * PackedQMoETensor at offset e of each array) and scales gate/up [E, I],
 * down [E, hidden]; out[t] = sum of weight * y_e(x_t) over the token's
 * experts in ascending expert order.  top_experts / top_weights
 * ([seq_len, top_k], nullable) receive the routing in rank order.
 * num_experts == 0 or top_k == 0 gives zeros (src/moe.rs:46-48);
 * top_k > num_experts is QMLA_ERR_SHAPE (the reference panics).          */
QMLA_API qmla_status qmla_moe_workspace_bytes(const qmla_moe_config *cfg, int32_t seq_len,
                                     size_t *bytes);
QMLA_API qmla_status qmla_moe_forward(const qmla_moe_config *cfg, const float *xs, int32_t seq_len,
                             const float *gate_weight, const uint8_t *gate_packed,
                             const float *gate_scales, const uint8_t *up_packed,
                             const float *up_scales, const uint8_t *down_packed,
                             const float *down_scales, float *out, int32_t *top_experts,
                             float *top_weights, void *workspace, size_t workspace_bytes,
                             qmla_stream stream);

#ifdef __cplusplus
}
#endif
#endif /* QMLA_H */
