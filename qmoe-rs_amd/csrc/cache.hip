// cache.hip -- the latent KV cache (replacement of KVCache,
// src/model.rs:86-105).
//
// The reference grows per-head decompressed k/v/k_rope tensors with
// Tensor::cat on every token (an O(T) copy per token per layer).  Here each
// token is one latent row [c_kv | k_pe] written once into a per-sequence
// contiguous range of a single HBM pool; appends touch only the new rows.

#include <algorithm>
#include <cstring>
#include <new>
#include <vector>

#include "internal.hpp"

namespace qmla {

namespace {

// One block per appended row.  Rows come from `src` as [n_seqs, n_new, w]
// in f32 or in the cache dtype.
template <typename SrcT, typename DstT>
__global__ void k_cache_append(const SrcT *__restrict__ src, DstT *__restrict__ pool,
                               const int64_t *__restrict__ offsets,
                               const int32_t *__restrict__ lens, int32_t seq0, int32_t n_new,
                               int64_t w) {
  int64_t row = blockIdx.x;
  int32_t s = (int32_t)(row / n_new);
  int32_t j = (int32_t)(row % n_new);
  int64_t dst_row = offsets[seq0 + s] + (int64_t)lens[seq0 + s] + j;
  const SrcT *in = src + row * w;
  DstT *out = pool + dst_row * w;
  for (int64_t c = threadIdx.x; c < w; c += blockDim.x) {
    if constexpr (sizeof(SrcT) == sizeof(DstT)) {
      out[c] = in[c];
    } else {
      out[c] = f32_to_bf16_bits(in[c]);
    }
  }
}

__global__ void k_cache_advance(int32_t *__restrict__ lens, int32_t seq0, int32_t n_seqs,
                                int32_t n_new) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n_seqs) lens[seq0 + i] += n_new;
}

}  // namespace

qmla_status check_append(const qmla_kv_cache *c, int32_t seq0, int32_t n_seqs, int32_t n_new) {
  QMLA_REQUIRE(n_seqs >= 0 && n_new >= 0, QMLA_ERR_INVALID_ARG, "negative count");
  QMLA_REQUIRE(seq0 >= 0 && seq0 + (int64_t)n_seqs <= c->num_seqs, QMLA_ERR_SHAPE,
               "sequences [%d, %d) outside the cache's %d", seq0, seq0 + n_seqs, c->num_seqs);
  for (int32_t i = seq0; i < seq0 + n_seqs; ++i)
    QMLA_REQUIRE((int64_t)c->h_lens[i] + n_new <= c->h_cap[i], QMLA_ERR_CAPACITY,
                 "sequence %d: length %d + %d new rows exceeds capacity %d", i, c->h_lens[i],
                 n_new, c->h_cap[i]);
  return QMLA_OK;
}

// Re-lays the pool out with capacities new_cap (each >= the old one): the
// live rows [0, len) of every sequence move to its new offset.  On failure
// the cache is left as it was.
qmla_status regrow(qmla_kv_cache *c, const std::vector<int32_t> &new_cap, hipStream_t s) {
  const size_t rb = c->row_bytes();
  std::vector<int64_t> off(c->num_seqs);
  int64_t total = 0;
  for (int32_t i = 0; i < c->num_seqs; ++i) {
    off[i] = total;
    total += new_cap[i];
  }
  void *pool = nullptr;
  QMLA_REQUIRE(hipMalloc(&pool, total > 0 ? (size_t)total * rb : 256) == hipSuccess, QMLA_ERR_OOM,
               "cannot allocate a %lld-row pool", (long long)total);
  auto bail = [&](const char *what) {
    (void)hipStreamSynchronize(s);
    (void)hipFree(pool);
    return fail(QMLA_ERR_HIP, "%s failed while growing the cache", what);
  };
  char *dst = static_cast<char *>(pool);
  const char *src = static_cast<const char *>(c->rows);
  for (int32_t i = 0; i < c->num_seqs; ++i)
    if (c->h_lens[i] > 0 &&
        hipMemcpyAsync(dst + off[i] * rb, src + c->h_offsets[i] * rb, (size_t)c->h_lens[i] * rb,
                       hipMemcpyDeviceToDevice, s) != hipSuccess)
      return bail("row copy");
  if (hipMemcpyAsync(c->d_offsets, off.data(), sizeof(int64_t) * c->num_seqs,
                     hipMemcpyHostToDevice, s) != hipSuccess ||
      hipMemcpyAsync(c->d_cap, new_cap.data(), sizeof(int32_t) * c->num_seqs,
                     hipMemcpyHostToDevice, s) != hipSuccess)
    return bail("table upload");
  // the copies and uploads read host vectors and the old pool: finish them
  if (hipStreamSynchronize(s) != hipSuccess) return bail("stream synchronize");
  (void)hipFree(c->rows);
  c->rows = pool;
  c->h_offsets = off;
  c->h_cap = new_cap;
  c->total_rows = total;
  return QMLA_OK;
}

qmla_status make_room(qmla_kv_cache *c, int32_t seq0, int32_t n_seqs, int32_t n_new,
                      hipStream_t stream) {
  if (c->grow && n_new > 0 && seq0 >= 0 && n_seqs >= 0 && seq0 + (int64_t)n_seqs <= c->num_seqs) {
    std::vector<int32_t> cap = c->h_cap;
    bool more = false;
    for (int32_t i = seq0; i < seq0 + n_seqs; ++i) {
      const int64_t need = (int64_t)c->h_lens[i] + n_new;
      if (need <= cap[i]) continue;
      QMLA_REQUIRE(need <= 0x7fffffff, QMLA_ERR_CAPACITY, "sequence %d: %lld rows", i,
                   (long long)need);
      cap[i] = (int32_t)std::min<int64_t>(0x7fffffff,
                                          std::max<int64_t>({need, 2 * (int64_t)cap[i], 16}));
      more = true;
    }
    if (more) QMLA_TRY(regrow(c, cap, stream));
  }
  return check_append(c, seq0, n_seqs, n_new);
}

qmla_status launch_cache_append(qmla_kv_cache *c, const void *rows, qmla_dtype rows_dtype,
                                int32_t seq0, int32_t n_seqs, int32_t n_new, hipStream_t stream) {
  QMLA_TRY(make_room(c, seq0, n_seqs, n_new, stream));
  int64_t nrows = (int64_t)n_seqs * n_new;
  if (nrows == 0) return QMLA_OK;
  QMLA_REQUIRE(rows != nullptr, QMLA_ERR_INVALID_ARG, "rows is NULL");
  QMLA_REQUIRE(nrows <= 0x7fffffff, QMLA_ERR_SHAPE, "too many rows in one append");
  dim3 grid((unsigned)nrows), block(128);
  if (c->dtype == QMLA_F32) {
    QMLA_REQUIRE(rows_dtype == QMLA_F32, QMLA_ERR_UNSUPPORTED,
                 "an f32 cache takes f32 rows only");
    k_cache_append<float, float><<<grid, block, 0, stream>>>(
        (const float *)rows, (float *)c->rows, c->d_offsets, c->d_lens, seq0, n_new,
        c->row_elems);
  } else if (rows_dtype == QMLA_F32) {
    k_cache_append<float, uint16_t><<<grid, block, 0, stream>>>(
        (const float *)rows, (uint16_t *)c->rows, c->d_offsets, c->d_lens, seq0, n_new,
        c->row_elems);
  } else {
    k_cache_append<uint16_t, uint16_t><<<grid, block, 0, stream>>>(
        (const uint16_t *)rows, (uint16_t *)c->rows, c->d_offsets, c->d_lens, seq0, n_new,
        c->row_elems);
  }
  QMLA_LAUNCH_CHECK("k_cache_append");
  return cache_advance(c, seq0, n_seqs, n_new, stream);
}

qmla_status cache_advance(qmla_kv_cache *c, int32_t seq0, int32_t n_seqs, int32_t n_new,
                          hipStream_t stream) {
  k_cache_advance<<<dim3((n_seqs + 255) / 256), dim3(256), 0, stream>>>(c->d_lens, seq0, n_seqs,
                                                                        n_new);
  QMLA_LAUNCH_CHECK("k_cache_advance");
  for (int32_t i = seq0; i < seq0 + n_seqs; ++i) c->h_lens[i] += n_new;
  return QMLA_OK;
}

}  // namespace qmla

using namespace qmla;

namespace {

void destroy_cache(qmla_kv_cache *c) {
  if (!c) return;
  if (c->rows) (void)hipFree(c->rows);
  if (c->d_offsets) (void)hipFree(c->d_offsets);
  if (c->d_lens) (void)hipFree(c->d_lens);
  if (c->d_cap) (void)hipFree(c->d_cap);
  delete c;
}

// Allocates the pool and tables of `c` (whose host fields are set) and
// uploads offsets, capacities and lengths.
qmla_status materialise(qmla_kv_cache *c, hipStream_t stream) {
  size_t pool = (size_t)c->total_rows * c->row_bytes();
  QMLA_HIP(hipMalloc(&c->rows, pool > 0 ? pool : 256));
  QMLA_HIP(hipMalloc((void **)&c->d_offsets, sizeof(int64_t) * c->num_seqs));
  QMLA_HIP(hipMalloc((void **)&c->d_lens, sizeof(int32_t) * c->num_seqs));
  QMLA_HIP(hipMalloc((void **)&c->d_cap, sizeof(int32_t) * c->num_seqs));
  QMLA_HIP(hipMemcpyAsync(c->d_offsets, c->h_offsets.data(), sizeof(int64_t) * c->num_seqs,
                          hipMemcpyHostToDevice, stream));
  QMLA_HIP(hipMemcpyAsync(c->d_lens, c->h_lens.data(), sizeof(int32_t) * c->num_seqs,
                          hipMemcpyHostToDevice, stream));
  QMLA_HIP(hipMemcpyAsync(c->d_cap, c->h_cap.data(), sizeof(int32_t) * c->num_seqs,
                          hipMemcpyHostToDevice, stream));
  QMLA_HIP(hipStreamSynchronize(stream));
  return QMLA_OK;
}

}  // namespace

extern "C" {

qmla_status qmla_cache_create(int32_t num_seqs, const int32_t *capacity, int32_t kv_lora_rank,
                              int32_t rope_dim, qmla_dtype dtype, qmla_kv_cache **out) {
  QMLA_REQUIRE(out && capacity, QMLA_ERR_INVALID_ARG, "NULL pointer");
  *out = nullptr;
  QMLA_REQUIRE(num_seqs > 0, QMLA_ERR_SHAPE, "num_seqs must be > 0");
  QMLA_REQUIRE(kv_lora_rank > 0 && rope_dim >= 0, QMLA_ERR_SHAPE, "bad latent dims %d/%d",
               kv_lora_rank, rope_dim);
  QMLA_REQUIRE(valid_dtype(dtype), QMLA_ERR_INVALID_ARG, "bad dtype %d", (int)dtype);
  QMLA_REQUIRE((kv_lora_rank + rope_dim) % 8 == 0, QMLA_ERR_UNSUPPORTED,
               "row width %d must be a multiple of 8", kv_lora_rank + rope_dim);
  int device = 0;
  QMLA_HIP(hipGetDevice(&device));
  qmla_kv_cache *c = new (std::nothrow) qmla_kv_cache();
  QMLA_REQUIRE(c, QMLA_ERR_OOM, "host allocation failed");
  c->device = device;
  c->num_seqs = num_seqs;
  c->r = kv_lora_rank;
  c->dr = rope_dim;
  c->dtype = dtype;
  c->row_elems = kv_lora_rank + rope_dim;
  c->h_offsets.resize(num_seqs);
  c->h_lens.assign(num_seqs, 0);
  c->h_cap.resize(num_seqs);
  int64_t total = 0;
  for (int32_t i = 0; i < num_seqs; ++i) {
    if (capacity[i] < 0) {
      delete c;
      return fail(QMLA_ERR_SHAPE, "capacity[%d] = %d is negative", i, capacity[i]);
    }
    c->h_offsets[i] = total;
    c->h_cap[i] = capacity[i];
    total += capacity[i];
  }
  c->total_rows = total;
  qmla_status st = materialise(c, nullptr);
  if (st != QMLA_OK) {
    destroy_cache(c);
    return st;
  }
  *out = c;
  return QMLA_OK;
}

qmla_status qmla_cache_destroy(qmla_kv_cache *cache) {
  destroy_cache(cache);
  return QMLA_OK;
}

qmla_status qmla_cache_clone(const qmla_kv_cache *src, qmla_kv_cache **out, qmla_stream stream) {
  QMLA_REQUIRE(src && out, QMLA_ERR_INVALID_ARG, "NULL pointer");
  *out = nullptr;
  qmla_kv_cache *c = new (std::nothrow) qmla_kv_cache();
  QMLA_REQUIRE(c, QMLA_ERR_OOM, "host allocation failed");
  c->device = src->device;
  c->num_seqs = src->num_seqs;
  c->r = src->r;
  c->dr = src->dr;
  c->dtype = src->dtype;
  c->row_elems = src->row_elems;
  c->total_rows = src->total_rows;
  c->h_offsets = src->h_offsets;
  c->h_lens = src->h_lens;
  c->h_cap = src->h_cap;
  c->grow = src->grow;
  hipStream_t s = as_stream(stream);
  // Wait for pending work on src's stream before reading its rows.
  if (hipStreamSynchronize(s) != hipSuccess) {
    delete c;
    return fail(QMLA_ERR_HIP, "stream synchronize failed");
  }
  qmla_status st = materialise(c, s);
  if (st == QMLA_OK) {
    size_t pool = (size_t)c->total_rows * c->row_bytes();
    if (pool && hipMemcpyAsync(c->rows, src->rows, pool, hipMemcpyDeviceToDevice, s) != hipSuccess)
      st = fail(QMLA_ERR_HIP, "pool copy failed");
    if (st == QMLA_OK &&
        hipMemcpyAsync(c->d_lens, src->d_lens, sizeof(int32_t) * c->num_seqs,
                       hipMemcpyDeviceToDevice, s) != hipSuccess)
      st = fail(QMLA_ERR_HIP, "length copy failed");
  }
  if (st != QMLA_OK) {
    destroy_cache(c);
    return st;
  }
  *out = c;
  return QMLA_OK;
}

qmla_status qmla_cache_append(qmla_kv_cache *cache, const void *rows, qmla_dtype rows_dtype,
                              int32_t n_seqs, int32_t n_new, qmla_stream stream) {
  QMLA_REQUIRE(cache, QMLA_ERR_INVALID_ARG, "cache is NULL");
  QMLA_REQUIRE(valid_dtype(rows_dtype), QMLA_ERR_INVALID_ARG, "bad rows dtype");
  return launch_cache_append(cache, rows, rows_dtype, 0, n_seqs, n_new, as_stream(stream));
}

qmla_status qmla_cache_append_seq(qmla_kv_cache *cache, int32_t seq, const void *rows,
                                  qmla_dtype rows_dtype, int32_t n_new, qmla_stream stream) {
  QMLA_REQUIRE(cache, QMLA_ERR_INVALID_ARG, "cache is NULL");
  QMLA_REQUIRE(valid_dtype(rows_dtype), QMLA_ERR_INVALID_ARG, "bad rows dtype");
  return launch_cache_append(cache, rows, rows_dtype, seq, 1, n_new, as_stream(stream));
}

qmla_status qmla_cache_set_lengths(qmla_kv_cache *cache, const int32_t *lengths,
                                   qmla_stream stream) {
  QMLA_REQUIRE(cache && lengths, QMLA_ERR_INVALID_ARG, "NULL pointer");
  for (int32_t i = 0; i < cache->num_seqs; ++i)
    QMLA_REQUIRE(lengths[i] >= 0 && lengths[i] <= cache->h_cap[i], QMLA_ERR_CAPACITY,
                 "length[%d] = %d outside [0, %d]", i, lengths[i], cache->h_cap[i]);
  std::memcpy(cache->h_lens.data(), lengths, sizeof(int32_t) * cache->num_seqs);
  // The host mirror is the source; copy synchronously so the caller may
  // reuse `lengths` at once.
  QMLA_HIP(hipMemcpyAsync(cache->d_lens, cache->h_lens.data(), sizeof(int32_t) * cache->num_seqs,
                          hipMemcpyHostToDevice, as_stream(stream)));
  QMLA_HIP(hipStreamSynchronize(as_stream(stream)));
  return QMLA_OK;
}

qmla_status qmla_cache_lengths(const qmla_kv_cache *cache, int32_t *lengths_out) {
  QMLA_REQUIRE(cache && lengths_out, QMLA_ERR_INVALID_ARG, "NULL pointer");
  std::memcpy(lengths_out, cache->h_lens.data(), sizeof(int32_t) * cache->num_seqs);
  return QMLA_OK;
}

qmla_status qmla_cache_reserve(qmla_kv_cache *cache, const int32_t *min_capacity,
                               qmla_stream stream) {
  QMLA_REQUIRE(cache && min_capacity, QMLA_ERR_INVALID_ARG, "NULL pointer");
  std::vector<int32_t> cap = cache->h_cap;
  bool more = false;
  for (int32_t i = 0; i < cache->num_seqs; ++i) {
    QMLA_REQUIRE(min_capacity[i] >= 0, QMLA_ERR_SHAPE, "min_capacity[%d] = %d is negative", i,
                 min_capacity[i]);
    if (min_capacity[i] > cap[i]) {
      cap[i] = min_capacity[i];
      more = true;
    }
  }
  return more ? regrow(cache, cap, as_stream(stream)) : QMLA_OK;
}

qmla_status qmla_cache_set_growth(qmla_kv_cache *cache, int32_t enable) {
  QMLA_REQUIRE(cache, QMLA_ERR_INVALID_ARG, "cache is NULL");
  cache->grow = enable != 0;
  return QMLA_OK;
}

qmla_status qmla_cache_capacity(const qmla_kv_cache *cache, int32_t *capacity_out) {
  QMLA_REQUIRE(cache && capacity_out, QMLA_ERR_INVALID_ARG, "NULL pointer");
  std::memcpy(capacity_out, cache->h_cap.data(), sizeof(int32_t) * cache->num_seqs);
  return QMLA_OK;
}

qmla_status qmla_cache_describe(const qmla_kv_cache *cache, qmla_cache_desc *out) {
  QMLA_REQUIRE(cache && out, QMLA_ERR_INVALID_ARG, "NULL pointer");
  out->num_seqs = cache->num_seqs;
  out->kv_lora_rank = cache->r;
  out->rope_dim = cache->dr;
  out->dtype = cache->dtype;
  out->row_elems = cache->row_elems;
  out->total_rows = cache->total_rows;
  out->rows = cache->rows;
  out->offsets = cache->d_offsets;
  out->lengths = cache->d_lens;
  out->capacity = cache->d_cap;
  return QMLA_OK;
}

}  // extern "C"
