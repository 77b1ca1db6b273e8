// cache.hip -- the latent KV cache (replacement of KVCache,
// src/model.rs:86-105).
//
// The reference grows per-head decompressed k/v/k_rope tensors with
// Tensor::cat on every token (an O(T) copy per token per layer).  Here each
// token is one latent row [c_kv | k_pe] written once into a page of its
// sequence; a sequence's pages are listed in a device block table.  Growing
// a sequence takes pages from a free list and writes their addresses into
// the table with one small kernel on the caller's stream: no live row is
// copied, nothing is re-laid out and the host never waits for the device.
// Pages come from HBM chunks allocated at creation (pool_rows), by
// qmla_cache_reserve / qmla_cache_reserve_pool, or -- only when the free
// list runs dry during an append in growth mode -- by a new chunk of half
// the pool again, at most 1 GiB (or the missing pages, if more).

#include <algorithm>
#include <cstring>
#include <new>
#include <vector>

#include "internal.hpp"

namespace qmla {

namespace {

constexpr int32_t kDefaultPageRows = 256;
constexpr int64_t kDefaultMaxLen = 163840;  // DeepSeek-V2's max_position_embeddings

// Block-table and capacity updates, passed by value so that the host arrays
// they come from can be reused at once (no copy from host memory is left in
// flight, no synchronisation).
constexpr int kWriteBatch = 64;
struct TableWrites {
  int32_t n_pages, n_caps;
  int32_t slot[kWriteBatch];  // index into the table
  int32_t seq[kWriteBatch];
  int32_t cap[kWriteBatch];
  uint64_t page[kWriteBatch];
};

__global__ __launch_bounds__(kWriteBatch) void k_table_write(TableWrites w,
                                                             uint64_t *__restrict__ pages,
                                                             int32_t *__restrict__ cap) {
  const int i = threadIdx.x;
  if (i < w.n_pages) pages[w.slot[i]] = w.page[i];
  if (i < w.n_caps) cap[w.seq[i]] = w.cap[i];
}

constexpr int kLenBatch = 256;
struct LenWrites {
  int32_t seq0, n;
  int32_t len[kLenBatch];
};

__global__ __launch_bounds__(kLenBatch) void k_set_lens(LenWrites w, int32_t *__restrict__ lens) {
  const int i = threadIdx.x;
  if (i < w.n) lens[w.seq0 + i] = w.len[i];
}

class TableWriter {
 public:
  TableWriter(qmla_kv_cache *c, hipStream_t s) : c_(c), s_(s) { w_.n_pages = w_.n_caps = 0; }
  qmla_status page(int64_t slot, uint64_t addr) {
    if (w_.n_pages == kWriteBatch) QMLA_TRY(flush());
    w_.slot[w_.n_pages] = (int32_t)slot;
    w_.page[w_.n_pages++] = addr;
    return QMLA_OK;
  }
  qmla_status cap(int32_t seq, int32_t v) {
    if (w_.n_caps == kWriteBatch) QMLA_TRY(flush());
    w_.seq[w_.n_caps] = seq;
    w_.cap[w_.n_caps++] = v;
    return QMLA_OK;
  }
  qmla_status flush() {
    if (w_.n_pages == 0 && w_.n_caps == 0) return QMLA_OK;
    k_table_write<<<dim3(1), dim3(kWriteBatch), 0, s_>>>(w_, c_->d_pages, c_->d_cap);
    QMLA_LAUNCH_CHECK("k_table_write");
    w_.n_pages = w_.n_caps = 0;
    return QMLA_OK;
  }

 private:
  qmla_kv_cache *c_;
  hipStream_t s_;
  TableWrites w_;
};

// One block per appended row.  Rows come from `src` as [n_seqs, n_new, w]
// in f32 or in the cache dtype.
template <typename SrcT, typename DstT>
__global__ void k_cache_append(const SrcT *__restrict__ src, PageTable tab,
                               const int32_t *__restrict__ lens, int32_t seq0, int32_t n_new,
                               int64_t w) {
  int64_t row = blockIdx.x;
  int32_t s = (int32_t)(row / n_new);
  int32_t j = (int32_t)(row % n_new);
  const SrcT *in = src + row * w;
  DstT *out = reinterpret_cast<DstT *>(
      tab.row(seq0 + s, (int64_t)lens[seq0 + s] + j, w * (int64_t)sizeof(DstT)));
  for (int64_t c = threadIdx.x; c < w; c += blockDim.x) {
    if constexpr (sizeof(SrcT) == sizeof(DstT)) {
      out[c] = in[c];
    } else {
      out[c] = f32_to_bf16_bits(in[c]);
    }
  }
}

// Rows [t0, t0 + n) of one sequence into a dense buffer, 16 B per lane.
__global__ __launch_bounds__(64) void k_cache_gather(PageTable tab, int32_t seq, int64_t t0,
                                                     int64_t row_bytes, uint8_t *__restrict__ out) {
  const int64_t t = blockIdx.x;
  const uint4 *src = reinterpret_cast<const uint4 *>(tab.row(seq, t0 + t, row_bytes));
  uint4 *dst = reinterpret_cast<uint4 *>(out + t * row_bytes);
  for (int64_t c = threadIdx.x; c < row_bytes / 16; c += blockDim.x) dst[c] = src[c];
}

__global__ void k_cache_advance(int32_t *__restrict__ lens, int32_t seq0, int32_t n_seqs,
                                int32_t n_new) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n_seqs) lens[seq0 + i] += n_new;
}

int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Adds a chunk of `pages` pages to the pool; its pages go onto the free
// list so that they are handed out in address order.
qmla_status add_chunk(qmla_kv_cache *c, int64_t pages) {
  if (pages <= 0) return QMLA_OK;
  void *p = nullptr;
  QMLA_REQUIRE(hipMalloc(&p, (size_t)pages * c->page_bytes()) == hipSuccess, QMLA_ERR_OOM,
               "cannot allocate %lld cache pages of %zu bytes", (long long)pages, c->page_bytes());
  c->chunks.push_back(p);
  c->pool_pages += pages;
  const uint64_t base = reinterpret_cast<uint64_t>(p);
  for (int64_t i = pages - 1; i >= 0; --i) c->free_pages.push_back(base + i * c->page_bytes());
  return QMLA_OK;
}

// Raises the capacity of sequences seq0 .. seq0 + n - 1 to at least want[i]
// rows: missing pages come from the free list (a new chunk when it is
// short) and their addresses reach the device table through k_table_write
// on `s`.  exact: the capacity becomes max(capacity, want[i]); otherwise it
// becomes every row of the pages the sequence holds.  Every check is made
// before anything changes.
qmla_status ensure_capacity(qmla_kv_cache *c, int32_t seq0, const std::vector<int64_t> &want,
                            bool exact, hipStream_t s) {
  const int32_t n = (int32_t)want.size();
  const int64_t P = c->page_rows, max_rows = (int64_t)c->table_width * P;
  int64_t extra = 0;
  for (int32_t i = 0; i < n; ++i) {
    const int32_t q = seq0 + i;
    if (want[i] <= c->h_cap[q]) continue;
    QMLA_REQUIRE(want[i] <= max_rows && want[i] <= 0x7fffffff, QMLA_ERR_CAPACITY,
                 "sequence %d: %lld rows exceed the cache's maximum length %lld", q,
                 (long long)want[i], (long long)std::min<int64_t>(max_rows, 0x7fffffff));
    extra += std::max<int64_t>(0, ceil_div(want[i], P) - c->h_npages[q]);
  }
  if (extra > (int64_t)c->free_pages.size()) {
    // the missing pages, or half the pool again up to 1 GiB, whichever is more
    const int64_t cap_pages = std::max<int64_t>(1, ((int64_t)1 << 30) / (int64_t)c->page_bytes());
    const int64_t grow = std::max<int64_t>(1, std::min(c->pool_pages / 2, cap_pages));
    QMLA_TRY(add_chunk(c, std::max(extra - (int64_t)c->free_pages.size(), grow)));
  }
  // Stage the new pages and capacities, launch every table write, and only
  // then commit them to the host mirror and the free list: a failed launch
  // leaves the host state as it was (the pages it staged stay free).
  struct Grant {
    int32_t seq, npages, cap;
  };
  std::vector<Grant> grants;
  std::vector<std::pair<int64_t, uint64_t>> pages;  // (table slot, page address)
  size_t taken = 0;
  for (int32_t i = 0; i < n; ++i) {
    const int32_t q = seq0 + i;
    if (want[i] <= c->h_cap[q]) continue;
    const int32_t need = (int32_t)ceil_div(want[i], P);
    for (int32_t j = c->h_npages[q]; j < need; ++j)
      pages.emplace_back((int64_t)q * c->table_width + j,
                         c->free_pages[c->free_pages.size() - 1 - taken++]);
    const int32_t npages = std::max(c->h_npages[q], need);
    grants.push_back({q, npages,
                      exact ? (int32_t)want[i]
                            : (int32_t)std::min<int64_t>((int64_t)npages * P, 0x7fffffff)});
  }
  TableWriter tw(c, s);
  for (const auto &p : pages) QMLA_TRY(tw.page(p.first, p.second));
  for (const Grant &g : grants) QMLA_TRY(tw.cap(g.seq, g.cap));
  QMLA_TRY(tw.flush());
  for (const auto &p : pages) c->h_pages[p.first] = p.second;
  c->free_pages.resize(c->free_pages.size() - taken);
  if (taken > 0) c->contiguous = false;
  for (const Grant &g : grants) {
    c->h_npages[g.seq] = g.npages;
    c->h_cap[g.seq] = g.cap;
  }
  return QMLA_OK;
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

qmla_status make_room(qmla_kv_cache *c, int32_t seq0, int32_t n_seqs, int32_t n_new,
                      hipStream_t stream) {
  if (c->grow && n_new > 0 && seq0 >= 0 && n_seqs >= 0 && seq0 + (int64_t)n_seqs <= c->num_seqs) {
    std::vector<int64_t> want(n_seqs);
    for (int32_t i = 0; i < n_seqs; ++i) want[i] = (int64_t)c->h_lens[seq0 + i] + n_new;
    QMLA_TRY(ensure_capacity(c, seq0, want, false, stream));
  }
  return check_append(c, seq0, n_seqs, n_new);
}

qmla_status launch_cache_append(qmla_kv_cache *c, const void *rows, qmla_dtype rows_dtype,
                                int32_t seq0, int32_t n_seqs, int32_t n_new, hipStream_t stream) {
  QMLA_REQUIRE(c->dtype == QMLA_BF16 || rows_dtype == QMLA_F32, QMLA_ERR_UNSUPPORTED,
               "an f32 cache takes f32 rows only");
  int64_t nrows = (int64_t)n_seqs * n_new;
  QMLA_REQUIRE(nrows == 0 || rows != nullptr, QMLA_ERR_INVALID_ARG, "rows is NULL");
  QMLA_REQUIRE(nrows <= 0x7fffffff, QMLA_ERR_SHAPE, "too many rows in one append");
  QMLA_TRY(make_room(c, seq0, n_seqs, n_new, stream));
  if (nrows == 0) return QMLA_OK;
  dim3 grid((unsigned)nrows), block(128);
  const PageTable tab = c->table();
  if (c->dtype == QMLA_F32) {
    k_cache_append<float, float><<<grid, block, 0, stream>>>(
        (const float *)rows, tab, c->d_lens, seq0, n_new, c->row_elems);
  } else if (rows_dtype == QMLA_F32) {
    k_cache_append<float, uint16_t><<<grid, block, 0, stream>>>(
        (const float *)rows, tab, c->d_lens, seq0, n_new, c->row_elems);
  } else {
    k_cache_append<uint16_t, uint16_t><<<grid, block, 0, stream>>>(
        (const uint16_t *)rows, tab, c->d_lens, seq0, n_new, c->row_elems);
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
  for (void *p : c->chunks) (void)hipFree(p);
  if (c->d_pages) (void)hipFree(c->d_pages);
  if (c->d_offsets) (void)hipFree(c->d_offsets);
  if (c->d_lens) (void)hipFree(c->d_lens);
  if (c->d_cap) (void)hipFree(c->d_cap);
  delete c;
}

// Host-side layout of a new cache: sequence i takes ceil(cap_i / P) pages
// of chunk 0 in order (row offset h_offsets[i]), the rest of chunk 0's
// `pool_pages` pages start free.
qmla_status plan_layout(qmla_kv_cache *c, const int32_t *cap, int64_t max_len, int64_t pool_rows,
                        int32_t page_rows) {
  if (page_rows == 0) page_rows = kDefaultPageRows;
  QMLA_REQUIRE(page_rows >= 32 && page_rows <= 65536 && (page_rows & (page_rows - 1)) == 0,
               QMLA_ERR_SHAPE, "page_rows %d must be a power of two in [32, 65536]", page_rows);
  QMLA_REQUIRE(max_len >= 0 && pool_rows >= 0, QMLA_ERR_SHAPE, "negative max_len or pool_rows");
  c->page_rows = page_rows;
  c->page_shift = __builtin_ctz((unsigned)page_rows);
  const int64_t P = page_rows;
  c->h_offsets.resize(c->num_seqs);
  c->h_lens.assign(c->num_seqs, 0);
  c->h_cap.resize(c->num_seqs);
  c->h_npages.resize(c->num_seqs);
  int64_t used = 0, longest = 0;
  for (int32_t i = 0; i < c->num_seqs; ++i) {
    QMLA_REQUIRE(cap[i] >= 0, QMLA_ERR_SHAPE, "capacity[%d] = %d is negative", i, cap[i]);
    c->h_offsets[i] = used * P;
    c->h_cap[i] = cap[i];
    c->h_npages[i] = (int32_t)ceil_div(cap[i], P);
    used += c->h_npages[i];
    longest = std::max<int64_t>(longest, cap[i]);
  }
  const int64_t width = ceil_div(std::max(longest, max_len > 0 ? max_len : kDefaultMaxLen), P);
  QMLA_REQUIRE((int64_t)c->num_seqs * width < 0x7fffffff, QMLA_ERR_SHAPE,
               "block table of %d sequences x %lld pages is too large", c->num_seqs,
               (long long)width);
  c->table_width = (int32_t)std::max<int64_t>(width, 1);
  c->pool_pages = std::max(used, ceil_div(pool_rows, P));
  c->total_rows = c->pool_pages * P;
  return QMLA_OK;
}

// Allocates chunk 0 and the device tables of `c` (host layout set), fills
// the block table and uploads it with the offsets, capacities and lengths.
qmla_status materialise(qmla_kv_cache *c, hipStream_t stream) {
  const int64_t P = c->page_rows;
  void *chunk = nullptr;
  const size_t pool = (size_t)c->pool_pages * c->page_bytes();
  QMLA_REQUIRE(hipMalloc(&chunk, pool > 0 ? pool : 256) == hipSuccess, QMLA_ERR_OOM,
               "cannot allocate a %lld-row cache pool", (long long)c->total_rows);
  c->chunks.push_back(chunk);
  const uint64_t base = reinterpret_cast<uint64_t>(chunk);
  const size_t rb = c->row_bytes();
  c->h_pages.assign((size_t)c->num_seqs * c->table_width, 0);
  int64_t used = 0;
  for (int32_t i = 0; i < c->num_seqs; ++i) {
    for (int32_t j = 0; j < c->h_npages[i]; ++j)
      c->h_pages[(size_t)i * c->table_width + j] = base + (c->h_offsets[i] + j * P) * rb;
    used += c->h_npages[i];
  }
  for (int64_t p = c->pool_pages - 1; p >= used; --p)
    c->free_pages.push_back(base + p * c->page_bytes());
  QMLA_HIP(hipMalloc((void **)&c->d_pages, sizeof(uint64_t) * c->h_pages.size()));
  QMLA_HIP(hipMalloc((void **)&c->d_offsets, sizeof(int64_t) * c->num_seqs));
  QMLA_HIP(hipMalloc((void **)&c->d_lens, sizeof(int32_t) * c->num_seqs));
  QMLA_HIP(hipMalloc((void **)&c->d_cap, sizeof(int32_t) * c->num_seqs));
  QMLA_HIP(hipMemcpyAsync(c->d_pages, c->h_pages.data(), sizeof(uint64_t) * c->h_pages.size(),
                          hipMemcpyHostToDevice, stream));
  QMLA_HIP(hipMemcpyAsync(c->d_offsets, c->h_offsets.data(), sizeof(int64_t) * c->num_seqs,
                          hipMemcpyHostToDevice, stream));
  QMLA_HIP(hipMemcpyAsync(c->d_lens, c->h_lens.data(), sizeof(int32_t) * c->num_seqs,
                          hipMemcpyHostToDevice, stream));
  QMLA_HIP(hipMemcpyAsync(c->d_cap, c->h_cap.data(), sizeof(int32_t) * c->num_seqs,
                          hipMemcpyHostToDevice, stream));
  QMLA_HIP(hipStreamSynchronize(stream));
  return QMLA_OK;
}

qmla_status new_cache(int32_t num_seqs, int32_t kv_lora_rank, int32_t rope_dim, qmla_dtype dtype,
                      qmla_kv_cache **out) {
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
  *out = c;
  return QMLA_OK;
}

}  // namespace

extern "C" {

qmla_status qmla_cache_create_paged(int32_t num_seqs, const int32_t *capacity, int64_t max_len,
                                    int64_t pool_rows, int32_t page_rows, int32_t kv_lora_rank,
                                    int32_t rope_dim, qmla_dtype dtype, qmla_kv_cache **out) {
  QMLA_REQUIRE(out && capacity, QMLA_ERR_INVALID_ARG, "NULL pointer");
  *out = nullptr;
  qmla_kv_cache *c = nullptr;
  QMLA_TRY(new_cache(num_seqs, kv_lora_rank, rope_dim, dtype, &c));
  qmla_status st = plan_layout(c, capacity, max_len, pool_rows, page_rows);
  if (st == QMLA_OK) st = materialise(c, nullptr);
  if (st != QMLA_OK) {
    destroy_cache(c);
    return st;
  }
  *out = c;
  return QMLA_OK;
}

qmla_status qmla_cache_create(int32_t num_seqs, const int32_t *capacity, int32_t kv_lora_rank,
                              int32_t rope_dim, qmla_dtype dtype, qmla_kv_cache **out) {
  return qmla_cache_create_paged(num_seqs, capacity, 0, 0, 0, kv_lora_rank, rope_dim, dtype, out);
}

qmla_status qmla_cache_destroy(qmla_kv_cache *cache) {
  destroy_cache(cache);
  return QMLA_OK;
}

qmla_status qmla_cache_clone(const qmla_kv_cache *src, qmla_kv_cache **out, qmla_stream stream) {
  QMLA_REQUIRE(src && out, QMLA_ERR_INVALID_ARG, "NULL pointer");
  *out = nullptr;
  qmla_kv_cache *c = nullptr;
  QMLA_TRY(new_cache(src->num_seqs, src->r, src->dr, src->dtype, &c));
  hipStream_t s = as_stream(stream);
  // The clone holds src's pages per sequence (capacities kept), packed in
  // order into one chunk; only live rows are copied.
  c->page_rows = src->page_rows;
  c->page_shift = src->page_shift;
  c->table_width = src->table_width;
  c->grow = src->grow;
  c->h_lens = src->h_lens;
  c->h_cap = src->h_cap;
  c->h_npages = src->h_npages;
  c->h_offsets.resize(c->num_seqs);
  int64_t used = 0;
  for (int32_t i = 0; i < c->num_seqs; ++i) {
    c->h_offsets[i] = used * c->page_rows;
    used += c->h_npages[i];
  }
  c->pool_pages = used;
  c->total_rows = used * c->page_rows;
  // Wait for pending work on src's stream before reading its rows.
  qmla_status st = hipStreamSynchronize(s) == hipSuccess
                       ? QMLA_OK
                       : fail(QMLA_ERR_HIP, "stream synchronize failed");
  if (st == QMLA_OK) st = materialise(c, s);
  const size_t pb = c->page_bytes(), rb = c->row_bytes();
  for (int32_t i = 0; st == QMLA_OK && i < c->num_seqs; ++i) {
    const int32_t live = (int32_t)ceil_div(c->h_lens[i], c->page_rows);
    const uint64_t *sp = src->h_pages.data() + (size_t)i * src->table_width;
    const uint64_t *dp = c->h_pages.data() + (size_t)i * c->table_width;
    // runs of pages consecutive in both pools go as one copy
    for (int32_t j = 0; st == QMLA_OK && j < live;) {
      int32_t k = j + 1;
      while (k < live && sp[k] == sp[k - 1] + pb && dp[k] == dp[k - 1] + pb) ++k;
      const int64_t rows = std::min<int64_t>((int64_t)k * c->page_rows, c->h_lens[i]) -
                           (int64_t)j * c->page_rows;
      if (hipMemcpyAsync(reinterpret_cast<void *>(dp[j]), reinterpret_cast<const void *>(sp[j]),
                         (size_t)rows * rb, hipMemcpyDeviceToDevice, s) != hipSuccess)
        st = fail(QMLA_ERR_HIP, "row copy failed");
      j = k;
    }
  }
  if (st == QMLA_OK && hipStreamSynchronize(s) != hipSuccess)
    st = fail(QMLA_ERR_HIP, "stream synchronize failed");
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
  // The lengths travel as kernel arguments: `lengths` may be reused at once
  // and the host does not wait.
  for (int32_t s0 = 0; s0 < cache->num_seqs; s0 += kLenBatch) {
    LenWrites w;
    w.seq0 = s0;
    w.n = std::min(kLenBatch, cache->num_seqs - s0);
    std::memcpy(w.len, lengths + s0, sizeof(int32_t) * w.n);
    k_set_lens<<<dim3(1), dim3(kLenBatch), 0, as_stream(stream)>>>(w, cache->d_lens);
    QMLA_LAUNCH_CHECK("k_set_lens");
  }
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
  std::vector<int64_t> want(cache->num_seqs);
  for (int32_t i = 0; i < cache->num_seqs; ++i) {
    QMLA_REQUIRE(min_capacity[i] >= 0, QMLA_ERR_SHAPE, "min_capacity[%d] = %d is negative", i,
                 min_capacity[i]);
    want[i] = min_capacity[i];
  }
  return ensure_capacity(cache, 0, want, true, as_stream(stream));
}

qmla_status qmla_cache_reserve_pool(qmla_kv_cache *cache, int64_t free_rows) {
  QMLA_REQUIRE(cache, QMLA_ERR_INVALID_ARG, "cache is NULL");
  QMLA_REQUIRE(free_rows >= 0, QMLA_ERR_SHAPE, "free_rows %lld is negative", (long long)free_rows);
  const int64_t need = ceil_div(free_rows, cache->page_rows) - (int64_t)cache->free_pages.size();
  return add_chunk(cache, need);
}

qmla_status qmla_cache_trim(qmla_kv_cache *cache, int32_t seq0, int32_t n_seqs,
                            qmla_stream stream) {
  QMLA_REQUIRE(cache, QMLA_ERR_INVALID_ARG, "cache is NULL");
  QMLA_REQUIRE(n_seqs >= 0 && seq0 >= 0 && seq0 + (int64_t)n_seqs <= cache->num_seqs,
               QMLA_ERR_SHAPE, "sequences [%d, %d) outside the cache's %d", seq0, seq0 + n_seqs,
               cache->num_seqs);
  const int32_t P = cache->page_rows;
  TableWriter tw(cache, as_stream(stream));
  for (int32_t q = seq0; q < seq0 + n_seqs; ++q) {
    const int32_t keep = (int32_t)ceil_div(cache->h_lens[q], P);
    if (keep >= cache->h_npages[q]) continue;
    for (int32_t j = cache->h_npages[q] - 1; j >= keep; --j)
      cache->free_pages.push_back(cache->h_pages[(size_t)q * cache->table_width + j]);
    cache->h_npages[q] = keep;
    cache->h_cap[q] = std::min(cache->h_cap[q], keep * P);
    QMLA_TRY(tw.cap(q, cache->h_cap[q]));
  }
  return tw.flush();
}

qmla_status qmla_cache_pool_info(const qmla_kv_cache *cache, int64_t *pool_rows,
                                 int64_t *free_rows) {
  QMLA_REQUIRE(cache, QMLA_ERR_INVALID_ARG, "cache is NULL");
  if (pool_rows) *pool_rows = cache->pool_pages * cache->page_rows;
  if (free_rows) *free_rows = (int64_t)cache->free_pages.size() * cache->page_rows;
  return QMLA_OK;
}

qmla_status qmla_cache_gather(const qmla_kv_cache *cache, int32_t seq, int32_t t0, int32_t n,
                              void *out, qmla_stream stream) {
  QMLA_REQUIRE(cache, QMLA_ERR_INVALID_ARG, "cache is NULL");
  QMLA_REQUIRE(seq >= 0 && seq < cache->num_seqs, QMLA_ERR_SHAPE, "sequence %d outside [0, %d)",
               seq, cache->num_seqs);
  QMLA_REQUIRE(t0 >= 0 && n >= 0 && (int64_t)t0 + n <= cache->h_cap[seq], QMLA_ERR_SHAPE,
               "rows [%d, %lld) outside sequence %d's capacity %d", t0, (long long)t0 + n, seq,
               cache->h_cap[seq]);
  if (n == 0) return QMLA_OK;
  QMLA_REQUIRE(out, QMLA_ERR_INVALID_ARG, "out is NULL");
  k_cache_gather<<<dim3(n), dim3(64), 0, as_stream(stream)>>>(
      cache->table(), seq, t0, (int64_t)cache->row_bytes(), static_cast<uint8_t *>(out));
  QMLA_LAUNCH_CHECK("k_cache_gather");
  return QMLA_OK;
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
  out->total_rows = cache->contiguous ? cache->total_rows : 0;
  out->rows = cache->contiguous ? cache->chunks[0] : nullptr;
  out->offsets = cache->contiguous ? cache->d_offsets : nullptr;
  out->lengths = cache->d_lens;
  out->capacity = cache->d_cap;
  out->pages = cache->d_pages;
  out->page_rows = cache->page_rows;
  out->table_width = cache->table_width;
  out->contiguous = cache->contiguous ? 1 : 0;
  out->reserved = 0;
  return QMLA_OK;
}

}  // extern "C"
