// decode.hip -- absorbed-latent MLA decode: work plan, f32 core, merge and
// the C entry points.
//
// Replaces the attention core of MlaAttention::forward_with_cache
// (src/model.rs:294-303: scores over the decompressed per-head cache,
// softmax, times V) by the absorbed form over the shared latent cache:
//   s_t = scale * (q_lat . c_t + q_rope . kpe_t),  o_lat = sum_t p_t c_t
// (the W_UK absorption into q_lat and the W_UV product on o_lat happen in
// the layer; see layer.hip).
//
// Work split: the tokens of all sequences, concatenated, are cut into
// `blocks` equal pieces (one or a few per compute unit); every (piece,
// sequence) overlap is a segment.  A sequence covered by one segment is
// written straight to the output; otherwise each segment writes a partial
// (o / l, log-sum-exp) slot and k_decode_merge combines them.

#include <algorithm>
#include <atomic>
#include <cmath>
#include <mutex>

#include "internal.hpp"

namespace qmla {

namespace {

constexpr int kPlanThreads = 1024;

// Exclusive scan of n ints held in LDS (in place); returns the total.
// Every thread of the block must call it.
__device__ int32_t block_exclusive_scan(int32_t *a, int32_t n, int32_t *tmp) {
  const int tid = threadIdx.x;
  const int per = (n + kPlanThreads - 1) / kPlanThreads;
  const int lo = min(n, tid * per), hi = min(n, lo + per);
  int32_t local = 0;
  for (int i = lo; i < hi; ++i) local += a[i];
  tmp[tid] = local;
  __syncthreads();
  // Hillis-Steele over the kPlanThreads partial sums.
  for (int off = 1; off < kPlanThreads; off <<= 1) {
    int32_t v = tid >= off ? tmp[tid - off] : 0;
    __syncthreads();
    tmp[tid] += v;
    __syncthreads();
  }
  int32_t run = tid > 0 ? tmp[tid - 1] : 0;
  const int32_t total = tmp[kPlanThreads - 1];
  for (int i = lo; i < hi; ++i) {
    int32_t v = a[i];
    a[i] = run;
    run += v;
  }
  __syncthreads();
  return total;
}

// One block builds the segment list.  LDS: P[batch] prefix, S[batch] slot
// base, C[blocks] segment counts, tmp[kPlanThreads].
__global__ __launch_bounds__(kPlanThreads) void k_decode_plan(const int32_t *__restrict__ lens,
                                                              int32_t pending, int32_t batch,
                                                              int32_t blocks, int32_t chunk,
                                                              DecodePlanView plan) {
  extern __shared__ int32_t sm[];
  int32_t *P = sm;               // [batch + 1]
  int32_t *S = P + batch + 1;    // [batch]
  int32_t *C = S + batch;        // [blocks + 1]
  int32_t *tmp = C + blocks + 1; // [kPlanThreads]
  const int tid = threadIdx.x;

  for (int b = tid; b < batch; b += kPlanThreads) P[b] = lens[b] + pending;
  __syncthreads();
  const int32_t N = block_exclusive_scan(P, batch, tmp);
  if (tid == 0) P[batch] = N;
  __syncthreads();

  // slots per sequence
  for (int b = tid; b < batch; b += kPlanThreads) {
    int32_t T = P[b + 1] - P[b];
    int32_t n = 0;
    if (T > 0) {
      int32_t first = min(P[b] / chunk, blocks - 1);
      int32_t last = min((P[b] + T - 1) / chunk, blocks - 1);
      n = last - first + 1;
    }
    S[b] = n;
    plan.seq_nslots[b] = n;
  }
  __syncthreads();
  (void)block_exclusive_scan(S, batch, tmp);
  for (int b = tid; b < batch; b += kPlanThreads) plan.seq_slot_base[b] = S[b];

  // segments per piece: sequences overlapping [start, end)
  for (int i = tid; i < blocks; i += kPlanThreads) {
    int32_t start = min(i * chunk, N);
    int32_t end = (i == blocks - 1) ? N : min((i + 1) * chunk, N);
    int32_t cnt = 0;
    if (start < end) {
      // first sequence whose end P[b+1] > start
      int32_t lo = 0, hi = batch - 1;
      while (lo < hi) {
        int32_t mid = (lo + hi) >> 1;
        if (P[mid + 1] > start) hi = mid; else lo = mid + 1;
      }
      for (int32_t b = lo; b < batch && P[b] < end; ++b)
        if (P[b + 1] > P[b]) ++cnt;
    }
    C[i] = cnt;
  }
  __syncthreads();
  const int32_t total_segs = block_exclusive_scan(C, blocks, tmp);
  for (int i = tid; i < blocks; i += kPlanThreads) plan.seg_start[i] = C[i];
  if (tid == 0) plan.seg_start[blocks] = total_segs;

  for (int i = tid; i < blocks; i += kPlanThreads) {
    int32_t start = min(i * chunk, N);
    int32_t end = (i == blocks - 1) ? N : min((i + 1) * chunk, N);
    if (start >= end) continue;
    int32_t lo = 0, hi = batch - 1;
    while (lo < hi) {
      int32_t mid = (lo + hi) >> 1;
      if (P[mid + 1] > start) hi = mid; else lo = mid + 1;
    }
    int32_t out = C[i];
    for (int32_t b = lo; b < batch && P[b] < end; ++b) {
      int32_t T = P[b + 1] - P[b];
      if (T <= 0) continue;
      int32_t first = min(P[b] / chunk, blocks - 1);
      int32_t nsl = plan.seq_nslots[b];
      DecodeSegment sg;
      sg.seq = b;
      sg.t0 = max(start, P[b]) - P[b];
      sg.t1 = min(end, P[b + 1]) - P[b];
      sg.slot = nsl == 1 ? -1 : S[b] + (i - first);
      plan.segs[out++] = sg;
    }
  }
}

// ---------------------------------------------------------------- f32 core
// One block per (piece, query row).  Per 64-token chunk: 4 threads per
// token form the 576-wide dot product, the chunk's scores update an online
// softmax, and each thread accumulates up to kColsPerThread latent columns.
constexpr int kF32Threads = 256;
constexpr int kF32Tok = 64;
constexpr int kColsPerThread = 4;  // r <= 1024

template <typename QT>
__device__ inline float load_q(const QT *p, int64_t i) {
  if constexpr (sizeof(QT) == 4) return p[i];
  else return bf16_bits_to_f32(p[i]);
}

template <typename QT>
__global__ __launch_bounds__(kF32Threads) void k_decode_f32(
    PageTable tab, const QT *__restrict__ q_lat, const QT *__restrict__ q_rope, int32_t rows, int32_t r,
    int32_t dr, float scale, DecodePlanView plan, float *__restrict__ out,
    float *__restrict__ out_lse, float *__restrict__ part_o, float *__restrict__ part_lse) {
  extern __shared__ float qs[];  // [r + dr]
  __shared__ float sc[kF32Tok];
  const int tid = threadIdx.x;
  const int piece = blockIdx.x;
  const int m = blockIdx.y;
  const int w = r + dr;
  const int32_t s0 = plan.seg_start[piece], s1 = plan.seg_start[piece + 1];
  for (int32_t si = s0; si < s1; ++si) {
    const DecodeSegment sg = plan.segs[si];
    const int64_t qrow = (int64_t)sg.seq * rows + m;
    __syncthreads();
    for (int c = tid; c < r; c += kF32Threads) qs[c] = load_q(q_lat, qrow * r + c);
    for (int c = tid; c < dr; c += kF32Threads) qs[r + c] = load_q(q_rope, qrow * dr + c);
    __syncthreads();
    // token t of the segment: row sg.t0 + t of the sequence, via its pages
    auto row_at = [&](int32_t t) {
      return reinterpret_cast<const float *>(tab.row(sg.seq, (int64_t)sg.t0 + t, (int64_t)w * 4));
    };
    const int32_t T = sg.t1 - sg.t0;
    float m_run = -INFINITY, l_run = 0.f;
    float acc[kColsPerThread];
#pragma unroll
    for (int k = 0; k < kColsPerThread; ++k) acc[k] = 0.f;
    for (int32_t t0 = 0; t0 < T; t0 += kF32Tok) {
      const int tt = tid >> 2, part = tid & 3;
      float d = 0.f;
      if (t0 + tt < T) {
        const float *row = row_at(t0 + tt);
        for (int c = part; c < w; c += 4) d += qs[c] * row[c];
      }
      d += __shfl_xor(d, 1);
      d += __shfl_xor(d, 2);
      if (part == 0) sc[tt] = (t0 + tt < T) ? d * scale : -INFINITY;
      __syncthreads();
      float cmax = -INFINITY;
      for (int j = 0; j < kF32Tok; ++j) cmax = fmaxf(cmax, sc[j]);
      const float m_new = fmaxf(m_run, cmax);
      const float alpha = (m_run == -INFINITY) ? 0.f : expf(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int k = 0; k < kColsPerThread; ++k) acc[k] *= alpha;
      const int nt = min(kF32Tok, T - t0);
      for (int j = 0; j < nt; ++j) {
        const float p = expf(sc[j] - m_new);
        l_run += p;
        const float *row = row_at(t0 + j);
#pragma unroll
        for (int k = 0; k < kColsPerThread; ++k) {
          const int c = tid + k * kF32Threads;
          if (c < r) acc[k] += p * row[c];
        }
      }
      m_run = m_new;
      __syncthreads();
    }
    const float inv = 1.f / l_run;
    const float lse = m_run + logf(l_run);
    if (sg.slot < 0) {
#pragma unroll
      for (int k = 0; k < kColsPerThread; ++k) {
        const int c = tid + k * kF32Threads;
        if (c < r) out[qrow * r + c] = acc[k] * inv;
      }
      if (out_lse && tid == 0) out_lse[qrow] = lse;
    } else {
      const int64_t prow = (int64_t)sg.slot * rows + m;
#pragma unroll
      for (int k = 0; k < kColsPerThread; ++k) {
        const int c = tid + k * kF32Threads;
        if (c < r) part_o[prow * r + c] = acc[k] * inv;
      }
      if (tid == 0) part_lse[prow] = lse;
    }
  }
}

// One block per (sequence, query row): log-sum-exp merge of the partial
// slots; empty sequences get zeros and lse = -inf.
__global__ __launch_bounds__(256) void k_decode_merge(int32_t rows, int32_t r, DecodePlanView plan,
                                                       const float *__restrict__ part_o,
                                                       const float *__restrict__ part_lse,
                                                       float *__restrict__ out,
                                                       float *__restrict__ out_lse,
                                                       int32_t *__restrict__ adv_lens, int32_t adv) {
  const int b = blockIdx.x, m = blockIdx.y, tid = threadIdx.x;
  // lengths grow by the pending tokens the decode attended (it has finished)
  if (adv_lens && m == 0 && tid == 0) adv_lens[b] += adv;
  const int32_t n = plan.seq_nslots[b];
  const int64_t qrow = (int64_t)b * rows + m;
  if (n == 1) return;
  if (n == 0) {
    for (int c = tid; c < r; c += blockDim.x) out[qrow * r + c] = 0.f;
    if (out_lse && tid == 0) out_lse[qrow] = -INFINITY;
    return;
  }
  const int32_t base = plan.seq_slot_base[b];
  float mx = -INFINITY;
  for (int k = 0; k < n; ++k) mx = fmaxf(mx, part_lse[(int64_t)(base + k) * rows + m]);
  float wsum = 0.f;
  for (int k = 0; k < n; ++k) wsum += expf(part_lse[(int64_t)(base + k) * rows + m] - mx);
  const float inv = 1.f / wsum;
  for (int c = tid; c < r; c += blockDim.x) {
    float a = 0.f;
    for (int k = 0; k < n; ++k) {
      const int64_t prow = (int64_t)(base + k) * rows + m;
      a += expf(part_lse[prow] - mx) * part_o[prow * r + c];
    }
    out[qrow * r + c] = a * inv;
  }
  if (out_lse && tid == 0) out_lse[qrow] = mx + logf(wsum);
}

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace

DecodeWorkspace decode_workspace_layout(int32_t batch, int32_t rows, int32_t r, int32_t blocks,
                                        bool mfma) {
  DecodeWorkspace w;
  w.slots = blocks + batch;
  size_t plan = mfma ? sizeof(int2) * (size_t)batch
                     : sizeof(int32_t) * (blocks + 1) +
                           sizeof(DecodeSegment) * (size_t)(blocks + batch) +
                           2 * sizeof(int32_t) * batch;
  const size_t prow = mfma ? (size_t)((rows + 31) / 32) * 32 : (size_t)rows;
  w.plan_bytes = align256(plan);
  w.part_o_off = w.plan_bytes;
  // partial outputs: f32, or bf16 on the MFMA path (its log-sum-exp stays f32)
  const size_t pelt = mfma ? sizeof(uint16_t) : sizeof(float);
  w.part_lse_off = w.part_o_off + align256(pelt * (size_t)w.slots * prow * r);
  w.total = w.part_lse_off + align256(sizeof(float) * (size_t)w.slots * prow);
  return w;
}

DecodePlanView decode_plan_view(void *ws, int32_t batch, int32_t blocks) {
  DecodePlanView v;
  char *p = static_cast<char *>(ws);
  v.seg_start = reinterpret_cast<int32_t *>(p);
  p += sizeof(int32_t) * (blocks + 1);
  p = reinterpret_cast<char *>((reinterpret_cast<uintptr_t>(p) + 15) & ~uintptr_t(15));
  v.segs = reinterpret_cast<DecodeSegment *>(p);
  p += sizeof(DecodeSegment) * (size_t)(blocks + batch);
  v.seq_slot_base = reinterpret_cast<int32_t *>(p);
  p += sizeof(int32_t) * batch;
  v.seq_nslots = reinterpret_cast<int32_t *>(p);
  return v;
}

qmla_status launch_decode_plan(const qmla_kv_cache *cache, int32_t pending, int32_t batch,
                               int32_t blocks, int32_t chunk, DecodePlanView plan,
                               hipStream_t stream) {
  size_t lds = sizeof(int32_t) * ((size_t)batch + 1 + batch + blocks + 1 + kPlanThreads);
  k_decode_plan<<<dim3(1), dim3(kPlanThreads), lds, stream>>>(cache->d_lens, pending, batch,
                                                             blocks, chunk, plan);
  QMLA_LAUNCH_CHECK("k_decode_plan");
  return QMLA_OK;
}

qmla_status launch_decode_merge(int32_t batch, int32_t rows, int32_t r, DecodePlanView plan,
                                const float *part_o, const float *part_lse, float *out,
                                float *out_lse, int32_t *adv_lens, int32_t adv,
                                hipStream_t stream) {
  k_decode_merge<<<dim3(batch, rows), dim3(256), 0, stream>>>(rows, r, plan, part_o, part_lse,
                                                             out, out_lse, adv_lens, adv);
  QMLA_LAUNCH_CHECK("k_decode_merge");
  return QMLA_OK;
}

qmla_status decode_shape_supported(const qmla_kv_cache *c, int32_t rows) {
  if (c->dtype == QMLA_BF16) {
    QMLA_REQUIRE(decode_mfma_supported(rows, c->r, c->dr), QMLA_ERR_UNSUPPORTED,
                 "bf16 decode for kv_lora_rank %d, rope %d", c->r, c->dr);
    QMLA_REQUIRE(rows <= 65535 * 128, QMLA_ERR_SHAPE, "too many query rows");
    return QMLA_OK;
  }
  QMLA_REQUIRE(c->r <= kF32Threads * kColsPerThread, QMLA_ERR_UNSUPPORTED,
               "kv_lora_rank %d > %d", c->r, kF32Threads * kColsPerThread);
  QMLA_REQUIRE(rows <= 65535, QMLA_ERR_SHAPE, "rows %d > 65535", rows);
  return QMLA_OK;
}

qmla_status launch_decode_f32(const DecodeArgs &a, hipStream_t stream) {
  QMLA_REQUIRE(a.r <= kF32Threads * kColsPerThread, QMLA_ERR_UNSUPPORTED,
               "kv_lora_rank %d > %d", a.r, kF32Threads * kColsPerThread);
  QMLA_REQUIRE(a.rows <= 65535, QMLA_ERR_SHAPE, "rows %d > 65535", a.rows);
  dim3 grid(a.blocks, a.rows), block(kF32Threads);
  size_t lds = sizeof(float) * (a.r + a.dr);
  const PageTable tab = a.cache->table();
  if (a.q_dtype == QMLA_F32) {
    k_decode_f32<float><<<grid, block, lds, stream>>>(
        tab, (const float *)a.q_lat, (const float *)a.q_rope, a.rows, a.r, a.dr, a.scale, a.plan,
        a.out, a.out_lse, a.part_o, a.part_lse);
  } else {
    k_decode_f32<uint16_t><<<grid, block, lds, stream>>>(
        tab, (const uint16_t *)a.q_lat, (const uint16_t *)a.q_rope, a.rows, a.r, a.dr, a.scale,
        a.plan, a.out, a.out_lse, a.part_o, a.part_lse);
  }
  QMLA_LAUNCH_CHECK("k_decode_f32");
  return QMLA_OK;
}

}  // namespace qmla

using namespace qmla;

namespace {

qmla_status validate_decode(const qmla_decode_dims *d, const qmla_kv_cache *c) {
  QMLA_REQUIRE(d && c, QMLA_ERR_INVALID_ARG, "NULL dims or cache");
  QMLA_REQUIRE(d->batch > 0 && d->batch <= c->num_seqs, QMLA_ERR_SHAPE,
               "batch %d outside [1, %d]", d->batch, c->num_seqs);
  QMLA_REQUIRE(d->batch <= kMaxPlanBatch, QMLA_ERR_UNSUPPORTED, "batch %d > %d", d->batch,
               kMaxPlanBatch);
  QMLA_REQUIRE(d->rows > 0, QMLA_ERR_SHAPE, "rows must be > 0");
  QMLA_REQUIRE(d->kv_lora_rank == c->r && d->rope_dim == c->dr, QMLA_ERR_SHAPE,
               "dims (%d, %d) differ from the cache's (%d, %d)", d->kv_lora_rank, d->rope_dim,
               c->r, c->dr);
  int64_t total = 0;
  for (int32_t i = 0; i < d->batch; ++i) total += c->h_lens[i];
  // the in-kernel plan adds decode_mfma_seg_tokens() virtual tokens per sequence
  const int64_t virt =
      total + (int64_t)d->batch * decode_mfma_seg_tokens(d->rows, d->kv_lora_rank, d->rope_dim);
  QMLA_REQUIRE(virt < (int64_t)1 << 31, QMLA_ERR_UNSUPPORTED, "%lld tokens in one call",
               (long long)total);
  return QMLA_OK;
}

// Number of pieces: enough to fill the device, but no piece shorter than a
// minimum so that per-piece overhead (q load, partial write) stays small.
// 128 tokens (four 32-token tiles): at batch 1, 256 and 1024 cached tokens
// step 2-3 us faster than with 256-token pieces; 64-token pieces make the
// 4096-token step 6 us slower (the merge of 64 partials).
int32_t choose_blocks(const qmla_decode_dims *d, const qmla_kv_cache *c, int32_t requested) {
  int64_t total = 0;
  for (int32_t i = 0; i < d->batch; ++i) total += c->h_lens[i];
  if (requested > 0) return std::min<int32_t>(requested, kMaxPlanBlocks);
  int cus = device_cu_count();
  if (cus <= 0) cus = 256;
  int per_cu = (c->dtype == QMLA_BF16 && decode_mfma_supported(d->rows, d->kv_lora_rank, d->rope_dim))
                   ? decode_mfma_blocks_per_cu(d->rows, d->kv_lora_rank, d->rope_dim)
                   : 4;
  int64_t target = (int64_t)cus * per_cu;
  const int64_t min_tokens = 128;
  int64_t by_work = (total + min_tokens - 1) / min_tokens;
  int64_t blocks = std::max<int64_t>(1, std::min(target, by_work));
  return (int32_t)std::min<int64_t>(blocks, kMaxPlanBlocks);
}

qmla_status decode_impl(const qmla_decode_dims *d, const qmla_kv_cache *c, qmla_dtype q_dtype,
                        const void *q_latent, const void *q_rope, double scale, float *out,
                        float *out_lse, int32_t splits, void *ws, size_t ws_bytes,
                        qmla_stream stream) {
  QMLA_TRY(validate_decode(d, c));
  QMLA_REQUIRE(valid_dtype(q_dtype), QMLA_ERR_INVALID_ARG, "bad q dtype");
  QMLA_REQUIRE(q_latent && out, QMLA_ERR_INVALID_ARG, "NULL q_latent or out");
  QMLA_REQUIRE(q_rope || d->rope_dim == 0, QMLA_ERR_INVALID_ARG, "NULL q_rope");
  QMLA_REQUIRE(splits >= 0, QMLA_ERR_INVALID_ARG, "negative split count");
  QMLA_REQUIRE(std::isfinite(scale), QMLA_ERR_INVALID_ARG, "non-finite scale");
  return decode_launch(d, c, q_dtype, q_latent, q_rope, scale, out, out_lse, splits, ws, ws_bytes,
                       0, false, as_stream(stream));
}

}  // namespace

qmla_status qmla::decode_launch(const qmla_decode_dims *d, const qmla_kv_cache *c,
                                qmla_dtype q_dtype, const void *q_latent, const void *q_rope,
                                double scale, float *out, float *out_lse, int32_t splits, void *ws,
                                size_t ws_bytes, int32_t pending, bool advance, hipStream_t s) {
  const int32_t blocks = choose_blocks(d, c, splits);
  const bool mfma = c->dtype == QMLA_BF16;
  if (mfma)
    QMLA_REQUIRE(decode_mfma_supported(d->rows, d->kv_lora_rank, d->rope_dim),
                 QMLA_ERR_UNSUPPORTED, "bf16 decode for kv_lora_rank %d, rope %d",
                 d->kv_lora_rank, d->rope_dim);
  DecodeWorkspace lay = decode_workspace_layout(d->batch, d->rows, d->kv_lora_rank, blocks, mfma);
  QMLA_REQUIRE(ws != nullptr && ws_bytes >= lay.total, QMLA_ERR_WORKSPACE,
               "workspace of %zu bytes < required %zu", ws_bytes, lay.total);
  DecodePlanView plan{};
  if (!mfma) {
    plan = decode_plan_view(ws, d->batch, blocks);
    int64_t total = 0;
    for (int32_t i = 0; i < d->batch; ++i) total += c->h_lens[i];
    int32_t chunk = (int32_t)std::max<int64_t>(1, (total + blocks - 1) / blocks);
    QMLA_TRY(launch_decode_plan(c, pending, d->batch, blocks, chunk, plan, s));
  }
  DecodeArgs a;
  a.cache = c;
  a.batch = d->batch;
  a.rows = d->rows;
  a.r = d->kv_lora_rank;
  a.dr = d->rope_dim;
  a.q_lat = q_latent;
  a.q_rope = q_rope;
  a.q_dtype = q_dtype;
  a.scale = (float)scale;
  a.out = out;
  a.out_lse = out_lse;
  a.plan = plan;
  a.seq_info = reinterpret_cast<int2 *>(ws);
  a.part_o = reinterpret_cast<float *>(static_cast<char *>(ws) + lay.part_o_off);
  a.part_lse = reinterpret_cast<float *>(static_cast<char *>(ws) + lay.part_lse_off);
  a.blocks = blocks;
  a.pending = pending;
  a.advance = advance;
  if (mfma) return launch_decode_mfma(a, s);  // decode + merge
  QMLA_TRY(launch_decode_f32(a, s));
  return launch_decode_merge(d->batch, d->rows, d->kv_lora_rank, plan, a.part_o, a.part_lse, out,
                             out_lse, advance ? c->d_lens : nullptr, pending, s);
}

namespace {

// ------------------------------------------- allocation-free decode -----
// Scratch of qmla_decode_absorbed_noalloc: the decode workspace (plan or
// per-sequence slot table, split partials and their log-sum-exp) lives in
// this file-scope device array instead of a caller buffer.  Each device the
// library runs on holds its own copy for the life of the process.  In host
// code `scratch` names a host-side stand-in, never the device copy: the
// device address comes from hipGetSymbolAddress, once per device, and only
// that pointer is handed to kernels.  Nothing in it needs clearing: every
// call writes each slot entry and partial it later reads.
constexpr size_t kNoAllocScratchBytes = QMLA_DECODE_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

constexpr int kMaxScratchDevices = 64;
std::atomic<void *> g_scratch_ptr[kMaxScratchDevices];
std::mutex g_scratch_mu;

// Device address of this device's scratch (resolved on the first call on
// the device, with it current).
qmla_status noalloc_scratch(void **out) {
  int dev = 0;
  QMLA_HIP(hipGetDevice(&dev));
  QMLA_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, QMLA_ERR_UNSUPPORTED,
               "device ordinal %d >= %d", dev, kMaxScratchDevices);
  void *p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (!p) {
      QMLA_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
      QMLA_REQUIRE(p != nullptr, QMLA_ERR_HIP, "no device address for the decode scratch");
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return QMLA_OK;
}

}  // namespace

extern "C" {

qmla_status qmla_decode_absorbed_noalloc(const qmla_decode_dims *dims, const qmla_kv_cache *cache,
                                         qmla_dtype q_dtype, const void *q_latent,
                                         const void *q_rope, double scale, float *out_latent,
                                         float *out_lse, qmla_stream stream) {
  QMLA_TRY(validate_decode(dims, cache));
  const int32_t blocks = choose_blocks(dims, cache, 0);
  const size_t need = decode_workspace_layout(dims->batch, dims->rows, dims->kv_lora_rank, blocks,
                                              cache->dtype == QMLA_BF16)
                          .total;
  QMLA_REQUIRE(need <= kNoAllocScratchBytes, QMLA_ERR_UNSUPPORTED,
               "decode needs %zu bytes of scratch; the allocation-free entry point has %zu "
               "(use qmla_decode_absorbed with a workspace)",
               need, kNoAllocScratchBytes);
  void *ws = nullptr;
  QMLA_TRY(noalloc_scratch(&ws));
  return decode_impl(dims, cache, q_dtype, q_latent, q_rope, scale, out_latent, out_lse, 0, ws,
                     kNoAllocScratchBytes, stream);
}

qmla_status qmla_decode_workspace_bytes_splits(const qmla_decode_dims *dims,
                                               const qmla_kv_cache *cache, int32_t num_splits,
                                               size_t *bytes) {
  QMLA_REQUIRE(bytes, QMLA_ERR_INVALID_ARG, "bytes is NULL");
  QMLA_TRY(validate_decode(dims, cache));
  QMLA_REQUIRE(num_splits >= 0, QMLA_ERR_INVALID_ARG, "negative split count");
  int32_t blocks = choose_blocks(dims, cache, num_splits);
  *bytes = decode_workspace_layout(dims->batch, dims->rows, dims->kv_lora_rank, blocks,
                                   cache->dtype == QMLA_BF16)
               .total;
  return QMLA_OK;
}

qmla_status qmla_decode_workspace_bytes(const qmla_decode_dims *dims, const qmla_kv_cache *cache,
                                        size_t *bytes) {
  return qmla_decode_workspace_bytes_splits(dims, cache, 0, bytes);
}

qmla_status qmla_decode_absorbed(const qmla_decode_dims *dims, const qmla_kv_cache *cache,
                                 qmla_dtype q_dtype, const void *q_latent, const void *q_rope,
                                 double scale, float *out_latent, float *out_lse, void *workspace,
                                 size_t workspace_bytes, qmla_stream stream) {
  return decode_impl(dims, cache, q_dtype, q_latent, q_rope, scale, out_latent, out_lse, 0,
                     workspace, workspace_bytes, stream);
}

qmla_status qmla_decode_absorbed_splits(const qmla_decode_dims *dims, const qmla_kv_cache *cache,
                                        qmla_dtype q_dtype, const void *q_latent,
                                        const void *q_rope, double scale, float *out_latent,
                                        float *out_lse, int32_t num_splits, void *workspace,
                                        size_t workspace_bytes, qmla_stream stream) {
  return decode_impl(dims, cache, q_dtype, q_latent, q_rope, scale, out_latent, out_lse,
                     num_splits, workspace, workspace_bytes, stream);
}

}  // extern "C"
