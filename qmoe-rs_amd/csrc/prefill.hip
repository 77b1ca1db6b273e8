// prefill.hip -- causal / chunked prefill attention: the f32 (parity-mode)
// kernel and the C entry points.
//
// Replaces fused_prefill_attn (src/attention_kernel.rs:64-107), which loops
// over query tiles of tile_size(S) rows (:3-11), materialises
// [b, h, tile, S] scores, adds the make_causal_mask (:14-31) -1e18 mask and
// runs a full softmax per row.  Here every (b, h, query tile) block streams
// key tiles through LDS with an online softmax; keys wholly above the causal
// diagonal are skipped, which is exact because exp(-1e18 - max) == 0.

#include <cmath>

#include "internal.hpp"

namespace qmla {

namespace {

constexpr int kPfRows = 64;     // query rows per block
constexpr int kPfKeys = 16;     // keys per LDS tile
constexpr int kPfThreads = 256; // 4 threads per query row
constexpr int kPfMaxQK = 256;   // dn + dr limit of this kernel
constexpr int kPfMaxV = 256;    // dv limit of this kernel

// grid (ceil(seq_q / 64), heads, batch)
template <int VPT>  // output columns per thread = ceil(dv / 4)
__global__ __launch_bounds__(kPfThreads) void k_prefill_f32(
    const float *__restrict__ q_nope, const float *__restrict__ q_rope,
    const float *__restrict__ k, const float *__restrict__ k_rope, const float *__restrict__ v,
    qmla_prefill_dims d, float scale, int causal, float *__restrict__ out) {
  const int dn = d.qk_nope, dr = d.qk_rope, dqk = dn + dr, dv = d.v_dim;
  __shared__ float ks[kPfKeys][kPfMaxQK + 1];
  __shared__ float vs[kPfKeys][kPfMaxV + 1];
  const int tid = threadIdx.x;
  const int rloc = tid >> 2, part = tid & 3;
  const int q0 = blockIdx.x * kPfRows;
  const int h = blockIdx.y, b = blockIdx.z;
  const int qi = q0 + rloc;
  const bool q_ok = qi < d.seq_q;
  const int64_t bh = (int64_t)b * d.heads + h;
  const int64_t bkr = (int64_t)b * d.k_rope_heads + (d.k_rope_heads == 1 ? 0 : h);

  // this thread's share of the query row: dims part, part+4, ...
  float q[kPfMaxQK / 4];
#pragma unroll
  for (int j = 0; j < kPfMaxQK / 4; ++j) {
    const int c = part + 4 * j;
    float x = 0.f;
    if (q_ok && c < dqk)
      x = c < dn ? q_nope[(bh * d.seq_q + qi) * dn + c] : q_rope[(bh * d.seq_q + qi) * dr + (c - dn)];
    q[j] = x;
  }
  float acc[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) acc[j] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  // last key any row of this block can see
  int kend = d.seq_k;
  if (causal) {
    const int last_row = min(q0 + kPfRows, d.seq_q) - 1 + d.q_offset;
    kend = min(kend, last_row + 1);
  }
  const int row_abs = d.q_offset + qi;
  for (int k0 = 0; k0 < kend; k0 += kPfKeys) {
    __syncthreads();
    for (int e = tid; e < kPfKeys * dqk; e += kPfThreads) {
      const int t = e / dqk, c = e - t * dqk;
      const int key = k0 + t;
      float x = 0.f;
      if (key < d.seq_k)
        x = c < dn ? k[(bh * d.seq_k + key) * dn + c] : k_rope[(bkr * d.seq_k + key) * dr + (c - dn)];
      ks[t][c] = x;
    }
    for (int e = tid; e < kPfKeys * dv; e += kPfThreads) {
      const int t = e / dv, c = e - t * dv;
      const int key = k0 + t;
      vs[t][c] = key < d.seq_k ? v[(bh * d.seq_k + key) * dv + c] : 0.f;
    }
    __syncthreads();
    float sc[kPfKeys];
    float cmax = -INFINITY;
#pragma unroll
    for (int t = 0; t < kPfKeys; ++t) {
      float a = 0.f;
#pragma unroll
      for (int j = 0; j < kPfMaxQK / 4; ++j) {
        const int c = part + 4 * j;
        if (c < dqk) a += q[j] * ks[t][c];
      }
      a += __shfl_xor(a, 1);
      a += __shfl_xor(a, 2);
      const int key = k0 + t;
      const bool vis = key < d.seq_k && (!causal || key <= row_abs);
      sc[t] = vis ? a * scale : -INFINITY;
      cmax = fmaxf(cmax, sc[t]);
    }
    const float m_new = fmaxf(m_run, cmax);
    if (m_new == -INFINITY) continue;  // nothing visible yet for this row
    const float alpha = m_run == -INFINITY ? 0.f : expf(m_run - m_new);
    l_run *= alpha;
#pragma unroll
    for (int j = 0; j < VPT; ++j) acc[j] *= alpha;
#pragma unroll
    for (int t = 0; t < kPfKeys; ++t) {
      const float p = expf(sc[t] - m_new);
      l_run += p;
#pragma unroll
      for (int j = 0; j < VPT; ++j) {
        const int c = part + 4 * j;
        if (c < dv) acc[j] += p * vs[t][c];
      }
    }
    m_run = m_new;
  }
  if (!q_ok) return;
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
  float *o = out + (bh * d.seq_q + qi) * dv;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const int c = part + 4 * j;
    if (c < dv) o[c] = acc[j] * inv;
  }
}

}  // namespace

qmla_status launch_prefill_f32(const qmla_prefill_dims &d, const float *q_nope, const float *q_rope,
                               const float *k, const float *k_rope, const float *v, float scale,
                               int causal, float *out, hipStream_t stream) {
  QMLA_REQUIRE(d.qk_nope + d.qk_rope <= kPfMaxQK && d.v_dim <= kPfMaxV, QMLA_ERR_UNSUPPORTED,
               "f32 prefill supports qk width <= %d and v width <= %d", kPfMaxQK, kPfMaxV);
  dim3 grid((d.seq_q + kPfRows - 1) / kPfRows, d.heads, d.batch), block(kPfThreads);
  const int vpt = (d.v_dim + 3) / 4;
  if (vpt <= 8)
    k_prefill_f32<8><<<grid, block, 0, stream>>>(q_nope, q_rope, k, k_rope, v, d, scale, causal, out);
  else if (vpt <= 32)
    k_prefill_f32<32><<<grid, block, 0, stream>>>(q_nope, q_rope, k, k_rope, v, d, scale, causal, out);
  else
    k_prefill_f32<64><<<grid, block, 0, stream>>>(q_nope, q_rope, k, k_rope, v, d, scale, causal, out);
  QMLA_LAUNCH_CHECK("k_prefill_f32");
  return QMLA_OK;
}

}  // namespace qmla

using namespace qmla;

namespace {

qmla_status validate_prefill(const qmla_prefill_dims *d, qmla_dtype dtype, const void *q_nope,
                             const void *q_rope, const void *k, const void *k_rope, const void *v,
                             double scale, int causal, const void *out) {
  QMLA_REQUIRE(d, QMLA_ERR_INVALID_ARG, "dims is NULL");
  QMLA_REQUIRE(valid_dtype(dtype), QMLA_ERR_INVALID_ARG, "bad dtype %d", (int)dtype);
  QMLA_REQUIRE(d->batch > 0 && d->heads > 0 && d->seq_q >= 0 && d->seq_k >= 0, QMLA_ERR_SHAPE,
               "bad batch/heads/seq (%d, %d, %d, %d)", d->batch, d->heads, d->seq_q, d->seq_k);
  QMLA_REQUIRE(d->batch <= 65535 && d->heads <= 65535, QMLA_ERR_SHAPE, "batch or heads > 65535");
  QMLA_REQUIRE(d->qk_nope > 0 && d->qk_rope >= 0 && d->v_dim > 0, QMLA_ERR_SHAPE,
               "bad head dims (%d, %d, %d)", d->qk_nope, d->qk_rope, d->v_dim);
  QMLA_REQUIRE(d->k_rope_heads == 1 || d->k_rope_heads == d->heads, QMLA_ERR_SHAPE,
               "k_rope_heads %d must be 1 or heads (%d)", d->k_rope_heads, d->heads);
  QMLA_REQUIRE(d->q_offset >= 0, QMLA_ERR_SHAPE, "q_offset %d < 0", d->q_offset);
  QMLA_REQUIRE(causal || d->q_offset == 0, QMLA_ERR_SHAPE, "q_offset needs causal");
  QMLA_REQUIRE(std::isfinite(scale), QMLA_ERR_INVALID_ARG, "non-finite scale");
  const bool empty = d->seq_q == 0;
  QMLA_REQUIRE(empty || (q_nope && k && v && out), QMLA_ERR_INVALID_ARG, "NULL tensor");
  QMLA_REQUIRE(empty || d->qk_rope == 0 || (q_rope && k_rope), QMLA_ERR_INVALID_ARG,
               "NULL rope tensor");
  return QMLA_OK;
}

}  // namespace

extern "C" {

qmla_status qmla_fused_prefill_attn(const qmla_prefill_dims *dims, qmla_dtype dtype,
                                    const void *q_nope, const void *q_rope, const void *k,
                                    const void *k_rope, const void *v, double scale, int causal,
                                    void *out, qmla_stream stream) {
  QMLA_TRY(validate_prefill(dims, dtype, q_nope, q_rope, k, k_rope, v, scale, causal, out));
  if (dims->seq_q == 0) return QMLA_OK;
  hipStream_t s = as_stream(stream);
  if (dims->seq_k == 0) {
    // no key at all: every row is empty
    return zero_bytes(out,
                      (size_t)dims->batch * dims->heads * dims->seq_q * dims->v_dim *
                          dtype_bytes(dtype),
                      s);
  }
  if (dtype == QMLA_F32)
    return launch_prefill_f32(*dims, (const float *)q_nope, (const float *)q_rope,
                              (const float *)k, (const float *)k_rope, (const float *)v,
                              (float)scale, causal, (float *)out, s);
  return launch_prefill_bf16(*dims, (const uint16_t *)q_nope, (const uint16_t *)q_rope,
                             (const uint16_t *)k, (const uint16_t *)k_rope, (const uint16_t *)v,
                             (float)scale, causal, (uint16_t *)out, s);
}

qmla_status qmla_reference_eager_attn(int32_t b, int32_t h, int32_t s, int32_t d, int32_t dv,
                                      qmla_dtype dtype, const void *q, const void *k,
                                      const void *v, double scale, int causal, void *out,
                                      qmla_stream stream) {
  qmla_prefill_dims dims{b, h, s, s, d, 0, dv, 1, 0};
  return qmla_fused_prefill_attn(&dims, dtype, q, nullptr, k, nullptr, v, scale, causal, out,
                                 stream);
}

qmla_status qmla_eager_prefill_attn(int32_t b, int32_t h, int32_t s, int32_t d, int32_t dv,
                                    qmla_dtype dtype, const void *q, const void *k, const void *v,
                                    double scale, int causal, void *out, qmla_stream stream) {
  return qmla_reference_eager_attn(b, h, s, d, dv, dtype, q, k, v, scale, causal, out, stream);
}

}  // extern "C"
