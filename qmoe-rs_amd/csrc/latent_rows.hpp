// latent_rows.hpp -- the new-token latent row of an MLA step
// (src/model.rs:270-291): kv_a = [c | k_pe] of one token becomes
//   [LayerNorm(c) | rope(k_pe, position)]
// and is written into its sequence's cache row (the KVCache::append of
// :99-104, :291, fused in).  Shared by the layer's standalone row kernel and
// the decode step's fused absorption launch.
#pragma once

#include "internal.hpp"

namespace qmla {

struct LatentRowsArgs {
  const float *kva;        // [tokens][r + dr] f32
  int s, r, dr;            // tokens per sequence, latent widths
  const float *ln_w, *ln_b;
  float eps;
  const float *inv_freq;   // [dr / 2]
  float mscale;
  PageTable table;         // cache pages (rows f32 or bf16 bits)
  bool bf16;
  const int32_t *lens;     // [sequences] current length (the new rows go after it)
  float *rows;             // optional f32 copy [tokens][r + dr], or null
  const float *kva1;       // optional second K-half of kva: the row is kva + kva1
};

// Sum over the block (all waves call it; blockDim.x a multiple of 64).
__device__ inline float latent_block_sum(float v, float *red) {
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  __syncthreads();
  if (l == 0) red[w] = v;
  __syncthreads();
  float t = 0.f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += red[i];
  return t;
}

// LDS a latent_row call needs: the row and 16 reduction slots.
__host__ __device__ inline size_t latent_row_lds_bytes(int r, int dr) {
  return sizeof(float) * ((size_t)r + dr + 16);
}

// Token `tok` = (b, i) of the call: its row goes to sequence b's cache row
// lens[b] + i (through the block table) at position lens[b] + i.  LayerNorm as
// candle_nn::LayerNorm (src/model.rs:136): mean, biased variance of the
// centred values, divide by sqrt(var + eps), weight, bias.  `lds` holds
// latent_row_lds_bytes(r, dr): the row is read from HBM once.
__device__ inline void latent_row(const LatentRowsArgs &a, int tok, float *lds) {
  const int b = tok / a.s, i = tok % a.s, r = a.r, dr = a.dr;
  const float *src = a.kva + (int64_t)tok * (r + dr);
  const float *src1 = a.kva1 ? a.kva1 + (int64_t)tok * (r + dr) : nullptr;
  float *x = lds, *red = lds + r + dr;
  for (int c = threadIdx.x; c < r + dr; c += blockDim.x) x[c] = src1 ? src[c] + src1[c] : src[c];
  __syncthreads();
  float *y = a.rows ? a.rows + (int64_t)tok * (r + dr) : nullptr;
  const int32_t len = a.lens[b];
  uint8_t *dst = a.table.row(b, (int64_t)len + i, (int64_t)(r + dr) * (a.bf16 ? 2 : 4));
  auto put = [&](int c, float v) {
    if (y) y[c] = v;
    if (a.bf16)
      reinterpret_cast<uint16_t *>(dst)[c] = f32_to_bf16_bits(v);
    else
      reinterpret_cast<float *>(dst)[c] = v;
  };
  float sum = 0.f;
  for (int c = threadIdx.x; c < r; c += blockDim.x) sum += x[c];
  const float mean = latent_block_sum(sum, red) / (float)r;
  float sq = 0.f;
  for (int c = threadIdx.x; c < r; c += blockDim.x) {
    const float d = x[c] - mean;
    sq += d * d;
  }
  const float var = latent_block_sum(sq, red) / (float)r;
  const float den = sqrtf(var + a.eps);
  for (int c = threadIdx.x; c < r; c += blockDim.x) {
    const float t = (x[c] - mean) / den * a.ln_w[c];
    put(c, a.ln_b ? t + a.ln_b[c] : t);
  }
  const float pos = (float)(len + i);
  for (int p = threadIdx.x; p < dr / 2; p += blockDim.x) {
    const float ang = pos * a.inv_freq[p];
    float cs, sn;
    rope_cs(ang, a.mscale, cs, sn);
    const float e = x[r + 2 * p], o = x[r + 2 * p + 1];
    put(r + 2 * p, e * cs - o * sn);
    put(r + 2 * p + 1, o * cs + e * sn);
  }
}

}  // namespace qmla
