/*
 * mla_oracle.c -- CPU restatement of qmoe-rs's MLA attention path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker).  Loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg; never by the
 * product library.  See mla_oracle.h for the per-function parity status.
 *
 * Built with -ffp-contract=off so that fp32 expressions round the way the
 * reference's separate tensor ops do (no fused multiply-add contraction).
 */
#include "mla_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ RNG -- */

/* SplitMix64 (Steele, Lea, Flood 2014; Vigna's reference C): output i of a
 * generator seeded with `seed` is mix(seed + (i+1) * golden). */
uint64_t orc_splitmix64_at(uint64_t seed, uint64_t i) {
  uint64_t z = seed + (i + 1) * 0x9E3779B97F4A7C15ULL;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

/* Box-Muller (cosine branch): element i uses outputs 2i and 2i+1. */
void orc_fill_normal(float *out, size_t n, uint64_t seed, double mean, double std_) {
  const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)n; ++i) {
    uint64_t a = orc_splitmix64_at(seed, 2 * (uint64_t)i);
    uint64_t b = orc_splitmix64_at(seed, 2 * (uint64_t)i + 1);
    double u1 = ((double)(a >> 11) + 1.0) * (1.0 / 9007199254740992.0); /* (0, 1] */
    double u2 = (double)(b >> 11) * (1.0 / 9007199254740992.0);         /* [0, 1) */
    double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
    out[i] = (float)(mean + std_ * z);
  }
}

/* Uniform integers in [lo, hi] by multiply-shift of the top 32 bits. */
void orc_fill_uniform_int(int32_t *out, size_t n, uint64_t seed, int32_t lo, int32_t hi) {
  uint64_t range = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
  for (size_t i = 0; i < n; ++i) {
    uint64_t x = orc_splitmix64_at(seed, i) >> 32;
    out[i] = (int32_t)((int64_t)lo + (int64_t)((x * range) >> 32));
  }
}

uint16_t orc_f32_to_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float orc_bf16_to_f32(uint16_t x) {
  uint32_t u = (uint32_t)x << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void orc_to_bf16(const float *in, uint16_t *out, size_t n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)n; ++i) out[i] = orc_f32_to_bf16(in[i]);
}

void orc_round_bf16(const float *in, float *out, size_t n) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < (long)n; ++i) out[i] = orc_bf16_to_f32(orc_f32_to_bf16(in[i]));
}

int orc_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void orc_set_num_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ------------------------------------------------------- scalar helpers -- */

/* src/model.rs:46-52 */
double orc_yarn_get_mscale(double scale, double mscale) {
  if (scale <= 1.0) return 1.0;
  return 0.1 * mscale * log(scale) + 1.0;
}

/* src/model.rs:160-173: factor 40, mscale 1.0, mscale_all_dim 0.707. */
void orc_mla_scales(int qk_nope, int qk_rope, double *rope_mscale, double *softmax_scale) {
  const double factor = 40.0, mscale = 1.0, mscale_all_dim = 0.707;
  if (rope_mscale)
    *rope_mscale =
        orc_yarn_get_mscale(factor, mscale) / orc_yarn_get_mscale(factor, mscale_all_dim);
  if (softmax_scale) {
    double q_head_dim = (double)(qk_nope + qk_rope);
    double base = pow(q_head_dim, -0.5);
    double m = orc_yarn_get_mscale(factor, mscale_all_dim);
    *softmax_scale = base * m * m;
  }
}

/* src/attention_kernel.rs:3-11 */
int orc_tile_size(int seq_len) {
  if (seq_len > 2048) return 16;
  if (seq_len > 1024) return 32;
  return 64;
}

/* ----------------------------------------------------------------- RoPE -- */

/* src/model.rs:55-66.  inv_freq is `1.0 / 10000f64.powf(2i/d) as f32`, an
 * f32 division (Rust's `as` binds tighter than `/`); the angle is the f32
 * product pos * inv_freq (a K=1 matmul); cos/sin are scaled by the f32
 * value of rope_mscale (candle's affine casts the f64 factor to f32). */
void orc_rope_table(int pos0, int n, int d, double mscale, float *out) {
  int half = d / 2;
  float ms = (float)mscale;
  float *inv = (float *)malloc(sizeof(float) * (size_t)(half > 0 ? half : 1));
  for (int i = 0; i < half; ++i) inv[i] = 1.0f / (float)pow(10000.0, 2.0 * i / (double)d);
  for (int p = 0; p < n; ++p) {
    float pos = (float)(pos0 + p);
    for (int i = 0; i < half; ++i) {
      float ang = pos * inv[i];
      out[(size_t)p * d + i] = cosf(ang) * ms;
      out[(size_t)p * d + half + i] = sinf(ang) * ms;
    }
  }
  free(inv);
}

/* src/model.rs:70-84: even/odd pairs (2i, 2i+1);
 *   even' = even*cos - odd*sin ; odd' = odd*cos + even*sin. */
void orc_apply_rope(const float *x, float *out, int outer, int s, int d, const float *table) {
  int half = d / 2;
  for (long o = 0; o < outer; ++o)
    for (int p = 0; p < s; ++p) {
      const float *xr = x + ((size_t)o * s + p) * d;
      float *yr = out + ((size_t)o * s + p) * d;
      const float *cs = table + (size_t)p * d;
      for (int i = 0; i < half; ++i) {
        float e = xr[2 * i], od = xr[2 * i + 1];
        float c = cs[i], sn = cs[half + i];
        float a = e * c, bb = od * sn, cc = od * c, dd = e * sn;
        yr[2 * i] = a - bb;
        yr[2 * i + 1] = cc + dd;
      }
    }
}

/* ------------------------------------------------------- dense building -- */

/* candle_nn::Linear: y = x W^T + b (src/model.rs:126-146 construct them). */
void orc_linear(const float *x, int rows, int in, const float *W, const float *b, int out,
                float *y) {
#pragma omp parallel for schedule(static)
  for (long i = 0; i < rows; ++i) {
    const float *xr = x + (size_t)i * in;
    for (int o = 0; o < out; ++o) {
      const float *w = W + (size_t)o * in;
      float acc = 0.0f;
      for (int k = 0; k < in; ++k) acc += xr[k] * w[k];
      y[(size_t)i * out + o] = b ? acc + b[o] : acc;
    }
  }
}

/* candle_nn::LayerNorm (src/model.rs:136): mean-removing, biased variance,
 * eps inside the square root, then weight and bias. */
void orc_layer_norm(const float *x, int rows, int n, const float *w, const float *b, double eps,
                    float *y) {
  float feps = (float)eps;
  for (long i = 0; i < rows; ++i) {
    const float *xr = x + (size_t)i * n;
    float *yr = y + (size_t)i * n;
    float sum = 0.0f;
    for (int k = 0; k < n; ++k) sum += xr[k];
    float mean = sum / (float)n;
    float sq = 0.0f;
    for (int k = 0; k < n; ++k) {
      float c = xr[k] - mean;
      sq += c * c;
    }
    float var = sq / (float)n;
    float den = sqrtf(var + feps);
    for (int k = 0; k < n; ++k) {
      float c = (xr[k] - mean) / den;
      float t = c * w[k];
      yr[k] = b ? t + b[k] : t;
    }
  }
}

/* candle_nn::ops::softmax(x, last dim): max, subtract, exp, sum, divide. */
void orc_softmax_rows(float *x, long rows, int n) {
  for (long i = 0; i < rows; ++i) {
    float *r = x + (size_t)i * n;
    float m = -INFINITY;
    for (int j = 0; j < n; ++j) m = r[j] > m ? r[j] : m;
    float sum = 0.0f;
    for (int j = 0; j < n; ++j) {
      r[j] = expf(r[j] - m);
      sum += r[j];
    }
    for (int j = 0; j < n; ++j) r[j] = r[j] / sum;
  }
}

/* ------------------------------------------------------------ attention -- */

/* The additive mask value: `mask * (-1e18f64)` on an f32 tensor. */
#define ORC_MASK_NEG ((float)-1e18)

/* src/attention_kernel.rs:110-134 */
void orc_reference_eager_attn(const float *q, const float *k, const float *v, int b, int h, int s,
                              int d, int dv, double scale, int causal, float *out) {
  float fscale = (float)scale;
#pragma omp parallel for collapse(2) schedule(static)
  for (int bi = 0; bi < b; ++bi)
    for (int hi = 0; hi < h; ++hi) {
      size_t bh = (size_t)bi * h + hi;
      const float *Q = q + bh * s * d, *K = k + bh * s * d, *V = v + bh * s * dv;
      float *O = out + bh * s * dv;
      float *sc = (float *)malloc(sizeof(float) * (size_t)s);
      for (int i = 0; i < s; ++i) {
        for (int j = 0; j < s; ++j) {
          float acc = 0.0f;
          for (int c = 0; c < d; ++c) acc += Q[(size_t)i * d + c] * K[(size_t)j * d + c];
          acc = acc * fscale;
          if (causal) acc = acc + ((i < j) ? ORC_MASK_NEG : 0.0f);
          sc[j] = acc;
        }
        orc_softmax_rows(sc, 1, s);
        for (int c = 0; c < dv; ++c) {
          float acc = 0.0f;
          for (int j = 0; j < s; ++j) acc += sc[j] * V[(size_t)j * dv + c];
          O[(size_t)i * dv + c] = acc;
        }
      }
      free(sc);
    }
}

/* src/attention_kernel.rs:64-107 with make_causal_mask (:14-31) rows offset
 * by q_offset.  The tile loop (:82-104) is kept: each tile's rows are formed
 * exactly as the reference forms them (scores_nope + scores_rope, then the
 * scale, then the mask). */
void orc_fused_prefill_attn(const float *q_nope, const float *q_rope, const float *k,
                            const float *k_rope, const float *v, int b, int h, int sq, int sk,
                            int dn, int dr, int dv, int krh, int q_offset, double scale,
                            int causal, float *out) {
  float fscale = (float)scale;
  int tile = orc_tile_size(sq);
#pragma omp parallel for collapse(2) schedule(static)
  for (int bi = 0; bi < b; ++bi)
    for (int hi = 0; hi < h; ++hi) {
      size_t bh = (size_t)bi * h + hi;
      size_t bkr = (size_t)bi * krh + (krh == 1 ? 0 : hi);
      const float *QN = q_nope + bh * sq * dn, *QR = q_rope + bh * sq * dr;
      const float *K = k + bh * sk * dn, *KR = k_rope + bkr * sk * dr, *V = v + bh * sk * dv;
      float *O = out + bh * sq * dv;
      float *sc = (float *)malloc(sizeof(float) * (size_t)sk);
      for (int t0 = 0; t0 < sq; t0 += tile) {
        int t1 = t0 + tile < sq ? t0 + tile : sq;
        for (int i = t0; i < t1; ++i) {
          int row = q_offset + i;
          for (int j = 0; j < sk; ++j) {
            float an = 0.0f, ar = 0.0f;
            for (int c = 0; c < dn; ++c) an += QN[(size_t)i * dn + c] * K[(size_t)j * dn + c];
            for (int c = 0; c < dr; ++c) ar += QR[(size_t)i * dr + c] * KR[(size_t)j * dr + c];
            float sv = (an + ar) * fscale;
            if (causal) sv = sv + ((row < j) ? ORC_MASK_NEG : 0.0f);
            sc[j] = sv;
          }
          orc_softmax_rows(sc, 1, sk);
          for (int c = 0; c < dv; ++c) {
            float acc = 0.0f;
            for (int j = 0; j < sk; ++j) acc += sc[j] * V[(size_t)j * dv + c];
            O[(size_t)i * dv + c] = acc;
          }
        }
      }
      free(sc);
    }
}

/* Textbook fp64 attention; masked keys are excluded outright (exp of
 * -1e18 - max is exactly zero in both precisions). */
void orc_prefill_attn_f64(const float *q_nope, const float *q_rope, const float *k,
                          const float *k_rope, const float *v, int b, int h, int sq, int sk,
                          int dn, int dr, int dv, int krh, int q_offset, double scale, int causal,
                          double *out) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int bi = 0; bi < b; ++bi)
    for (int hi = 0; hi < h; ++hi) {
      size_t bh = (size_t)bi * h + hi;
      size_t bkr = (size_t)bi * krh + (krh == 1 ? 0 : hi);
      const float *QN = q_nope + bh * sq * dn, *QR = q_rope + bh * sq * dr;
      const float *K = k + bh * sk * dn, *KR = k_rope + bkr * sk * dr, *V = v + bh * sk * dv;
      double *O = out + bh * sq * dv;
      double *sc = (double *)malloc(sizeof(double) * (size_t)sk);
      for (int i = 0; i < sq; ++i) {
        int row = q_offset + i;
        int jmax = causal ? (row + 1 < sk ? row + 1 : sk) : sk;
        double m = -INFINITY;
        for (int j = 0; j < jmax; ++j) {
          double a = 0.0;
          for (int c = 0; c < dn; ++c) a += (double)QN[(size_t)i * dn + c] * K[(size_t)j * dn + c];
          for (int c = 0; c < dr; ++c) a += (double)QR[(size_t)i * dr + c] * KR[(size_t)j * dr + c];
          sc[j] = a * scale;
          if (sc[j] > m) m = sc[j];
        }
        double sum = 0.0;
        for (int j = 0; j < jmax; ++j) {
          sc[j] = exp(sc[j] - m);
          sum += sc[j];
        }
        for (int c = 0; c < dv; ++c) {
          double acc = 0.0;
          for (int j = 0; j < jmax; ++j) acc += sc[j] * V[(size_t)j * dv + c];
          O[(size_t)i * dv + c] = jmax > 0 ? acc / sum : 0.0;
        }
      }
      free(sc);
    }
}

/* --------------------------------------------------- MLA layer (ref) ----- */

/* src/model.rs:178-190: kv_b = Linear(c); reshape [n, H, dn+dv]; split. */
void orc_compute_kv(const orc_mla_layer *L, const float *c, long n, float *k, float *v) {
  int H = L->heads, dn = L->dn, dv = L->dv, w = dn + dv;
  float *kvb = (float *)malloc(sizeof(float) * (size_t)n * H * w);
  orc_linear(c, (int)n, L->r, L->wkvb, L->bkvb, H * w, kvb);
  for (long t = 0; t < n; ++t)
    for (int hh = 0; hh < H; ++hh) {
      const float *src = kvb + ((size_t)t * H + hh) * w;
      memcpy(k + ((size_t)t * H + hh) * dn, src, sizeof(float) * dn);
      memcpy(v + ((size_t)t * H + hh) * dv, src + dn, sizeof(float) * dv);
    }
  free(kvb);
}

/* src/model.rs:270-273 (projection, split, LayerNorm) and :281-288 (RoPE of
 * the shared rope part at positions pos0 + i). */
void orc_mla_latent_rows(const orc_mla_layer *L, const float *xs, int b, int s, int pos0,
                         float *rows) {
  int r = L->r, dr = L->dr, w = r + dr;
  long n = (long)b * s;
  float *kva = (float *)malloc(sizeof(float) * (size_t)n * w);
  float *tab = (float *)malloc(sizeof(float) * (size_t)s * (dr > 0 ? dr : 1));
  float *tmp = (float *)malloc(sizeof(float) * (size_t)s * (dr > 0 ? dr : 1));
  orc_linear(xs, (int)n, L->hidden, L->wkva, L->bkva, w, kva);
  orc_rope_table(pos0, s, dr, L->rope_mscale, tab);
  for (int bi = 0; bi < b; ++bi) {
    for (int i = 0; i < s; ++i) {
      const float *src = kva + ((size_t)bi * s + i) * w;
      float *dst = rows + ((size_t)bi * s + i) * w;
      orc_layer_norm(src, 1, r, L->ln_w, L->ln_b, L->ln_eps, dst);
      memcpy(tmp + (size_t)i * dr, src + r, sizeof(float) * dr);
    }
    orc_apply_rope(tmp, tmp, 1, s, dr, tab);
    for (int i = 0; i < s; ++i)
      memcpy(rows + ((size_t)bi * s + i) * w + r, tmp + (size_t)i * dr, sizeof(float) * dr);
  }
  free(kva);
  free(tab);
  free(tmp);
}

void orc_decompress_cache(const orc_mla_layer *L, const float *latent, int b, int T, float *k,
                          float *v, float *k_rope) {
  int H = L->heads, dn = L->dn, dv = L->dv, dr = L->dr, r = L->r, w = r + dr;
  float *c = (float *)malloc(sizeof(float) * (size_t)T * r + 1);
  float *kt = (float *)malloc(sizeof(float) * (size_t)T * H * dn + 1);
  float *vt = (float *)malloc(sizeof(float) * (size_t)T * H * dv + 1);
  for (int bi = 0; bi < b; ++bi) {
    for (int t = 0; t < T; ++t)
      memcpy(c + (size_t)t * r, latent + ((size_t)bi * T + t) * w, sizeof(float) * r);
    orc_compute_kv(L, c, T, kt, vt);
    for (int hh = 0; hh < H; ++hh)
      for (int t = 0; t < T; ++t) {
        size_t o = (((size_t)bi * H + hh) * T + t);
        memcpy(k + o * dn, kt + ((size_t)t * H + hh) * dn, sizeof(float) * dn);
        memcpy(v + o * dv, vt + ((size_t)t * H + hh) * dv, sizeof(float) * dv);
        memcpy(k_rope + o * dr, latent + ((size_t)bi * T + t) * w + r, sizeof(float) * dr);
      }
  }
  free(c);
  free(kt);
  free(vt);
}

/* Shared front half of forward_prefill / forward_with_cache:
 * q projection, split, RoPE of q_rope at positions pos0 + i
 * (src/model.rs:199-203 / :263-267).  q_nope [b,H,s,dn], q_rope [b,H,s,dr]. */
static void orc_mla_queries(const orc_mla_layer *L, const float *xs, int b, int s, int pos0,
                            float *q_nope, float *q_rope) {
  int H = L->heads, dn = L->dn, dr = L->dr, w = dn + dr;
  long n = (long)b * s;
  float *q = (float *)malloc(sizeof(float) * (size_t)n * H * w);
  float *tab = (float *)malloc(sizeof(float) * (size_t)s * (dr > 0 ? dr : 1));
  orc_linear(xs, (int)n, L->hidden, L->wq, L->bq, H * w, q);
  for (int bi = 0; bi < b; ++bi)
    for (int i = 0; i < s; ++i)
      for (int hh = 0; hh < H; ++hh) {
        const float *src = q + (((size_t)bi * s + i) * H + hh) * w;
        size_t o = (((size_t)bi * H + hh) * s + i);
        memcpy(q_nope + o * dn, src, sizeof(float) * dn);
        memcpy(q_rope + o * dr, src + dn, sizeof(float) * dr);
      }
  orc_rope_table(pos0, s, dr, L->rope_mscale, tab);
  orc_apply_rope(q_rope, q_rope, b * H, s, dr, tab);
  free(q);
  free(tab);
}

/* context [b,H,s,dv] -> transpose/reshape [b,s,H*dv] -> o_proj
 * (src/model.rs:248-249 and :304-306). */
static void orc_mla_output(const orc_mla_layer *L, const float *ctx, int b, int s, float *out) {
  int H = L->heads, dv = L->dv;
  float *t = (float *)malloc(sizeof(float) * (size_t)b * s * H * dv);
  for (int bi = 0; bi < b; ++bi)
    for (int hh = 0; hh < H; ++hh)
      for (int i = 0; i < s; ++i)
        memcpy(t + (((size_t)bi * s + i) * H + hh) * dv, ctx + (((size_t)bi * H + hh) * s + i) * dv,
               sizeof(float) * dv);
  orc_linear(t, b * s, H * dv, L->wo, L->bo, L->hidden, out);
  free(t);
}

/* src/model.rs:256-307 */
void orc_mla_forward_with_cache(const orc_mla_layer *L, const float *xs, int b, int s,
                                const float *k, const float *v, const float *k_rope, int Tc,
                                float *out, float *new_k, float *new_v, float *new_k_rope) {
  int H = L->heads, dn = L->dn, dr = L->dr, dv = L->dv, r = L->r, w = r + dr;
  int T = Tc + s;
  float *qn = (float *)malloc(sizeof(float) * (size_t)b * H * s * dn + 1);
  float *qr = (float *)malloc(sizeof(float) * (size_t)b * H * s * dr + 1);
  orc_mla_queries(L, xs, b, s, Tc, qn, qr);

  /* new latent rows (LayerNorm'd c, roped k_pe), then decompression */
  float *rows = (float *)malloc(sizeof(float) * (size_t)b * s * w + 1);
  orc_mla_latent_rows(L, xs, b, s, Tc, rows);
  float *ka = (float *)malloc(sizeof(float) * (size_t)b * H * T * dn + 1);
  float *va = (float *)malloc(sizeof(float) * (size_t)b * H * T * dv + 1);
  float *kra = (float *)malloc(sizeof(float) * (size_t)b * H * T * dr + 1);
  float *c = (float *)malloc(sizeof(float) * (size_t)s * r + 1);
  float *kt = (float *)malloc(sizeof(float) * (size_t)s * H * dn + 1);
  float *vt = (float *)malloc(sizeof(float) * (size_t)s * H * dv + 1);
  for (int bi = 0; bi < b; ++bi) {
    for (int i = 0; i < s; ++i) memcpy(c + (size_t)i * r, rows + ((size_t)bi * s + i) * w, sizeof(float) * r);
    orc_compute_kv(L, c, s, kt, vt);
    for (int hh = 0; hh < H; ++hh) {
      size_t bh = (size_t)bi * H + hh;
      /* KVCache::append = cat along the sequence dim (src/model.rs:99-104) */
      if (Tc > 0) {
        memcpy(ka + bh * T * dn, k + bh * Tc * dn, sizeof(float) * (size_t)Tc * dn);
        memcpy(va + bh * T * dv, v + bh * Tc * dv, sizeof(float) * (size_t)Tc * dv);
        memcpy(kra + bh * T * dr, k_rope + bh * Tc * dr, sizeof(float) * (size_t)Tc * dr);
      }
      for (int i = 0; i < s; ++i) {
        memcpy(ka + (bh * T + Tc + i) * dn, kt + ((size_t)i * H + hh) * dn, sizeof(float) * dn);
        memcpy(va + (bh * T + Tc + i) * dv, vt + ((size_t)i * H + hh) * dv, sizeof(float) * dv);
        memcpy(kra + (bh * T + Tc + i) * dr, rows + ((size_t)bi * s + i) * w + r, sizeof(float) * dr);
      }
    }
  }
  /* scores over all T keys, no mask (src/model.rs:297-302) */
  float *ctx = (float *)malloc(sizeof(float) * (size_t)b * H * s * dv + 1);
  orc_fused_prefill_attn(qn, qr, ka, kra, va, b, H, s, T, dn, dr, dv, H, 0, L->softmax_scale, 0,
                         ctx);
  orc_mla_output(L, ctx, b, s, out);
  if (new_k) memcpy(new_k, ka, sizeof(float) * (size_t)b * H * T * dn);
  if (new_v) memcpy(new_v, va, sizeof(float) * (size_t)b * H * T * dv);
  if (new_k_rope) memcpy(new_k_rope, kra, sizeof(float) * (size_t)b * H * T * dr);
  free(qn); free(qr); free(rows); free(ka); free(va); free(kra); free(c); free(kt); free(vt);
  free(ctx);
}

/* src/model.rs:193-253 (fused_attn branch, causal). */
void orc_mla_forward_prefill(const orc_mla_layer *L, const float *xs, int b, int s, float *out,
                             float *k, float *v, float *k_rope) {
  int H = L->heads, dn = L->dn, dr = L->dr, dv = L->dv, r = L->r, w = r + dr;
  float *qn = (float *)malloc(sizeof(float) * (size_t)b * H * s * dn + 1);
  float *qr = (float *)malloc(sizeof(float) * (size_t)b * H * s * dr + 1);
  orc_mla_queries(L, xs, b, s, 0, qn, qr);
  float *rows = (float *)malloc(sizeof(float) * (size_t)b * s * w + 1);
  orc_mla_latent_rows(L, xs, b, s, 0, rows);
  float *ka = (float *)malloc(sizeof(float) * (size_t)b * H * s * dn + 1);
  float *va = (float *)malloc(sizeof(float) * (size_t)b * H * s * dv + 1);
  float *kra = (float *)malloc(sizeof(float) * (size_t)b * H * s * dr + 1);
  orc_decompress_cache(L, rows, b, s, ka, va, kra);
  float *ctx = (float *)malloc(sizeof(float) * (size_t)b * H * s * dv + 1);
  orc_fused_prefill_attn(qn, qr, ka, kra, va, b, H, s, s, dn, dr, dv, H, 0, L->softmax_scale, 1,
                         ctx);
  orc_mla_output(L, ctx, b, s, out);
  if (k) memcpy(k, ka, sizeof(float) * (size_t)b * H * s * dn);
  if (v) memcpy(v, va, sizeof(float) * (size_t)b * H * s * dv);
  if (k_rope) memcpy(k_rope, kra, sizeof(float) * (size_t)b * H * s * dr);
  free(qn); free(qr); free(rows); free(ka); free(va); free(kra); free(ctx);
}

/* ------------------------------------------- absorbed latent decode ------ */

/* Rows are processed in blocks of ORC_RB query rows so that each cache row
 * is read once per block (this is also the CPU baseline's inner loop). */
#define ORC_RB 8

void orc_decode_absorbed(const float *q_lat, const float *q_rope, const float *cache,
                         const int64_t *offsets, const int32_t *lens, int nseq, int M, int r,
                         int dr, double scale, float *out, float *lse) {
  int w = r + dr;
  int nblk = (M + ORC_RB - 1) / ORC_RB;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int sq = 0; sq < nseq; ++sq)
    for (int blk = 0; blk < nblk; ++blk) {
      int T = lens[sq];
      const float *C = cache + (size_t)offsets[sq] * w;
      int m0 = blk * ORC_RB, m1 = m0 + ORC_RB < M ? m0 + ORC_RB : M, nb = m1 - m0;
      float *sc = (float *)malloc(sizeof(float) * (size_t)ORC_RB * (T > 0 ? T : 1));
      double acc[ORC_RB][1024];
      double mx[ORC_RB], sum[ORC_RB];
      for (int i = 0; i < nb; ++i) {
        mx[i] = -INFINITY;
        sum[i] = 0.0;
        for (int c = 0; c < r; ++c) acc[i][c] = 0.0;
      }
      for (int t = 0; t < T; ++t) {
        const float *row = C + (size_t)t * w;
        for (int i = 0; i < nb; ++i) {
          const float *ql = q_lat + ((size_t)sq * M + m0 + i) * r;
          const float *qr = q_rope + ((size_t)sq * M + m0 + i) * dr;
          float a = 0.0f;
          for (int c = 0; c < r; ++c) a += ql[c] * row[c];
          float b2 = 0.0f;
          for (int c = 0; c < dr; ++c) b2 += qr[c] * row[r + c];
          float s = (a + b2) * (float)scale;
          sc[(size_t)i * T + t] = s;
          if (s > mx[i]) mx[i] = s;
        }
      }
      for (int t = 0; t < T; ++t) {
        const float *row = C + (size_t)t * w;
        for (int i = 0; i < nb; ++i) {
          double p = exp((double)sc[(size_t)i * T + t] - mx[i]);
          sum[i] += p;
          for (int c = 0; c < r; ++c) acc[i][c] += p * row[c];
        }
      }
      for (int i = 0; i < nb; ++i) {
        float *o = out + ((size_t)sq * M + m0 + i) * r;
        for (int c = 0; c < r; ++c) o[c] = T > 0 ? (float)(acc[i][c] / sum[i]) : 0.0f;
        if (lse) lse[(size_t)sq * M + m0 + i] = T > 0 ? (float)(mx[i] + log(sum[i])) : -INFINITY;
      }
      free(sc);
    }
}

void orc_decode_absorbed_f64(const float *q_lat, const float *q_rope, const float *cache,
                             const int64_t *offsets, const int32_t *lens, int nseq, int M, int r,
                             int dr, double scale, double *out, double *lse) {
  int w = r + dr;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int sq = 0; sq < nseq; ++sq)
    for (int m = 0; m < M; ++m) {
      int T = lens[sq];
      const float *C = cache + (size_t)offsets[sq] * w;
      const float *ql = q_lat + ((size_t)sq * M + m) * r;
      const float *qr = q_rope + ((size_t)sq * M + m) * dr;
      double *sc = (double *)malloc(sizeof(double) * (size_t)(T > 0 ? T : 1));
      double mx = -INFINITY;
      for (int t = 0; t < T; ++t) {
        const float *row = C + (size_t)t * w;
        double a = 0.0;
        for (int c = 0; c < r; ++c) a += (double)ql[c] * row[c];
        for (int c = 0; c < dr; ++c) a += (double)qr[c] * row[r + c];
        sc[t] = a * scale;
        if (sc[t] > mx) mx = sc[t];
      }
      double sum = 0.0;
      for (int t = 0; t < T; ++t) {
        sc[t] = exp(sc[t] - mx);
        sum += sc[t];
      }
      double *o = out + ((size_t)sq * M + m) * r;
      for (int c = 0; c < r; ++c) {
        double a = 0.0;
        for (int t = 0; t < T; ++t) a += sc[t] * C[(size_t)t * w + c];
        o[c] = T > 0 ? a / sum : 0.0;
      }
      if (lse) lse[(size_t)sq * M + m] = T > 0 ? mx + log(sum) : -INFINITY;
      free(sc);
    }
}

/* q_lat[h][c] = sum_j q_nope[h][j] * Wkvb[h(dn+dv) + j][c] */
void orc_absorb_q(const orc_mla_layer *L, const float *q_nope, long n, float *q_lat) {
  int H = L->heads, dn = L->dn, dv = L->dv, r = L->r;
#pragma omp parallel for collapse(2) schedule(static)
  for (long i = 0; i < n; ++i)
    for (int hh = 0; hh < H; ++hh) {
      const float *qn = q_nope + ((size_t)i * H + hh) * dn;
      const float *W = L->wkvb + (size_t)hh * (dn + dv) * r;
      float *o = q_lat + ((size_t)i * H + hh) * r;
      for (int c = 0; c < r; ++c) {
        double a = 0.0;
        for (int j = 0; j < dn; ++j) a += (double)qn[j] * W[(size_t)j * r + c];
        o[c] = (float)a;
      }
    }
}

/* o[h][j] = sum_c Wkvb[h(dn+dv) + dn + j][c] * o_lat[h][c] + bkvb[h(dn+dv) + dn + j] */
void orc_unabsorb_out(const orc_mla_layer *L, const float *o_lat, long n, float *o) {
  int H = L->heads, dn = L->dn, dv = L->dv, r = L->r;
#pragma omp parallel for collapse(2) schedule(static)
  for (long i = 0; i < n; ++i)
    for (int hh = 0; hh < H; ++hh) {
      const float *ol = o_lat + ((size_t)i * H + hh) * r;
      const float *W = L->wkvb + ((size_t)hh * (dn + dv) + dn) * r;
      const float *bb = L->bkvb ? L->bkvb + (size_t)hh * (dn + dv) + dn : NULL;
      float *oo = o + ((size_t)i * H + hh) * dv;
      for (int j = 0; j < dv; ++j) {
        double a = 0.0;
        for (int c = 0; c < r; ++c) a += (double)W[(size_t)j * r + c] * ol[c];
        oo[j] = (float)(a + (bb ? bb[j] : 0.0));
      }
    }
}

void orc_mla_forward_with_latent(const orc_mla_layer *L, const float *xs, int b, int s,
                                 const float *latent, int Tc, float *out, float *new_rows) {
  int H = L->heads, dn = L->dn, dr = L->dr, dv = L->dv, r = L->r, w = r + dr;
  int T = Tc + s, M = s * H;
  float *qn = (float *)malloc(sizeof(float) * (size_t)b * H * s * dn + 1);
  float *qr = (float *)malloc(sizeof(float) * (size_t)b * H * s * dr + 1);
  orc_mla_queries(L, xs, b, s, Tc, qn, qr);
  /* reorder [b,H,s,.] -> [b,s,H,.] query rows (row m = i*H + h) */
  float *qn2 = (float *)malloc(sizeof(float) * (size_t)b * M * dn + 1);
  float *qr2 = (float *)malloc(sizeof(float) * (size_t)b * M * dr + 1);
  for (int bi = 0; bi < b; ++bi)
    for (int hh = 0; hh < H; ++hh)
      for (int i = 0; i < s; ++i) {
        size_t src = ((size_t)bi * H + hh) * s + i, dst = ((size_t)bi * s + i) * H + hh;
        memcpy(qn2 + dst * dn, qn + src * dn, sizeof(float) * dn);
        memcpy(qr2 + dst * dr, qr + src * dr, sizeof(float) * dr);
      }
  float *ql = (float *)malloc(sizeof(float) * (size_t)b * M * r + 1);
  orc_absorb_q(L, qn2, (long)b * s, ql);
  float *rows = (float *)malloc(sizeof(float) * (size_t)b * s * w + 1);
  orc_mla_latent_rows(L, xs, b, s, Tc, rows);
  float *all = (float *)malloc(sizeof(float) * (size_t)b * T * w + 1);
  for (int bi = 0; bi < b; ++bi) {
    if (Tc > 0)
      memcpy(all + (size_t)bi * T * w, latent + (size_t)bi * Tc * w, sizeof(float) * (size_t)Tc * w);
    memcpy(all + ((size_t)bi * T + Tc) * w, rows + (size_t)bi * s * w, sizeof(float) * (size_t)s * w);
  }
  int64_t *offs = (int64_t *)malloc(sizeof(int64_t) * (size_t)b);
  int32_t *lens = (int32_t *)malloc(sizeof(int32_t) * (size_t)b);
  for (int bi = 0; bi < b; ++bi) {
    offs[bi] = (int64_t)bi * T;
    lens[bi] = T;
  }
  float *olat = (float *)malloc(sizeof(float) * (size_t)b * M * r + 1);
  orc_decode_absorbed(ql, qr2, all, offs, lens, b, M, r, dr, L->softmax_scale, olat, NULL);
  float *o = (float *)malloc(sizeof(float) * (size_t)b * M * dv + 1);
  orc_unabsorb_out(L, olat, (long)b * s, o); /* [b, s, H, dv] == [b, s, H*dv] */
  orc_linear(o, b * s, H * dv, L->wo, L->bo, L->hidden, out);
  if (new_rows) memcpy(new_rows, rows, sizeof(float) * (size_t)b * s * w);
  free(qn); free(qr); free(qn2); free(qr2); free(ql); free(rows); free(all); free(offs);
  free(lens); free(olat); free(o);
}
