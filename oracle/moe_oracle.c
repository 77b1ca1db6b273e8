/*
 * moe_oracle.c -- CPU restatement of qmoe-rs's 2-bit packed MoE path
 * (src/simd.rs, src/tensor.rs, src/moe.rs).
 *
 * TEST INFRASTRUCTURE ONLY (the checker).  Loaded by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg; never by the
 * product library.  Parity status per function is listed in moe_oracle.h.
 * Built with -ffp-contract=off: the reference's `sum += w * a` is a separate
 * f32 multiply and add.
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* src/simd.rs:6-45.  Lane q of the f32x4 accumulator sums code q of every
 * byte times activation 4i + q (:17-41); reduce_sum adds the lanes in lane
 * order (:44). */
float orc_fused_dequantize_and_dot(const uint8_t *packed, size_t n_bytes, const float *act,
                                   size_t n_act, float scale) {
  size_t n = n_bytes < n_act / 4 ? n_bytes : n_act / 4; /* :15 */
  float lane[4] = {0.f, 0.f, 0.f, 0.f};
  for (size_t i = 0; i < n; ++i) {
    uint8_t byte = packed[i];
    for (int q = 0; q < 4; ++q) {
      float w = (float)((byte >> (2 * q)) & 3) - 1.0f; /* :22-31 */
      float p = w * act[4 * i + q];
      lane[q] = lane[q] + p; /* :40 */
    }
  }
  float s = 0.f;
  for (int q = 0; q < 4; ++q) s = s + lane[q];
  return s * scale;
}

/* src/tensor.rs:64-95 (forward_simd_raw :99-121 is the same loop). */
void orc_packed_forward(const uint8_t *packed, const float *scales, int out_f, int in_f,
                        const float *x, int batch, float *out) {
  size_t bpr = (size_t)in_f / 4; /* :74 */
  for (int b = 0; b < batch; ++b)
    for (int i = 0; i < out_f; ++i)
      out[(size_t)b * out_f + i] = orc_fused_dequantize_and_dot(
          packed + (size_t)i * bpr, bpr, x + (size_t)b * in_f, (size_t)in_f, scales[i]);
}

typedef struct {
  int idx;
  float v;
} orc_logit;

/* sort_by(b.1.partial_cmp(&a.1)) is a stable descending sort (src/moe.rs:71):
 * equal logits keep ascending expert order. */
static int orc_logit_desc(const void *pa, const void *pb) {
  const orc_logit *a = (const orc_logit *)pa, *b = (const orc_logit *)pb;
  if (a->v > b->v) return -1;
  if (a->v < b->v) return 1;
  return a->idx - b->idx;
}

/* SwiGLU expert on one token (src/moe.rs:100-119); writes hidden_dim values. */
static void orc_expert(const orc_moe_config *c, int e, const float *x, const uint8_t *gate_packed,
                       const float *gate_scales, const uint8_t *up_packed, const float *up_scales,
                       const uint8_t *down_packed, const float *down_scales, float *g, float *u,
                       float *y) {
  int H = c->hidden_dim, I = c->intermediate_dim;
  size_t gsz = (size_t)I * (H / 4), dsz = (size_t)H * (I / 4);
  orc_packed_forward(gate_packed + e * gsz, gate_scales + (size_t)e * I, I, H, x, 1, g); /* :102 */
  orc_packed_forward(up_packed + e * gsz, up_scales + (size_t)e * I, I, H, x, 1, u);     /* :103 */
  for (int i = 0; i < I; ++i) {
    float gi = g[i];
    float swish = gi * (1.0f / (1.0f + expf(-gi))); /* :113 */
    g[i] = swish * u[i];                            /* :114 */
  }
  orc_packed_forward(down_packed + e * dsz, down_scales + (size_t)e * H, H, I, g, 1, y); /* :118 */
}

/* src/moe.rs:40-130. */
void orc_moe_forward(const orc_moe_config *c, const float *xs, int T, const float *gate_weight,
                     const uint8_t *gate_packed, const float *gate_scales,
                     const uint8_t *up_packed, const float *up_scales,
                     const uint8_t *down_packed, const float *down_scales, float *out,
                     int32_t *top_idx, float *top_w) {
  int E = c->num_experts, K = c->top_k, H = c->hidden_dim, I = c->intermediate_dim;
  memset(out, 0, sizeof(float) * (size_t)T * H); /* :47, :86 */
  if (E == 0) return;
  orc_logit *lg = (orc_logit *)malloc(sizeof(orc_logit) * (size_t)E);
  /* bins, stored per token: sel[t][j] = (expert, weight) */
  int32_t *sel = (int32_t *)malloc(sizeof(int32_t) * ((size_t)T * K + 1));
  float *selw = (float *)malloc(sizeof(float) * ((size_t)T * K + 1));
  for (int t = 0; t < T; ++t) {
    const float *x = xs + (size_t)t * H;
    for (int e = 0; e < E; ++e) { /* :51 gate logits = xs . gate_weight^T */
      const float *w = gate_weight + (size_t)e * H;
      float s = 0.f;
      for (int h = 0; h < H; ++h) s = s + x[h] * w[h];
      lg[e].idx = e;
      lg[e].v = s;
    }
    qsort(lg, (size_t)E, sizeof(orc_logit), orc_logit_desc); /* :64-71 */
    float mx = -INFINITY;
    for (int e = 0; e < E; ++e) mx = fmaxf(mx, lg[e].v); /* :74 */
    float sum = 0.f;
    for (int e = 0; e < E; ++e) sum = sum + expf(lg[e].v - mx); /* :75 */
    for (int j = 0; j < K; ++j) {                                /* :76-81 */
      sel[(size_t)t * K + j] = lg[j].idx;
      selw[(size_t)t * K + j] = expf(lg[j].v - mx) / sum;
      if (top_idx) top_idx[(size_t)t * K + j] = lg[j].idx;
      if (top_w) top_w[(size_t)t * K + j] = selw[(size_t)t * K + j];
    }
  }
  float *g = (float *)malloc(sizeof(float) * ((size_t)I + 1));
  float *u = (float *)malloc(sizeof(float) * ((size_t)I + 1));
  float *y = (float *)malloc(sizeof(float) * ((size_t)H + 1));
  for (int e = 0; e < E; ++e)   /* :89 experts in index order */
    for (int t = 0; t < T; ++t) /* :96 a bin holds its tokens in order */
      for (int j = 0; j < K; ++j) {
        if (sel[(size_t)t * K + j] != e) continue;
        orc_expert(c, e, xs + (size_t)t * H, gate_packed, gate_scales, up_packed, up_scales,
                   down_packed, down_scales, g, u, y);
        float w = selw[(size_t)t * K + j];
        float *o = out + (size_t)t * H;
        for (int h = 0; h < H; ++h) o[h] = o[h] + y[h] * w; /* :122-125 */
      }
  free(lg); free(sel); free(selw); free(g); free(u); free(y);
}
