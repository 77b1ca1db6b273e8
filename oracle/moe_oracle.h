/*
 * moe_oracle.h -- CPU restatement of qmoe-rs's 2-bit packed MoE path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker); built into liboracle.so with the
 * attention oracle.  Parity status of each function:
 *   orc_fused_dequantize_and_dot  pinned: the reference's known-answer test
 *       (src/simd.rs:51-65) and closed forms (all codes 0/1/2/3).
 *   orc_packed_forward            pinned: a dense float64 matmul of the
 *       unpacked weights (numpy, independent code path).
 *   orc_moe_forward               pinned: a float64 numpy restatement with a
 *       stable arg-sort, tie cases and the top_k = num_experts closed form.
 */
#ifndef QMLA_MOE_ORACLE_H
#define QMLA_MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fused_dequantize_and_dot (src/simd.rs:6-45): codes w = (byte >> 2q) & 3
 * map to w - 1; four f32 lane sums over min(n_bytes, n_act / 4) bytes, then
 * the lane sum times scale.                                               */
float orc_fused_dequantize_and_dot(const uint8_t *packed, size_t n_bytes, const float *act,
                                   size_t n_act, float scale);

/* PackedQMoETensor::forward_simd (src/tensor.rs:64-95): out[b][i] =
 * dot(row i of packed [out_f, in_f / 4], x[b]) * scales[i].              */
void orc_packed_forward(const uint8_t *packed, const float *scales, int out_f, int in_f,
                        const float *x, int batch, float *out);

/* QMoELayer::forward (src/moe.rs:40-130).  Expert e's tensors are slices of
 * gate_packed/up_packed [E, I, H/4], down_packed [E, H, I/4] and the scale
 * arrays [E, I] / [E, H].  top_idx/top_w (nullable, [seq, top_k]) receive
 * the routing in descending-logit order.                                 */
typedef struct {
  int num_experts, top_k, hidden_dim, intermediate_dim;
} orc_moe_config;

void orc_moe_forward(const orc_moe_config *cfg, const float *xs, int seq_len,
                     const float *gate_weight, const uint8_t *gate_packed,
                     const float *gate_scales, const uint8_t *up_packed, const float *up_scales,
                     const uint8_t *down_packed, const float *down_scales, float *out,
                     int32_t *top_idx, float *top_w);

#ifdef __cplusplus
}
#endif
#endif
