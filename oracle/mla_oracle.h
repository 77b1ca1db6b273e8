/*
 * mla_oracle.h -- CPU restatement of qmoe-rs's MLA attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker for the HIP
 * implementation in qmoe-rs_amd/.  Only tests/, __graft_entry__.smoke() and
 * the cpu_baseline leg of bench.py may load it; the product path never links,
 * loads or falls back to it.
 *
 * Every function cites the reference file:line it restates (paths are
 * relative to the qmoe-rs source tree).  fp32 functions follow the
 * reference's operation order; *_f64 functions are textbook double-precision
 * twins used to pin the fp32 restatement and the GPU kernels.
 *
 * Layout conventions (all row-major, contiguous):
 *   attention tensors  [b, h, s, d]          (the reference's transposed views)
 *   activations        [b, s, hidden]
 *   Linear weight      [out, in]  (y = x W^T + b, candle_nn::Linear)
 *   latent cache row   [c_kv (r) | k_pe (dr)]  (k_pe already roped)
 *
 * Parity status per function is recorded next to each declaration:
 *   "pinned by: ..." names the independent checks in tests/test_oracle.py.
 */
#ifndef QMLA_ORACLE_H
#define QMLA_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- RNG ----
 * Portable deterministic generator shared by tests, fixtures and bench:
 * SplitMix64 -> Box-Muller in fp64 -> f32.  Element i of a tensor seeded
 * with `seed` depends only on (seed, i), so slices can be regenerated.
 * pinned by: SplitMix64 published test vector; moments of 1e6 draws.      */
uint64_t orc_splitmix64_at(uint64_t seed, uint64_t i);
void orc_fill_normal(float *out, size_t n, uint64_t seed, double mean, double std_);
void orc_fill_uniform_int(int32_t *out, size_t n, uint64_t seed, int32_t lo, int32_t hi);
/* round-to-nearest-even f32 -> bf16 (NaN kept quiet) and back.
 * pinned by: hand-picked tie/overflow cases.                              */
uint16_t orc_f32_to_bf16(float x);
float orc_bf16_to_f32(uint16_t x);
void orc_to_bf16(const float *in, uint16_t *out, size_t n);
void orc_round_bf16(const float *in, float *out, size_t n);

/* ------------------------------------------------------- scalar helpers -- */
/* yarn_get_mscale, src/model.rs:46-52.  pinned by: closed-form constants.  */
double orc_yarn_get_mscale(double scale, double mscale);
/* MlaAttention::new rope_mscale / softmax_scale, src/model.rs:160-173.
 * pinned by: closed-form constants 1.085726399 / 0.114721387.             */
void orc_mla_scales(int qk_nope, int qk_rope, double *rope_mscale, double *softmax_scale);
/* tile_size, src/attention_kernel.rs:3-11.  pinned by: boundary values.    */
int orc_tile_size(int seq_len);

/* ----------------------------------------------------------------- RoPE --
 * precompute_rope_freqs, src/model.rs:55-66: out [seq_len, d] =
 * [cos(pos*inv_freq)*mscale | sin(pos*inv_freq)*mscale], inv_freq computed
 * 1.0f / (float)10000^(2i/d).  Rows [pos0, pos0+n) are produced.
 * pinned by: position-0 identity, pair-norm scaling, relative-position
 * invariance of <rope(q,m), rope(k,n)>.                                   */
void orc_rope_table(int pos0, int n, int d, double mscale, float *out);
/* apply_rope, src/model.rs:70-84: x [outer, s, d] with interleaved pairs
 * (2i, 2i+1); table [s, d] as above.  In-place allowed (out == x).        */
void orc_apply_rope(const float *x, float *out, int outer, int s, int d, const float *table);

/* ------------------------------------------------------ dense building --
 * candle_nn::Linear (x W^T + b) as used by every projection in
 * src/model.rs:126-146.  pinned by: fp64 twin on random data.             */
void orc_linear(const float *x, int rows, int in, const float *W, const float *b, int out,
                float *y);
/* candle_nn::LayerNorm, src/model.rs:136 (eps 1e-6, weight and bias):
 * (x - mean) / sqrt(var + eps) * w + b with biased variance.
 * pinned by: zero-mean/unit-variance invariant and a hand-computed vector. */
void orc_layer_norm(const float *x, int rows, int n, const float *w, const float *b, double eps,
                    float *y);
/* candle_nn::ops::softmax over the last dim (max-subtract, exp, sum, div).
 * pinned by: uniform rows, one-hot limit.                                 */
void orc_softmax_rows(float *x, long rows, int n);

/* ------------------------------------------------------------ attention --
 * reference_eager_attn, src/attention_kernel.rs:110-134 (also the intended
 * math of eager_prefill_attn :34-57): softmax(q k^T * scale [+ mask]) v,
 * causal mask -1e18 where row < col.  q,k [b,h,s,d], v [b,h,s,dv].
 * pinned by: fp64 brute force, closed forms (row 0 == v[0]; q = 0 gives
 * prefix means), key-permutation invariance.                              */
void orc_reference_eager_attn(const float *q, const float *k, const float *v, int b, int h, int s,
                              int d, int dv, double scale, int causal, float *out);

/* fused_prefill_attn, src/attention_kernel.rs:64-107, generalised:
 *   scores = (q_nope k^T + q_rope k_rope^T) * scale, then the causal mask of
 *   make_causal_mask (:14-31) with absolute query row = q_offset + i and key
 *   column j masked (-1e18) when row < col, softmax, times v; queries are
 *   processed in tiles of tile_size(sq) rows (:79-104).
 * Shapes: q_nope [b,h,sq,dn], q_rope [b,h,sq,dr], k [b,h,sk,dn],
 *         k_rope [b,krh,sk,dr] (krh = 1 broadcasts one rope key to all
 *         heads, krh = h is the reference's expanded layout), v [b,h,sk,dv],
 *         out [b,h,sq,dv].  The reference itself is q_offset = 0, sq = sk.
 * pinned by: the reference's own tiling-invariance cases
 * (:169-197, same generator, same tolerance) against the eager form, and
 * the fp64 twin below.                                                    */
void orc_fused_prefill_attn(const float *q_nope, const float *q_rope, const float *k,
                            const float *k_rope, const float *v, int b, int h, int sq, int sk,
                            int dn, int dr, int dv, int krh, int q_offset, double scale,
                            int causal, float *out);
/* Double-precision brute force of the same function (no tiling).          */
void orc_prefill_attn_f64(const float *q_nope, const float *q_rope, const float *k,
                          const float *k_rope, const float *v, int b, int h, int sq, int sk,
                          int dn, int dr, int dv, int krh, int q_offset, double scale, int causal,
                          double *out);

/* --------------------------------------------------- MLA layer (ref) ----- */
typedef struct {
  int hidden, heads, dn, dr, dv, r;
  const float *wq, *bq;     /* q_proj            [H*(dn+dr), hidden]  src/model.rs:126-130 */
  const float *wkva, *bkva; /* kv_a_proj_with_mqa [r+dr, hidden]      src/model.rs:131-135 */
  const float *ln_w, *ln_b; /* kv_a_layernorm    [r]                  src/model.rs:136     */
  const float *wkvb, *bkvb; /* kv_b_proj         [H*(dn+dv), r]       src/model.rs:137-141 */
  const float *wo, *bo;     /* o_proj            [hidden, H*dv]       src/model.rs:142-146 */
  double rope_mscale, softmax_scale, ln_eps;
} orc_mla_layer;

/* compute_kv, src/model.rs:178-190, applied to latent rows c [n, r]:
 * k [n, H, dn], v [n, H, dv] (token-major, as kv_b_proj's reshape).       */
void orc_compute_kv(const orc_mla_layer *L, const float *c, long n, float *k, float *v);

/* Latent rows of the new tokens, src/model.rs:270-273 and :281-288 (the
 * rope part before head broadcast): rows [b, s, r+dr] = [LayerNorm(kv_a[:r])
 * | rope(kv_a[r:], position pos0 + i)].                                    */
void orc_mla_latent_rows(const orc_mla_layer *L, const float *xs, int b, int s, int pos0,
                         float *rows);

/* Expand a latent cache into the reference KVCache tensors
 * (src/model.rs:86-105, filled at :250 / :291): latent [b, T, r+dr] ->
 * k [b,H,T,dn], v [b,H,T,dv], k_rope [b,H,T,dr] (head-broadcast).          */
void orc_decompress_cache(const orc_mla_layer *L, const float *latent, int b, int T, float *k,
                          float *v, float *k_rope);

/* MlaAttention::forward_with_cache, src/model.rs:256-307, reference
 * (decompressed) form.  xs [b, s, hidden]; cache k/v/k_rope [b,H,Tc,.] with
 * Tc cached tokens; out [b, s, hidden].  If new_k/new_v/new_k_rope are
 * non-NULL the appended cache [b,H,Tc+s,.] is written there (KVCache::append,
 * :99-104).  No causal mask among the s new tokens (:297-302).            */
void orc_mla_forward_with_cache(const orc_mla_layer *L, const float *xs, int b, int s,
                                const float *k, const float *v, const float *k_rope, int Tc,
                                float *out, float *new_k, float *new_v, float *new_k_rope);

/* MlaAttention::forward_prefill, src/model.rs:193-253 (fused_attn branch,
 * :221-225).  xs [b, s, hidden] -> out [b, s, hidden]; optional cache out
 * k [b,H,s,dn], v [b,H,s,dv], k_rope [b,H,s,dr].                          */
void orc_mla_forward_prefill(const orc_mla_layer *L, const float *xs, int b, int s, float *out,
                             float *k, float *v, float *k_rope);

/* ------------------------------------------- absorbed latent decode ------
 * The absorption identity (no reference code; it is an exact algebraic
 * rewrite of src/model.rs:297-303): for head h and token t,
 *   s_t = scale * (q_lat . c_t + q_rope . kpe_t),  o_lat = sum softmax(s)_t c_t
 * q_lat [nseq, M, r], q_rope [nseq, M, dr] (M query rows per sequence: heads
 * x new tokens, every row attends every cached token, as :297-302);
 * cache rows [*, r+dr] fp32, sequence i occupying rows
 * [offsets[i], offsets[i] + lens[i]).  out [nseq, M, r], lse [nseq, M]
 * (natural log of the softmax denominator incl. the max), may be NULL.
 * pinned by: fp64 twin; equality with the decompressed reference path
 * through orc_absorb_q / orc_unabsorb_out (tests/test_oracle.py).         */
void orc_decode_absorbed(const float *q_lat, const float *q_rope, const float *cache,
                         const int64_t *offsets, const int32_t *lens, int nseq, int M, int r,
                         int dr, double scale, float *out, float *lse);
void orc_decode_absorbed_f64(const float *q_lat, const float *q_rope, const float *cache,
                             const int64_t *offsets, const int32_t *lens, int nseq, int M, int r,
                             int dr, double scale, double *out, double *lse);
/* q_lat[h] = W_UK^h^T q_nope[h]  (W_UK^h = kv_b_proj rows [h(dn+dv), h(dn+dv)+dn)).
 * q_nope [n, H, dn] -> q_lat [n, H, r].                                    */
void orc_absorb_q(const orc_mla_layer *L, const float *q_nope, long n, float *q_lat);
/* o[h] = W_UV^h o_lat[h] + b_V^h -> [n, H, dv]                            */
void orc_unabsorb_out(const orc_mla_layer *L, const float *o_lat, long n, float *o);

/* Absorbed-form MLA decode step (the form the GPU layer computes):
 * same inputs/outputs as orc_mla_forward_with_cache but over a latent cache
 * latent [b, Tc, r+dr]; new latent rows are written to new_rows [b, s, r+dr]
 * if non-NULL.                                                              */
void orc_mla_forward_with_latent(const orc_mla_layer *L, const float *xs, int b, int s,
                                 const float *latent, int Tc, float *out, float *new_rows);

/* OpenMP thread count used by the parallel loops above (for reporting).   */
int orc_num_threads(void);
void orc_set_num_threads(int n); /* OpenMP threads for later calls (n > 0) */

#ifdef __cplusplus
}
#endif
#endif
