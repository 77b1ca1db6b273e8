// layer.hip -- MlaAttention (src/model.rs:107-307) with device-resident
// weights, in f32.
//
// forward_with_cache (src/model.rs:256-307) runs in absorbed form over the
// latent cache:
//   q = xs Wq^T + bq; q_rope roped at positions len + i       (:263-267)
//   kv_a = xs Wkva^T + bkva; c = LayerNorm(kv_a[:r]);
//   k_pe = rope(kv_a[r:])                                      (:270-288)
//   append [c | k_pe] to the latent cache                      (:291)
//   q_lat[h] = W_UK^h^T q_nope[h]       (W_UK^h = kv_b rows [h(dn+dv), +dn))
//   o_lat = absorbed attention core (decode.hip)               (:294-303)
//   o[h] = W_UV^h o_lat[h] + b_V^h ; out = o Wo^T + bo         (:303-306)
// The b_K part of kv_b's bias adds q_nope . b_K^h to every score of a row,
// a constant that softmax removes, so it never enters the absorbed form.
//
// forward_prefill (src/model.rs:193-253) decompresses K and V for the new
// tokens (compute_kv, :178-190) and runs the causal prefill kernel with the
// rope key stored once (k_rope_heads = 1) instead of broadcast per head.

#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <functional>
#include <mutex>
#include <new>
#include <thread>
#include <vector>

#include <rocblas/rocblas.h>

#include "latent_rows.hpp"

struct qmla_layer {
  qmla_layer_config cfg{};
  float *wq = nullptr, *bq = nullptr, *wkva = nullptr, *bkva = nullptr, *ln_w = nullptr,
        *ln_b = nullptr, *wkvb = nullptr, *bkvb = nullptr, *wo = nullptr, *bo = nullptr;
  float *inv_freq = nullptr;  // [dr / 2], src/model.rs:56-58
  // Fragment-major bf16 hi/lo halves of the decode-step projections
  // (skinny_gemm.hip), packed from:
  //   w1   [H(dn+dr) + r + dr][hidden]  q_proj rows, then kv_a_proj_with_mqa rows
  //   wuk  [H][r][dn]                   W_UK^h transposed (kv_b rows h(dn+dv) .. +dn)
  //   wuv  [H][dv][r]                   W_UV^h (kv_b rows h(dn+dv)+dn .. +dv)
  //   wo   [hidden][H dv]               o_proj
  //   wkvb [H(dn+dv)][r]               kv_b_proj (the prefill's compute_kv)
  void *w1f = nullptr, *wukf = nullptr, *wuvf = nullptr, *wof = nullptr, *wkvbf = nullptr;
  float *b1 = nullptr;   // [bq | bkva]
  float *buv = nullptr;  // [H][dv]: b_V^h
  bool skinny = false;   // the split weights exist (every K a multiple of 16)
  // bf16 operands in the hand-written projection kernels (the weights' hi
  // halves and bf16 activations, f32 accumulation); qmla_layer_set_
  // projection_dtype.  The rocBLAS paths and the materialise call stay exact.
  bool proj_bf16 = false;
  // Split-form rows of wq, wkva, wkvb and wo for the GEMMs of products with
  // many rows: row n of a [N][K] weight becomes [w_hi | w_hi | w_lo | b_hi,
  // b_lo, 0...] in bf16 (split_cols(K) columns; hi = bf16(v), lo = bf16(v -
  // hi); the bias columns are 0 without a bias).
  uint16_t *wq_x = nullptr, *wkva_x = nullptr, *wkvb_x = nullptr, *wo_x = nullptr;
  std::vector<void *> allocs;
  // rocBLAS handles for the GEMM path (prefill, and decode shapes the skinny
  // kernel does not take).  A call takes a free one and sets its stream, so
  // calls on different streams run concurrently up to kBlasHandles.
  static constexpr int kBlasHandles = 4;
  struct BlasSlot {
    rocblas_handle h = nullptr;
    std::mutex mu;
  };
  mutable std::array<BlasSlot, kBlasHandles> blas;
};

namespace qmla {

namespace {

// ------------------------------------------------------------ f32 GEMM
constexpr int kSkinnyRows = 64;  // products with at most this many rows go split-K
// The projections are plain GEMMs and go to rocBLAS (full f32: no reduced-
// precision math mode is set on the handle).
// C[z][m][n] = sum_k A[z][m][k] * B[z][k][n] (+ bias[z][n]); B is read as
// B[k][n] = Bt[n][k] when trans_b (the Linear layout W[out][in]).  All
// matrices are row-major with leading dimensions ld* and per-z strides s*.
struct GemmArgs {
  const float *A;
  const float *B;
  const float *bias;
  float *C;
  int M, N, K;
  int64_t lda, ldb, ldc;
  int64_t sA, sB, sC, sBias;  // per-z strides
};

// C[z][m][n] = bias[z][n], ahead of a GEMM that accumulates with beta = 1
// (grid: x over the M * N elements of one z, y over z).
__global__ __launch_bounds__(256) void k_bias_fill(float *__restrict__ C,
                                                   const float *__restrict__ bias, int64_t MN,
                                                   int N, int64_t ldc, int64_t sC,
                                                   int64_t sBias) {
  const int64_t z = blockIdx.y;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= MN) return;
  const int64_t m = i / N, n = i % N;
  C[z * sC + m * ldc + n] = bias[z * sBias + n];
}

// Row-major C = A op(B) is column-major C^T = op(B)^T A^T: rocBLAS gets
// (m, n, k) = (N, M, K) with B as its first operand.
qmla_status gemm(const qmla_layer *L, const GemmArgs &g, int batch, bool trans_b, hipStream_t s) {
  if (g.M == 0 || g.N == 0) return QMLA_OK;
  const int64_t MN = (int64_t)g.M * g.N;
  QMLA_REQUIRE(batch <= 65535 && (MN + 255) / 256 <= 0x7fffffff, QMLA_ERR_SHAPE,
               "GEMM too large");
  float beta = 0.f;
  if (g.bias) {
    dim3 grid((unsigned)((MN + 255) / 256), batch);
    k_bias_fill<<<grid, dim3(256), 0, s>>>(g.C, g.bias, MN, g.N, g.ldc, g.sC, g.sBias);
    QMLA_LAUNCH_CHECK("k_bias_fill");
    beta = 1.f;
  }
  const float one = 1.f;
  // a free handle, or (all busy) the one this thread maps to; the handle's
  // stream is set per call
  qmla_layer::BlasSlot *slot = nullptr;
  std::unique_lock<std::mutex> lock;
  for (auto &b : L->blas) {
    std::unique_lock<std::mutex> l(b.mu, std::try_to_lock);
    if (l.owns_lock()) {
      slot = &b;
      lock = std::move(l);
      break;
    }
  }
  if (!slot) {
    slot = &L->blas[std::hash<std::thread::id>{}(std::this_thread::get_id()) %
                    qmla_layer::kBlasHandles];
    lock = std::unique_lock<std::mutex>(slot->mu);
  }
  rocblas_status st = rocblas_set_stream(slot->h, s);
  if (st == rocblas_status_success)
    st = rocblas_sgemm_strided_batched(
        slot->h, trans_b ? rocblas_operation_transpose : rocblas_operation_none,
        rocblas_operation_none, g.N, g.M, g.K, &one, g.B, (rocblas_int)g.ldb, g.sB, g.A,
        (rocblas_int)g.lda, g.sA, &beta, g.C, (rocblas_int)g.ldc, g.sC, batch);
  QMLA_REQUIRE(st == rocblas_status_success, QMLA_ERR_HIP, "rocBLAS sgemm: %s",
               rocblas_status_to_string(st));
  return QMLA_OK;
}

// K slices for a skinny product (few rows, long K): rocBLAS tiles such a
// GEMM over N only, which leaves most of the device idle (32-48 workgroups
// for the decode-step projections).  Splitting K into S slices of >= 256
// multiplies the grid by S; the slices' partial products are then summed.
inline int split_k_slices(int M, int K) {
  int S = 1;
  if (M <= kSkinnyRows)
    while (S < 16 && K % (2 * S) == 0 && K / (2 * S) >= 256) S *= 2;
  return S;
}

// y[m][n] = bias[n] + sum_s part[s][m][n], in slice order (deterministic).
__global__ __launch_bounds__(256) void k_split_k_sum(const float *__restrict__ part, int S,
                                                     int64_t MN, int N,
                                                     const float *__restrict__ bias,
                                                     float *__restrict__ y) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= MN) return;
  float acc = bias ? bias[i % N] : 0.f;
  for (int s = 0; s < S; ++s) acc += part[s * MN + i];
  y[i] = acc;
}

// y = x W^T + b for x [M, K], W [N, K] (candle_nn::Linear).  Skinny
// products with room in `part` (S * M * N floats) go split-K.
qmla_status linear(const qmla_layer *L, const float *x, int M, int K, const float *W,
                   const float *b, int N, float *y, hipStream_t s, float *part = nullptr,
                   size_t part_elems = 0) {
  const int S = split_k_slices(M, K);
  if (S > 1 && part && (size_t)S * M * N <= part_elems) {
    const int KS = K / S;
    // slice z: part[z] = x[:, z KS : (z+1) KS] W[:, z KS : (z+1) KS]^T
    GemmArgs g{x, W, nullptr, part, M, N, KS, K, K, N, KS, KS, (int64_t)M * N, 0};
    QMLA_TRY(gemm(L, g, S, true, s));
    const int64_t MN = (int64_t)M * N;
    k_split_k_sum<<<dim3((unsigned)((MN + 255) / 256)), dim3(256), 0, s>>>(part, S, MN, N, b, y);
    QMLA_LAUNCH_CHECK("k_split_k_sum");
    return QMLA_OK;
  }
  GemmArgs g{x, W, b, y, M, N, K, K, K, N, 0, 0, 0, 0};
  return gemm(L, g, 1, true, s);
}


// ------------------------------------------------------- split bf16 GEMM
// A product with many rows runs on bf16 GEMMs with f32 accumulation instead
// of an f32 GEMM:  x w = x_hi w_hi + x_lo w_hi + x_hi w_lo, with hi =
// bf16(v) (round to nearest even) and lo = bf16(v - hi) for both operands.
// The dropped x_lo w_lo and the bits past lo keep ~2^-16 of each product,
// the same f32-exact form as the skinny decode-step GEMM.  The three
// products and the bias are one GEMM over K' = split_cols(K) columns:
//   x' = [x_hi | x_lo | x_hi | 1, 1, 0...],  w' = [w_hi | w_hi | w_lo | b_hi, b_lo, 0...]
// so the output is written once.  On this part bf16 GEMMs run ~5-10x
// faster than f32 ones at prefill sizes.
constexpr int kSplitRows = 256;  // products with at least this many rows split

// 3K columns of halves, the two bias columns, zeros up to a multiple of 64
// (the GEMM kernels' K tile).
__host__ __device__ inline int split_cols(int K) { return (3 * K + 2 + 63) / 64 * 64; }

// x'[m] (split_cols(K) bf16 per row, contiguous) from x[m * ldx + k].
__global__ __launch_bounds__(256) void k_split_rows(const float *__restrict__ x, int64_t ldx,
                                                    int64_t M, int K, uint16_t *__restrict__ xs) {
  const int KX = split_cols(K);
  const int64_t n = M * K;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256) {
    const int64_t m = i / K, k = i - m * K;
    const float v = x[m * ldx + k];
    const uint16_t h = f32_to_bf16_bits(v);
    uint16_t *row = xs + m * KX;
    row[k] = h;
    row[K + k] = f32_to_bf16_bits(v - bf16_bits_to_f32(h));
    row[2 * K + k] = h;
    if (k < KX - 3 * K) row[3 * K + k] = k < 2 ? (uint16_t)0x3f80 : (uint16_t)0;  // 1.0, 1.0, 0...
  }
}

// Bytes of scratch the split of an [M][K] activation needs.
inline size_t split_bytes(int64_t M, int64_t K) {
  return (size_t)M * split_cols((int)K) * sizeof(uint16_t);
}

qmla_status split_act(const float *x, int64_t ldx, int M, int K, void *xs, hipStream_t s) {
  const int64_t n = (int64_t)M * K;
  if (n == 0) return QMLA_OK;
  // k_split_rows writes the pad columns from the first K lanes of a row
  QMLA_REQUIRE(split_cols(K) - 3 * K <= K, QMLA_ERR_SHAPE, "split of K = %d", K);
  const unsigned blocks = (unsigned)std::min<int64_t>((n + 255) / 256, 16384);
  k_split_rows<<<dim3(blocks), dim3(256), 0, s>>>(x, ldx, M, K, static_cast<uint16_t *>(xs));
  QMLA_LAUNCH_CHECK("k_split_rows");
  return QMLA_OK;
}

// A free rocBLAS handle of the layer (or this thread's, when all are busy),
// locked for the caller.
qmla_layer::BlasSlot *take_blas(const qmla_layer *L, std::unique_lock<std::mutex> &lock) {
  for (auto &bs : L->blas) {
    std::unique_lock<std::mutex> l(bs.mu, std::try_to_lock);
    if (l.owns_lock()) {
      lock = std::move(l);
      return &bs;
    }
  }
  auto *slot = &L->blas[std::hash<std::thread::id>{}(std::this_thread::get_id()) %
                        qmla_layer::kBlasHandles];
  lock = std::unique_lock<std::mutex>(slot->mu);
  return slot;
}

// C[z][m][n] = x'[z][m] . w'[z][n] (the split product with its bias), all
// row-major: x' [M][K'] per z at stride sX, w' [N][K'] per z at stride sW
// (ld ldw), C [M][N] (ld ldc) at stride sC, K' = split_cols(K).
qmla_status gemm_split(const qmla_layer *L, const uint16_t *xs, int64_t sX, int M, int K,
                       const uint16_t *wx, int64_t ldw, int64_t sW, int N, float *C, int64_t ldc,
                       int64_t sC, int batch, hipStream_t s) {
  if (M == 0 || N == 0) return QMLA_OK;
  QMLA_REQUIRE(batch >= 1 && batch <= 65535, QMLA_ERR_SHAPE, "GEMM batch %d", batch);
  const int KX = split_cols(K);
  std::unique_lock<std::mutex> lock;
  qmla_layer::BlasSlot *slot = take_blas(L, lock);
  rocblas_status st = rocblas_set_stream(slot->h, s);
  const float one = 1.f, zero = 0.f;
  // row-major C = x' w'^T is column-major C^T = w' x'^T: (m, n, k) = (N, M, K')
  if (st == rocblas_status_success)
    st = rocblas_gemm_strided_batched_ex(
        slot->h, rocblas_operation_transpose, rocblas_operation_none, N, M, KX, &one, wx,
        rocblas_datatype_bf16_r, (rocblas_int)ldw, sW, xs, rocblas_datatype_bf16_r, KX, sX,
        &zero, C, rocblas_datatype_f32_r, (rocblas_int)ldc, sC, C, rocblas_datatype_f32_r,
        (rocblas_int)ldc, sC, batch, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  QMLA_REQUIRE(st == rocblas_status_success, QMLA_ERR_HIP, "rocBLAS gemm_ex: %s",
               rocblas_status_to_string(st));
  return QMLA_OK;
}

// y = x W^T + b: the split form for many rows when the split weight exists
// (x' already in xs when `split` is false), else linear().
qmla_status project(const qmla_layer *L, const float *x, int M, int K, const float *W,
                    const uint16_t *Wx, const float *b, int N, float *y, hipStream_t s,
                    float *part, size_t part_elems, void *xs, bool split = true) {
  if (M >= kSplitRows && K >= 64 && Wx && xs) {
    if (split) QMLA_TRY(split_act(x, K, M, K, xs, s));
    return gemm_split(L, static_cast<const uint16_t *>(xs), 0, M, K, Wx, split_cols(K), 0, N, y,
                      N, 0, 1, s);
  }
  return linear(L, x, M, K, W, b, N, y, s, part, part_elems);
}

// Latent rows of new tokens, written straight into the cache (the append of
// src/model.rs:99-104 fused in): one block per token (latent_rows.hpp).
__global__ __launch_bounds__(256) void k_latent_rows(LatentRowsArgs a) {
  extern __shared__ float lds[];  // latent_row_lds_bytes(r, dr)
  latent_row(a, blockIdx.x, lds);
}

// forward_prefill's latent rows (src/model.rs:206-219), one wave per token:
// the cache row [LayerNorm(c) | rope(k_pe)] at position i of its (empty)
// sequence; the split GEMM's activation records of LayerNorm(c) (kv_b_proj's
// input, K = r: record (tok / 32, c / 16), lane tok % 32 + 32 ((c / 8) % 2),
// hi and lo halves, or with rec_lo = 0 (bf16 operands) hi-only records of
// 1 KB); and rope(k_pe) as the attention's k_rope [b, 1, s, dr]
// in bf16 or f32.  The sequences start empty (forward_prefill checks it),
// so positions are the token indices, lens is not read, and the wave of
// each sequence's token 0 sets its length to s.  The grid covers n rounded
// up to 32 tokens (the padding rows of the records are zeroed).  r % 32 == 0,
// r <= 512 U, dr % 8 == 0.
template <typename KT, int U>
__global__ __launch_bounds__(256) void k_prefill_rows(LatentRowsArgs a, int n, uint8_t *rec,
                                                      int rec_lo, KT *k_rope, int32_t *lens) {
  const int tok = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int r = a.r, dr = a.dr, C8 = r / 8, KS = r / 16;
  const int RB = rec_lo ? 2048 : 1024;  // bytes per record
  if (tok >= n) {
    // the padding rows of the last 32-row record group: zeros
    if (tok >= (n + 31) / 32 * 32) return;
    for (int c8 = lane; c8 < C8; c8 += 64) {
      uint8_t *rp =
          rec + ((int64_t)(tok >> 5) * KS + (c8 >> 1)) * RB + ((tok & 31) + 32 * (c8 & 1)) * 16;
      *reinterpret_cast<u32x4_t *>(rp) = u32x4_t{0, 0, 0, 0};
      if (rec_lo) *reinterpret_cast<u32x4_t *>(rp + 1024) = u32x4_t{0, 0, 0, 0};
    }
    return;
  }
  const int b = tok / a.s, i = tok - b * a.s;
  const float *src = a.kva + (int64_t)tok * (r + dr);
  uint8_t *dst = a.table.row(b, i, (int64_t)(r + dr) * (a.bf16 ? 2 : 4));
  // LayerNorm as candle_nn::LayerNorm (src/model.rs:136): mean, biased
  // variance of the centred values, divide by sqrt(var + eps), weight, bias
  constexpr int kMaxC8 = U;  // r <= 512 U: each lane holds U groups of 8
  floatx4_t x[kMaxC8][2];
  float sum = 0.f;
#pragma unroll
  for (int u = 0; u < kMaxC8; ++u) {
    const int c8 = lane + 64 * u;
    if (c8 < C8) {
      x[u][0] = *reinterpret_cast<const floatx4_t *>(src + 8 * c8);
      x[u][1] = *reinterpret_cast<const floatx4_t *>(src + 8 * c8 + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) sum += x[u][0][e] + x[u][1][e];
    }
  }
  for (int off = 32; off > 0; off >>= 1) sum += __shfl_xor(sum, off);
  const float mean = sum / (float)r;
  float sq = 0.f;
#pragma unroll
  for (int u = 0; u < kMaxC8; ++u)
    if (lane + 64 * u < C8)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = x[u][e >> 2][e & 3] - mean;
        sq += d * d;
      }
  for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off);
  const float inv = 1.f / sqrtf(sq / (float)r + a.eps);
#pragma unroll
  for (int u = 0; u < kMaxC8; ++u) {
    const int c8 = lane + 64 * u;
    if (c8 >= C8) continue;
    float v[8], w[8], bb[8];
    uint16_t hi[8], lo[8];
    *reinterpret_cast<floatx4_t *>(w) = *reinterpret_cast<const floatx4_t *>(a.ln_w + 8 * c8);
    *reinterpret_cast<floatx4_t *>(w + 4) =
        *reinterpret_cast<const floatx4_t *>(a.ln_w + 8 * c8 + 4);
    if (a.ln_b) {
      *reinterpret_cast<floatx4_t *>(bb) = *reinterpret_cast<const floatx4_t *>(a.ln_b + 8 * c8);
      *reinterpret_cast<floatx4_t *>(bb + 4) =
          *reinterpret_cast<const floatx4_t *>(a.ln_b + 8 * c8 + 4);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) bb[e] = 0.f;
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v[e] = (x[u][e >> 2][e & 3] - mean) * inv * w[e] + bb[e];
      hi[e] = f32_to_bf16_bits(v[e]);
      lo[e] = f32_to_bf16_bits(v[e] - bf16_bits_to_f32(hi[e]));
    }
    if (a.bf16) {
      *reinterpret_cast<u32x4_t *>(dst + 16 * c8) =
          u32x4_t{hi[0] | ((uint32_t)hi[1] << 16), hi[2] | ((uint32_t)hi[3] << 16),
                  hi[4] | ((uint32_t)hi[5] << 16), hi[6] | ((uint32_t)hi[7] << 16)};
    } else {
      *reinterpret_cast<floatx4_t *>(dst + 32 * c8) = floatx4_t{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<floatx4_t *>(dst + 32 * c8 + 16) = floatx4_t{v[4], v[5], v[6], v[7]};
    }
    uint8_t *rp = rec + ((int64_t)(tok >> 5) * KS + (c8 >> 1)) * RB + ((tok & 31) + 32 * (c8 & 1)) * 16;
    *reinterpret_cast<u32x4_t *>(rp) =
        u32x4_t{hi[0] | ((uint32_t)hi[1] << 16), hi[2] | ((uint32_t)hi[3] << 16),
                hi[4] | ((uint32_t)hi[5] << 16), hi[6] | ((uint32_t)hi[7] << 16)};
    if (rec_lo)
      *reinterpret_cast<u32x4_t *>(rp + 1024) =
          u32x4_t{lo[0] | ((uint32_t)lo[1] << 16), lo[2] | ((uint32_t)lo[3] << 16),
                  lo[4] | ((uint32_t)lo[5] << 16), lo[6] | ((uint32_t)lo[7] << 16)};
  }
  const float pos = (float)i;
  for (int p = lane; p < dr / 2; p += 64) {
    const float ang = pos * a.inv_freq[p];
    float cs, sn;
    rope_cs(ang, a.mscale, cs, sn);
    const float e = src[r + 2 * p], o = src[r + 2 * p + 1];
    const float re = e * cs - o * sn, ro = o * cs + e * sn;
    if (a.bf16) {
      reinterpret_cast<uint16_t *>(dst)[r + 2 * p] = f32_to_bf16_bits(re);
      reinterpret_cast<uint16_t *>(dst)[r + 2 * p + 1] = f32_to_bf16_bits(ro);
    } else {
      reinterpret_cast<float *>(dst)[r + 2 * p] = re;
      reinterpret_cast<float *>(dst)[r + 2 * p + 1] = ro;
    }
    if constexpr (sizeof(KT) == 2) {
      k_rope[(int64_t)tok * dr + 2 * p] = f32_to_bf16_bits(re);
      k_rope[(int64_t)tok * dr + 2 * p + 1] = f32_to_bf16_bits(ro);
    } else {
      k_rope[(int64_t)tok * dr + 2 * p] = re;
      k_rope[(int64_t)tok * dr + 2 * p + 1] = ro;
    }
  }
  if (i == 0 && lane == 0) lens[b] = a.s;
}

LatentRowsArgs latent_rows_args(const qmla_layer *L, const float *kva, int seq, float *rows,
                                qmla_kv_cache *cache) {
  const auto &g = L->cfg;
  LatentRowsArgs a{};
  a.kva = kva;
  a.s = seq;
  a.r = g.kv_lora_rank;
  a.dr = g.qk_rope;
  a.ln_w = L->ln_w;
  a.ln_b = L->ln_b;
  a.eps = (float)g.ln_eps;
  a.inv_freq = L->inv_freq;
  a.mscale = (float)g.rope_mscale;
  a.table = cache->table();
  a.bf16 = cache->dtype == QMLA_BF16;
  a.lens = cache->d_lens;
  a.rows = rows;
  return a;
}

// LayerNorm + RoPE of the n new tokens into the cache (sequence b's tokens
// at positions lens[b] + i), then the lengths advance (the caller checked
// the room already).
qmla_status latent_to_cache(const qmla_layer *L, const float *kva, int batch, int seq,
                            float *rows, qmla_kv_cache *cache, hipStream_t s) {
  k_latent_rows<<<dim3(batch * seq), dim3(256),
                  latent_row_lds_bytes(L->cfg.kv_lora_rank, L->cfg.qk_rope), s>>>(
      latent_rows_args(L, kva, seq, rows, cache));
  QMLA_LAUNCH_CHECK("k_latent_rows");
  return cache_advance(cache, 0, batch, seq, s);
}

// Element stores of the prefill operands: f32 as is, or bf16 (round to
// nearest even) for the bf16 MFMA prefill.
__device__ __forceinline__ void put(float *p, float v) { *p = v; }
__device__ __forceinline__ void put(uint16_t *p, float v) { *p = f32_to_bf16_bits(v); }
__device__ __forceinline__ float get(const float *p) { return *p; }
__device__ __forceinline__ float get(const uint16_t *p) { return bf16_bits_to_f32(*p); }

// Split q [b*s, H, dn+dr] into q_nope and roped q_rope (src/model.rs:263-267
// and :199-203); sequence b's token i sits at position lens[b] + i (its
// cached length before this step's append).  Output layouts by `bhs`:
//   bhs = 0: q_nope [b, s, H, dn], q_rope [b, s, H, dr]  (decode rows i*H + h)
//   bhs = 1: q_nope [b, H, s, dn], q_rope [b, H, s, dr]  (prefill layout)
template <typename OutT>
__global__ __launch_bounds__(64) void k_split_rope_q(const float *__restrict__ q, int s, int H,
                                                      int dn, int dr,
                                                      const float *__restrict__ inv_freq,
                                                      float mscale,
                                                      const int32_t *__restrict__ lens, int bhs,
                                                      OutT *__restrict__ q_nope,
                                                      OutT *__restrict__ q_rope) {
  const int tok = blockIdx.x, h = blockIdx.y;
  const int b = tok / s, i = tok % s;
  const float *src = q + ((int64_t)tok * H + h) * (dn + dr);
  const int64_t o = bhs ? ((int64_t)b * H + h) * s + i : (int64_t)tok * H + h;
  for (int c = threadIdx.x; c < dn; c += blockDim.x) put(q_nope + o * dn + c, src[c]);
  const float pos = (float)(lens[b] + i);
  for (int p = threadIdx.x; p < dr / 2; p += blockDim.x) {
    const float ang = pos * inv_freq[p];
    float cs, sn;
    rope_cs(ang, mscale, cs, sn);
    const float e = src[dn + 2 * p], od = src[dn + 2 * p + 1];
    put(q_rope + o * dr + 2 * p, e * cs - od * sn);
    put(q_rope + o * dr + 2 * p + 1, od * cs + e * sn);
  }
}

// kvb [b*s, H, dn+dv] -> k [b, H, s, dn], v [b, H, s, dv]  (compute_kv's
// reshape + transpose, src/model.rs:181-188 and :213-215)
template <typename OutT>
__global__ __launch_bounds__(128) void k_split_kv(const float *__restrict__ kvb, int s, int H,
                                                   int dn, int dv, OutT *__restrict__ k,
                                                   OutT *__restrict__ v) {
  const int tok = blockIdx.x, h = blockIdx.y;
  const int b = tok / s, i = tok % s;
  const float *src = kvb + ((int64_t)tok * H + h) * (dn + dv);
  const int64_t o = ((int64_t)b * H + h) * s + i;
  for (int c = threadIdx.x; c < dn; c += blockDim.x) put(k + o * dn + c, src[c]);
  for (int c = threadIdx.x; c < dv; c += blockDim.x) put(v + o * dv + c, src[dn + c]);
}

// rows [b*s, r+dr] -> k_rope [b, 1, s, dr]
template <typename OutT>
__global__ __launch_bounds__(64) void k_rows_rope(const float *__restrict__ rows, int r, int dr,
                                                   OutT *__restrict__ k_rope) {
  const int tok = blockIdx.x;
  for (int c = threadIdx.x; c < dr; c += blockDim.x)
    put(k_rope + (int64_t)tok * dr + c, rows[(int64_t)tok * (r + dr) + r + c]);
}

// ctx [b, H, s, dv] -> [b, s, H*dv] f32  (src/model.rs:248)
template <typename InT>
__global__ __launch_bounds__(128) void k_merge_heads(const InT *__restrict__ ctx, int s, int H,
                                                      int dv, float *__restrict__ o) {
  const int tok = blockIdx.x, h = blockIdx.y;
  const int b = tok / s, i = tok % s;
  const InT *src = ctx + (((int64_t)b * H + h) * s + i) * dv;
  float *dst = o + ((int64_t)tok * H + h) * dv;
  for (int c = threadIdx.x; c < dv; c += blockDim.x) dst[c] = get(src + c);
}

// Materialising the reference KVCache (src/model.rs:86-105) from latent rows:
// the c_kv part of sequence seq0 + b's first T rows as f32 [n, T, r] (the
// A operand of the kv_b_proj GEMMs).
template <typename SrcT>
__global__ __launch_bounds__(256) void k_latent_c_f32(PageTable tab, int seq0, int T, int r,
                                                      int dr, float *__restrict__ dst) {
  const int t = blockIdx.x, b = blockIdx.y;
  const SrcT *src =
      reinterpret_cast<const SrcT *>(tab.row(seq0 + b, t, (int64_t)(r + dr) * sizeof(SrcT)));
  float *o = dst + ((int64_t)b * T + t) * r;
  for (int c = threadIdx.x; c < r; c += blockDim.x) {
    if constexpr (sizeof(SrcT) == 2)
      o[c] = bf16_bits_to_f32(src[c]);
    else
      o[c] = src[c];
  }
}

// The c_kv part of the cache rows in split form ([n, T] rows of
// split_cols(r) bf16: [c_hi | c_lo | c_hi | 1, 1, 0...]), the activations
// of the split kv_b_proj GEMMs.
template <typename SrcT>
__global__ __launch_bounds__(256) void k_latent_c_split(PageTable tab, int seq0, int T, int r,
                                                        int dr, uint16_t *__restrict__ xs) {
  const int t = blockIdx.x, b = blockIdx.y;
  const SrcT *src =
      reinterpret_cast<const SrcT *>(tab.row(seq0 + b, t, (int64_t)(r + dr) * sizeof(SrcT)));
  uint16_t *row = xs + ((int64_t)b * T + t) * split_cols(r);
  for (int c = threadIdx.x; c < r; c += blockDim.x) {
    float x;
    if constexpr (sizeof(SrcT) == 2)
      x = bf16_bits_to_f32(src[c]);
    else
      x = src[c];
    const uint16_t h = f32_to_bf16_bits(x);
    row[c] = h;
    row[r + c] = f32_to_bf16_bits(x - bf16_bits_to_f32(h));
    row[2 * r + c] = h;
  }
  for (int c = threadIdx.x; c < split_cols(r) - 3 * r; c += blockDim.x)
    row[3 * r + c] = c < 2 ? (uint16_t)0x3f80 : (uint16_t)0;
}

// k_rope [n, H, T, dr]: the stored (roped) k_pe of each token broadcast to
// every head, as the reference's expand at src/model.rs:217-219 / :281-285.
template <typename SrcT>
__global__ __launch_bounds__(256) void k_broadcast_rope(PageTable tab, int seq0, int T, int H,
                                                        int r, int dr,
                                                        float *__restrict__ k_rope) {
  const int t = blockIdx.x, b = blockIdx.y;
  const SrcT *src =
      reinterpret_cast<const SrcT *>(tab.row(seq0 + b, t, (int64_t)(r + dr) * sizeof(SrcT))) + r;
  for (int e = threadIdx.x; e < H * dr; e += blockDim.x) {
    const int h = e / dr, c = e % dr;
    float v;
    if constexpr (sizeof(SrcT) == 2)
      v = bf16_bits_to_f32(src[c]);
    else
      v = src[c];
    k_rope[(((int64_t)b * H + h) * T + t) * dr + c] = v;
  }
}

// Builds and uploads the fragment-major split projection weights of the
// decode step (once, at layer creation).
qmla_status make_skinny_weights(qmla_layer *L, const float *wq, const float *bq,
                                const float *wkva, const float *bkva, const float *wkvb,
                                const float *bkvb, const float *wo) {
  const auto &g = L->cfg;
  const int H = g.heads, dn = g.qk_nope, dr = g.qk_rope, dv = g.v_dim, r = g.kv_lora_rank;
  const int hid = g.hidden, nq = H * (dn + dr), nk = r + dr;
  auto upload = [&](const void *src, size_t bytes, void **dst) -> qmla_status {
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) return fail(QMLA_ERR_OOM, "weight allocation failed");
    L->allocs.push_back(p);
    *dst = p;
    if (hipMemcpy(p, src, bytes, hipMemcpyHostToDevice) != hipSuccess)
      return fail(QMLA_ERR_HIP, "weight upload failed");
    return QMLA_OK;
  };
  auto put = [&](const float *W, int64_t ldw, int64_t sw, int N, int K, int Z,
                 void **dst) -> qmla_status {
    std::vector<uint8_t> frag(skinny_frag_bytes(N, K, Z));
    skinny_pack(W, ldw, sw, N, K, Z, frag.data());
    return upload(frag.data(), frag.size(), dst);
  };
  std::vector<float> w((size_t)(nq + nk) * hid);
  std::memcpy(w.data(), wq, sizeof(float) * nq * hid);
  std::memcpy(w.data() + (size_t)nq * hid, wkva, sizeof(float) * nk * hid);
  QMLA_TRY(put(w.data(), hid, 0, nq + nk, hid, 1, &L->w1f));
  std::vector<float> b(nq + nk, 0.f);
  if (bq) std::memcpy(b.data(), bq, sizeof(float) * nq);
  if (bkva) std::memcpy(b.data() + nq, bkva, sizeof(float) * nk);
  QMLA_TRY(upload(b.data(), b.size() * 4, (void **)&L->b1));
  // W_UK^h transposed: wuk[h][i][d] = wkvb[h (dn + dv) + d][i]
  w.assign((size_t)H * r * dn, 0.f);
  for (int h = 0; h < H; ++h)
    for (int d = 0; d < dn; ++d)
      for (int i = 0; i < r; ++i)
        w[((size_t)h * r + i) * dn + d] = wkvb[((size_t)h * (dn + dv) + d) * r + i];
  QMLA_TRY(put(w.data(), dn, (int64_t)r * dn, r, dn, H, &L->wukf));
  // W_UV^h = kv_b rows h (dn + dv) + dn .. + dv, and its bias b_V^h
  QMLA_TRY(put(wkvb + (size_t)dn * r, r, (int64_t)(dn + dv) * r, dv, r, H, &L->wuvf));
  b.assign((size_t)H * dv, 0.f);
  if (bkvb)
    for (int h = 0; h < H; ++h)
      for (int i = 0; i < dv; ++i) b[(size_t)h * dv + i] = bkvb[(size_t)h * (dn + dv) + dn + i];
  QMLA_TRY(upload(b.data(), b.size() * 4, (void **)&L->buv));
  QMLA_TRY(put(wo, (int64_t)H * dv, 0, hid, H * dv, 1, &L->wof));
  QMLA_TRY(put(wkvb, r, 0, H * (dn + dv), r, 1, &L->wkvbf));
  L->skinny = true;
  return QMLA_OK;
}

// forward_prefill runs its projections on the split GEMM (split_gemm.hip)
// when the fragment-major weights exist and every product's widths suit it.
bool use_split_gemm(const qmla_layer *L) {
  const auto &g = L->cfg;
  const int H = g.heads, dn = g.qk_nope, dr = g.qk_rope, dv = g.v_dim, r = g.kv_lora_rank;
  return L->skinny && L->wkvbf && r <= 512 &&
         split_gemm_supported(H * (dn + dr) + r + dr, g.hidden) &&
         split_gemm_supported(H * (dn + dv), r) && split_gemm_supported(g.hidden, H * dv) &&
         dn % 4 == 0 && dr % 8 == 0 && dv % 32 == 0;
}

// The decode step runs its projections on the skinny kernel when every
// product has a K the kernel takes and the token count is small.
bool use_skinny(const qmla_layer *L, int n) {
  const auto &g = L->cfg;
  // q_proj | kv_a splits its K (hidden) in two halves
  return L->skinny && n <= kSkinnyRows && g.hidden % 32 == 0 &&
         skinny_supported(32, g.hidden / 2) && skinny_supported(32, g.qk_nope) &&
         skinny_supported(32, g.kv_lora_rank) && skinny_supported(32, g.heads * g.v_dim);
}

// Arguments of a skinny product y = x W^T (+ bias) with the FINAL store:
// x [Z][M][K] (row stride ldx, z-stride sx), y [Z][M][N] (ldy, sy).
// o_proj of the decode step with its K range split over kOprojGroups
// blocks per 32-output tile (4 x the blocks streaming the weight); the
// groups' partial planes are added in group order by k_add_planes.
constexpr int kOprojGroups = 4;

// out[i] = sum over g < G of planes[g plane + i] (in g order), four
// elements per thread.
__global__ __launch_bounds__(256) void k_add_planes(const float *__restrict__ planes, int G,
                                                    int64_t plane, int64_t n4,
                                                    float *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n4) return;
  floatx4_t v = reinterpret_cast<const floatx4_t *>(planes)[i];
  for (int g = 1; g < G; ++g) {
    const floatx4_t p = reinterpret_cast<const floatx4_t *>(planes + g * plane)[i];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] += p[e];
  }
  reinterpret_cast<floatx4_t *>(out)[i] = v;
}

SkinnyGemmArgs skinny_args(const void *w_frag, const float *x, int64_t ldx, int64_t sx,
                           const float *bias, int64_t sb, float *y, int64_t ldy, int64_t sy,
                           int M, int N, int K, int Z) {
  SkinnyGemmArgs a{};
  a.w_frag = w_frag;
  a.x = x;
  a.ldx = ldx;
  a.sx = sx;
  a.bias = bias;
  a.sb = sb;
  a.y = y;
  a.ldy = ldy;
  a.sy = sy;
  a.M = M;
  a.N = N;
  a.K = K;
  a.Z = Z;
  a.mode = kSkinnyFinal;
  return a;
}

inline size_t al(size_t x) { return (x + 255) & ~size_t(255); }

struct LayerWs {
  size_t q, kva, rows, qn, qr, qlat, olat, o, dec, kvb, k, v, kr, ctx, pack, pack2, sgpart, part,
      part_elems, xsplit,
      qn1, qr1, kva1,
      total;
};

// Which forward call a carve-up serves.  The two calls share the
// projection regions; the decode-only regions (q_lat, o_lat, the decode
// core's partials) and the prefill-only ones (LayerNorm'd rows, kv_b_proj
// output, k, v, k_rope, context) overlay one another, so a workspace sized
// for both is the larger of the two, not their sum.
enum class WsFor { kDecode, kPrefill, kBoth };

// Scratch carve-up shared by the size queries and the two forward calls.
LayerWs layer_ws(const qmla_layer *L, int32_t batch, int32_t seq, size_t dec_bytes, WsFor use) {
  const auto &g = L->cfg;
  const size_t n = (size_t)batch * seq, H = g.heads;
  LayerWs w{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    size_t o = off;
    off += al(bytes);
    return o;
  };
  // forward_prefill on the hand-written split GEMMs writes q, k, v and the
  // cache rows from the GEMM epilogues: it needs neither the f32 q, the
  // rocBLAS split of the activations, the LayerNorm'd rows nor the kv_b
  // output, only the activation records
  const bool sg = use_split_gemm(L) && n >= (size_t)kSplitGemmMinRows;
  const bool sg_only = sg && use == WsFor::kPrefill;
  w.q = take(sg_only ? 1 : sizeof(float) * n * H * (g.qk_nope + g.qk_rope));
  w.kva = take(sizeof(float) * n * (g.kv_lora_rank + g.qk_rope));
  w.qn = take(sizeof(float) * n * H * g.qk_nope);
  w.qr = take(sizeof(float) * n * H * g.qk_rope + 4);
  // o: [n][H dv] f32, or o_proj's packed B operand of 32 token rows (the
  // same 4 bytes per element, 32 rows at least)
  w.o = take(sizeof(float) * std::max<size_t>(n, 32) * H * g.v_dim);
  // split-K partials of the skinny projections (16 slices at most)
  const size_t widest = std::max<size_t>({(size_t)H * (g.qk_nope + g.qk_rope),
                                          (size_t)(g.kv_lora_rank + g.qk_rope), (size_t)g.hidden});
  w.part_elems = n <= (size_t)kSkinnyRows ? 16 * n * widest : 0;
  w.part = take(sizeof(float) * (w.part_elems ? w.part_elems : 1));
  // bf16 halves of a projection's activations (rocBLAS split GEMMs, many rows)
  const size_t kmax = std::max<size_t>({(size_t)g.hidden, H * g.v_dim, (size_t)g.kv_lora_rank});
  w.xsplit =
      take(n >= (size_t)kSplitRows && !sg_only ? split_bytes((int64_t)n, (int64_t)kmax) : 1);
  const size_t shared = off;
  size_t dec_end = shared, pre_end = shared;
  if (use != WsFor::kPrefill) {
    w.qlat = take(sizeof(float) * n * H * g.kv_lora_rank);
    w.olat = take(sizeof(float) * n * H * g.kv_lora_rank);
    w.dec = take(dec_bytes);
    // the second K-half of the skinny q_proj | kv_a product
    if (n <= (size_t)kSkinnyRows) {
      w.qn1 = take(sizeof(float) * n * H * g.qk_nope);
      w.qr1 = take(sizeof(float) * n * H * g.qk_rope);
      w.kva1 = take(sizeof(float) * n * (g.kv_lora_rank + g.qk_rope));
    }
    dec_end = off;
  }
  if (use != WsFor::kDecode) {
    off = shared;
    w.rows = take(sg ? 1 : sizeof(float) * n * (g.kv_lora_rank + g.qk_rope));
    w.kvb = take(sg ? 1 : sizeof(float) * n * H * (g.qk_nope + g.v_dim));
    w.k = take(sizeof(float) * n * H * g.qk_nope);
    w.v = take(sizeof(float) * n * H * g.v_dim);
    w.kr = take(sizeof(float) * n * g.qk_rope + 4);
    w.ctx = take(sizeof(float) * n * H * g.v_dim);
    // the activation records of the hand-written split GEMM: the current
    // product's, and kv_b_proj's (written by the latent rows kernel)
    w.pack = take(sg ? split_gemm_pack_bytes((int)n, (int)kmax) : 1);
    w.pack2 = take(sg ? split_gemm_pack_bytes((int)n, g.kv_lora_rank) : 1);
    // the split GEMMs' K-slice partial sums (few rows), one product at a time
    const int N1 = (int)H * (g.qk_nope + g.qk_rope) + g.kv_lora_rank + g.qk_rope;
    const int Nkv = (int)H * (g.qk_nope + g.v_dim);
    w.sgpart = take(sg ? std::max({split_gemm_part_bytes((int)n, N1, g.hidden),
                                   split_gemm_part_bytes((int)n, Nkv, g.kv_lora_rank),
                                   split_gemm_part_bytes((int)n, g.hidden, (int)H * g.v_dim),
                                   (size_t)1})
                       : 1);
    pre_end = off;
  }
  w.total = std::max(dec_end, pre_end);
  return w;
}

qmla_status check_layer_call(const qmla_layer *L, const float *xs, int32_t batch, int32_t seq,
                             const qmla_kv_cache *c, const float *out) {
  QMLA_REQUIRE(L && c, QMLA_ERR_INVALID_ARG, "NULL layer or cache");
  QMLA_REQUIRE(batch > 0 && seq > 0, QMLA_ERR_SHAPE, "batch and seq must be > 0");
  QMLA_REQUIRE(xs && out, QMLA_ERR_INVALID_ARG, "NULL xs or out");
  // the kernels move rows in 16-byte vectors
  QMLA_REQUIRE((reinterpret_cast<uintptr_t>(xs) | reinterpret_cast<uintptr_t>(out)) % 16 == 0,
               QMLA_ERR_INVALID_ARG, "xs and out must be 16-byte aligned");
  QMLA_REQUIRE(batch <= c->num_seqs, QMLA_ERR_SHAPE, "batch %d > cache sequences %d", batch,
               c->num_seqs);
  QMLA_REQUIRE(c->r == L->cfg.kv_lora_rank && c->dr == L->cfg.qk_rope, QMLA_ERR_SHAPE,
               "cache latent dims (%d, %d) differ from the layer's (%d, %d)", c->r, c->dr,
               L->cfg.kv_lora_rank, L->cfg.qk_rope);
  QMLA_REQUIRE(c->dtype == QMLA_F32 || c->dtype == QMLA_BF16, QMLA_ERR_UNSUPPORTED,
               "the layer needs an f32 or bf16 latent cache");
  return QMLA_OK;
}

// Sequences seq0 .. seq0 + n - 1 of one uniform length T (the reference's
// KVCache holds one tensor per kind, so every sequence has the same T).
qmla_status check_materialise(const qmla_layer *L, const qmla_kv_cache *c, int32_t seq0,
                              int32_t n, int32_t *T) {
  QMLA_REQUIRE(L && c, QMLA_ERR_INVALID_ARG, "NULL layer or cache");
  QMLA_REQUIRE(n > 0 && seq0 >= 0 && seq0 + (int64_t)n <= c->num_seqs, QMLA_ERR_SHAPE,
               "sequences [%d, %d) outside the cache's %d", seq0, seq0 + n, c->num_seqs);
  QMLA_REQUIRE(c->r == L->cfg.kv_lora_rank && c->dr == L->cfg.qk_rope, QMLA_ERR_SHAPE,
               "cache latent dims (%d, %d) differ from the layer's (%d, %d)", c->r, c->dr,
               L->cfg.kv_lora_rank, L->cfg.qk_rope);
  QMLA_REQUIRE(c->dtype == QMLA_F32 || c->dtype == QMLA_BF16, QMLA_ERR_UNSUPPORTED,
               "bad cache dtype");
  for (int32_t i = seq0 + 1; i < seq0 + n; ++i)
    QMLA_REQUIRE(c->h_lens[i] == c->h_lens[seq0], QMLA_ERR_SHAPE,
                 "sequence lengths differ (%d vs %d): a KVCache tensor has one length",
                 c->h_lens[i], c->h_lens[seq0]);
  *T = c->h_lens[seq0];
  return QMLA_OK;
}

// Whether materialise runs compute_kv in split form (sequences of many
// tokens), and its scratch: the c_kv rows as f32 or in split form.
bool materialise_split(const qmla_layer *L, int32_t T) { return T >= kSplitRows && L->wkvb_x; }

size_t materialise_ws_bytes(const qmla_layer *L, const qmla_kv_cache *c, int32_t n, int32_t T) {
  if (materialise_split(L, T)) return split_bytes((int64_t)n * T, c->r);
  return sizeof(float) * (size_t)n * T * c->r;
}

// Decode workspace for the largest piece count the decode may choose
// (device CUs x pieces per CU), so the size does not creep up with the
// context and a caller can size the workspace once per (batch, seq).  The
// cache's dtype fixes the decode path: bf16 partials on the MFMA decode,
// f32 ones on the f32 decode.
size_t decode_bytes_for(const qmla_layer *L, const qmla_kv_cache *c, int32_t batch,
                        int32_t seq) {
  int cus = device_cu_count();
  if (cus <= 0) cus = 256;
  const int32_t rows = seq * L->cfg.heads, r = L->cfg.kv_lora_rank, dr = L->cfg.qk_rope;
  const bool mfma = c->dtype == QMLA_BF16;
  const int per_cu = mfma && decode_mfma_supported(rows, r, dr)
                         ? decode_mfma_blocks_per_cu(rows, r, dr)
                         : 4;
  const int32_t blocks = (int32_t)std::min<int64_t>((int64_t)cus * per_cu, kMaxPlanBlocks);
  return decode_workspace_layout(batch, rows, r, blocks, mfma).total;
}

}  // namespace
}  // namespace qmla

using namespace qmla;

extern "C" {

qmla_status qmla_layer_default_scales(qmla_layer_config *cfg) {
  QMLA_REQUIRE(cfg, QMLA_ERR_INVALID_ARG, "cfg is NULL");
  // src/model.rs:46-52 and :160-173
  auto mscale = [](double scale, double m) { return scale <= 1.0 ? 1.0 : 0.1 * m * std::log(scale) + 1.0; };
  const double factor = 40.0;
  cfg->rope_mscale = mscale(factor, 1.0) / mscale(factor, 0.707);
  const double m = mscale(factor, 0.707);
  cfg->softmax_scale = std::pow((double)(cfg->qk_nope + cfg->qk_rope), -0.5) * m * m;
  cfg->ln_eps = 1e-6;
  return QMLA_OK;
}

qmla_status qmla_layer_create(const qmla_layer_config *cfg, const float *wq, const float *bq,
                              const float *wkva, const float *bkva, const float *ln_w,
                              const float *ln_b, const float *wkvb, const float *bkvb,
                              const float *wo, const float *bo, qmla_layer **out) {
  QMLA_REQUIRE(cfg && out, QMLA_ERR_INVALID_ARG, "NULL cfg or out");
  *out = nullptr;
  QMLA_REQUIRE(wq && wkva && ln_w && wkvb && wo, QMLA_ERR_INVALID_ARG, "NULL weight");
  const auto &g = *cfg;
  QMLA_REQUIRE(g.hidden > 0 && g.heads > 0 && g.qk_nope > 0 && g.qk_rope >= 0 && g.v_dim > 0 &&
                   g.kv_lora_rank > 0,
               QMLA_ERR_SHAPE, "bad layer dims");
  QMLA_REQUIRE(g.qk_rope % 2 == 0, QMLA_ERR_SHAPE, "qk_rope must be even");
  QMLA_REQUIRE((g.kv_lora_rank + g.qk_rope) % 8 == 0, QMLA_ERR_UNSUPPORTED,
               "kv_lora_rank + qk_rope must be a multiple of 8");
  qmla_layer *L = new (std::nothrow) qmla_layer();
  QMLA_REQUIRE(L, QMLA_ERR_OOM, "host allocation failed");
  L->cfg = g;
  for (auto &b : L->blas)
    if (rocblas_create_handle(&b.h) != rocblas_status_success) {
      for (auto &c : L->blas)
        if (c.h) (void)rocblas_destroy_handle(c.h);
      delete L;
      return fail(QMLA_ERR_HIP, "rocBLAS handle creation failed");
    }
  const int H = g.heads;
  struct W {
    float **dst;
    const float *src;
    size_t n;
  } ws[] = {
      {&L->wq, wq, (size_t)H * (g.qk_nope + g.qk_rope) * g.hidden},
      {&L->bq, bq, (size_t)H * (g.qk_nope + g.qk_rope)},
      {&L->wkva, wkva, (size_t)(g.kv_lora_rank + g.qk_rope) * g.hidden},
      {&L->bkva, bkva, (size_t)(g.kv_lora_rank + g.qk_rope)},
      {&L->ln_w, ln_w, (size_t)g.kv_lora_rank},
      {&L->ln_b, ln_b, (size_t)g.kv_lora_rank},
      {&L->wkvb, wkvb, (size_t)H * (g.qk_nope + g.v_dim) * g.kv_lora_rank},
      {&L->bkvb, bkvb, (size_t)H * (g.qk_nope + g.v_dim)},
      {&L->wo, wo, (size_t)g.hidden * H * g.v_dim},
      {&L->bo, bo, (size_t)g.hidden},
  };
  qmla_status st = QMLA_OK;
  for (auto &w : ws) {
    if (!w.src) continue;  // optional bias
    void *p = nullptr;
    if (hipMalloc(&p, w.n * sizeof(float)) != hipSuccess) {
      st = fail(QMLA_ERR_OOM, "weight allocation failed");
      break;
    }
    L->allocs.push_back(p);
    *w.dst = static_cast<float *>(p);
    if (hipMemcpy(p, w.src, w.n * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
      st = fail(QMLA_ERR_HIP, "weight upload failed");
      break;
    }
  }
  if (st == QMLA_OK && g.qk_rope > 0) {
    // inv_freq[i] = 1.0f / (float)10000^(2i/d)  (src/model.rs:56-58)
    std::vector<float> inv(g.qk_rope / 2);
    for (int i = 0; i < g.qk_rope / 2; ++i)
      inv[i] = 1.0f / (float)std::pow(10000.0, 2.0 * i / (double)g.qk_rope);
    void *p = nullptr;
    if (hipMalloc(&p, inv.size() * sizeof(float)) != hipSuccess ||
        hipMemcpy(p, inv.data(), inv.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess)
      st = fail(QMLA_ERR_HIP, "inv_freq upload failed");
    if (p) L->allocs.push_back(p);
    L->inv_freq = static_cast<float *>(p);
  }
  if (st == QMLA_OK) {
    // split-form rows of the four projections (with their biases)
    struct Half {
      uint16_t **dst;
      const float *w, *b;
      int N, K;
    } hs[] = {
        {&L->wq_x, wq, bq, H * (g.qk_nope + g.qk_rope), g.hidden},
        {&L->wkva_x, wkva, bkva, g.kv_lora_rank + g.qk_rope, g.hidden},
        {&L->wkvb_x, wkvb, bkvb, H * (g.qk_nope + g.v_dim), g.kv_lora_rank},
        {&L->wo_x, wo, bo, g.hidden, H * g.v_dim},
    };
    std::vector<uint16_t> hl;
    for (auto &h : hs) {
      const int KX = split_cols(h.K);
      hl.assign((size_t)h.N * KX, 0);
      for (int n = 0; n < h.N; ++n) {
        uint16_t *row = hl.data() + (size_t)n * KX;
        for (int k = 0; k < h.K; ++k) {
          const float v = h.w[(size_t)n * h.K + k];
          const uint16_t hi = f32_to_bf16_bits(v);
          row[k] = hi;
          row[h.K + k] = hi;
          row[2 * h.K + k] = f32_to_bf16_bits(v - bf16_bits_to_f32(hi));
        }
        if (h.b) {
          const uint16_t bh = f32_to_bf16_bits(h.b[n]);
          row[3 * h.K] = bh;
          row[3 * h.K + 1] = f32_to_bf16_bits(h.b[n] - bf16_bits_to_f32(bh));
        }
      }
      void *p = nullptr;
      if (hipMalloc(&p, hl.size() * sizeof(uint16_t)) != hipSuccess) {
        st = fail(QMLA_ERR_OOM, "weight allocation failed");
        break;
      }
      L->allocs.push_back(p);
      if (hipMemcpy(p, hl.data(), hl.size() * sizeof(uint16_t), hipMemcpyHostToDevice) !=
          hipSuccess) {
        st = fail(QMLA_ERR_HIP, "weight upload failed");
        break;
      }
      *h.dst = static_cast<uint16_t *>(p);
    }
  }
  if (st == QMLA_OK && g.hidden % 16 == 0 && g.qk_nope % 16 == 0 && g.kv_lora_rank % 16 == 0 &&
      (g.heads * g.v_dim) % 16 == 0)
    st = make_skinny_weights(L, wq, bq, wkva, bkva, wkvb, bkvb, wo);
  if (st != QMLA_OK) {
    for (void *p : L->allocs) (void)hipFree(p);
    for (auto &b : L->blas) (void)rocblas_destroy_handle(b.h);
    delete L;
    return st;
  }
  *out = L;
  return QMLA_OK;
}

qmla_status qmla_layer_set_projection_dtype(qmla_layer *layer, qmla_dtype dtype) {
  QMLA_REQUIRE(layer, QMLA_ERR_INVALID_ARG, "NULL layer");
  QMLA_REQUIRE(dtype == QMLA_F32 || dtype == QMLA_BF16, QMLA_ERR_INVALID_ARG,
               "projection dtype %d", (int)dtype);
  layer->proj_bf16 = dtype == QMLA_BF16;
  return QMLA_OK;
}

qmla_status qmla_layer_destroy(qmla_layer *layer) {
  if (!layer) return QMLA_OK;
  for (void *p : layer->allocs) (void)hipFree(p);
  for (auto &b : layer->blas)
    if (b.h) (void)rocblas_destroy_handle(b.h);
  delete layer;
  return QMLA_OK;
}

qmla_status qmla_layer_workspace_bytes(const qmla_layer *layer, const qmla_kv_cache *cache,
                                       int32_t batch, int32_t seq, size_t *bytes) {
  QMLA_REQUIRE(layer && cache && bytes, QMLA_ERR_INVALID_ARG, "NULL pointer");
  QMLA_REQUIRE(batch > 0 && seq > 0 && batch <= cache->num_seqs, QMLA_ERR_SHAPE,
               "bad batch/seq");
  *bytes = layer_ws(layer, batch, seq, decode_bytes_for(layer, cache, batch, seq), WsFor::kBoth)
               .total;
  return QMLA_OK;
}

qmla_status qmla_layer_prefill_workspace_bytes(const qmla_layer *layer,
                                               const qmla_kv_cache *cache, int32_t batch,
                                               int32_t seq, size_t *bytes) {
  QMLA_REQUIRE(layer && cache && bytes, QMLA_ERR_INVALID_ARG, "NULL pointer");
  QMLA_REQUIRE(batch > 0 && seq > 0 && batch <= cache->num_seqs, QMLA_ERR_SHAPE,
               "bad batch/seq");
  *bytes = layer_ws(layer, batch, seq, 0, WsFor::kPrefill).total;
  return QMLA_OK;
}

qmla_status qmla_layer_forward_with_cache(const qmla_layer *L, const float *xs, int32_t batch,
                                          int32_t seq, qmla_kv_cache *cache, float *out,
                                          void *workspace, size_t workspace_bytes,
                                          qmla_stream stream) {
  QMLA_TRY(check_layer_call(L, xs, batch, seq, cache, out));
  // f32 cache: f32 decode core.  bf16 cache: the new rows are rounded to
  // bf16 on append and the core is the bf16 MFMA decode (q rounded to bf16,
  // f32 accumulation) for the latent shapes it serves.  Every check runs
  // before the cache is touched: a rejected call leaves lengths, capacity
  // and rows as they were.
  const auto &g = L->cfg;
  const int H = g.heads, dn = g.qk_nope, dr = g.qk_rope, dv = g.v_dim, r = g.kv_lora_rank;
  QMLA_REQUIRE((int64_t)seq * H <= 0x7fffffff, QMLA_ERR_SHAPE, "seq x heads too large");
  QMLA_TRY(decode_shape_supported(cache, seq * H));
  const size_t dec_bytes = decode_bytes_for(L, cache, batch, seq);
  const LayerWs w = layer_ws(L, batch, seq, dec_bytes, WsFor::kDecode);
  QMLA_REQUIRE(workspace && workspace_bytes >= w.total, QMLA_ERR_WORKSPACE,
               "workspace of %zu bytes < required %zu", workspace_bytes, w.total);
  QMLA_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, QMLA_ERR_WORKSPACE,
               "the workspace must be 256-byte aligned (device allocations are)");
  QMLA_TRY(make_room(cache, 0, batch, seq, as_stream(stream)));
  char *ws = static_cast<char *>(workspace);
  float *q = (float *)(ws + w.q), *kva = (float *)(ws + w.kva);
  float *qn = (float *)(ws + w.qn), *qr = (float *)(ws + w.qr), *qlat = (float *)(ws + w.qlat);
  float *olat = (float *)(ws + w.olat), *o = (float *)(ws + w.o);
  float *part = (float *)(ws + w.part);
  hipStream_t s = as_stream(stream);
  const int n = batch * seq;

  if (use_skinny(L, n)) {
    // The projections on the skinny MFMA kernel, 32 token rows per launch;
    // six dependent launches for one new token per sequence:
    //   q_proj | kv_a (q split and roped in the epilogue) -> W_UK absorption
    //   with the new latent cache rows in extra blocks -> decode core ->
    //   merge (+ length advance) -> W_UV -> o_proj
    // q_proj | kv_a runs with its K range split over two block groups; its
    // two halves land in two planes that the next launch adds (the
    // absorption's operand load, the latent row blocks for kv_a, and its
    // GEMM blocks for the roped q_rope).
    float *qn1 = (float *)(ws + w.qn1), *qr1 = (float *)(ws + w.qr1);
    float *kva1 = (float *)(ws + w.kva1);
    for (int m0 = 0; m0 < n; m0 += 32) {
      SkinnyGemmArgs a = skinny_args(L->w1f, xs + (size_t)m0 * g.hidden, g.hidden, 0, L->b1, 0,
                                     nullptr, 0, 0, std::min(32, n - m0), H * (dn + dr) + r + dr,
                                     g.hidden, 1);
      a.mode = kSkinnyQkv;
      a.m0 = m0;
      a.seq = seq;
      a.heads = H;
      a.dn = dn;
      a.dr = dr;
      a.q_nope = qn;
      a.q_rope = qr;
      a.kva = kva;
      a.kva_ld = r + dr;
      a.lens = cache->d_lens;
      a.inv_freq = L->inv_freq;
      a.mscale = (float)g.rope_mscale;
      a.groups = 2;
      a.q_nope1 = qn1;
      a.q_rope1 = qr1;
      a.kva1 = kva1;
      a.bf16ops = L->proj_bf16 ? 1 : 0;
      QMLA_TRY(launch_skinny_gemm(a, s));
    }
    // q_lat[t, h, :] = W_UK^h^T q_nope[t, h, :]   (z = head), and the latent
    // rows [LayerNorm(c) | rope(k_pe)] of the n new tokens into the cache
    LatentRowsArgs rows = latent_rows_args(L, kva, seq, nullptr, cache);
    rows.kva1 = kva1;
    for (int m0 = 0; m0 < n; m0 += 32) {
      SkinnyGemmArgs uk = skinny_args(L->wukf, qn + (size_t)m0 * H * dn, (int64_t)H * dn, dn,
                                      nullptr, 0, qlat + (size_t)m0 * H * r, (int64_t)H * r, r,
                                      std::min(32, n - m0), r, dn, H);
      uk.x2 = qn1 + (size_t)m0 * H * dn;
      uk.bf16ops = L->proj_bf16 ? 1 : 0;
      if (m0 == 0) {
        // the roped q_rope's two halves
        uk.add_dst = qr;
        uk.add_src = qr1;
        uk.add_n = (int64_t)n * H * dr;
      }
      QMLA_TRY(launch_skinny_gemm(uk, s, m0 == 0 ? &rows : nullptr, n));
    }
    // the new rows sit past the device lengths: the decode attends
    // lens + seq tokens and its merge advances the lengths.  The host
    // mirror moves with them (the split plan counts the new tokens); if the
    // decode is not launched, the merge never advances the device lengths,
    // so the mirror goes back and both keep the old lengths.
    for (int32_t i = 0; i < batch; ++i) cache->h_lens[i] += seq;
    qmla_decode_dims dd{batch, seq * H, r, dr};
    const qmla_status st = decode_launch(&dd, cache, QMLA_F32, qlat, qr, g.softmax_scale, olat,
                                         nullptr, 0, ws + w.dec, dec_bytes, seq, true, s);
    if (st != QMLA_OK) {
      for (int32_t i = 0; i < batch; ++i) cache->h_lens[i] -= seq;
      return st;
    }
    // o[t, h, :] = W_UV^h o_lat[t, h, :] + b_V^h, written as o_proj's
    // packed B operand (32 token rows x H dv: 4 (H dv) bytes), then o_proj
    for (int m0 = 0; m0 < n; m0 += 32) {
      const int M = std::min(32, n - m0);
      SkinnyGemmArgs uv = skinny_args(L->wuvf, olat + (size_t)m0 * H * r, (int64_t)H * r, r,
                                      L->buv, dv, o, 0, dv, M, dv, r, H);
      uv.mode = kSkinnyPackB;
      uv.bf16ops = L->proj_bf16 ? 1 : 0;  // o_proj below then reads the hi halves only
      QMLA_TRY(launch_skinny_gemm(uv, s));
      const int64_t plane = (int64_t)M * g.hidden;
      const bool split = g.hidden % 4 == 0 && (H * dv) % (16 * kOprojGroups) == 0 &&
                         skinny_supported(M, H * dv / kOprojGroups) &&
                         (size_t)kOprojGroups * plane <= w.part_elems;
      SkinnyGemmArgs op = skinny_args(L->wof, o, 0, 0, L->bo, 0,
                                      split ? part : out + (size_t)m0 * g.hidden, g.hidden, 0, M,
                                      g.hidden, H * dv, 1);
      op.x_packed = true;
      op.bf16ops = L->proj_bf16 ? 1 : 0;
      if (split) {
        op.groups = kOprojGroups;
        op.sgrp = plane;
      }
      QMLA_TRY(launch_skinny_gemm(op, s));
      if (split) {
        const int64_t n4 = plane / 4;
        k_add_planes<<<dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, s>>>(
            part, kOprojGroups, plane, n4, out + (size_t)m0 * g.hidden);
        QMLA_LAUNCH_CHECK("k_add_planes");
      }
    }
    return QMLA_OK;
  }

  void *xsp = ws + w.xsplit;
  // q_proj and kv_a_proj_with_mqa share one split of xs
  QMLA_TRY(project(L, xs, n, g.hidden, L->wq, L->wq_x, L->bq, H * (dn + dr), q, s, part,
                   w.part_elems, xsp));
  QMLA_TRY(project(L, xs, n, g.hidden, L->wkva, L->wkva_x, L->bkva, r + dr, kva, s, part,
                   w.part_elems, xsp, false));
  // q's positions are the lengths before this step's append (src/model.rs:267)
  k_split_rope_q<float><<<dim3(n, H), dim3(64), 0, s>>>(q, seq, H, dn, dr, L->inv_freq,
                                                       (float)g.rope_mscale, cache->d_lens, 0, qn,
                                                       qr);
  QMLA_LAUNCH_CHECK("k_split_rope_q");
  QMLA_TRY(latent_to_cache(L, kva, batch, seq, nullptr, cache, s));
  // q_lat[t, h, :] = q_nope[t, h, :] W_UK^h   (batched over heads)
  {
    GemmArgs a{qn, L->wkvb, nullptr, qlat, n, r, dn, (int64_t)H * dn, r, (int64_t)H * r,
               dn, (int64_t)(dn + dv) * r, r, 0};
    QMLA_TRY(gemm(L, a, H, false, s));
  }
  qmla_decode_dims dd{batch, seq * H, r, dr};
  QMLA_TRY(qmla_decode_absorbed(&dd, cache, QMLA_F32, qlat, qr, g.softmax_scale, olat, nullptr,
                                ws + w.dec, dec_bytes, stream));
  // o[t, h, :] = W_UV^h o_lat[t, h, :] + b_V^h
  {
    GemmArgs a{olat, L->wkvb + (size_t)dn * r, L->bkvb ? L->bkvb + dn : nullptr, o, n, dv, r,
               (int64_t)H * r, r, (int64_t)H * dv, r, (int64_t)(dn + dv) * r, dv,
               (int64_t)(dn + dv)};
    QMLA_TRY(gemm(L, a, H, true, s));
  }
  QMLA_TRY(project(L, o, n, H * dv, L->wo, L->wo_x, L->bo, g.hidden, out, s, part,
                   w.part_elems, xsp));
  return QMLA_OK;
}

qmla_status qmla_layer_forward_prefill(const qmla_layer *L, const float *xs, int32_t batch,
                                       int32_t seq, qmla_kv_cache *cache, float *out,
                                       void *workspace, size_t workspace_bytes,
                                       qmla_stream stream) {
  QMLA_TRY(check_layer_call(L, xs, batch, seq, cache, out));
  for (int32_t i = 0; i < batch; ++i)
    QMLA_REQUIRE(cache->h_lens[i] == 0, QMLA_ERR_SHAPE,
                 "forward_prefill starts a sequence: cache length %d of sequence %d must be 0",
                 cache->h_lens[i], i);
  const auto &g = L->cfg;
  const int H = g.heads, dn = g.qk_nope, dr = g.qk_rope, dv = g.v_dim, r = g.kv_lora_rank;
  const LayerWs w = layer_ws(L, batch, seq, 0, WsFor::kPrefill);
  QMLA_REQUIRE(workspace && workspace_bytes >= w.total, QMLA_ERR_WORKSPACE,
               "workspace of %zu bytes < required %zu", workspace_bytes, w.total);
  QMLA_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, QMLA_ERR_WORKSPACE,
               "the workspace must be 256-byte aligned (device allocations are)");
  QMLA_TRY(make_room(cache, 0, batch, seq, as_stream(stream)));
  char *ws = static_cast<char *>(workspace);
  float *q = (float *)(ws + w.q), *kva = (float *)(ws + w.kva), *rows = (float *)(ws + w.rows);
  float *qn = (float *)(ws + w.qn), *qr = (float *)(ws + w.qr), *kvb = (float *)(ws + w.kvb);
  float *k = (float *)(ws + w.k), *v = (float *)(ws + w.v), *kr = (float *)(ws + w.kr);
  float *ctx = (float *)(ws + w.ctx), *o = (float *)(ws + w.o);
  float *part = (float *)(ws + w.part);
  hipStream_t s = as_stream(stream);
  const int n = batch * seq;

  // With a bf16 cache the attention runs on the bf16 MFMA prefill: q, k, v
  // and k_rope are written in bf16 (round to nearest even) into the same
  // regions.  An f32 cache keeps the f32 path throughout.
  const bool bfa = cache->dtype == QMLA_BF16 && prefill_bf16_supported(dn, dr, dv);
  if (use_split_gemm(L) && n >= kSplitGemmMinRows) {
    // Four launches around the attention, all hand-written:
    //   q_proj | kv_a (q split per head and roped in the epilogue, kv_a rows
    //   raw) -> latent rows (LayerNorm, RoPE, cache write) -> kv_b_proj (k, v
    //   per head in the epilogue) -> attention -> o_proj (reading the
    //   head-major context directly)
    SplitGemmArgs a{};
    a.M = n;
    a.seq = seq;
    a.heads = H;
    a.dn = dn;
    a.dr = dr;
    a.dv = dv;
    a.out_bf16 = bfa ? 1 : 0;
    a.ksplit = 1;  // the launcher picks the K slices
    a.part = (float *)(ws + w.sgpart);
    a.bf16ops = L->proj_bf16 ? 1 : 0;
    SplitGemmArgs qa = a;
    qa.w_frag = L->w1f;
    qa.N = H * (dn + dr) + r + dr;
    qa.K = g.hidden;
    qa.x = xs;
    qa.ldx = g.hidden;
    qa.bias = L->b1;
    qa.epi = kSgEpiQkv;
    qa.out0 = qn;
    qa.out1 = qr;
    qa.kva = kva;
    qa.kva_ld = r + dr;
    qa.lens = cache->d_lens;  // 0 here: forward_prefill starts its sequences
    qa.inv_freq = L->inv_freq;
    qa.mscale = (float)g.rope_mscale;
    void *pack = ws + w.pack;
    QMLA_TRY(launch_split_gemm(qa, pack, s));
    // the latent rows: cache rows, kv_b_proj's activation records and k_rope
    uint8_t *krec = reinterpret_cast<uint8_t *>(ws + w.pack2);
    {
      const LatentRowsArgs la = latent_rows_args(L, kva, seq, nullptr, cache);
      const dim3 grid((n + 31) / 32 * 8);  // 4 tokens a block, n rounded up to 32
      // r <= 512 (use_split_gemm): one group of 8 values per lane
      const int rec_lo = L->proj_bf16 ? 0 : 1;
      if (bfa)
        k_prefill_rows<uint16_t, 1><<<grid, dim3(256), 0, s>>>(la, n, krec, rec_lo,
                                                               (uint16_t *)kr, cache->d_lens);
      else
        k_prefill_rows<float, 1><<<grid, dim3(256), 0, s>>>(la, n, krec, rec_lo, kr,
                                                            cache->d_lens);
      QMLA_LAUNCH_CHECK("k_prefill_rows");
      for (int32_t i = 0; i < batch; ++i) cache->h_lens[i] += seq;
    }
    SplitGemmArgs ka = a;
    ka.w_frag = L->wkvbf;
    ka.N = H * (dn + dv);
    ka.K = r;
    ka.bias = L->bkvb;
    ka.epi = kSgEpiKvb;
    ka.out0 = k;
    ka.out1 = v;
    QMLA_TRY(launch_split_gemm_packed(ka, krec, s));
    qmla_prefill_dims pd{batch, H, seq, seq, dn, dr, dv, 1, 0};
    // the bf16 attention can write the context straight as o_proj's
    // activation records (whole 32-token blocks per sequence)
    const bool ctx_rec = bfa && seq % 32 == 0 && prefill_bf16_records_supported(dn, dr, dv);
    if (bfa)
      QMLA_TRY(launch_prefill_bf16(pd, (const uint16_t *)qn, (const uint16_t *)qr,
                                   (const uint16_t *)k, (const uint16_t *)kr, (const uint16_t *)v,
                                   (float)g.softmax_scale, 1,
                                   ctx_rec ? (uint16_t *)pack : (uint16_t *)ctx, s,
                                   ctx_rec ? 1 : 0));
    else
      QMLA_TRY(launch_prefill_f32(pd, qn, qr, k, kr, v, (float)g.softmax_scale, 1, ctx, s));
    SplitGemmArgs oa = a;
    oa.w_frag = L->wof;
    oa.N = g.hidden;
    oa.K = H * dv;
    oa.x = ctx;
    oa.x_heads = 1;
    oa.x_bf16 = bfa ? 1 : 0;
    oa.bias = L->bo;
    oa.epi = kSgEpiFinal;
    oa.y = out;
    oa.ldy = g.hidden;
    if (ctx_rec) return launch_split_gemm_packed(oa, pack, s, /*hi_only=*/true);
    return launch_split_gemm(oa, pack, s);
  }

  void *xsp = ws + w.xsplit;
  // q_proj and kv_a_proj_with_mqa share one split of xs
  QMLA_TRY(project(L, xs, n, g.hidden, L->wq, L->wq_x, L->bq, H * (dn + dr), q, s, part,
                   w.part_elems, xsp));
  QMLA_TRY(project(L, xs, n, g.hidden, L->wkva, L->wkva_x, L->bkva, r + dr, kva, s, part,
                   w.part_elems, xsp, false));
  if (bfa)
    k_split_rope_q<uint16_t><<<dim3(n, H), dim3(64), 0, s>>>(
        q, seq, H, dn, dr, L->inv_freq, (float)g.rope_mscale, cache->d_lens, 1, (uint16_t *)qn,
        (uint16_t *)qr);
  else
    k_split_rope_q<float><<<dim3(n, H), dim3(64), 0, s>>>(
        q, seq, H, dn, dr, L->inv_freq, (float)g.rope_mscale, cache->d_lens, 1, qn, qr);
  QMLA_LAUNCH_CHECK("k_split_rope_q");
  // the latent replacement of the KVCache returned at src/model.rs:250 (the
  // f32 rows also feed compute_kv below)
  QMLA_TRY(latent_to_cache(L, kva, batch, seq, rows, cache, s));
  // compute_kv on the LayerNorm'd latent (src/model.rs:178-190)
  if (n >= kSplitRows && r >= 64) {
    QMLA_TRY(split_act(rows, r + dr, n, r, xsp, s));
    QMLA_TRY(gemm_split(L, static_cast<const uint16_t *>(xsp), 0, n, r, L->wkvb_x, split_cols(r),
                        0, H * (dn + dv), kvb, H * (dn + dv), 0, 1, s));
  } else {
    GemmArgs a{rows, L->wkvb, L->bkvb, kvb, n, H * (dn + dv), r, r + dr, r, (int64_t)H * (dn + dv),
               0, 0, 0, 0};
    QMLA_TRY(gemm(L, a, 1, true, s));
  }
  qmla_prefill_dims pd{batch, H, seq, seq, dn, dr, dv, 1, 0};
  if (bfa) {
    k_split_kv<uint16_t><<<dim3(n, H), dim3(128), 0, s>>>(kvb, seq, H, dn, dv, (uint16_t *)k,
                                                         (uint16_t *)v);
    QMLA_LAUNCH_CHECK("k_split_kv");
    if (dr > 0) {
      k_rows_rope<uint16_t><<<dim3(n), dim3(64), 0, s>>>(rows, r, dr, (uint16_t *)kr);
      QMLA_LAUNCH_CHECK("k_rows_rope");
    }
    QMLA_TRY(launch_prefill_bf16(pd, (const uint16_t *)qn, (const uint16_t *)qr,
                                 (const uint16_t *)k, (const uint16_t *)kr, (const uint16_t *)v,
                                 (float)g.softmax_scale, 1, (uint16_t *)ctx, s));
    k_merge_heads<uint16_t><<<dim3(n, H), dim3(128), 0, s>>>((const uint16_t *)ctx, seq, H, dv, o);
  } else {
    k_split_kv<float><<<dim3(n, H), dim3(128), 0, s>>>(kvb, seq, H, dn, dv, k, v);
    QMLA_LAUNCH_CHECK("k_split_kv");
    if (dr > 0) {
      k_rows_rope<float><<<dim3(n), dim3(64), 0, s>>>(rows, r, dr, kr);
      QMLA_LAUNCH_CHECK("k_rows_rope");
    }
    QMLA_TRY(launch_prefill_f32(pd, qn, qr, k, kr, v, (float)g.softmax_scale, 1, ctx, s));
    k_merge_heads<float><<<dim3(n, H), dim3(128), 0, s>>>(ctx, seq, H, dv, o);
  }
  QMLA_LAUNCH_CHECK("k_merge_heads");
  QMLA_TRY(project(L, o, n, H * dv, L->wo, L->wo_x, L->bo, g.hidden, out, s, part,
                   w.part_elems, xsp));
  return QMLA_OK;
}

qmla_status qmla_cache_materialise_workspace_bytes(const qmla_layer *layer,
                                                   const qmla_kv_cache *cache, int32_t seq0,
                                                   int32_t n_seqs, size_t *bytes) {
  QMLA_REQUIRE(bytes, QMLA_ERR_INVALID_ARG, "bytes is NULL");
  int32_t T = 0;
  QMLA_TRY(check_materialise(layer, cache, seq0, n_seqs, &T));
  *bytes = materialise_ws_bytes(layer, cache, n_seqs, T);
  return QMLA_OK;
}

qmla_status qmla_cache_materialise(const qmla_layer *L, const qmla_kv_cache *cache,
                                   int32_t seq0, int32_t n_seqs, float *k, float *v,
                                   float *k_rope, void *workspace, size_t workspace_bytes,
                                   qmla_stream stream) {
  int32_t T = 0;
  QMLA_TRY(check_materialise(L, cache, seq0, n_seqs, &T));
  const size_t need = materialise_ws_bytes(L, cache, n_seqs, T);
  QMLA_REQUIRE(need == 0 || (workspace && workspace_bytes >= need), QMLA_ERR_WORKSPACE,
               "workspace of %zu bytes < required %zu", workspace_bytes, need);
  if (T == 0) return QMLA_OK;
  const auto &g = L->cfg;
  const int H = g.heads, dn = g.qk_nope, dr = g.qk_rope, dv = g.v_dim, r = g.kv_lora_rank;
  hipStream_t s = as_stream(stream);
  QMLA_REQUIRE(n_seqs <= 65535, QMLA_ERR_SHAPE, "n_seqs %d > 65535", n_seqs);
  const bool bf = cache->dtype == QMLA_BF16;
  if (k_rope && dr > 0) {
    if (bf)
      k_broadcast_rope<uint16_t><<<dim3(T, n_seqs), dim3(256), 0, s>>>(cache->table(), seq0, T, H,
                                                                        r, dr, k_rope);
    else
      k_broadcast_rope<float><<<dim3(T, n_seqs), dim3(256), 0, s>>>(cache->table(), seq0, T, H, r,
                                                                     dr, k_rope);
    QMLA_LAUNCH_CHECK("k_broadcast_rope");
  }
  if (!k && !v) return QMLA_OK;
  if (materialise_split(L, T)) {
    // the c_kv rows in split form, then compute_kv (src/model.rs:178-190)
    // per sequence as one split GEMM batched over heads (bias included)
    uint16_t *xs = static_cast<uint16_t *>(workspace);
    if (bf)
      k_latent_c_split<uint16_t><<<dim3(T, n_seqs), dim3(256), 0, s>>>(cache->table(), seq0, T, r,
                                                                        dr, xs);
    else
      k_latent_c_split<float><<<dim3(T, n_seqs), dim3(256), 0, s>>>(cache->table(), seq0, T, r, dr,
                                                                     xs);
    QMLA_LAUNCH_CHECK("k_latent_c_split");
    const int KX = split_cols(r);
    const int64_t sW = (int64_t)(dn + dv) * KX;
    for (int32_t b = 0; b < n_seqs; ++b) {
      const uint16_t *xb = xs + (size_t)b * T * KX;
      if (k)
        QMLA_TRY(gemm_split(L, xb, 0, T, r, L->wkvb_x, KX, sW, dn, k + (size_t)b * H * T * dn, dn,
                            (int64_t)T * dn, H, s));
      if (v)
        QMLA_TRY(gemm_split(L, xb, 0, T, r, L->wkvb_x + (size_t)dn * KX, KX, sW, dv,
                            v + (size_t)b * H * T * dv, dv, (int64_t)T * dv, H, s));
    }
    return QMLA_OK;
  }
  // the c_kv rows, gathered from the pages into [n, T, r] f32
  float *lat = static_cast<float *>(workspace);
  if (bf)
    k_latent_c_f32<uint16_t><<<dim3(T, n_seqs), dim3(256), 0, s>>>(cache->table(), seq0, T, r,
                                                                    dr, lat);
  else
    k_latent_c_f32<float><<<dim3(T, n_seqs), dim3(256), 0, s>>>(cache->table(), seq0, T, r, dr,
                                                                 lat);
  QMLA_LAUNCH_CHECK("k_latent_c_f32");
  // compute_kv (src/model.rs:178-190) per sequence, batched over heads:
  //   k[b][h] = c_b W_UK^h^T + b_K^h,  v[b][h] = c_b W_UV^h^T + b_V^h
  for (int32_t b = 0; b < n_seqs; ++b) {
    const float *A = lat + (size_t)b * T * r;
    const int64_t lda = r;
    if (k) {
      GemmArgs a{A, L->wkvb, L->bkvb, k + (size_t)b * H * T * dn, T, dn, r, lda, r, dn,
                 0, (int64_t)(dn + dv) * r, (int64_t)T * dn, (int64_t)(dn + dv)};
      QMLA_TRY(gemm(L, a, H, true, s));
    }
    if (v) {
      GemmArgs a{A, L->wkvb + (size_t)dn * r, L->bkvb ? L->bkvb + dn : nullptr,
                 v + (size_t)b * H * T * dv, T, dv, r, lda, r, dv,
                 0, (int64_t)(dn + dv) * r, (int64_t)T * dv, (int64_t)(dn + dv)};
      QMLA_TRY(gemm(L, a, H, true, s));
    }
  }
  return QMLA_OK;
}

}  // extern "C"
