// skinny_gemm.hip -- the Linear projections of an MLA decode step
// (MlaAttention::forward_with_cache, src/model.rs:263-306: q_proj,
// kv_a_proj_with_mqa, the W_UK absorption, W_UV and o_proj) for at most 32
// token rows at a time.
//
// Such a product y[m][n] = sum_k x[m][k] W[n][k] + b[n] (M <= 32 rows, N and
// K in the thousands) is a stream of the weights: every weight is used M
// times.  It runs on bf16 MFMA in an f32-exact split form.  A weight w is
// stored as two bf16 halves w_hi = bf16(w), w_lo = bf16(w - w_hi) (the same
// four bytes per weight as f32, split once when the layer is created), and
// the activations are split the same way in registers, so that
//   x w = x_hi w_hi + x_lo w_hi + x_hi w_lo  (+ x_lo w_lo, below 2^-16 |x w|)
// takes three v_mfma_f32_32x32x16_bf16 with f32 accumulation.  The products
// keep ~16 significant bits of each operand (relative error ~2^-16 per
// product, f32 accumulation), well inside the f32 path's tolerance.  With
// bf16 operands (SkinnyGemmArgs::bf16ops) only w_hi and bf16(x) enter: one
// MFMA per step, and only the hi half of each weight record is read.
//
// Weight layout (fragment-major, built when the layer is created): for z,
// 32-output block nb and 16-wide k-step ks, one 2 KB record at
// ((z * NB + nb) * KS + ks) * 2048 holds the A operand of that MFMA step
// exactly as the wave's lanes read it -- lane l's 16 bytes are the 8 bf16
// weights W[32 nb + l % 32][16 ks + 8 (l / 32) .. + 7], first the hi halves
// of all 64 lanes (1 KB), then the lo halves (1 KB).  Outputs past N are
// zero rows.  Every weight load is thus one contiguous 1 KB wave access,
// and a wave's whole K-slice is one contiguous run.
//
// Work split: block (nb, z) owns 32 outputs (n) of one z (a head for the
// batched per-head products), or half of their K range when the product is
// split over two block groups (twice the blocks: the 114-tile q_proj |
// kv_a product otherwise leaves more than half of the 256 CUs idle, and
// its consumers add the two halves); its NW (<= 8) waves take consecutive
// K-slices.  Each wave streams its A fragments (hi and lo) from HBM into
// registers, two chunks of kChunk steps in flight, reads its B fragments
// (16 k x 32 tokens) from the f32 activations, and accumulates
// C^T[32 n][32 m] in 16 registers.  The NW partial tiles are summed through LDS in slice order
// (deterministic, no atomics) and the block's epilogue adds the bias and
// writes the output in the layout its consumer reads:
//   FINAL  y[m][n]
//   PACKB  the output as the bf16 hi/lo B operand of a following product
//          (hi halves only with bf16 operands)
//          (fragment-major, output index z sy + n as its k), so that product
//          reads its activations as contiguous records without splitting
//   QKV    q_proj | kv_a_proj_with_mqa concatenated: head-split q_nope,
//          roped q_rope (positions lens[b] + i, src/model.rs:263-267) and
//          the raw kv_a rows.
// A launch may carry extra blocks that write the new tokens' latent cache
// rows (latent_rows.hpp), so that the row work of a decode step rides on
// the absorption product's launch instead of a launch of its own.

#include <algorithm>
#include <type_traits>

#include "latent_rows.hpp"

namespace qmla {

namespace {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// (x_hi, x_lo) bf16 halves of 8 f32 values: hi = bf16(x) (round to nearest
// even), lo = bf16(x - hi).
__device__ __forceinline__ void split8(const floatx4_t &a, const floatx4_t &b, bf16x8_t &hi,
                                       bf16x8_t &lo) {
  float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const __bf16 h = (__bf16)v[i];
    hi[i] = h;
    lo[i] = (__bf16)(v[i] - (float)h);
  }
}

// bf16(x) of 8 f32 values (round to nearest even).
__device__ __forceinline__ void hi8(const floatx4_t &a, const floatx4_t &b, bf16x8_t &hi) {
  const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
#pragma unroll
  for (int i = 0; i < 8; ++i) hi[i] = (__bf16)v[i];
}

constexpr int kChunk = 4;  // k-steps of 16 per load group (two groups in flight)

// Byte offset of activation (m, k) in the fragment-major B layout: per
// 16-wide k-step a 2 KB record, hi halves of the 64 lanes then lo halves;
// lane m + 32 h holds k = 16 ks + 8 h .. + 7.
__device__ __forceinline__ int64_t packed_b_offset(int m, int64_t k) {
  return (k >> 4) * 2048 + (int64_t)(m + 32 * ((k >> 3) & 1)) * 16 + (k & 7) * 2;
}

// XM: how the B operand is read -- kXF32 f32 x, kXPacked the pre-split
// fragment-major records, kXSum the f32 sum x + x2 of two planes.  B16: bf16
// operands (the weights' hi halves and bf16(x), one MFMA per step).
constexpr int kXF32 = 0, kXPacked = 1, kXSum = 2;

template <int NW, int XM, bool B16>
__global__ __launch_bounds__(NW * 64) void k_skinny_gemm(SkinnyGemmArgs a, LatentRowsArgs rows,
                                                         int n_rows) {
  // LDS: the waves' partial tiles, or a latent row block's row
  extern __shared__ float smem[];
  float(*red)[16][64] = reinterpret_cast<float(*)[16][64]>(smem);
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int NB = (a.N + 31) / 32;
  // the latent row blocks go first (plane z = 0), then the product's
  if (blockIdx.x < (unsigned)n_rows) {
    if (blockIdx.y == 0) latent_row(rows, blockIdx.x, smem);
    return;
  }
  // tile nb, K-half grp (groups = 2) of plane z
  const int nbg = blockIdx.x - n_rows, z = blockIdx.y;
  if (a.add_n) {
    const int64_t stride = (int64_t)(gridDim.x - n_rows) * gridDim.y * blockDim.x;
    const int64_t i0 = ((int64_t)z * (gridDim.x - n_rows) + nbg) * blockDim.x + threadIdx.x;
    for (int64_t i = i0; i < a.add_n; i += stride) a.add_dst[i] += a.add_src[i];
  }
  const int nb = nbg / a.groups, grp = nbg - nb * a.groups;
  const int n0 = nb * 32;
  const int row = lane & 31, h = lane >> 5;
  const int KS = a.K / 16;
  const int steps = KS / a.groups / NW;  // this wave's k-steps
  const int ks0 = grp * (KS / a.groups) + wave * steps;
  // B columns (tokens) past M load a clamped copy whose outputs are dropped.
  const int64_t brow = min(row, a.M - 1);
  const uint8_t *wf = reinterpret_cast<const uint8_t *>(a.w_frag) +
                      (((int64_t)z * NB + nb) * KS + ks0) * 2048 + lane * 16;
  const float *xp = a.x + z * a.sx + brow * a.ldx + ks0 * 16 + 8 * h;
  const float *xp2 = XM == kXSum ? a.x2 + z * a.sx + brow * a.ldx + ks0 * 16 + 8 * h : nullptr;
  // XP: the activations come pre-split in the fragment-major B layout
  const uint8_t *xf = reinterpret_cast<const uint8_t *>(a.x) + (int64_t)ks0 * 2048 + lane * 16;

  floatx16_t acc;
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.f;
  bf16x8_t ah[2][kChunk], al[2][kChunk];
  floatx4_t xa[2][kChunk], xb[2][kChunk];
  // Loads are unconditional (steps past the wave's last one re-read the
  // last step and their MFMAs are skipped), so that the compiler counts the
  // loads in flight exactly and waits only for the chunk it computes on.
  auto load = [&](int buf, int s0) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      const int st = min(s0 + c, steps - 1);
      const uint8_t *f = wf + (int64_t)st * 2048;
      ah[buf][c] = *reinterpret_cast<const bf16x8_t *>(f);
      if constexpr (!B16) al[buf][c] = *reinterpret_cast<const bf16x8_t *>(f + 1024);
      if constexpr (XM == kXPacked) {
        xa[buf][c] = *reinterpret_cast<const floatx4_t *>(xf + (int64_t)st * 2048);
        if constexpr (!B16)
          xb[buf][c] = *reinterpret_cast<const floatx4_t *>(xf + (int64_t)st * 2048 + 1024);
      } else if constexpr (XM == kXSum) {
        xa[buf][c] = *reinterpret_cast<const floatx4_t *>(xp + st * 16) +
                     *reinterpret_cast<const floatx4_t *>(xp2 + st * 16);
        xb[buf][c] = *reinterpret_cast<const floatx4_t *>(xp + st * 16 + 4) +
                     *reinterpret_cast<const floatx4_t *>(xp2 + st * 16 + 4);
      } else {
        xa[buf][c] = *reinterpret_cast<const floatx4_t *>(xp + st * 16);
        xb[buf][c] = *reinterpret_cast<const floatx4_t *>(xp + st * 16 + 4);
      }
    }
  };
  auto compute = [&](int buf, int s0) __attribute__((always_inline)) {
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      if (s0 + c < steps) {
        bf16x8_t xh, xl;
        if constexpr (XM == kXPacked) {
          xh = __builtin_bit_cast(bf16x8_t, xa[buf][c]);
          if constexpr (!B16) xl = __builtin_bit_cast(bf16x8_t, xb[buf][c]);
        } else if constexpr (B16) {
          hi8(xa[buf][c], xb[buf][c], xh);
        } else {
          split8(xa[buf][c], xb[buf][c], xh, xl);
        }
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[buf][c], xh, acc, 0, 0, 0);
        if constexpr (!B16) {
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah[buf][c], xl, acc, 0, 0, 0);
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al[buf][c], xh, acc, 0, 0, 0);
        }
      }
    }
  };
  // two chunks in flight: the loads of chunk i + 1 go out before the MFMAs
  // of chunk i
  load(0, 0);
  int s0 = 0;
  for (; s0 + 2 * kChunk < steps; s0 += 2 * kChunk) {
    load(1, s0 + kChunk);
    compute(0, s0);
    load(0, s0 + 2 * kChunk);
    compute(1, s0 + kChunk);
  }
  if (s0 + kChunk < steps) {
    load(1, s0 + kChunk);
    compute(0, s0);
    compute(1, s0 + kChunk);
  } else {
    compute(0, s0);
  }
  // element j of lane l: output n0 + 8 (j / 4) + 4 (l / 32) + j % 4, token l % 32
#pragma unroll
  for (int j = 0; j < 16; ++j) red[wave][j][lane] = acc[j];
  __syncthreads();
  const float *bias = a.bias && grp == 0 ? a.bias + z * a.sb : nullptr;
  // epilogue over pairs (j, j + 1), j even: adjacent outputs of one token
  for (int e = threadIdx.x; e < 8 * 64; e += NW * 64) {
    const int j = 2 * (e >> 6), l = e & 63;
    float v0 = 0.f, v1 = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      v0 += red[w][j][l];
      v1 += red[w][j + 1][l];
    }
    const int m = l & 31;
    const int n = n0 + 8 * (j >> 2) + 4 * (l >> 5) + (j & 3);  // even
    if (m >= a.M || n >= a.N) continue;
    if (bias) {
      v0 += bias[n];
      if (n + 1 < a.N) v1 += bias[n + 1];
    }
    if (a.mode == kSkinnyFinal) {
      float *y = a.y + z * a.sy + grp * a.sgrp + (int64_t)m * a.ldy + n;
      y[0] = v0;
      if (n + 1 < a.N) y[1] = v1;
      continue;
    }
    if (a.mode == kSkinnyPackB) {
      // output (m, z sy + n) as the bf16 hi/lo B operand of the next product
      uint8_t *yb = reinterpret_cast<uint8_t *>(a.y);
      const int64_t k = z * a.sy + n;
      const float v[2] = {v0, v1};
      for (int q = 0; q < 2 && n + q < a.N; ++q) {
        const uint16_t hi = f32_to_bf16_bits(v[q]);
        const uint16_t lo = f32_to_bf16_bits(v[q] - bf16_bits_to_f32(hi));
        const int64_t off = packed_b_offset(m, k + q);
        *reinterpret_cast<uint16_t *>(yb + off) = hi;
        if constexpr (!B16) *reinterpret_cast<uint16_t *>(yb + off + 1024) = lo;
      }
      continue;
    }
    // kSkinnyQkv: n in [0, H (dn + dr)) is q_proj's output, the rest kv_a
    const int qw = a.dn + a.dr, hq = a.heads * qw;
    const int mg = a.m0 + m;  // token index in the whole call
    if (n >= hq) {
      float *y = (grp ? a.kva1 : a.kva) + (int64_t)mg * a.kva_ld + (n - hq);
      y[0] = v0;
      y[1] = v1;
      continue;
    }
    const int hd = n / qw, d = n - hd * qw;
    if (d < a.dn) {
      float *y = (grp ? a.q_nope1 : a.q_nope) + ((int64_t)mg * a.heads + hd) * a.dn + d;
      y[0] = v0;
      y[1] = v1;
    } else {
      // interleaved pair (2p, 2p + 1) of q_rope (src/model.rs:70-84); the
      // rotation is linear, so each K-half is rotated on its own
      const int p = (d - a.dn) >> 1;
      const int b = mg / a.seq, i = mg - b * a.seq;
      const float pos = (float)(a.lens[b] + i);
      const float ang = pos * a.inv_freq[p];
      float cs, sn;
      rope_cs(ang, a.mscale, cs, sn);
      float *y = (grp ? a.q_rope1 : a.q_rope) + ((int64_t)mg * a.heads + hd) * a.dr + 2 * p;
      y[0] = v0 * cs - v1 * sn;
      y[1] = v1 * cs + v0 * sn;
    }
  }
}

}  // namespace

// Waves per block: the split of a block's K range, up to 8, with each
// wave's range a multiple of 16 and at least 64 wide when K allows.  Eight
// waves time ~10% below sixteen at K = 2048 (a block's time is set by what
// one CU moves -- its weight slab plus the activations -- and sixteen waves
// only add the reduction through LDS).
int skinny_waves(int K) {
  int nw = 8;
  while (nw > 1 && (K % (16 * nw) != 0 || K / nw < 64)) nw >>= 1;
  return K % (16 * nw) == 0 ? nw : 0;
}

size_t skinny_frag_bytes(int N, int K, int Z) {
  return (size_t)Z * ((N + 31) / 32) * (K / 16) * 2048;
}

void skinny_pack(const float *W, int64_t ldw, int64_t sw, int N, int K, int Z, uint8_t *out) {
  const int NB = (N + 31) / 32, KS = K / 16;
  for (int z = 0; z < Z; ++z)
    for (int nb = 0; nb < NB; ++nb)
      for (int ks = 0; ks < KS; ++ks) {
        uint16_t *rec = reinterpret_cast<uint16_t *>(out + (((size_t)z * NB + nb) * KS + ks) * 2048);
        for (int l = 0; l < 64; ++l) {
          const int n = nb * 32 + (l & 31), k = ks * 16 + 8 * (l >> 5);
          for (int e = 0; e < 8; ++e) {
            const float w = n < N ? W[z * sw + (int64_t)n * ldw + k + e] : 0.f;
            const uint16_t hi = f32_to_bf16_bits(w);
            rec[l * 8 + e] = hi;
            rec[512 + l * 8 + e] = f32_to_bf16_bits(w - bf16_bits_to_f32(hi));
          }
        }
      }
}

bool skinny_supported(int M, int K) { return M >= 1 && M <= 32 && K > 0 && skinny_waves(K) > 0; }

qmla_status launch_skinny_gemm(const SkinnyGemmArgs &a, hipStream_t stream,
                               const LatentRowsArgs *rows, int n_rows) {
  const int G = a.groups ? a.groups : 1;
  QMLA_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, QMLA_ERR_SHAPE, "skinny GEMM groups %d", G);
  QMLA_REQUIRE(a.K % (16 * G) == 0 && skinny_supported(a.M, a.K / G), QMLA_ERR_UNSUPPORTED,
               "skinny GEMM M %d K %d groups %d", a.M, a.K, G);
  QMLA_REQUIRE(a.N > 0 && a.Z > 0 && a.Z <= 65535, QMLA_ERR_SHAPE, "skinny GEMM N %d Z %d", a.N,
               a.Z);
  QMLA_REQUIRE(a.mode != kSkinnyQkv || (a.N % 2 == 0 && a.dn % 2 == 0 && a.dr % 2 == 0),
               QMLA_ERR_SHAPE, "q/kv split needs even widths");
  QMLA_REQUIRE(G == 1 || (a.mode == kSkinnyQkv && G == 2 && a.q_nope1 && a.q_rope1 && a.kva1) ||
                   (a.mode == kSkinnyFinal && a.sgrp >= (int64_t)a.Z * a.sy &&
                    a.sgrp >= (int64_t)a.M * a.ldy),
               QMLA_ERR_SHAPE, "a K split needs a destination plane per group");
  QMLA_REQUIRE(!(a.x_packed && a.x2), QMLA_ERR_SHAPE, "packed activations have one plane");
  const int nw = skinny_waves(a.K / G);
  const int extra = rows ? n_rows : 0;
  LatentRowsArgs ra{};
  if (rows) ra = *rows;
  SkinnyGemmArgs args = a;
  args.groups = G;
  dim3 grid((unsigned)((a.N + 31) / 32 * G + extra), (unsigned)a.Z);
  const size_t lds = std::max(sizeof(float) * nw * 16 * 64,
                              rows ? latent_row_lds_bytes(rows->r, rows->dr) : 0);
  if (a.x_packed) QMLA_REQUIRE(a.Z == 1, QMLA_ERR_SHAPE, "packed activations need Z = 1");
  auto go2 = [&](auto xm, auto b16) {
    constexpr int XM = decltype(xm)::value;
    constexpr bool B16 = decltype(b16)::value;
    switch (nw) {
      case 8: k_skinny_gemm<8, XM, B16><<<grid, dim3(512), lds, stream>>>(args, ra, extra); break;
      case 4: k_skinny_gemm<4, XM, B16><<<grid, dim3(256), lds, stream>>>(args, ra, extra); break;
      case 2: k_skinny_gemm<2, XM, B16><<<grid, dim3(128), lds, stream>>>(args, ra, extra); break;
      default: k_skinny_gemm<1, XM, B16><<<grid, dim3(64), lds, stream>>>(args, ra, extra); break;
    }
  };
  auto go = [&](auto xm) {
    if (a.bf16ops)
      go2(xm, std::true_type{});
    else
      go2(xm, std::false_type{});
  };
  if (a.x_packed)
    go(std::integral_constant<int, kXPacked>{});
  else if (a.x2)
    go(std::integral_constant<int, kXSum>{});
  else
    go(std::integral_constant<int, kXF32>{});
  QMLA_LAUNCH_CHECK("k_skinny_gemm");
  return QMLA_OK;
}

}  // namespace qmla
