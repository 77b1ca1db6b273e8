// decode_mfma.hip -- bf16 MFMA core of the absorbed-latent MLA decode.
//
// Replaces the batched GEMVs of MlaAttention::forward_with_cache
// (src/model.rs:297-303) for a bf16 latent cache.  All heads share one
// latent row per token, so a block keeps up to 128 query rows (4 waves x
// 32) resident and streams each cached token through LDS exactly once:
//
//   S^T[t][h] = sum_k C[t][k] Q[h][k]         (32x32x16 MFMA, M = tokens)
//   p = exp2(S^T * scale*log2(e) - m)          (online softmax, f32)
//   O^T[c][h] += sum_t V^T[c][t] P^T[t][h]    (32x32x16 MFMA, M = latent cols)
//
// with V = C[:, :r].  The S^T accumulator layout (lane = head, 16 tokens
// per lane) is exactly the B-operand layout P^T needs, so P never leaves
// registers; V^T comes from the token-major tile via ds_read_b64_tr_b16.
//
// Tiles of 32 tokens are copied global -> LDS by direct-to-LDS loads
// (global_load_lds_dwordx4) into an NSTAGE ring, so several tiles are in
// flight without staging registers.  LDS rows are padded to 73 16-byte
// chunks (1168 B), which keeps the A-operand reads (16 rows x 16 B per
// quarter-wave) free of bank conflicts.

#include <cmath>

#include "internal.hpp"

namespace qmla {

namespace {

constexpr int kTok = 32;  // tokens per tile

template <int R, int DR>
struct DecodeShape {
  static constexpr int W = R + DR;                  // latent row width
  static constexpr int KSTEPS = W / 16;             // S k-steps
  static constexpr int CB = R / 32;                 // PV column blocks
  static constexpr int CHUNKS = W / 8;              // 16-byte chunks per row
  static constexpr int RS = CHUNKS + 1;             // padded LDS row stride (chunks)
  static constexpr int INSTR = (kTok * RS + 63) / 64;  // DMA instructions per tile
  static constexpr int SLOTS = INSTR * 64;          // 16-byte slots per stage
  static_assert(R % 32 == 0 && W % 16 == 0, "unsupported latent shape");
};

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ void wait_vmcnt_dyn(int n) {
  // n is wave-uniform; dispatch to an immediate.
  switch (n) {
#define QMLA_W(k) case k: wait_vmcnt<k>(); break;
    QMLA_W(0) QMLA_W(1) QMLA_W(2) QMLA_W(3) QMLA_W(4) QMLA_W(5) QMLA_W(6) QMLA_W(7)
    QMLA_W(8) QMLA_W(9) QMLA_W(10) QMLA_W(11) QMLA_W(12) QMLA_W(13) QMLA_W(14) QMLA_W(15)
    QMLA_W(16) QMLA_W(17) QMLA_W(18) QMLA_W(19) QMLA_W(20) QMLA_W(21) QMLA_W(22) QMLA_W(23)
    QMLA_W(24) QMLA_W(25) QMLA_W(26) QMLA_W(27) QMLA_W(28) QMLA_W(29) QMLA_W(30) QMLA_W(31)
    QMLA_W(32) QMLA_W(33) QMLA_W(34) QMLA_W(35) QMLA_W(36) QMLA_W(37) QMLA_W(38) QMLA_W(39)
    QMLA_W(40) QMLA_W(41) QMLA_W(42) QMLA_W(43) QMLA_W(44) QMLA_W(45) QMLA_W(46) QMLA_W(47)
    QMLA_W(48) QMLA_W(49) QMLA_W(50) QMLA_W(51) QMLA_W(52) QMLA_W(53) QMLA_W(54) QMLA_W(55)
    QMLA_W(56) QMLA_W(57) QMLA_W(58) QMLA_W(59) QMLA_W(60) QMLA_W(61) QMLA_W(62)
#undef QMLA_W
    default: wait_vmcnt<0>(); break;
  }
}

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4;
typedef __attribute__((address_space(3))) bf16x8_t lds_bf16x8;

// o *= alpha for a 16-float MFMA accumulator.  Done through inline asm with
// AGPR operands, one value at a time through a VGPR, so the 256 accumulator
// registers of a wave stay in AGPRs (a VALU multiply on them would make the
// register allocator move them to arch VGPRs, which do not have room).
__device__ __forceinline__ void agpr_scale16(floatx16_t &o, float alpha) {
  float e[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) e[i] = o[i];
  float tmp;
#define QMLA_S1(i) "v_accvgpr_read_b32 %16, %" #i "\n v_mul_f32 %16, %16, %17\n v_accvgpr_write_b32 %" #i ", %16\n"
  asm volatile(QMLA_S1(0) QMLA_S1(1) QMLA_S1(2) QMLA_S1(3) QMLA_S1(4) QMLA_S1(5) QMLA_S1(6)
                   QMLA_S1(7) QMLA_S1(8) QMLA_S1(9) QMLA_S1(10) QMLA_S1(11) QMLA_S1(12)
                       QMLA_S1(13) QMLA_S1(14) QMLA_S1(15)
               : "+a"(e[0]), "+a"(e[1]), "+a"(e[2]), "+a"(e[3]), "+a"(e[4]), "+a"(e[5]),
                 "+a"(e[6]), "+a"(e[7]), "+a"(e[8]), "+a"(e[9]), "+a"(e[10]), "+a"(e[11]),
                 "+a"(e[12]), "+a"(e[13]), "+a"(e[14]), "+a"(e[15]), "=&v"(tmp)
               : "v"(alpha));
#undef QMLA_S1
#pragma unroll
  for (int i = 0; i < 16; ++i) o[i] = e[i];
}

__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v;
  v[0] = (__bf16)a;  // v_cvt_pk_bf16_f32: round to nearest even
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// Issue this wave's share of the DMA instructions for one tile.  Slot s of
// the stage holds chunk (s % RS) of tile row (s / RS); pad slots and rows
// past the segment end re-load a valid chunk (never read back).
template <class SH, int NW>
__device__ __forceinline__ void issue_tile(const uint8_t *__restrict__ seq_base, int tile_t0,
                                           int seg_t1, lds_char *stage, int wave, int lane) {
  for (int ins = wave; ins < SH::INSTR; ins += NW) {
    const int s = ins * 64 + lane;
    int t = s / SH::RS, c = s - t * SH::RS;
    if (t >= kTok || c >= SH::CHUNKS) {
      t = 0;
      c = 0;
    }
    int tok = tile_t0 + t;
    tok = tok < seg_t1 ? tok : seg_t1 - 1;
    const uint8_t *src = seq_base + (int64_t)tok * (SH::W * 2) + c * 16;
    __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)(stage + ins * 1024), 16, 0,
                                     0);
  }
}

template <class SH, int NW>
__device__ __forceinline__ constexpr int instr_of_wave(int wave) {
  return (SH::INSTR - wave + NW - 1) / NW;
}

template <int R, int DR, typename QT>
__device__ __forceinline__ bf16x8_t load_q8(const QT *__restrict__ q_lat,
                                            const QT *__restrict__ q_rope, int64_t qrow, int d0) {
  const QT *src = d0 < R ? q_lat + qrow * R + d0 : q_rope + qrow * DR + (d0 - R);
  if constexpr (sizeof(QT) == 2) {
    return *reinterpret_cast<const bf16x8_t *>(src);
  } else {
    const floatx4_t a = *reinterpret_cast<const floatx4_t *>(src);
    const floatx4_t b = *reinterpret_cast<const floatx4_t *>(src + 4);
    u32x4_t p;
    p[0] = pack2_bf16(a[0], a[1]);
    p[1] = pack2_bf16(a[2], a[3]);
    p[2] = pack2_bf16(b[0], b[1]);
    p[3] = pack2_bf16(b[2], b[3]);
    return __builtin_bit_cast(bf16x8_t, p);
  }
}

template <int R, int DR, int NW, int NSTAGE, typename QT>
__global__ __launch_bounds__(NW * 64) void k_decode_mfma(
    const uint8_t *__restrict__ pool, const int64_t *__restrict__ offsets,
    const QT *__restrict__ q_lat, const QT *__restrict__ q_rope, int32_t rows,
    float scale_log2, DecodePlanView plan, float *__restrict__ out, float *__restrict__ out_lse,
    float *__restrict__ part_o, float *__restrict__ part_lse) {
  using SH = DecodeShape<R, DR>;
  constexpr int STAGE_BYTES = SH::SLOTS * 16;
  constexpr int ROW_BYTES = SH::RS * 16;
  extern __shared__ __attribute__((aligned(16))) char ring_raw[];
  lds_char *ring = (lds_char *)ring_raw;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int n = lane & 31;     // head (query row) within the wave = MFMA column
  const int half = lane >> 5;  // which 8-wide k half of an MFMA operand
  const int row = blockIdx.y * (NW * 32) + wave * 32 + n;  // query row
  const bool row_ok = row < rows;
  const int row_c = row_ok ? row : rows - 1;
  const int piece = blockIdx.x;
  const int my_instr = instr_of_wave<SH, NW>(wave);

  // Per-lane LDS byte offsets inside a stage.
  //  S^T A operand (tokens x dims): row n, chunk 2*kk + half -> + kk*32.
  const int a_off = (n * SH::RS + half) * 16;
  //  V^T A operand via ds_read_b64_tr_b16: 16-lane group g reads 4 tokens x
  //  16 columns; lane sl supplies token tok_a + ..., columns col_in..+3.
  const int g = lane >> 4, sl = lane & 15;
  const int tok_a = (g >= 2 ? 4 : 0) + (sl >> 2);
  const int col_in = (g & 1) * 16 + 4 * (sl & 3);
  const int v_off = tok_a * ROW_BYTES + (col_in >> 3) * 16 + (col_in & 7) * 2;

  const int32_t s0 = plan.seg_start[piece], s1 = plan.seg_start[piece + 1];
  for (int32_t si = s0; si < s1; ++si) {
    const DecodeSegment sg = plan.segs[si];
    const int64_t qrow = (int64_t)sg.seq * rows + row;
    const int64_t qrow_c = (int64_t)sg.seq * rows + row_c;
    const uint8_t *seq_base = pool + offsets[sg.seq] * (int64_t)(SH::W * 2);

    // Q fragment = B operand of S^T: dims kk*16 + 8*half .. +7 of this row.
    bf16x8_t qf[SH::KSTEPS];
#pragma unroll
    for (int kk = 0; kk < SH::KSTEPS; ++kk) {
      bf16x8_t v = load_q8<R, DR, QT>(q_lat, q_rope, qrow_c, kk * 16 + half * 8);
      u32x4_t u = __builtin_bit_cast(u32x4_t, v);
      const uint32_t keep = row_ok ? 0xffffffffu : 0u;
      u[0] &= keep;
      u[1] &= keep;
      u[2] &= keep;
      u[3] &= keep;
      qf[kk] = __builtin_bit_cast(bf16x8_t, u);
    }

    floatx16_t o[SH::CB];
#pragma unroll
    for (int cb = 0; cb < SH::CB; ++cb)
#pragma unroll
      for (int j = 0; j < 16; ++j) o[cb][j] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    const int T = sg.t1 - sg.t0;
    const int ntiles = (T + kTok - 1) / kTok;
    const int seg_end = sg.t1;
#pragma unroll
    for (int p = 0; p < NSTAGE - 1; ++p)
      if (p < ntiles)
        issue_tile<SH, NW>(seq_base, sg.t0 + p * kTok, seg_end, ring + p * STAGE_BYTES, wave,
                           lane);

    for (int it = 0; it < ntiles; ++it) {
      const int nxt = it + NSTAGE - 1;
      if (nxt < ntiles)
        issue_tile<SH, NW>(seq_base, sg.t0 + nxt * kTok, seg_end,
                           ring + (nxt % NSTAGE) * STAGE_BYTES, wave, lane);
      // Tiles it+1 .. min(nxt, ntiles-1) may stay in flight.
      const int ahead = (nxt < ntiles ? nxt : ntiles - 1) - it;
      wait_vmcnt_dyn(ahead * my_instr);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);

      const lds_char *stage = ring + (it % NSTAGE) * STAGE_BYTES;
      const lds_char *pa = stage + a_off;
      const lds_char *pv = stage + v_off;
      // ---- S^T = C Q^T over the 32 tokens of this tile
      floatx16_t s;
#pragma unroll
      for (int j = 0; j < 16; ++j) s[j] = 0.f;
#pragma unroll
      for (int kk = 0; kk < SH::KSTEPS; ++kk) {
        const bf16x8_t a = *reinterpret_cast<const lds_bf16x8 *>(pa + kk * 32);
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[kk], s, 0, 0, 0);
      }
      // Keep 4 operand reads in flight ahead of the MFMA chain.
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int kk = 0; kk < SH::KSTEPS - 4; ++kk) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
      __builtin_amdgcn_sched_barrier(0);
      // ---- online softmax (log2 domain); lane holds 16 tokens of head n
      const int tile_t0 = it * kTok;  // relative to the segment
      float mt = -INFINITY;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int tok = tile_t0 + 8 * (j >> 2) + 4 * half + (j & 3);
        const float x = tok < T ? s[j] * scale_log2 : -INFINITY;
        s[j] = x;
        mt = fmaxf(mt, x);
      }
      mt = xor32_max(mt);
      // Lazy rescaling: keep the running reference unless the tile max
      // exceeds it by more than 8 (a factor 256); p stays <= 256.
      if (m_run == -INFINITY || mt > m_run + 8.f) {
        const float m_new = fmaxf(mt, m_run);
        const float alpha = m_run == -INFINITY ? 0.f : exp2f(m_run - m_new);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int cb = 0; cb < SH::CB; ++cb) agpr_scale16(o[cb], alpha);
      }
      u32x4_t pk[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p0 = exp2f(s[ks * 8 + 2 * i] - m_run);
          const float p1 = exp2f(s[ks * 8 + 2 * i + 1] - m_run);
          l_run += p0 + p1;
          pk[ks][i] = pack2_bf16(p0, p1);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      // ---- O^T += V^T P^T
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8_t pb = __builtin_bit_cast(bf16x8_t, pk[ks]);
#pragma unroll
        for (int cb = 0; cb < SH::CB; ++cb) {
          const lds_char *p1 = pv + ks * 16 * ROW_BYTES + cb * 64;
          const bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)p1);
          const bf16x4_t hi =
              __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)(p1 + 8 * ROW_BYTES));
          const bf16x8_t a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          o[cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb, o[cb], 0, 0, 0);
        }
      }
      // Keep 3 MFMAs' worth of transposed reads in flight.
      __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
      for (int i = 0; i < 2 * SH::CB - 3; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 3, 0);
      __builtin_amdgcn_sched_barrier(0);
      // Every wave must be done reading this stage before it is refilled.
      __builtin_amdgcn_s_waitcnt((0xF) | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
      __builtin_amdgcn_s_barrier();
    }

    // ---- finalise: combine the two half-waves' denominators
    l_run = xor32_sum(l_run);
    const float inv = 1.f / l_run;
    const float lse = (m_run + log2f(l_run)) * 0.69314718055994531f;
    if (row_ok) {
      float *dst;
      if (sg.slot < 0) {
        dst = out + qrow * R;
        if (out_lse && half == 0) out_lse[qrow] = lse;
      } else {
        const int64_t prow = (int64_t)sg.slot * rows + row;
        dst = part_o + prow * R;
        if (half == 0) part_lse[prow] = lse;
      }
#pragma unroll
      for (int cb = 0; cb < SH::CB; ++cb)
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
          floatx4_t v;
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = o[cb][jq * 4 + i] * inv;
          *reinterpret_cast<floatx4_t *>(dst + cb * 32 + 8 * jq + 4 * half) = v;
        }
    }
  }
}

template <int R, int DR, int NW, int NSTAGE>
qmla_status launch_shape(const DecodeArgs &a, hipStream_t stream) {
  using SH = DecodeShape<R, DR>;
  const size_t lds = (size_t)NSTAGE * SH::SLOTS * 16;
  const int passes = (a.rows + NW * 32 - 1) / (NW * 32);
  dim3 grid(a.blocks, passes), block(NW * 64);
  const float sl2 = a.scale * 1.4426950408889634f;
  const uint8_t *pool = static_cast<const uint8_t *>(a.cache->rows);
  if (a.q_dtype == QMLA_BF16) {
    auto k = k_decode_mfma<R, DR, NW, NSTAGE, uint16_t>;
    QMLA_HIP(hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 (int)lds));
    k<<<grid, block, lds, stream>>>(pool, a.cache->d_offsets, (const uint16_t *)a.q_lat,
                                    (const uint16_t *)a.q_rope, a.rows, sl2, a.plan, a.out,
                                    a.out_lse, a.part_o, a.part_lse);
  } else {
    auto k = k_decode_mfma<R, DR, NW, NSTAGE, float>;
    QMLA_HIP(hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 (int)lds));
    k<<<grid, block, lds, stream>>>(pool, a.cache->d_offsets, (const float *)a.q_lat,
                                    (const float *)a.q_rope, a.rows, sl2, a.plan, a.out,
                                    a.out_lse, a.part_o, a.part_lse);
  }
  QMLA_LAUNCH_CHECK("k_decode_mfma");
  return QMLA_OK;
}

template <int R, int DR>
qmla_status launch_dims(const DecodeArgs &a, hipStream_t stream) {
  if (a.rows <= 32) return launch_shape<R, DR, 1, 2>(a, stream);
  if (a.rows <= 64) return launch_shape<R, DR, 2, 2>(a, stream);
  return launch_shape<R, DR, 4, 4>(a, stream);
}

}  // namespace

bool decode_mfma_supported(int32_t rows, int32_t r, int32_t dr) {
  (void)rows;
  return (r == 512 && dr == 64) || (r == 64 && dr == 16) || (r == 128 && dr == 32);
}

int decode_mfma_blocks_per_cu(int32_t rows) { return rows <= 64 ? 2 : 1; }

qmla_status launch_decode_mfma(const DecodeArgs &a, hipStream_t stream) {
  QMLA_REQUIRE(a.rows <= 65535 * 128, QMLA_ERR_SHAPE, "too many query rows");
  if (a.r == 512 && a.dr == 64) return launch_dims<512, 64>(a, stream);
  if (a.r == 64 && a.dr == 16) return launch_dims<64, 16>(a, stream);
  if (a.r == 128 && a.dr == 32) return launch_dims<128, 32>(a, stream);
  return fail(QMLA_ERR_UNSUPPORTED, "bf16 decode for kv_lora_rank %d, rope %d", a.r, a.dr);
}

}  // namespace qmla
