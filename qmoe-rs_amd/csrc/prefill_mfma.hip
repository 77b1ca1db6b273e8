// prefill_mfma.hip -- bf16 MFMA flash prefill (causal, chunk offset).
//
// Replaces the tiled candle matmuls of fused_prefill_attn
// (src/attention_kernel.rs:64-107) for bf16 inputs with f32 accumulation.
// Per block: 4 waves x 64 query rows of one (b, h).  Per 32-key tile:
//
//   S^T[key][q] = sum_d K[key][d] Q[q][d]       d over [k_nope | k_rope]
//   P^T = exp2(S^T * scale*log2(e) - m)          online softmax, f32
//   O^T[c][q] += sum_key V^T[c][key] P^T[key][q]
//
// As in the decode kernel, the S^T accumulator (lane = query row, 16 keys
// per lane) is used directly as the B operand of the P.V product, and V^T
// is read from the key-major tile with ds_read_b64_tr_b16.  Each wave
// covers two 32-row column blocks so every K / V^T operand read feeds two
// MFMAs.  Key tiles above a wave's causal horizon are skipped (exact: the
// reference's -1e18 mask gives exp() == 0); blocks are issued heaviest
// first so the causal triangle balances across compute units.

#include <cmath>

#include "internal.hpp"

namespace qmla {

namespace {

constexpr int kPKeys = 32;      // keys per tile
constexpr int kPWaves = 4;
constexpr int kPRowsWave = 64;  // two 32-row MFMA column blocks
constexpr int kPRows = kPWaves * kPRowsWave;
constexpr int kPStages = 4;

typedef __attribute__((address_space(3))) void lds_void_p;
typedef __attribute__((address_space(3))) char lds_char_p;
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4_p;
typedef __attribute__((address_space(3))) bf16x8_t lds_bf16x8_p;

template <int DN_, int DR_, int DV_>
struct PrefillShape {
  static constexpr int DN = DN_, DR = DR_, DV = DV_;
  static constexpr int DQK = DN + DR;
  static constexpr int KSTEPS = DQK / 16;
  static constexpr int CB = DV / 32;
  static constexpr int NCH = DN / 8;            // 16-byte chunks of k_nope
  static constexpr int KCH = DQK / 8;           // 16-byte chunks of a K row
  static constexpr int KRS = KCH + 1;           // padded K row stride (chunks)
  static constexpr int VCH = DV / 8;
  static constexpr int VRS = VCH + 1;           // padded V row stride (chunks)
  static constexpr int KSLOTS = kPKeys * KRS;
  static constexpr int VSLOTS = kPKeys * VRS;
  static constexpr int INSTR = (KSLOTS + VSLOTS + 63) / 64;
  static constexpr int STAGE_BYTES = INSTR * 64 * 16;
  static constexpr int V_BASE = KSLOTS * 16;    // byte offset of the V tile in a stage
  static_assert(DN % 8 == 0 && DR % 8 == 0 && DQK % 16 == 0 && DV % 32 == 0, "bad dims");
  static_assert((INSTR + kPWaves - 1) / kPWaves * (kPStages - 1) < 64, "vmcnt overflow");
};

template <int N>
__device__ __forceinline__ void pwait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ void pwait_vmcnt_dyn(int n) {
  switch (n) {
#define QMLA_W(k) case k: pwait_vmcnt<k>(); break;
    QMLA_W(0) QMLA_W(1) QMLA_W(2) QMLA_W(3) QMLA_W(4) QMLA_W(5) QMLA_W(6) QMLA_W(7)
    QMLA_W(8) QMLA_W(9) QMLA_W(10) QMLA_W(11) QMLA_W(12) QMLA_W(13) QMLA_W(14) QMLA_W(15)
    QMLA_W(16) QMLA_W(17) QMLA_W(18) QMLA_W(19) QMLA_W(20) QMLA_W(21) QMLA_W(22) QMLA_W(23)
    QMLA_W(24) QMLA_W(25) QMLA_W(26) QMLA_W(27) QMLA_W(28) QMLA_W(29) QMLA_W(30) QMLA_W(31)
    QMLA_W(32) QMLA_W(33) QMLA_W(34) QMLA_W(35) QMLA_W(36) QMLA_W(37) QMLA_W(38) QMLA_W(39)
#undef QMLA_W
    default: pwait_vmcnt<0>(); break;
  }
}

// o *= alpha on an MFMA accumulator kept in AGPRs (see decode_mfma.hip).
__device__ __forceinline__ void pagpr_scale16(floatx16_t &o, float alpha) {
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

__device__ __forceinline__ uint32_t ppack2_bf16(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v;
  v[0] = (__bf16)a;  // v_cvt_pk_bf16_f32, round to nearest even
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// One stage = K tile (32 keys x [k_nope | k_rope], padded rows) followed by
// the V tile (32 keys x dv, padded rows).  Slot s of the stage is written by
// DMA instruction s / 64, lane s % 64.  Keys past seq_k and pad slots
// re-load a valid chunk that is never read back.
template <class SH>
__device__ __forceinline__ void pissue_tile(const uint8_t *__restrict__ kb,
                                            const uint8_t *__restrict__ krb,
                                            const uint8_t *__restrict__ vb, int key0, int seq_k,
                                            lds_char_p *stage, int wave, int lane) {
  for (int ins = wave; ins < SH::INSTR; ins += kPWaves) {
    const int s = ins * 64 + lane;
    const uint8_t *src;
    if (s < SH::KSLOTS) {
      const int t = s / SH::KRS, c = s - t * SH::KRS;
      int key = key0 + t;
      key = key < seq_k ? key : seq_k - 1;
      if (c < SH::NCH)
        src = kb + (int64_t)key * (SH::DN * 2) + c * 16;
      else if (c < SH::KCH)
        src = krb + (int64_t)key * (SH::DR * 2) + (c - SH::NCH) * 16;
      else
        src = kb + (int64_t)key * (SH::DN * 2);
    } else {
      const int sv = s - SH::KSLOTS;
      int t = sv / SH::VRS, c = sv - t * SH::VRS;
      if (t >= kPKeys || c >= SH::VCH) {
        t = 0;
        c = 0;
      }
      int key = key0 + t;
      key = key < seq_k ? key : seq_k - 1;
      src = vb + (int64_t)key * (SH::DV * 2) + c * 16;
    }
    __builtin_amdgcn_global_load_lds((const void *)src, (lds_void_p *)(stage + ins * 1024), 16, 0,
                                     0);
  }
}

template <class SH>
__device__ __forceinline__ bf16x8_t load_q_frag(const uint16_t *__restrict__ qn,
                                                const uint16_t *__restrict__ qr, int64_t qrow,
                                                int d0) {
  const uint16_t *src = d0 < SH::DN ? qn + qrow * SH::DN + d0 : qr + qrow * SH::DR + (d0 - SH::DN);
  return *reinterpret_cast<const bf16x8_t *>(src);
}

// grid.x = batch * heads * n_qtiles (heaviest query tiles first when causal)
template <int DN, int DR, int DV>
__global__ __launch_bounds__(kPWaves * 64) void k_prefill_mfma(
    const uint16_t *__restrict__ q_nope, const uint16_t *__restrict__ q_rope,
    const uint16_t *__restrict__ k, const uint16_t *__restrict__ k_rope,
    const uint16_t *__restrict__ v, qmla_prefill_dims d, float scale_log2, int causal,
    uint16_t *__restrict__ out, int n_qtiles) {
  using SH = PrefillShape<DN, DR, DV>;
  constexpr int VROW = SH::VRS * 16;
  extern __shared__ __attribute__((aligned(16))) char pring_raw[];
  lds_char_p *ring = (lds_char_p *)pring_raw;
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int n = lane & 31, half = lane >> 5;

  const int BH = d.batch * d.heads;
  const int L = blockIdx.x;
  const int qt = causal ? (n_qtiles - 1 - L / BH) : (L / BH);
  const int bh = L % BH;
  const int b = bh / d.heads, h = bh - b * d.heads;
  const int q0 = qt * kPRows;
  const int wrow0 = q0 + wave * kPRowsWave;

  const int64_t bhq = (int64_t)bh * d.seq_q;
  const int64_t bhk = (int64_t)bh * d.seq_k;
  const int64_t bkr = ((int64_t)b * d.k_rope_heads + (d.k_rope_heads == 1 ? 0 : h)) * d.seq_k;
  const uint8_t *kb = reinterpret_cast<const uint8_t *>(k + bhk * DN);
  const uint8_t *krb = reinterpret_cast<const uint8_t *>(k_rope + bkr * DR);
  const uint8_t *vb = reinterpret_cast<const uint8_t *>(v + bhk * DV);

  // Q fragments (B operand of S^T) for the wave's two 32-row column blocks.
  bf16x8_t qf[2][SH::KSTEPS];
  bool rok[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int row = wrow0 + nb * 32 + n;
    rok[nb] = row < d.seq_q;
    const int64_t qrow = bhq + (rok[nb] ? row : d.seq_q - 1);
    const uint32_t keep = rok[nb] ? 0xffffffffu : 0u;
#pragma unroll
    for (int kk = 0; kk < SH::KSTEPS; ++kk) {
      u32x4_t u = __builtin_bit_cast(u32x4_t, load_q_frag<SH>(q_nope, q_rope, qrow, kk * 16 + half * 8));
      u[0] &= keep;
      u[1] &= keep;
      u[2] &= keep;
      u[3] &= keep;
      qf[nb][kk] = __builtin_bit_cast(bf16x8_t, u);
    }
  }

  floatx16_t o[2][SH::CB];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
#pragma unroll
    for (int cb = 0; cb < SH::CB; ++cb)
#pragma unroll
      for (int j = 0; j < 16; ++j) o[nb][cb][j] = 0.f;
  float m_run[2] = {-INFINITY, -INFINITY}, l_run[2] = {0.f, 0.f};

  // key horizon (exclusive) of the block and of this wave
  int kend_blk = d.seq_k, kend_w = d.seq_k;
  if (causal) {
    kend_blk = min(d.seq_k, d.q_offset + min(q0 + kPRows, d.seq_q));
    kend_w = min(d.seq_k, d.q_offset + min(wrow0 + kPRowsWave, d.seq_q));
  }
  if (wrow0 >= d.seq_q) kend_w = 0;  // no query row in this wave
  const int ntiles = (kend_blk + kPKeys - 1) / kPKeys;
  const int my_instr = (SH::INSTR - wave + kPWaves - 1) / kPWaves;

  const int a_off = (n * SH::KRS + half) * 16;
  const int g = lane >> 4, sl = lane & 15;
  const int tok_a = (g >= 2 ? 4 : 0) + (sl >> 2);
  const int col_in = (g & 1) * 16 + 4 * (sl & 3);
  const int v_off = SH::V_BASE + tok_a * VROW + (col_in >> 3) * 16 + (col_in & 7) * 2;
  const int row_abs0 = d.q_offset + wrow0 + n;  // absolute row of column block 0

#pragma unroll
  for (int p = 0; p < kPStages - 1; ++p)
    if (p < ntiles)
      pissue_tile<SH>(kb, krb, vb, p * kPKeys, d.seq_k, ring + p * SH::STAGE_BYTES, wave, lane);

  for (int it = 0; it < ntiles; ++it) {
    const int nxt = it + kPStages - 1;
    if (nxt < ntiles)
      pissue_tile<SH>(kb, krb, vb, nxt * kPKeys, d.seq_k,
                      ring + (nxt % kPStages) * SH::STAGE_BYTES, wave, lane);
    const int ahead = (nxt < ntiles ? nxt : ntiles - 1) - it;
    pwait_vmcnt_dyn(ahead * my_instr);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    const int key0 = it * kPKeys;
    if (key0 < kend_w) {  // wave-uniform: tile not above this wave's horizon
      const lds_char_p *stage = ring + (it % kPStages) * SH::STAGE_BYTES;
      const lds_char_p *pa = stage + a_off;
      const lds_char_p *pv = stage + v_off;
      floatx16_t s[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
#pragma unroll
        for (int j = 0; j < 16; ++j) s[nb][j] = 0.f;
#pragma unroll
      for (int kk = 0; kk < SH::KSTEPS; ++kk) {
        const bf16x8_t a = *reinterpret_cast<const lds_bf16x8_p *>(pa + kk * 32);
        s[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[0][kk], s[0], 0, 0, 0);
        s[1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[1][kk], s[1], 0, 0, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
      for (int kk = 0; kk < SH::KSTEPS - 2; ++kk) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
      __builtin_amdgcn_sched_barrier(0);

      u32x4_t pk[2][2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int row_abs = row_abs0 + nb * 32;
        float mt = -INFINITY;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const int key = key0 + 8 * (j >> 2) + 4 * half + (j & 3);
          const bool vis = key < d.seq_k && (!causal || key <= row_abs);
          const float x = vis ? s[nb][j] * scale_log2 : -INFINITY;
          s[nb][j] = x;
          mt = fmaxf(mt, x);
        }
        mt = xor32_max(mt);
        // Lazy rescale (threshold 8 in log2 units, p <= 256).  Key 0 is
        // visible to every row, so the first tile makes m_run finite.
        if (m_run[nb] == -INFINITY || mt > m_run[nb] + 8.f) {
          const float m_new = fmaxf(mt, m_run[nb]);
          const float alpha = m_run[nb] == -INFINITY ? 0.f : exp2f(m_run[nb] - m_new);
          m_run[nb] = m_new;
          l_run[nb] *= alpha;
#pragma unroll
          for (int cb = 0; cb < SH::CB; ++cb) pagpr_scale16(o[nb][cb], alpha);
        }
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p0 = exp2f(s[nb][ks * 8 + 2 * i] - m_run[nb]);
            const float p1 = exp2f(s[nb][ks * 8 + 2 * i + 1] - m_run[nb]);
            l_run[nb] += p0 + p1;
            pk[nb][ks][i] = ppack2_bf16(p0, p1);
          }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bf16x8_t pb0 = __builtin_bit_cast(bf16x8_t, pk[0][ks]);
        const bf16x8_t pb1 = __builtin_bit_cast(bf16x8_t, pk[1][ks]);
#pragma unroll
        for (int cb = 0; cb < SH::CB; ++cb) {
          const lds_char_p *p1 = pv + ks * 16 * VROW + cb * 64;
          const bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_p *)p1);
          const bf16x4_t hi =
              __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4_p *)(p1 + 8 * VROW));
          const bf16x8_t a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
          o[0][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb0, o[0][cb], 0, 0, 0);
          o[1][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pb1, o[1][cb], 0, 0, 0);
        }
      }
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int i = 0; i < 2 * SH::CB - 2; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
    __builtin_amdgcn_s_waitcnt((0xF) | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
    __builtin_amdgcn_s_barrier();
  }

  // finalise
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const float l = xor32_sum(l_run[nb]);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    if (!rok[nb]) continue;
    uint16_t *dst = out + (bhq + wrow0 + nb * 32 + n) * DV;
#pragma unroll
    for (int cb = 0; cb < SH::CB; ++cb)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        u32x2_t w;
        w[0] = ppack2_bf16(o[nb][cb][jq * 4 + 0] * inv, o[nb][cb][jq * 4 + 1] * inv);
        w[1] = ppack2_bf16(o[nb][cb][jq * 4 + 2] * inv, o[nb][cb][jq * 4 + 3] * inv);
        *reinterpret_cast<u32x2_t *>(dst + cb * 32 + 8 * jq + 4 * half) = w;
      }
  }
}

template <int DN, int DR, int DV>
qmla_status launch_prefill_shape(const qmla_prefill_dims &d, const uint16_t *q_nope,
                                 const uint16_t *q_rope, const uint16_t *k,
                                 const uint16_t *k_rope, const uint16_t *v, float scale,
                                 int causal, uint16_t *out, hipStream_t stream) {
  using SH = PrefillShape<DN, DR, DV>;
  const int n_qtiles = (d.seq_q + kPRows - 1) / kPRows;
  const int64_t nblocks = (int64_t)d.batch * d.heads * n_qtiles;
  QMLA_REQUIRE(nblocks <= 0x7fffffff, QMLA_ERR_SHAPE, "too many query tiles");
  const size_t lds = (size_t)kPStages * SH::STAGE_BYTES;
  auto kern = k_prefill_mfma<DN, DR, DV>;
  QMLA_TRY(ensure_dynamic_lds((const void *)kern, lds));
  kern<<<dim3((unsigned)nblocks), dim3(kPWaves * 64), lds, stream>>>(
      q_nope, q_rope, k, k_rope, v, d, scale * 1.4426950408889634f, causal, out, n_qtiles);
  QMLA_LAUNCH_CHECK("k_prefill_mfma");
  return QMLA_OK;
}

}  // namespace

qmla_status launch_prefill_bf16(const qmla_prefill_dims &d, const uint16_t *q_nope,
                                const uint16_t *q_rope, const uint16_t *k,
                                const uint16_t *k_rope, const uint16_t *v, float scale,
                                int causal, uint16_t *out, hipStream_t stream) {
  const int dn = d.qk_nope, dr = d.qk_rope, dv = d.v_dim;
  if (dn == 128 && dr == 64 && dv == 128)
    return launch_prefill_shape<128, 64, 128>(d, q_nope, q_rope, k, k_rope, v, scale, causal, out,
                                              stream);
  if (dn == 32 && dr == 16 && dv == 32)
    return launch_prefill_shape<32, 16, 32>(d, q_nope, q_rope, k, k_rope, v, scale, causal, out,
                                            stream);
  if (dn == 16 && dr == 16 && dv == 32)
    return launch_prefill_shape<16, 16, 32>(d, q_nope, q_rope, k, k_rope, v, scale, causal, out,
                                            stream);
  if (dn == 32 && dr == 0 && dv == 32)
    return launch_prefill_shape<32, 0, 32>(d, q_nope, q_rope, k, k_rope, v, scale, causal, out,
                                           stream);
  if (dn == 64 && dr == 64 && dv == 64)
    return launch_prefill_shape<64, 64, 64>(d, q_nope, q_rope, k, k_rope, v, scale, causal, out,
                                            stream);
  return fail(QMLA_ERR_UNSUPPORTED,
              "bf16 prefill for (qk_nope, qk_rope, v_dim) = (%d, %d, %d); supported: "
              "(128,64,128) (64,64,64) (32,16,32) (16,16,32) (32,0,32)",
              dn, dr, dv);
}

}  // namespace qmla
