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

constexpr int kTok = 32;      // tokens per tile
constexpr int kPrefetch = 3;  // LDS operand reads issued ahead of their MFMA

// LDS stage layout for one 32-token tile:
//  * c_kv region: token rows of R bf16 (2R bytes).  Each DMA instruction
//    (64 lanes x 16 B) fills one 1 KB group of 1024 / 2R rows; groups are
//    padded by 16 B (1040 B stride for R = 512) so the S^T operand reads
//    (16 rows x 16 B per quarter-wave) fall in distinct bank groups.
//  * rope region: 32 rows x DR bf16, chunk positions XOR-swizzled by row.
template <int R, int DR>
struct DecodeShape {
  static constexpr int W = R + DR;                    // latent row width
  static constexpr int KSTEPS = W / 16;               // S k-steps (16 dims each)
  static constexpr int KV_STEPS = R / 16;             // ... of which over c_kv
  static constexpr int CB = R / 32;                   // PV column blocks
  static constexpr int ROW_B = R * 2;                 // c_kv bytes per token
  static constexpr int RPG = 1024 / ROW_B;            // c_kv rows per DMA group
  static constexpr int GS = 1024 + 16;                // padded group stride
  static constexpr int KV_INSTR = kTok / RPG;         // DMA instructions for c_kv
  static constexpr int KV_BYTES = KV_INSTR * GS;
  static constexpr int RCH = DR / 8;                  // rope chunks per token
  static constexpr int ROPE_INSTR = kTok * DR * 2 / 1024;
  static constexpr int INSTR = KV_INSTR + ROPE_INSTR;
  static constexpr int STAGE_BYTES = KV_BYTES + ROPE_INSTR * 1024;
  static_assert(R == 64 || R == 128 || R == 256 || R == 512, "kv_lora_rank");
  static_assert(DR == 16 || DR == 32 || DR == 64, "rope dim");
  // Token t of a tile lives in c_kv row slot pi(t) (for one row per group):
  // pi(t) = (t & 16) | (t & 3) << 2 | (t >> 2) & 3.  With the 1040-byte row
  // stride this makes both LDS read patterns conflict-free on the 64-bank
  // LDS: the S^T operand reads (16 consecutive tokens, same 16-byte chunk)
  // hit 16 distinct row offsets mod 256 B, and the transposed V^T reads
  // (4 consecutive tokens x 64 contiguous bytes per 32 lanes) hit rows whose
  // offsets are 64 B apart mod 256 B.  pi(t + 8) = pi(t) + 2 for t % 16 < 8.
  static __device__ __forceinline__ int slot(int t) {
    return RPG == 1 ? ((t & 16) | ((t & 3) << 2) | ((t >> 2) & 3)) : t;
  }
  // byte offset of token row t in the c_kv region
  static __device__ __forceinline__ int kv_row(int t) {
    const int r = slot(t);
    return (r / RPG) * GS + (r % RPG) * ROW_B;
  }
  // row-offset (bytes) between tokens t + 8 and t (t % 16 < 8), and t + 16 and t
  static constexpr int HI8 = RPG == 1 ? 2 * GS : (8 / RPG) * GS;
  static constexpr int HI16 = RPG == 1 ? 16 * GS : (16 / RPG) * GS;
};

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
// vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt_hi[15:14]).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ void wait_vmcnt_dyn(int n) {
  // n is wave-uniform (scalar); dispatch to an immediate.
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

// Waits until at most k tiles of this wave's DMA are outstanding.  With an
// even split (every wave issues INSTR / NW instructions per tile) the count
// is a compile-time multiple; otherwise dispatch on the runtime count.
template <class SH, int NW>
__device__ __forceinline__ void wait_tiles(int k, int my_instr) {
  if constexpr (SH::INSTR % NW == 0) {
    constexpr int MI = SH::INSTR / NW;
    if (k <= 0)
      wait_vmcnt<0>();
    else if (k == 1)
      wait_vmcnt<MI>();
    else
      wait_vmcnt<(2 * MI < 63 ? 2 * MI : 63)>();
  } else {
    wait_vmcnt_dyn(k * my_instr);
  }
}

typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) bf16x4_t lds_bf16x4;
typedef __attribute__((address_space(3))) bf16x8_t lds_bf16x8;

// S^T accumulation chain in arch VGPRs.  Any AGPR operand in a function makes
// the compiler pick the AGPR form for every MFMA builtin, which would put
// this 16-register accumulator next to the 256 O^T accumulators in the AGPR
// file and spill Q; issuing the S^T MFMAs through inline asm with "v"
// constraints keeps it in VGPRs.  Hazards: the first MFMA of a chain takes
// srcC = 0 (no VALU -> MFMA srcC dependence); each following one reads the
// previous result as srcC with exactly the same registers (forwarded, no
// wait states); VALU reads of the result are preceded by s_nop padding
// (mfma_s_drain) longer than the MFMA's 8 passes.
__device__ __forceinline__ floatx16_t mfma_s_first(const bf16x8_t &a, const bf16x8_t &b) {
  floatx16_t d;
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
  return d;
}
__device__ __forceinline__ void mfma_s_acc(floatx16_t &d, const bf16x8_t &a, const bf16x8_t &b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_s_drain(floatx16_t &d) {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" : "+v"(d));
}

__device__ __forceinline__ uint32_t pack2_bf16(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v;
  v[0] = (__bf16)a;  // v_cvt_pk_bf16_f32: round to nearest even
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// Issue this wave's share of the DMA instructions for one tile.  Tokens past
// the segment end re-load the segment's last row (masked later, never used).
template <class SH, int NW>
__device__ __forceinline__ void issue_tile(const uint8_t *__restrict__ seq_base, int tile_t0,
                                           int seg_t1, lds_char *stage, int wave, int lane) {
  // With NW dividing both instruction counts, whether instruction ins0+wave
  // exists and which region it fills is known per unrolled step.
  constexpr bool EVEN = SH::INSTR % NW == 0 && SH::KV_INSTR % NW == 0;
#pragma unroll
  for (int ins0 = 0; ins0 < SH::INSTR; ins0 += NW) {
    const int ins = ins0 + wave;
    if (EVEN || ins < SH::INSTR) {
      int t, c, base_b;
      lds_char *dst;
      if (EVEN ? ins0 < SH::KV_INSTR : ins < SH::KV_INSTR) {
        t = ins * SH::RPG + lane / (SH::ROW_B / 16);
        c = lane % (SH::ROW_B / 16);
        base_b = 0;
        dst = stage + (SH::RPG == 1 ? SH::kv_row(ins) : ins * SH::GS);
      } else {
        const int q = ins - SH::KV_INSTR;
        t = q * (64 / SH::RCH) + lane / SH::RCH;
        c = (lane % SH::RCH) ^ (t & (SH::RCH - 1));
        base_b = SH::ROW_B;
        dst = stage + SH::KV_BYTES + q * 1024;
      }
      int tok = tile_t0 + t;
      tok = tok < seg_t1 ? tok : seg_t1 - 1;
      const uint8_t *src = seq_base + (int64_t)tok * (SH::W * 2) + base_b + c * 16;
      __builtin_amdgcn_global_load_lds((const void *)src, (lds_void *)dst, 16, 0, 0);
    }
  }
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

// Per-lane LDS read addressing (see DecodeShape).
template <class SH>
struct LaneAddr {
  int a_base;     // S^T operand, c_kv part: + kk*32
  int rope_row;   // S^T operand, rope part: row base inside the rope region
  int rope_mask;  // row & (RCH - 1): XOR swizzle of rope chunks
  int half;
  int v_base;     // V^T operand: + ks-block and cb offsets

  __device__ __forceinline__ bf16x8_t s_read(const lds_char *st, int kk) const {
    if (kk < SH::KV_STEPS)
      return *reinterpret_cast<const lds_bf16x8 *>(st + a_base + kk * 32);
    const int c = (2 * (kk - SH::KV_STEPS) + half) ^ rope_mask;
    return *reinterpret_cast<const lds_bf16x8 *>(st + SH::KV_BYTES + rope_row + c * 16);
  }
  // PV operand i = ks * CB + cb: tokens 16 ks + {tok_a, tok_a + 8}, 32 columns
  __device__ __forceinline__ bf16x8_t pv_read(const lds_char *st, int i) const {
    const int ks = i / SH::CB, cb = i % SH::CB;
    const lds_char *p = st + v_base + ks * SH::HI16 + cb * 64;
    const bf16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)p);
    const bf16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4 *)(p + SH::HI8));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  }
};

// One pipelined body: S^T of the next tile (DO_S) interleaved with O^T +=
// V^T P^T of the current tile (DO_PV).  Operand reads run two MFMAs ahead.
template <class SH, bool DO_S, bool DO_PV>
__device__ __forceinline__ void body(const LaneAddr<SH> &la, const lds_char *st_s,
                                     const lds_char *st_pv, const bf16x8_t (&qf)[SH::KSTEPS],
                                     floatx16_t &s, const bf16x8_t (&pb)[2],
                                     floatx16_t (&o)[SH::CB]) {
  constexpr int NS = DO_S ? SH::KSTEPS : 0;
  constexpr int NP = DO_PV ? 2 * SH::CB : 0;
  constexpr int N = NS > NP ? NS : NP;
  constexpr int D = kPrefetch;
  bf16x8_t sa[D + 1], pa[D + 1];
#pragma unroll
  for (int i = 0; i < D; ++i) {
    if (i < NS) sa[i] = la.s_read(st_s, i);
    if (i < NP) pa[i] = la.pv_read(st_pv, i);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) {
    if (i < NS) {
      if (i + D < NS) sa[(i + D) % (D + 1)] = la.s_read(st_s, i + D);
      if (i == 0)
        s = mfma_s_first(sa[0], qf[0]);
      else
        mfma_s_acc(s, sa[i % (D + 1)], qf[i]);
    }
    if (i < NP) {
      if (i + D < NP) pa[(i + D) % (D + 1)] = la.pv_read(st_pv, i + D);
      o[i % SH::CB] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa[i % (D + 1)], pb[i / SH::CB],
                                                              o[i % SH::CB], 0, 0, 0);
    }
  }
  if constexpr (DO_S) mfma_s_drain(s);
}

// Online softmax of one tile's S^T (lane = head, 16 tokens) in the log2
// domain.  The running reference m is set by the first tile (or given by a
// restart) and then kept: probabilities are exp2(s - m) <= 2^16 as long as no
// row's maximum exceeds m by more than kRefSlack.  When one does (rare), the
// function returns true and the block restarts the segment with the larger
// reference (see the kernel).  The O^T accumulators are therefore only ever
// MFMA-accumulated, read at the end or zeroed at a segment start -- never
// rescaled in registers, which keeps all 256 of them in AGPRs.
constexpr float kRefSlack = 16.f;

template <class SH>
__device__ __forceinline__ bool softmax_tile(floatx16_t &s, float scale_log2, int tile_t0, int T,
                                             int half, float &m_run, float &l_run,
                                             bf16x8_t (&pb)[2], float &mt_out) {
  float mt = -INFINITY;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int tok = tile_t0 + 8 * (j >> 2) + 4 * half + (j & 3);
    const float x = tok < T ? s[j] * scale_log2 : -INFINITY;
    s[j] = x;
    mt = fmaxf(mt, x);
  }
  mt = xor32_max(mt);
  mt_out = mt;
  if (m_run == -INFINITY) {
    m_run = mt;  // first tile of the segment (or after a flush): o and l are zero
  } else if (__ballot(mt > m_run + kRefSlack) != 0) {
    return true;
  }
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    u32x4_t pk;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p0 = exp2f(s[ks * 8 + 2 * i] - m_run);
      const float p1 = exp2f(s[ks * 8 + 2 * i + 1] - m_run);
      l_run += p0 + p1;
      pk[i] = pack2_bf16(p0, p1);
    }
    pb[ks] = __builtin_bit_cast(bf16x8_t, pk);
  }
  return false;
}

// True when any wave of the block raised its reference-overflow flag.
template <int NW>
__device__ __forceinline__ bool any_flag(const volatile int *flags) {
  int v = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) v |= flags[w];
  return v != 0;
}

template <int R, int DR, int NW, int NSTAGE, typename QT>
__global__ __launch_bounds__(NW * 64) void k_decode_mfma(
    const uint8_t *__restrict__ pool, const int64_t *__restrict__ offsets,
    const QT *__restrict__ q_lat, const QT *__restrict__ q_rope, int32_t rows,
    float scale_log2, DecodePlanView plan, float *__restrict__ out, float *__restrict__ out_lse,
    float *__restrict__ part_o, float *__restrict__ part_lse) {
  using SH = DecodeShape<R, DR>;
  static_assert(NSTAGE >= 3, "the pipelined loop keeps two stages resident");
  extern __shared__ __attribute__((aligned(16))) char ring_raw[];
  __shared__ int ovf_flag[NW];
  lds_char *ring = (lds_char *)ring_raw;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n = lane & 31;     // head (query row) within the wave = MFMA column
  const int half = lane >> 5;  // which 8-wide k half of an MFMA operand
  const int row = blockIdx.y * (NW * 32) + wave * 32 + n;  // query row
  const bool row_ok = row < rows;
  const int row_c = row_ok ? row : rows - 1;
  const int piece = blockIdx.x;
  const int my_instr = (SH::INSTR - wave + NW - 1) / NW;

  LaneAddr<SH> la;
  la.a_base = SH::kv_row(n) + half * 16;
  la.rope_row = n * (DR * 2);
  la.rope_mask = n & (SH::RCH - 1);
  la.half = half;
  {
    const int g = lane >> 4, sl = lane & 15;
    const int tok_a = (g >= 2 ? 4 : 0) + (sl >> 2);
    const int col_in = (g & 1) * 16 + 4 * (sl & 3);
    la.v_base = SH::kv_row(tok_a) + (col_in >> 3) * 16 + (col_in & 7) * 2;
  }

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
      u32x4_t u = __builtin_bit_cast(u32x4_t, load_q8<R, DR, QT>(q_lat, q_rope, qrow_c,
                                                                  kk * 16 + half * 8));
      const uint32_t keep = row_ok ? 0xffffffffu : 0u;
      u[0] &= keep;
      u[1] &= keep;
      u[2] &= keep;
      u[3] &= keep;
      qf[kk] = __builtin_bit_cast(bf16x8_t, u);
    }

    const int T = sg.t1 - sg.t0;
    const int ntiles = (T + kTok - 1) / kTok;
    auto stage = [&](int t) { return ring + (t % NSTAGE) * SH::STAGE_BYTES; };

    floatx16_t o[SH::CB];
    floatx16_t s;
    bf16x8_t pb[2];
    float m_run, l_run;
    float m_init = -INFINITY;  // reference to (re)start the segment with
    for (;;) {
#pragma unroll
      for (int cb = 0; cb < SH::CB; ++cb)
#pragma unroll
        for (int j = 0; j < 16; ++j) o[cb][j] = 0.f;
      m_run = m_init;
      l_run = 0.f;
      if (lane == 0) ovf_flag[wave] = 0;

      // prologue: NSTAGE-1 tiles in flight, then S and softmax of tile 0
#pragma unroll
      for (int p = 0; p < NSTAGE - 1; ++p)
        if (p < ntiles) issue_tile<SH, NW>(seq_base, sg.t0 + p * kTok, sg.t1, stage(p), wave, lane);
      wait_tiles<SH, NW>(min(NSTAGE - 2, ntiles - 1), my_instr);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      body<SH, true, false>(la, stage(0), stage(0), qf, s, pb, o);
      float mt;
      // tile 0 never overflows: m_init is -inf or covers every tile's max
      (void)softmax_tile<SH>(s, scale_log2, 0, T, half, m_run, l_run, pb, mt);
      float m_cand = fmaxf(m_run, mt);  // max over all tiles of the segment

      // steady state: S^T of tile it+1 interleaved with P.V of tile it.  A
      // reference overflow only raises a flag (the tile's P is left stale and
      // the segment is redone below): the loop keeps a single exit.
      for (int it = 0; it + 1 < ntiles; ++it) {
        // tile it+1 must be complete; tile it+2 (if issued) may stay in flight
        wait_tiles<SH, NW>(min(NSTAGE - 3, ntiles - 2 - it), my_instr);
        // All waves are past iteration it-1: stage (it-1) % NSTAGE is free and
        // tile it+1 is visible to every wave.
        __builtin_amdgcn_s_waitcnt((0xF) | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        const int nxt = it + NSTAGE - 1;
        if (nxt < ntiles)
          issue_tile<SH, NW>(seq_base, sg.t0 + nxt * kTok, sg.t1, stage(nxt), wave, lane);
        __builtin_amdgcn_sched_barrier(0);
        body<SH, true, true>(la, stage(it + 1), stage(it), qf, s, pb, o);
        __builtin_amdgcn_sched_barrier(0);
        if (softmax_tile<SH>(s, scale_log2, (it + 1) * kTok, T, half, m_run, l_run, pb, mt) &&
            lane == 0)
          ovf_flag[wave] = 1;
        m_cand = fmaxf(m_cand, mt);
        __builtin_amdgcn_sched_barrier(0);
      }
      // P.V of the last tile
      body<SH, false, true>(la, stage(ntiles - 1), stage(ntiles - 1), qf, s, pb, o);
      // Every wave is done with the stages (the next segment's or attempt's
      // prologue refills them) and every overflow flag is visible.
      __builtin_amdgcn_s_waitcnt((0xF) | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
      __builtin_amdgcn_s_barrier();
      if (!any_flag<NW>(ovf_flag)) break;
      // Rare: some row's maximum outgrew the reference.  Redo the segment
      // with a reference covering every tile's maximum (cannot overflow).
      __builtin_amdgcn_s_barrier();  // all waves have read the flags
      m_init = m_cand;
    }

    // ---- finalise: combine the two half-waves' denominators and write
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
  const size_t lds = (size_t)NSTAGE * SH::STAGE_BYTES;
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
  if (a.rows <= 32) return launch_shape<R, DR, 1, 3>(a, stream);
  if (a.rows <= 64) return launch_shape<R, DR, 2, 4>(a, stream);
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
