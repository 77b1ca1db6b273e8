// prefill_mfma.hip -- bf16 MFMA flash prefill (causal, chunk offset).
//
// Replaces the tiled candle matmuls of fused_prefill_attn
// (src/attention_kernel.rs:64-107) for bf16 inputs with f32 accumulation.
// A block holds 4 waves x 64 query rows of one (b, h) and streams 32-key
// tiles of [k_nope | k_rope] and v through an LDS ring.  Per wave and tile:
//
//   S^T[key][q] = sum_d K[key][d] Q[q][d]      2 x KSTEPS MFMAs (Q in VGPRs)
//   P^T = exp2(S^T * scale*log2(e) - m)         softmax, f32
//   O^T[c][q] += sum_key V^T[c][key] P^T[key][q]
//
// The S^T accumulator (lane = query row, 16 keys per lane) is the B operand
// of the P.V product, and V^T comes from the key-major tile through
// ds_read_b64_tr_b16.  The loop is software-pipelined: iteration it
// computes S^T of tile it+1, then P.V of tile it with the softmax of tile
// it+1 spread over its MFMAs.  The softmax keeps a lazy fixed reference per
// row (the first tile's maximum; a block whose later scores exceed it by
// more than kPSlack redoes its tiles with the true maximum), so the O^T
// accumulators are never rescaled inside the loop.  Key tiles above a wave's
// causal horizon are skipped (exact: the reference's -1e18 mask gives
// exp() == 0); blocks are issued heaviest first so the causal triangle
// balances across compute units.

#include <cmath>
#include <type_traits>
#include <utility>

#include "mfma_pipe.hpp"

namespace qmla {

namespace {

using namespace pipe;

constexpr int kPKeys = 32;      // keys per tile
constexpr int kPWaves = 4;
constexpr int kPRowsWave = 64;  // two 32-row MFMA column blocks
constexpr int kPRows = kPWaves * kPRowsWave;
constexpr int kPStages = 4;
constexpr int kPAhead = 4;      // S^T operand reads issued ahead of their MFMAs
constexpr int kPvAheadP = 3;    // V^T fragments issued ahead of their MFMAs
constexpr float kPSlack = 16.f;

// One LDS region of a stage: 32 key rows of ROWB bytes, filled by 1 KB DMA
// instructions (RPI rows each).  Chunk positions are XOR-swizzled by row so
// that the operand reads are free of bank conflicts without padding:
//  * K regions (S^T operand: 16 rows read the same 16-byte chunk): chunk c
//    of row r sits at c ^ ((r / RB) & (CPR - 1)), RB = rows per 256-byte bank
//    cycle -- rows sharing a bank window get distinct chunk positions.
//  * V region (V^T operand: 4 consecutive rows x one 64-byte group per half
//    wave): group g of row r sits at g ^ ((r / RB) & (GPR - 1)).
// The DMA realises the swizzle on the source side: the lane writing LDS
// position p of row r loads the chunk whose swizzled position is p.
template <int ROWB>
struct Region {
  static_assert(ROWB == 0 || (ROWB >= 32 && ROWB <= 1024 && (ROWB & (ROWB - 1)) == 0), "row bytes");
  static constexpr int CPR = ROWB / 16;
  static constexpr int RPI = ROWB ? 1024 / ROWB : 1;
  static constexpr int INSTR = 32 * ROWB / 1024;
  static constexpr int BYTES = 32 * ROWB;
  static constexpr int RB = ROWB >= 256 ? 1 : (ROWB ? 256 / ROWB : 1);
  static constexpr int GPR = ROWB / 64;
  static __device__ __forceinline__ int kpos(int r, int c) { return c ^ ((r / RB) & (CPR - 1)); }
  static __device__ __forceinline__ int vgrp(int r, int g) {
    return GPR > 1 ? (g ^ ((r / RB) & (GPR - 1))) : g;
  }
};

template <int DN_, int DR_, int DV_>
struct PrefillShape {
  static constexpr int DN = DN_, DR = DR_, DV = DV_;
  static constexpr int DQK = DN + DR;
  static constexpr int KSTEPS = DQK / 16;   // S^T k-steps
  static constexpr int NSTEPS = DN / 16;    // ... of which over k_nope
  static constexpr int CB = DV / 32;        // P.V column blocks
  using KN = Region<DN * 2>;
  using KR = Region<DR * 2>;
  using VR = Region<DV * 2>;
  static constexpr int KN_OFF = 0;
  static constexpr int KR_OFF = KN::BYTES;
  static constexpr int V_OFF = KN::BYTES + KR::BYTES;
  static constexpr int STAGE_BYTES = KN::BYTES + KR::BYTES + VR::BYTES;
  static constexpr int INSTR = KN::INSTR + KR::INSTR + VR::INSTR;
  static constexpr int MI = (INSTR + kPWaves - 1) / kPWaves;  // DMA slots per wave
  static constexpr bool EVEN = KN::INSTR % kPWaves == 0 && KR::INSTR % kPWaves == 0 &&
                               VR::INSTR % kPWaves == 0;
  static_assert(DN % 16 == 0 && DR % 16 == 0 && DV % 32 == 0 && DN >= 16 && DV >= 32, "dims");
  static_assert(MI * (kPStages - 1) < 64, "vmcnt range");
};

// Uniform parts of one tile's DMA: base pointers of the three source rows
// (key0 of the tile), the LDS stage, and the last valid key (tile-relative).
struct PTileDma {
  const uint8_t *kn, *kr, *v;
  uint32_t stage;
  int last;
};

// Per-lane part of region instruction i: source offset of the chunk that
// lands at this lane's LDS position (swizzle inverted), clamped rows.
template <class RG, bool VSWZ>
__device__ __forceinline__ uint32_t region_src(int i, int lane, int last) {
  const int r = i * RG::RPI + lane / RG::CPR;
  const int p = lane % RG::CPR;
  const int j = VSWZ ? ((RG::vgrp(r, p >> 2) << 2) | (p & 3)) : RG::kpos(r, p);
  return (uint32_t)(min(r, last) * (RG::CPR * 16) + j * 16);
}

// DMA slot k of this wave: instruction k * kPWaves + wave of the tile.
template <class SH>
__device__ __forceinline__ void pissue_one(const PTileDma &d, int k, int wave, int lane) {
  const int ins0 = k * kPWaves, ins = ins0 + wave;
  if (!SH::EVEN && ins >= SH::INSTR) return;
  constexpr int E1 = SH::KN::INSTR, E2 = SH::KN::INSTR + SH::KR::INSTR;
  const uint32_t st = fresh(d.stage);
  if (SH::EVEN ? ins0 < E1 : ins < E1) {
    dma16(fresh(d.kn), region_src<typename SH::KN, false>(ins, lane, d.last),
          st + SH::KN_OFF + ins * 1024);
  } else if (SH::EVEN ? ins0 < E2 : ins < E2) {
    if constexpr (SH::KR::INSTR > 0)
      dma16(fresh(d.kr), region_src<typename SH::KR, false>(ins - E1, lane, d.last),
            st + SH::KR_OFF + (ins - E1) * 1024);
  } else {
    dma16(fresh(d.v), region_src<typename SH::VR, true>(ins - E2, lane, d.last),
          st + SH::V_OFF + (ins - E2) * 1024);
  }
}

template <class SH>
__device__ __forceinline__ void pissue_tile(const PTileDma &d, int wave, int lane) {
#pragma unroll
  for (int k = 0; k < SH::MI; ++k) pissue_one<SH>(d, k, wave, lane);
}

// Waits until at most k tiles of this wave's DMA are outstanding.
template <class SH>
__device__ __forceinline__ void pwait_tiles(int k, int my_instr) {
  if constexpr (SH::EVEN) {
    if (k <= 0)
      wait_vmcnt<0>();
    else if (k == 1)
      wait_vmcnt<SH::MI>();
    else
      wait_vmcnt<(2 * SH::MI < 63 ? 2 * SH::MI : 63)>();
  } else {
    wait_vmcnt_dyn(k * my_instr);
  }
}

// Per-lane LDS byte offsets (relative to a stage) of the MFMA operands.
template <class SH>
struct PLane {
  uint32_t s[SH::KSTEPS];  // S^T operand of k-step kk (row n, 8 dims at 8*half)
  uint32_t v[SH::CB];      // V^T operand of column block cb (k-step / hi via immediates)
};

template <class SH>
__device__ __forceinline__ PLane<SH> plane_offsets(int lane) {
  PLane<SH> la;
  const int n = lane & 31, half = lane >> 5;
#pragma unroll
  for (int kk = 0; kk < SH::KSTEPS; ++kk) {
    if (kk < SH::NSTEPS)
      la.s[kk] = SH::KN_OFF + n * (SH::DN * 2) + SH::KN::kpos(n, 2 * kk + half) * 16;
    else
      la.s[kk] = SH::KR_OFF + n * (SH::DR * 2) + SH::KR::kpos(n, 2 * (kk - SH::NSTEPS) + half) * 16;
  }
  const int g = lane >> 4, sl = lane & 15;
  const int tok_a = (g >= 2 ? 4 : 0) + (sl >> 2);
  const int col_in = (g & 1) * 16 + 4 * (sl & 3);  // element within a 32-column block
#pragma unroll
  for (int cb = 0; cb < SH::CB; ++cb)
    la.v[cb] = SH::V_OFF + tok_a * (SH::DV * 2) + SH::VR::vgrp(tok_a, cb) * 64 + col_in * 2;
  return la;
}

// S^T of one tile for both column blocks: 2 x KSTEPS MFMAs into VGPR
// accumulators, operand reads kPAhead steps ahead; with DMA, this wave's
// slots for the tile in `d` are spread over the MFMAs.
template <class SH, bool DMA>
__device__ __forceinline__ void ps_phase(const PLane<SH> &la, uint32_t st,
                                         const bf16x8_t (&qf)[2][SH::KSTEPS], floatx16_t (&s)[2],
                                         const PTileDma &d, int wave, int lane) {
  constexpr int D = kPAhead < SH::KSTEPS ? kPAhead : SH::KSTEPS;
  bf16x8_t a[D + 1];
  [&]<int... K>(std::integer_sequence<int, K...>) {
    ([&] { if constexpr (K < D) a[K] = ds_b128<0>(st + la.s[K]); }(), ...);
    ([&] {
      constexpr int kk = K;
      constexpr int after = (kk + D - 1 < SH::KSTEPS - 1 ? D - 1 : SH::KSTEPS - 1 - kk);
      wait_lgkm<after>();
      arrived(a[kk % (D + 1)]);
      if constexpr (kk == 0) {
        s[0] = mfma_s_first(a[0], qf[0][0]);
        s[1] = mfma_s_first(a[0], qf[1][0]);
      } else {
        mfma_s_acc(s[0], a[kk % (D + 1)], qf[0][kk]);
        mfma_s_acc(s[1], a[kk % (D + 1)], qf[1][kk]);
      }
      if constexpr (DMA) {
#pragma unroll
        for (int k = 0; k < SH::MI; ++k)
          if ((k * SH::KSTEPS) / SH::MI == kk) pissue_one<SH>(d, k, wave, lane);
      }
      if constexpr (kk + D < SH::KSTEPS) a[(kk + D) % (D + 1)] = ds_b128<0>(st + la.s[kk + D]);
    }(), ...);
  }(std::make_integer_sequence<int, SH::KSTEPS>{});
  mfma_s_drain(s[0]);
  mfma_s_drain(s[1]);
}

// V^T fragment j = (k-step ks, column block i): two transposing reads.
template <class SH, int J>
__device__ __forceinline__ bf16x8_t pv_frag(const PLane<SH> &la, uint32_t st) {
  constexpr int ks = J / SH::CB, cb = J % SH::CB;
  return ds_tr2<ks * 16 * (SH::DV * 2), 8 * (SH::DV * 2)>(st + la.v[cb]);
}

// O^T += V^T P^T for both column blocks: 2 x 2 x CB MFMAs into the AGPR
// accumulators, V^T fragments streamed kPvAheadP ahead.
template <class SH>
__device__ __forceinline__ void ppv_phase(const PLane<SH> &la, uint32_t st,
                                          const bf16x8_t (&pb)[2][2], floatx16_t (&o)[2][SH::CB]) {
  constexpr int NA = 2 * SH::CB;
  constexpr int DA = kPvAheadP < NA ? kPvAheadP : NA;
  bf16x8_t a[DA + 1];
  [&]<int... J>(std::integer_sequence<int, J...>) {
    ([&] { if constexpr (J < DA) a[J] = pv_frag<SH, J>(la, st); }(), ...);
    ([&] {
      constexpr int j = J;
      constexpr int after = 2 * (j + DA - 1 < NA - 1 ? DA - 1 : NA - 1 - j);
      wait_lgkm<after>();
      arrived(a[j % (DA + 1)]);
      constexpr int ks = j / SH::CB, cb = j % SH::CB;
      o[0][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[j % (DA + 1)], pb[0][ks], o[0][cb], 0, 0, 0);
      o[1][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[j % (DA + 1)], pb[1][ks], o[1][cb], 0, 0, 0);
      if constexpr (j + DA < NA) a[(j + DA) % (DA + 1)] = pv_frag<SH, j + DA>(la, st);
    }(), ...);
  }(std::make_integer_sequence<int, NA>{});
}

// Key (within the tile) of S^T accumulator element j of this lane.
__device__ __forceinline__ int ptile_key(int j, int half) {
  return 8 * (j >> 2) + 4 * half + (j & 3);
}

// Raw maximum of this lane's 16 scores of column block nb; with MASK, keys
// at or past seq_k or (causal) after the row's absolute position are out.
template <bool MASK>
__device__ __forceinline__ float ptile_max(const floatx16_t &s, int key0, int half, int vis_lim) {
  float x[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) x[j] = (!MASK || key0 + ptile_key(j, half) < vis_lim) ? s[j] : -INFINITY;
  const float a = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
  const float b = fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7]));
  const float c = fmaxf(fmaxf(x[8], x[9]), fmaxf(x[10], x[11]));
  const float e = fmaxf(fmaxf(x[12], x[13]), fmaxf(x[14], x[15]));
  return fmaxf(fmaxf(a, b), fmaxf(c, e));
}

// p = exp2(s * sl2 - m) as the two bf16 B-operand fragments; adds to l.
template <bool MASK>
__device__ __forceinline__ void ptile_p(const floatx16_t &s, float sl2, float m, int key0,
                                        int half, int vis_lim, float &l, bf16x8_t (&pb)[2]) {
  float p[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    p[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j], sl2, -m));
    if (MASK) p[j] = key0 + ptile_key(j, half) < vis_lim ? p[j] : 0.f;
  }
  float q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = p[2 * i] + p[2 * i + 1];
  l += ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    u32x4_t pk;
#pragma unroll
    for (int i = 0; i < 4; ++i) pk[i] = pack2_bf16(p[ks * 8 + 2 * i], p[ks * 8 + 2 * i + 1]);
    pb[ks] = __builtin_bit_cast(bf16x8_t, pk);
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
  extern __shared__ __attribute__((aligned(16))) char pring_raw[];
  lds_char *ring = (lds_char *)pring_raw;
  const uint32_t ring_u = lds_u32(ring);
  const uint32_t ovf_flags = ring_u + kPStages * SH::STAGE_BYTES;  // kPWaves words
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n = lane & 31, half = lane >> 5;
  // A negative scale is applied as |scale| with the sign folded into q
  // (exact in bf16), so the raw score maximum is also the scaled one.
  const uint32_t q_sign = scale_log2 < 0.f ? 0x80008000u : 0u;
  const float sl2 = fabsf(scale_log2);

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
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int row = wrow0 + nb * 32 + n;
    const bool ok = row < d.seq_q;
    const int64_t qrow = bhq + (ok ? row : d.seq_q - 1);
    const uint32_t keep = ok ? 0xffffffffu : 0u;
#pragma unroll
    for (int kk = 0; kk < SH::KSTEPS; ++kk) {
      u32x4_t u = __builtin_bit_cast(u32x4_t, load_q_frag<SH>(q_nope, q_rope, qrow, kk * 16 + half * 8));
#pragma unroll
      for (int i = 0; i < 4; ++i) u[i] = (u[i] ^ q_sign) & keep;
      qf[nb][kk] = __builtin_bit_cast(bf16x8_t, u);
    }
  }

  // key horizon (exclusive) of the block and of this wave
  int kend_blk = d.seq_k, kend_w = d.seq_k;
  if (causal) {
    kend_blk = min(d.seq_k, d.q_offset + min(q0 + kPRows, d.seq_q));
    kend_w = min(d.seq_k, d.q_offset + min(wrow0 + kPRowsWave, d.seq_q));
  }
  if (wrow0 >= d.seq_q) kend_w = 0;  // no query row in this wave
  const int ntb = (kend_blk + kPKeys - 1) / kPKeys;  // tiles of the block
  const int ntw = (kend_w + kPKeys - 1) / kPKeys;    // tiles of this wave
  const int my_instr = (SH::INSTR - wave + kPWaves - 1) / kPWaves;
  const PLane<SH> la = plane_offsets<SH>(lane);
  // a tile needs the mask if one of its keys is invisible to some row of
  // the wave: past seq_k, or (causal) after the wave's first row
  const int mask_from = causal ? min(d.seq_k, d.q_offset + wrow0 + 1) : d.seq_k;
  int vis_lim[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
    vis_lim[nb] = causal ? min(d.seq_k, d.q_offset + wrow0 + nb * 32 + n + 1) : d.seq_k;
  auto tile_dma = [&](int t) {
    const int key0 = t * kPKeys;
    return PTileDma{kb + (int64_t)key0 * (DN * 2), krb + (int64_t)key0 * (DR * 2),
                    vb + (int64_t)key0 * (DV * 2), ring_u + (t % kPStages) * SH::STAGE_BYTES,
                    d.seq_k - 1 - key0};
  };
  auto stage_u = [&](int t) { return ring_u + (uint32_t)((t % kPStages) * SH::STAGE_BYTES); };

  floatx16_t o[2][SH::CB];
  floatx16_t s[2];
  bf16x8_t pb[2][2], pn[2][2];
  float m_ref[2], l_run[2], m_raw[2];
  float m_init[2] = {-INFINITY, -INFINITY};
  for (;;) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
      for (int cb = 0; cb < SH::CB; ++cb)
#pragma unroll
        for (int j = 0; j < 16; ++j) o[nb][cb][j] = 0.f;
      l_run[nb] = 0.f;
      m_raw[nb] = -INFINITY;
      m_ref[nb] = m_init[nb];
    }
    if (lane == 0) ds_w32(ovf_flags + 4 * wave, 0u);

    // prologue: kPStages-1 tiles in flight, then S and softmax of tile 0
#pragma unroll
    for (int p = 0; p < kPStages - 1; ++p)
      if (p < ntb) pissue_tile<SH>(tile_dma(p), wave, lane);
    pwait_tiles<SH>(min(kPStages - 2, ntb - 1), my_instr);
    wait_lgkm<0>();
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if (ntw > 0) {
      ps_phase<SH, false>(la, stage_u(0), qf, s, PTileDma{}, wave, lane);
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        m_raw[nb] = ptile_max<true>(s[nb], 0, half, vis_lim[nb]);
        // key 0 is visible to every row: the first tile's maximum is finite
        if (m_ref[nb] == -INFINITY) m_ref[nb] = xor32_max(m_raw[nb]) * sl2;
        ptile_p<true>(s[nb], sl2, m_ref[nb], 0, half, vis_lim[nb], l_run[nb], pb[nb]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);

    // Iteration it: S^T of tile it+1, then P.V of tile it with the softmax
    // of tile it+1 spread over its MFMAs.  MODE 0: unmasked tile it+1 with
    // its DMA slots spread over S^T; MODE 1: masked tile it+1, DMA up
    // front; MODE 2: this wave is past its horizon for tile it+1 (P.V of
    // tile it only, or nothing).
    auto step = [&](auto mode_c, int it) __attribute__((always_inline)) {
      constexpr int MODE = decltype(mode_c)::value;
      const int nxt = it + kPStages - 1;
      pwait_tiles<SH>(min(kPStages - 3, ntb - 2 - it), my_instr);
      // every wave is past iteration it-1 (stage (it-1) % kPStages is free)
      // and tile it+1 is visible to every wave
      wait_lgkm<0>();
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (MODE == 0) {
        ps_phase<SH, true>(la, stage_u(it + 1), qf, s, tile_dma(nxt), wave, lane);
      } else {
        if (nxt < ntb) pissue_tile<SH>(tile_dma(nxt), wave, lane);
        if constexpr (MODE == 1) ps_phase<SH, false>(la, stage_u(it + 1), qf, s, PTileDma{}, wave, lane);
      }
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (MODE == 2) {
        if (it < ntw) ppv_phase<SH>(la, stage_u(it), pb, o);
      } else {
        const int key0 = (it + 1) * kPKeys;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          m_raw[nb] = fmaxf(m_raw[nb], ptile_max<MODE == 1>(s[nb], key0, half, vis_lim[nb]));
        ppv_phase<SH>(la, stage_u(it), pb, o);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          ptile_p<MODE == 1>(s[nb], sl2, m_ref[nb], key0, half, vis_lim[nb], l_run[nb], pn[nb]);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          pb[nb][0] = pn[nb][0];
          pb[nb][1] = pn[nb][1];
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    };
    for (int it = 0; it + 1 < ntb; ++it) {
      const int key1 = (it + 1) * kPKeys;
      if (it + 1 >= ntw)
        step(std::integral_constant<int, 2>{}, it);
      else if (key1 + kPKeys > mask_from || it + kPStages - 1 >= ntb)
        step(std::integral_constant<int, 1>{}, it);
      else
        step(std::integral_constant<int, 0>{}, it);
    }
    // P.V of the last tile
    if (ntb - 1 < ntw) {
      wait_lgkm<0>();
      ppv_phase<SH>(la, stage_u(ntb - 1), pb, o);
    }

    // Overflow check: each row's scaled maximum against its reference.
    bool ovf = false;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) ovf |= xor32_max(m_raw[nb]) * sl2 > m_ref[nb] + kPSlack;
    if (__ballot(ovf) != 0 && lane == 0) ds_w32(ovf_flags + 4 * wave, 1u);
    wait_lgkm<0>();
    __builtin_amdgcn_s_barrier();
    uint32_t f[kPWaves];
#pragma unroll
    for (int w = 0; w < kPWaves; ++w) f[w] = ds_r32(ovf_flags + 4 * w);
    wait_lgkm<0>();
    uint32_t any = 0;
#pragma unroll
    for (int w = 0; w < kPWaves; ++w) {
      arrived32(f[w]);
      any |= f[w];
    }
    if (__builtin_amdgcn_readfirstlane(any) == 0) break;
    // Rare: redo the block's tiles with every row's true maximum.
    __builtin_amdgcn_s_barrier();  // all waves have read the flags
    m_init[0] = xor32_max(m_raw[0]) * sl2;
    m_init[1] = xor32_max(m_raw[1]) * sl2;
  }
  // the final P.V MFMAs complete before their accumulators are read
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");

  // finalise
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const float l = xor32_sum(l_run[nb]);
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const int row = wrow0 + nb * 32 + n;
    if (row >= d.seq_q) continue;
    uint16_t *dst = out + (bhq + row) * DV;
#pragma unroll
    for (int cb = 0; cb < SH::CB; ++cb)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        u32x2_t w;
        w[0] = pack2_bf16(o[nb][cb][jq * 4 + 0] * inv, o[nb][cb][jq * 4 + 1] * inv);
        w[1] = pack2_bf16(o[nb][cb][jq * 4 + 2] * inv, o[nb][cb][jq * 4 + 3] * inv);
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
  const size_t lds = (size_t)kPStages * SH::STAGE_BYTES + kPWaves * 4;
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
