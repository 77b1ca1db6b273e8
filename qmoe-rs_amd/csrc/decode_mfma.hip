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
// flight without staging registers.  The token rows of a stage are placed
// so that both the A-operand reads and the transposed V^T reads are free
// of LDS bank conflicts (see DecodeShape).

#include <cmath>
#include <type_traits>
#include <utility>

#include "mfma_pipe.hpp"

namespace qmla {

namespace {

using namespace pipe;

constexpr int kTok = 32;      // tokens per tile
constexpr int kPrefetch = 8;  // S^T operand reads issued ahead of their MFMA

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

// Per-lane LDS byte offsets of the MFMA operands (see DecodeShape).
template <class SH>
struct LaneAddr {
  static constexpr int ROPE_STEPS = SH::KSTEPS - SH::KV_STEPS;
  uint32_t s_kv;                  // S^T operand, c_kv part: + kk*32
  uint32_t s_rope[ROPE_STEPS];    // S^T operand, rope k-steps (XOR-swizzled chunks)
  uint32_t v;                     // V^T operand: + ks/cb offsets
  uint32_t p_rd, p_wr;            // P^T rows: read (row group) / write (own rows)
  int half;
};

template <class SH, int KK>
__device__ __forceinline__ bf16x8_t s_read(const LaneAddr<SH> &la, uint32_t st_kv,
                                           uint32_t st_base) {
  if constexpr (KK < SH::KV_STEPS)
    return ds_b128<KK * 32>(st_kv);
  else
    return ds_b128<0>(st_base + la.s_rope[KK - SH::KV_STEPS]);
}

// DMA of a full tile (all 32 tokens inside the segment), issued in
// per-wave instruction slots: a uniform tile base plus per-lane offsets
// that are the same for every tile, so no per-tile vector address math.
// Per-wave uniform parts of the DMA addresses.  Instruction ins = k*NW +
// wave of a tile splits into a compile-time part (slot k) and these wave
// terms: for one row per group, pi(k*NW + wave) = pi(k*NW) + 4*wave because
// NW <= 4 only touches the low two bits of the token.
struct WaveDma {
  int src_kv, src_rope;  // source byte offsets (row terms)
  int dst_kv, dst_rope;  // LDS byte offsets inside a stage
};

template <class SH, int NW>
__device__ __forceinline__ WaveDma wave_dma(int wave) {
  static_assert(NW == 1 || NW == 2 || NW == 4, "wave count");
  WaveDma w;
  w.src_kv = wave * SH::RPG * (SH::W * 2);
  w.src_rope = wave * (64 / SH::RCH) * (SH::W * 2);
  w.dst_kv = SH::RPG == 1 ? 4 * wave * SH::GS : wave * SH::GS;
  w.dst_rope = wave * 1024;
  return w;
}

struct FullTileDma {
  const uint8_t *tile_base;
  lds_char *stage;
  int wave;
  uint32_t v_kv, v_rope;
  WaveDma w;
};

template <class SH, int NW>
struct DmaSlots {
  static constexpr int MI = (SH::INSTR + NW - 1) / NW;  // slots per wave
  static constexpr bool EVEN = SH::INSTR % NW == 0 && SH::KV_INSTR % NW == 0;
};

// Slot k of this wave: DMA instruction k * NW + wave of the tile.
template <class SH, int NW>
__device__ __forceinline__ void issue_full_one(const FullTileDma &d, int k) {
  constexpr bool EVEN = DmaSlots<SH, NW>::EVEN;
  const int ins0 = k * NW, ins = ins0 + d.wave;
  if (EVEN || ins < SH::INSTR) {
    const uint8_t *tb = fresh(d.tile_base);
    const uint32_t st = fresh(lds_u32(d.stage));
    if (EVEN ? ins0 < SH::KV_INSTR : ins < SH::KV_INSTR) {
      // rows ins*RPG .. +RPG-1, lane covers row ins*RPG + lane/(ROW_B/16)
      dma16(tb + (ins0 * SH::RPG * (SH::W * 2) + d.w.src_kv), d.v_kv,
            st + (uint32_t)((SH::RPG == 1 ? SH::kv_row(ins0) : ins0 * SH::GS) + d.w.dst_kv));
    } else {
      // q0 = rope instruction index of wave 0 (negative for a wave whose
      // first rope instruction follows wave 0's last c_kv one)
      const int q0 = ins0 - SH::KV_INSTR;
      dma16(tb + (q0 * (64 / SH::RCH) * (SH::W * 2) + d.w.src_rope), d.v_rope,
            st + (uint32_t)(SH::KV_BYTES + q0 * 1024 + d.w.dst_rope));
    }
  }
}

// S^T of one tile: KSTEPS dependent MFMAs into the VGPR accumulator s,
// operands read kPrefetch steps ahead (LDS latency is ~3-4 MFMAs).  With
// DMA, this wave's instruction slots for the tile in `d` are spread evenly
// over the MFMAs so the vector-memory issue hides under them.
template <class SH, int NW, bool DMA>
__device__ __forceinline__ void s_phase(const LaneAddr<SH> &la, const lds_char *st,
                                        const bf16x8_t (&qf)[SH::KSTEPS], floatx16_t &s,
                                        const FullTileDma &d) {
  constexpr int D = kPrefetch < SH::KSTEPS ? kPrefetch : SH::KSTEPS;
  constexpr int MI = DmaSlots<SH, NW>::MI;
  const uint32_t st_base = lds_u32(st);
  const uint32_t st_kv = st_base + la.s_kv;
  bf16x8_t a[D + 1];
  [&]<int... K>(std::integer_sequence<int, K...>) {
    ([&] { if constexpr (K < D) a[K] = s_read<SH, K>(la, st_kv, st_base); }(), ...);
    ([&] {
      constexpr int kk = K;
      // reads issued after read kk
      constexpr int after = (kk + D - 1 < SH::KSTEPS - 1 ? D - 1 : SH::KSTEPS - 1 - kk);
      wait_lgkm<after>();
      arrived(a[kk % (D + 1)]);
      if constexpr (kk == 0)
        s = mfma_s_first(a[0], qf[0]);
      else
        mfma_s_acc(s, a[kk % (D + 1)], qf[kk]);
      if constexpr (DMA) {
#pragma unroll
        for (int k = 0; k < MI; ++k)
          if ((k * SH::KSTEPS) / MI == kk) issue_full_one<SH, NW>(d, k);
      }
      if constexpr (kk + D < SH::KSTEPS) a[(kk + D) % (D + 1)] = s_read<SH, kk + D>(la, st_kv, st_base);
    }(), ...);
  }(std::make_integer_sequence<int, SH::KSTEPS>{});
  mfma_s_drain(s);
}

// Split of the O^T accumulation over the block's waves.  Every wave owns
// the S^T / softmax of its 32 query rows; the P.V product is split by
// (row block, column block) instead, so that each wave reads only its share
// of V^T from LDS and takes P^T for all rows from a small LDS buffer.  With
// CW column groups and RW = NW / CW row groups, wave w accumulates column
// blocks w % CW + i * CW (i < NCB) for row blocks w / CW + r * RW (r < NRB).
template <int R, int NW>
struct PvSplit {
  static constexpr int CB = R / 32;
  static constexpr int CW = CB < NW ? CB : NW;
  static constexpr int RW = NW / CW;
  static constexpr int NCB = CB / CW;
  static constexpr int NRB = NW / RW;
  static_assert(NCB * NRB == CB, "accumulator count");
};

// P^T staging: one 80-byte row per query row holding the four 16-byte
// B-operand chunks (k-step ks, half h) at ks*32 + h*16.  The 16-byte pad
// spreads 16 consecutive rows over distinct LDS bank groups.
constexpr int kPRow = 80;

template <class SH>
__device__ __forceinline__ void p_write(const LaneAddr<SH> &la, uint32_t pbuf,
                                        const bf16x8_t (&pn)[2]) {
  ds_w128<0>(pbuf + la.p_wr, pn[0]);
  ds_w128<32>(pbuf + la.p_wr, pn[1]);
}

// O^T += V^T P^T for this wave's share of one tile: NCB x NRB x 2 MFMAs
// into the AGPR accumulators.  P^T fragments of both k-steps are loaded
// first, then the V^T fragments stream kPvAhead ahead of their MFMAs.
constexpr int kPvAhead = 3;

template <class SH, class PS, int J>
__device__ __forceinline__ bf16x8_t v_frag(uint32_t vb) {
  constexpr int ks = J / PS::NCB, i = J % PS::NCB;
  return ds_tr2<ks * SH::HI16 + i * PS::CW * 64, SH::HI8>(vb);
}

// mid.part<j>() runs after the MFMAs of V^T fragment j (the softmax of the
// next tile, spread over the MFMAs: this wave is alone on its SIMD, so its
// VALU work hides only under its own MFMAs).
// LDS read order of pv_phase: the P^T fragments of k-step 0 (NRB reads)
// and V^T fragments 0 .. DA-1 (two reads each) up front; after the MFMAs of
// fragment j, V^T fragment j + DA, and after those of fragment 0 the P^T
// fragments of k-step 1 (first needed by fragment NCB).  wait_after(j) =
// reads issued after the last one fragment j needs, at its wait.
template <int NA, int DA, int NRB, int NCB>
struct PvOrder {
  static constexpr int issued_before(int j) {
    int n = NRB + 2 * DA;
    for (int i = 0; i < j; ++i) n += (i + DA < NA ? 2 : 0) + (i == 0 ? NRB : 0);
    return n;
  }
  static constexpr int last_a(int j) { return j < DA ? NRB + 2 * j + 1 : issued_before(j - DA) + 1; }
  static constexpr int last_p1() { return issued_before(0) + (DA < NA ? 2 : 0) + NRB - 1; }
  static constexpr int wait_after(int j) {
    int need = last_a(j);
    if (j == 0 && NRB - 1 > need) need = NRB - 1;
    if (j == NCB && last_p1() > need) need = last_p1();
    return issued_before(j) - 1 - need;
  }
};

// mid.part<j>() runs after the MFMAs of V^T fragment j (the softmax of the
// next tile, spread over the MFMAs: this wave is alone on its SIMD, so its
// VALU work hides only under its own MFMAs).
template <class SH, class PS, class MID>
__device__ __forceinline__ void pv_phase(const LaneAddr<SH> &la, const lds_char *st,
                                         uint32_t pbuf, int cw,
                                         floatx16_t (&o)[PS::NCB][PS::NRB], MID &mid) {
  constexpr int NA = 2 * PS::NCB;  // V^T fragments (k-step, column block)
  constexpr int DA = kPvAhead < NA ? kPvAhead : NA;
  using ORD = PvOrder<NA, DA, PS::NRB, PS::NCB>;
  const uint32_t vb = lds_u32(st) + la.v + cw * 64;
  const uint32_t pb = pbuf + la.p_rd;
  bf16x8_t b[2][PS::NRB], a[DA + 1];
  auto read_p = [&](auto ks_c) __attribute__((always_inline)) {
    constexpr int KS = decltype(ks_c)::value;
    [&]<int... R>(std::integer_sequence<int, R...>) {
      ((b[KS][R] = ds_b128<R * PS::RW * 32 * kPRow + KS * 32>(pb)), ...);
    }(std::make_integer_sequence<int, PS::NRB>{});
  };
  read_p(std::integral_constant<int, 0>{});
  [&]<int... J>(std::integer_sequence<int, J...>) {
    ([&] { if constexpr (J < DA) a[J] = v_frag<SH, PS, J>(vb); }(), ...);
    ([&] {
      constexpr int j = J;
      constexpr int after = ORD::wait_after(j);
      static_assert(after >= 0 && after <= 15, "lgkmcnt");
      wait_lgkm<after>();
      arrived(a[j % (DA + 1)]);
      if constexpr (j == 0 || j == PS::NCB) {
#pragma unroll
        for (int r = 0; r < PS::NRB; ++r) arrived(b[j == 0 ? 0 : 1][r]);
      }
#pragma unroll
      for (int r = 0; r < PS::NRB; ++r)
        o[j % PS::NCB][r] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            a[j % (DA + 1)], b[j / PS::NCB][r], o[j % PS::NCB][r], 0, 0, 0);
      mid.template part<j, NA>();
      if constexpr (j + DA < NA) a[(j + DA) % (DA + 1)] = v_frag<SH, PS, j + DA>(vb);
      if constexpr (j == 0) read_p(std::integral_constant<int, 1>{});
      __builtin_amdgcn_sched_barrier(0);
    }(), ...);
  }(std::make_integer_sequence<int, NA>{});
}

struct NoMid {
  template <int J, int N>
  __device__ __forceinline__ void part() {}
};

// Online softmax in the log2 domain with a lazy fixed reference.  The
// reference m (scaled units) is the first tile's row maximum, or the one a
// restart hands in, and then stays fixed: p = exp2(s * scale_log2 - m).
// Each lane tracks the largest 16-token partial sum of p it forms, an upper
// bound of every p in it; after the segment the block checks it against
// kOverflow, and in the rare case of an overflow redoes the segment with a
// reference at or above the true maximum (see the kernel).  The O^T
// accumulators are therefore only ever MFMA-accumulated, zeroed at a
// segment start or read at the end -- never rescaled in registers, which
// keeps all 256 of them in AGPRs -- and the per-tile softmax has no branch,
// so it splits into pieces spread over the P.V MFMAs.
constexpr float kOverflow = 65536.f;  // largest p kept (2^16) before a restart
// The narrow kernel (4 scores per lane and tile) checks row maxima instead:
// a score above m + kRefSlack restarts its segment.
constexpr float kRefSlack = 16.f;

// Token (within the tile) of S^T accumulator element j of this lane.
__device__ __forceinline__ int tile_tok(int j, int half) {
  return 8 * (j >> 2) + 4 * half + (j & 3);
}

// Raw (unscaled) maximum of this lane's 16 scores; with MASK, tokens at or
// past `valid` are ignored.
template <bool MASK>
__device__ __forceinline__ float tile_max(const floatx16_t &s, int valid, int half) {
  float x[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) x[j] = (!MASK || tile_tok(j, half) < valid) ? s[j] : -INFINITY;
  float m01 = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
  float m23 = fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7]));
  float m45 = fmaxf(fmaxf(x[8], x[9]), fmaxf(x[10], x[11]));
  float m67 = fmaxf(fmaxf(x[12], x[13]), fmaxf(x[14], x[15]));
  return fmaxf(fmaxf(m01, m23), fmaxf(m45, m67));
}

// p = exp2(s * sl2 - m) packed into the two bf16 B-operand fragments of
// P^T; adds the lane's 16-token mass to l and folds it into tmax.  sl2 >= 0.
// part<I, N>() computes the I-th of N pieces: score pairs i with
// i * N / 8 == I, and the totals with the last piece.
template <bool MASK>
struct TileSoftmax {
  const floatx16_t &s;
  float sl2, m;
  int valid, half;
  float &l, &tmax;
  bf16x8_t (&pb)[2];
  float q[8];
  u32x4_t pk[2];

  template <int I, int N>
  __device__ __forceinline__ void part() {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i * N / 8 != I) continue;
      float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * i], sl2, -m));
      float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * i + 1], sl2, -m));
      if (MASK) {
        p0 = tile_tok(2 * i, half) < valid ? p0 : 0.f;
        p1 = tile_tok(2 * i + 1, half) < valid ? p1 : 0.f;
      }
      q[i] = p0 + p1;
      pk[i / 4][i % 4] = pack2_bf16(p0, p1);
    }
    if constexpr (I == N - 1) {
      const float t = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
      l += t;
      tmax = fmaxf(tmax, t);
      pb[0] = __builtin_bit_cast(bf16x8_t, pk[0]);
      pb[1] = __builtin_bit_cast(bf16x8_t, pk[1]);
    }
  }
};

template <bool MASK>
__device__ __forceinline__ void tile_p(const floatx16_t &s, float sl2, float m, int valid,
                                       int half, float &l, float &tmax, bf16x8_t (&pb)[2]) {
  TileSoftmax<MASK> t{s, sl2, m, valid, half, l, tmax, pb};
  t.template part<0, 1>();
}

template <class SH, int NW>
__device__ __forceinline__ void issue_full_tile(const FullTileDma &d) {
#pragma unroll
  for (int k = 0; k < DmaSlots<SH, NW>::MI; ++k) issue_full_one<SH, NW>(d, k);
}

// First row of the tile of a sequence starting at token t, a multiple of
// kTok: the plan cuts sequences at multiples of kTok and a page holds a
// multiple of kTok rows, so the tile's rows are consecutive in one page.
// `prow` is the sequence's block-table row; t is uniform, so this is one
// scalar load.
template <class SH>
__device__ __forceinline__ const uint8_t *tile_rows(const uint64_t *__restrict__ prow, int shift,
                                                    int t) {
  const uint64_t page = prow[t >> shift];
  return reinterpret_cast<const uint8_t *>(page) + (int64_t)(t & ((1 << shift) - 1)) * (SH::W * 2);
}

// DMA of the segment's last, partial tile: tokens past `last` (the last
// valid token, relative to the tile) re-load that token's row, which the
// softmax masks.  Sources are the uniform tile base plus 32-bit per-lane
// offsets; the LDS position (and rope swizzle) stays that of the unclamped
// token.
template <class SH, int NW>
__device__ __forceinline__ void issue_clamped_tile(const uint8_t *__restrict__ tile_base,
                                                   lds_char *stage, int wave, int lane_in,
                                                   int last, const WaveDma &w) {
  constexpr bool EVEN = DmaSlots<SH, NW>::EVEN;
  const int lane = vfresh(lane_in);
#pragma unroll
  for (int ins0 = 0; ins0 < SH::INSTR; ins0 += NW) {
    const int ins = ins0 + wave;
    if (EVEN || ins < SH::INSTR) {
      int t, c, base_b, dst;
      if (EVEN ? ins0 < SH::KV_INSTR : ins < SH::KV_INSTR) {
        t = ins * SH::RPG + lane / (SH::ROW_B / 16);
        c = lane % (SH::ROW_B / 16);
        base_b = 0;
        dst = (SH::RPG == 1 ? SH::kv_row(ins0) : ins0 * SH::GS) + w.dst_kv;
      } else {
        const int q = ins - SH::KV_INSTR;
        t = q * (64 / SH::RCH) + lane / SH::RCH;
        c = (lane % SH::RCH) ^ (t & (SH::RCH - 1));
        base_b = SH::ROW_B;
        dst = SH::KV_BYTES + (ins0 - SH::KV_INSTR) * 1024 + w.dst_rope;
      }
      dma16(fresh(tile_base), (uint32_t)(min(t, last) * (SH::W * 2) + base_b + c * 16),
            fresh(lds_u32(stage)) + (uint32_t)dst);
    }
  }
}

template <class SH, int NW>
__device__ __forceinline__ void issue_any_tile(const uint8_t *__restrict__ tile_base, int tile_t0,
                                               int seg_t1, lds_char *stage, int wave, int lane,
                                               uint32_t v_kv, uint32_t v_rope, const WaveDma &w) {
  if (tile_t0 + kTok <= seg_t1)
    issue_full_tile<SH, NW>(FullTileDma{tile_base, stage, wave, v_kv, v_rope, w});
  else
    issue_clamped_tile<SH, NW>(tile_base, stage, wave, lane, seg_t1 - 1 - tile_t0, w);
}

// True when any wave of the block raised its reference-overflow flag
// (flags: NW words at LDS address `flags`; written before a barrier).
template <int NW>
__device__ __forceinline__ bool any_flag(uint32_t flags) {
  uint32_t v[NW];
#pragma unroll
  for (int w = 0; w < NW; ++w) v[w] = ds_r32(flags + 4 * w);
  wait_lgkm<0>();
  uint32_t f = 0;
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    arrived32(v[w]);
    f |= v[w];
  }
  return __builtin_amdgcn_readfirstlane(f) != 0;
}

// ---- in-kernel split plan.  The concatenated tokens of the batch are cut
// into gridDim.x pieces of `chunk` tokens; piece i covers [i*chunk,
// (i+1)*chunk).  Each sequence is preceded by seg_tokens virtual tokens in
// this stream: a segment costs a fixed setup (Q load, prologue, partial
// store) on top of its tiles, and a piece that starts a new sequence gets
// correspondingly fewer real tokens.  A (piece, sequence) overlap of real
// tokens is a segment; every segment
// writes a partial result to its own slot: sequence b owns slots
// sb[b] .. sb[b] + ns[b] - 1 (ns[b] = pieces it touches), in piece order.
// Each block derives its own segments (no separate planning launch): the
// length prefix sums are rebuilt in the idle stage ring, and up to kSegCap
// segment descriptors are kept in LDS; a block with more segments plans
// again when its list runs out.  The block whose piece holds a sequence's
// first token (blockIdx.y == 0) records {sb, ns} for the merge.
constexpr int kSegCap = 64;

struct SegDesc {
  int32_t seq, t0, t1, slot;
};

// Exclusive scan of a[0..n) in LDS; returns the total.  Up to 512 values
// are scanned by wave 0 alone (lane-local runs, then a shuffle scan: one
// barrier in all); longer arrays by all NT threads (log-step, two barriers
// per step).
// The piece of this block.  Blocks are dealt to the 8 XCDs round-robin, so
// block i maps to piece (i % 8) * (grid / 8) + i / 8: consecutive pieces,
// i.e. the pieces of one sequence, sit on one XCD and its query rows come
// from that XCD's L2 after the first load (16-head decode 41.0-41.4 ->
// 40.5-40.8 us per step in a same-box A/B; the 128-head decode within noise).
__device__ __forceinline__ int decode_piece() {
  const int g = gridDim.x, b = blockIdx.x;
  return (g & 7) ? b : (b & 7) * (g >> 3) + (b >> 3);
}

template <int NT>
__device__ int32_t lds_exscan(int32_t *a, int32_t n, int32_t *tmp) {
  if (n <= 512) {
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      const int per = (n + 63) / 64;
      const int lo = min(n, lane * per), hi = min(n, lo + per);
      int32_t local = 0;
      for (int i = lo; i < hi; ++i) local += a[i];
      int32_t incl = local;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int32_t v = __shfl_up(incl, off);
        if (lane >= off) incl += v;
      }
      int32_t run = incl - local;
      for (int i = lo; i < hi; ++i) {
        const int32_t v = a[i];
        a[i] = run;
        run += v;
      }
      if (lane == 63) tmp[0] = incl;
    }
    __syncthreads();
    return tmp[0];
  }
  const int tid = threadIdx.x;
  const int per = (n + NT - 1) / NT;
  const int lo = min(n, tid * per), hi = min(n, lo + per);
  int32_t local = 0;
  for (int i = lo; i < hi; ++i) local += a[i];
  tmp[tid] = local;
  __syncthreads();
  for (int off = 1; off < NT; off <<= 1) {
    const int32_t v = tid >= off ? tmp[tid - off] : 0;
    __syncthreads();
    tmp[tid] += v;
    __syncthreads();
  }
  int32_t run = tid > 0 ? tmp[tid - 1] : 0;
  const int32_t total = tmp[NT - 1];
  for (int i = lo; i < hi; ++i) {
    const int32_t v = a[i];
    a[i] = run;
    run += v;
  }
  __syncthreads();
  return total;
}

// One planning round: fills list[0..count) with this block's segments of
// sequences >= from, sets *next to the first sequence not listed (batch
// when done).  scratch: 2 * (batch + 1) + NT int32 of idle LDS.  In the
// virtual stream, sequence b occupies [P[b], P[b + 1]) with its real
// tokens at [v0, v0 + L) = [P[b] + seg_tokens, P[b + 1]).  Sequences are
// cut only at tile boundaries (multiples of kTok from the sequence start):
// the tile starting at virtual position v belongs to the piece holding v,
// so every segment starts at a multiple of kTok and each of its tiles lies
// in one cache page.  A piece is at least kTok long, so the pieces holding
// a sequence's tile starts are consecutive and each gets a non-empty segment.
template <int NT>
__device__ void plan_round(const int32_t *__restrict__ lens, int32_t pending, int32_t batch,
                           int32_t from, int32_t seg_tokens, int32_t *scratch, SegDesc *list,
                           int32_t *meta, int2 *__restrict__ seq_info) {
  const int tid = threadIdx.x;
  const int blocks = gridDim.x, piece = decode_piece();
  int32_t *P = scratch, *SB = scratch + batch + 1, *tmp = SB + batch + 1;
  for (int b = tid; b < batch; b += NT) P[b] = lens[b] + pending + seg_tokens;
  __syncthreads();
  const int32_t N = lds_exscan<NT>(P, batch, tmp);
  if (tid == 0) P[batch] = N;
  const int32_t chunk = max(kTok, (N + blocks - 1) / blocks);
  __syncthreads();
  // pieces holding the tile starts of a sequence with real tokens [v0, v0 + L)
  auto touched = [&](int32_t v0, int32_t L) {
    return L > 0 ? (v0 + (L - 1) / kTok * kTok) / chunk - v0 / chunk + 1 : 0;
  };
  // sequence-relative cut at virtual position x: the first tile start >= x
  auto cut = [&](int32_t x, int32_t v0, int32_t L) {
    return x <= v0 ? 0 : min(L, (x - v0 + kTok - 1) / kTok * kTok);
  };
  for (int b = tid; b < batch; b += NT) {
    const int32_t v0 = P[b] + seg_tokens;
    SB[b] = touched(v0, P[b + 1] - v0);
  }
  __syncthreads();
  (void)lds_exscan<NT>(SB, batch, tmp);
  if (from == 0 && blockIdx.y == 0) {
    for (int b = tid; b < batch; b += NT) {
      const int32_t v0 = P[b] + seg_tokens;
      if (min(v0 / chunk, blocks - 1) == piece)
        seq_info[b] = make_int2(SB[b], touched(v0, P[b + 1] - v0));
    }
  }
  if (tid == 0) {
    const int32_t start = min(piece * chunk, N), end = min(start + chunk, N);
    // first sequence >= from whose tokens reach past start
    int32_t lo = from, hi = batch;
    while (lo < hi) {
      const int32_t mid = (lo + hi) >> 1;
      if (P[mid + 1] > start) hi = mid; else lo = mid + 1;
    }
    int32_t cnt = 0, b = lo;
    for (; b < batch && P[b] + seg_tokens < end && cnt < kSegCap; ++b) {
      const int32_t v0 = P[b] + seg_tokens, L = P[b + 1] - v0;
      const int32_t t0 = cut(start, v0, L), t1 = cut(end, v0, L);
      if (t1 <= t0) continue;  // empty sequence, or no tile start inside the piece
      list[cnt++] = SegDesc{b, t0, t1, SB[b] + (piece - v0 / chunk)};
    }
    meta[0] = cnt;
    meta[1] = (b < batch && P[b] + seg_tokens < end) ? b : batch;
  }
  __syncthreads();
}

// The same plan for batch <= 64, computed by every wave in registers (lane b
// = sequence b): two shuffle scans and a ballot instead of LDS round trips
// and barriers, so the first tiles are requested sooner.  A piece then holds
// at most 64 <= kSegCap segments: one round.  Segment i is the i-th set bit
// of mask, in ascending sequence order as in plan_round.
struct WavePlan {
  uint64_t mask;
  int32_t t0, t1, slot;  // this lane's sequence
};

__device__ __forceinline__ int32_t wave_incl_scan(int32_t x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int32_t v = __shfl_up(x, off);
    if (lane >= off) x += v;
  }
  return x;
}

__device__ WavePlan plan_wave(const int32_t *__restrict__ lens, int32_t pending, int32_t batch,
                              int32_t seg_tokens, int2 *__restrict__ seq_info) {
  static_assert(kSegCap >= 64, "one round per piece");
  const int lane = threadIdx.x & 63;
  const int blocks = gridDim.x, piece = decode_piece();
  const bool live = lane < batch;
  const int32_t x = live ? lens[lane] + pending + seg_tokens : 0;
  const int32_t incl = wave_incl_scan(x);  // P[b + 1]
  const int32_t N = __shfl(incl, 63);
  const int32_t chunk = max(kTok, (N + blocks - 1) / blocks);
  const int32_t v0 = incl - x + seg_tokens, L = x - seg_tokens;
  const int32_t first = v0 / chunk;
  const int32_t touched = live && L > 0 ? (v0 + (L - 1) / kTok * kTok) / chunk - first + 1 : 0;
  const int32_t sb = wave_incl_scan(touched) - touched;
  if (blockIdx.y == 0 && (threadIdx.x >> 6) == 0 && live && min(first, blocks - 1) == piece)
    seq_info[lane] = make_int2(sb, touched);
  const int32_t start = min(piece * chunk, N), end = min(start + chunk, N);
  auto cut = [&](int32_t c) { return c <= v0 ? 0 : min(L, (c - v0 + kTok - 1) / kTok * kTok); };
  WavePlan w;
  w.t0 = cut(start);
  w.t1 = cut(end);
  w.slot = sb + (piece - first);
  w.mask = __ballot(live && incl > start && v0 < end && w.t1 > w.t0);
  return w;
}

// One planning round of a block: the segment count; next_seq = the first
// sequence of the next round (batch when there is none).
template <int NT>
__device__ __forceinline__ int32_t plan_segments(const int32_t *__restrict__ lens, int32_t pending,
                                                 int32_t batch, int32_t &next_seq,
                                                 int32_t seg_tokens, int32_t *scratch,
                                                 SegDesc *list, int32_t *meta,
                                                 int2 *__restrict__ seq_info, WavePlan &wp) {
  if (batch <= 64) {
    wp = plan_wave(lens, pending, batch, seg_tokens, seq_info);
    next_seq = batch;
    return __builtin_popcountll(wp.mask);
  }
  plan_round<NT>(lens, pending, batch, next_seq, seg_tokens, scratch, list, meta, seq_info);
  next_seq = __builtin_amdgcn_readfirstlane(meta[1]);
  return __builtin_amdgcn_readfirstlane(meta[0]);
}

// Segment si of the round (called for si = 0, 1, ... in order).
__device__ __forceinline__ SegDesc plan_segment(int32_t si, int32_t batch, const SegDesc *list,
                                                WavePlan &wp) {
  SegDesc sg;
  if (batch <= 64) {
    const int ln = __builtin_ctzll(wp.mask);
    wp.mask &= wp.mask - 1;
    sg.seq = ln;
    sg.t0 = __builtin_amdgcn_readlane(wp.t0, ln);
    sg.t1 = __builtin_amdgcn_readlane(wp.t1, ln);
    sg.slot = __builtin_amdgcn_readlane(wp.slot, ln);
  } else {
    const SegDesc d = list[si];
    sg.seq = __builtin_amdgcn_readfirstlane(d.seq);
    sg.t0 = __builtin_amdgcn_readfirstlane(d.t0);
    sg.t1 = __builtin_amdgcn_readfirstlane(d.t1);
    sg.slot = __builtin_amdgcn_readfirstlane(d.slot);
  }
  return sg;
}

// Dynamic LDS of one block: the NSTAGE tile ring, the P^T staging rows,
// the per-row softmax denominators exchanged at the end of a segment, the
// per-wave reference-overflow flags and the segment list (+ 2 words).
template <int R, int DR, int NW, int NSTAGE>
constexpr size_t decode_lds_bytes() {
  return (size_t)NSTAGE * DecodeShape<R, DR>::STAGE_BYTES + NW * 32 * kPRow + NW * 32 * 4 +
         NW * 4 + kSegCap * sizeof(SegDesc) + 16;
}

// Partial results: slot-major, then 32-row block, then 32-column block; a
// block is 1024 bf16 (2 KB, rounded to nearest even; the log-sum-exp stays
// f32) in the MFMA accumulator order [jq][lane][4] (element j of lane l:
// row l % 32, column 8 (j / 4) + 4 (l / 32) + j % 4), so each store
// instruction writes 512 B contiguously.  part_lse: [slot][rows padded to 32].
template <int R, int DR, int NW, int NSTAGE, typename QT>
__global__ __launch_bounds__(NW * 64) void k_decode_mfma(
    const uint64_t *__restrict__ pages, int32_t pt_width, int32_t pt_shift,
    const int32_t *__restrict__ lens, int32_t batch, const QT *__restrict__ q_lat,
    const QT *__restrict__ q_rope, int32_t rows, float scale_log2, int32_t seg_tokens,
    int32_t pending, int2 *__restrict__ seq_info, uint16_t *__restrict__ part_o,
    float *__restrict__ part_lse) {
  using SH = DecodeShape<R, DR>;
  using PS = PvSplit<R, NW>;
  static_assert(NSTAGE >= 3, "the pipelined loop keeps two stages resident");
  extern __shared__ __attribute__((aligned(16))) char ring_raw[];
  lds_char *ring = (lds_char *)ring_raw;
  lds_char *pbuf = ring + NSTAGE * SH::STAGE_BYTES;
  const uint32_t l_rows = lds_u32(pbuf + NW * 32 * kPRow);  // NW*32 floats
  const uint32_t ovf_flags = l_rows + NW * 32 * 4;         // NW words
  lds_char *seg_lds = pbuf + NW * 32 * kPRow + NW * 32 * 4 + NW * 4;
  SegDesc *seg_list = (SegDesc *)seg_lds;                   // kSegCap entries
  int32_t *seg_meta = (int32_t *)(seg_lds + kSegCap * sizeof(SegDesc));
  const int row_blocks = (rows + 31) / 32;  // of the padded partial layout
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n = lane & 31;     // row within a 32-row block = MFMA column
  const int half = lane >> 5;  // which 8-wide k half of an MFMA operand
  const int row0 = blockIdx.y * (NW * 32);  // first query row of this block
  const int row = row0 + wave * 32 + n;     // this lane's softmax row
  const bool row_ok = row < rows;
  const int row_c = row_ok ? row : rows - 1;
  const int cw = wave % PS::CW, rg = wave / PS::CW;  // P.V share of this wave
  const int my_instr = (SH::INSTR - wave + NW - 1) / NW;
  // A negative scale is applied as |scale| with the sign folded into q
  // (exact in bf16), so the raw score maximum is also the scaled one.
  const uint32_t q_sign = scale_log2 < 0.f ? 0x80008000u : 0u;
  const float sl2 = fabsf(scale_log2);

  LaneAddr<SH> la;
  la.s_kv = SH::kv_row(n) + half * 16;
#pragma unroll
  for (int rk = 0; rk < LaneAddr<SH>::ROPE_STEPS; ++rk)
    la.s_rope[rk] = SH::KV_BYTES + n * (DR * 2) + (((2 * rk + half) ^ (n & (SH::RCH - 1))) * 16);
  {
    const int g = lane >> 4, sl = lane & 15;
    const int tok_a = (g >= 2 ? 4 : 0) + (sl >> 2);
    const int col_in = (g & 1) * 16 + 4 * (sl & 3);
    la.v = SH::kv_row(tok_a) + (col_in >> 3) * 16 + (col_in & 7) * 2;
  }
  la.p_rd = (32 * rg + n) * kPRow + half * 16;
  la.p_wr = (32 * wave + n) * kPRow + half * 16;
  la.half = half;
  const uint32_t pbuf_u = lds_u32(pbuf);
  // per-lane source offsets of a full tile's DMA (see issue_tile)
  const uint32_t v_kv = (lane / (SH::ROW_B / 16)) * (SH::W * 2) + (lane % (SH::ROW_B / 16)) * 16;
  const WaveDma wd = wave_dma<SH, NW>(wave);
  const uint32_t v_rope = (lane / SH::RCH) * (SH::W * 2) + SH::ROW_B +
                          ((lane % SH::RCH) ^ ((lane / SH::RCH) & (SH::RCH - 1))) * 16;

  int32_t next_seq = 0;
  do {
  WavePlan wp;
  const int32_t nseg = plan_segments<NW * 64>(lens, pending, batch, next_seq, seg_tokens,
                                              (int32_t *)ring_raw, seg_list, seg_meta, seq_info, wp);
  for (int32_t si = 0; si < nseg; ++si) {
    const SegDesc sg = plan_segment(si, batch, seg_list, wp);
    const int64_t qrow_c = (int64_t)sg.seq * rows + row_c;
    const uint64_t *prow = pages + (int64_t)sg.seq * pt_width;
    const int T = sg.t1 - sg.t0;
    const int ntiles = (T + kTok - 1) / kTok;
    auto stage = [&](int t) { return ring + (t % NSTAGE) * SH::STAGE_BYTES; };
    // prologue: NSTAGE-1 tiles in flight (issued before the Q loads so the
    // two latencies overlap; a restart issues them again)
    auto prologue = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int p = 0; p < NSTAGE - 1; ++p)
        if (p < ntiles)
          issue_any_tile<SH, NW>(tile_rows<SH>(prow, pt_shift, sg.t0 + p * kTok), sg.t0 + p * kTok,
                                 sg.t1, stage(p), wave, lane, v_kv, v_rope, wd);
    };
    prologue();

    // Q fragment = B operand of S^T: dims kk*16 + 8*half .. +7 of this row.
    bf16x8_t qf[SH::KSTEPS];
    const uint32_t keep = row_ok ? 0xffffffffu : 0u;
#pragma unroll
    for (int kk = 0; kk < SH::KSTEPS; ++kk) {
      u32x4_t u = __builtin_bit_cast(u32x4_t, load_q8<R, DR, QT>(q_lat, q_rope, qrow_c,
                                                                  kk * 16 + half * 8));
#pragma unroll
      for (int i = 0; i < 4; ++i) u[i] = (u[i] ^ q_sign) & keep;
      qf[kk] = __builtin_bit_cast(bf16x8_t, u);
    }

    floatx16_t o[PS::NCB][PS::NRB];
    floatx16_t s;
    bf16x8_t pn[2];
    float m_run, l_run, t_max;
    float m_init = -INFINITY;  // reference to (re)start the segment with
    for (;;) {
#pragma unroll
      for (int i = 0; i < PS::NCB; ++i)
#pragma unroll
        for (int r = 0; r < PS::NRB; ++r)
#pragma unroll
          for (int j = 0; j < 16; ++j) o[i][r][j] = 0.f;
      l_run = 0.f;
      if (lane == 0) ds_w32(ovf_flags + 4 * wave, 0u);

      // prologue in flight (re-issued on a restart), then S and softmax of tile 0
      if (m_init != -INFINITY) prologue();
      wait_tiles<SH, NW>(min(NSTAGE - 2, ntiles - 1), my_instr);
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      s_phase<SH, NW, false>(la, stage(0), qf, s, FullTileDma{});
      t_max = 0.f;
      m_run = m_init == -INFINITY ? xor32_max(tile_max<true>(s, T, half)) * sl2 : m_init;
      tile_p<true>(s, sl2, m_run, T, half, l_run, t_max, pn);
      __builtin_amdgcn_sched_barrier(0);

      // Steady state, iteration it: publish P of tile it, S^T of tile it+1,
      // then P.V of tile it with the softmax of tile it+1 spread over its
      // MFMAs.  FAST iterations (the prefetched tile it+NSTAGE-1 is a full
      // tile and tile it+1 is not the last) spread their DMA over the S^T
      // MFMAs and carry no mask; the at most NSTAGE-1 tail iterations issue
      // their (possibly clamped) DMA up front and mask the scores.
      auto step = [&](auto fast, int it) __attribute__((always_inline)) {
        constexpr bool FAST = decltype(fast)::value;
        const int nxt = it + NSTAGE - 1;
        // rows of tile nxt, loaded ahead of barrier A, whose wait covers it
        const uint8_t *nxt_rows =
            tile_rows<SH>(prow, pt_shift, sg.t0 + min(nxt, ntiles - 1) * kTok);
        // tile it+1 must be complete; tile it+2 (if issued) may stay in flight
        if constexpr (FAST)
          wait_tiles<SH, NW>(NSTAGE - 3, my_instr);
        else
          wait_tiles<SH, NW>(min(NSTAGE - 3, ntiles - 2 - it), my_instr);
        // Barrier A: every wave is past iteration it-1, so stage (it-1) %
        // NSTAGE and the P^T rows are free, and tile it+1 is visible.
        __builtin_amdgcn_s_waitcnt((0xF) | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (!FAST && nxt < ntiles)
          issue_any_tile<SH, NW>(nxt_rows, sg.t0 + nxt * kTok, sg.t1, stage(nxt), wave, lane,
                                 v_kv, v_rope, wd);
        p_write(la, pbuf_u, pn);
        __builtin_amdgcn_sched_barrier(0);
        s_phase<SH, NW, FAST>(la, stage(it + 1), qf, s,
                              FullTileDma{nxt_rows, stage(nxt), wave, v_kv, v_rope, wd});
        // Barrier B: P^T of tile it is complete in LDS.
        __builtin_amdgcn_s_waitcnt((0xF) | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        const int valid = T - (it + 1) * kTok;
        TileSoftmax<!FAST> sm{s, sl2, m_run, valid, half, l_run, t_max, pn};
        pv_phase<SH, PS>(la, stage(it), pbuf_u, cw, o, sm);
        __builtin_amdgcn_sched_barrier(0);
      };
      int it = 0;
      for (; it + NSTAGE + 1 <= ntiles; ++it) step(std::true_type{}, it);
      for (; it + 1 < ntiles; ++it) step(std::false_type{}, it);
      // P.V of the last tile
      __builtin_amdgcn_s_waitcnt((0xF) | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
      __builtin_amdgcn_s_barrier();
      p_write(la, pbuf_u, pn);
      __builtin_amdgcn_s_waitcnt((0xF) | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
      __builtin_amdgcn_s_barrier();
      {
        NoMid none;
        pv_phase<SH, PS>(la, stage(ntiles - 1), pbuf_u, cw, o, none);
      }

      // Overflow check: some p of the row above kOverflow.
      const float t_row = xor32_max(t_max);
      const bool ovf = __ballot(t_row > kOverflow) != 0;  // every lane votes
      if (ovf && lane == 0) ds_w32(ovf_flags + 4 * wave, 1u);
      // Every wave is done with the stages and the P^T rows (the next
      // segment's or attempt's prologue refills them) and every overflow
      // flag is visible.
      __builtin_amdgcn_s_waitcnt((0xF) | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
      __builtin_amdgcn_s_barrier();
      if (!any_flag<NW>(ovf_flags)) break;
      // Rare: some row's scores outgrew the reference.  Redo the segment
      // with a reference at or above every row's true maximum (each p <=
      // its 16-token sum <= t_row), so no p of the second pass exceeds 1.
      __builtin_amdgcn_s_barrier();  // all waves have read the flags
      m_init = m_run + log2f(t_row);
    }

    // ---- finalise: denominators of this wave's rows, shared with the
    // waves holding other parts of those rows' O^T.  Lane-derived addresses
    // are formed here from an opaque lane index (nothing kept across the
    // loop for them).
    const int fl = vfresh(lane), fn = fl & 31, fh = fl >> 5;
    l_run = xor32_sum(l_run);
    const float lse = (m_run + log2f(l_run)) * 0.69314718055994531f;
    const int frow = row0 + wave * 32 + fn;
    if (fh == 0) ds_w32(l_rows + 4 * (wave * 32 + fn), __builtin_bit_cast(uint32_t, l_run));
    const int slot = sg.slot;
    // rows past the padded partial layout (a wave beyond the last 32-row
    // block of this pass) store nothing
    if (fh == 0 && frow < row_blocks * 32) part_lse[(int64_t)slot * (row_blocks * 32) + frow] = lse;
    __builtin_amdgcn_s_waitcnt((0xF) | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
    __builtin_amdgcn_s_barrier();
    // every denominator first: no LDS access between the output stores
    float inv[PS::NRB];
    {
      uint32_t lv[PS::NRB];
#pragma unroll
      for (int r = 0; r < PS::NRB; ++r) lv[r] = ds_r32(l_rows + 4 * (32 * (rg + r * PS::RW) + fn));
      wait_lgkm<0>();
#pragma unroll
      for (int r = 0; r < PS::NRB; ++r) {
        arrived32(lv[r]);
        inv[r] = 1.f / __builtin_bit_cast(float, lv[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < PS::NRB; ++r) {
      const int rb = blockIdx.y * NW + rg + r * PS::RW;  // 32-row block of the padded rows
      if (rb >= row_blocks) continue;
      uint16_t *blk = part_o + (((int64_t)slot * row_blocks + rb) * (R / 32)) * 1024 + fl * 4;
#pragma unroll
      for (int i = 0; i < PS::NCB; ++i) {
        const int cb = cw + i * PS::CW;
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
          u32x2_t v;
          v[0] = pack2_bf16(o[i][r][jq * 4] * inv[r], o[i][r][jq * 4 + 1] * inv[r]);
          v[1] = pack2_bf16(o[i][r][jq * 4 + 2] * inv[r], o[i][r][jq * 4 + 3] * inv[r]);
          *reinterpret_cast<u32x2_t *>(blk + cb * 1024 + jq * 256) = v;
        }
      }
    }
    // l_rows is rewritten by the next segment only after its prologue barrier
  }
  // the next planning round reuses the stage ring: every wave is done with it
  __builtin_amdgcn_s_waitcnt((0xF) | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
  __builtin_amdgcn_s_barrier();
  } while (next_seq < batch);
}

// Log-sum-exp merge of the partial slots into the row-major output.  One
// wave per (sequence, 32-row block, 32-column block): per-row weights
// exp(lse_s - max) from the slots' lse, the weighted sum of the slots' 4 KB
// blocks, then an LDS transpose so the output is written as whole 128-byte
// row segments.  Sequences without tokens get zeros and lse = -inf.
template <int R>
__global__ __launch_bounds__(256) void k_decode_merge_frag(
    int32_t rows, int32_t row_blocks, const int2 *__restrict__ seq_info,
    const uint16_t *__restrict__ part_o, const float *__restrict__ part_lse, float *__restrict__ out,
    float *__restrict__ out_lse, int32_t *__restrict__ adv_lens, int32_t adv, int32_t adv_n) {
  constexpr int CB = R / 32;
  // lengths that the decode read as lens + pending become lens + pending
  // here, after the decode kernel (which read them) has finished
  if (adv_lens && blockIdx.x == 0 && blockIdx.y == 0)
    for (int i = threadIdx.x; i < adv_n; i += blockDim.x) adv_lens[i] += adv;
  __shared__ float tile[4][32][33];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int cb = blockIdx.y * 4 + wave;
  if (cb >= CB) return;
  const int b = blockIdx.x / row_blocks, rb = blockIdx.x % row_blocks;
  const int n = lane & 31, half = lane >> 5;
  const int row = rb * 32 + n;
  const int2 si = seq_info[b];
  const int32_t sb = si.x, ns = si.y;
  const int rows_pad = row_blocks * 32;
  float acc[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) acc[j] = 0.f;
  float mx = -INFINITY, wsum = 0.f;
  auto blk_of = [&](int k) {
    return part_o + (((int64_t)(sb + k) * row_blocks + rb) * CB + cb) * 1024 + lane * 4;
  };
  // slot k's weight w times its bf16 block, added in slot order
  auto add = [&](float w, const u32x2_t (&v)[4]) __attribute__((always_inline)) {
    wsum += w;
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
      acc[jq * 4 + 0] += w * __builtin_bit_cast(float, v[jq][0] << 16);
      acc[jq * 4 + 1] += w * __builtin_bit_cast(float, v[jq][0] & 0xffff0000u);
      acc[jq * 4 + 2] += w * __builtin_bit_cast(float, v[jq][1] << 16);
      acc[jq * 4 + 3] += w * __builtin_bit_cast(float, v[jq][1] & 0xffff0000u);
    }
  };
  // Up to kUp slots: every lse and block is requested at once, one round
  // trip instead of a chain of them.  Same-box traces against the loop
  // alone: the 128-head merge 14.0-14.1 -> 13.3-13.6 us, the 16-head one
  // (8-9 slots) 4.84 -> 4.76 us; kUp = 10 timed the same.  More slots:
  // loops unrolled so that several slots' loads are in flight at once.
  constexpr int kUp = 16;
  if (ns <= kUp) {
    float ls[kUp];
    u32x2_t pv[kUp][4];
#pragma unroll
    for (int k = 0; k < kUp; ++k) {
      if (k < ns) {
        ls[k] = part_lse[(int64_t)(sb + k) * rows_pad + row];
        const uint16_t *blk = blk_of(k);
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) pv[k][jq] = *reinterpret_cast<const u32x2_t *>(blk + jq * 256);
      }
    }
#pragma unroll
    for (int k = 0; k < kUp; ++k)
      if (k < ns) mx = fmaxf(mx, ls[k]);
#pragma unroll
    for (int k = 0; k < kUp; ++k)
      if (k < ns) add(expf(ls[k] - mx), pv[k]);
  } else {
#pragma unroll 4
    for (int k = 0; k < ns; ++k) mx = fmaxf(mx, part_lse[(int64_t)(sb + k) * rows_pad + row]);
#pragma unroll 4
    for (int k = 0; k < ns; ++k) {
      const uint16_t *blk = blk_of(k);
      u32x2_t v[4];
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) v[jq] = *reinterpret_cast<const u32x2_t *>(blk + jq * 256);
      add(expf(part_lse[(int64_t)(sb + k) * rows_pad + row] - mx), v);
    }
  }
  const float inv = ns > 0 ? 1.f / wsum : 0.f;
#pragma unroll
  for (int jq = 0; jq < 4; ++jq)
#pragma unroll
    for (int e = 0; e < 4; ++e) tile[wave][n][8 * jq + 4 * half + e] = acc[jq * 4 + e] * inv;
  if (cb == 0 && half == 0 && out_lse && row < rows)
    out_lse[(int64_t)b * rows + row] = ns > 0 ? mx + logf(wsum) : -INFINITY;
  __builtin_amdgcn_wave_barrier();
  // lane l: rows l / 8 + 8 k, columns 4 (l % 8) .. + 3
  const int c4 = (lane & 7) * 4;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int rl = (lane >> 3) + 8 * k;
    const int orow = rb * 32 + rl;
    if (orow < rows) {
      floatx4_t v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = tile[wave][rl][c4 + e];
      *reinterpret_cast<floatx4_t *>(out + ((int64_t)b * rows + orow) * R + cb * 32 + c4) = v;
    }
  }
}

// ---- narrow decode: one 32-row block (rows <= 32), all four SIMDs ------
// With few query rows the MFMA work per token is small, so a block puts
// four waves on one 32-row block instead of one wave: wave w computes S^T
// over its quarter of the latent dims (KSTEPS / 4 k-steps); the four
// partial S^T are summed through LDS; wave v takes the softmax of
// accumulator elements 4v..4v+3 (tokens 8v + 4 half + 0..3 of each lane's
// row); P^T goes through the P^T staging rows; and the P.V product is split
// by column, wave w owning column blocks w * CB/4 .. (w + 1) * CB/4 - 1.
// Three barriers per tile and no software pipelining: this path is bound
// by HBM by a wide margin, and the kNarrowStages-tile ring keeps
// kNarrowStages - 1 tiles in flight.
constexpr int kNarrowStages = 3;
constexpr int kNarrowRed = 4 * 4 * 64 * 16;  // partial S^T: [wave][quarter][lane] x 16 B

// Partial S^T of one tile over the KQ k-steps at per-lane stage offsets sa;
// dma(kk) runs after MFMA kk (DMA slots spread under the MFMAs).
template <int KQ, class DMAF>
__device__ __forceinline__ void narrow_s_phase(uint32_t st, const uint32_t (&sa)[KQ],
                                               const bf16x8_t (&qf)[KQ], floatx16_t &s,
                                               DMAF &&dma) {
  constexpr int D = KQ < 4 ? KQ : 4;
  bf16x8_t a[D + 1];
  [&]<int... K>(std::integer_sequence<int, K...>) {
    ([&] { if constexpr (K < D) a[K] = ds_b128<0>(st + sa[K]); }(), ...);
    ([&] {
      constexpr int kk = K;
      constexpr int after = (kk + D - 1 < KQ - 1 ? D - 1 : KQ - 1 - kk);
      wait_lgkm<after>();
      arrived(a[kk % (D + 1)]);
      if constexpr (kk == 0)
        s = mfma_s_first(a[0], qf[0]);
      else
        mfma_s_acc(s, a[kk % (D + 1)], qf[kk]);
      dma(kk);
      if constexpr (kk + D < KQ) a[(kk + D) % (D + 1)] = ds_b128<0>(st + sa[kk + D]);
    }(), ...);
  }(std::make_integer_sequence<int, KQ>{});
  mfma_s_drain(s);
}

// Quarter q (elements 4q .. 4q+3) of an S^T accumulator to LDS.
template <int Q>
__device__ __forceinline__ void red_write(uint32_t addr, const floatx16_t &s) {
  const floatx4_t v = __builtin_shufflevector(s, s, 4 * Q, 4 * Q + 1, 4 * Q + 2, 4 * Q + 3);
  asm volatile("ds_write_b128 %0, %1" : : "v"(addr), "v"(v));
}

template <int R, int DR>
constexpr size_t narrow_lds_bytes() {
  return (size_t)kNarrowStages * DecodeShape<R, DR>::STAGE_BYTES + kNarrowRed + 32 * kPRow +
         4 * 32 * 4 + 4 * 4 + kSegCap * sizeof(SegDesc) + 16;
}

template <int R, int DR, typename QT>
__global__ __launch_bounds__(256) void k_decode_narrow(
    const uint64_t *__restrict__ pages, int32_t pt_width, int32_t pt_shift,
    const int32_t *__restrict__ lens, int32_t batch, const QT *__restrict__ q_lat,
    const QT *__restrict__ q_rope, int32_t rows, float scale_log2, int32_t seg_tokens,
    int32_t pending, int2 *__restrict__ seq_info, uint16_t *__restrict__ part_o,
    float *__restrict__ part_lse) {
  using SH = DecodeShape<R, DR>;
  constexpr int NW = 4, NSTAGE = kNarrowStages;
  constexpr int KQ = SH::KSTEPS / NW;  // k-steps of this wave's S^T quarter
  constexpr int NCB = SH::CB / NW;     // P.V column blocks of this wave
  static_assert(SH::KSTEPS % NW == 0 && SH::CB % NW == 0, "narrow split");
  extern __shared__ __attribute__((aligned(16))) char ring_raw[];
  lds_char *ring = (lds_char *)ring_raw;
  const uint32_t ring_u = lds_u32(ring);
  const uint32_t red_u = ring_u + NSTAGE * SH::STAGE_BYTES;
  const uint32_t pbuf_u = red_u + kNarrowRed;
  const uint32_t xrow_u = pbuf_u + 32 * kPRow;  // [wave][32 rows] f32 exchange
  const uint32_t flags_u = xrow_u + 4 * 32 * 4;  // NW words
  lds_char *seg_lds = ring + (flags_u + 4 * NW - ring_u);
  SegDesc *seg_list = (SegDesc *)seg_lds;
  int32_t *seg_meta = (int32_t *)(seg_lds + kSegCap * sizeof(SegDesc));
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int n = lane & 31, half = lane >> 5;
  const bool row_ok = n < rows;
  const int row_c = row_ok ? n : rows - 1;
  const int my_instr = (SH::INSTR - wave + NW - 1) / NW;
  const uint32_t q_sign = scale_log2 < 0.f ? 0x80008000u : 0u;
  const float sl2 = fabsf(scale_log2);

  // S^T operand offsets (within a stage) of this wave's k-steps
  uint32_t sa[KQ];
#pragma unroll
  for (int kk = 0; kk < KQ; ++kk) {
    const int ks = wave * KQ + kk;
    if (ks < SH::KV_STEPS) {
      sa[kk] = SH::kv_row(n) + half * 16 + ks * 32;
    } else {
      const int rk = ks - SH::KV_STEPS;
      sa[kk] = SH::KV_BYTES + n * (DR * 2) + (((2 * rk + half) ^ (n & (SH::RCH - 1))) * 16);
    }
  }
  // V^T operand base of this wave's column blocks
  uint32_t v_off;
  {
    const int g = lane >> 4, sl = lane & 15;
    const int tok_a = (g >= 2 ? 4 : 0) + (sl >> 2);
    const int col_in = (g & 1) * 16 + 4 * (sl & 3);
    v_off = SH::kv_row(tok_a) + (col_in >> 3) * 16 + (col_in & 7) * 2 + wave * NCB * 64;
  }
  // P^T staging: B-operand chunk (k-step ks, half h) of row n at n*kPRow +
  // ks*32 + h*16; this wave's softmax fills positions 4 (wave % 2) .. +3 of
  // chunk (wave / 2, half).
  const uint32_t p_wr = pbuf_u + n * kPRow + (wave >> 1) * 32 + half * 16 + (wave & 1) * 8;
  const uint32_t p_rd = pbuf_u + n * kPRow + half * 16;
  const uint32_t red_wr = red_u + (uint32_t)((wave * 4) * 64 + lane) * 16;
  const uint32_t red_rd = red_u + (uint32_t)(wave * 64 + lane) * 16;  // + w * 4 * 64 * 16
  const uint32_t v_kv = (lane / (SH::ROW_B / 16)) * (SH::W * 2) + (lane % (SH::ROW_B / 16)) * 16;
  const WaveDma wd = wave_dma<SH, NW>(wave);
  const uint32_t v_rope = (lane / SH::RCH) * (SH::W * 2) + SH::ROW_B +
                          ((lane % SH::RCH) ^ ((lane / SH::RCH) & (SH::RCH - 1))) * 16;

  int32_t next_seq = 0;
  do {
  WavePlan wp;
  const int32_t nseg = plan_segments<NW * 64>(lens, pending, batch, next_seq, seg_tokens,
                                              (int32_t *)ring_raw, seg_list, seg_meta, seq_info, wp);
  for (int32_t si = 0; si < nseg; ++si) {
    const SegDesc sg = plan_segment(si, batch, seg_list, wp);
    const int64_t qrow_c = (int64_t)sg.seq * rows + row_c;
    const uint64_t *prow = pages + (int64_t)sg.seq * pt_width;
    const int T = sg.t1 - sg.t0;
    const int ntiles = (T + kTok - 1) / kTok;
    auto stage = [&](int t) { return ring + (t % NSTAGE) * SH::STAGE_BYTES; };
    // prologue DMA before the Q loads (latencies overlap); re-issued on a restart
    auto prologue = [&]() __attribute__((always_inline)) {
#pragma unroll
      for (int p = 0; p < NSTAGE - 1; ++p)
        if (p < ntiles)
          issue_any_tile<SH, NW>(tile_rows<SH>(prow, pt_shift, sg.t0 + p * kTok), sg.t0 + p * kTok,
                                 sg.t1, stage(p), wave, lane, v_kv, v_rope, wd);
    };
    prologue();
    bf16x8_t qf[KQ];
    const uint32_t keep = row_ok ? 0xffffffffu : 0u;
#pragma unroll
    for (int kk = 0; kk < KQ; ++kk) {
      u32x4_t u = __builtin_bit_cast(
          u32x4_t, load_q8<R, DR, QT>(q_lat, q_rope, qrow_c, (wave * KQ + kk) * 16 + half * 8));
#pragma unroll
      for (int i = 0; i < 4; ++i) u[i] = (u[i] ^ q_sign) & keep;
      qf[kk] = __builtin_bit_cast(bf16x8_t, u);
    }
    floatx16_t o[NCB];
    floatx16_t s;
    float m_ref = 0.f, l_run, m_raw;
    float m_init = -INFINITY;
    for (;;) {
#pragma unroll
      for (int i = 0; i < NCB; ++i)
#pragma unroll
        for (int j = 0; j < 16; ++j) o[i][j] = 0.f;
      l_run = 0.f;
      m_raw = -INFINITY;
      if (lane == 0) ds_w32(flags_u + 4 * wave, 0u);
      if (m_init != -INFINITY) prologue();
      for (int it = 0; it < ntiles; ++it) {
        const int nxt = it + NSTAGE - 1;
        // rows of tile nxt, loaded ahead of the wait below, which covers it
        const uint8_t *nxt_rows =
            tile_rows<SH>(prow, pt_shift, sg.t0 + min(nxt, ntiles - 1) * kTok);
        // tile it complete and visible; P.V of tile it-1 done everywhere
        wait_tiles<SH, NW>(min(NSTAGE - 2, ntiles - 1 - it), my_instr);
        wait_lgkm<0>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // DMA of tile nxt: a full tile's slots go under the S^T MFMAs, a
        // partial (clamped) one is issued up front
        const bool full_nxt = nxt < ntiles && (nxt + 1) * kTok <= T;
        if (nxt < ntiles && !full_nxt)
          issue_any_tile<SH, NW>(nxt_rows, sg.t0 + nxt * kTok, sg.t1, stage(nxt), wave, lane, v_kv,
                                 v_rope, wd);
        const FullTileDma fd{nxt_rows, stage(nxt), wave, v_kv, v_rope, wd};
        const uint32_t st = lds_u32(stage(it));
        // partial S^T over this wave's k-steps, to LDS by quarter
        narrow_s_phase<KQ>(st, sa, qf, s, [&](int kk) __attribute__((always_inline)) {
          constexpr int MI = DmaSlots<SH, NW>::MI;
#pragma unroll
          for (int k = 0; k < MI; ++k)
            if ((k * KQ) / MI == kk && full_nxt) issue_full_one<SH, NW>(fd, k);
        });
        red_write<0>(red_wr, s);
        red_write<1>(red_wr + 1 * 64 * 16, s);
        red_write<2>(red_wr + 2 * 64 * 16, s);
        red_write<3>(red_wr + 3 * 64 * 16, s);
        wait_lgkm<0>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // full scores of accumulator elements 4 wave .. 4 wave + 3
        float sc[4] = {0.f, 0.f, 0.f, 0.f};
        {
          // (read as floats: element-wise bit casts of a vector lane are
          // avoided -- the compiler here returned lane 0 for them)
          floatx4_t r[4];
#pragma unroll
          for (int w = 0; w < 4; ++w)
            asm volatile("ds_read_b128 %0, %1" : "=v"(r[w]) : "v"(red_rd + w * 4 * 64 * 16));
          wait_lgkm<0>();
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            asm volatile("" : "+v"(r[w]));
#pragma unroll
            for (int e = 0; e < 4; ++e) sc[e] += r[w][e];
          }
        }
        const int valid = T - it * kTok;
        const int tok0 = 8 * wave + 4 * half;
        float mx = -INFINITY;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (tok0 + e < valid) mx = fmaxf(mx, sc[e]);
        if (it == 0) {
          // reference: the first tile's row maximum over all 32 tokens
          const float mrow = xor32_max(mx);
          if (half == 0) ds_w32(xrow_u + 4 * (wave * 32 + n), __builtin_bit_cast(uint32_t, mrow));
          wait_lgkm<0>();
          __builtin_amdgcn_s_barrier();
          uint32_t xv[4];
#pragma unroll
          for (int w = 0; w < 4; ++w) xv[w] = ds_r32(xrow_u + 4 * (w * 32 + n));
          wait_lgkm<0>();
          float mf = -INFINITY;
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            arrived32(xv[w]);
            mf = fmaxf(mf, __builtin_bit_cast(float, xv[w]));
          }
          m_ref = m_init == -INFINITY ? mf * sl2 : m_init;
        }
        m_raw = fmaxf(m_raw, mx);
        float p[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          p[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[e], sl2, -m_ref));
          p[e] = tok0 + e < valid ? p[e] : 0.f;
        }
        l_run += (p[0] + p[1]) + (p[2] + p[3]);
        {
          u32x2_t pw;
          pw[0] = pack2_bf16(p[0], p[1]);
          pw[1] = pack2_bf16(p[2], p[3]);
          asm volatile("ds_write_b64 %0, %1" : : "v"(p_wr), "v"(pw));
        }
        wait_lgkm<0>();
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        // P.V of this wave's column blocks
        {
          const bf16x8_t b0 = ds_b128<0>(p_rd), b1 = ds_b128<32>(p_rd);
          const uint32_t vb = st + v_off;
          bf16x8_t va[2 * NCB];
          [&]<int... J>(std::integer_sequence<int, J...>) {
            ((va[J] = ds_tr2<(J / NCB) * SH::HI16 + (J % NCB) * 64, SH::HI8>(vb)), ...);
          }(std::make_integer_sequence<int, 2 * NCB>{});
          wait_lgkm<0>();
          bf16x8_t bb[2] = {b0, b1};
          arrived(bb[0]);
          arrived(bb[1]);
#pragma unroll
          for (int j = 0; j < 2 * NCB; ++j) {
            arrived(va[j]);
            o[j % NCB] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va[j], bb[j / NCB], o[j % NCB], 0, 0, 0);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      // Overflow check: this wave's maximum against the reference.
      const float m_seg = xor32_max(m_raw) * sl2;
      const bool ovf = __ballot(m_seg > m_ref + kRefSlack) != 0;
      if (ovf && lane == 0) ds_w32(flags_u + 4 * wave, 1u);
      wait_lgkm<0>();
      __builtin_amdgcn_s_barrier();
      if (!any_flag<NW>(flags_u)) break;
      // Rare: redo the segment with every row's true maximum.
      {
        const float mrow = xor32_max(m_raw);
        if (half == 0) ds_w32(xrow_u + 4 * (wave * 32 + n), __builtin_bit_cast(uint32_t, mrow));
        wait_lgkm<0>();
        __builtin_amdgcn_s_barrier();
        uint32_t xv[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) xv[w] = ds_r32(xrow_u + 4 * (w * 32 + n));
        wait_lgkm<0>();
        float mf = -INFINITY;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          arrived32(xv[w]);
          mf = fmaxf(mf, __builtin_bit_cast(float, xv[w]));
        }
        m_init = mf * sl2;
      }
      __builtin_amdgcn_s_barrier();  // every wave has read the flags and maxima
    }
    // the final P.V MFMAs complete before their accumulators are read
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    // ---- finalise: row sums over the four waves' tokens
    const int fl = vfresh(lane), fn = fl & 31, fh = fl >> 5;
    const float lpart = xor32_sum(l_run);
    if (fh == 0) ds_w32(xrow_u + 4 * (wave * 32 + fn), __builtin_bit_cast(uint32_t, lpart));
    wait_lgkm<0>();
    __builtin_amdgcn_s_barrier();
    float l_row = 0.f;
    {
      uint32_t xv[4];
#pragma unroll
      for (int w = 0; w < 4; ++w) xv[w] = ds_r32(xrow_u + 4 * (w * 32 + fn));
      wait_lgkm<0>();
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        arrived32(xv[w]);
        l_row += __builtin_bit_cast(float, xv[w]);
      }
    }
    const int slot = sg.slot;
    if (wave == 0 && fh == 0)
      part_lse[(int64_t)slot * 32 + fn] = (m_ref + log2f(l_row)) * 0.69314718055994531f;
    const float inv = 1.f / l_row;
    uint16_t *blk = part_o + ((int64_t)slot * SH::CB) * 1024 + fl * 4;
#pragma unroll
    for (int i = 0; i < NCB; ++i) {
      const int cb = wave * NCB + i;
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        u32x2_t v;
        v[0] = pack2_bf16(o[i][jq * 4] * inv, o[i][jq * 4 + 1] * inv);
        v[1] = pack2_bf16(o[i][jq * 4 + 2] * inv, o[i][jq * 4 + 3] * inv);
        *reinterpret_cast<u32x2_t *>(blk + cb * 1024 + jq * 256) = v;
      }
    }
    // xrow and the stages are rewritten by the next segment only after its
    // first barrier
    wait_lgkm<0>();
    __builtin_amdgcn_s_barrier();
  }
  // the next planning round reuses the stage ring: every wave is done with it
  __builtin_amdgcn_s_waitcnt((0xF) | (0x7 << 4) | (0x0 << 8) | (0x3 << 14));
  __builtin_amdgcn_s_barrier();
  } while (next_seq < batch);
}

template <int R>
qmla_status launch_merge(const DecodeArgs &a, hipStream_t stream) {
  const int row_blocks = (a.rows + 31) / 32;
  dim3 mgrid((unsigned)(a.batch * row_blocks), (R / 32 + 3) / 4);
  k_decode_merge_frag<R><<<mgrid, dim3(256), 0, stream>>>(
      a.rows, row_blocks, a.seq_info, (const uint16_t *)a.part_o, a.part_lse, a.out, a.out_lse,
      a.advance ? a.cache->d_lens : nullptr, a.pending, a.batch);
  QMLA_LAUNCH_CHECK("k_decode_merge_frag");
  return QMLA_OK;
}

template <int R, int DR, int NW, int NSTAGE>
qmla_status launch_shape(const DecodeArgs &a, hipStream_t stream) {
  static_assert(decode_lds_bytes<R, DR, NW, NSTAGE>() <= 160 * 1024, "LDS budget");
  const size_t lds = decode_lds_bytes<R, DR, NW, NSTAGE>();
  const int passes = (a.rows + NW * 32 - 1) / (NW * 32);
  dim3 grid(a.blocks, passes), block(NW * 64);
  const float sl2 = a.scale * 1.4426950408889634f;
  const int32_t seg_tokens = decode_mfma_seg_tokens(a.rows, R, DR);
  const PageTable tab = a.cache->table();
  if (a.q_dtype == QMLA_BF16) {
    auto k = k_decode_mfma<R, DR, NW, NSTAGE, uint16_t>;
    QMLA_TRY(ensure_dynamic_lds((const void *)k, lds));
    k<<<grid, block, lds, stream>>>(tab.pages, tab.width, tab.shift, a.cache->d_lens, a.batch,
                                    (const uint16_t *)a.q_lat, (const uint16_t *)a.q_rope, a.rows,
                                    sl2, seg_tokens, a.pending, a.seq_info, (uint16_t *)a.part_o, a.part_lse);
  } else {
    auto k = k_decode_mfma<R, DR, NW, NSTAGE, float>;
    QMLA_TRY(ensure_dynamic_lds((const void *)k, lds));
    k<<<grid, block, lds, stream>>>(tab.pages, tab.width, tab.shift, a.cache->d_lens, a.batch,
                                    (const float *)a.q_lat, (const float *)a.q_rope, a.rows, sl2,
                                    seg_tokens, a.pending, a.seq_info, (uint16_t *)a.part_o, a.part_lse);
  }
  QMLA_LAUNCH_CHECK("k_decode_mfma");
  return launch_merge<R>(a, stream);
}

template <int R, int DR>
qmla_status launch_narrow(const DecodeArgs &a, hipStream_t stream) {
  const size_t lds = narrow_lds_bytes<R, DR>();
  dim3 grid(a.blocks, 1), block(256);
  const float sl2 = a.scale * 1.4426950408889634f;
  const int32_t seg_tokens = decode_mfma_seg_tokens(a.rows, R, DR);
  const PageTable tab = a.cache->table();
  if (a.q_dtype == QMLA_BF16) {
    auto k = k_decode_narrow<R, DR, uint16_t>;
    QMLA_TRY(ensure_dynamic_lds((const void *)k, lds));
    k<<<grid, block, lds, stream>>>(tab.pages, tab.width, tab.shift, a.cache->d_lens, a.batch,
                                    (const uint16_t *)a.q_lat, (const uint16_t *)a.q_rope, a.rows,
                                    sl2, seg_tokens, a.pending, a.seq_info, (uint16_t *)a.part_o, a.part_lse);
  } else {
    auto k = k_decode_narrow<R, DR, float>;
    QMLA_TRY(ensure_dynamic_lds((const void *)k, lds));
    k<<<grid, block, lds, stream>>>(tab.pages, tab.width, tab.shift, a.cache->d_lens, a.batch,
                                    (const float *)a.q_lat, (const float *)a.q_rope, a.rows, sl2,
                                    seg_tokens, a.pending, a.seq_info, (uint16_t *)a.part_o, a.part_lse);
  }
  QMLA_LAUNCH_CHECK("k_decode_narrow");
  return launch_merge<R>(a, stream);
}

template <int R, int DR>
qmla_status launch_dims(const DecodeArgs &a, hipStream_t stream) {
  if constexpr (R == 512 && DR == 64)
    if (decode_narrow_path(a.rows, R, DR)) return launch_narrow<R, DR>(a, stream);
  if (a.rows <= 32) return launch_shape<R, DR, 1, 3>(a, stream);
  if (a.rows <= 64) return launch_shape<R, DR, 2, 4>(a, stream);
  return launch_shape<R, DR, 4, 4>(a, stream);
}

}  // namespace

bool decode_mfma_supported(int32_t rows, int32_t r, int32_t dr) {
  (void)rows;
  return (r == 512 && dr == 64) || (r == 64 && dr == 16) || (r == 128 && dr == 32);
}

// The narrow path (one 32-row block over all four SIMDs) serves r = 512 /
// dr = 64 with at most 32 query rows; its 3-stage ring allows one block per
// compute unit.
bool decode_narrow_path(int32_t rows, int32_t r, int32_t dr) {
  return rows <= 32 && r == 512 && dr == 64;
}

int decode_mfma_blocks_per_cu(int32_t rows, int32_t r, int32_t dr) {
  if (decode_narrow_path(rows, r, dr)) return 1;
  return rows <= 64 ? 2 : 1;
}

// Virtual tokens charged per sequence start in the split plan: the fixed
// cost of a segment (Q load, prologue latency, l exchange, partial store)
// over the loop's cost per token -- ~32K clocks over ~100 clocks per token
// at 128 rows, ~8K clocks over ~35 for the narrow path.
int32_t decode_mfma_seg_tokens(int32_t rows, int32_t r, int32_t dr) {
  if (decode_narrow_path(rows, r, dr)) return 256;
  return rows > 64 ? 320 : 64;
}

qmla_status launch_decode_mfma(const DecodeArgs &a, hipStream_t stream) {
  QMLA_REQUIRE(a.rows <= 65535 * 128, QMLA_ERR_SHAPE, "too many query rows");
  if (a.r == 512 && a.dr == 64) return launch_dims<512, 64>(a, stream);
  if (a.r == 64 && a.dr == 16) return launch_dims<64, 16>(a, stream);
  if (a.r == 128 && a.dr == 32) return launch_dims<128, 32>(a, stream);
  return fail(QMLA_ERR_UNSUPPORTED, "bf16 decode for kv_lora_rank %d, rope %d", a.r, a.dr);
}

}  // namespace qmla
