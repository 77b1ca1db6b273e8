// prefill_mfma.hip -- bf16 MFMA flash prefill (causal, chunk offset).
//
// Replaces the tiled candle matmuls of fused_prefill_attn
// (src/attention_kernel.rs:64-107) for bf16 inputs with f32 accumulation.
// A block holds 8 waves x 32 query rows of one (b, h) and streams 32-key
// tiles of [k_nope | k_rope] and v through an LDS ring.  Per wave and tile:
//
//   S^T[key][q] = sum_d K[key][d] Q[q][d]      KSTEPS MFMAs (Q in VGPRs)
//   P^T = exp2(S^T * scale*log2(e) - m)         softmax, f32
//   O^T[c][q] += sum_key V^T[c][key] P^T[key][q]
//
// The S^T accumulator (lane = query row, 16 keys per lane) is the B operand
// of the P.V product, and V^T comes from the key-major tile through
// ds_read_b64_tr_b16.  Each wave fits in half a SIMD's register file, so
// two waves share a SIMD: waves 0-3 (group 0) and 4-7 (group 1), one of
// each per SIMD.  The block advances in barrier-separated steps; in every
// step one group computes S^T of a tile (MFMA and LDS bound) while the
// other computes the softmax of its previous S^T (VALU) and then the P.V
// of the tile before (MFMA), so one wave's softmax runs under the other
// wave's MFMAs.  Group 1 runs one step behind group 0.
//
// The softmax keeps a lazy fixed reference per row (the first tile's
// maximum; a block in which some probability exceeds kPOverflow redoes its
// tiles with a reference at or above the true maximum), so the O^T
// accumulators are never rescaled inside the loop.  Only the first tile
// takes a maximum: later tiles are checked through the largest 16-key
// partial sum of p, an upper bound of every p in it.  Key tiles above a wave's causal horizon are
// skipped (exact: the reference's -1e18 mask gives exp() == 0); blocks are
// issued heaviest first so the causal triangle balances across compute
// units.

#include <cmath>
#include <type_traits>
#include <utility>

#include "mfma_pipe.hpp"

namespace qmla {

namespace {

using namespace pipe;

__device__ __forceinline__ void ds_w64(uint32_t addr, u32x2_t v) {
  asm volatile("ds_write_b64 %0, %1" : : "v"(addr), "v"(v));
}

constexpr int kPKeys = 32;      // keys per tile
constexpr int kPWaves = 8;      // two groups of four
constexpr int kPDmaWaves = 4;   // group 1 issues every tile's DMA
constexpr int kPRows = kPWaves * 32;
constexpr int kPStages = 4;     // tile ring depth
constexpr int kPAhead = 5;      // S^T operand reads issued ahead of their MFMAs
constexpr int kPvAheadP = 2;    // V^T fragments issued ahead of their MFMAs
constexpr float kPOverflow = 65536.f;  // largest p kept (2^16) before a restart

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
template <int ROWB_>
struct Region {
  static_assert(ROWB_ == 0 || (ROWB_ >= 32 && ROWB_ <= 1024 && (ROWB_ & (ROWB_ - 1)) == 0), "row bytes");
  static constexpr int ROWB = ROWB_;
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
  static constexpr int MI = (INSTR + kPDmaWaves - 1) / kPDmaWaves;  // DMA slots per wave
  // every region boundary falls on a slot boundary: slot k's region is a
  // compile-time fact, the same for every DMA wave
  static constexpr bool EVEN = KN::INSTR % kPDmaWaves == 0 && KR::INSTR % kPDmaWaves == 0 &&
                               VR::INSTR % kPDmaWaves == 0;
  static_assert(DN % 16 == 0 && DR % 16 == 0 && DV % 32 == 0 && DN >= 16 && DV >= 32, "dims");
  static_assert(MI * (kPStages - 1) < 64, "vmcnt range");
  static_assert(kPStages >= 4 && kPStages <= 7, "ring depth");
};

// Uniform parts of one tile's DMA: base pointers of the three source rows
// (key0 of the tile), the LDS stage, and the last valid key (tile-relative).
struct PTileDma {
  const uint8_t *kn, *kr, *v;
  uint32_t stage;
  int last;
};

// Per-lane part of region instruction i: source offset (within the tile)
// of the chunk that lands at this lane's LDS position (swizzle inverted).
template <class RG, bool VSWZ>
__device__ __forceinline__ uint32_t region_src(int i, int lane) {
  const int r = i * RG::RPI + lane / RG::CPR;
  const int p = lane % RG::CPR;
  const int j = VSWZ ? ((RG::vgrp(r, p >> 2) << 2) | (p & 3)) : RG::kpos(r, p);
  return (uint32_t)(r * RG::ROWB + j * 16);
}

// The same offset with its key row clamped to `last` (0..31): rows past
// seq_k read the last valid row.  The chunk stays within its row.
template <int ROWB>
__device__ __forceinline__ uint32_t clamp_row(uint32_t voff, int last) {
  return min(voff, (uint32_t)(last * ROWB) + (voff & (ROWB - 1)));
}

// Per-lane source offset of DMA slot k of this wave (instruction k *
// kPDmaWaves + dw of a tile, dw = wave - 4), unclamped; 0 for a slot the
// wave does not own.
template <class SH>
__device__ __forceinline__ uint32_t pslot_voff(int k, int wave, int lane) {
  const int ins = k * kPDmaWaves + wave;
  constexpr int E1 = SH::KN::INSTR, E2 = SH::KN::INSTR + SH::KR::INSTR;
  if (ins < E1) return region_src<typename SH::KN, false>(ins, lane);
  if constexpr (SH::KR::INSTR > 0)
    if (ins < E2) return region_src<typename SH::KR, false>(ins - E1, lane);
  if (ins < SH::INSTR) return region_src<typename SH::VR, true>(ins - E2, lane);
  return 0;
}

// DMA slot K of this wave for the tile in d (voff from pslot_voff).
// CLAMP: rows past d.last re-load row d.last (the tile's last valid key);
// a full tile (d.last >= 31) needs no clamp.
template <class SH, int K, bool CLAMP>
__device__ __forceinline__ void pissue_one(const PTileDma &d, int wave, uint32_t voff) {
  constexpr int E1 = SH::KN::INSTR, E2 = SH::KN::INSTR + SH::KR::INSTR;
  constexpr int INS0 = K * kPDmaWaves;
  const int ins = INS0 + wave;
  if (!SH::EVEN && ins >= SH::INSTR) return;
  const uint32_t st = fresh(d.stage);
  const int last = CLAMP ? min(d.last, 31) : 31;
  auto cl = [&](auto rb) { return CLAMP ? clamp_row<decltype(rb)::value>(voff, last) : voff; };
  if (SH::EVEN ? INS0 < E1 : ins < E1) {
    dma16(fresh(d.kn), cl(std::integral_constant<int, SH::KN::ROWB>{}),
          st + SH::KN_OFF + ins * 1024);
  } else if (SH::EVEN ? INS0 < E2 : ins < E2) {
    if constexpr (SH::KR::INSTR > 0)
      dma16(fresh(d.kr), cl(std::integral_constant<int, SH::KR::ROWB>{}),
            st + SH::KR_OFF + (ins - E1) * 1024);
  } else {
    dma16(fresh(d.v), cl(std::integral_constant<int, SH::VR::ROWB>{}),
          st + SH::V_OFF + (ins - E2) * 1024);
  }
}

// Every slot of this wave for the tile in d, clamped unless it is full.
template <class SH>
__device__ __forceinline__ void pissue_tile(const PTileDma &d, int wave,
                                            const uint32_t (&voff)[SH::MI]) {
  [&]<int... K>(std::integer_sequence<int, K...>) {
    if (d.last >= 31)
      (pissue_one<SH, K, false>(d, wave, voff[K]), ...);
    else
      (pissue_one<SH, K, true>(d, wave, voff[K]), ...);
  }(std::make_integer_sequence<int, SH::MI>{});
}

// Waits until at most k tiles (0 <= k <= kPStages - 2) of this wave's DMA
// are outstanding; my_instr = the wave's DMA instructions per tile.
template <class SH>
__device__ __forceinline__ void pwait_tiles(int k, int my_instr) {
  constexpr int MAXN = (kPStages - 2) * SH::MI;
  static_assert(MAXN < 64, "vmcnt range");
  const int n = k <= 0 ? 0 : k * my_instr;
  bool done = false;
  [&]<int... N>(std::integer_sequence<int, N...>) {
    (void)((N > 0 && !done && n == N ? (wait_vmcnt<N>(), done = true) : false), ...);
  }(std::make_integer_sequence<int, MAXN + 1>{});
  if (!done) wait_vmcnt<0>();
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

// S^T of one tile for the wave's 32 rows: one chain of KSTEPS MFMAs into a
// VGPR accumulator, operand reads kPAhead steps ahead.  With DMA, the
// wave's DMA slots of the full tile in d are spread over the MFMAs.
template <class SH, bool DMA>
__device__ __forceinline__ void ps_phase(const PLane<SH> &la, uint32_t st,
                                         const bf16x8_t (&qf)[SH::KSTEPS], floatx16_t &s,
                                         const PTileDma &d, int dw,
                                         const uint32_t (&voff)[SH::MI]) {
  constexpr int D = kPAhead < SH::KSTEPS ? kPAhead : SH::KSTEPS;
  bf16x8_t a[D + 1];
  __builtin_amdgcn_s_setprio(2);
  [&]<int... K>(std::integer_sequence<int, K...>) {
    ([&] { if constexpr (K < D) a[K] = ds_b128<0>(st + la.s[K]); }(), ...);
    ([&] {
      constexpr int kk = K;
      constexpr int after = (kk + D - 1 < SH::KSTEPS - 1 ? D - 1 : SH::KSTEPS - 1 - kk);
      wait_lgkm<after>();
      arrived(a[kk % (D + 1)]);
      if constexpr (kk == 0)
        s = mfma_s_first(a[0], qf[0]);
      else
        mfma_s_acc(s, a[kk % (D + 1)], qf[kk]);
      if constexpr (DMA)
        [&]<int... M>(std::integer_sequence<int, M...>) {
          ([&] {
            if constexpr ((M * SH::KSTEPS) / SH::MI == kk) pissue_one<SH, M, false>(d, dw, voff[M]);
          }(), ...);
        }(std::make_integer_sequence<int, SH::MI>{});
      if constexpr (kk + D < SH::KSTEPS) a[(kk + D) % (D + 1)] = ds_b128<0>(st + la.s[kk + D]);
    }(), ...);
  }(std::make_integer_sequence<int, SH::KSTEPS>{});
  __builtin_amdgcn_s_setprio(0);
  mfma_s_drain(s);
}

// V^T fragment j = (k-step ks, column block i): two transposing reads.
template <class SH, int J>
__device__ __forceinline__ bf16x8_t pv_frag(const PLane<SH> &la, uint32_t st) {
  constexpr int ks = J / SH::CB, cb = J % SH::CB;
  return ds_tr2<ks * 16 * (SH::DV * 2), 8 * (SH::DV * 2)>(st + la.v[cb]);
}

// O^T += V^T P^T: 2 x CB MFMAs, V^T fragments streamed kPvAheadP ahead.
// Each MFMA reads its accumulator CB MFMAs after the one that wrote it; P^T
// (VALU-written) is consumed a full step after it was formed.
// mid() runs after the first fragments are requested (their LDS latency
// overlaps it).
template <class SH, class MID>
__device__ __forceinline__ void ppv_phase(const PLane<SH> &la, uint32_t st, const bf16x8_t (&pb)[2],
                                          floatx16_t (&o)[SH::CB], MID &&mid) {
  constexpr int NA = 2 * SH::CB;
  constexpr int DA = kPvAheadP < NA ? kPvAheadP : NA;
  bf16x8_t a[DA + 1];
  [&]<int... J>(std::integer_sequence<int, J...>) {
    ([&] { if constexpr (J < DA) a[J] = pv_frag<SH, J>(la, st); }(), ...);
    mid();
    ([&] {
      constexpr int j = J;
      constexpr int after = 2 * (j + DA - 1 < NA - 1 ? DA - 1 : NA - 1 - j);
      wait_lgkm<after>();
      arrived(a[j % (DA + 1)]);
      constexpr int ks = j / SH::CB, cb = j % SH::CB;
      // in place (asm): the accumulators never move between registers
      mfma_s_acc(o[cb], a[j % (DA + 1)], pb[ks]);
      if constexpr (j + DA < NA) a[(j + DA) % (DA + 1)] = pv_frag<SH, j + DA>(la, st);
    }(), ...);
  }(std::make_integer_sequence<int, NA>{});
}

// S^T accumulator element j of lane (n, half) holds key 8 (j / 4) + 4 half
// + j % 4 of the tile for query row n.

// Raw maximum of this lane's 16 scores; with MASK, keys at or past seq_k or
// (causal) after the row's absolute position are out.
template <bool MASK>
__device__ __forceinline__ float ptile_max(const floatx16_t &s, int key0, int half, int vis_lim) {
  // keys of this lane: key0 + 4 half + 8 (j / 4) + j % 4; rel < 0 <=> visible
  const int rel = MASK ? vfresh(key0 + 4 * half - vis_lim) : 0;
  float x[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) x[j] = (!MASK || rel + 8 * (j >> 2) + (j & 3) < 0) ? s[j] : -INFINITY;
  const float a = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
  const float b = fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7]));
  const float c = fmaxf(fmaxf(x[8], x[9]), fmaxf(x[10], x[11]));
  const float e = fmaxf(fmaxf(x[12], x[13]), fmaxf(x[14], x[15]));
  return fmaxf(fmaxf(a, b), fmaxf(c, e));
}

// p = exp2(s * sl2 - m) as the two bf16 B-operand fragments; adds the
// lane's 16-key sum to l and folds it into the running maximum tmax.
template <bool MASK>
__device__ __forceinline__ void ptile_p(const floatx16_t &s, float sl2, float m, int key0,
                                        int half, int vis_lim, float &l, float &tmax,
                                        bf16x8_t (&pb)[2]) {
  const int rel = MASK ? vfresh(key0 + 4 * half - vis_lim) : 0;
  float p[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    p[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j], sl2, -m));
    if (MASK) p[j] = rel + 8 * (j >> 2) + (j & 3) < 0 ? p[j] : 0.f;
  }
  float q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = p[2 * i] + p[2 * i + 1];
  const float t = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
  l += t;
  tmax = fmaxf(tmax, t);
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
//
// Schedule.  Step k (0 <= k < 2 * ntb + 3, a barrier before each) is local
// step k - g of a group-g wave.  Local step 2j: S^T of tile j.  Local step
// 2j + 1: softmax of tile j, then P.V of tile j - 1.  Tile j is therefore
// read last in global step 2j + 4 (group 1's P.V, its local step 2j + 3),
// and the DMA of tile j + kPStages into its stage is issued in step 2j + 5
// (odd steps k >= 3 issue tile (k - 5) / 2 + kPStages; the prologue issues
// tiles 0 .. kPStages - 2): the barrier before step 2j + 5 is what keeps
// that DMA behind the last read, so every step needs its barrier.  Before
// step 2m every wave waits for its share of tile m, so tile m is complete
// in LDS when group 0 reads it.
template <int DN, int DR, int DV>
__global__ __launch_bounds__(kPWaves * 64) void k_prefill_mfma(
    const uint16_t *__restrict__ q_nope, const uint16_t *__restrict__ q_rope,
    const uint16_t *__restrict__ k, const uint16_t *__restrict__ k_rope,
    const uint16_t *__restrict__ v, qmla_prefill_dims d, float scale_log2, int causal,
    uint16_t *__restrict__ out, int n_qtiles, int pair_tiles, int out_records) {
  using SH = PrefillShape<DN, DR, DV>;
  extern __shared__ __attribute__((aligned(16))) char pring_raw[];
  lds_char *ring = (lds_char *)pring_raw;
  const uint32_t ring_u = lds_u32(ring);
  const uint32_t ovf_flags = ring_u + kPStages * SH::STAGE_BYTES;  // kPWaves words
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = wave >> 2;
  const int lane = tid & 63;
  const int n = lane & 31, half = lane >> 5;
  // A negative scale is applied as |scale| with the sign folded into q
  // (exact in bf16), so the raw score maximum is also the scaled one.
  const uint32_t q_sign = scale_log2 < 0.f ? 0x80008000u : 0u;
  const float sl2 = fabsf(scale_log2);

  // Block order.  Query tiles are ranked by work (rank 0 = heaviest when
  // causal).  Unpaired: rank by rank.  Paired (pair_tiles, when K/V exceed
  // the Infinity Cache): rank pair by rank pair, and within a pair the two
  // tiles of one (b, h) get block indices 8 apart -- blocks are dealt to the
  // 8 XCDs round-robin, so both land on the same XCD at nearly the same
  // time and the second one's K/V reads hit that XCD's L2.
  const int BH = d.batch * d.heads;
  const int L = blockIdx.x;
  int rank, bh;
  if (!pair_tiles) {
    rank = L / BH;
    bh = L % BH;
  } else if ((BH & 7) == 0 && L < 2 * BH * (n_qtiles >> 1)) {
    const int pr = L / (2 * BH), rem = L - pr * 2 * BH;
    const int x = rem & 7, r = rem >> 3;
    rank = 2 * pr + (r & 1);
    bh = (r >> 1) * 8 + x;
  } else if ((BH & 7) == 0) {
    rank = n_qtiles - 1;  // odd tile count: the last rank alone
    bh = L - 2 * BH * (n_qtiles >> 1);
  } else {
    rank = L / BH;
    bh = L % BH;
  }
  const int qt = causal ? n_qtiles - 1 - rank : rank;
  const int b = bh / d.heads, h = bh - b * d.heads;
  const int q0 = qt * kPRows;
  // The two waves sharing a SIMD (w, w + 4) own 32-row blocks r and 7 - r:
  // on the causal diagonal every SIMD then keeps one busy wave to the end.
  const int row_first = q0 + 32 * (grp == 0 ? (wave & 3) : 7 - (wave & 3));

  const int64_t bhq = (int64_t)bh * d.seq_q;
  const int64_t bhk = (int64_t)bh * d.seq_k;
  const int64_t bkr = ((int64_t)b * d.k_rope_heads + (d.k_rope_heads == 1 ? 0 : h)) * d.seq_k;
  const uint8_t *kb = reinterpret_cast<const uint8_t *>(k + bhk * DN);
  const uint8_t *krb = reinterpret_cast<const uint8_t *>(k_rope + bkr * DR);
  const uint8_t *vb = reinterpret_cast<const uint8_t *>(v + bhk * DV);

  // key horizon (exclusive) of the block and of this wave
  int kend_blk = d.seq_k, kend_w = d.seq_k;
  if (causal) {
    kend_blk = min(d.seq_k, d.q_offset + min(q0 + kPRows, d.seq_q));
    kend_w = min(d.seq_k, d.q_offset + min(row_first + 32, d.seq_q));
  }
  if (row_first >= d.seq_q) kend_w = 0;  // no query row in this wave
  const int ntb = (kend_blk + kPKeys - 1) / kPKeys;  // tiles of the block
  const int ntw = (kend_w + kPKeys - 1) / kPKeys;    // tiles of this wave
  // group 1's waves issue the DMA (slot k of wave dw: instruction k * 4 + dw)
  const int dw = wave & 3;
  const int my_instr = grp == 1 ? (SH::INSTR - dw + kPDmaWaves - 1) / kPDmaWaves : 0;
  const PLane<SH> la = plane_offsets<SH>(lane);
  uint32_t voff[SH::MI];
#pragma unroll
  for (int i = 0; i < SH::MI; ++i) voff[i] = pslot_voff<SH>(i, dw, lane);
  // a tile needs the mask if one of its keys is invisible to some row of
  // the wave: past seq_k, or (causal) after the wave's first row
  const int mask_from = causal ? min(d.seq_k, d.q_offset + row_first + 1) : d.seq_k;
  const int vis_lim = causal ? min(d.seq_k, d.q_offset + row_first + n + 1) : d.seq_k;
  auto tile_dma = [&](int t) {
    const int key0 = t * kPKeys;
    return PTileDma{kb + (int64_t)key0 * (DN * 2), krb + (int64_t)key0 * (DR * 2),
                    vb + (int64_t)key0 * (DV * 2), ring_u + (t % kPStages) * SH::STAGE_BYTES,
                    d.seq_k - 1 - key0};
  };
  auto stage_u = [&](int t) { return ring_u + (uint32_t)((t % kPStages) * SH::STAGE_BYTES); };

  // Q fragments (B operand of S^T) of the wave's 32 rows.
  bf16x8_t qf[SH::KSTEPS];
  {
    const int row = row_first + n;
    const bool ok = row < d.seq_q;
    const int64_t qrow = bhq + (ok ? row : d.seq_q - 1);
    const uint32_t keep = ok ? 0xffffffffu : 0u;
#pragma unroll
    for (int kk = 0; kk < SH::KSTEPS; ++kk) {
      u32x4_t u = __builtin_bit_cast(u32x4_t, load_q_frag<SH>(q_nope, q_rope, qrow, kk * 16 + half * 8));
#pragma unroll
      for (int i = 0; i < 4; ++i) u[i] = (u[i] ^ q_sign) & keep;
      qf[kk] = __builtin_bit_cast(bf16x8_t, u);
    }
  }

  floatx16_t o[SH::CB];
  floatx16_t s;
  bf16x8_t pb[2], pn[2];
  float m_ref = -INFINITY, l_run, t_max;
  float m_init = -INFINITY;
  const int nsteps = 2 * ntb + 3;
  for (;;) {
#pragma unroll
    for (int cb = 0; cb < SH::CB; ++cb)
#pragma unroll
      for (int j = 0; j < 16; ++j) o[cb][j] = 0.f;
    l_run = 0.f;
    t_max = 0.f;
    if (lane == 0) ds_w32(ovf_flags + 4 * wave, 0u);

#pragma unroll
    for (int p = 0; p < kPStages - 1; ++p)
      if (grp == 1 && p < ntb) pissue_tile<SH>(tile_dma(p), dw, voff);

    // softmax of tile j (its S^T is in s) into pout; tile 0 sets the
    // reference (key 0 is visible to every row, so its maximum is finite)
    auto sm = [&](auto mask_c, int j, bf16x8_t (&pout)[2]) __attribute__((always_inline)) {
      constexpr bool MASK = decltype(mask_c)::value;
      const int key0 = j * kPKeys;
      ptile_p<MASK>(s, sl2, m_ref, key0, half, vis_lim, l_run, t_max, pout);
    };
    auto sm0 = [&](auto mask_c) __attribute__((always_inline)) {
      constexpr bool MASK = decltype(mask_c)::value;
      const float mr = ptile_max<MASK>(s, 0, half, vis_lim);
      m_ref = m_init == -INFINITY ? xor32_max(mr) * sl2 : m_init;
      ptile_p<MASK>(s, sl2, m_ref, 0, half, vis_lim, l_run, t_max, pb);
    };

    // Step k: vmcnt wait (even k), barrier.  At odd steps k >= 3, group 1
    // issues tile (k - 5) / 2 + kPStages, spread over its S^T MFMAs when it
    // has an S^T in that step.
    int k = 0;
    auto head = [&]() __attribute__((always_inline)) {
      if ((k & 1) == 0) {
        // tile k/2 complete (this wave's share); later tiles may stay in flight
        const int m = k >> 1;
        const int last = min(ntb - 1, max(kPStages - 2, m + kPStages - 3));
        // steady state: kPStages - 3 whole tiles of MI slots (group 0 has none)
        if (SH::EVEN && last - m == kPStages - 3)
          wait_vmcnt<(kPStages - 3) * SH::MI>();
        else
          pwait_tiles<SH>(last - m, my_instr);
      }
      wait_lgkm<0>();
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      ++k;
    };
    // tile DMA'd in the step just begun (k - 1), or ntb if none
    auto dma_tile = [&]() {
      return (grp == 1 && k >= 4 && (k & 1) == 0) ? (k - 6) / 2 + kPStages : ntb;
    };
    auto dma_only = [&]() __attribute__((always_inline)) {
      const int t = dma_tile();
      if (t < ntb) pissue_tile<SH>(tile_dma(t), dw, voff);
    };
    // The wave's local steps: S^T of tile j, then softmax of tile j with the
    // P.V of tile j - 1.  Tiles before jm need no mask.
    const int jm = min(ntw, mask_from / kPKeys);  // first tile needing the mask
    if (grp == 1) head();  // group 1 starts one step late
    if (ntw > 0) {
      head();
      ps_phase<SH, false>(la, stage_u(0), qf, s, PTileDma{}, dw, voff);
      head();
      if (jm == 0)
        sm0(std::true_type{});
      else
        sm0(std::false_type{});
      __builtin_amdgcn_sched_barrier(0);
      // Local steps 2j, 2j + 1: S^T of tile j (with this step's DMA, if
      // any), then the P.V of tile j - 1 (P^T in pin) with the softmax of
      // tile j into pout.  A partial tile's DMA goes out before the S^T.
      auto body = [&](auto mask_c, int j, bf16x8_t (&pin)[2], bf16x8_t (&pout)[2])
                      __attribute__((always_inline)) {
        head();
        const int t = dma_tile();
        const PTileDma td = tile_dma(t);
        if (t < ntb && td.last >= 31) {
          ps_phase<SH, true>(la, stage_u(j), qf, s, td, dw, voff);
        } else {
          if (t < ntb) pissue_tile<SH>(td, dw, voff);
          ps_phase<SH, false>(la, stage_u(j), qf, s, td, dw, voff);
        }
        __builtin_amdgcn_sched_barrier(0);
        head();
        ppv_phase<SH>(la, stage_u(j - 1), pin, o,
                      [&]() __attribute__((always_inline)) { sm(mask_c, j, pout); });
        __builtin_amdgcn_sched_barrier(0);
      };
      // two tiles per trip, so the P^T fragments alternate between pb and
      // pn without copies; after an odd tile count the last ones move to pb
      auto run = [&](auto mask_c, int j, int jend) __attribute__((always_inline)) {
        for (; j + 1 < jend; j += 2) {
          body(mask_c, j, pb, pn);
          body(mask_c, j + 1, pn, pb);
        }
        if (j < jend) {
          body(mask_c, j, pb, pn);
          pb[0] = pn[0];
          pb[1] = pn[1];
        }
      };
      run(std::false_type{}, 1, jm);
      run(std::true_type{}, max(jm, 1), ntw);
      head();  // no S^T of tile ntw
      dma_only();
      head();
      ppv_phase<SH>(la, stage_u(ntw - 1), pb, o, [] {});
      __builtin_amdgcn_sched_barrier(0);
    }
    while (k < nsteps) {
      head();
      dma_only();
    }

    // Overflow check: some p of the row above kPOverflow.
    const float t_row = xor32_max(t_max);
    const bool ovf = ntw > 0 && t_row > kPOverflow;
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
    // Rare: redo the block's tiles with a reference at or above every
    // row's true maximum (each p <= its 16-key sum <= t_row), so no p of
    // the second pass exceeds 1.
    __builtin_amdgcn_s_barrier();  // all waves have read the flags
    m_init = m_ref + log2f(t_row);
  }
  // the final P.V MFMAs complete before their accumulators are read
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");

  // finalise: O / l in bf16.  Lane (n, half) holds 4 consecutive columns
  // of row n per (cb, jq); stored as they are, each store instruction
  // would write 16 bytes into each of 32 rows.  When it fits, the wave's
  // 32 rows go through its own region of the idle ring instead (every wave
  // is past its last ring read: the overflow check's barrier), and each
  // store instruction writes whole consecutive rows, 1 KB.
  const float l = xor32_sum(l_run);
  const float inv = l > 0.f ? 1.f / l : 0.f;
  constexpr int STR = DV * 2 + 16;  // staged row stride in bytes (padded: fewer bank conflicts)
  if constexpr (kPWaves * 32 * STR <= kPStages * SH::STAGE_BYTES) {
    const uint32_t wb = ring_u + (uint32_t)(wave * 32 * STR);
#pragma unroll
    for (int cb = 0; cb < SH::CB; ++cb)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        u32x2_t w;
        w[0] = pack2_bf16(o[cb][jq * 4 + 0] * inv, o[cb][jq * 4 + 1] * inv);
        w[1] = pack2_bf16(o[cb][jq * 4 + 2] * inv, o[cb][jq * 4 + 3] * inv);
        ds_w64(wb + n * STR + (cb * 32 + 8 * jq + 4 * half) * 2, w);
      }
    constexpr int CPR = DV / 8;        // 16-byte chunks per row
    constexpr int RPI = 64 / CPR;      // rows per store instruction
    constexpr int NI = 32 / RPI;       // store instructions per wave
    static_assert(DV % 16 == 0 && DV / 16 == NI, "one record per store instruction");
    bf16x8_t rows[NI];
    wait_lgkm<0>();
    if (out_records) {
      // The context as o_proj's activation records (hi halves only): the
      // rows [b s][H dv], record (token block, k-step), lane l holding row
      // l % 32 at k = 16 ks + 8 (l / 32) .. + 7.  seq_q % 32 == 0, so the
      // wave's 32 rows are one token block (host check).
      if (row_first < d.seq_q) {
#pragma unroll
        for (int i = 0; i < NI; ++i)
          rows[i] = ds_b128<0>(wb + (lane & 31) * STR + (2 * i + (lane >> 5)) * 16);
        wait_lgkm<0>();
        const int64_t tb = ((int64_t)b * d.seq_q + row_first) / 32;
        uint8_t *rec = reinterpret_cast<uint8_t *>(out) +
                       ((tb * d.heads + h) * NI) * 1024 + lane * 16;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          arrived(rows[i]);
          *reinterpret_cast<bf16x8_t *>(rec + i * 1024) = rows[i];
        }
      }
      return;
    }
    const int lr = lane / CPR, lc = lane % CPR;
#pragma unroll
    for (int i = 0; i < NI; ++i) rows[i] = ds_b128<0>(wb + (i * RPI + lr) * STR + lc * 16);
    wait_lgkm<0>();
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      arrived(rows[i]);
      const int r = row_first + i * RPI + lr;
      if (r < d.seq_q) *reinterpret_cast<bf16x8_t *>(out + (bhq + r) * DV + lc * 8) = rows[i];
    }
  } else {
    if (out_records) return;  // the host allows records only with the staged store
    const int row = row_first + n;
    if (row < d.seq_q) {
      uint16_t *dst = out + (bhq + row) * DV;
#pragma unroll
      for (int cb = 0; cb < SH::CB; ++cb)
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
          u32x2_t w;
          w[0] = pack2_bf16(o[cb][jq * 4 + 0] * inv, o[cb][jq * 4 + 1] * inv);
          w[1] = pack2_bf16(o[cb][jq * 4 + 2] * inv, o[cb][jq * 4 + 3] * inv);
          *reinterpret_cast<u32x2_t *>(dst + cb * 32 + 8 * jq + 4 * half) = w;
        }
    }
  }
}

template <int DN, int DR, int DV>
qmla_status launch_prefill_shape(const qmla_prefill_dims &d, const uint16_t *q_nope,
                                 const uint16_t *q_rope, const uint16_t *k,
                                 const uint16_t *k_rope, const uint16_t *v, float scale,
                                 int causal, uint16_t *out, hipStream_t stream,
                                 int out_records) {
  using SH = PrefillShape<DN, DR, DV>;
  constexpr bool kStaged = kPWaves * 32 * (DV * 2 + 16) <= kPStages * SH::STAGE_BYTES;
  QMLA_REQUIRE(!out_records || (kStaged && DV % 16 == 0 && DV / 16 == 32 / (64 / (DV / 8)) &&
                                d.seq_q % 32 == 0),
               QMLA_ERR_UNSUPPORTED, "context records need dv 128 and seq_q %% 32 == 0");
  const int n_qtiles = (d.seq_q + kPRows - 1) / kPRows;
  const int64_t nblocks = (int64_t)d.batch * d.heads * n_qtiles;
  QMLA_REQUIRE(nblocks <= 0x7fffffff, QMLA_ERR_SHAPE, "too many query tiles");
  const size_t lds = (size_t)kPStages * SH::STAGE_BYTES + kPWaves * 4;
  static_assert((size_t)kPStages * SH::STAGE_BYTES + kPWaves * 4 <= 160 * 1024, "LDS");
  // Pair the query tiles of each (b, h) on one XCD only when the K/V
  // stream does not fit the 256 MB Infinity Cache (otherwise re-reads hit
  // it anyway and the plain heaviest-first order balances better).
  const int64_t kv_bytes = (int64_t)d.batch * d.heads * d.seq_k * (DN + DV) * 2 +
                           (int64_t)d.batch * d.k_rope_heads * d.seq_k * DR * 2;
  const int pair_tiles = n_qtiles > 1 && kv_bytes > ((int64_t)256 << 20) ? 1 : 0;
  auto kern = k_prefill_mfma<DN, DR, DV>;
  QMLA_TRY(ensure_dynamic_lds((const void *)kern, lds));
  kern<<<dim3((unsigned)nblocks), dim3(kPWaves * 64), lds, stream>>>(
      q_nope, q_rope, k, k_rope, v, d, scale * 1.4426950408889634f, causal, out, n_qtiles,
      pair_tiles, out_records);
  QMLA_LAUNCH_CHECK("k_prefill_mfma");
  return QMLA_OK;
}

}  // namespace

bool prefill_bf16_supported(int dn, int dr, int dv) {
  return (dn == 128 && dr == 64 && dv == 128) || (dn == 32 && dr == 16 && dv == 32) ||
         (dn == 16 && dr == 16 && dv == 32) || (dn == 32 && dr == 0 && dv == 32) ||
         (dn == 64 && dr == 64 && dv == 64);
}

bool prefill_bf16_records_supported(int dn, int dr, int dv) {
  auto staged = [](auto shape) {
    using SH = decltype(shape);
    return kPWaves * 32 * (SH::DV * 2 + 16) <= kPStages * SH::STAGE_BYTES;
  };
  if (dn == 128 && dr == 64 && dv == 128) return staged(PrefillShape<128, 64, 128>{});
  if (dn == 32 && dr == 16 && dv == 32) return staged(PrefillShape<32, 16, 32>{});
  if (dn == 16 && dr == 16 && dv == 32) return staged(PrefillShape<16, 16, 32>{});
  if (dn == 32 && dr == 0 && dv == 32) return staged(PrefillShape<32, 0, 32>{});
  if (dn == 64 && dr == 64 && dv == 64) return staged(PrefillShape<64, 64, 64>{});
  return false;
}

qmla_status launch_prefill_bf16(const qmla_prefill_dims &d, const uint16_t *q_nope,
                                const uint16_t *q_rope, const uint16_t *k,
                                const uint16_t *k_rope, const uint16_t *v, float scale,
                                int causal, uint16_t *out, hipStream_t stream, int out_records) {
  const int dn = d.qk_nope, dr = d.qk_rope, dv = d.v_dim;
  if (dn == 128 && dr == 64 && dv == 128)
    return launch_prefill_shape<128, 64, 128>(d, q_nope, q_rope, k, k_rope, v, scale, causal, out,
                                              stream, out_records);
  if (dn == 32 && dr == 16 && dv == 32)
    return launch_prefill_shape<32, 16, 32>(d, q_nope, q_rope, k, k_rope, v, scale, causal, out,
                                            stream, out_records);
  if (dn == 16 && dr == 16 && dv == 32)
    return launch_prefill_shape<16, 16, 32>(d, q_nope, q_rope, k, k_rope, v, scale, causal, out,
                                            stream, out_records);
  if (dn == 32 && dr == 0 && dv == 32)
    return launch_prefill_shape<32, 0, 32>(d, q_nope, q_rope, k, k_rope, v, scale, causal, out,
                                           stream, out_records);
  if (dn == 64 && dr == 64 && dv == 64)
    return launch_prefill_shape<64, 64, 64>(d, q_nope, q_rope, k, k_rope, v, scale, causal, out,
                                            stream, out_records);
  return fail(QMLA_ERR_UNSUPPORTED,
              "bf16 prefill for (qk_nope, qk_rope, v_dim) = (%d, %d, %d); supported: "
              "(128,64,128) (64,64,64) (32,16,32) (16,16,32) (32,0,32)",
              dn, dr, dv);
}

}  // namespace qmla
