// split_gemm.hip -- the projections of an MLA layer call over many token
// rows (MlaAttention::forward_prefill, src/model.rs:197-249: q_proj with
// kv_a_proj_with_mqa, kv_b_proj inside compute_kv, o_proj) as f32-exact
// GEMMs on bf16 MFMA, with the layer's layout work fused into the epilogue.
//
// y[m][n] = sum_k x[m][k] W[n][k] + b[n] in the split form of
// skinny_gemm.hip: every operand is stored as bf16 halves, hi = bf16(v) and
// lo = bf16(v - hi), and every 32 x 32 x 16 step is three
// v_mfma_f32_32x32x16_bf16 with f32 accumulation:
//   x w = x_hi w_hi + x_lo w_hi + x_hi w_lo   (x_lo w_lo < 2^-16 |x w|)
// When x is bf16 (the bf16 attention's context) x_lo is zero: the x records
// carry no lo half and the second product is skipped.  With bf16 operands
// (SplitGemmArgs::bf16ops) both lo halves are left out: x_hi w_hi alone,
// one MFMA per step, hi-only records of both operands in LDS.
//
// Operands as fragment-major records.  A record is one MFMA operand of a
// 32-row block and a 16-wide k-step, exactly as the wave's lanes read it:
// lane l's 16 bytes are the 8 bf16 values of row 32 b + l % 32 at k = 16 ks
// + 8 (l / 32) .. + 7, first the hi halves of the 64 lanes (1 KB), then the
// lo halves (1 KB).  The weights are packed once when the layer is created
// (skinny_pack); the activations are packed per call by k_pack_rows (a
// pass that reads x once) or written as records by the kernel that
// produces them (the prefill's latent rows kernel for kv_b_proj, the bf16
// attention's epilogue for o_proj), so that the GEMM moves both operands
// with direct-to-LDS DMA of contiguous 1 KB runs and holds nothing in
// flight in registers.
//
// Block: 8 waves (two per SIMD; SgCfg::NWV) on a BN x BM output tile; wave (wn, wm)
// owns NBW 32-output blocks x MBW 32-row blocks (BN = 32 NBW WN, BM = 32
// MBW WM).  K goes in chunks of KSC k-steps through an NST-deep LDS ring:
// the DMA of chunk c + NST - 1 is issued while chunk c is multiplied,
// spread over its MFMAs, and one barrier per chunk publishes the next
// stage and frees the oldest.  Blocks are dealt to XCDs in groups of tiles
// that share weights and activations (see the tile order below).  Many
// rows run 256 x 256 tiles (each wave 128 outputs x 64 rows, one k-step per
// chunk, three stages: 96 KB of LDS); fewer rows 64 x 128 tiles.
//
// Few rows: K is split over up to 8 blocks per tile, whose raw partial sums
// a second launch (k_sg_reduce) adds in slice order before the epilogue.
//
// Epilogues (lane l of a 32 x 32 accumulator holds row m = l % 32 and
// outputs n = 8 (j / 4) + 4 (l / 32) + j % 4, j < 16: four runs of 4
// consecutive outputs), staged through the idle LDS ring so that rows
// leave as contiguous segments:
//   FINAL  y[m ldy + n] (+ bias), f32
//   QKV    [q_proj | kv_a_proj_with_mqa]: q_nope and the roped q_rope in
//          the attention's [b, H, s, d] layout (positions lens[b] + s,
//          src/model.rs:199-203), bf16 or f32; the raw kv_a rows f32
//   KVB    kv_b_proj: k [b, H, s, dn] and v [b, H, s, dv] (compute_kv's
//          reshape and transpose, src/model.rs:181-188, :213-215)
#include <cmath>
#include <type_traits>
#include <utility>

#include "mfma_pipe.hpp"

namespace qmla {

namespace {

constexpr int kSgGn = 4, kSgGm = 8;  // tiles of an XCD group (n x m)
constexpr int kFrag = 2048;          // one record: hi 1 KB, lo 1 KB

// Barrier after this wave's LDS traffic has completed, without a memory
// fence (the DMA in flight stays in flight).
__device__ __forceinline__ void sg_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
}

template <typename T>
__device__ __forceinline__ void sg_put4(T *p, const float (&v)[4]);

template <>
__device__ __forceinline__ void sg_put4<float>(float *p, const float (&v)[4]) {
  *reinterpret_cast<floatx4_t *>(p) = floatx4_t{v[0], v[1], v[2], v[3]};
}

template <>
__device__ __forceinline__ void sg_put4<uint16_t>(uint16_t *p, const float (&v)[4]) {
  u32x2_t w;
  w[0] = pack_bf16x2(v[0], v[1]);
  w[1] = pack_bf16x2(v[2], v[3]);
  *reinterpret_cast<u32x2_t *>(p) = w;
}

// ---- activation records.  Record (mb, ks) of x: lane l holds x[32 mb + l %
// 32][16 ks + 8 (l / 32) .. + 7]; rows past M are zero.  One thread per
// lane of a record, 4 records per 256-thread block.  XM: kSgXRow f32 rows
// x[m ldx + k]; kSgXHeads* the attention context [b, H, s, dv] read as the
// row [b s][H dv] (k = h dv + d), bf16 or f32.  LO: the records carry lo
// halves (not for bf16 x, nor for bf16 operands).
constexpr int kSgXRow = 0, kSgXHeadsBf16 = 1, kSgXHeadsF32 = 2;

template <int XM, bool LO>
__global__ __launch_bounds__(256) void k_pack_rows(SplitGemmArgs a, uint8_t *__restrict__ rec) {
  static_assert(!(LO && XM == kSgXHeadsBf16), "bf16 x has no lo halves");
  constexpr int RB = LO ? 2048 : 1024;  // bytes per record
  const int KS = a.K / 16;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);  // < 2^31 (host check)
  const int nrec = (a.M + 31) / 32 * KS;
  if (r >= nrec) return;
  const int lane = threadIdx.x & 63;
  const int mb = r / KS, ks = r - mb * KS;
  const int m = mb * 32 + (lane & 31), k = ks * 16 + 8 * (lane >> 5);
  uint8_t *dst = rec + (int64_t)r * RB + lane * 16;
  if (m >= a.M) {
    *reinterpret_cast<u32x4_t *>(dst) = u32x4_t{0, 0, 0, 0};
    if constexpr (LO) *reinterpret_cast<u32x4_t *>(dst + 1024) = u32x4_t{0, 0, 0, 0};
    return;
  }
  if constexpr (XM == kSgXHeadsBf16) {
    const int b = m / a.seq, s = m - b * a.seq, hd = k / a.dv;
    const uint16_t *src = reinterpret_cast<const uint16_t *>(a.x) +
                          (((int64_t)b * a.heads + hd) * a.seq + s) * a.dv + (k - hd * a.dv);
    *reinterpret_cast<u32x4_t *>(dst) = *reinterpret_cast<const u32x4_t *>(src);
  } else {
    const float *src;
    if constexpr (XM == kSgXRow) {
      src = reinterpret_cast<const float *>(a.x) + (int64_t)m * a.ldx + k;
    } else {
      const int b = m / a.seq, s = m - b * a.seq, hd = k / a.dv;
      src = reinterpret_cast<const float *>(a.x) + (((int64_t)b * a.heads + hd) * a.seq + s) * a.dv +
            (k - hd * a.dv);
    }
    const floatx4_t v0 = *reinterpret_cast<const floatx4_t *>(src);
    const floatx4_t v1 = *reinterpret_cast<const floatx4_t *>(src + 4);
    const float v[8] = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
    u32x4_t hi, lo;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t h0 = f32_to_bf16_bits(v[2 * i]), h1 = f32_to_bf16_bits(v[2 * i + 1]);
      hi[i] = h0 | ((uint32_t)h1 << 16);
      const uint16_t l0 = f32_to_bf16_bits(v[2 * i] - bf16_bits_to_f32(h0));
      const uint16_t l1 = f32_to_bf16_bits(v[2 * i + 1] - bf16_bits_to_f32(h1));
      lo[i] = l0 | ((uint32_t)l1 << 16);
    }
    *reinterpret_cast<u32x4_t *>(dst) = hi;
    if constexpr (LO) *reinterpret_cast<u32x4_t *>(dst + 1024) = lo;
  }
}

// The epilogue's destination of four consecutive outputs n0 .. n0 + 3
// (n0 % 4 == 0), split into a column part, computed once per column group,
// and a row part.  Kinds: rows of y (FINAL), q_nope, q_rope (pair p) and the
// kv_a rows (QKV), k and v (KVB).
enum SgKind { kSgY, kSgQNope, kSgQRope, kSgKva, kSgK, kSgV };
struct SgCol {
  int kind;
  int p;         // q_rope: first pair of the four outputs
  int64_t coff;  // column part of the element offset
};

template <int EPI>
__device__ __forceinline__ SgCol sg_col(const SplitGemmArgs &a, int n0) {
  SgCol c{kSgY, 0, n0};
  if constexpr (EPI == kSgEpiQkv) {
    const int qw = a.dn + a.dr, nq = a.heads * qw;
    if (n0 >= nq) {
      c.kind = kSgKva;
      c.coff = n0 - nq;
    } else {
      // head hd's rows of [b, H, s, d]: ((b H + hd) s_len + s) d_w + d is the
      // row part (b H s_len + s) d_w plus the column part hd s_len d_w + d
      const int hd = n0 / qw, d = n0 - hd * qw;
      if (d < a.dn) {
        c.kind = kSgQNope;
        c.coff = (int64_t)hd * a.seq * a.dn + d;
      } else {
        c.kind = kSgQRope;
        c.p = (d - a.dn) >> 1;
        c.coff = (int64_t)hd * a.seq * a.dr + (d - a.dn);
      }
    }
  } else if constexpr (EPI == kSgEpiKvb) {
    const int kw = a.dn + a.dv, hd = n0 / kw, d = n0 - hd * kw;
    if (d < a.dn) {
      c.kind = kSgK;
      c.coff = (int64_t)hd * a.seq * a.dn + d;
    } else {
      c.kind = kSgV;
      c.coff = (int64_t)hd * a.seq * a.dv + (d - a.dn);
    }
  }
  return c;
}

// Stores v (bias included) for row m, token s of sequence b, at column
// group c.
template <int EPI, typename OutT>
__device__ __forceinline__ void sg_write(const SplitGemmArgs &a, const SgCol &c, int m, int b,
                                         int s, const float (&v)[4]) {
  if constexpr (EPI == kSgEpiFinal) {
    sg_put4<float>(a.y + (int64_t)m * a.ldy + c.coff, v);
  } else {
    const int64_t rowp = (int64_t)b * a.heads * a.seq + s;
    if constexpr (EPI == kSgEpiQkv) {
      if (c.kind == kSgKva) {
        sg_put4<float>(a.kva + (int64_t)m * a.kva_ld + c.coff, v);
      } else if (c.kind == kSgQNope) {
        sg_put4<OutT>(reinterpret_cast<OutT *>(a.out0) + rowp * a.dn + c.coff, v);
      } else {
        // interleaved pairs (2p, 2p + 1) of q_rope at position lens[b] + s
        // (src/model.rs:70-84, :199-203)
        const float pos = (float)(a.lens[b] + s);
        float r[4];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          float cs, sn;
          rope_cs(pos * a.inv_freq[c.p + u], a.mscale, cs, sn);
          r[2 * u] = v[2 * u] * cs - v[2 * u + 1] * sn;
          r[2 * u + 1] = v[2 * u + 1] * cs + v[2 * u] * sn;
        }
        sg_put4<OutT>(reinterpret_cast<OutT *>(a.out1) + rowp * a.dr + c.coff, r);
      }
    } else {  // kSgEpiKvb
      if (c.kind == kSgK)
        sg_put4<OutT>(reinterpret_cast<OutT *>(a.out0) + rowp * a.dn + c.coff, v);
      else
        sg_put4<OutT>(reinterpret_cast<OutT *>(a.out1) + rowp * a.dv + c.coff, v);
    }
  }
}

// Split-K: the sum of the slices' partials in slice order, the bias, then
// the epilogue; one thread per four outputs of a row.
template <int EPI, typename OutT>
__global__ __launch_bounds__(256) void k_sg_reduce(SplitGemmArgs a) {
  const int NQ = a.N / 4;
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= (int64_t)a.M * NQ) return;
  const int m = (int)(t / NQ), n0 = 4 * (int)(t - (int64_t)m * NQ);
  const int64_t plane = (int64_t)a.M * a.N;
  const float *src = a.part + (int64_t)m * a.N + n0;
  floatx4_t acc = *reinterpret_cast<const floatx4_t *>(src);
  for (int z = 1; z < a.ksplit; ++z) {
    const floatx4_t p = *reinterpret_cast<const floatx4_t *>(src + z * plane);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += p[e];
  }
  float v[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = acc[e] + (a.bias ? a.bias[n0 + e] : 0.f);
  const int b = m / a.seq;
  sg_write<EPI, OutT>(a, sg_col<EPI>(a, n0), m, b, m - b * a.seq, v);
}

// Tile shape and pipeline of one instantiation: NBW x MBW 32-blocks per
// wave, NWV waves (WN along N, NWV / WN along M), KSC k-steps of 16 per
// chunk and NST chunks in the LDS ring.
template <int NBW_, int MBW_, int WN_, int KSC_, int NST_, int NWV_ = 8>
struct SgCfg {
  static constexpr int NBW = NBW_, MBW = MBW_, WN = WN_, KSC = KSC_, NST = NST_, NWV = NWV_;
};

// XLO / WLO: the activation / weight records' lo halves take part (x_lo w_hi
// and x_hi w_lo); both off is the bf16-operand product.
template <class CF, bool XLO, bool WLO, int EPI, typename OutT>
__global__ __launch_bounds__(CF::NWV * 64) void k_split_gemm(SplitGemmArgs a, const uint8_t *xrec) {
  constexpr int NBW = CF::NBW, MBW = CF::MBW, WN = CF::WN, KSC = CF::KSC, NST = CF::NST;
  constexpr int NWV = CF::NWV, WM = NWV / WN;
  constexpr int MBT = MBW * WM, NBT = NBW * WN;  // 32-row / 32-output blocks of the tile
  constexpr int BM = 32 * MBT, BN = 32 * NBT;
  constexpr int XR = XLO ? 2048 : 1024;           // LDS bytes per activation record
  constexpr int WR = WLO ? 2048 : 1024;           // ... per weight record
  constexpr int WI = KSC * NBT * (WLO ? 2 : 1);   // weight DMA instructions per chunk
  constexpr int WSEG = KSC * NBT * WR;            // a stage's weight records
  constexpr int STAGE = WSEG + KSC * MBT * XR;    // ... and activation records
  constexpr int NDMA = STAGE / 1024;              // DMA instructions per chunk
  // ... per wave; when NDMA is not a multiple of NWV, the waves past the
  // last instruction repeat it (the same bytes into the same place)
  constexpr int DW = (NDMA + NWV - 1) / NWV;
  extern __shared__ __attribute__((aligned(16))) char sg_lds[];
  const uint32_t ring_u = (uint32_t)(uintptr_t)(sg_lds);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wn = wave % WN, wm = wave / WN;
  // XCD-aware tile order: blocks are dealt to the 8 XCDs round-robin, so
  // the k-th block of XCD x is blockIdx.x = 8 k + x.  Each XCD takes groups
  // of kSgGn x kSgGm tiles (group g = 8 (k / G) + x, G = kSgGn kSgGm); the G
  // blocks of a group run together on one XCD and advance through K side by
  // side, so each chunk of a weight tile or activation tile comes from
  // memory once and is re-read from that XCD's L2 by the group's other
  // blocks.
  const int NT = (a.N + BN - 1) / BN, MT = (a.M + BM - 1) / BM;
  const int GNT = (NT + kSgGn - 1) / kSgGn;
  const int L = blockIdx.x, xcd = L & 7, kk = L >> 3;
  const int grp = (kk / (kSgGn * kSgGm)) * 8 + xcd, pos = kk % (kSgGn * kSgGm);
  const int bn = (grp % GNT) * kSgGn + pos % kSgGn, bm = (grp / GNT) * kSgGm + pos / kSgGn;
  if (bn >= NT || bm >= MT) return;  // a slot of a partial group
  const int NB = (a.N + 31) / 32, MB = (a.M + 31) / 32, KS = a.K / 16;
  // this block's K slice: chunks [cz, cz + NC) of the KS / KSC
  const int NC = KS / KSC / a.ksplit, cz = blockIdx.y * NC;

  // DMA slot u of this wave: instruction i = wave DW + u of the chunk.
  // Instructions [0, WI) move weight records (record j KSC + ks of tile
  // block j, hi [then lo]), the rest activation records (tile row block j,
  // k-step ks, hi [then lo]).  Tile blocks past N or M re-load the last
  // block (their outputs are dropped).
  auto dma_one = [&](int c, int u) __attribute__((always_inline)) {
    const uint32_t st = ring_u + (uint32_t)((c % NST) * STAGE);
    {
      const int i = NDMA % NWV ? min(wave * DW + u, NDMA - 1) : wave * DW + u;
      const uint8_t *src;
      if (i < WI) {
        const int rec = WLO ? i >> 1 : i, half = WLO ? i & 1 : 0;
        const int j = rec / KSC, ks = rec % KSC;
        const int nb = min(bn * NBT + j, NB - 1);
        src = reinterpret_cast<const uint8_t *>(a.w_frag) +
              ((int64_t)nb * KS + KSC * (cz + c) + ks) * kFrag + half * 1024;
      } else {
        const int xi = i - WI;
        const int rec = XLO ? xi >> 1 : xi, half = XLO ? xi & 1 : 0;
        const int j = rec / KSC, ks = rec % KSC;
        const int mb = min(bm * MBT + j, MB - 1);
        src = xrec + ((int64_t)mb * KS + KSC * (cz + c) + ks) * XR + half * 1024;
      }
      pipe::dma16(pipe::fresh(src), (uint32_t)(lane * 16), pipe::fresh(st + (uint32_t)(i * 1024)));
    }
  };
  auto dma = [&](int c) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < DW; ++u) dma_one(c, u);
  };

  floatx16_t acc[NBW][MBW];
#pragma unroll
  for (int i = 0; i < NBW; ++i)
#pragma unroll
    for (int j = 0; j < MBW; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

  // Chunk c's products.  With dc >= 0, the DMA slots of chunk dc are spread
  // over the products (slot u after output pair u * PAIRS / DW): a DMA
  // instruction stalls its wave's issue while the memory system is busy,
  // and spread out it stalls between MFMAs instead of ahead of them.
  constexpr int PAIRS = KSC * NBW * MBW;
  auto compute = [&](int c, int dc) __attribute__((always_inline)) {
    const char *st = sg_lds + (c % NST) * STAGE + lane * 16;
#pragma unroll
    for (int ks = 0; ks < KSC; ++ks) {
      bf16x8_t xh[MBW], xl[MBW], wh[NBW], wl[NBW];
#pragma unroll
      for (int i = 0; i < NBW; ++i) {
        const char *f = st + ((wn * NBW + i) * KSC + ks) * WR;
        wh[i] = *reinterpret_cast<const bf16x8_t *>(f);
        if constexpr (WLO) wl[i] = *reinterpret_cast<const bf16x8_t *>(f + 1024);
      }
#pragma unroll
      for (int j = 0; j < MBW; ++j) {
        const char *f = st + WSEG + ((wm * MBW + j) * KSC + ks) * XR;
        xh[j] = *reinterpret_cast<const bf16x8_t *>(f);
        if constexpr (XLO) xl[j] = *reinterpret_cast<const bf16x8_t *>(f + 1024);
      }
#pragma unroll
      for (int i = 0; i < NBW; ++i)
#pragma unroll
        for (int j = 0; j < MBW; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wh[i], xh[j], acc[i][j], 0, 0, 0);
          if constexpr (XLO)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wh[i], xl[j], acc[i][j], 0, 0, 0);
          if constexpr (WLO)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wl[i], xh[j], acc[i][j], 0, 0, 0);
          const int pr = (ks * NBW + i) * MBW + j;
#pragma unroll
          for (int u = 0; u < DW; ++u)
            if (dc >= 0 && (u * PAIRS) / DW == pr) dma_one(dc, u);
        }
    }
  };

  // ---- pipeline: before chunk c is multiplied, this wave's DMA for it
  // must be done (the DW instructions of each of the up to NST - 2 later
  // chunks already requested may stay in flight), then a barrier publishes
  // every wave's share and, since every wave is past chunk c - 1, frees its
  // stage for chunk c + NST - 1.
  static_assert((NST - 2) * DW < 64, "vmcnt range");
#pragma unroll
  for (int p = 0; p < NST - 1; ++p)
    if (p < NC) dma(p);
  for (int c = 0; c < NC; ++c) {
    pipe::wait_vmcnt_dyn(min(NST - 2, NC - 1 - c) * DW);
    sg_barrier();
    compute(c, c + NST - 1 < NC ? c + NST - 1 : -1);
  }

  // ---- epilogue, staged through the idle ring.  Stored straight from the
  // accumulators, each store instruction would write 16 bytes into each of
  // 32 rows; instead each wave writes its accumulators for PN outputs of
  // 32 rows into its own staging rows and reads them back as whole row
  // segments (16 lanes per 64 outputs), so each store instruction covers
  // RPI rows of contiguous outputs.  Per-row and per-column address parts
  // are computed once (incremental sequence positions, one division per
  // pass).
  sg_barrier();  // every wave is done with the ring
  constexpr int PA = NBW >= 2 ? 2 : 1;  // accumulator columns per pass
  constexpr int PN = 32 * PA;           // outputs per pass
  constexpr int SROW = PN * 4 + 16;     // staged row stride in bytes (padded)
  constexpr int CPR = PN / 4;           // 16-byte chunks per staged row
  constexpr int RPI = 64 / CPR;         // rows per read instruction
  constexpr int NI = 32 / RPI;
  // (the launch sizes the ring for the staging rows when they need more)
  char *wst = sg_lds + wave * 32 * SROW;
  const int half = lane >> 5, mr = lane & 31;
  const int lrow = lane / CPR, lch = lane % CPR;
  const bool partial = a.ksplit > 1;
  // one call per row block j, with compile-time j and pass indices so that
  // the accumulators stay in registers
  auto row_block = [&](auto jc) __attribute__((always_inline)) {
    constexpr int j = decltype(jc)::value;
    const int m0 = bm * BM + (wm * MBW + j) * 32;
    if (m0 >= a.M) return;
    // this lane's rows m0 + lrow + RPI ii: sequence b and position s
    int rb[NI], rs[NI];
    {
      const int mf = m0 + lrow;
      int b = mf / a.seq, sq = mf - b * a.seq;
#pragma unroll
      for (int ii = 0; ii < NI; ++ii) {
        rb[ii] = b;
        rs[ii] = sq;
        sq += RPI;
        while (sq >= a.seq) {
          sq -= a.seq;
          ++b;
        }
      }
    }
    auto pass = [&](auto pc) __attribute__((always_inline)) {
      constexpr int pp = decltype(pc)::value;
      // the pass's accumulators into this wave's staging rows
#pragma unroll
      for (int ii = 0; ii < PA; ++ii)
#pragma unroll
        for (int jq = 0; jq < 4; ++jq)
          *reinterpret_cast<floatx4_t *>(wst + mr * SROW + (ii * 32 + 8 * jq + 4 * half) * 4) =
              floatx4_t{acc[pp * PA + ii][j][4 * jq], acc[pp * PA + ii][j][4 * jq + 1],
                        acc[pp * PA + ii][j][4 * jq + 2], acc[pp * PA + ii][j][4 * jq + 3]};
      // this lane's four outputs n0 .. n0 + 3 of the pass: destination and
      // column part of the address
      const int n0 = bn * BN + (wn * NBW + pp * PA) * 32 + lch * 4;
      const bool col_ok = n0 < a.N;
      SgCol col{kSgY, 0, n0};
      float bias4[4] = {0.f, 0.f, 0.f, 0.f};
      if (!partial && col_ok) {
        if (a.bias)
#pragma unroll
          for (int e = 0; e < 4; ++e) bias4[e] = a.bias[n0 + e];
        col = sg_col<EPI>(a, n0);
      }
      pipe::wait_lgkm<0>();  // the staging writes are done
#pragma unroll
      for (int ii = 0; ii < NI; ++ii) {
        const int r = lrow + RPI * ii, m = m0 + r;
        const floatx4_t q = *reinterpret_cast<const floatx4_t *>(wst + r * SROW + lch * 16);
        if (m >= a.M || !col_ok) continue;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = q[e] + bias4[e];
        if (partial) {
          sg_put4<float>(a.part + ((int64_t)blockIdx.y * a.M + m) * a.N + n0, v);
          continue;
        }
        sg_write<EPI, OutT>(a, col, m, rb[ii], rs[ii], v);
      }
      // the next pass rewrites the staging rows after this lane's reads
      pipe::wait_lgkm<0>();
    };
    [&]<int... P>(std::integer_sequence<int, P...>) {
      (pass(std::integral_constant<int, P>{}), ...);
    }(std::make_integer_sequence<int, NBW / PA>{});
  };
  [&]<int... J>(std::integer_sequence<int, J...>) {
    (row_block(std::integral_constant<int, J>{}), ...);
  }(std::make_integer_sequence<int, MBW>{});
}

// The ring, or the epilogue's staging rows (8 waves x 32 rows of 32 or 64
// f32 outputs, padded) when they need more.
template <class CF, bool XLO, bool WLO>
constexpr size_t sg_lds_bytes() {
  constexpr int MBT = CF::MBW * (CF::NWV / CF::WN), NBT = CF::NBW * CF::WN;
  constexpr size_t ring =
      (size_t)CF::NST * CF::KSC * (NBT * (WLO ? 2048 : 1024) + MBT * (XLO ? 2048 : 1024));
  constexpr size_t staging = (size_t)CF::NWV * 32 * (32 * (CF::NBW >= 2 ? 2 : 1) * 4 + 16);
  return ring > staging ? ring : staging;
}

template <class CF, bool XLO, bool WLO>
qmla_status sg_launch(const SplitGemmArgs &a, const uint8_t *xrec, hipStream_t s) {
  constexpr int BN = 32 * CF::NBW * CF::WN, BM = 32 * CF::MBW * (CF::NWV / CF::WN);
  static_assert(sg_lds_bytes<CF, XLO, WLO>() <= 160 * 1024, "LDS");
  // whole groups of kSgGn x kSgGm tile slots, dealt to the 8 XCDs
  const int64_t gn = ((a.N + BN - 1) / BN + kSgGn - 1) / kSgGn;
  const int64_t gm = ((a.M + BM - 1) / BM + kSgGm - 1) / kSgGm;
  const int64_t groups = (gn * gm + 7) / 8 * 8;
  const int64_t blocks = groups * kSgGn * kSgGm;
  QMLA_REQUIRE(blocks <= 0x7fffffff, QMLA_ERR_SHAPE, "split GEMM grid of %lld blocks",
               (long long)blocks);
  const size_t lds = sg_lds_bytes<CF, XLO, WLO>();
  QMLA_REQUIRE(a.K % (16 * CF::KSC) == 0, QMLA_ERR_UNSUPPORTED,
               "split GEMM K %d is not a whole number of %d-wide chunks", a.K, 16 * CF::KSC);
  QMLA_REQUIRE(a.ksplit >= 1 && a.ksplit <= 65535 && (a.K / 16 / CF::KSC) % a.ksplit == 0 &&
                   (a.ksplit == 1 || a.part),
               QMLA_ERR_SHAPE, "split GEMM: %d K slices", a.ksplit);
  const int64_t outs = (int64_t)a.M * (a.N / 4);  // reduce threads
  QMLA_REQUIRE(outs / 256 + 1 <= 0x7fffffff, QMLA_ERR_SHAPE, "split GEMM reduce grid");
  auto go = [&](auto kern, auto reduce) -> qmla_status {
    QMLA_TRY(ensure_dynamic_lds((const void *)kern, lds));
    kern<<<dim3((unsigned)blocks, (unsigned)a.ksplit), dim3(CF::NWV * 64), lds, s>>>(a, xrec);
    QMLA_LAUNCH_CHECK("k_split_gemm");
    if (a.ksplit > 1) {
      reduce<<<dim3((unsigned)((outs + 255) / 256)), dim3(256), 0, s>>>(a);
      QMLA_LAUNCH_CHECK("k_sg_reduce");
    }
    return QMLA_OK;
  };
  switch (a.epi) {
    case kSgEpiQkv:
      if (a.out_bf16)
        return go(k_split_gemm<CF, XLO, WLO, kSgEpiQkv, uint16_t>, k_sg_reduce<kSgEpiQkv, uint16_t>);
      return go(k_split_gemm<CF, XLO, WLO, kSgEpiQkv, float>, k_sg_reduce<kSgEpiQkv, float>);
    case kSgEpiKvb:
      if (a.out_bf16)
        return go(k_split_gemm<CF, XLO, WLO, kSgEpiKvb, uint16_t>, k_sg_reduce<kSgEpiKvb, uint16_t>);
      return go(k_split_gemm<CF, XLO, WLO, kSgEpiKvb, float>, k_sg_reduce<kSgEpiKvb, float>);
    default:
      return go(k_split_gemm<CF, XLO, WLO, kSgEpiFinal, float>, k_sg_reduce<kSgEpiFinal, float>);
  }
}

}  // namespace

bool split_gemm_supported(int N, int K) { return N > 0 && N % 4 == 0 && K > 0 && K % 32 == 0; }

size_t split_gemm_pack_bytes(int M, int K) {
  return (size_t)((M + 31) / 32) * (K / 16) * kFrag;
}

// Below the 256 x 256 tiling, a product whose 64 x 128 tiles leave the
// device short of blocks (fewer than 256) splits K (powers of two, up to 8)
// until about 512 blocks are in flight, keeping at least 8 chunks of 32 k
// per slice: each block streams its slice of K with a latency-bound ring,
// so more, shorter blocks finish sooner.  The second launch that adds the
// slices costs 4-8 us, which a product with K < 1024 does not win back
// (kv_b_proj, K = 512: 18.4 -> 15.0 + 4.2 us at 256 rows).
int split_gemm_slices(int M, int N, int K) {
  if (M >= kSplitGemmBigRows || M <= 0 || N <= 0 || K < 1024) return 1;
  const int64_t tiles = (int64_t)((N + 63) / 64) * ((M + 127) / 128);
  if (tiles >= 256) return 1;
  const int nc = K / 32;  // chunks of the 64 x 128 tiling
  int s = 1;
  while (s < 8 && tiles * s * 2 <= 512 && nc % (2 * s) == 0 && nc / (2 * s) >= 8) s *= 2;
  return s;
}

size_t split_gemm_part_bytes(int M, int N, int K) {
  const int s = split_gemm_slices(M, N, K);
  return s > 1 ? (size_t)s * M * N * sizeof(float) : 0;
}

namespace {
qmla_status sg_check(const SplitGemmArgs &a) {
  QMLA_REQUIRE(split_gemm_supported(a.N, a.K) && a.M > 0, QMLA_ERR_UNSUPPORTED,
               "split GEMM M %d N %d K %d", a.M, a.N, a.K);
  QMLA_REQUIRE(a.seq > 0, QMLA_ERR_SHAPE, "split GEMM seq %d", a.seq);
  QMLA_REQUIRE(a.x_heads == 0 || (a.dv > 0 && a.dv % 16 == 0 && a.K == a.heads * a.dv),
               QMLA_ERR_SHAPE, "split GEMM head-major x: dv %d, K %d", a.dv, a.K);
  QMLA_REQUIRE(a.epi != kSgEpiQkv || (a.dn % 4 == 0 && a.dr % 4 == 0 && a.lens && a.inv_freq),
               QMLA_ERR_SHAPE, "split GEMM q split needs widths that are multiples of 4");
  QMLA_REQUIRE(a.epi != kSgEpiKvb || (a.dn % 4 == 0 && a.dv % 4 == 0), QMLA_ERR_SHAPE,
               "split GEMM k/v split needs widths that are multiples of 4");
  return QMLA_OK;
}

// Many rows: 256 x 256 tiles; fewer: 64 x 128 tiles, so that the grid
// still fills the device (at 2048 rows a 256 x 256 tiling of q_proj |
// kv_a has 120 blocks).
qmla_status sg_run(const SplitGemmArgs &a0, const uint8_t *xrec, bool xlo, hipStream_t s) {
  using Big = SgCfg<4, 2, 2, 1, 3>;
  // bf16 operands: two k-steps per chunk, so that a barrier still spans 16
  // MFMAs per wave (the layer prefill 0.432 -> 0.427 ms in a same-box A/B)
  using BigB16 = SgCfg<4, 2, 2, 2, 3>;
  using Small = SgCfg<1, 1, 2, 2, 3>;
  static_assert(Small::KSC == 2, "split_gemm_slices counts chunks of 32 k");
  SplitGemmArgs a = a0;
  a.ksplit = split_gemm_slices(a.M, a.N, a.K);
  QMLA_REQUIRE(a.ksplit == 1 || a.part, QMLA_ERR_WORKSPACE,
               "split GEMM of %d x %d x %d needs %zu bytes of partial sums", a.M, a.N, a.K,
               split_gemm_part_bytes(a.M, a.N, a.K));
  if (a.bf16ops) {
    if (a.M >= kSplitGemmBigRows) return sg_launch<BigB16, false, false>(a, xrec, s);
    return sg_launch<Small, false, false>(a, xrec, s);
  }
  if (a.M >= kSplitGemmBigRows)
    return xlo ? sg_launch<Big, true, true>(a, xrec, s) : sg_launch<Big, false, true>(a, xrec, s);
  return xlo ? sg_launch<Small, true, true>(a, xrec, s) : sg_launch<Small, false, true>(a, xrec, s);
}
}  // namespace

qmla_status launch_split_gemm_packed(const SplitGemmArgs &a, const void *xrec, hipStream_t s,
                                     bool hi_only) {
  QMLA_TRY(sg_check(a));
  QMLA_REQUIRE(xrec, QMLA_ERR_SHAPE, "packed activations without records");
  return sg_run(a, static_cast<const uint8_t *>(xrec), !hi_only && !a.bf16ops, s);
}

qmla_status launch_split_gemm(const SplitGemmArgs &a, void *pack, hipStream_t s) {
  QMLA_TRY(sg_check(a));
  QMLA_REQUIRE(pack, QMLA_ERR_SHAPE, "split GEMM without a pack buffer");
  // the activations as records (one pass over x)
  const int64_t recs = (int64_t)((a.M + 31) / 32) * (a.K / 16);
  QMLA_REQUIRE(recs + 3 <= 0x7fffffff, QMLA_ERR_SHAPE, "split GEMM pack grid");
  uint8_t *xrec = static_cast<uint8_t *>(pack);
  const dim3 pg((unsigned)((recs + 3) / 4)), pb(256);
  const bool xlo = !(a.x_heads && a.x_bf16) && !a.bf16ops;
  if (a.x_heads && a.x_bf16)
    k_pack_rows<kSgXHeadsBf16, false><<<pg, pb, 0, s>>>(a, xrec);
  else if (a.x_heads == 0)
    xlo ? k_pack_rows<kSgXRow, true><<<pg, pb, 0, s>>>(a, xrec)
        : k_pack_rows<kSgXRow, false><<<pg, pb, 0, s>>>(a, xrec);
  else
    xlo ? k_pack_rows<kSgXHeadsF32, true><<<pg, pb, 0, s>>>(a, xrec)
        : k_pack_rows<kSgXHeadsF32, false><<<pg, pb, 0, s>>>(a, xrec);
  QMLA_LAUNCH_CHECK("k_pack_rows");
  return sg_run(a, xrec, xlo, s);
}

}  // namespace qmla
