// moe_packed.hip -- the 2-bit packed expert GEMV and the QMoE layer forward
// on gfx950: PackedQMoETensor::forward_simd (src/tensor.rs:64-95) over
// fused_dequantize_and_dot (src/simd.rs:6-45), and QMoELayer::forward
// (src/moe.rs:40-130).
//
// Packed format (src/simd.rs:20-31): row i of an [out, in] tensor is in/4
// bytes; weight 4j + q of the row is bits 2q..2q+1 of byte j, a code c in
// 0..3 standing for c - 1.
//
// Exact integer form.  An activation vector x (f32, length K) is turned
// into integers q_k = rint(x_k 2^e) with max |q_k| <= 2^22 (e per vector),
// written as three signed 8-bit digits q = d0 + 2^8 d1 + 2^16 d2.  Then
//   sum_k (c_k - 1) x_k = 2^-e (sum_p 2^(8p) sum_k c_k d_p,k  -  sum_k q_k)
// where every inner sum is an exact int32 from the int8 MFMA
// (v_mfma_i32_32x32x32_i8): the A operand is the codes themselves (one
// shift and one mask turn a 32-bit word of 16 codes into 4 bytes-per-lane
// registers), the B operand the digits of up to 10 vectors (3 columns each
// of the 32).  The only rounding is x -> q (2^-23 of the vector's largest
// element) and the final conversion to f32, so the result is as accurate as
// the reference's f32 sum.
//
// k order.  A lane (row m, half h) of a wave loads 16 bytes of row m at byte
// 32 g + 16 h (group g of 128 codes); word c of them (c = 0..3) feeds the
// MFMA of chunk 4g + c, and its register v byte b holds code 16 c + 4 b + v
// of the word, i.e. k = 128 g + 64 h + 16 c + 4 b + v.  The digits are
// written to LDS in that order, so a lane's B operand is 16 contiguous
// bytes (one ds_read_b128).
#include <cmath>

#include "internal.hpp"

namespace qmla {
namespace {

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));

constexpr int kTokTile = 10;   // vectors per MFMA tile (3 digit columns each)
constexpr int kSlab = 4096;    // codes of B staged in LDS at once (128 KB)
constexpr int kMfmaWaves = 4;  // waves per block; each owns 32 rows
constexpr int kMfmaThreads = 64 * kMfmaWaves;
constexpr int kMaxExperts = 4096;
constexpr int kSelLds = 2048;  // routing tables up to this many pairs are read into LDS
constexpr int kMaxK = 1 << 20;


struct PackedArgs {
  const uint8_t *w[2];      // packed [experts][M][K / 4]
  const float *scale[2];    // [experts][M]
  int64_t w_stride;         // bytes per expert
  int64_t s_stride;         // scales per expert
  int32_t M, K;
  const float *x;           // [vectors][ld_x] f32
  int64_t ld_x;
  int32_t src_div;          // source vector of slot s = s / src_div
  const int2 *ebin;         // per expert {first bin position, pairs} (grid y = expert x
                            //   slices); null: grid y = tiles of kTokTile over `count` slots
  int32_t slices;           // with bins: blocks sharing an expert's bin; block
                            //   (e, s) takes its tiles s, s + slices, ...
  const int32_t *slots;     // bin position -> slot (null: identity)
  const int32_t *sel;       // instead of ebin/slots: expert e's bin is the pairs p with
  int32_t npairs;           //   sel[p] == e, ascending (each block reads it itself)
  const float *logits;      // instead of sel: gate logits [npairs / topk][n_experts]; the
  int32_t n_experts, topk;  //   block ranks every token's experts itself (table in LDS)
  int32_t *sel_out;         // with logits: block (0, slice 0) of expert e writes the
  float *selw_out;          //   routing of e's pairs (expert, softmax weight), and the
  int32_t *user_idx;        //   caller's copies when non-null
  float *user_w;
  int32_t count;
  float *out;               // out[slot * ld_out + row]
  int64_t ld_out;
  const uint32_t *src_max;  // optional: max |x| bits per source vector (skips pass 1),
  int32_t src_max_parts;    //   as src_max_parts partial maxima each
  uint32_t *out_max;        // optional: max |out| bits of this block's rows per slot,
                            //   out_max[slot * gridDim.x + blockIdx.x]
};

struct TileInfo {
  int expert, start, ntok;
};

// The block's expert and its bin range [first, first + count): with bins,
// grid y is (expert, slice) and the block walks every slices-th tile of the
// expert's bin starting at its slice; without, grid y is one tile of the
// `count` slots.
__device__ __forceinline__ bool binned(const PackedArgs &a) { return a.ebin || a.sel || a.logits; }

__device__ __forceinline__ int block_expert(const PackedArgs &a) {
  return binned(a) ? (int)blockIdx.y / a.slices : 0;
}

__device__ __forceinline__ int block_slice(const PackedArgs &a) {
  return binned(a) ? (int)blockIdx.y % a.slices : 0;
}

// Expert e's bin read from the routing table (the pairs p with sel[p] == e,
// ascending p): returns its size, and with `out` lists the pairs at bin
// positions [t0, t0 + n) into out[0..n).  Each thread scans a contiguous run
// of the table; a block scan of the runs' counts orders them.  Every thread
// of the block calls it (two barriers); tmp holds kMfmaWaves ints.
__device__ int sel_bin(const int32_t *sel, int np, int e, int t0, int n, int *out, int *tmp) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (np + kMfmaThreads - 1) / kMfmaThreads;
  const int lo = min(np, tid * per), hi = min(np, lo + per);
  int c = 0;
  for (int p = lo; p < hi; ++p) c += sel[p] == e;
  int incl = c;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(incl, o);
    if (lane >= o) incl += u;
  }
  if (lane == 63) tmp[wave] = incl;
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kMfmaWaves; ++w) {
    base += w < wave ? tmp[w] : 0;
    total += tmp[w];
  }
  if (out) {
    int r = base + incl - c;
    for (int p = lo; p < hi && r < t0 + n; ++p)
      if (sel[p] == e) {
        if (r >= t0) out[r - t0] = p;
        ++r;
      }
  }
  __syncthreads();
  return total;
}

constexpr int kRankTokens = 256;  // tokens the GEMV blocks rank themselves (LDS table)
static_assert(kRankTokens <= kMfmaThreads, "rank_tokens gives every token a thread");

// rank[t] = rank of expert e among token t's E logits lg[t][*]: the number of
// experts before it in (logit descending, index ascending) order, the
// reference's stable descending sort (src/moe.rs:51-82); NaN ranks as -inf.
// T <= kRankTokens; pow2 groups of threads share a token and add their
// counts with LDS atomics into rank[], which the caller zeroed before a
// barrier.  Every thread of the block calls it (one barrier).
__device__ void rank_tokens(const float *lg, int T, int E, int e, int *rank) {
  const int tid = threadIdx.x;
  int g = 1;
  while (g * 2 * T <= kMfmaThreads) g *= 2;
  const int t = tid / g, part = tid - t * g;
  if (t < T) {
    const float *l = lg + t * E;
    const float v = l[e] != l[e] ? -INFINITY : l[e];
    int r = 0;
    for (int j = part; j < E; j += g) {
      const float u = l[j] != l[j] ? -INFINITY : l[j];
      r += (u > v) || (u == v && j < e);
    }
    if (r) atomicAdd(&rank[t], r);
  }
  __syncthreads();
}

// sel_bin over the token ranks of expert e instead of a routing table: the
// bin is the pairs t * topk + rank[t] of the tokens with rank[t] < topk,
// ascending (the order sel_bin gives for the table those ranks make).
__device__ int rank_bin(const int *rank, int T, int topk, int t0, int n, int *out, int *tmp) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (T + kMfmaThreads - 1) / kMfmaThreads;
  const int lo = min(T, tid * per), hi = min(T, lo + per);
  int c = 0;
  for (int t = lo; t < hi; ++t) c += rank[t] < topk;
  int incl = c;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int u = __shfl_up(incl, o);
    if (lane >= o) incl += u;
  }
  if (lane == 63) tmp[wave] = incl;
  __syncthreads();
  int base = 0, total = 0;
#pragma unroll
  for (int w = 0; w < kMfmaWaves; ++w) {
    base += w < wave ? tmp[w] : 0;
    total += tmp[w];
  }
  if (out) {
    int r = base + incl - c;
    for (int t = lo; t < hi && r < t0 + n; ++t)
      if (rank[t] < topk) {
        if (r >= t0) out[r - t0] = t * topk + rank[t];
        ++r;
      }
  }
  __syncthreads();
  return total;
}

__device__ __forceinline__ void block_range(const PackedArgs &a, int &first, int &count) {
  if (a.ebin) {
    const int2 eb = a.ebin[blockIdx.y / a.slices];
    first = eb.x;
    count = eb.y;
  } else {
    first = blockIdx.y * kTokTile;
    count = min(kTokTile, a.count - first);
  }
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt out of range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ u32x4_t gload16(const uint8_t *p) {
  return *reinterpret_cast<const u32x4_t *>(p);
}

__device__ __forceinline__ i32x4_t decode_codes(uint32_t w) {
  return i32x4_t{(int)(w & 0x03030303u), (int)((w >> 2) & 0x03030303u),
                 (int)((w >> 4) & 0x03030303u), (int)((w >> 6) & 0x03030303u)};
}

constexpr int kBadExp = 0x7fffffff;  // exponent marking a vector with inf/NaN

// Expert GEMV over one tile of vectors.  NMAT = 1: out = dot * scale.
// NMAT = 2 (gate, up): out = swish(dot_0 * s_0) * (dot_1 * s_1)
// (src/moe.rs:102-115).  Block: 4 waves x 32 rows; grid (row blocks,
// experts) with each block walking its expert's tiles, or (row blocks,
// tiles) without bins.
// The block turns its <= 10 f32 vectors into digit planes itself: pass 1
// finds each vector's largest magnitude (its exponent e) unless the producer
// handed it over (src_max), pass 2 writes the digits of each slab of K into
// LDS in the lane order of the B operand and sums q per vector.
// NG > 0: K = 128 NG in one slab with a compile-time ring of weight
// groups, the first ones requested at entry so their HBM latency overlaps
// the quantisation.  NG = 0: any K % 128 == 0, a ring of D groups in flight.
template <int NMAT, int NG>
__global__ __launch_bounds__(kMfmaThreads) void k_packed_mfma(PackedArgs a) {
  extern __shared__ __attribute__((aligned(16))) int8_t lds_b[];  // [chunk][h][32][16]
  __shared__ int64_t voff[kTokTile];
  __shared__ int vslot[kTokTile];
  __shared__ unsigned vmax[kTokTile];
  __shared__ int vexp[kTokTile];
  __shared__ unsigned long long vsum[kTokTile];
  __shared__ unsigned bmax[kTokTile];
  __shared__ int sel_list[kTokTile];
  __shared__ int sel_tmp[kMfmaWaves];
  __shared__ int32_t sel_lds[kSelLds];
  __shared__ int rank_lds[kRankTokens];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int n = lane & 31, h = lane >> 5;
  const int m0 = (blockIdx.x * kMfmaWaves + wave) * 32;
  const bool wave_ok = m0 < a.M;
  const bool row_ok = m0 + n < a.M;
  const int bpr = a.K >> 2;
  const int expert = block_expert(a), slice = block_slice(a);
  const uint8_t *wp[NMAT];
#pragma unroll
  for (int i = 0; i < NMAT; ++i)
    wp[i] = a.w[i] + expert * a.w_stride + (int64_t)(row_ok ? m0 + n : 0) * bpr + 16 * h;

  // Loads are branch-free (rows past M read row 0, ring slots past the slab
  // re-read its last group; neither result is used) so that the compiler
  // keeps them in flight instead of waiting behind each branch.  The first
  // groups are requested before the block knows its tokens: the expert is
  // the grid position, so the weight stream starts while the bins are read.
  constexpr int D = 4;
  constexpr int PD = NMAT == 1 ? 8 : 6;  // groups in flight, fixed group count
  constexpr int NR = NG > 0 ? (NG < PD ? NG : PD) : D;
  u32x4_t ring[NR][NMAT];
  const int ng0 = min(kSlab, a.K) >> 7;
  // Slice 0 requests its first weight groups before it reads its bin; the
  // other slices of an expert (which have work only for bins of more than
  // one tile) request theirs once they know they have a tile.
  if (slice == 0) {
#pragma unroll
    for (int d = 0; d < NR; ++d)
#pragma unroll
      for (int i = 0; i < NMAT; ++i)
        ring[d][i] = gload16(wp[i] + (NG > 0 ? d : min(d, ng0 - 1)) * 32);
  }

  int first = 0, count;
  // the routing table, read once (into LDS when it fits); or the logits
  // (always in LDS: the host takes this path only when they fit)
  const int32_t *bins = a.sel;
  const float *lg = reinterpret_cast<const float *>(sel_lds);
  const int ntok_r = a.logits ? a.npairs / a.topk : 0;
  if (a.logits) {
    for (int i = tid; i < ntok_r * a.n_experts; i += kMfmaThreads)
      sel_lds[i] = __float_as_int(a.logits[i]);
    for (int t = tid; t < ntok_r; t += kMfmaThreads) rank_lds[t] = 0;
    __syncthreads();
  } else if (a.sel && a.npairs <= kSelLds) {
    for (int p = tid; p < a.npairs; p += kMfmaThreads) sel_lds[p] = a.sel[p];
    __syncthreads();
    bins = sel_lds;
  }
  if (a.logits) {
    rank_tokens(lg, ntok_r, a.n_experts, expert, rank_lds);
    count = rank_bin(rank_lds, ntok_r, a.topk, 0, 0, nullptr, sel_tmp);
  } else if (a.sel) {
    count = sel_bin(bins, a.npairs, expert, 0, 0, nullptr, sel_tmp);
  } else {
    block_range(a, first, count);
  }
  if (a.sel_out && slice == 0) {
    // This expert's part of the routing table, for the launches after this
    // one: (expert, weight) at pair t * topk + rank.  The weight is the
    // softmax over all experts' logits (src/moe.rs:51-82), one wave per
    // token with k_moe_route's lane order and reductions; the expert's row
    // blocks share the tokens (token t: row block t % gridDim.x).
    const int E = a.n_experts, lane = tid & 63, wave = tid >> 6;
    for (int t = blockIdx.x + (int)gridDim.x * wave; t < ntok_r;
         t += (int)gridDim.x * kMfmaWaves) {
      if (rank_lds[t] >= a.topk) continue;
      const float *l = lg + t * E;
      float mx = -INFINITY;
      for (int j = lane; j < E; j += 64) mx = fmaxf(mx, l[j]);
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
      float se = 0.f;
      for (int j = lane; j < E; j += 64) se += expf(l[j] - mx);
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) se += __shfl_xor(se, o);
      if (lane == 0) {
        const float w = expf(l[expert] - mx) / se;
        const int o = t * a.topk + rank_lds[t];
        a.sel_out[o] = expert;
        a.selw_out[o] = w;
        if (a.user_idx) a.user_idx[o] = expert;
        if (a.user_w) a.user_w[o] = w;
      }
    }
  }
  const int tt0 = slice * kTokTile;
  if (count <= tt0) {  // no tile for this block: drain the requested groups
    wait_vm<0>();
    return;
  }
  // without bins the grid position is the block's only tile (count <= kTokTile)
  const int tstep = binned(a) ? a.slices * kTokTile : kTokTile;
  for (int tt = tt0; tt < count; tt += tstep) {
  const TileInfo ti{expert, first + tt, min(kTokTile, count - tt)};
  if (tt != tt0 || slice != 0) {
    // a later tile of this block: the LDS of the last one is free once every
    // wave is past its epilogue; its weights come again (from L2)
    if (tt != tt0) __syncthreads();
#pragma unroll
    for (int d = 0; d < NR; ++d)
#pragma unroll
      for (int i = 0; i < NMAT; ++i)
        ring[d][i] = gload16(wp[i] + (NG > 0 ? d : min(d, ng0 - 1)) * 32);
  }

  if (a.logits)
    rank_bin(rank_lds, ntok_r, a.topk, tt, ti.ntok, sel_list, sel_tmp);
  else if (a.sel)
    sel_bin(bins, a.npairs, expert, tt, ti.ntok, sel_list, sel_tmp);
  if (tid < kTokTile) {
    vmax[tid] = 0;
    vsum[tid] = 0;
    if (tid < ti.ntok) {
      const int pos = ti.start + tid;
      const int slot = a.sel || a.logits ? sel_list[tid] : a.slots ? a.slots[pos] : pos;
      const int src = slot / a.src_div;
      vslot[tid] = slot;
      voff[tid] = (int64_t)src * a.ld_x;
      if (a.src_max) {
        unsigned m = 0;
        for (int j = 0; j < a.src_max_parts; ++j)
          m = max(m, a.src_max[(int64_t)src * a.src_max_parts + j]);
        vmax[tid] = m;
      }
    }
    bmax[tid] = 0;
  }
  __syncthreads();

  const int K4 = a.K >> 2;
  if (!a.src_max) {
    // Pass 1: largest |x| of each vector (as f32 bits; inf/NaN compare above).
    const int items = ti.ntok * K4;
    constexpr int U = 8;
    unsigned run = 0;
    int cur = -1;
    for (int base = 0; base < items; base += kMfmaThreads * U) {
      u32x4_t v[U];
      int tt[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = min(base + tid + kMfmaThreads * u, items - 1);
        const int tu = i / K4;
        v[u] = *reinterpret_cast<const u32x4_t *>(a.x + voff[tu] + 4 * (i - tu * K4));
        tt[u] = base + tid + kMfmaThreads * u < items ? tu : -1;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (tt[u] < 0) continue;
        if (tt[u] != cur) {
          if (cur >= 0) atomicMax(&vmax[cur], run);
          cur = tt[u];
          run = 0;
        }
        const u32x4_t m = v[u] & 0x7fffffffu;
        run = max(run, max(max(m[0], m[1]), max(m[2], m[3])));
      }
    }
    if (cur >= 0) atomicMax(&vmax[cur], run);
    __syncthreads();
  }
  if (tid < ti.ntok) {
    const unsigned mb = vmax[tid] & 0x7fffffffu;
    int e = 0;
    if (mb >= 0x7f800000u) {
      e = kBadExp;
    } else if (mb != 0) {
      int ex;
      frexpf(__uint_as_float(mb), &ex);  // max |x| < 2^ex
      e = 22 - ex;                       // max |q| <= 2^22
    }
    vexp[tid] = e;
  }

  i32x16_t acc[NMAT];
#pragma unroll
  for (int i = 0; i < NMAT; ++i) acc[i] = i32x16_t{};

  for (int k0 = 0; k0 < a.K; k0 += kSlab) {
    const int ks = min(kSlab, a.K - k0);
    const int nch = ks >> 5;
    __syncthreads();
    // Pass 2: digit planes of the slab.  Item (t, half, chunk) covers 16
    // consecutive k of vector t and fills columns 3t .. 3t+2.
    {
      const int items = ti.ntok * 2 * nch;
      unsigned long long qs = 0;
      int cur = -1;
      constexpr int U2 = 2;  // items whose loads are issued together
      for (int i0 = tid; i0 < items; i0 += kMfmaThreads * U2) {
        floatx4_t f[U2][4];
#pragma unroll
        for (int u = 0; u < U2; ++u) {
          const int i = min(i0 + kMfmaThreads * u, items - 1);
          const int t = i % ti.ntok, r = i / ti.ntok;
          const int cg = (k0 >> 5) + (r >> 1);
          const float *src = a.x + voff[t] + 128 * (cg >> 2) + 64 * (r & 1) + 16 * (cg & 3);
#pragma unroll
          for (int j = 0; j < 4; ++j) f[u][j] = *reinterpret_cast<const floatx4_t *>(src + 4 * j);
        }
#pragma unroll
        for (int u = 0; u < U2; ++u) {
          const int i = i0 + kMfmaThreads * u;
          if (i >= items) break;
          const int t = i % ti.ntok, r = i / ti.ntok;
          const int h2 = r & 1, c = r >> 1;
          const int e = vexp[t];
          uint32_t w0[4] = {0, 0, 0, 0}, w1[4] = {0, 0, 0, 0}, w2[4] = {0, 0, 0, 0};
          long long sq = 0;
#pragma unroll
          for (int j = 0; j < 16; ++j) {  // j = 4 b + v -> byte b of word v
            const int q = e == kBadExp ? 0 : (int)rintf(ldexpf(f[u][j >> 2][j & 3], e));
            const int d0 = ((q + 128) & 255) - 128;
            const int q1 = (q - d0) >> 8;
            const int d1 = ((q1 + 128) & 255) - 128;
            const int d2 = (q1 - d1) >> 8;
            const int v = j & 3, sh = 8 * (j >> 2);
            w0[v] |= (uint32_t)(d0 & 255) << sh;
            w1[v] |= (uint32_t)(d1 & 255) << sh;
            w2[v] |= (uint32_t)(d2 & 255) << sh;
            sq += q;
          }
          i32x4_t *dst = reinterpret_cast<i32x4_t *>(lds_b + (((c * 2 + h2) * 32 + 3 * t) << 4));
          dst[0] = i32x4_t{(int)w0[0], (int)w0[1], (int)w0[2], (int)w0[3]};
          dst[1] = i32x4_t{(int)w1[0], (int)w1[1], (int)w1[2], (int)w1[3]};
          dst[2] = i32x4_t{(int)w2[0], (int)w2[1], (int)w2[2], (int)w2[3]};
          if (t != cur) {
            if (cur >= 0) atomicAdd(&vsum[cur], qs);
            cur = t;
            qs = 0;
          }
          qs += (unsigned long long)sq;
        }
      }
      if (cur >= 0) atomicAdd(&vsum[cur], qs);
      // columns of absent vectors and the two spare columns
      const int spare = 32 - 3 * ti.ntok;
      for (int i = tid; i < spare * 2 * nch; i += kMfmaThreads) {
        const int col = 3 * ti.ntok + i % spare, r = i / spare;
        *reinterpret_cast<i32x4_t *>(lds_b + ((r * 32 + col) << 4)) = i32x4_t{0, 0, 0, 0};
      }
    }
    __syncthreads();
    // Nothing but weight loads is in flight from here on: without this
    // drain the compiler keeps waits at the loop head for loads of the
    // passes above, which would also hold the weight ring.  The weights
    // were requested before pass 1.
    wait_vm<0>();
    if (!wave_ok) continue;
    if constexpr (NG > 0) {
#pragma unroll
      for (int g = 0; g < NG; ++g) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const i32x4_t b = *reinterpret_cast<const i32x4_t *>(
              lds_b + ((((g * 4 + c) * 2 + h) * 32 + n) << 4));
#pragma unroll
          for (int i = 0; i < NMAT; ++i)
            acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(decode_codes(ring[g % NR][i][c]), b,
                                                           acc[i], 0, 0, 0);
        }
        if (g + NR < NG) {  // compile-time: refill the slot with group g + NR
#pragma unroll
          for (int i = 0; i < NMAT; ++i) ring[g % NR][i] = gload16(wp[i] + (g + NR) * 32);
        }
        // pin the refill here: the scheduler would otherwise sink it next
        // to its use and leave one group in flight
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      const int ng = ks >> 7;
      const int gk0 = k0 >> 7;
      if (k0 > 0) {
#pragma unroll
        for (int d = 0; d < D; ++d)
#pragma unroll
          for (int i = 0; i < NMAT; ++i)
            ring[d][i] = gload16(wp[i] + (gk0 + min(d, ng - 1)) * 32);
      }
      // Branch-free body (the group count is padded to a multiple of D;
      // padding groups multiply zero codes), so that the compiler's waits
      // stay per group instead of collapsing at each branch.
      for (int g0 = 0; g0 < ng; g0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
          const int g = g0 + d;
          const bool live = g < ng;
          const int gl = min(g, ng - 1);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const i32x4_t b = *reinterpret_cast<const i32x4_t *>(
                lds_b + ((((gl * 4 + c) * 2 + h) * 32 + n) << 4));
#pragma unroll
            for (int i = 0; i < NMAT; ++i)
              acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                  decode_codes(live ? ring[d][i][c] : 0u), b, acc[i], 0, 0, 0);
          }
          // the slot is free once its codes are decoded: refill it in place
#pragma unroll
          for (int i = 0; i < NMAT; ++i)
            ring[d][i] = gload16(wp[i] + (gk0 + min(g + D, ng - 1)) * 32);
        }
      }
    }
  }
  // Epilogue.  The accumulators go through LDS (the B area, free once
  // every wave is past its MFMAs) so that each lane finishes whole outputs:
  // row rl = lane % 32 of the wave's 32, vectors lane / 32, + 2, ...  The
  // three digit columns are combined once per output and each vector's 32
  // rows leave as one 128-byte store.  Idle waves (rows past M) stay to the
  // end for the block barriers.
  __syncthreads();
  int *accs = reinterpret_cast<int *>(lds_b) + wave * (NMAT * 16 * 64);
  if (wave_ok) {
#pragma unroll
    for (int i = 0; i < NMAT; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) accs[(i * 16 + r) * 64 + lane] = acc[i][r];
  }
  // accumulator element (row rl, column c) sits in register
  // r = 4 (rl / 8) + rl % 4 of lane c + 32 ((rl / 4) % 2)
  const int rl = lane & 31;
  const int rr = 4 * (rl >> 3) + (rl & 3), lb = 32 * ((rl >> 2) & 1);
  const int row = m0 + rl;
  const bool row_live = wave_ok && row < a.M;
  const int rowc = min(row, a.M - 1);
  const float sc0 = a.scale[0][expert * a.s_stride + rowc];
  const float sc1 = a.scale[NMAT - 1][expert * a.s_stride + rowc];
  for (int t = lane >> 5; t < ti.ntok; t += 2) {
    const int e = vexp[t];
    const long long qsum = (long long)vsum[t];
    float dot[NMAT];
#pragma unroll
    for (int i = 0; i < NMAT; ++i) {
      const int *ar = accs + (i * 16 + rr) * 64 + lb + 3 * t;
      const long long tot = (long long)ar[0] + ((long long)ar[1] << 8) + ((long long)ar[2] << 16);
      dot[i] = e == kBadExp ? __builtin_nanf("") : (float)ldexp((double)(tot - qsum), -e);
    }
    float y;
    if constexpr (NMAT == 1) {
      y = dot[0] * sc0;
    } else {
      const float g = dot[0] * sc0;
      const float u = dot[1] * sc1;
      y = (g * (1.0f / (1.0f + expf(-g)))) * u;
    }
    if (row_live) {
      a.out[(int64_t)vslot[t] * a.ld_out + row] = y;
      if (a.out_max) atomicMax(&bmax[t], __float_as_uint(y) & 0x7fffffffu);  // LDS
    }
  }
  if (a.out_max) {  // this block's partial maximum per vector, no global atomics
    __syncthreads();
    if (tid < ti.ntok) a.out_max[(int64_t)vslot[tid] * gridDim.x + blockIdx.x] = bmax[tid];
  }
  }  // tiles of the block
}

// Fallback for in_features that are not a multiple of 128: one thread per
// output row, the reference's four lane sums in its order (src/simd.rs:17-44,
// separate multiply and add), so its results are those of the reference.
template <int NMAT>
__global__ __launch_bounds__(256) void k_packed_generic(PackedArgs a) {
  int first, count;
  block_range(a, first, count);
  const int row = blockIdx.x * 256 + threadIdx.x;
  if (row >= a.M) return;
  const int bpr = a.K >> 2;
  const TileInfo ti{block_expert(a), first, count};
  const int stride = a.ebin ? a.slices : 1;  // slices >= 1 whenever bins are given
  for (int t = block_slice(a); t < ti.ntok; t += stride) {
    const int pos = ti.start + t;
    const int slot = a.slots ? a.slots[pos] : pos;
    const float *xv = a.x + (int64_t)(slot / a.src_div) * a.ld_x;
    float dot[NMAT];
#pragma unroll
    for (int i = 0; i < NMAT; ++i) {
      const uint8_t *wr = a.w[i] + ti.expert * a.w_stride + (int64_t)row * bpr;
      float l0 = 0.f, l1 = 0.f, l2 = 0.f, l3 = 0.f;
      for (int j = 0; j < bpr; ++j) {
        const uint32_t by = wr[j];
        l0 = __fadd_rn(l0, __fmul_rn((float)(by & 3u) - 1.0f, xv[4 * j]));
        l1 = __fadd_rn(l1, __fmul_rn((float)((by >> 2) & 3u) - 1.0f, xv[4 * j + 1]));
        l2 = __fadd_rn(l2, __fmul_rn((float)((by >> 4) & 3u) - 1.0f, xv[4 * j + 2]));
        l3 = __fadd_rn(l3, __fmul_rn((float)(by >> 6) - 1.0f, xv[4 * j + 3]));
      }
      dot[i] = __fmul_rn(__fadd_rn(__fadd_rn(__fadd_rn(l0, l1), l2), l3),
                         a.scale[i][ti.expert * a.s_stride + row]);
    }
    float *o = a.out + (int64_t)slot * a.ld_out;
    if constexpr (NMAT == 1) {
      o[row] = dot[0];
    } else {
      const float g = dot[0];
      o[row] = __fmul_rn(__fmul_rn(g, 1.0f / (1.0f + expf(-g))), dot[1]);
    }
  }
}

// Gate logits, top-k and routing weights of one token per block
// (src/moe.rs:51-82): logits over every expert (16 waves, two experts per
// wave at a time with all their loads in flight together), rank by (logit
// desc, index asc) -- the order of the reference's stable descending sort --,
// softmax over all experts, top_k weights.  Also the largest |x| (f32 bits)
// of the token, for the expert GEMVs' quantisation.
__global__ __launch_bounds__(1024) void k_moe_route(const float *__restrict__ xs,
                                                    const float *__restrict__ gw, int E, int H,
                                                    int topk, int32_t *__restrict__ sel,
                                                    float *__restrict__ selw,
                                                    int32_t *__restrict__ user_idx,
                                                    float *__restrict__ user_w,
                                                    uint32_t *__restrict__ xmax) {
  __shared__ float lg[kMaxExperts];
  __shared__ float stat[2];
  const int t = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const float *x = xs + (int64_t)t * H;
  const bool vec = (H & 3) == 0 && (((uintptr_t)xs | (uintptr_t)gw) & 15) == 0;
  uint32_t xm = 0;
  for (int e0 = wave; e0 < E; e0 += 32) {
    const int e1 = e0 + 16;
    const float *w0 = gw + (int64_t)e0 * H;
    const float *w1 = gw + (int64_t)min(e1, E - 1) * H;
    float s0 = 0.f, s1 = 0.f;
    if (vec) {
      const int H4 = H >> 2;
      constexpr int U = 8;
      for (int base = 0; base < H4; base += 64 * U) {
        floatx4_t xv[U], a0[U], a1[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int i = min(base + lane + 64 * u, H4 - 1);  // branch-free loads
          xv[u] = reinterpret_cast<const floatx4_t *>(x)[i];
          a0[u] = reinterpret_cast<const floatx4_t *>(w0)[i];
          a1[u] = reinterpret_cast<const floatx4_t *>(w1)[i];
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
          if (base + lane + 64 * u < H4) {
            s0 += xv[u][0] * a0[u][0] + xv[u][1] * a0[u][1] + xv[u][2] * a0[u][2] +
                  xv[u][3] * a0[u][3];
            s1 += xv[u][0] * a1[u][0] + xv[u][1] * a1[u][1] + xv[u][2] * a1[u][2] +
                  xv[u][3] * a1[u][3];
#pragma unroll
            for (int j = 0; j < 4; ++j) xm = max(xm, __float_as_uint(xv[u][j]) & 0x7fffffffu);
          }
      }
    } else {
      for (int k = lane; k < H; k += 64) {
        s0 += x[k] * w0[k];
        s1 += x[k] * w1[k];
        xm = max(xm, __float_as_uint(x[k]) & 0x7fffffffu);
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      s0 += __shfl_xor(s0, o);
      s1 += __shfl_xor(s1, o);
    }
    if (lane == 0) {
      lg[e0] = s0;
      if (e1 < E) lg[e1] = s1;
    }
  }
  if (wave == 0) {  // wave 0 read all of x in its first pass (E >= 1)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) xm = max(xm, (uint32_t)__shfl_xor((int)xm, o));
    if (lane == 0) xmax[t] = xm;
  }
  __syncthreads();
  if (wave == 0) {
    float mx = -INFINITY;
    for (int e = lane; e < E; e += 64) mx = fmaxf(mx, lg[e]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    float se = 0.f;
    for (int e = lane; e < E; e += 64) se += expf(lg[e] - mx);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) se += __shfl_xor(se, o);
    if (lane == 0) {
      stat[0] = mx;
      stat[1] = se;
    }
  }
  __syncthreads();
  const float mx = stat[0], se = stat[1];
  // NaN logits rank as -inf, so the ranks stay a permutation of 0..E-1
  // and every (token, rank < top_k) entry is written exactly once.
  for (int e = threadIdx.x; e < E; e += 1024) {
    const float v = lg[e] != lg[e] ? -INFINITY : lg[e];
    int rank = 0;
    for (int j = 0; j < E; ++j) {
      const float u = lg[j] != lg[j] ? -INFINITY : lg[j];
      rank += (u > v) || (u == v && j < e);
    }
    if (rank < topk) {
      const float w = expf(lg[e] - mx) / se;
      const int64_t o = (int64_t)t * topk + rank;
      sel[o] = e;
      selw[o] = w;
      if (user_idx) user_idx[o] = e;
      if (user_w) user_w[o] = w;
    }
  }
}

// Gate logits only, one wave per (token, expert): grid (ceil(E / 4), T) of
// 4 waves, so a token's E gate rows are read by E / 4 CUs rather than one.
// Each wave's dot product runs the same lane and chunk order as
// k_moe_route's, so the logits are the same bits.  Wave 0 of block (0, t)
// also finds the token's largest |x| (f32 bits) for the expert GEMVs.  The
// GEMV blocks rank the experts themselves (PackedArgs::logits).
__global__ __launch_bounds__(256) void k_moe_logits(const float *__restrict__ xs,
                                                    const float *__restrict__ gw, int E, int H,
                                                    float *__restrict__ logits,
                                                    uint32_t *__restrict__ xmax) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.x * 4 + wave, t = blockIdx.y;
  if (e >= E) return;
  const float *x = xs + (int64_t)t * H;
  const float *w0 = gw + (int64_t)e * H;
  const bool vec = (H & 3) == 0 && (((uintptr_t)xs | (uintptr_t)gw) & 15) == 0;
  const bool want_max = blockIdx.x == 0 && wave == 0;
  uint32_t xm = 0;
  float s0 = 0.f;
  if (vec) {
    const int H4 = H >> 2;
    constexpr int U = 8;
    for (int base = 0; base < H4; base += 64 * U) {
      floatx4_t xv[U], a0[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int i = min(base + lane + 64 * u, H4 - 1);  // branch-free loads
        xv[u] = reinterpret_cast<const floatx4_t *>(x)[i];
        a0[u] = reinterpret_cast<const floatx4_t *>(w0)[i];
      }
#pragma unroll
      for (int u = 0; u < U; ++u)
        if (base + lane + 64 * u < H4) {
          s0 += xv[u][0] * a0[u][0] + xv[u][1] * a0[u][1] + xv[u][2] * a0[u][2] +
                xv[u][3] * a0[u][3];
#pragma unroll
          for (int j = 0; j < 4; ++j) xm = max(xm, __float_as_uint(xv[u][j]) & 0x7fffffffu);
        }
    }
  } else {
    for (int k = lane; k < H; k += 64) {
      s0 += x[k] * w0[k];
      xm = max(xm, __float_as_uint(x[k]) & 0x7fffffffu);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s0 += __shfl_xor(s0, o);
  if (lane == 0) logits[(int64_t)t * E + e] = s0;
  if (want_max) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) xm = max(xm, (uint32_t)__shfl_xor((int)xm, o));
    if (lane == 0) xmax[t] = xm;
  }
}

// Exclusive prefix sum over a 1024-thread block (one value per thread).
__device__ long long block_scan1024(long long v, long long *tmp) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  long long incl = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const long long u = __shfl_up(incl, o);
    if (lane >= o) incl += u;
  }
  if (lane == 63) tmp[wave] = incl;
  __syncthreads();
  long long base = 0;
  for (int w = 0; w < wave; ++w) base += tmp[w];
  __syncthreads();
  return base + incl - v;
}

// Token binning (src/moe.rs:56-82 expert_bins): per-expert counts, bin
// offsets ({first, count} per expert) and the bin position -> slot list.
// Order within a bin does not change any result (each pair is computed
// alone).
__global__ __launch_bounds__(1024) void k_moe_bin(const int32_t *__restrict__ sel, int npairs,
                                                  int E, int2 *__restrict__ ebin,
                                                  int32_t *__restrict__ pair_slot) {
  __shared__ int cnt[kMaxExperts];
  __shared__ int cur[kMaxExperts];
  __shared__ long long tmp[16];
  for (int e = threadIdx.x; e < E; e += 1024) cnt[e] = 0;
  __syncthreads();
  for (int p = threadIdx.x; p < npairs; p += 1024) {
    const int e = sel[p];
    if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
  }
  __syncthreads();
  // thread j owns experts 4j .. 4j + 3 (E <= 4096)
  long long mine = 0;
  int c4[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = 4 * threadIdx.x + i;
    c4[i] = e < E ? cnt[e] : 0;
    mine += c4[i];
  }
  int off = (int)block_scan1024(mine, tmp);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int e = 4 * threadIdx.x + i;
    if (e < E) {
      cur[e] = off;
      ebin[e] = int2{off, c4[i]};
    }
    off += c4[i];
  }
  __syncthreads();
  for (int p = threadIdx.x; p < npairs; p += 1024) {
    const int e = sel[p];
    if (e < 0 || e >= E) continue;
    const int pos = atomicAdd(&cur[e], 1);
    pair_slot[pos] = p;
  }
}

// out[t] = sum over the token's experts in ascending expert order of
// y[slot] * weight, starting from zero (src/moe.rs:86, :89, :121-125).
__global__ __launch_bounds__(256) void k_moe_combine(const float *__restrict__ y,
                                                     const int32_t *__restrict__ sel,
                                                     const float *__restrict__ selw, int T,
                                                     int topk, int H, float *__restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)T * H) return;
  const int t = (int)(idx / H), hh = (int)(idx - (int64_t)t * H);
  const int32_t *st = sel + (int64_t)t * topk;
  float acc = 0.f;
  int last = -1;
  for (int r = 0; r < topk; ++r) {
    int best = -1, be = 0x7fffffff;
    for (int j = 0; j < topk; ++j)
      if (st[j] > last && st[j] < be) {
        be = st[j];
        best = j;
      }
    if (best < 0) break;
    last = be;
    const int64_t slot = (int64_t)t * topk + best;
    acc = __fadd_rn(acc, __fmul_rn(y[slot * H + hh], selw[slot]));
  }
  out[idx] = acc;
}

__global__ void k_fill_zero(float *p, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0.f;
}

// ------------------------------------------------------------------- host

inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

bool mfma_ok(int32_t K) { return K > 0 && K % 128 == 0 && K <= kMaxK; }

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// B operand slab, reused by the epilogue for the accumulators (4 waves x
// NMAT x 16 registers x 64 lanes x 4 bytes)
size_t mfma_lds_bytes(int32_t K, int nmat) {
  return std::max((size_t)std::min(K, kSlab) * 32, (size_t)kMfmaWaves * nmat * 16 * 64 * 4);
}

int mfma_row_blocks(int32_t M) { return (M + 32 * kMfmaWaves - 1) / (32 * kMfmaWaves); }

constexpr int64_t kMaxTileGrid = 65535;  // grid y limit
constexpr int64_t kMaxSlices = 64;       // blocks sharing one expert's bin

template <int NMAT, int NG>
qmla_status launch_mfma(const PackedArgs &a, int64_t tile_grid, hipStream_t s) {
  const size_t lds = mfma_lds_bytes(a.K, NMAT);
  QMLA_TRY(ensure_dynamic_lds((const void *)k_packed_mfma<NMAT, NG>, lds));
  const dim3 grid(mfma_row_blocks(a.M), (unsigned)tile_grid);
  hipLaunchKernelGGL((k_packed_mfma<NMAT, NG>), grid, dim3(kMfmaThreads), lds, s, a);
  QMLA_LAUNCH_CHECK("k_packed_mfma");
  return QMLA_OK;
}

template <int NMAT>
qmla_status launch_packed(const PackedArgs &a, int64_t tile_grid, bool mfma, hipStream_t s) {
  if (tile_grid <= 0 || a.M <= 0) return QMLA_OK;
  QMLA_REQUIRE(tile_grid <= kMaxTileGrid, QMLA_ERR_UNSUPPORTED,
               "grid of %lld tiles or experts (at most %lld)", (long long)tile_grid,
               (long long)kMaxTileGrid);
  if (mfma) {
    // whole-K prefetch for the common widths (NMAT x NG x 16 B a lane)
    switch (a.K >> 7) {
      case 2: return launch_mfma<NMAT, 2>(a, tile_grid, s);
      case 4: return launch_mfma<NMAT, 4>(a, tile_grid, s);
      case 8: return launch_mfma<NMAT, 8>(a, tile_grid, s);
      case 11: return launch_mfma<NMAT, 11>(a, tile_grid, s);
      case 12: return launch_mfma<NMAT, 12>(a, tile_grid, s);
      case 16: return launch_mfma<NMAT, 16>(a, tile_grid, s);
      default: return launch_mfma<NMAT, 0>(a, tile_grid, s);
    }
  }
  const dim3 grid((a.M + 255) / 256, (unsigned)tile_grid);
  hipLaunchKernelGGL(k_packed_generic<NMAT>, grid, dim3(256), 0, s, a);
  QMLA_LAUNCH_CHECK("k_packed_generic");
  return QMLA_OK;
}

qmla_status check_packed_dims(int32_t out_f, int32_t in_f, int32_t batch) {
  QMLA_REQUIRE(out_f >= 0 && in_f >= 0 && batch >= 0, QMLA_ERR_SHAPE,
               "negative size (out_features %d, in_features %d, batch %d)", out_f, in_f, batch);
  QMLA_REQUIRE(in_f <= kMaxK, QMLA_ERR_UNSUPPORTED, "in_features %d above %d", in_f, kMaxK);
  return QMLA_OK;
}

struct MoeWs {
  size_t sel, selw, ebin, slots, xmax, logits, hmax, h, y, total;
};

MoeWs moe_ws(const qmla_moe_config &c, int32_t T) {
  const int64_t P = (int64_t)T * c.top_k;
  const int64_t H = c.hidden_dim, I = c.intermediate_dim;
  MoeWs w{};
  size_t o = 0;
  auto take = [&](size_t bytes) {
    const size_t at = o;
    o += align256(bytes);
    return at;
  };
  w.sel = take(sizeof(int32_t) * P);
  w.selw = take(sizeof(float) * P);
  w.ebin = take(sizeof(int2) * c.num_experts);
  w.slots = take(sizeof(int32_t) * P);
  w.xmax = take(sizeof(uint32_t) * T);
  w.logits = take(sizeof(float) * T * c.num_experts);
  w.hmax = take(sizeof(uint32_t) * P * mfma_row_blocks(I));
  w.h = take(sizeof(float) * P * I);
  w.y = take(sizeof(float) * P * H);
  w.total = o;
  return w;
}

qmla_status check_moe(const qmla_moe_config *c, int32_t T) {
  QMLA_REQUIRE(c != nullptr, QMLA_ERR_INVALID_ARG, "config is null");
  QMLA_REQUIRE(T >= 0 && c->num_experts >= 0 && c->top_k >= 0 && c->hidden_dim > 0 &&
                   c->intermediate_dim > 0,
               QMLA_ERR_SHAPE, "bad sizes (seq %d, experts %d, top_k %d, hidden %d, inter %d)", T,
               c->num_experts, c->top_k, c->hidden_dim, c->intermediate_dim);
  QMLA_REQUIRE(c->top_k <= c->num_experts || c->num_experts == 0, QMLA_ERR_SHAPE,
               "top_k %d above num_experts %d", c->top_k, c->num_experts);
  QMLA_REQUIRE(c->num_experts <= kMaxExperts, QMLA_ERR_UNSUPPORTED, "num_experts %d above %d",
               c->num_experts, kMaxExperts);
  QMLA_REQUIRE(c->hidden_dim <= kMaxK && c->intermediate_dim <= kMaxK, QMLA_ERR_UNSUPPORTED,
               "hidden/intermediate above %d", kMaxK);
  QMLA_REQUIRE((int64_t)T * c->top_k <= (int64_t)1 << 30, QMLA_ERR_UNSUPPORTED,
               "seq_len x top_k too large");
  return QMLA_OK;
}

}  // namespace
}  // namespace qmla

using namespace qmla;

extern "C" {

qmla_status qmla_packed_forward_workspace_bytes(int32_t out_features, int32_t in_features,
                                                int32_t batch, size_t *bytes) {
  clear_error();
  QMLA_REQUIRE(bytes != nullptr, QMLA_ERR_INVALID_ARG, "bytes is null");
  QMLA_TRY(check_packed_dims(out_features, in_features, batch));
  *bytes = 0;  // every kernel works in registers and LDS
  return QMLA_OK;
}

qmla_status qmla_packed_forward(const uint8_t *packed, const float *scales, int32_t out_features,
                                int32_t in_features, const float *x, int32_t batch, float *out,
                                void *workspace, size_t workspace_bytes, qmla_stream stream) {
  clear_error();
  (void)workspace;
  (void)workspace_bytes;
  QMLA_TRY(check_packed_dims(out_features, in_features, batch));
  if (out_features == 0 || batch == 0) return QMLA_OK;
  QMLA_REQUIRE(packed != nullptr || in_features < 4, QMLA_ERR_INVALID_ARG, "packed is null");
  QMLA_REQUIRE(scales != nullptr && x != nullptr && out != nullptr, QMLA_ERR_INVALID_ARG,
               "null pointer argument");
  PackedArgs a{};
  a.w[0] = a.w[1] = packed;
  a.scale[0] = a.scale[1] = scales;
  a.M = out_features;
  a.K = in_features;
  a.x = x;
  a.ld_x = in_features;
  a.src_div = 1;
  a.count = batch;
  a.out = out;
  a.ld_out = out_features;
  const bool mfma = mfma_ok(in_features) && aligned16(packed) && aligned16(x);
  return launch_packed<1>(a, ((int64_t)batch + kTokTile - 1) / kTokTile, mfma, as_stream(stream));
}

qmla_status qmla_moe_workspace_bytes(const qmla_moe_config *cfg, int32_t seq_len, size_t *bytes) {
  clear_error();
  QMLA_REQUIRE(bytes != nullptr, QMLA_ERR_INVALID_ARG, "bytes is null");
  QMLA_TRY(check_moe(cfg, seq_len));
  *bytes = moe_ws(*cfg, seq_len).total;
  return QMLA_OK;
}

qmla_status qmla_moe_forward(const qmla_moe_config *cfg, const float *xs, int32_t seq_len,
                             const float *gate_weight, const uint8_t *gate_packed,
                             const float *gate_scales, const uint8_t *up_packed,
                             const float *up_scales, const uint8_t *down_packed,
                             const float *down_scales, float *out, int32_t *top_experts,
                             float *top_weights, void *workspace, size_t workspace_bytes,
                             qmla_stream stream) {
  clear_error();
  QMLA_TRY(check_moe(cfg, seq_len));
  const qmla_moe_config c = *cfg;
  const int32_t T = seq_len, H = c.hidden_dim, I = c.intermediate_dim;
  if (T == 0) return QMLA_OK;
  QMLA_REQUIRE(xs != nullptr && out != nullptr, QMLA_ERR_INVALID_ARG, "xs or out is null");
  const hipStream_t s = as_stream(stream);
  const int64_t n_out = (int64_t)T * H;
  if (c.num_experts == 0 || c.top_k == 0) {  // src/moe.rs:46-48 (no expert adds anything)
    hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)((n_out + 255) / 256)), dim3(256), 0, s, out,
                       n_out);
    QMLA_LAUNCH_CHECK("k_fill_zero");
    return QMLA_OK;
  }
  QMLA_REQUIRE(gate_weight && gate_packed && gate_scales && up_packed && up_scales &&
                   down_packed && down_scales,
               QMLA_ERR_INVALID_ARG, "null weight pointer");
  const MoeWs w = moe_ws(c, T);
  QMLA_REQUIRE(workspace != nullptr && workspace_bytes >= w.total, QMLA_ERR_WORKSPACE,
               "workspace of %zu bytes, %zu needed", workspace_bytes, w.total);
  char *ws = static_cast<char *>(workspace);
  auto at = [&](size_t off) { return static_cast<void *>(ws + off); };
  int32_t *sel = static_cast<int32_t *>(at(w.sel));
  float *selw = static_cast<float *>(at(w.selw));
  int2 *ebin = static_cast<int2 *>(at(w.ebin));
  int32_t *slots = static_cast<int32_t *>(at(w.slots));
  float *hbuf = static_cast<float *>(at(w.h));
  float *ybuf = static_cast<float *>(at(w.y));
  const int32_t P = T * c.top_k;

  uint32_t *xmax = static_cast<uint32_t *>(at(w.xmax));
  uint32_t *hmax = static_cast<uint32_t *>(at(w.hmax));
  float *logits = static_cast<float *>(at(w.logits));
  const bool fast_gu = mfma_ok(H) && aligned16(gate_packed) && aligned16(up_packed) &&
                       aligned16(xs);
  const bool fast_dn = mfma_ok(I) && aligned16(down_packed) && aligned16(hbuf);
  // The MFMA GEMV blocks read their expert's bin from the routing table
  // themselves; the per-row fallback walks prebuilt bins.
  const bool block_bins = fast_gu && fast_dn;
  // Decode-sized calls (the logits fit the blocks' LDS table): only the
  // logits are computed up front, over a wide grid, and the gate/up blocks
  // rank the experts and write the routing table.  Otherwise one block per
  // token computes logits, ranks and weights.
  const bool rank_in_gemv =
      block_bins && T <= kRankTokens && (int64_t)T * c.num_experts <= kSelLds;
  if (rank_in_gemv) {
    hipLaunchKernelGGL(k_moe_logits, dim3((unsigned)((c.num_experts + 3) / 4), (unsigned)T),
                       dim3(256), 0, s, xs, gate_weight, c.num_experts, H, logits, xmax);
    QMLA_LAUNCH_CHECK("k_moe_logits");
  } else {
    hipLaunchKernelGGL(k_moe_route, dim3(T), dim3(1024), 0, s, xs, gate_weight, c.num_experts, H,
                       c.top_k, sel, selw, top_experts, top_weights, xmax);
    QMLA_LAUNCH_CHECK("k_moe_route");
  }
  if (!block_bins) {
    hipLaunchKernelGGL(k_moe_bin, dim3(1), dim3(1024), 0, s, sel, P, c.num_experts, ebin, slots);
    QMLA_LAUNCH_CHECK("k_moe_bin");
  }
  PackedArgs gu{};
  gu.w[0] = gate_packed;
  gu.w[1] = up_packed;
  gu.scale[0] = gate_scales;
  gu.scale[1] = up_scales;
  gu.w_stride = (int64_t)I * (H / 4);
  gu.s_stride = I;
  gu.M = I;
  gu.K = H;
  gu.x = xs;
  gu.ld_x = H;
  gu.src_div = c.top_k;
  gu.ebin = block_bins ? nullptr : ebin;
  gu.slots = block_bins ? nullptr : slots;
  gu.sel = block_bins && !rank_in_gemv ? sel : nullptr;
  gu.npairs = P;
  if (rank_in_gemv) {
    gu.logits = logits;
    gu.n_experts = c.num_experts;
    gu.topk = c.top_k;
    gu.sel_out = sel;
    gu.selw_out = selw;
    gu.user_idx = top_experts;
    gu.user_w = top_weights;
  }
  gu.out = hbuf;
  gu.ld_out = I;
  gu.src_max = xmax;
  gu.src_max_parts = 1;
  gu.out_max = fast_gu && fast_dn ? hmax : nullptr;
  // Split each expert's bin over `slices` blocks when the pairs outnumber
  // the experts' first tiles (prefill-sized calls, skewed routing); a
  // decode-sized call keeps one block per expert and row block.
  {
    const int64_t tiles = ((int64_t)P + kTokTile - 1) / kTokTile;
    int64_t sl = (tiles + c.num_experts - 1) / c.num_experts;
    sl = std::max<int64_t>(1, std::min<int64_t>({sl, kMaxSlices, kMaxTileGrid / c.num_experts}));
    gu.slices = (int32_t)sl;
  }
  QMLA_REQUIRE(gu.slices >= 1, QMLA_ERR_SHAPE, "bin slices");
  QMLA_TRY(launch_packed<2>(gu, (int64_t)c.num_experts * gu.slices, fast_gu, s));

  PackedArgs dn = gu;
  // the down GEMV reads the routing table the gate/up launch completed
  dn.sel = block_bins ? sel : nullptr;
  dn.logits = nullptr;
  dn.sel_out = nullptr;
  dn.selw_out = nullptr;
  dn.user_idx = nullptr;
  dn.user_w = nullptr;
  dn.w[0] = dn.w[1] = down_packed;
  dn.scale[0] = dn.scale[1] = down_scales;
  dn.w_stride = (int64_t)H * (I / 4);
  dn.s_stride = H;
  dn.M = H;
  dn.K = I;
  dn.x = hbuf;
  dn.ld_x = I;
  dn.src_div = 1;
  dn.out = ybuf;
  dn.ld_out = H;
  dn.src_max = fast_gu && fast_dn ? hmax : nullptr;
  dn.src_max_parts = mfma_row_blocks(I);
  dn.out_max = nullptr;
  QMLA_TRY(launch_packed<1>(dn, (int64_t)c.num_experts * dn.slices, fast_dn, s));

  hipLaunchKernelGGL(k_moe_combine, dim3((unsigned)((n_out + 255) / 256)), dim3(256), 0, s, ybuf,
                     sel, selw, T, c.top_k, H, out);
  QMLA_LAUNCH_CHECK("k_moe_combine");
  return QMLA_OK;
}

}  // extern "C"
