// internal.hpp -- objects shared between the translation units of libqmla.
#pragma once

#include <vector>

#include "common.hpp"

namespace qmla {

// Block table of a paged latent cache: token t of sequence s is row
// t & (2^shift - 1) of page pages[s * width + (t >> shift)] (a device
// address).  Pages hold 2^shift rows, a multiple of the 32-token tile of the
// MFMA decode, so a tile that starts at a multiple of 32 lies in one page.
struct PageTable {
  const uint64_t *pages;  // device [sequences][width]
  int32_t width;
  int32_t shift;
  __device__ __forceinline__ uint8_t *row(int32_t seq, int64_t t, int64_t row_bytes) const {
    const uint64_t page = pages[(int64_t)seq * width + (t >> shift)];
    return reinterpret_cast<uint8_t *>(page) + (t & ((int64_t(1) << shift) - 1)) * row_bytes;
  }
};

}  // namespace qmla

// Latent KV cache: one row [c_kv | k_pe] per token in pages of page_rows
// rows taken from HBM chunks; sequence i owns the pages listed in its block
// table row, h_npages[i] of them.  Lengths and the table are kept on the
// device (read by kernels) and mirrored on the host (validation and page
// bookkeeping without a device sync).
struct qmla_kv_cache {
  int device = 0;
  int32_t num_seqs = 0;
  int32_t r = 0;
  int32_t dr = 0;
  qmla_dtype dtype = QMLA_F32;
  int64_t row_elems = 0;
  int32_t page_rows = 0;
  int32_t page_shift = 0;
  int32_t table_width = 0;       // pages one sequence can hold
  uint64_t *d_pages = nullptr;   // device [num_seqs][table_width] page addresses
  int32_t *d_lens = nullptr;     // device [num_seqs]
  int32_t *d_cap = nullptr;      // device [num_seqs]
  std::vector<uint64_t> h_pages;
  std::vector<int32_t> h_npages;
  std::vector<int32_t> h_lens;
  std::vector<int32_t> h_cap;    // capacity (rows), <= h_npages * page_rows
  std::vector<void *> chunks;    // HBM chunks the pages come from
  int64_t pool_pages = 0;        // pages over all chunks
  std::vector<uint64_t> free_pages;  // unowned pages (taken from the back)
  // Layout at creation: chunks[0] holds every sequence's pages in order,
  // sequence i from row offset h_offsets[i].  Holds while `contiguous`.
  int64_t total_rows = 0;        // rows of chunks[0]
  int64_t *d_offsets = nullptr;  // device [num_seqs]
  std::vector<int64_t> h_offsets;
  bool contiguous = true;
  bool grow = false;  // appends past capacity take more pages instead of failing

  size_t elem_bytes() const { return dtype == QMLA_BF16 ? 2 : 4; }
  size_t row_bytes() const { return (size_t)row_elems * elem_bytes(); }
  size_t page_bytes() const { return (size_t)page_rows * row_bytes(); }
  qmla::PageTable table() const { return qmla::PageTable{d_pages, table_width, page_shift}; }
};

namespace qmla {

inline bool valid_dtype(qmla_dtype d) { return d == QMLA_F32 || d == QMLA_BF16; }
inline size_t dtype_bytes(qmla_dtype d) { return d == QMLA_BF16 ? 2 : 4; }

// Zeroes `bytes` bytes at dst (any alignment) with a kernel on stream s.
// Used instead of hipMemsetAsync wherever a caller may capture the call
// into a HIP graph: a kernel node replays exactly as recorded.
qmla_status zero_bytes(void *dst, size_t bytes, hipStream_t s);

// ------------------------------------------------------------ decode plan
// The token range of sequences 0..batch-1 (concatenated, N tokens) is cut
// into `blocks` contiguous pieces of `chunk` tokens (the last one takes the
// remainder).  A piece may cover parts of several sequences; each (piece,
// sequence) overlap is a segment with its own partial-result slot.
struct DecodeSegment {
  int32_t seq;
  int32_t t0;    // first token (sequence-relative)
  int32_t t1;    // one past the last token
  int32_t slot;  // partial slot, or -1 when the segment is its sequence's only one
};

struct DecodePlanView {
  int32_t *seg_start;      // [blocks + 1] first segment of each piece
  DecodeSegment *segs;     // [blocks + batch]
  int32_t *seq_slot_base;  // [batch]
  int32_t *seq_nslots;     // [batch] 0 (empty), 1 (written directly), >= 2 (merge)
};

// Workspace layout for a decode call with `blocks` pieces:
//   plan (seg_start, segs, seq tables), then slots x rows x r f32 partial
//   outputs and slots x rows f32 partial log-sum-exp.
// The bf16 MFMA path plans inside its kernel: instead of the plan it keeps
// per-sequence {first slot, slot count} (int2 x batch), and its partial rows
// are padded to a multiple of 32 (fragment-major layout, see decode_mfma).
struct DecodeWorkspace {
  size_t plan_bytes = 0;
  size_t part_o_off = 0;
  size_t part_lse_off = 0;
  size_t total = 0;
  int32_t slots = 0;
};

DecodeWorkspace decode_workspace_layout(int32_t batch, int32_t rows, int32_t r, int32_t blocks,
                                        bool mfma);
DecodePlanView decode_plan_view(void *ws, int32_t batch, int32_t blocks);

qmla_status launch_decode_plan(const qmla_kv_cache *cache, int32_t pending, int32_t batch,
                               int32_t blocks, int32_t chunk, DecodePlanView plan,
                               hipStream_t stream);
// The decode of qmla_decode_absorbed[_splits] with `pending` tokens per
// sequence already written past the device lengths (see DecodeArgs); with
// `advance` the lengths grow by `pending` once the merge has run.  The
// caller has validated the shapes; the host length mirror is the caller's.
qmla_status decode_launch(const qmla_decode_dims *d, const qmla_kv_cache *c, qmla_dtype q_dtype,
                          const void *q_latent, const void *q_rope, double scale, float *out,
                          float *out_lse, int32_t splits, void *ws, size_t ws_bytes,
                          int32_t pending, bool advance, hipStream_t stream);
qmla_status launch_decode_merge(int32_t batch, int32_t rows, int32_t r, DecodePlanView plan,
                                const float *part_o, const float *part_lse, float *out,
                                float *out_lse, int32_t *adv_lens, int32_t adv,
                                hipStream_t stream);

// Attention cores (decode_f32.hip / decode_mfma.hip).
struct DecodeArgs {
  const qmla_kv_cache *cache;
  int32_t batch, rows, r, dr;
  const void *q_lat;  // [batch, rows, r]  f32 or bf16 (q_dtype)
  const void *q_rope; // [batch, rows, dr]
  qmla_dtype q_dtype;
  float scale;
  float *out;         // [batch, rows, r]
  float *out_lse;     // [batch, rows] or null
  DecodePlanView plan;  // f32 path
  int2 *seq_info;       // MFMA path: [batch] {first slot, slot count}
  float *part_o;
  float *part_lse;
  int32_t blocks;
  // Tokens already written past each of the batch's device lengths (the
  // layer's new rows): the decode attends lens + pending tokens, and with
  // `advance` the merge then adds pending to the lengths.
  int32_t pending;
  bool advance;
};
// Largest batch and piece count one decode call plans for.
constexpr int32_t kMaxPlanBatch = 8192;
constexpr int32_t kMaxPlanBlocks = 8192;
qmla_status launch_decode_f32(const DecodeArgs &a, hipStream_t stream);
qmla_status launch_decode_mfma(const DecodeArgs &a, hipStream_t stream);
bool decode_mfma_supported(int32_t rows, int32_t r, int32_t dr);
// Whether a decode with `rows` query rows per sequence over cache `c` has a
// core (bf16 MFMA shapes, f32 width and row limits); checks no lengths.
qmla_status decode_shape_supported(const qmla_kv_cache *c, int32_t rows);
// Pieces per compute unit the MFMA decode kernel runs concurrently.
bool decode_narrow_path(int32_t rows, int32_t r, int32_t dr);
int decode_mfma_blocks_per_cu(int32_t rows, int32_t r, int32_t dr);
int32_t decode_mfma_seg_tokens(int32_t rows, int32_t r, int32_t dr);

// Prefill attention (prefill_*.hip).
qmla_status launch_prefill_f32(const qmla_prefill_dims &d, const float *q_nope,
                               const float *q_rope, const float *k, const float *k_rope,
                               const float *v, float scale, int causal, float *out,
                               hipStream_t stream);
// (dn, dr, dv) combinations the bf16 MFMA prefill takes.
bool prefill_bf16_supported(int dn, int dr, int dv);
// Shapes whose bf16 prefill can write the context as records (below).
bool prefill_bf16_records_supported(int dn, int dr, int dv);
// With out_records, out receives the context as the split GEMM's activation
// records of the rows [b s][H dv] (hi halves only; dv 128, seq_q % 32 == 0)
// instead of [b, H, s, dv].
qmla_status launch_prefill_bf16(const qmla_prefill_dims &d, const uint16_t *q_nope,
                                const uint16_t *q_rope, const uint16_t *k,
                                const uint16_t *k_rope, const uint16_t *v, float scale,
                                int causal, uint16_t *out, hipStream_t stream,
                                int out_records = 0);

// Skinny projections (skinny_gemm.hip): y[m][n] = sum_k x[m][k] W[n][k]
// (+ bias[n]) for M <= 32 token rows, per z (a head) with z-strides; W in
// the fragment-major bf16 hi/lo layout of skinny_pack.  Epilogue modes:
constexpr int kSkinnyFinal = 0;  // y[z sy + m ldy + n]
constexpr int kSkinnyQkv = 1;    // [q_proj | kv_a_proj_with_mqa] -> q_nope, roped q_rope, kva
constexpr int kSkinnyPackB = 2;  // y: the next product's B operand, k = z sy + n (2 KB per 16 k)
struct SkinnyGemmArgs {
  const void *w_frag;  // fragment-major bf16 hi/lo weights (skinny_pack)
  const float *x;      // [Z][M][K]: row stride ldx, z-stride sx; or, with
  int64_t ldx, sx;     // x_packed, a PACKB output (Z = 1)
  bool x_packed;
  const float *bias;   // [Z][N], z-stride sb, or null
  int64_t sb;
  float *y;            // FINAL: [Z][M][N], row stride ldy, z-stride sy
  int64_t ldy, sy;
  int M, N, K, Z;
  int mode;
  // QKV: token m of this launch is token m0 + m of the call, sequence
  // (m0 + m) / seq, position lens[seq] + (m0 + m) % seq.
  int m0, seq, heads, dn, dr;
  float *q_nope;  // [tokens][heads][dn]
  float *q_rope;  // [tokens][heads][dr]
  float *kva;     // [tokens][kva_ld]
  int64_t kva_ld;
  const int32_t *lens;
  const float *inv_freq;
  float mscale;
  // K split over `groups` (1, 2, 4 or 8) blocks per 32-output tile; group 0
  // adds the bias.  QKV (2 groups): group 1 writes its half to q_nope1,
  // q_rope1 and kva1, and the consumers add the two halves.  FINAL: group g
  // writes its partial sums to y + g sgrp, and the caller adds the planes.
  int groups;
  float *q_nope1, *q_rope1, *kva1;
  int64_t sgrp;
  // optional second plane of x (f32, x's strides): the operand is x + x2
  const float *x2;
  // Optional elementwise work spread over the product's blocks (about one
  // element per thread): add_dst[i] += add_src[i] for i < add_n.
  float *add_dst;
  const float *add_src;
  int64_t add_n;
  // bf16 operands: the weights' hi halves and bf16(x), one MFMA per step
  // (a PACKB output then carries its hi halves only)
  int bf16ops;
};
struct LatentRowsArgs;
int skinny_waves(int K);
// Fragment-major hi/lo packing of W [Z][N][K] (row stride ldw, z-stride sw,
// f32, host memory) into out (skinny_frag_bytes(N, K, Z) bytes).
size_t skinny_frag_bytes(int N, int K, int Z);
void skinny_pack(const float *W, int64_t ldw, int64_t sw, int N, int K, int Z, uint8_t *out);
bool skinny_supported(int M, int K);
// With `rows`, the launch also writes the latent cache rows of n_rows new
// tokens (latent_rows.hpp) in extra blocks.
qmla_status launch_skinny_gemm(const SkinnyGemmArgs &a, hipStream_t stream,
                               const LatentRowsArgs *rows = nullptr, int n_rows = 0);

// Projections of many token rows (split_gemm.hip): y[m][n] = sum_k x[m][k]
// W[n][k] + bias[n], W in the fragment-major layout of skinny_pack (Z = 1),
// f32-exact on bf16 MFMA.  Epilogue modes:
constexpr int kSgEpiFinal = 0;  // y[m ldy + n], f32
constexpr int kSgEpiQkv = 1;    // [q_proj | kv_a]: out0 = q_nope, out1 = roped q_rope
                                //   ([b, H, s, d], bf16 or f32), kva f32 rows
constexpr int kSgEpiKvb = 2;    // kv_b_proj: out0 = k [b, H, s, dn], out1 = v [b, H, s, dv]
struct SplitGemmArgs {
  const void *w_frag;  // fragment-major bf16 hi/lo records of W [N][K]
  int M, N, K;
  // x: f32 rows x[m ldx + k] (x_heads = 0), or the attention context
  // [b, heads, seq, dv] as rows [b seq][heads dv] (x_heads = 1; bf16 when
  // x_bf16, else f32)
  const void *x;
  int64_t ldx;
  int x_heads, x_bf16;
  const float *bias;  // [N] or null
  int epi;
  float *y;           // FINAL
  int64_t ldy;
  int out_bf16;       // QKV / KVB outputs in bf16 (else f32)
  // row m is token s = m % seq of sequence b = m / seq
  int seq, heads, dn, dr, dv;
  void *out0, *out1;
  float *kva;         // QKV: kv_a rows [M][kva_ld]
  int64_t kva_ld;
  const int32_t *lens;     // QKV: token s of sequence b sits at position lens[b] + s
  const float *inv_freq;   // [dr / 2]
  float mscale;
  // split-K: ksplit slices of K each write raw partial sums part[z][M][N]
  // (f32), which a second launch adds in slice order before the epilogue
  int ksplit;
  float *part;
  // bf16 operands: the weights' and activations' hi halves only (records of
  // 1 KB, no lo halves), one MFMA per step, f32 accumulation
  int bf16ops;
};
bool split_gemm_supported(int N, int K);
// K slices the split GEMM uses for an M x N x K product (1 when its tiles
// already fill the device), and the partial-sum bytes they need.
int split_gemm_slices(int M, int N, int K);
size_t split_gemm_part_bytes(int M, int N, int K);
// Rows from which the split GEMM runs its 256 x 256 tiles, and below which
// the layer keeps its rocBLAS path (few rows stream the weights; the split
// GEMM's tiles would leave most of the device idle).
constexpr int kSplitGemmBigRows = 4096;
constexpr int kSplitGemmMinRows = 128;
// Scratch for the activation records of an [M][K] product.
size_t split_gemm_pack_bytes(int M, int K);
// Packs x into `pack` (split_gemm_pack_bytes(M, K) bytes), then runs the GEMM.
qmla_status launch_split_gemm(const SplitGemmArgs &a, void *pack, hipStream_t stream);
// The GEMM over activation records a producer already wrote (split_gemm_
// pack_bytes(M, K) bytes at most; a.x unused): hi | lo records of f32
// activations, or with hi_only (or a.bf16ops) hi-only records of 1 KB.
qmla_status launch_split_gemm_packed(const SplitGemmArgs &a, const void *xrec, hipStream_t stream,
                                     bool hi_only = false);

// Cache row writer shared by the cache API and the layer: copies/converts
// n_seqs x n_new rows (row-major [n_seqs, n_new, row_elems]) into sequences
// seq0 .. seq0 + n_seqs - 1 at their current device lengths, then advances
// those lengths by n_new.
qmla_status launch_cache_append(qmla_kv_cache *cache, const void *rows, qmla_dtype rows_dtype,
                                int32_t seq0, int32_t n_seqs, int32_t n_new, hipStream_t stream);
qmla_status check_append(const qmla_kv_cache *cache, int32_t seq0, int32_t n_seqs, int32_t n_new);
// Lengths of sequences seq0 .. seq0 + n_seqs - 1 grow by n_new (device
// table in stream order, host mirror now), after their rows were written.
qmla_status cache_advance(qmla_kv_cache *cache, int32_t seq0, int32_t n_seqs, int32_t n_new,
                          hipStream_t stream);
// check_append, after growing the sequences that need it when the cache's
// growth mode is on.
qmla_status make_room(qmla_kv_cache *cache, int32_t seq0, int32_t n_seqs, int32_t n_new,
                      hipStream_t stream);

}  // namespace qmla
