// Launch-side declarations of the det-path HIP kernels (gfx950).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace det {

// Weight storage of one det matrix on the device.
enum Storage : int { kInt8 = 8, kI16 = 16, kI32 = 32 };

struct DevMatrix {
  uint64_t rows = 0, cols = 0;
  int storage = kInt8;
  // int8 form, tile-major: 16-row tiles, each stored as kpad/128 steps of
  // 2048 bytes in the exact order one wavefront loads them (lane l = 16*g + i
  // holds row 16*tile + i, columns [128*step + 32*g, +32)). Rows are padded
  // to a multiple of 16 and columns to kpad (a multiple of 128) with zeros.
  // Per-row integer scale and row sum (sum of q) accompany it.
  uint64_t kpad = 0;
  int8_t* q = nullptr;
  int32_t* scale = nullptr;
  int32_t* rowsum = nullptr;
  // row sums over each column part of kLimbPartCols (the prefill GEMM's
  // limb decomposition is chosen per part): part p of row r at
  // rowsum_p[p * rowsum_p_ld + r]
  int32_t* rowsum_p = nullptr;
  uint64_t rowsum_p_ld = 0;
  // Digit planes: W[r][c] = scale[r] * sum_p 256^p d_p[r][c] with int8
  // digits d_p (planes = 1: the int8 form above). Plane p of tile t is the
  // virtual tile t * planes + p in the tile-major layout (each tile's planes
  // are consecutive, every plane kpad/128 tile-steps), so kernels read a
  // planes-digit matrix as an int8 matrix of planes * 16 rows per tile and
  // combine a row's planes with shifts of 8 p bits. rowsum is the row sum of
  // sum_p 256^p d_p (within int32 by the row-mass bound).
  int planes = 1;
  // width class of the uploaded values (8: factored int8 x scale, 16, 32)
  int value_width = 8;
  // wide form: w[rows][cols] as int16 or int32 Wgt bits.
  void* w = nullptr;
  bool owns = true;  // false for row-range views
};

// Columns per part of the prefill GEMM's per-part limb decomposition.
constexpr uint64_t kLimbPartCols = 256;
// More parts than this (K above 16384) take four limbs throughout.
constexpr uint64_t kLimbMaxParts = 64;
__host__ __device__ inline uint64_t limb_parts(uint64_t kpad) { return (kpad + kLimbPartCols - 1) / kLimbPartCols; }

// A view of rows [r0, r0+n) of a matrix (shares storage). For int8 storage
// r0 must be a multiple of 16 (tile aligned).
DevMatrix row_view(const DevMatrix& m, uint64_t r0, uint64_t n);
// Byte offset of q[r][c] in the tile-major int8 layout: 16-row tiles of
// 128-column steps (2 KB tile-steps). Columns [32g, 32g + 32) of tile row i
// are MFMA lane l = 16g + i's operand bytes; their first 16 sit at 16 l and
// the second 16 at kTileHalfBytes + 16 l, so each of a lane's two 16-byte
// operand loads reads one contiguous 1 KB half of the tile-step (64 lanes x
// 16 bytes); 32-byte-strided lane addresses stream from HBM about 9 % slower.
constexpr uint64_t kTileHalfBytes = 1024;
__host__ __device__ inline uint64_t tiled_offset(uint64_t kpad, uint64_t r, uint64_t c) {
  const uint64_t tile = r >> 4, i = r & 15, step = c >> 7, g = (c >> 5) & 3, h = (c >> 4) & 1, b = c & 15;
  return (tile * (kpad >> 7) + step) * 2048 + h * kTileHalfBytes + (g * 16 + i) * 16 + b;
}
// The virtual row of digit plane p of row r in a planes-digit matrix.
__host__ __device__ inline uint64_t digit_row(uint64_t r, int planes, int p) {
  return (((r >> 4) * uint64_t(planes) + uint64_t(p)) << 4) | (r & 15);
}

// Activation limb planes for the int8 path: for each token row, four int8
// planes of kpad bytes (byte j of a ^ 0x00808080, zero padded).
void launch_act_limbs(const int32_t* act, uint64_t m, uint64_t k, uint64_t ld_act, uint64_t kpad,
                      int8_t* limbs, hipStream_t s);

// out[t][n] = requantize(sum_k act[t][k] * W[n][k]) for t < m; the raw
// wrapped accumulators go to acc_out instead when it is non-null.
// `limbs` is scratch of at least m * 4 * kpad bytes (int8 path only).
void launch_linear(const DevMatrix& W, const int32_t* act, uint64_t m, uint64_t ld_act, int32_t* out,
                   uint64_t ld_out, int64_t* acc_out, int8_t* limbs, hipStream_t s);

// Int8 GEMM for a slab of m activation rows (prefill): the activations are
// first expanded into tiled limb rows in a_tiled (gemm_act_bytes(m, W.kpad)
// bytes), then 128 x 128 MFMA blocks accumulate exactly. Output as for
// launch_linear (requantized rows, or raw Q32.32 accumulators to acc_out).
uint64_t gemm_act_bytes(uint64_t m, uint64_t kpad);
// The two halves of launch_gemm, so one limb expansion can feed several
// matrices with the same input width.
void launch_gemm_limbs(const int32_t* act, uint64_t m, uint64_t k, uint64_t ld_act, uint64_t kpad, int8_t* a_tiled,
                       hipStream_t s);
// split: the rows of W go to three outputs (rows [0, r1) to out with stride
// ld_out, [r1, r2) to out1, [r2, rows) to out2, each requantized), e.g. the
// fused [q; k; v] projection into the q, k and v row buffers.
struct RowSplit {
  int32_t* out1 = nullptr;
  int32_t* out2 = nullptr;
  uint64_t ld1 = 0, ld2 = 0, r1 = 0, r2 = 0;
};
// K split of grids that leave CUs idle (small m): chunk c of the K range
// writes its wrapping Q32.32 share of every output to planes[c][m][rows]
// (gemm_plane_bytes(W, m) bytes; the wrapping sum of the chunks is the
// accumulator exactly), and a second kernel sums them into the outputs.
// planes == nullptr keeps the single pass.
struct KSplit {
  uint32_t chunks = 1;
  int64_t* planes = nullptr;
};
uint32_t gemm_kchunks(const DevMatrix& W, uint64_t m);
uint64_t gemm_plane_bytes(const DevMatrix& W, uint64_t m);
void launch_gemm_tiled(const DevMatrix& W, uint64_t m, int32_t* out, uint64_t ld_out, int64_t* acc_out,
                       const int8_t* a_tiled, hipStream_t s, const RowSplit* split = nullptr,
                       int64_t* planes = nullptr);
void launch_gemm(const DevMatrix& W, const int32_t* act, uint64_t m, uint64_t ld_act, int32_t* out, uint64_t ld_out,
                 int64_t* acc_out, int8_t* a_tiled, hipStream_t s, int64_t* planes = nullptr);
// The gate/up projection with the GELU product in the GEMM epilogue: W holds
// tiles of 8 gate rows followed by the matching 8 up rows (the decode step's
// interleaved gate/up matrix), and out[t][f] = mul_sat(gelu(gate_f), up_f)
// for f < W.rows / 2 (stride ld_out); a_tiled from launch_gemm_limbs.
void launch_gemm_tiled_gelu(const DevMatrix& W, uint64_t m, int32_t* out, uint64_t ld_out, const int8_t* a_tiled,
                            hipStream_t s);

// Batch-1 int8 GEMV for the fused decode step (int8 storage, fits LDS):
// act_i64 requantizes wrapped accumulators on load; epilogue 1 applies
// mul_sat(gelu(gate), up) to an interleaved gate/up matrix (out has rows/2);
// epilogue 2 writes mul_sat(gelu(row), mul[row]) (int32 activations only).
bool gemv_fits_lds(const DevMatrix& W, uint64_t m);
void launch_gemv_decode(const DevMatrix& W, const void* act, bool act_i64, int epilogue, int32_t* out,
                        hipStream_t s, const int32_t* mul = nullptr);
// Decode GEMV (one activation row) into wrapping Q32.32 accumulators that must
// be zero on entry; K is split across workgroups with exact atomic adds.
void launch_gemv_decode_acc(const DevMatrix& W, const void* act, bool act_i64, int64_t* acc, hipStream_t s);
// Whether launch_gemv_decode_acc writes W's accumulators with plain stores
// (complete rows, no zero needed on entry) rather than atomic partial sums.
bool gemv_decode_acc_plain(const DevMatrix& W);
// Decode GEMV from an activation given as limb planes (4 planes of W.kpad
// bytes). acc != null: wrapping Q32.32 sums added atomically (zero on entry);
// else requantized to out, or with epilogue 1 (interleaved gate/up matrix)
// out[f] = mul_sat(gelu(gate_f), up_f), also written as limb planes
// (stride out_kpad) to out_limbs.
void launch_gemv_dec(const DevMatrix& W, const int8_t* limbs, int32_t* out, int64_t* acc, int epilogue,
                     int8_t* out_limbs, uint64_t out_kpad, hipStream_t s);
// Operand-major limb layout of the batched decode GEMV (k_gemv_rega): the
// limbs of token t's row of kpad columns sit in the MFMA A operands that read
// them. Tokens go in passes of 16 (pass p = t / 16, slot s = t % 16); column
// c belongs to half-step hs = 2 (c / 128) + (c / 16) % 2, and limb j of it
// is byte c % 16 of lane 16 ((c / 32) % 4) + 4 (s % 4) + j's 16-byte operand
// of token group s / 4. A pass takes 64 kpad bytes (as many as 16 tokens'
// limb planes), every half-step 4 KB: 1 KB per token group, one contiguous
// wave load per operand.
__host__ __device__ inline uint64_t om_offset(uint64_t kpad, uint64_t t, uint64_t c, int j) {
  const uint64_t s = t & 15;
  const uint64_t hs = 2 * (c >> 7) + ((c >> 4) & 1);
  const uint64_t lane = 16 * ((c >> 5) & 3) + 4 * (s & 3) + uint64_t(j);
  return (((t >> 4) * (kpad >> 6) + hs) * 4 + (s >> 2)) * 1024 + lane * 16 + (c & 15);
}
// The same for ntok activation rows (token t: limb planes 4t..4t+3), every
// weight tile serving up to 16 tokens; token t's outputs go to
// out + t * out_ld, acc + t * acc_ld and planes 4t..4t+3 of out_limbs.
// limbs_om (optional): the same activations also in the operand-major layout,
// which passes of 5-16 tokens then read instead of the planes. out_om
// (epilogue 1, with out_limbs): the outputs' limbs are also written in that
// layout (stride out_kpad) by every pass of 5 or more tokens.
void launch_gemv_dec_batch(const DevMatrix& W, const int8_t* limbs, uint32_t ntok, int32_t* out, uint64_t out_ld,
                           int64_t* acc, uint64_t acc_ld, int epilogue, int8_t* out_limbs, uint64_t out_kpad,
                           hipStream_t s, const int8_t* limbs_om = nullptr, int8_t* out_om = nullptr);
// The same into Q32.32 accumulators (acc + t * acc_ld, added atomically)
// from activation rows given as wrapped Q32.32 accumulators (acc_in + t *
// in_ld, requantized on load): no limb planes in between. Applies when
// gemv_dec_batch_in64_ok: int8 or digit-plane weights with K a multiple of
// 128, in_ld even, at least 5 tokens in every pass of 16.
bool gemv_dec_batch_in64_ok(const DevMatrix& W, uint32_t ntok, uint64_t in_ld);
void launch_gemv_dec_batch_in64(const DevMatrix& W, const int64_t* acc_in, uint64_t in_ld, uint32_t ntok,
                                int64_t* acc, uint64_t acc_ld, hipStream_t s);

// The residual norm that precedes a batch-1 decode GEMV, computed by the GEMV
// itself: x' = add_sat(x_in, rmsnorm(requant(src)) * w_post) [* scalar], and
// the GEMV's input is rmsnorm(x') * w_next. x' goes to x_out (and row_out when
// set); x_out must not alias x_in. clear (optional) is zeroed by the launch.
// All arrays hold H values (16-byte aligned), H % 4 == 0.
struct DecNormIn {
  const int64_t* src = nullptr;  // complete Q32.32 accumulators of the sub-block output
  const int32_t* x_in = nullptr;
  const int32_t* w_post = nullptr;
  const int32_t* w_next = nullptr;
  int32_t* x_out = nullptr;
  int32_t* row_out = nullptr;
  int64_t* clear = nullptr;
  uint64_t clear_n = 0;
  uint64_t H = 0;
  int64_t eps = 0;
  int32_t scalar = 0;
  int has_scalar = 0;
};
// Whether W (int8, cols == H, K up to 4096, a few tiles per CU) fits the fused kernel.
bool gemv_norm_fits(const DevMatrix& W, uint64_t H);
// epilogue 0: Q32.32 accumulators to acc_out (plain stores); epilogue 1:
// interleaved gate/up matrix, out[f] = mul_sat(gelu(gate_f), up_f) and its
// limb planes (stride out_kpad) to out_limbs.
void launch_gemv_norm(const DecNormIn& ni, const DevMatrix& W, int epilogue, int64_t* acc_out, int32_t* out,
                      int8_t* out_limbs, uint64_t out_kpad, hipStream_t s);

void launch_rmsnorm(int32_t* x, uint64_t rows, uint64_t cols, uint64_t ld, const int32_t* w,
                    int64_t eps, hipStream_t s);
// dst = add_sat(rmsnorm(src), res) row by row (dst may equal src or res).
void launch_rmsnorm_add(int32_t* dst, const int32_t* src, const int32_t* res, uint64_t rows, uint64_t cols,
                        uint64_t ld, const int32_t* w, int64_t eps, hipStream_t s);
// dst = rmsnorm(src) row by row (dst may equal src).
// x = add_sat(rmsnorm(src) * w1, x); normed = rmsnorm(x) * w2 (one pass for
// rows of 2049-4096 columns, else the two launches above).
void launch_rmsnorm_add_norm(int32_t* x, const int32_t* src, int32_t* normed, uint64_t rows, uint64_t cols,
                             uint64_t ld, const int32_t* w1, const int32_t* w2, int64_t eps, hipStream_t s,
                             bool has_scalar = false, int32_t scalar = 0);
void launch_rmsnorm_to(int32_t* dst, const int32_t* src, uint64_t rows, uint64_t cols, uint64_t ld, const int32_t* w,
                       int64_t eps, hipStream_t s);
void launch_rope(int32_t* x, uint64_t rows, uint64_t ld, uint64_t heads, uint64_t head_dim,
                 uint64_t half, const int64_t* inv_freq, uint64_t pos0, uint64_t pos_step,
                 hipStream_t s);

// Per-query cache window for batched decode (one query per sequence).
struct AttnSeq {
  const int32_t* k;  // the sequence's cache rows
  const int32_t* v;
  uint64_t base;     // physical row of window row 0
  uint64_t wrap;     // ring capacity (window row r at (base + r) mod wrap), 0 for a linear cache
  uint64_t count;    // window rows
};

struct AttnArgs {
  const int32_t* q;  // query rows: q + t*q_ld + h*hd
  uint64_t q_ld;
  const int32_t* k;  // key rows: k + phys(r)*kv_ld + kvh*hd
  const int32_t* v;
  uint64_t kv_ld;
  uint64_t ring_start, ring_cap;  // phys(r) = ring_cap ? (ring_start + r) % ring_cap : r
  int32_t* out;  // out + t*out_ld + h*hd
  uint64_t out_ld;
  uint32_t hd, num_heads, groups;
  uint32_t n_queries;
  // rows for query t: [start_t, start_t + count_t) where, in causal mode,
  // end_t = t + 1 + causal_offset, start_t = window ? max(0, end_t - window) : 0,
  // both clamped to [0, avail); in fixed mode every query uses [fix_start, fix_start+fix_count).
  int causal;
  uint64_t window, causal_offset, avail;
  uint64_t fix_start, fix_count;
  // batched decode: query t uses seqs[t] (k, v, window) instead of the fields
  // above; fix_count then holds the longest window of the batch
  const AttnSeq* seqs;
  // work area for the MFMA form of causal attention (attn_mfma_bytes(*this)
  // bytes; without it the vector-ALU kernel runs)
  void* work;
  uint64_t work_bytes;
  // limb blocks already written into that work area by the producer of the
  // rows (attn_mfma_plan's qlimbs / klimbs): 1 the Q blocks, 2 the K blocks
  uint32_t split_done;
};
// Windows longer than kMaxAttentionRows are rejected by the callers.
constexpr uint64_t kMaxAttentionRows = 16000;
void launch_attention(const AttnArgs& a, hipStream_t s);

// Causal attention over a linear cache on int8 MFMA (attention.hip): the
// work area it needs (0 where it does not apply: ring caches, batched
// windows, head dims not a multiple of 64 or above 512, fewer than 16
// queries, unaligned rows), and the launch, false when it does not apply.
uint64_t attn_mfma_bytes(const AttnArgs& a);
bool launch_attention_mfma(const AttnArgs& a, void* work, uint64_t work_bytes, hipStream_t s);
struct AttnMfmaArgs;
// The MFMA form's layout of a.work (false where the form does not apply).
bool attn_mfma_plan(const AttnArgs& a, AttnMfmaArgs& m);
// MFMA operand limb blocks of Q / K rows (one 1 KB block per 16-row tile,
// 64-dim substep and limb: lane 16 g + i holds row i, dims [64 s + 16 g, +16)
// as bytes j of x ^ 0x808080, the four-limb split x = sum_j c_j 256^j + C4).
constexpr int64_t kAttnC4 = 8421504;
constexpr uint32_t kAttnOp = 1024;
// 16 consecutive values of a row -> limb j's 16 bytes as four words w[j][0..3]
// (byte j of x ^ 0x808080, four values per word) and the sum of x - C4
__device__ inline int64_t attn_split16(const int32_t (&x)[16], uint32_t (&w)[4][4]) {
  int64_t s = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int d = 0; d < 4; ++d) w[j][d] = 0;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const uint32_t u = uint32_t(x[e]) ^ 0x00808080u;
    s += int64_t(x[e]) - kAttnC4;
#pragma unroll
    for (int j = 0; j < 4; ++j) w[j][e >> 2] |= ((u >> (8 * j)) & 0xffu) << (8 * (e & 3));
  }
  return s;
}
struct AttnMfmaArgs {
  uint32_t hd, groups;
  uint64_t n_queries, avail, window, causal_offset;
  uint64_t nqt, nkt, nks, srow;  // query / key tiles of 16, key substeps of 64, score row stride
  int32_t* out;
  uint64_t out_ld;
  int8_t* qlimbs;
  int8_t* klimbs;
  int8_t* vlimbs;
  int64_t* qsum;
  int64_t* ksum;
  int64_t* vblk;
  int32_t* scores;
  int32_t* resid;
  uint32_t* argm;
};

// Elementwise ops (saturating Q16.16).
void launch_add_sat(int32_t* dst, const int32_t* src, uint64_t n, hipStream_t s);
void launch_gelu_mul(int32_t* gate, const int32_t* up, uint64_t n, hipStream_t s);
void launch_scale(int32_t* x, uint64_t n, int32_t scalar, hipStream_t s);
void launch_softcap(int32_t* x, uint64_t n, int32_t cap, hipStream_t s);

// Embedding-style gather: out[t][c] = mul_sat(Wgt(M[ids[t]][col0 + c]), scale).
// RoPE with one position per row (positions on the device).
void launch_rope_rows(int32_t* x, uint64_t rows, uint64_t ld, uint64_t heads, uint64_t hd, uint64_t half,
                      const int64_t* inv_freq, const uint64_t* positions, hipStream_t s);

// Head norms of M tokens' q / k / v rows and RoPE of the q and k rows in one
// launch (q: [M][nh * hd], k and v: [M][nkv * hd]; v may be null); the same
// results as launch_rmsnorm over each row set followed by launch_rope /
// launch_rope_rows. Returns false (nothing launched) for shapes it does not
// take: head dim above 512 or a rotation of more than 256 pairs.
constexpr uint32_t kHeadRopeMaxHalf = 256;
struct HeadNormRope {
  int32_t *q, *k, *v;
  const int32_t *q_gain, *k_gain;  // null: no gain
  uint32_t nh, nkv, hd, half;      // half: rotated pairs per head (0: no rotation)
  int64_t eps;
  const int64_t* inv_freq;
  uint64_t pos0;                   // token t at position pos0 + t, unless
  const uint64_t* positions;       // one device position per token
  // optional cache copies of the final k and v rows: token t >= kv_from to
  // row t % kv_cap (kv_ring) or t of kc / vc (row width nkv * hd)
  int32_t *kc = nullptr, *vc = nullptr;
  uint64_t kv_from = 0, kv_cap = 0;
  int kv_ring = 0;
  // optional MFMA attention operands of the final rows (attn_mfma_plan):
  // q rows to qlimbs / qsum (nqt tiles per head), k rows to klimbs / ksum
  // (nkt tiles per KV head); rows from m up to whole tiles are written as
  // zero blocks and zero sums
  int8_t *qlimbs = nullptr, *klimbs = nullptr;
  int64_t *qsum = nullptr, *ksum = nullptr;
  uint64_t nqt = 0, nkt = 0;
  uint64_t rows = 0;  // tokens with rows (the grid covers nqt * 16 when qlimbs is set)
};
bool launch_head_norm_rope(const HeadNormRope& a, uint64_t m, hipStream_t s);
// Row i of k and v (width w) to kdst[i] / vdst[i] (device arrays of row pointers).
void launch_kv_append(const int32_t* k, const int32_t* v, uint64_t w, uint64_t n, int32_t* const* kdst,
                      int32_t* const* vdst, hipStream_t s);
// out[r] = first index of the maximum of row r of x [rows][n]; scratch holds
// argmax_rows_scratch(rows, n) int64 keys.
uint64_t argmax_rows_scratch(uint64_t rows, uint64_t n);
void launch_argmax_rows(const int32_t* x, uint64_t rows, uint64_t n, int64_t* scratch, uint32_t* out, hipStream_t s);
void launch_gather_rows(const DevMatrix& M, const uint32_t* ids, uint64_t m, uint64_t col0,
                        uint64_t ncols, int32_t scale, int32_t* out, uint64_t ld_out, hipStream_t s,
                        uint64_t ids_stride = 1);

// First index of the maximum; `scratch` holds >= 2*ceil(n/1024) int64 values.
void launch_argmax(const int32_t* x, uint64_t n, int64_t* scratch, uint32_t* out, hipStream_t s);

}  // namespace det
