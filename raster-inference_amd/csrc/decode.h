// Fused batch-1 decode step (graph-captured) kernels for the det path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace det {

// Per-step values the captured decode graph reads from device memory.
struct StepState {
  uint64_t position;  // index of the token being decoded (number of tokens before it)
  uint32_t token;
  uint32_t pad;
};

// One RoPE inverse-frequency table; its cos/sin pairs for the step position
// occupy trig[2 * offset, 2 * (offset + pairs)).
struct RopeTable {
  const int64_t* inv_freq;
  uint32_t pairs, offset;
};

// One sequence's cache of one layer in a batched step.
struct DecSeqCache {
  int32_t* k;
  int32_t* v;
  uint64_t cap;
};

// Integer softmax statistics of one query head over its window
// (ops.rs:230-258): the first argmax, the exp sum with its reciprocal, and the
// residual ONE - sum(weights) that the argmax row's weight receives.
struct AttnStat {
  int32_t mx;     // maximum score
  uint32_t mi;    // window row of its first occurrence
  int64_t sum;    // sum of exp terms
  uint64_t rec;   // 2^96 / sum, 0 when the generic division is needed
  int32_t resid;  // added (saturating) to the weight of row mi
  int32_t pad;
};

// One decode step's attention for one layer: head norms, RoPE and KV append
// of the fused projection rows, then scores, integer softmax and weighted sums.
struct AttnDecArgs {
  int64_t* qkv;         // fused projection accumulators [q heads | k heads | v heads (if has_v)]; cleared here
  const int32_t* q_norm;
  const int32_t* k_norm;
  const int32_t* trig;  // this layer's (cos, sin) pairs at the step position
  int64_t eps;
  uint64_t rotary;
  int has_v;            // the projection has v rows (else k_eq_v: values are the un-gained key norms)
  int own_cache;        // 0: reads a donor's cache and the projection has query rows only
  int32_t* k;           // attention cache (own or donor) [cap][nkv*hd]
  int32_t* v;
  const StepState* st;
  uint64_t cap, window;
  uint64_t max_rows;  // row stride of the scores scratch (>= cap)
  int ring;
  uint32_t hd, nh, nkv;
  int32_t* scores;  // scratch [nh][max_rows]
  int64_t* acc;     // [nh][hd] wrapped weighted sums (requantized by the O projection)
  int scores_in_lds;  // the statistics kernel keeps G x lds_stride exp terms in LDS
  uint64_t lds_stride;  // LDS row stride of the kept terms (>= every window)
  int64_t* keys;        // [nh][key_chunks] argmax key of each kAttnScoreRows chunk of scores
  uint64_t key_chunks;  // >= max_rows / kAttnScoreRows
  AttnStat* stats;      // [nh]
  // Batched steps (grid z = sequence): caches[seq] replaces k, v and cap (cap
  // above then only sizes the grid), and st, trig, qkv, scores and acc advance
  // by one StepState and by the strides below per sequence.
  const DecSeqCache* caches;
  uint64_t trig_stride, qkv_stride, scores_stride, acc_stride, keys_stride, stats_stride;
  uint32_t nseq;
  // kAttnScoreRows chunks per scores / weighted-sum workgroup (1, 2 or 4; 0
  // picks by cache size). Any choice gives the same results.
  uint32_t rows_mul;
};

// Limits of the fused decode kernels.
constexpr uint32_t kDecMaxHeadDim = 512;
constexpr uint32_t kDecMaxGroup = 8;
constexpr uint64_t kDecMaxHidden = 15360;  // 1024 threads x 15 elements per single-workgroup row kernel
constexpr uint32_t kAttnScoreRows = 32;     // window rows per scores workgroup (512 threads)
constexpr uint32_t kAttnWsumRows = 32;      // window rows per softmax / weighted-sum workgroup

// The normalised rows are written as int32 (normed) and as limb planes
// (limbs, plane stride kpad) for the decode GEMV; with om (optional) also in
// the batched GEMV's operand-major layout (om_offset, row i = token i).
// With nseq > 1, sequence i uses st[i] and rows i of x, dec_in and normed
// (stride H) and limb planes 4i..4i+3 (stride kpad).
void launch_dec_embed(const DevMatrix& E, const StepState* st, int32_t scale, uint64_t H, int32_t* x, int32_t* dec_in,
                      const int32_t* w_in, int64_t eps, int32_t* normed, int8_t* limbs, uint64_t kpad, hipStream_t s,
                      uint32_t nseq = 1, int8_t* om = nullptr);
// x = add_sat(x_src, rmsnorm(requant(src), w_post)) [* scalar]; normed = rmsnorm(x, w_next);
// src (wrapping Q32.32 accumulators) is cleared after use. x_src defaults to
// x (in place). x_out (optional) receives a copy of the new x (row stride H
// per sequence).
// Without w_next, x_limbs also writes x's limb planes to limbs. om as for
// launch_dec_embed.
void launch_dec_residual_norm(int64_t* src, int32_t* x, int32_t* normed, const int32_t* w_post, bool has_scalar,
                              int32_t scalar, const int32_t* w_next, uint64_t H, int64_t eps, int8_t* limbs,
                              uint64_t kpad, hipStream_t s, uint32_t nseq = 1, int32_t* x_out = nullptr,
                              const int32_t* x_src = nullptr, bool x_limbs = false, int8_t* om = nullptr);
// Limb planes (plane stride kpad, 4 planes per row) of nseq int32 rows of k
// columns (row stride ld); with gate_in, of mul_sat(gelu(x), gate_in) per
// element (gate_in row stride in_ld): the per-layer input gate.
void launch_dec_row_limbs(const int32_t* x, uint64_t k, uint64_t ld, uint32_t nseq, int8_t* limbs, uint64_t kpad,
                          hipStream_t s, const int32_t* gate_in = nullptr, uint64_t in_ld = 0, int8_t* om = nullptr);
void launch_dec_attention(const AttnDecArgs& a, hipStream_t s);
// Whether launch_dec_attention runs the statistics as a separate pass.
bool dec_attention_split(const AttnDecArgs& a);
// part 0: head norms, RoPE, KV append and scores; part 1: softmax statistics;
// part 2: weights and weighted sums; part 3: parts 1 and 2 in one kernel whose
// workgroups each rebuild the statistics (for grids that fit the device once)
void launch_dec_attention_part(const AttnDecArgs& a, int part, hipStream_t s);
// Writes the step position and token and every RoPE table's cos/sin pairs at
// that position (trig: 2 * total_pairs int32).
void launch_dec_set_step(StepState* st, uint64_t position, uint32_t token, const RopeTable* tables, uint32_t ntables,
                         uint32_t total_pairs, int32_t* trig, hipStream_t s);
void launch_dec_softcap(int32_t* x, uint64_t n, int32_t cap, hipStream_t s);
// Batched steps: the cos/sin pairs of every RoPE table at each sequence's
// position st[i].position, into trig + i * 2 * total_pairs.
void launch_dec_set_trig(const StepState* st, uint32_t nseq, const RopeTable* tables, uint32_t ntables,
                         uint32_t total_pairs, int32_t* trig, hipStream_t s);
// Requantizes the wrapped weighted sums acc[t][0..k) (row stride ld) of nseq
// sequences into limb planes (token t: planes 4t..4t+3, stride kpad; zero
// past k) for the O projection GEMV, and clears acc.
void launch_dec_acc_limbs(int64_t* acc, uint64_t k, uint64_t ld, uint32_t nseq, int8_t* limbs, uint64_t kpad,
                          hipStream_t s);
// Up to kMaxRowPtrs device rows gathered into one buffer: row i (width[i]
// int32 values at src[i]) goes to dst + i * stride. Passed by value as the
// kernel argument, so no descriptor upload precedes the launch.
constexpr uint32_t kMaxRowPtrs = 128;
struct RowPtrs {
  const int32_t* src[kMaxRowPtrs];
  uint32_t width[kMaxRowPtrs];
  uint32_t n;
  uint32_t stride;
};
void launch_gather_row_ptrs(const RowPtrs& g, int32_t* dst, hipStream_t s);
// dst[i][0..w) = src[i * w ..] for i < n (device array of row pointers).
void launch_copy_rows(const int32_t* src, uint64_t w, uint64_t n, int32_t* const* dst, hipStream_t s);
// Writes `bytes` (a multiple of 8) of host data to device memory at dst by
// kernel arguments, 3.5 KB per launch: stream-ordered, nothing staged in
// host memory the device reads later.
void launch_set_bytes(void* dst, const void* src, size_t bytes, hipStream_t s);

}  // namespace det
