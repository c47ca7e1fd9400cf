// Fused batch-1 decode step kernels (decode_transition on MI355X).
//
// One decode step is a fixed kernel sequence that reads the step position and
// token from device memory, so the whole step is captured once as a HIP graph
// and replayed. KV rows live at canonical slots (token t at t % capacity for
// sliding-window rings, t for linear caches), so every window bound is a
// function of the position alone.
//
// Semantics follow det_layer_decode (det_kernels.rs:866-1133) exactly; every
// reduction is an integer reduction whose result does not depend on order.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <stdexcept>

#include "decode.h"
#include "det_arith.h"
#include "kernels.h"
#include "wave.h"

namespace det {

// Wavefront reductions (DPP; every lane gets the result).
__device__ __forceinline__ int64_t wsum_sat(int64_t v) { return wave_sum_sat64(v); }  // non-negative terms
__device__ __forceinline__ int64_t wsum_wrap(int64_t v) { return wave_sum_wrap64(v); }
__device__ __forceinline__ int64_t wmax(int64_t v) { return wave_max64(v); }

// rms scale (ops.rs:406-425) of a row spread over the block, from each
// thread's saturating partial sum of squares. The saturating sum of
// non-negative terms is min(total, i64::MAX) in any order. One wave reduces the
// wave partials and computes the scale once; it reaches the block through LDS.
template <int NT>
__device__ __forceinline__ int32_t blk_rms_scale(int64_t ss, uint64_t n, int64_t eps, int64_t* red, int32_t* bc) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  ss = wsum_sat(ss);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  if (wave == 0) {
    int64_t t = lane < NT / 64 ? red[lane] : 0;
    t = wsum_sat(t);
    if (lane == 0) *bc = rms_scale_from_sumsq(t, uint32_t(n), eps);
  }
  __syncthreads();
  return *bc;
}

__device__ __forceinline__ int32_t wgt_bits(const DevMatrix& M, uint64_t r, uint64_t c) {
  if (M.storage == kInt8) {
    uint32_t v = 0;
    for (int p = 0; p < M.planes; ++p) v += uint32_t(int32_t(M.q[tiled_offset(M.kpad, digit_row(r, M.planes, p), c)])) << (8 * p);
    return int32_t(v * uint32_t(M.scale[r]));
  }
  if (M.storage == kI16) return int32_t(static_cast<const int16_t*>(M.w)[r * M.cols + c]);
  return static_cast<const int32_t*>(M.w)[r * M.cols + c];
}

// Row kernels: one workgroup of NT threads, element c = tid + NT * e held in
// registers (e < EPT, so rows up to NT * EPT), every global read issued first.
// The normalised row is written as int32 and as the four limb planes (plane
// stride kpad) that the next decode GEMV reads; with om also in the batched
// GEMV's operand-major layout (om_offset, token t of the batch).
// The operand-major bytes of the workgroup's one token are staged in LDS
// (oms) in their global order: 64-byte chunk (hs, g) holds limbs 0-3 of
// columns 128 (hs / 2) + 32 g + 16 (hs % 2) + [0, 16), which om_offset puts
// in four consecutive 16-byte lane operands; om_flush then copies whole
// 16-byte pieces (scattered global byte stores were slower).
__device__ __forceinline__ void put_limbs(int8_t* limbs, uint64_t kpad, uint64_t c, int32_t v, uint8_t* oms) {
  const uint32_t u = uint32_t(v) ^ 0x00808080u;
#pragma unroll
  for (int j = 0; j < 4; ++j) limbs[j * kpad + c] = int8_t(uint8_t(u >> (8 * j)));
  if (oms) {
    const uint64_t q = ((2 * (c >> 7) + ((c >> 4) & 1)) * 4 + ((c >> 5) & 3)) * 64 + (c & 15);
#pragma unroll
    for (int j = 0; j < 4; ++j) oms[q + 16 * j] = uint8_t(u >> (8 * j));
  }
}
__device__ __forceinline__ void put_row(int32_t* row, int8_t* limbs, uint64_t kpad, uint64_t c, int32_t v,
                                        uint8_t* oms) {
  row[c] = v;
  put_limbs(limbs, kpad, c, v, oms);
}
// After the staging writes (every thread calls it): token t's operand-major
// bytes from oms to om.
template <int NT>
__device__ __forceinline__ void om_flush(const uint8_t* oms, int8_t* om, uint64_t kpad, uint64_t t) {
  __syncthreads();
  const uint64_t pieces = kpad / 4;  // 16-byte pieces: 4 limbs x kpad bytes
  for (uint64_t q = threadIdx.x; q < pieces; q += NT) {
    const uint64_t chunk = q >> 2, j = q & 3, hs = chunk >> 2, g = chunk & 3;
    const uint64_t c0 = 128 * (hs >> 1) + 32 * g + 16 * (hs & 1);
    *reinterpret_cast<int4*>(om + om_offset(kpad, t, c0, int(j))) = *reinterpret_cast<const int4*>(oms + q * 16);
  }
}

// Embed the step token (gemma/io.rs:2446-2518) and normalise it for layer 0.
template <int NT, int EPT>
__global__ __launch_bounds__(NT) void k_dec_embed(DevMatrix E, const StepState* __restrict__ st, int32_t scale,
                                                   uint64_t H, int32_t* __restrict__ x, int32_t* __restrict__ dec_in,
                                                   const int32_t* __restrict__ w_in, int64_t eps,
                                                   int32_t* __restrict__ normed, int8_t* __restrict__ limbs,
                                                   uint64_t kpad, int8_t* __restrict__ om) {
  __shared__ int64_t red[NT / 64];
  __shared__ int32_t bc;
  __shared__ __attribute__((aligned(16))) uint8_t oms_buf[4 * NT * EPT];
  uint8_t* oms = om ? oms_buf : nullptr;
  const uint32_t seq = blockIdx.y;
  x += uint64_t(seq) * H;
  dec_in += uint64_t(seq) * H;
  normed += uint64_t(seq) * H;
  limbs += uint64_t(seq) * 4 * kpad;
  const uint32_t tok = st[seq].token;
  int32_t v[EPT], w[EPT];
  int64_t ss = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const uint64_t c = threadIdx.x + uint64_t(NT) * e;
    const bool in = c < H;
    w[e] = in ? w_in[c] : 0;
    v[e] = in ? mul_sat(wgt_bits(E, tok, c), scale) : 0;
    if (in) {
      x[c] = v[e];
      dec_in[c] = v[e];
    }
    ss = add_sat64_nn(ss, sq_term(v[e]));
  }
  const int32_t sc = blk_rms_scale<NT>(ss, H, eps, red, &bc);
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const uint64_t c = threadIdx.x + uint64_t(NT) * e;
    if (c < H) put_row(normed, limbs, kpad, c, mul_sat(mul_sat(v[e], sc), w[e]), oms);
  }
  if (om) om_flush<NT>(oms, om, kpad, seq);
}

// Residual add of a normalised sub-block output, then the next input norm:
// x = add_sat(x_src, rmsnorm(requant(src), w_post)) (times the layer scalar at the end of a
// layer); normed = rmsnorm(x, w_next) (det_kernels.rs:1058-1075, 1108-1133).
// src holds the projection's wrapping accumulators and is cleared after use.
// x_src may equal x (each thread reads its elements before writing them).
// Without w_next only x is written (the next norm is left to a later kernel),
// and with x_limbs also x's limb planes (the input of a GEMV on x itself).
template <int NT, int EPT>
__global__ __launch_bounds__(NT) void k_dec_residual_norm(int64_t* __restrict__ src, const int32_t* x_src,
                                                           int32_t* x, int32_t* __restrict__ normed,
                                                           const int32_t* __restrict__ w_post, int has_scalar,
                                                           int32_t scalar, const int32_t* __restrict__ w_next,
                                                           uint64_t H, int64_t eps, int8_t* __restrict__ limbs,
                                                           uint64_t kpad, int32_t* __restrict__ x_out, int x_limbs,
                                                           int8_t* __restrict__ om) {
  __shared__ int64_t red[NT / 64];
  __shared__ int32_t bc;
  __shared__ __attribute__((aligned(16))) uint8_t oms_buf[4 * NT * EPT];
  uint8_t* oms = om ? oms_buf : nullptr;
  const uint32_t seq = blockIdx.y;
  src += uint64_t(seq) * H;
  x_src += uint64_t(seq) * H;
  x += uint64_t(seq) * H;
  normed += uint64_t(seq) * H;
  limbs += uint64_t(seq) * 4 * kpad;
  if (x_out) x_out += uint64_t(seq) * H;
  int32_t o[EPT], xv[EPT], wp[EPT], wn[EPT];
  int64_t ss = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const uint64_t c = threadIdx.x + uint64_t(NT) * e;
    const bool in = c < H;
    o[e] = in ? requant(src[c]) : 0;
    if (in) src[c] = 0;
    xv[e] = in ? x_src[c] : 0;
    wp[e] = in ? w_post[c] : 0;
    wn[e] = in && w_next ? w_next[c] : 0;
  }
#pragma unroll
  for (int e = 0; e < EPT; ++e) ss = add_sat64_nn(ss, sq_term(o[e]));
  const int32_t s1 = blk_rms_scale<NT>(ss, H, eps, red, &bc);
  ss = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const uint64_t c = threadIdx.x + uint64_t(NT) * e;
    int32_t v = add_sat(xv[e], mul_sat(mul_sat(o[e], s1), wp[e]));
    if (has_scalar) v = mul_sat(v, scalar);
    xv[e] = v;
    if (c < H) x[c] = v;
    if (x_out && c < H) x_out[c] = v;
    ss = add_sat64_nn(ss, sq_term(c < H ? v : 0));
  }
  if (!w_next) {  // uniform over the workgroup
    if (x_limbs)
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const uint64_t c = threadIdx.x + uint64_t(NT) * e;
        if (c < H) put_limbs(limbs, kpad, c, xv[e], oms);
      }
    if (x_limbs && om) om_flush<NT>(oms, om, kpad, seq);
    return;
  }
  const int32_t s2 = blk_rms_scale<NT>(ss, H, eps, red, &bc);
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const uint64_t c = threadIdx.x + uint64_t(NT) * e;
    if (c < H) put_row(normed, limbs, kpad, c, mul_sat(mul_sat(xv[e], s2), wn[e]), oms);
  }
  if (om) om_flush<NT>(oms, om, kpad, seq);
}

// Window of the attention cache at this step (cache_windows + key_start,
// det_kernels.rs:297-311, 1005-1008), from the canonical slot placement:
// window row j sits at slot base + j, wrapped once around a ring of cap slots.
// The step's own token is the last window row, at slot `slot`.
struct Window {
  uint64_t base, cnt, pos, slot;
};
__device__ __forceinline__ Window attn_window(const AttnDecArgs& a) {
  Window w;
  w.pos = a.st->position;
  const uint64_t n = w.pos + 1;
  const uint64_t len = a.ring ? (n < a.cap ? n : a.cap) : n;
  const uint64_t start = (a.ring && n > a.cap) ? n % a.cap : 0;
  const uint64_t ks = a.window ? (len > a.window ? len - a.window : 0) : 0;
  w.cnt = len - ks;
  w.base = start + ks;
  if (w.base >= a.cap) w.base -= a.cap;
  w.slot = a.ring ? w.pos % a.cap : w.pos;
  return w;
}
__device__ __forceinline__ uint64_t phys_row(const AttnDecArgs& a, const Window& w, uint64_t j) {
  const uint64_t p = w.base + j;
  return p >= a.cap ? p - a.cap : p;
}
// Argmax key of a score at window row j: larger score first, then smaller j
// (argmax_first order).
__device__ __forceinline__ int64_t score_key(int32_t score, uint64_t j) {
  return int64_t(uint64_t(int64_t(score)) << 32 | (0xffffffffull - j));
}

// One head row of the fused projection, normalised by one wavefront
// (det_kernels.rs:952-998): x = requant(acc) (the accumulators are read
// here and cleared later), y = rmsnorm(x) * gain; the un-gained norm goes to
// `plain` when given (k_eq_v values).
// A head row's accumulators and gains as one lane reads them (element
// lane + 64 k, k < MAXHD / 64), so that they can be fetched before other loads
// are issued. Every load goes to a clamped address (elements past hd re-read
// the last one and are masked to zero; without gains the row itself is read
// and masked), so that no load is predicated and the wait counts before the
// first use stay exact.
template <uint32_t MAXHD>
struct HeadRowIn {
  int64_t acc[MAXHD / 64];
  int32_t gain[MAXHD / 64];
};
template <uint32_t MAXHD>
__device__ __forceinline__ void load_head_row(const int64_t* __restrict__ src, uint32_t hd,
                                              const int32_t* __restrict__ gain, uint32_t lane, HeadRowIn<MAXHD>& in) {
  const int32_t* gp = gain ? gain : reinterpret_cast<const int32_t*>(src);
#pragma unroll
  for (int k = 0; k < int(MAXHD / 64); ++k) {
    const uint32_t d = lane + 64 * k;
    const uint32_t dc = d < hd ? d : hd - 1;
    in.acc[k] = src[dc];
    in.gain[k] = gp[dc];
  }
#pragma unroll
  for (int k = 0; k < int(MAXHD / 64); ++k) {
    const bool on = lane + 64 * k < hd;
    in.acc[k] = on ? in.acc[k] : 0;
    in.gain[k] = (on && gain) ? in.gain[k] : 0;
  }
}
template <uint32_t MAXHD, class DP, class PP>
__device__ __forceinline__ void norm_head_row(const HeadRowIn<MAXHD>& in, uint32_t hd, int64_t eps, bool has_gain,
                                              DP dst, PP plain, uint32_t lane) {
  constexpr int kPer = MAXHD / 64;
  int32_t xv[kPer];
  int64_t ss = 0;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    xv[k] = requant(in.acc[k]);  // zero past hd
    ss = add_sat64_nn(ss, sq_term(xv[k]));
  }
  ss = wsum_sat(ss);
  const int32_t sc = rms_scale_from_sumsq(ss, hd, eps);
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const uint32_t d = lane + 64 * k;
    if (d < hd) {
      const int32_t v = mul_sat(xv[k], sc);
      dst[d] = has_gain ? mul_sat(v, in.gain[k]) : v;
      if (plain) plain[d] = v;
    }
  }
}

// This workgroup's sequence view of a (possibly batched) launch: grid z picks
// the sequence, its cache and its slices of the per-step buffers.
// (The cache pointers may come from the per-sequence table, so the kernels
// access the caches through global_ptr.)
__device__ __forceinline__ void seq_view(AttnDecArgs& a) {
  const uint32_t seq = blockIdx.z;
  a.st += seq;
  a.trig += seq * a.trig_stride;
  a.qkv += seq * a.qkv_stride;
  a.scores += seq * a.scores_stride;
  a.acc += seq * a.acc_stride;
  a.keys += seq * a.keys_stride;
  a.stats += seq * a.stats_stride;
  if (a.caches) {
    const DecSeqCache c = a.caches[seq];
    a.k = c.k;
    a.v = c.v;
    a.cap = c.cap;
  }
}

// Scores of every query head of one KV head over P chunks of kAttnScoreRows
// window rows (ops.rs:318-333: wrapping dot product, requantized), 512
// threads. The
// workgroup first builds the normalised, rotated queries of its heads in LDS
// (one wavefront per head row); the workgroup whose rows include the step's
// own token also normalises and rotates the new key row, appends key and
// value rows to the cache at the canonical slot and scores that row from LDS.
// Sixteen lanes share one key row per chunk; the key rows of all P chunks are
// fetched at the start. Workgroup 0 also zeroes the heads' weighted-sum
// accumulators. The argmax key of every chunk goes to keys.
template <bool VEC, int P, uint32_t MAXHD, bool OH = false>
__global__ __launch_bounds__(512) void k_dec_attn_scores(AttnDecArgs a) {
  __shared__ int32_t ql[kDecMaxGroup * kDecMaxHeadDim];
  __shared__ int32_t kn[kDecMaxHeadDim];
  __shared__ int64_t ck[P][kDecMaxGroup][kAttnScoreRows];
  seq_view(a);
  // OH: one query head per workgroup (grid x = query head), else every query
  // head of KV head blockIdx.x: GW heads from h_first. Only the writer (the
  // first head's workgroup under OH) stores the new key and value rows.
  const uint32_t G = a.nh / a.nkv, hd = a.hd;
  const uint32_t kvh = OH ? blockIdx.x / G : blockIdx.x;
  const uint32_t GW = OH ? 1u : G, h_first = OH ? blockIdx.x : kvh * G;
  const bool writer = !OH || blockIdx.x % G == 0;
  // head-norm jobs: 0..GW-1 the queries, GW the new key, GW + 1 the new value
  // (the writer only).
  // This wave's first job's accumulators are read before anything else (the
  // key-row loads below would otherwise be waited for first); the key and
  // value rows are read even where this workgroup turns out not to hold the
  // step's own row, and then go unused.
  const uint32_t wv = threadIdx.x >> 6;
  const uint32_t njobs_max = GW + (a.own_cache ? ((a.has_v && writer) ? 2u : 1u) : 0u);
  HeadRowIn<MAXHD> pre;
  auto job_src = [&](uint32_t job) {
    return job < GW ? a.qkv + (uint64_t(h_first) + job) * hd
                    : a.qkv + (uint64_t(a.nh) + (job == GW ? 0 : a.nkv) + kvh) * hd;
  };
  auto job_gain = [&](uint32_t job) { return job < GW ? a.q_norm : (job == GW ? a.k_norm : nullptr); };
  const uint32_t pj = wv < njobs_max ? wv : 0;  // (idle waves read job 0's row and drop it)
  load_head_row(job_src(pj), hd, job_gain(pj), threadIdx.x & 63, pre);
  // cos/sin of this thread's first two rotation slots, also read ahead of the
  // key rows (later slots, for rows x half > 1024, load theirs in the rotation
  // loop)
  // (unconditional loads, straight into their registers: without rotation
  // they read the accumulator row instead and go unused)
  const uint32_t half = uint32_t(a.rotary / 2);
  const int32_t* trig = half ? a.trig : reinterpret_cast<const int32_t*>(a.qkv);
  const uint32_t hmod = half ? half : 1;
  int32_t tc[2], ts[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const uint32_t i = (threadIdx.x + 512 * u) % hmod;
    tc[u] = trig[2 * i];
    ts[u] = trig[2 * i + 1];
  }
  const Window win = attn_window(a);
  const uint64_t r0 = uint64_t(blockIdx.y) * P * kAttnScoreRows;
  const uint64_t qoff = uint64_t(h_first) * hd;
  if (blockIdx.y == 0)
    for (uint32_t i = threadIdx.x; i < GW * hd; i += 512) a.acc[qoff + i] = 0;
  if (r0 >= win.cnt) return;
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t cur = win.cnt - 1;  // window row of the step's own token
  const bool has_new = a.own_cache && cur >= r0 && cur < r0 + P * kAttnScoreRows;
  const uint64_t kvw = uint64_t(a.nkv) * hd;
  // this lane group's key row of every chunk, fetched while the head rows are normalised
  const uint32_t grp = threadIdx.x >> 4, li = threadIdx.x & 15;
  constexpr int kPer = MAXHD / 16;  // key elements per lane (head_dim <= MAXHD)
  int32_t kr[P][kPer];
  bool valid[P], own_row[P];
#pragma unroll
  for (int p = 0; p < P; ++p) {
    const uint64_t j = r0 + p * kAttnScoreRows + grp;
    valid[p] = j < win.cnt;
    own_row[p] = has_new && j == cur;
    const bool kload = valid[p] && !own_row[p];
    // (clamped addresses, masked values: no predicated loads)
    const global_ptr<const int32_t> krow = to_global(a.k) + (kload ? phys_row(a, win, j) : 0) * kvw + uint64_t(kvh) * hd;
    if (VEC) {
#pragma unroll
      for (int t = 0; t < kPer / 4; ++t) {
        const uint32_t d = 4 * li + 64 * t;
        const int4 v = load_int4(krow + (d < hd ? d : hd - 4));
        const bool on = kload && d < hd;
        kr[p][4 * t] = on ? v.x : 0, kr[p][4 * t + 1] = on ? v.y : 0;
        kr[p][4 * t + 2] = on ? v.z : 0, kr[p][4 * t + 3] = on ? v.w : 0;
      }
    } else {
#pragma unroll
      for (int t = 0; t < kPer; ++t) {
        const uint32_t d = li + 16 * t;
        const int32_t v = krow[d < hd ? d : hd - 1];
        kr[p][t] = (kload && d < hd) ? v : 0;
      }
    }
  }
  // head rows: jobs 0..GW-1 are the queries, then the new key (and value) rows
  const uint32_t nkeys = has_new ? ((a.has_v && writer) ? 2 : 1) : 0;
  const global_ptr<int32_t> kslot = to_global(a.k) + win.slot * kvw + uint64_t(kvh) * hd;
  const global_ptr<int32_t> vslot = to_global(a.v) + win.slot * kvw + uint64_t(kvh) * hd;
  const global_ptr<int32_t> no_row = nullptr;
  auto norm_job = [&](uint32_t job, const HeadRowIn<MAXHD>& in) {
    const bool gained = job_gain(job) != nullptr;
    if (job < GW) {
      norm_head_row(in, hd, a.eps, gained, ql + job * hd, no_row, lane);
    } else if (job == GW) {
      norm_head_row(in, hd, a.eps, gained, kn, (a.has_v || !writer) ? no_row : vslot, lane);
    } else {
      norm_head_row(in, hd, a.eps, gained, vslot, no_row, lane);
    }
  };
  // the wave's first job straight from the preloaded registers (a copy into a
  // loop variable would wait for every load in flight, key rows included)
  if (wave < GW + nkeys) norm_job(wave, pre);
  for (uint32_t job = wave + 8; job < GW + nkeys; job += 8) {
    HeadRowIn<MAXHD> in;
    load_head_row(job_src(job), hd, job_gain(job), lane, in);
    norm_job(job, in);
  }
  __syncthreads();
  if (half && win.pos != 0) {
    const uint32_t rows = GW + (has_new ? 1 : 0);
    for (uint32_t idx = threadIdx.x, u = 0; idx < rows * half; idx += 512, ++u) {
      const uint32_t r = idx / half, i = idx % half;
      int32_t* y = r < GW ? ql + r * hd : kn;
      const int32_t c = u == 0 ? tc[0] : (u == 1 ? tc[1] : a.trig[2 * i]);
      const int32_t s = u == 0 ? ts[0] : (u == 1 ? ts[1] : a.trig[2 * i + 1]);
      const int32_t lhs = y[i], rhs = y[i + half];
      y[i] = sub_sat(mul_sat(lhs, c), mul_sat(rhs, s));
      y[i + half] = add_sat(mul_sat(rhs, c), mul_sat(lhs, s));
    }
    __syncthreads();
  }
  if (has_new && writer)
    for (uint32_t d = threadIdx.x; d < hd; d += 512) kslot[d] = kn[d];
#pragma unroll
  for (int p = 0; p < P; ++p)
    if (own_row[p]) {
      if (VEC) {
#pragma unroll
        for (int t = 0; t < kPer / 4; ++t) {
          const uint32_t d = 4 * li + 64 * t;
          if (d < hd)
            kr[p][4 * t] = kn[d], kr[p][4 * t + 1] = kn[d + 1], kr[p][4 * t + 2] = kn[d + 2], kr[p][4 * t + 3] = kn[d + 3];
        }
      } else {
#pragma unroll
        for (int t = 0; t < kPer; ++t) {
          const uint32_t d = li + 16 * t;
          if (d < hd) kr[p][t] = kn[d];
        }
      }
    }
  for (uint32_t g = 0; g < GW; ++g) {
    const int32_t* qg = ql + g * hd;
    int64_t accs[P];
    if (VEC) {
      // every chunk's products from one read of each query quad, in four
      // independent wrapping chains per chunk (the sum is exact in any order);
      // past hd the key values are zero, and the query read is clamped into
      // the row
      int64_t part[P][4];
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int c = 0; c < 4; ++c) part[p][c] = 0;
#pragma unroll
      for (int t = 0; t < kPer / 4; ++t) {
        const uint32_t d = 4 * li + 64 * t;
        const int4 q = *reinterpret_cast<const int4*>(qg + (d < hd ? d : 0));
#pragma unroll
        for (int p = 0; p < P; ++p) {
          const int c = t & 3;
          part[p][c] = mac(part[p][c], q.x, kr[p][4 * t]);
          part[p][c] = mac(part[p][c], q.y, kr[p][4 * t + 1]);
          part[p][c] = mac(part[p][c], q.z, kr[p][4 * t + 2]);
          part[p][c] = mac(part[p][c], q.w, kr[p][4 * t + 3]);
        }
      }
#pragma unroll
      for (int p = 0; p < P; ++p)
        accs[p] = int64_t(uint64_t(part[p][0]) + uint64_t(part[p][1]) + uint64_t(part[p][2]) + uint64_t(part[p][3]));
    } else {
#pragma unroll
      for (int p = 0; p < P; ++p) {
        int64_t acc = 0;
#pragma unroll
        for (int t = 0; t < kPer; ++t) {
          const uint32_t d = li + 16 * t;
          if (d < hd) acc = mac(acc, qg[d], kr[p][t]);
        }
        accs[p] = acc;
      }
    }
#pragma unroll
    for (int p = 0; p < P; ++p) accs[p] = int64_t(row16_reduce(uint64_t(accs[p]), OpWrapAdd()));  // the 16 lanes of a key row
#pragma unroll
    for (int p = 0; p < P; ++p) {
      const int64_t acc = accs[p];
      if (li == 0) {
        const uint64_t j = r0 + p * kAttnScoreRows + grp;
        const int32_t sc = requant(acc);
        if (valid[p]) a.scores[(uint64_t(h_first) + g) * a.max_rows + j] = sc;
        ck[p][g][grp] = valid[p] ? score_key(sc, j) : INT64_MIN;
      }
    }
  }
  __syncthreads();
  // every chunk's argmax key per head (the maximum of the chunk maxima is the
  // window's first argmax); chunks past the window are never read
  if (threadIdx.x < P * GW) {
    const uint32_t p = threadIdx.x / GW, g = threadIdx.x % GW;
    const uint64_t c = uint64_t(blockIdx.y) * P + p;
    if (c * kAttnScoreRows < win.cnt) {
      int64_t best = ck[p][g][0];
      for (uint32_t r = 1; r < kAttnScoreRows; ++r) best = ck[p][g][r] > best ? ck[p][g][r] : best;
      a.keys[(uint64_t(h_first) + g) * a.key_chunks + c] = best;
    }
  }
}

// Integer softmax statistics (ops.rs:230-258) of every query head of one KV
// head over its whole window, 1024 threads, 16 / G waves per head: the first
// argmax (from the scores kernel's chunk maxima), the exp sum (non-negative
// terms with a total below 2^63, so the saturating sum is the plain sum) with
// its reciprocal, and the sum of every weight of the window, whose
// complement to ONE the reference adds to the argmax row's weight. With room
// in LDS each exp term is kept there for the weight pass (2^32, the argmax
// row's term, stored as 0xffffffff: every other term is at most 2^32 - 2^16).
template <bool OH = false>
__global__ __launch_bounds__(1024) void k_dec_attn_stats(AttnDecArgs a) {
  extern __shared__ int32_t sl_dyn[];
  __shared__ int64_t red[16];
  __shared__ int64_t hkey[kDecMaxGroup], hsum[kDecMaxGroup];
  __shared__ uint64_t hrec[kDecMaxGroup];
  seq_view(a);
  const Window win = attn_window(a);
  // OH: one query head per workgroup (grid x = query head); else every query
  // head of KV head blockIdx.x: GW heads from h_first
  const uint32_t G = a.nh / a.nkv;
  const uint32_t GW = OH ? 1u : G, h_first = OH ? blockIdx.x : blockIdx.x * G;
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t wph = 16 / GW, g = wave / wph, wi = wave % wph;
  const bool active = g < GW;
  const uint64_t stride = 64 * uint64_t(wph);
  const uint64_t head = uint64_t(h_first) + (active ? g : 0);
  const uint64_t nch = (win.cnt + kAttnScoreRows - 1) / kAttnScoreRows;
  int64_t best = INT64_MIN;
  if (active)
    for (uint64_t c = wi * 64 + lane; c < nch; c += stride) {
      const int64_t k = a.keys[head * a.key_chunks + c];
      best = k > best ? k : best;
    }
  best = wmax(best);
  if (lane == 0) red[wave] = best;
  __syncthreads();
  if (threadIdx.x < GW) {
    int64_t k = red[threadIdx.x * wph];
    for (uint32_t w = 1; w < wph; ++w) k = red[threadIdx.x * wph + w] > k ? red[threadIdx.x * wph + w] : k;
    hkey[threadIdx.x] = k;
  }
  __syncthreads();
  const int32_t mx = int32_t(hkey[active ? g : 0] >> 32);
  const int32_t* scg = a.scores + head * a.max_rows;
  int32_t* scl = a.scores_in_lds ? sl_dyn + uint64_t(active ? g : 0) * a.lds_stride : nullptr;
  int64_t s = 0;
  if (active)
    for (uint64_t r = wi * 64 + lane; r < win.cnt; r += stride) {
      const int64_t e = softmax_exp(scg[r], mx);
      s += e;
      if (scl) scl[r] = int32_t(e == kOneAcc ? 0xffffffffu : uint32_t(e));
    }
  s = wsum_wrap(s);
  __syncthreads();  // red[] from the argmax has been read
  if (lane == 0) red[wave] = s;
  __syncthreads();
  if (threadIdx.x < GW) {
    int64_t t = 0;
    for (uint32_t w = 0; w < wph; ++w) t += red[threadIdx.x * wph + w];
    hsum[threadIdx.x] = t;
    hrec[threadIdx.x] = t < (int64_t(1) << 61) ? softmax_recip(t) : 0;  // 0: generic division
  }
  __syncthreads();
  int64_t ws = 0;
  if (active) {
    const int64_t S = hsum[g];
    const uint64_t M = hrec[g];
    for (uint64_t r = wi * 64 + lane; r < win.cnt; r += stride) {
      int64_t e;
      if (scl) {
        const uint32_t u = uint32_t(scl[r]);
        e = u == 0xffffffffu ? kOneAcc : int64_t(u);
      } else {
        e = softmax_exp(scg[r], mx);
      }
      ws += M ? softmax_weight_r(e, S, M) : softmax_weight(e, S);
    }
  }
  ws = wsum_wrap(ws);
  __syncthreads();  // red[] from the exp sums has been read
  if (lane == 0) red[wave] = ws;
  __syncthreads();
  if (threadIdx.x < GW) {
    int64_t t = 0;
    for (uint32_t w = 0; w < wph; ++w) t += red[threadIdx.x * wph + w];
    const int64_t key = hkey[threadIdx.x];
    AttnStat st;
    st.mx = int32_t(key >> 32);
    st.mi = uint32_t(0xffffffffull - (uint64_t(key) & 0xffffffffull));
    st.sum = hsum[threadIdx.x];
    st.rec = hrec[threadIdx.x];
    st.resid = sub_sat(kOneAct, sat32(t));
    st.pad = 0;
    a.stats[uint64_t(h_first) + threadIdx.x] = st;
  }
}

// Weights (ops.rs:245-258, from the head statistics) and weighted sums
// (ops.rs:336-351) over P chunks of kAttnWsumRows window rows for every query
// head of one KV head, 1024 threads; each workgroup adds its wrapping partial
// sums to the accumulators atomically (exact in any order). Workgroup 0
// clears the projection accumulators read by the scores kernel.
template <int P, uint32_t MAXHD>
__global__ __launch_bounds__(1024) void k_dec_attn_wsum(AttnDecArgs a) {
  constexpr uint32_t R = P * kAttnWsumRows;  // window rows of this workgroup
  __shared__ int32_t wl[kDecMaxGroup][R];
  __shared__ int64_t part[3][1024];
  seq_view(a);
  const Window win = attn_window(a);
  const uint32_t kvh = blockIdx.x, G = a.nh / a.nkv, hd = a.hd;
  if (blockIdx.y == 0) {
    for (uint32_t i = threadIdx.x; i < G * hd; i += 1024) a.qkv[uint64_t(kvh) * G * hd + i] = 0;
    if (a.own_cache)
      for (uint32_t i = threadIdx.x; i < hd; i += 1024) {
        a.qkv[(uint64_t(a.nh) + kvh) * hd + i] = 0;
        if (a.has_v) a.qkv[(uint64_t(a.nh) + a.nkv + kvh) * hd + i] = 0;
      }
  }
  const uint64_t r0 = uint64_t(blockIdx.y) * R;
  if (r0 >= win.cnt) return;
  const uint64_t nr = win.cnt - r0 < R ? win.cnt - r0 : R;
  const uint64_t kvw = uint64_t(a.nkv) * hd;
  // weight of row (gg, rr) = idx of the G x R block, R <= 1024 / G for P <= 8:
  // this thread's statistics and score are read before the value rows (loads
  // complete in issue order and the value rows are needed last), at clamped
  // addresses so that no load is predicated
  const uint32_t idx0 = threadIdx.x, gg0 = idx0 / R, rr0 = idx0 % R;
  const uint64_t head0 = uint64_t(kvh) * G + (idx0 < G * R ? gg0 : 0);
  const AttnStat st0 = a.stats[head0];
  const int32_t sc0 = a.scores[head0 * a.max_rows + r0 + (rr0 < nr ? rr0 : nr - 1)];
  asm volatile("" ::: "memory");
  // value rows: slice sl takes rows 8 sl .. 8 sl + 7 of every chunk, dims dl and dl + 256
  const uint32_t sl = threadIdx.x >> 8, dl = threadIdx.x & 255;
  constexpr int JJ = MAXHD > 256 ? 2 : 1;  // dims dl (and dl + 256)
  int32_t vp[P][JJ][kAttnWsumRows / 4];
  const global_ptr<const int32_t> vcache = to_global(a.v) + uint64_t(kvh) * hd;
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int jj = 0; jj < JJ; ++jj)
#pragma unroll
      for (int k = 0; k < int(kAttnWsumRows / 4); ++k) {
        const uint32_t d = dl + 256 * jj;
        const uint64_t rr = p * kAttnWsumRows + sl * (kAttnWsumRows / 4) + k;
        vp[p][jj][k] = vcache[phys_row(a, win, r0 + (rr < nr ? rr : nr - 1)) * kvw + (d < hd ? d : hd - 1)];
      }
  asm volatile("" ::: "memory");
  auto weight = [&](const AttnStat& st, int32_t score, uint64_t r) {
    const int64_t e = softmax_exp(score, st.mx);
    int32_t w = st.rec ? softmax_weight_r(e, st.sum, st.rec) : softmax_weight(e, st.sum);
    if (r == st.mi) w = add_sat(w, st.resid);
    return w;
  };
  if (idx0 < G * R) wl[gg0][rr0] = rr0 < nr ? weight(st0, sc0, r0 + rr0) : 0;
  for (uint32_t idx = threadIdx.x + 1024; idx < G * R; idx += 1024) {
    const uint32_t gg = idx / R, rr = idx % R;
    const uint64_t head = uint64_t(kvh) * G + gg;
    wl[gg][rr] = rr < nr ? weight(a.stats[head], a.scores[head * a.max_rows + r0 + rr], r0 + rr) : 0;
  }
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int jj = 0; jj < JJ; ++jj)
#pragma unroll
      for (int k = 0; k < int(kAttnWsumRows / 4); ++k) {
        const uint64_t rr = p * kAttnWsumRows + sl * (kAttnWsumRows / 4) + k;
        if (!(dl + 256 * jj < hd && rr < nr)) vp[p][jj][k] = 0;
      }
  __syncthreads();
  // weighted sums: 4 row slices per dim, combined in LDS for up to 1024 / dstr
  // heads per pass, one atomic per (head, dim)
  const uint32_t dstr = hd > 256 ? 512 : 256;
  const uint32_t hpp = 1024 / dstr;
  for (uint32_t h0 = 0; h0 < G; h0 += hpp) {
    const uint32_t hn = G - h0 < hpp ? G - h0 : hpp;
    if (sl > 0)
      for (uint32_t hh = 0; hh < hn; ++hh) {
        int64_t p0 = 0, p1 = 0;
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
          for (int k = 0; k < int(kAttnWsumRows / 4); ++k) {
            const int32_t w = wl[h0 + hh][p * kAttnWsumRows + sl * (kAttnWsumRows / 4) + k];
            p0 = mac(p0, vp[p][0][k], w);
            if (JJ > 1) p1 = mac(p1, vp[p][JJ - 1][k], w);
          }
        part[sl - 1][hh * dstr + dl] = p0;
        if (dstr == 512) part[sl - 1][hh * dstr + 256 + dl] = p1;
      }
    __syncthreads();
    if (sl == 0)
      for (uint32_t hh = 0; hh < hn; ++hh) {
        int64_t p0 = 0, p1 = 0;
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
          for (int k = 0; k < int(kAttnWsumRows / 4); ++k) {
            const int32_t w = wl[h0 + hh][p * kAttnWsumRows + k];
            p0 = mac(p0, vp[p][0][k], w);
            if (JJ > 1) p1 = mac(p1, vp[p][JJ - 1][k], w);
          }
#pragma unroll
        for (int q = 0; q < 3; ++q) {
          p0 = int64_t(uint64_t(p0) + uint64_t(part[q][hh * dstr + dl]));
          if (dstr == 512) p1 = int64_t(uint64_t(p1) + uint64_t(part[q][hh * dstr + 256 + dl]));
        }
        int64_t* out = a.acc + (uint64_t(kvh) * G + h0 + hh) * hd;
        if (dl < hd) atomicAdd(reinterpret_cast<unsigned long long*>(out + dl), static_cast<unsigned long long>(p0));
        if (dl + 256 < hd)
          atomicAdd(reinterpret_cast<unsigned long long*>(out + dl + 256), static_cast<unsigned long long>(p1));
      }
    __syncthreads();
  }
}

// Single-kernel form for small grids (one sequence, short windows): integer
// softmax (ops.rs:230-258) and weighted sum (ops.rs:336-351) over
// P chunks of kAttnWsumRows window rows for every query head of one KV head,
// 1024 threads. Each workgroup rebuilds the heads' statistics over the whole
// window, with 16 / G waves per head: the first argmax from the scores
// kernel's per-chunk argmax keys (every wave of a head reduces all of them,
// so no barrier), the exp sum from the scores (the first NS of each thread's
// rows held in registers from the start), then weights its own rows and
// adds its wrapping partial sums to the accumulators atomically (exact in any
// order). The workgroup holding a head's argmax row also sums every weight of
// the window and applies the residual ONE - sum to that row, as the reference
// does before the weighted sum. Workgroup 0 clears the projection
// accumulators read by the scores kernel.
template <int P, uint32_t MAXHD, bool OH = false>
__global__ __launch_bounds__(1024) void k_dec_attn_softmax_wsum(AttnDecArgs a) {
  constexpr uint32_t R = P * kAttnWsumRows;  // window rows of this workgroup
  constexpr int NS = 4;                       // score rows per thread held in registers
  __shared__ int64_t red[16];
  __shared__ int64_t hsum[kDecMaxGroup];
  __shared__ uint64_t hrec[kDecMaxGroup];
  __shared__ int64_t el[kDecMaxGroup][R];
  __shared__ int32_t wl[kDecMaxGroup][R];
  __shared__ int64_t part[3][1024];
  seq_view(a);
  const Window win = attn_window(a);
  // OH: one query head per workgroup (grid x = query head); else every
  // query head of KV head blockIdx.x. GW heads from h_first.
  const uint32_t G = a.nh / a.nkv, hd = a.hd;
  const uint32_t kvh = OH ? blockIdx.x / G : blockIdx.x;
  const uint32_t GW = OH ? 1u : G, h_first = OH ? blockIdx.x : kvh * G;
  if (blockIdx.y == 0) {
    for (uint32_t i = threadIdx.x; i < GW * hd; i += 1024) a.qkv[uint64_t(h_first) * hd + i] = 0;
    if (a.own_cache && (!OH || blockIdx.x % G == 0))
      for (uint32_t i = threadIdx.x; i < hd; i += 1024) {
        a.qkv[(uint64_t(a.nh) + kvh) * hd + i] = 0;
        if (a.has_v) a.qkv[(uint64_t(a.nh) + a.nkv + kvh) * hd + i] = 0;
      }
  }
  const uint64_t r0 = uint64_t(blockIdx.y) * R;
  if (r0 >= win.cnt) return;
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint64_t nr = win.cnt - r0 < R ? win.cnt - r0 : R;
  const uint64_t kvw = uint64_t(a.nkv) * hd;
  // this wave's head and its rows r = wi * 64 + lane + stride * n
  const uint32_t wph = 16 / GW, g = wave / wph, wi = wave % wph;
  const bool active = g < GW;
  const uint64_t stride = 64 * uint64_t(wph);
  const uint64_t head = uint64_t(h_first) + (active ? g : 0);
  const int32_t* scg = a.scores + head * a.max_rows;
  const uint64_t nch = (win.cnt + kAttnScoreRows - 1) / kAttnScoreRows;
  // The chunk keys and the first NS of this thread's scores are read before
  // the value rows (loads complete in issue order, and the value rows are
  // needed last); clamped addresses, so that no load is predicated.
  const int64_t* keys = a.keys + head * a.key_chunks;
  const int64_t k0 = keys[lane < nch ? lane : nch - 1];
  int32_t sv[NS];
#pragma unroll
  for (int n = 0; n < NS; ++n) {
    const uint64_t r = wi * 64 + lane + stride * n;
    sv[n] = scg[r < win.cnt ? r : win.cnt - 1];
  }
  asm volatile("" ::: "memory");  // (keeps these loads ahead of the value rows)
  // value rows: slice sl takes rows 8 sl .. 8 sl + 7 of every chunk, dims dl and dl + 256
  const uint32_t sl = threadIdx.x >> 8, dl = threadIdx.x & 255;
  constexpr int JJ = MAXHD > 256 ? 2 : 1;  // dims dl (and dl + 256)
  int32_t vp[P][JJ][kAttnWsumRows / 4];
  const global_ptr<const int32_t> vcache = to_global(a.v) + uint64_t(kvh) * hd;
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int jj = 0; jj < JJ; ++jj)
#pragma unroll
      for (int k = 0; k < int(kAttnWsumRows / 4); ++k) {
        const uint32_t d = dl + 256 * jj;
        const uint64_t rr = p * kAttnWsumRows + sl * (kAttnWsumRows / 4) + k;
        vp[p][jj][k] = vcache[phys_row(a, win, r0 + (rr < nr ? rr : nr - 1)) * kvw + (d < hd ? d : hd - 1)];
      }
  asm volatile("" ::: "memory");
  // the head's first argmax: the largest chunk key (every wave of the head
  // reduces all of them)
  int64_t best = lane < nch ? k0 : INT64_MIN;
  for (uint64_t c = lane + 64; c < nch; c += 64) best = keys[c] > best ? keys[c] : best;
  best = wmax(best);
  const int32_t mx = int32_t(best >> 32);
  const uint64_t mi = 0xffffffffull - (uint64_t(best) & 0xffffffffull);
  // exp terms (non-negative, total below 2^63: the saturating sum is the plain
  // sum); this workgroup's rows go to LDS
  int64_t ev[NS];
  int64_t s = 0;
  if (active) {
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      const uint64_t r = wi * 64 + lane + stride * n;
      ev[n] = r < win.cnt ? softmax_exp(sv[n], mx) : 0;
      s += ev[n];
      if (r >= r0 && r < r0 + nr) el[g][r - r0] = ev[n];
    }
    for (uint64_t r = wi * 64 + lane + stride * NS; r < win.cnt; r += stride) {
      const int64_t e = softmax_exp(scg[r], mx);
      s += e;
      if (r >= r0 && r < r0 + nr) el[g][r - r0] = e;
    }
  }
  s = wsum_wrap(s);
  if (lane == 0) red[wave] = s;
  __syncthreads();
  if (threadIdx.x < GW) {
    int64_t t = 0;
    for (uint32_t w = 0; w < wph; ++w) t += red[threadIdx.x * wph + w];
    hsum[threadIdx.x] = t;
    hrec[threadIdx.x] = t < (int64_t(1) << 61) ? softmax_recip(t) : 0;  // 0: generic division
  }
  // (masked once the loads are all issued)
#pragma unroll
  for (int p = 0; p < P; ++p)
#pragma unroll
    for (int jj = 0; jj < JJ; ++jj)
#pragma unroll
      for (int k = 0; k < int(kAttnWsumRows / 4); ++k) {
        const uint64_t rr = p * kAttnWsumRows + sl * (kAttnWsumRows / 4) + k;
        if (!(dl + 256 * jj < hd && rr < nr)) vp[p][jj][k] = 0;
      }
  __syncthreads();
  // raw weights of this workgroup's rows
  for (uint32_t idx = threadIdx.x; idx < GW * R; idx += 1024) {
    const uint32_t gg = idx / R, rr = idx % R;
    const uint64_t M = hrec[gg];
    wl[gg][rr] = rr < nr ? (M ? softmax_weight_r(el[gg][rr], hsum[gg], M) : softmax_weight(el[gg][rr], hsum[gg])) : 0;
  }
  // residual for heads whose argmax row is in this chunk: their waves sum
  // every weight of the window
  const bool owner = active && mi >= r0 && mi < r0 + nr;
  int64_t ws = 0;
  if (owner) {
    const int64_t S = hsum[g];
    const uint64_t M = hrec[g];
#pragma unroll
    for (int n = 0; n < NS; ++n) {
      const uint64_t r = wi * 64 + lane + stride * n;
      if (r < win.cnt) ws += M ? softmax_weight_r(ev[n], S, M) : softmax_weight(ev[n], S);
    }
    for (uint64_t r = wi * 64 + lane + stride * NS; r < win.cnt; r += stride) {
      const int64_t e = softmax_exp(scg[r], mx);
      ws += M ? softmax_weight_r(e, S, M) : softmax_weight(e, S);
    }
  }
  ws = wsum_wrap(ws);
  __syncthreads();  // red[] from the exp sums has been read
  if (lane == 0) red[wave] = ws;
  __syncthreads();
  if (active && wi == 0 && lane == 0 && owner) {
    int64_t t = 0;
    for (uint32_t w = 0; w < wph; ++w) t += red[g * wph + w];
    wl[g][mi - r0] = add_sat(wl[g][mi - r0], sub_sat(kOneAct, sat32(t)));
  }
  __syncthreads();
  // weighted sums: 4 row slices per dim, combined in LDS for up to 1024 / dstr
  // heads per pass, one atomic per (head, dim)
  const uint32_t dstr = hd > 256 ? 512 : 256;
  const uint32_t hpp = 1024 / dstr;
  for (uint32_t h0 = 0; h0 < GW; h0 += hpp) {
    const uint32_t hn = GW - h0 < hpp ? GW - h0 : hpp;
    if (sl > 0)
      for (uint32_t hh = 0; hh < hn; ++hh) {
        int64_t p0 = 0, p1 = 0;
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
          for (int k = 0; k < int(kAttnWsumRows / 4); ++k) {
            const int32_t w = wl[h0 + hh][p * kAttnWsumRows + sl * (kAttnWsumRows / 4) + k];
            p0 = mac(p0, vp[p][0][k], w);
            if (JJ > 1) p1 = mac(p1, vp[p][JJ - 1][k], w);
          }
        part[sl - 1][hh * dstr + dl] = p0;
        if (dstr == 512) part[sl - 1][hh * dstr + 256 + dl] = p1;
      }
    __syncthreads();
    if (sl == 0)
      for (uint32_t hh = 0; hh < hn; ++hh) {
        int64_t p0 = 0, p1 = 0;
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
          for (int k = 0; k < int(kAttnWsumRows / 4); ++k) {
            const int32_t w = wl[h0 + hh][p * kAttnWsumRows + k];
            p0 = mac(p0, vp[p][0][k], w);
            if (JJ > 1) p1 = mac(p1, vp[p][JJ - 1][k], w);
          }
#pragma unroll
        for (int q = 0; q < 3; ++q) {
          p0 = int64_t(uint64_t(p0) + uint64_t(part[q][hh * dstr + dl]));
          if (dstr == 512) p1 = int64_t(uint64_t(p1) + uint64_t(part[q][hh * dstr + 256 + dl]));
        }
        int64_t* out = a.acc + (uint64_t(h_first) + h0 + hh) * hd;
        if (dl < hd) atomicAdd(reinterpret_cast<unsigned long long*>(out + dl), static_cast<unsigned long long>(p0));
        if (dl + 256 < hd)
          atomicAdd(reinterpret_cast<unsigned long long*>(out + dl + 256), static_cast<unsigned long long>(p1));
      }
    __syncthreads();
  }
}

// Writes the step position and token (passed as kernel arguments) for the
// graph-captured step that follows on the same stream, and the cos/sin pairs
// of every RoPE table at that position (ops.rs:613-680 per pair).
__global__ __launch_bounds__(256) void k_dec_set_step(StepState* __restrict__ st, uint64_t position, uint32_t token,
                                                      const RopeTable* __restrict__ tables, uint32_t ntables,
                                                      uint32_t total_pairs, int32_t* __restrict__ trig) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i == 0) {
    st->position = position;
    st->token = token;
  }
  if (i >= total_pairs) return;
  for (uint32_t t = 0; t < ntables; ++t) {
    const RopeTable tb = tables[t];
    if (i >= tb.offset && i < tb.offset + tb.pairs) {
      int32_t c, s;
      sin_cos(rope_angle(position, tb.inv_freq[i - tb.offset]), &c, &s);
      trig[2 * uint64_t(i)] = c;
      trig[2 * uint64_t(i) + 1] = s;
    }
  }
}

// Batched form: positions from st[seq] (grid y = sequence).
__global__ __launch_bounds__(256) void k_dec_set_trig(const StepState* __restrict__ st,
                                                      const RopeTable* __restrict__ tables, uint32_t ntables,
                                                      uint32_t total_pairs, int32_t* __restrict__ trig) {
  const uint32_t i = blockIdx.x * 256 + threadIdx.x;
  if (i >= total_pairs) return;
  const uint64_t position = st[blockIdx.y].position;
  trig += uint64_t(blockIdx.y) * 2 * total_pairs;
  for (uint32_t t = 0; t < ntables; ++t) {
    const RopeTable tb = tables[t];
    if (i >= tb.offset && i < tb.offset + tb.pairs) {
      int32_t c, s;
      sin_cos(rope_angle(position, tb.inv_freq[i - tb.offset]), &c, &s);
      trig[2 * uint64_t(i)] = c;
      trig[2 * uint64_t(i) + 1] = s;
    }
  }
}

// Weighted-sum accumulators of one sequence (grid y) to the O projection's
// limb planes, 4 columns per thread; the accumulators are cleared for the
// next step.
__global__ __launch_bounds__(256) void k_dec_acc_limbs(int64_t* __restrict__ acc, uint64_t k, uint64_t ld,
                                                       int8_t* __restrict__ limbs, uint64_t kpad) {
  const uint64_t c0 = (uint64_t(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (c0 >= kpad) return;
  const uint64_t t = blockIdx.y;
  int64_t* row = acc + t * ld;
  uint32_t packed[4] = {0, 0, 0, 0};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint64_t c = c0 + e;
    if (c < k) {
      const uint32_t u = uint32_t(requant(row[c])) ^ 0x00808080u;
      row[c] = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) packed[j] |= ((u >> (8 * j)) & 0xffu) << (8 * e);
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) *reinterpret_cast<uint32_t*>(limbs + (t * 4 + j) * kpad + c0) = packed[j];
}

// Limb planes of n int32 rows (grid y = row t, x at x + t * ld), 4 columns
// per thread; with GATE the row is first the per-layer input gate's
// mul_sat(gelu(x), in) (det_kernels.rs:1108-1128) with in at in + t * in_ld.
// Columns k..kpad-1 get zero bytes (their weights are zero).
template <bool GATE>
__global__ __launch_bounds__(256) void k_dec_row_limbs(const int32_t* __restrict__ x, uint64_t k, uint64_t ld,
                                                       const int32_t* __restrict__ in, uint64_t in_ld,
                                                       int8_t* __restrict__ limbs, uint64_t kpad,
                                                       int8_t* __restrict__ om) {
  const uint64_t c0 = (uint64_t(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (c0 >= kpad) return;
  const uint64_t t = blockIdx.y;
  uint32_t packed[4] = {0, 0, 0, 0};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint64_t c = c0 + e;
    if (c < k) {
      int32_t v = x[t * ld + c];
      if (GATE) v = mul_sat(gelu_act(v), in[t * in_ld + c]);
      const uint32_t u = uint32_t(v) ^ 0x00808080u;
#pragma unroll
      for (int j = 0; j < 4; ++j) packed[j] |= ((u >> (8 * j)) & 0xffu) << (8 * e);
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) *reinterpret_cast<uint32_t*>(limbs + (t * 4 + j) * kpad + c0) = packed[j];
  // (columns c0 .. c0 + 3 are four consecutive bytes of one operand)
  if (om)
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<uint32_t*>(om + om_offset(kpad, t, c0, j)) = packed[j];
}

// Up to kSetWords 64-bit words by value (within the 4 KB of kernel arguments).
constexpr uint32_t kSetWords = 448;
struct SetWords {
  uint64_t w[kSetWords];
};
__global__ __launch_bounds__(256) void k_set_words(uint64_t* __restrict__ dst, uint32_t n, SetWords v) {
  for (uint32_t i = threadIdx.x; i < n; i += 256) dst[i] = v.w[i];
}

__global__ void k_copy_rows(const int32_t* __restrict__ src, uint64_t w, int32_t* const* __restrict__ dst) {
  const uint64_t c = (uint64_t(blockIdx.x) * blockDim.x + threadIdx.x) * 4;
  if (c >= w) return;
  const int32_t* s = src + uint64_t(blockIdx.y) * w;
  int32_t* d = dst[blockIdx.y];
  if (c + 4 <= w && (w & 3) == 0) {
    *reinterpret_cast<int4*>(d + c) = *reinterpret_cast<const int4*>(s + c);
  } else {
    for (uint64_t e = c; e < w && e < c + 4; ++e) d[e] = s[e];
  }
}

// Row i of the output (stride g.stride) = g.width[i] int32 values at g.src[i];
// one workgroup per row.
__global__ void k_gather_row_ptrs(RowPtrs g, int32_t* __restrict__ dst) {
  const uint32_t r = blockIdx.x;
  const int32_t* s = g.src[r];
  int32_t* d = dst + uint64_t(r) * g.stride;
  for (uint32_t c = threadIdx.x; c < g.width[r]; c += blockDim.x) d[c] = s[c];
}

__global__ void k_dec_softcap(int32_t* __restrict__ x, uint64_t n, int32_t cap) {
  const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) x[i] = softcap_act(x[i], cap);
}

// ---------------------------------------------------------------------------
static inline unsigned nblk(uint64_t n, unsigned per) { return unsigned((n + per - 1) / per); }

// Row kernels run 1024 threads with the fewest elements per thread that
// cover the row (2, 3, 4, 8 or 15; up to kDecMaxHidden).
#define DET_ROW_DISPATCH(KERNEL, ...)                                                     \
  do {                                                                                    \
    if (H <= 2048)                                                                        \
      hipLaunchKernelGGL((KERNEL<1024, 2>), dim3(1, nseq), dim3(1024), 0, s, __VA_ARGS__); \
    else if (H <= 3072)                                                                   \
      hipLaunchKernelGGL((KERNEL<1024, 3>), dim3(1, nseq), dim3(1024), 0, s, __VA_ARGS__); \
    else if (H <= 4096)                                                                   \
      hipLaunchKernelGGL((KERNEL<1024, 4>), dim3(1, nseq), dim3(1024), 0, s, __VA_ARGS__); \
    else if (H <= 8192)                                                                   \
      hipLaunchKernelGGL((KERNEL<1024, 8>), dim3(1, nseq), dim3(1024), 0, s, __VA_ARGS__); \
    else                                                                                  \
      hipLaunchKernelGGL((KERNEL<1024, 15>), dim3(1, nseq), dim3(1024), 0, s, __VA_ARGS__);\
  } while (0)
void launch_dec_embed(const DevMatrix& E, const StepState* st, int32_t scale, uint64_t H, int32_t* x, int32_t* dec_in,
                      const int32_t* w_in, int64_t eps, int32_t* normed, int8_t* limbs, uint64_t kpad, hipStream_t s,
                      uint32_t nseq, int8_t* om) {
  DET_ROW_DISPATCH(k_dec_embed, E, st, scale, H, x, dec_in, w_in, eps, normed, limbs, kpad, om);
}
void launch_dec_residual_norm(int64_t* src, int32_t* x, int32_t* normed, const int32_t* w_post, bool has_scalar,
                              int32_t scalar, const int32_t* w_next, uint64_t H, int64_t eps, int8_t* limbs,
                              uint64_t kpad, hipStream_t s, uint32_t nseq, int32_t* x_out, const int32_t* x_src,
                              bool x_limbs, int8_t* om) {
  DET_ROW_DISPATCH(k_dec_residual_norm, src, x_src ? x_src : x, x, normed, w_post, int(has_scalar), scalar, w_next, H,
                   eps, limbs, kpad, x_out, int(x_limbs && !w_next), om);
}
#undef DET_ROW_DISPATCH
// Window chunks per attention workgroup: a.rows_mul when set (1, 2 or 4),
// else the largest that still leaves a workgroup for every CU (a single
// sequence is latency-bound and keeps one chunk per workgroup; batched steps
// share each workgroup's head norms, RoPE and atomic adds over more rows); at
// most 2 for head dims above 256 (register room).
static uint32_t attn_rows_mul(const AttnDecArgs& a) {
  const uint32_t cap = a.hd > 256 ? 2 : 4;
  uint32_t p;
  if (a.rows_mul == 1 || a.rows_mul == 2 || a.rows_mul == 4) {
    p = a.rows_mul;
  } else {
    const uint64_t wgs = uint64_t(a.nkv) * nblk(a.cap, kAttnScoreRows) * (a.nseq ? a.nseq : 1);
    p = wgs >= 4 * 256 ? 4 : (wgs >= 2 * 256 ? 2 : 1);
  }
  return p < cap ? p : cap;
}
#define DET_ATTN_P(P, HD, KERNEL, ...)                                                       \
  do {                                                                                       \
    if ((HD) <= 256) {                                                                       \
      if ((P) == 4) hipLaunchKernelGGL((KERNEL<4, 256>), __VA_ARGS__);                       \
      else if ((P) == 2) hipLaunchKernelGGL((KERNEL<2, 256>), __VA_ARGS__);                  \
      else hipLaunchKernelGGL((KERNEL<1, 256>), __VA_ARGS__);                                \
    } else {                                                                                 \
      if ((P) == 2) hipLaunchKernelGGL((KERNEL<2, kDecMaxHeadDim>), __VA_ARGS__);            \
      else hipLaunchKernelGGL((KERNEL<1, kDecMaxHeadDim>), __VA_ARGS__);                     \
    }                                                                                        \
  } while (0)
template <bool VEC, bool OH>
static void launch_scores(const AttnDecArgs& a, uint32_t P, dim3 grid, hipStream_t s) {
  if (a.hd <= 256) {
    if (P == 4) hipLaunchKernelGGL((k_dec_attn_scores<VEC, 4, 256, OH>), grid, dim3(512), 0, s, a);
    else if (P == 2) hipLaunchKernelGGL((k_dec_attn_scores<VEC, 2, 256, OH>), grid, dim3(512), 0, s, a);
    else hipLaunchKernelGGL((k_dec_attn_scores<VEC, 1, 256, OH>), grid, dim3(512), 0, s, a);
  } else {
    if (P == 2) hipLaunchKernelGGL((k_dec_attn_scores<VEC, 2, kDecMaxHeadDim, OH>), grid, dim3(512), 0, s, a);
    else hipLaunchKernelGGL((k_dec_attn_scores<VEC, 1, kDecMaxHeadDim, OH>), grid, dim3(512), 0, s, a);
  }
}
void launch_dec_attention_part(const AttnDecArgs& a, int part, hipStream_t s) {
  // grids cover the cache capacity (every window fits in it); idle chunks exit
  const uint32_t ns = a.nseq ? a.nseq : 1;
  const uint32_t P = attn_rows_mul(a);
  if (part == 0) {
    // one query head per workgroup while that grid fits the device in one
    // pass (each workgroup's dot products cover one head instead of all heads
    // of a KV head)
    const uint64_t chunks = nblk(a.cap, P * kAttnScoreRows);
    const bool oh = uint64_t(a.nh) * chunks * ns <= 256;
    const dim3 grid(oh ? a.nh : a.nkv, unsigned(chunks), ns);
    if (a.hd % 64 == 0) {
      if (oh) launch_scores<true, true>(a, P, grid, s);
      else launch_scores<true, false>(a, P, grid, s);
    } else {
      if (oh) launch_scores<false, true>(a, P, grid, s);
      else launch_scores<false, false>(a, P, grid, s);
    }
  } else if (part == 1) {
    if (uint64_t(a.nh) * ns <= 256) {
      // one query head per workgroup: a quarter of the exp terms per
      // workgroup for four heads per KV head, and one head's terms fit in LDS
      // for windows up to 8192 rows
      AttnDecArgs b = a;
      b.scores_in_lds = b.lds_stride * 4 <= 32768;
      hipLaunchKernelGGL(k_dec_attn_stats<true>, dim3(a.nh, 1, ns), dim3(1024), b.scores_in_lds ? b.lds_stride * 4 : 0,
                         s, b);
    } else {
      const size_t lds = a.scores_in_lds ? size_t(a.nh / a.nkv) * a.lds_stride * 4 : 0;
      hipLaunchKernelGGL(k_dec_attn_stats<false>, dim3(a.nkv, 1, ns), dim3(1024), lds, s, a);
    }
  } else if (part == 2) {
    DET_ATTN_P(P, a.hd, k_dec_attn_wsum, dim3(a.nkv, nblk(a.cap, P * kAttnWsumRows), ns), dim3(1024), 0, s, a);
  } else if (uint64_t(a.nh) * nblk(a.cap, P * kAttnWsumRows) * ns <= 256) {
    // one query head per workgroup while that grid still fits the device in
    // one pass: each workgroup's exp terms (the window of its heads, vector
    // ALU bound) are those of one head instead of all heads of a KV head
    const dim3 grid(a.nh, nblk(a.cap, P * kAttnWsumRows), ns);
    if (a.hd <= 256) {
      if (P == 4) hipLaunchKernelGGL((k_dec_attn_softmax_wsum<4, 256, true>), grid, dim3(1024), 0, s, a);
      else if (P == 2) hipLaunchKernelGGL((k_dec_attn_softmax_wsum<2, 256, true>), grid, dim3(1024), 0, s, a);
      else hipLaunchKernelGGL((k_dec_attn_softmax_wsum<1, 256, true>), grid, dim3(1024), 0, s, a);
    } else {
      if (P == 2) hipLaunchKernelGGL((k_dec_attn_softmax_wsum<2, kDecMaxHeadDim, true>), grid, dim3(1024), 0, s, a);
      else hipLaunchKernelGGL((k_dec_attn_softmax_wsum<1, kDecMaxHeadDim, true>), grid, dim3(1024), 0, s, a);
    }
  } else {
    DET_ATTN_P(P, a.hd, k_dec_attn_softmax_wsum, dim3(a.nkv, nblk(a.cap, P * kAttnWsumRows), ns), dim3(1024), 0, s, a);
  }
}
#undef DET_ATTN_P
// The weighted-sum workgroups of the single-kernel form each rebuild the
// window statistics; that redundancy is free while the grid fits the device
// in one pass, beyond it a separate statistics pass is cheaper.
bool dec_attention_split(const AttnDecArgs& a) {
  const uint64_t wgs = uint64_t(a.nkv) * nblk(a.cap, attn_rows_mul(a) * kAttnWsumRows) * (a.nseq ? a.nseq : 1);
  return wgs > 256;
}
void launch_dec_attention(const AttnDecArgs& a, hipStream_t s) {
  launch_dec_attention_part(a, 0, s);
  if (dec_attention_split(a)) {
    launch_dec_attention_part(a, 1, s);
    launch_dec_attention_part(a, 2, s);
  } else {
    launch_dec_attention_part(a, 3, s);
  }
}
void launch_dec_set_step(StepState* st, uint64_t position, uint32_t token, const RopeTable* tables, uint32_t ntables,
                         uint32_t total_pairs, int32_t* trig, hipStream_t s) {
  hipLaunchKernelGGL(k_dec_set_step, dim3(total_pairs ? nblk(total_pairs, 256) : 1), dim3(256), 0, s, st, position,
                     token, tables, ntables, total_pairs, trig);
}
void launch_gather_row_ptrs(const RowPtrs& g, int32_t* dst, hipStream_t s) {
  if (g.n) hipLaunchKernelGGL(k_gather_row_ptrs, dim3(g.n), dim3(256), 0, s, g, dst);
}
void launch_dec_softcap(int32_t* x, uint64_t n, int32_t cap, hipStream_t s) {
  hipLaunchKernelGGL(k_dec_softcap, dim3(nblk(n, 256)), dim3(256), 0, s, x, n, cap);
}
void launch_dec_set_trig(const StepState* st, uint32_t nseq, const RopeTable* tables, uint32_t ntables,
                         uint32_t total_pairs, int32_t* trig, hipStream_t s) {
  if (total_pairs && nseq)
    hipLaunchKernelGGL(k_dec_set_trig, dim3(nblk(total_pairs, 256), nseq), dim3(256), 0, s, st, tables, ntables,
                       total_pairs, trig);
}
void launch_dec_acc_limbs(int64_t* acc, uint64_t k, uint64_t ld, uint32_t nseq, int8_t* limbs, uint64_t kpad,
                          hipStream_t s) {
  if (nseq && kpad) hipLaunchKernelGGL(k_dec_acc_limbs, dim3(nblk(kpad / 4, 256), nseq), dim3(256), 0, s, acc, k, ld, limbs, kpad);
}
void launch_dec_row_limbs(const int32_t* x, uint64_t k, uint64_t ld, uint32_t nseq, int8_t* limbs, uint64_t kpad,
                          hipStream_t s, const int32_t* gate_in, uint64_t in_ld, int8_t* om) {
  if (!nseq || !kpad) return;
  if (kpad % 4) throw std::invalid_argument("launch_dec_row_limbs: kpad must be a multiple of 4");
  if (gate_in)
    hipLaunchKernelGGL(k_dec_row_limbs<true>, dim3(nblk(kpad / 4, 256), nseq), dim3(256), 0, s, x, k, ld, gate_in,
                       in_ld, limbs, kpad, om);
  else
    hipLaunchKernelGGL(k_dec_row_limbs<false>, dim3(nblk(kpad / 4, 256), nseq), dim3(256), 0, s, x, k, ld, x, 0,
                       limbs, kpad, om);
}
void launch_copy_rows(const int32_t* src, uint64_t w, uint64_t n, int32_t* const* dst, hipStream_t s) {
  if (n && w) hipLaunchKernelGGL(k_copy_rows, dim3(nblk((w + 3) / 4, 256), unsigned(n)), dim3(256), 0, s, src, w, dst);
}
void launch_set_bytes(void* dst, const void* src, size_t bytes, hipStream_t s) {
  const auto* w = static_cast<const uint8_t*>(src);
  auto* d = static_cast<uint64_t*>(dst);
  for (size_t off = 0; off < bytes / 8; off += kSetWords) {
    const uint32_t n = uint32_t(std::min<size_t>(kSetWords, bytes / 8 - off));
    SetWords v{};
    std::memcpy(v.w, w + off * 8, size_t(n) * 8);
    hipLaunchKernelGGL(k_set_words, dim3(1), dim3(256), 0, s, d + off, n, v);
  }
}

}  // namespace det
