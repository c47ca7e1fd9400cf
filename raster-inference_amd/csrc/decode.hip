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

#include "decode.h"
#include "det_arith.h"
#include "kernels.h"

namespace det {

constexpr int kRowThreads = 1024;

__device__ __forceinline__ int64_t wsum_sat(int64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = add_sat64(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ int64_t wsum_wrap(int64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = int64_t(uint64_t(v) + uint64_t(__shfl_xor(v, o, 64)));
  return v;
}
__device__ __forceinline__ int64_t wmax(int64_t v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const int64_t w = __shfl_xor(v, o, 64);
    v = w > v ? w : v;
  }
  return v;
}
// op 1: saturating sum of non-negative terms, op 2: max. All threads get the result.
template <int NT>
__device__ __forceinline__ int64_t blk_reduce(int64_t v, int op, int64_t* red) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = op == 1 ? wsum_sat(v) : wmax(v);
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  int64_t r = red[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) r = op == 1 ? add_sat64(r, red[w]) : (red[w] > r ? red[w] : r);
  return r;
}
// rms scale of a row held in LDS (ops.rs:406-425)
template <int NT>
__device__ __forceinline__ int32_t blk_rms_scale(const int32_t* v, uint64_t n, int64_t eps, int64_t* red) {
  int64_t ss = 0;
  for (uint64_t c = threadIdx.x; c < n; c += NT) ss = add_sat64(ss, sq_term(v[c]));
  ss = blk_reduce<NT>(ss, 1, red);
  return rms_scale_from_sumsq(ss, uint32_t(n), eps);
}

__device__ __forceinline__ int32_t wgt_bits(const DevMatrix& M, uint64_t r, uint64_t c) {
  if (M.storage == kInt8) return int32_t(M.q[tiled_offset(M.kpad, r, c)]) * M.scale[r];
  if (M.storage == kI16) return int32_t(static_cast<const int16_t*>(M.w)[r * M.cols + c]);
  return static_cast<const int32_t*>(M.w)[r * M.cols + c];
}

// Embed the step token (gemma/io.rs:2446-2518) and normalise it for layer 0.
__global__ __launch_bounds__(kRowThreads) void k_dec_embed(DevMatrix E, const StepState* __restrict__ st,
                                                          int32_t scale, uint64_t H, int32_t* __restrict__ x,
                                                          int32_t* __restrict__ dec_in, const int32_t* __restrict__ w_in,
                                                          int64_t eps, int32_t* __restrict__ normed) {
  extern __shared__ int32_t row[];
  __shared__ int64_t red[kRowThreads / 64];
  const uint32_t tok = st->token;
  for (uint64_t c = threadIdx.x; c < H; c += kRowThreads) {
    const int32_t v = mul_sat(wgt_bits(E, tok, c), scale);
    row[c] = v;
    x[c] = v;
    dec_in[c] = v;
  }
  __syncthreads();
  const int32_t sc = blk_rms_scale<kRowThreads>(row, H, eps, red);
  for (uint64_t c = threadIdx.x; c < H; c += kRowThreads) normed[c] = mul_sat(mul_sat(row[c], sc), w_in[c]);
}

// After the O projection: x = add_sat(rmsnorm(o, w_post), x); normed = rmsnorm(x, w_pre)
// (det_kernels.rs:1058-1075).
__global__ __launch_bounds__(kRowThreads) void k_dec_mid(const int32_t* __restrict__ o, int32_t* __restrict__ x,
                                                        int32_t* __restrict__ normed, const int32_t* __restrict__ w_post,
                                                        const int32_t* __restrict__ w_pre, uint64_t H, int64_t eps) {
  extern __shared__ int32_t row[];
  __shared__ int64_t red[kRowThreads / 64];
  for (uint64_t c = threadIdx.x; c < H; c += kRowThreads) row[c] = o[c];
  __syncthreads();
  const int32_t s1 = blk_rms_scale<kRowThreads>(row, H, eps, red);
  __syncthreads();
  for (uint64_t c = threadIdx.x; c < H; c += kRowThreads) {
    const int32_t v = add_sat(x[c], mul_sat(mul_sat(row[c], s1), w_post[c]));
    row[c] = v;
    x[c] = v;
  }
  __syncthreads();
  const int32_t s2 = blk_rms_scale<kRowThreads>(row, H, eps, red);
  for (uint64_t c = threadIdx.x; c < H; c += kRowThreads) normed[c] = mul_sat(mul_sat(row[c], s2), w_pre[c]);
}

// End of layer: x = add_sat(x, rmsnorm(ff, w_post_ff)); optional layer scalar;
// normed = rmsnorm(x, w_next) for the next layer's input norm (or the final norm).
__global__ __launch_bounds__(kRowThreads) void k_dec_end(const int32_t* __restrict__ ff, int32_t* __restrict__ x,
                                                        int32_t* __restrict__ normed, const int32_t* __restrict__ w_post,
                                                        int has_scalar, int32_t scalar, const int32_t* __restrict__ w_next,
                                                        uint64_t H, int64_t eps) {
  extern __shared__ int32_t row[];
  __shared__ int64_t red[kRowThreads / 64];
  for (uint64_t c = threadIdx.x; c < H; c += kRowThreads) row[c] = ff[c];
  __syncthreads();
  const int32_t s1 = blk_rms_scale<kRowThreads>(row, H, eps, red);
  __syncthreads();
  for (uint64_t c = threadIdx.x; c < H; c += kRowThreads) {
    int32_t v = add_sat(x[c], mul_sat(mul_sat(row[c], s1), w_post[c]));
    if (has_scalar) v = mul_sat(v, scalar);
    row[c] = v;
    x[c] = v;
  }
  __syncthreads();
  const int32_t s2 = blk_rms_scale<kRowThreads>(row, H, eps, red);
  for (uint64_t c = threadIdx.x; c < H; c += kRowThreads) normed[c] = mul_sat(mul_sat(row[c], s2), w_next[c]);
}

// Head norms, RoPE and KV append for one step (det_kernels.rs:952-998):
// block r < nh: query head r; then nkv key heads; then nkv value heads.
__global__ __launch_bounds__(64) void k_dec_qkv_post(QkvPostArgs a) {
  extern __shared__ int32_t y[];
  const int lane = threadIdx.x;
  const uint32_t r = blockIdx.x;
  const uint64_t pos = a.st->position;
  const uint64_t hd = a.hd, kvw = uint64_t(a.nkv) * hd;
  const int32_t* src;
  const int32_t* w = nullptr;
  int32_t* dst;
  bool rope = a.rotary > 0;
  const uint64_t slot = a.ring ? pos % a.cap : pos;
  if (r < a.nh) {
    src = a.qkv + uint64_t(r) * hd;
    w = a.q_norm;
    dst = a.qbuf + uint64_t(r) * hd;
  } else if (r < a.nh + a.nkv) {
    const uint64_t h = r - a.nh;
    src = a.qkv + (uint64_t(a.nh) + h) * hd;
    w = a.k_norm;
    dst = a.kc + slot * kvw + h * hd;
  } else {
    const uint64_t h = r - a.nh - a.nkv;
    src = a.qkv + (uint64_t(a.nh) + (a.has_v ? a.nkv : 0) + h) * hd;
    dst = a.vc + slot * kvw + h * hd;
    rope = false;
  }
  int64_t ss = 0;
  for (uint64_t d = lane; d < hd; d += 64) ss = add_sat64(ss, sq_term(src[d]));
  ss = wsum_sat(ss);
  const int32_t sc = rms_scale_from_sumsq(ss, uint32_t(hd), a.eps);
  for (uint64_t d = lane; d < hd; d += 64) {
    const int32_t v = mul_sat(src[d], sc);
    y[d] = w ? mul_sat(v, w[d]) : v;
  }
  __syncthreads();
  if (rope && pos != 0) {
    const uint64_t half = a.rotary / 2;
    for (uint64_t i = lane; i < half; i += 64) {
      int32_t c, s;
      sin_cos(rope_angle(pos, a.inv_freq[i]), &c, &s);
      const int32_t lhs = y[i], rhs = y[i + half];
      y[i] = sub_sat(mul_sat(lhs, c), mul_sat(rhs, s));
      y[i + half] = add_sat(mul_sat(rhs, c), mul_sat(lhs, s));
    }
    __syncthreads();
  }
  for (uint64_t d = lane; d < hd; d += 64) dst[d] = y[d];
}

// Window of the attention cache at this step (cache_windows + key_start,
// det_kernels.rs:297-311, 1005-1008), from the canonical slot placement.
struct Window {
  uint64_t start, len, ks, cnt;
};
__device__ __forceinline__ Window attn_window(const AttnDecArgs& a) {
  const uint64_t n = a.st->position + 1;
  Window w;
  w.len = a.ring ? (n < a.cap ? n : a.cap) : n;
  w.start = a.ring ? (n - w.len) % a.cap : 0;
  w.ks = a.window ? (w.len > a.window ? w.len - a.window : 0) : 0;
  w.cnt = w.len - w.ks;
  return w;
}
__device__ __forceinline__ uint64_t phys_row(const AttnDecArgs& a, const Window& w, uint64_t j) {
  const uint64_t l = w.ks + j;
  return a.ring ? (w.start + l) % a.cap : l;
}

// Scores for all query heads of one KV head over a chunk of 32 window rows.
__global__ __launch_bounds__(256) void k_dec_attn_scores(AttnDecArgs a) {
  const Window win = attn_window(a);
  const uint32_t kvh = blockIdx.x;
  const uint64_t r0 = uint64_t(blockIdx.y) * 32;
  if (r0 >= win.cnt) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t G = a.nh / a.nkv, hd = a.hd;
  const uint64_t kvw = uint64_t(a.nkv) * hd;
  // each lane owns dims [4*lane + 256*j, +4)
  constexpr int kMaxJ = 2;  // hd <= 512
  constexpr int kMaxG = 8;
  int32_t qv[kMaxG][kMaxJ][4];
#pragma unroll
  for (int g = 0; g < kMaxG; ++g)
#pragma unroll
    for (int j = 0; j < kMaxJ; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t d = 4 * lane + 256 * j + e;
        qv[g][j][e] = (uint32_t(g) < G && d < hd) ? a.q[(uint64_t(kvh) * G + g) * hd + d] : 0;
      }
  for (uint64_t u = 0; u < 8; ++u) {
    const uint64_t j_row = r0 + wave * 8 + u;
    if (j_row >= win.cnt) break;
    const int32_t* krow = a.k + phys_row(a, win, j_row) * kvw + uint64_t(kvh) * hd;
    int64_t acc[kMaxG];
#pragma unroll
    for (int g = 0; g < kMaxG; ++g) acc[g] = 0;
#pragma unroll
    for (int j = 0; j < kMaxJ; ++j) {
      const uint32_t d0 = 4 * lane + 256 * j;
      if (d0 < hd) {
        const int4 kv = *reinterpret_cast<const int4*>(krow + d0);
        const int32_t kk[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
        for (int g = 0; g < kMaxG; ++g)
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[g] = mac(acc[g], qv[g][j][e], kk[e]);
      }
    }
#pragma unroll
    for (int g = 0; g < kMaxG; ++g) {
      if (uint32_t(g) >= G) break;
      const int64_t t = wsum_wrap(acc[g]);
      if (lane == 0) a.scores[(uint64_t(kvh) * G + g) * a.max_rows + j_row] = requant(t);
    }
  }
}

// Integer softmax per query head (ops.rs:230-258); zeroes the head's output
// accumulators for the weighted-sum pass.
__global__ __launch_bounds__(256) void k_dec_attn_softmax(AttnDecArgs a) {
  __shared__ int64_t red[4];
  const Window win = attn_window(a);
  const uint32_t h = blockIdx.x;
  const int32_t* sc = a.scores + uint64_t(h) * a.max_rows;
  int32_t* wt = a.weights + uint64_t(h) * a.max_rows;
  for (uint64_t d = threadIdx.x; d < a.hd; d += 256) a.acc[uint64_t(h) * a.hd + d] = 0;
  int64_t best = INT64_MIN;
  for (uint64_t r = threadIdx.x; r < win.cnt; r += 256) {
    const int64_t key = (int64_t(sc[r]) * 4294967296ll) | int64_t(0xffffffffu - uint32_t(r));
    best = key > best ? key : best;
  }
  best = blk_reduce<256>(best, 2, red);
  const uint32_t mi = 0xffffffffu - uint32_t(uint64_t(best));
  const int32_t mx = sc[mi];
  int64_t sum = 0;
  for (uint64_t r = threadIdx.x; r < win.cnt; r += 256) sum = add_sat64(sum, softmax_exp(sc[r], mx));
  sum = blk_reduce<256>(sum, 1, red);
  int64_t ws = 0;
  for (uint64_t r = threadIdx.x; r < win.cnt; r += 256) {
    const int32_t w = softmax_weight(softmax_exp(sc[r], mx), sum);
    wt[r] = w;
    ws = add_sat64(ws, int64_t(w));
  }
  ws = blk_reduce<256>(ws, 1, red);
  __syncthreads();
  if (threadIdx.x == 0) wt[mi] = add_sat(wt[mi], sub_sat(kOneAct, sat32(ws)));
}

// Weighted sum over a chunk of 64 window rows for every query head of one KV
// head; partial wrapping i64 sums are added atomically (exact in any order).
__global__ __launch_bounds__(256) void k_dec_attn_wsum(AttnDecArgs a) {
  __shared__ int32_t wl[8][64];
  const Window win = attn_window(a);
  const uint32_t kvh = blockIdx.x;
  const uint64_t r0 = uint64_t(blockIdx.y) * 64;
  if (r0 >= win.cnt) return;
  const uint64_t nr = win.cnt - r0 < 64 ? win.cnt - r0 : 64;
  const uint32_t G = a.nh / a.nkv, hd = a.hd;
  const uint64_t kvw = uint64_t(a.nkv) * hd;
  for (uint32_t idx = threadIdx.x; idx < G * 64; idx += 256) {
    const uint32_t g = idx / 64, r = idx % 64;
    wl[g][r] = r < nr ? a.weights[(uint64_t(kvh) * G + g) * a.max_rows + r0 + r] : 0;
  }
  __syncthreads();
  for (uint32_t d = threadIdx.x; d < hd; d += 256) {
    int64_t acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint64_t r = 0; r < nr; ++r) {
      const int32_t v = a.v[phys_row(a, win, r0 + r) * kvw + uint64_t(kvh) * hd + d];
#pragma unroll
      for (int g = 0; g < 8; ++g)
        if (uint32_t(g) < G) acc[g] = mac(acc[g], v, wl[g][r]);
    }
#pragma unroll
    for (int g = 0; g < 8; ++g)
      if (uint32_t(g) < G)
        atomicAdd(reinterpret_cast<unsigned long long*>(a.acc + (uint64_t(kvh) * G + g) * hd + d),
                  static_cast<unsigned long long>(acc[g]));
  }
}

// Writes the step position and token (passed as kernel arguments) for the
// graph-captured step that follows on the same stream.
__global__ void k_dec_set_step(StepState* __restrict__ st, uint64_t position, uint32_t token) {
  if (threadIdx.x == 0) {
    st->position = position;
    st->token = token;
  }
}

__global__ void k_dec_softcap(int32_t* __restrict__ x, uint64_t n, int32_t cap) {
  const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) x[i] = softcap_act(x[i], cap);
}

// ---------------------------------------------------------------------------
static inline unsigned nblk(uint64_t n, unsigned per) { return unsigned((n + per - 1) / per); }

void launch_dec_embed(const DevMatrix& E, const StepState* st, int32_t scale, uint64_t H, int32_t* x, int32_t* dec_in,
                      const int32_t* w_in, int64_t eps, int32_t* normed, hipStream_t s) {
  hipLaunchKernelGGL(k_dec_embed, dim3(1), dim3(kRowThreads), H * 4, s, E, st, scale, H, x, dec_in, w_in, eps, normed);
}
void launch_dec_mid(const int32_t* o, int32_t* x, int32_t* normed, const int32_t* w_post, const int32_t* w_pre,
                    uint64_t H, int64_t eps, hipStream_t s) {
  hipLaunchKernelGGL(k_dec_mid, dim3(1), dim3(kRowThreads), H * 4, s, o, x, normed, w_post, w_pre, H, eps);
}
void launch_dec_end(const int32_t* ff, int32_t* x, int32_t* normed, const int32_t* w_post, bool has_scalar,
                    int32_t scalar, const int32_t* w_next, uint64_t H, int64_t eps, hipStream_t s) {
  hipLaunchKernelGGL(k_dec_end, dim3(1), dim3(kRowThreads), H * 4, s, ff, x, normed, w_post, int(has_scalar), scalar,
                     w_next, H, eps);
}
void launch_dec_qkv_post(const QkvPostArgs& a, bool own_cache, hipStream_t s) {
  const unsigned blocks = a.nh + (own_cache ? 2 * a.nkv : 0);
  hipLaunchKernelGGL(k_dec_qkv_post, dim3(blocks), dim3(64), a.hd * 4, s, a);
}
void launch_dec_attention(const AttnDecArgs& a, hipStream_t s) {
  // grids cover the cache capacity (every window fits in it); idle chunks exit
  hipLaunchKernelGGL(k_dec_attn_scores, dim3(a.nkv, nblk(a.cap, 32)), dim3(256), 0, s, a);
  hipLaunchKernelGGL(k_dec_attn_softmax, dim3(a.nh), dim3(256), 0, s, a);
  hipLaunchKernelGGL(k_dec_attn_wsum, dim3(a.nkv, nblk(a.cap, 64)), dim3(256), 0, s, a);
}
void launch_dec_set_step(StepState* st, uint64_t position, uint32_t token, hipStream_t s) {
  hipLaunchKernelGGL(k_dec_set_step, dim3(1), dim3(64), 0, s, st, position, token);
}
void launch_dec_softcap(int32_t* x, uint64_t n, int32_t cap, hipStream_t s) {
  hipLaunchKernelGGL(k_dec_softcap, dim3(nblk(n, 256)), dim3(256), 0, s, x, n, cap);
}

}  // namespace det
