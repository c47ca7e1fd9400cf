// Causal prefill attention on int8 MFMA (det_attention_prefill,
// det_kernels.rs:575-651): the q.k and weight.v products of every (head,
// query) row exactly, as wrapping int64 sums, from int8 limb products.
//
// An int32 x is split into four signed bytes with an offset,
//   x = c0 + 256 c1 + 65536 c2 + 2^24 c3 + C4,  C4 = 8421504,
// c_j the signed bytes of x ^ 0x808080; a softmax weight w, which lies in
// [-2^23, 2^23), into three,
//   w = a0 + 256 a1 + 65536 a2 + 32896,  a_j the signed bytes of (w + 2^23) ^ 0x808080.
// With x' = x - C4 (and w' = w - 32896):
//   sum_d q_d k_d = sum_{i,j} 256^(i+j) sum_d c_i(q_d) c_j(k_d)
//                   + C4 sum_d q'_d + C4 sum_d k'_d + hd C4^2,
//   sum_r w_r v_r = sum_{i,j} 256^(i+j) sum_r a_i(w_r) c_j(v_r)
//                   + C4 sum_r w'_r + 32896 sum_r v'_r + R 32896 C4
// in wrapping int64 (R the keys summed over). The limb products with the
// same i + j share one int32 MFMA accumulator: at most four pairs of
// 128 x 128 over at most 512 head dims (q.k), three pairs over at most
// 16000 keys (weight.v), both below 2^31. The softmax between the two is the
// integer softmax of the reference, one wave per row.
//
// Pipeline (one launch each): limb tiles of Q, of K and of V (transposed,
// dims x keys) with their offset sums; the scores of every (head, query, key
// in the window) into a work area; the softmax of every row in place (and
// the residual of its first argmax row); the weighted sums.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "det_arith.h"
#include "kernels.h"
#include "wave.h"

namespace det {

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int64_t kC4 = kAttnC4;  // offset of the four-limb split
constexpr int64_t kC3 = 32896;     // offset of the three-limb split
constexpr uint32_t kOp = kAttnOp;  // one MFMA operand block: 64 lanes x 16 bytes

// Sortable key for "max value, first index": larger value wins, then smaller index.
__device__ inline int64_t first_max_key(int32_t value, uint32_t index) {
  return (int64_t(value) * 4294967296ll) | int64_t(0xffffffffu - index);
}

// Query rows t in [0, n_queries) attend to keys [start_t, end_t).
struct AttnRange {
  uint64_t start, end;
};
__device__ inline AttnRange attn_range(const AttnMfmaArgs& a, uint64_t t) {
  uint64_t end = t + 1 + a.causal_offset;
  uint64_t start = (a.window && end > a.window) ? end - a.window : 0;
  if (start > a.avail) start = a.avail;
  if (end > a.avail) end = a.avail;
  return {start, end > start ? end : start};
}

// 16 int32 -> four 16-byte limb vectors (byte j of x ^ 0x808080) and the sum of x - C4
__device__ inline int64_t split4(const int32_t (&x)[16], v4i (&limb)[4]) {
  uint32_t w[4][4];
  const int64_t s = attn_split16(x, w);
#pragma unroll
  for (int j = 0; j < 4; ++j) limb[j] = v4i{int(w[j][0]), int(w[j][1]), int(w[j][2]), int(w[j][3])};
  return s;
}

// Q or K rows to limb blocks. Block (row tile T, substep s, limb j) at
// ((T * nsub + s) * 4 + j) * kOp: lane l holds row 16 T + (l & 15), dims
// [64 s + 16 (l >> 4), +16). One wave per substep; sums[row] = sum_d (x_d - C4).
// Rows past n take x = C4 (x' = 0: zero limbs, zero sum). grid (heads, tiles),
// block 64 * nsub.
__global__ __launch_bounds__(512) void k_attn_split_rows(const int32_t* __restrict__ x, uint64_t ld, uint64_t n,
                                                         uint32_t hd, uint64_t ntiles, int8_t* __restrict__ limbs,
                                                         int64_t* __restrict__ sums) {
  __shared__ int64_t part[8][16];
  const uint32_t h = blockIdx.x, T = blockIdx.y, s = threadIdx.x >> 6, l = threadIdx.x & 63;
  const uint32_t nsub = hd / 64;
  const uint64_t row = uint64_t(T) * 16 + (l & 15);
  const uint32_t d0 = 64 * s + 16 * (l >> 4);
  int32_t v[16];
  if (row < n) {
    const int4* p = reinterpret_cast<const int4*>(x + row * ld + uint64_t(h) * hd + d0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int4 t = p[q];
      v[4 * q] = t.x, v[4 * q + 1] = t.y, v[4 * q + 2] = t.z, v[4 * q + 3] = t.w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 16; ++e) v[e] = int32_t(kC4);
  }
  v4i limb[4];
  int64_t sm = split4(v, limb);
  int8_t* blk = limbs + ((uint64_t(h) * ntiles + T) * nsub + s) * 4 * kOp + l * 16;
#pragma unroll
  for (int j = 0; j < 4; ++j) *reinterpret_cast<v4i*>(blk + j * kOp) = limb[j];
  // the four lane groups of a row, then the substeps
  sm += __shfl_xor(sm, 16, 64);
  sm += __shfl_xor(sm, 32, 64);
  if (l < 16) part[s][l] = sm;
  __syncthreads();
  if (threadIdx.x < 16) {
    int64_t t = 0;
    for (uint32_t q = 0; q < nsub; ++q) t += part[q][threadIdx.x];
    sums[uint64_t(h) * ntiles * 16 + uint64_t(T) * 16 + threadIdx.x] = t;
  }
}

// V to transposed limb blocks: block (dim tile D, key substep ks, limb j) at
// ((D * nks + ks) * 4 + j) * kOp: lane l holds dim 16 D + (l & 15), keys
// [64 ks + 16 (l >> 4), +16) (keys past avail hold v = C4). vblk[ks][dim] =
// sum over the substep's keys of v - C4. grid (kv heads, nks), block 64 *
// min(hd / 16, 16) (waves loop over the dim tiles).
__global__ __launch_bounds__(1024) void k_attn_split_v(const int32_t* __restrict__ v, uint64_t ld, uint64_t avail,
                                                       uint32_t hd, uint64_t nks, int8_t* __restrict__ limbs,
                                                       int64_t* __restrict__ vblk) {
  const uint32_t kvh = blockIdx.x, ks = blockIdx.y, l = threadIdx.x & 63;
  const uint32_t ndt = hd / 16, nw = blockDim.x >> 6;
  for (uint32_t D = threadIdx.x >> 6; D < ndt; D += nw) {
    const uint32_t dim = 16 * D + (l & 15);
    const uint64_t k0 = uint64_t(ks) * 64 + 16 * (l >> 4);
    int32_t x[16];
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      const uint64_t r = k0 + e;
      x[e] = r < avail ? v[r * ld + uint64_t(kvh) * hd + dim] : int32_t(kC4);
    }
    v4i limb[4];
    int64_t sm = split4(x, limb);
    int8_t* blk = limbs + ((uint64_t(kvh) * ndt + D) * nks + ks) * 4 * kOp + l * 16;
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<v4i*>(blk + j * kOp) = limb[j];
    sm += __shfl_xor(sm, 16, 64);
    sm += __shfl_xor(sm, 32, 64);
    if (l < 16) vblk[(uint64_t(kvh) * nks + ks) * hd + dim] = sm;
  }
}

// Scores: block (kv head, query tile T, group of 8 key tiles), wave w on key
// tile 8 kg + w. The block's query limb blocks (all G heads, 4 KB per head
// and head-dim substep) are read once into LDS and shared by the waves; each
// wave holds its key tile's limb blocks in registers and goes through the
// heads. Lane l holds, in component r, query 16 T + 4 (l >> 4) + r and key
// 16 J + (l & 15). Scores outside a query's window are not written.
// grid (kv heads, query tiles, ceil(key tiles / 8)), block 512, LDS
// G * NSUB * 4 KB.
template <int NSUB>
__global__ __launch_bounds__(512) void k_attn_scores_mfma(AttnMfmaArgs a) {
  extern __shared__ v4i qsh[];  // [g][s][i][lane]
  const uint32_t kvh = blockIdx.x, T = blockIdx.y, wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const uint32_t G = a.groups;
  const uint64_t t_lo = uint64_t(T) * 16;
  const uint64_t t_hi = t_lo + 15 < a.n_queries ? t_lo + 15 : a.n_queries - 1;
  const uint64_t kmin = attn_range(a, t_lo).start, kmax = attn_range(a, t_hi).end;
  const uint64_t kg0 = uint64_t(blockIdx.z) * 128;  // the group's first key
  if (kg0 >= kmax || kg0 + 128 <= kmin) return;    // (workgroup-uniform)
  // the query limb blocks of the G heads
  constexpr uint32_t per_head = NSUB * 4 * 64;  // v4i per head
  for (uint32_t idx = threadIdx.x; idx < G * per_head; idx += 512) {
    const uint32_t g = idx / per_head, rest = idx % per_head;
    const uint64_t h = uint64_t(kvh) * G + g;
    qsh[idx] = reinterpret_cast<const v4i*>(a.qlimbs + (h * a.nqt + T) * NSUB * 4 * kOp)[rest];
  }
  __syncthreads();
  const uint32_t J = blockIdx.z * 8 + wave;
  const uint64_t key0 = uint64_t(J) * 16;
  if (J >= a.nkt || key0 >= kmax || key0 + 16 <= kmin) return;  // (no barriers below)
  const uint64_t key = key0 + (l & 15);
  const int64_t ks = a.ksum[uint64_t(kvh) * a.nkt * 16 + key];
  const uint64_t cconst = uint64_t(NSUB) * 64 * uint64_t(kC4) * uint64_t(kC4);
  const int8_t* kb = a.klimbs + (uint64_t(kvh) * a.nkt + J) * NSUB * 4 * kOp + l * 16;
  v4i b[NSUB][4];
#pragma unroll
  for (int s = 0; s < NSUB; ++s)
#pragma unroll
    for (int j = 0; j < 4; ++j) b[s][j] = *reinterpret_cast<const v4i*>(kb + (s * 4 + j) * kOp);
  for (uint32_t g = 0; g < G; ++g) {
    v4i acc[7];
#pragma unroll
    for (int s = 0; s < 7; ++s) acc[s] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < NSUB; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const v4i q = qsh[((g * NSUB + s) * 4 + i) * 64 + l];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i + j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(q, b[s][j], acc[i + j], 0, 0, 0);
      }
    const uint32_t h = kvh * G + g;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint64_t t = t_lo + 4 * (l >> 4) + r;
      if (t >= a.n_queries) continue;
      const AttnRange w = attn_range(a, t);
      if (key < w.start || key >= w.end) continue;
      uint64_t dot = 0;
#pragma unroll
      for (int s = 0; s < 7; ++s) dot += uint64_t(int64_t(acc[s][r])) << (8 * s);
      dot += uint64_t(kC4) * uint64_t(ks) + uint64_t(kC4) * uint64_t(a.qsum[uint64_t(h) * a.nqt * 16 + t]) + cconst;
      a.scores[(uint64_t(h) * a.n_queries + t) * a.srow + key] = requant(int64_t(dot));
    }
  }
}

template <int NSUB>
void launch_scores_nsub(const AttnMfmaArgs& m, uint64_t nkv, hipStream_t s) {
  const uint32_t lds = m.groups * NSUB * 4 * kOp;
  static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_attn_scores_mfma<NSUB>),
                                                     hipFuncAttributeMaxDynamicSharedMemorySize, 4 * NSUB * 4 * kOp);
  (void)attr;
  const dim3 grid(unsigned(nkv), unsigned(m.nqt), unsigned((m.nkt + 7) / 8));
  hipLaunchKernelGGL(k_attn_scores_mfma<NSUB>, grid, dim3(512), lds, s, m);
}

// Softmax of every (head, query) row in place, one wave per row (the
// reference's first argmax, exp sum, weights; the residual that brings the
// weights to one is kept per row, for the weighted sums to add to the first
// argmax row). The first 512 scores of a row and their exp terms stay in
// registers. grid (heads, ceil(queries / 4)), block 256.
__global__ __launch_bounds__(256) void k_attn_softmax_rows(AttnMfmaArgs a) {
  constexpr int CR = 8;  // cached entries per lane
  const uint32_t h = blockIdx.x, l = threadIdx.x & 63;
  const uint64_t t = uint64_t(blockIdx.y) * 4 + (threadIdx.x >> 6);
  if (t >= a.n_queries) return;
  const AttnRange w = attn_range(a, t);
  int32_t* row = a.scores + (uint64_t(h) * a.n_queries + t) * a.srow + w.start;
  const uint64_t cnt = w.end - w.start;
  if (cnt == 0) {  // (callers keep every window non-empty)
    if (l == 0) a.resid[uint64_t(h) * a.n_queries + t] = 0, a.argm[uint64_t(h) * a.n_queries + t] = 0xffffffffu;
    return;
  }
  int32_t sc[CR];
#pragma unroll
  for (int c = 0; c < CR; ++c) {
    const uint64_t r = l + 64 * uint64_t(c);
    sc[c] = row[r < cnt ? r : cnt - 1];
  }
  int64_t best = INT64_MIN;
#pragma unroll
  for (int c = 0; c < CR; ++c) {
    const uint64_t r = l + 64 * uint64_t(c);
    const int64_t k = first_max_key(sc[c], uint32_t(r));
    best = r < cnt && k > best ? k : best;
  }
  for (uint64_t r = l + 64 * CR; r < cnt; r += 64) {
    const int64_t k = first_max_key(row[r], uint32_t(r));
    best = k > best ? k : best;
  }
  best = wave_max64(best);
  const uint32_t mi = 0xffffffffu - uint32_t(uint64_t(best));
  const int32_t mx = int32_t(best >> 32);  // the maximum score itself
  int64_t e[CR];
  int64_t sum = 0;
#pragma unroll
  for (int c = 0; c < CR; ++c) {
    const uint64_t r = l + 64 * uint64_t(c);
    e[c] = r < cnt ? softmax_exp(sc[c], mx) : 0;
    sum += e[c];
  }
  for (uint64_t r = l + 64 * CR; r < cnt; r += 64) sum += softmax_exp(row[r], mx);  // below 2^63
  sum = wave_sum_wrap64(sum);
  const uint64_t M = sum < (int64_t(1) << 61) ? softmax_recip(sum) : 0;
  int64_t ws = 0;
#pragma unroll
  for (int c = 0; c < CR; ++c) {
    const uint64_t r = l + 64 * uint64_t(c);
    if (r < cnt) {
      const int32_t wt = M ? softmax_weight_r(e[c], sum, M) : softmax_weight(e[c], sum);
      row[r] = wt;
      ws += wt;
    }
  }
  for (uint64_t r = l + 64 * CR; r < cnt; r += 64) {
    const int64_t ex = softmax_exp(row[r], mx);
    const int32_t wt = M ? softmax_weight_r(ex, sum, M) : softmax_weight(ex, sum);
    row[r] = wt;  // each entry is read and written by the same lane
    ws += wt;
  }
  ws = wave_sum_wrap64(ws);
  if (l == 0) {
    a.resid[uint64_t(h) * a.n_queries + t] = sub_sat(kOneAct, sat32(ws));
    a.argm[uint64_t(h) * a.n_queries + t] = uint32_t(w.start + mi);
  }
}

// Weighted sums: block (kv head, query tile T, group of 8 dim tiles), wave w
// on dim tile 8 dg + w for all GB (= group size, at most 4) query heads.
// Each key substep of the tile's union window, waves 0 .. GB-1 turn one
// head's weights (zero outside a query's window, the residual added at its
// first argmax row) into three limb operands in LDS (double-buffered), and
// every wave multiplies them with its dim tile's V limbs. Lane l holds, in
// component r, query 16 T + 4 (l >> 4) + r and dim 16 D + (l & 15).
// grid (kv heads, query tiles, ceil(dim tiles / 8)), block 512.
template <int GB>
__global__ __launch_bounds__(512) void k_attn_wsum_mfma(AttnMfmaArgs a) {
  __shared__ v4i wlimb[2][GB][3][64];
  __shared__ int64_t wq[GB][16];
  const uint32_t kvh = blockIdx.x, T = blockIdx.y, wave = threadIdx.x >> 6, l = threadIdx.x & 63;
  const uint32_t ndt = a.hd / 16, D = blockIdx.z * 8 + wave;
  const bool d_on = D < ndt;
  const uint32_t G = a.groups;
  const uint64_t t_lo = uint64_t(T) * 16;
  const uint64_t t_hi = t_lo + 15 < a.n_queries ? t_lo + 15 : a.n_queries - 1;
  const uint64_t kmin = attn_range(a, t_lo).start, kmax = attn_range(a, t_hi).end;
  const uint64_t ks0 = kmin / 64, ks1 = (kmax + 63) / 64;  // key substeps of the tile's union window
  // converting waves (wave < GB): head g = wave, query tq = lane & 15
  const bool conv = wave < uint32_t(GB);
  const uint64_t tq = t_lo + (l & 15);
  const bool tq_on = tq < a.n_queries;
  const AttnRange wr = attn_range(a, tq_on ? tq : a.n_queries - 1);
  const uint64_t hq = uint64_t(kvh * G + (conv ? wave : 0)) * a.n_queries + (tq_on ? tq : 0);
  const int32_t res = conv && tq_on ? a.resid[hq] : 0;
  const uint32_t am = conv && tq_on ? a.argm[hq] : 0xffffffffu;
  const int32_t* wrow = a.scores + hq * a.srow;
  int64_t wsm = 0;
  auto convert = [&](uint64_t ks, int buf) {
    const uint64_t kb = ks * 64 + 16 * (l >> 4);
    const int4* wp = reinterpret_cast<const int4*>(wrow + kb);
    uint32_t wl[3][4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int4 x = wp[q4];
      const int32_t xs[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint64_t key = kb + 4 * q4 + e;
        int32_t wt = (tq_on && key >= wr.start && key < wr.end) ? xs[e] : 0;
        if (key == am) wt = add_sat(wt, res);
        wsm += int64_t(wt) - kC3;
        const uint32_t u = (uint32_t(wt) + 0x800000u) ^ 0x00808080u;
#pragma unroll
        for (int i = 0; i < 3; ++i) wl[i][q4] |= ((u >> (8 * i)) & 0xffu) << (8 * e);
      }
    }
#pragma unroll
    for (int i = 0; i < 3; ++i)
      wlimb[buf][wave][i][l] = v4i{int(wl[i][0]), int(wl[i][1]), int(wl[i][2]), int(wl[i][3])};
  };
  const uint32_t dim = 16 * (d_on ? D : ndt - 1) + (l & 15);
  const int8_t* vb = a.vlimbs + (uint64_t(kvh) * ndt + (d_on ? D : ndt - 1)) * a.nks * 4 * kOp + l * 16;
  int64_t vs = 0;
  for (uint64_t ks = ks0; ks < ks1; ++ks) vs += a.vblk[(uint64_t(kvh) * a.nks + ks) * a.hd + dim];
  v4i acc[GB][6];
#pragma unroll
  for (int g = 0; g < GB; ++g)
#pragma unroll
    for (int s = 0; s < 6; ++s) acc[g][s] = v4i{0, 0, 0, 0};
  if (conv && ks0 < ks1) convert(ks0, 0);
  __syncthreads();
  for (uint64_t ks = ks0; ks < ks1; ++ks) {
    const int buf = int((ks - ks0) & 1);
    v4i b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) b[j] = *reinterpret_cast<const v4i*>(vb + (ks * 4 + j) * kOp);
    // the next substep's limbs go to the other buffer while this one's MFMAs run
    if (conv && ks + 1 < ks1) convert(ks + 1, buf ^ 1);
#pragma unroll
    for (int g = 0; g < GB; ++g)
#pragma unroll
      for (int i = 0; i < 3; ++i) {
        const v4i ai = wlimb[buf][g][i][l];
#pragma unroll
        for (int j = 0; j < 4; ++j)
          acc[g][i + j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ai, b[j], acc[g][i + j], 0, 0, 0);
      }
    __syncthreads();
  }
  // sum of w - 32896 per query and head, over the four key groups of the converting wave
  if (conv) {
    int64_t sq = wsm;
    sq += __shfl_xor(sq, 16, 64);
    sq += __shfl_xor(sq, 32, 64);
    if (l < 16) wq[wave][l] = sq;
  }
  __syncthreads();
  if (!d_on) return;
  const uint64_t rconst = (ks1 - ks0) * 64 * uint64_t(kC3) * uint64_t(kC4);
#pragma unroll
  for (int g = 0; g < GB; ++g) {
    const uint32_t h = kvh * G + g;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t qi = 4 * (l >> 4) + r;
      const uint64_t t = t_lo + qi;
      uint64_t dot = 0;
#pragma unroll
      for (int s = 0; s < 6; ++s) dot += uint64_t(int64_t(acc[g][s][r])) << (8 * s);
      dot += uint64_t(kC4) * uint64_t(wq[g][qi]) + uint64_t(kC3) * uint64_t(vs) + rconst;
      if (t < a.n_queries) a.out[t * a.out_ld + uint64_t(h) * a.hd + dim] = requant(int64_t(dot));
    }
  }
}

}  // namespace

// Work area of the MFMA path (zero when it does not apply): limb blocks of Q,
// K and V, their offset sums, the score rows and the per-row residuals.
uint64_t attn_mfma_bytes(const AttnArgs& a) {
  if (a.seqs || !a.causal || a.ring_cap || a.hd % 64 != 0 || a.hd > 512 || a.num_heads == 0 || a.groups == 0 ||
      a.num_heads % a.groups != 0 || a.groups > 4 ||
      a.n_queries < 16 || a.avail == 0 || a.q_ld % 4 != 0 || a.kv_ld % 4 != 0 ||
      reinterpret_cast<uintptr_t>(a.q) % 16 != 0 || reinterpret_cast<uintptr_t>(a.k) % 16 != 0)
    return 0;
  const uint64_t nh = a.num_heads, nkv = nh / a.groups, nsub = a.hd / 64;
  const uint64_t nqt = (a.n_queries + 15) / 16, nkt = (a.avail + 15) / 16, nks = (a.avail + 63) / 64;
  const uint64_t srow = nks * 64;
  uint64_t b = 0;
  b += nh * nqt * nsub * 4 * kOp;            // Q limbs
  b += nkv * nkt * nsub * 4 * kOp;           // K limbs
  b += nkv * (a.hd / 16) * nks * 4 * kOp;    // V limbs
  b += nh * nqt * 16 * 8 + nkv * nkt * 16 * 8 + nkv * nks * a.hd * 8;  // offset sums
  b += nh * a.n_queries * srow * 4;          // scores / weights
  b += nh * a.n_queries * 8;                 // residuals and argmax rows
  return b + 4096;
}

bool attn_mfma_plan(const AttnArgs& a, AttnMfmaArgs& m) {
  const uint64_t need = attn_mfma_bytes(a);
  void* work = a.work;
  if (need == 0 || !work || a.work_bytes < need) return false;
  m = AttnMfmaArgs{};
  const uint64_t nh = a.num_heads, nkv = nh / a.groups, nsub = a.hd / 64;
  m.hd = a.hd;
  m.groups = a.groups;
  m.n_queries = a.n_queries;
  m.avail = a.avail;
  m.window = a.window;
  m.causal_offset = a.causal_offset;
  m.nqt = (a.n_queries + 15) / 16;
  m.nkt = (a.avail + 15) / 16;
  m.nks = (a.avail + 63) / 64;
  m.srow = m.nks * 64;
  m.out = a.out;
  m.out_ld = a.out_ld;
  auto carve = [&](uint64_t bytes) {
    uint8_t* p = static_cast<uint8_t*>(work);
    work = p + ((bytes + 255) / 256) * 256;
    return p;
  };
  m.qlimbs = reinterpret_cast<int8_t*>(carve(nh * m.nqt * nsub * 4 * kOp));
  m.klimbs = reinterpret_cast<int8_t*>(carve(nkv * m.nkt * nsub * 4 * kOp));
  m.vlimbs = reinterpret_cast<int8_t*>(carve(nkv * (a.hd / 16) * m.nks * 4 * kOp));
  m.qsum = reinterpret_cast<int64_t*>(carve(nh * m.nqt * 16 * 8));
  m.ksum = reinterpret_cast<int64_t*>(carve(nkv * m.nkt * 16 * 8));
  m.vblk = reinterpret_cast<int64_t*>(carve(nkv * m.nks * a.hd * 8));
  m.scores = reinterpret_cast<int32_t*>(carve(nh * a.n_queries * m.srow * 4));
  m.resid = reinterpret_cast<int32_t*>(carve(nh * a.n_queries * 4));
  m.argm = reinterpret_cast<uint32_t*>(carve(nh * a.n_queries * 4));
  return true;
}

bool launch_attention_mfma(const AttnArgs& a, void* work, uint64_t work_bytes, hipStream_t s) {
  AttnArgs aw = a;
  aw.work = work;
  aw.work_bytes = work_bytes;
  AttnMfmaArgs m;
  if (!attn_mfma_plan(aw, m)) return false;
  const uint64_t nh = a.num_heads, nkv = nh / a.groups, nsub = a.hd / 64;
  const unsigned th = unsigned(64 * nsub);
  // Q rows: heads are the row segments of q; K rows: kv heads of k (unless
  // the rows' producer wrote their blocks)
  if (!(a.split_done & 1))
    hipLaunchKernelGGL(k_attn_split_rows, dim3(unsigned(nh), unsigned(m.nqt)), dim3(th), 0, s, a.q, a.q_ld,
                       uint64_t(a.n_queries), a.hd, m.nqt, m.qlimbs, m.qsum);
  if (!(a.split_done & 2))
    hipLaunchKernelGGL(k_attn_split_rows, dim3(unsigned(nkv), unsigned(m.nkt)), dim3(th), 0, s, a.k, a.kv_ld,
                       a.avail, a.hd, m.nkt, m.klimbs, m.ksum);
  const unsigned vth = unsigned(64 * std::min<uint64_t>(a.hd / 16, 16));
  hipLaunchKernelGGL(k_attn_split_v, dim3(unsigned(nkv), unsigned(m.nks)), dim3(vth), 0, s, a.v, a.kv_ld, a.avail,
                     a.hd, m.nks, m.vlimbs, m.vblk);
  const dim3 wgrid(unsigned(nkv), unsigned(m.nqt), unsigned((a.hd / 16 + 7) / 8));
  switch (nsub) {
    case 1: launch_scores_nsub<1>(m, nkv, s); break;
    case 2: launch_scores_nsub<2>(m, nkv, s); break;
    case 3: launch_scores_nsub<3>(m, nkv, s); break;
    case 4: launch_scores_nsub<4>(m, nkv, s); break;
    case 5: launch_scores_nsub<5>(m, nkv, s); break;
    case 6: launch_scores_nsub<6>(m, nkv, s); break;
    case 7: launch_scores_nsub<7>(m, nkv, s); break;
    default: launch_scores_nsub<8>(m, nkv, s); break;
  }
  hipLaunchKernelGGL(k_attn_softmax_rows, dim3(unsigned(nh), unsigned((a.n_queries + 3) / 4)), dim3(256), 0, s, m);
  switch (a.groups) {
    case 1: hipLaunchKernelGGL(k_attn_wsum_mfma<1>, wgrid, dim3(512), 0, s, m); break;
    case 2: hipLaunchKernelGGL(k_attn_wsum_mfma<2>, wgrid, dim3(512), 0, s, m); break;
    case 3: hipLaunchKernelGGL(k_attn_wsum_mfma<3>, wgrid, dim3(512), 0, s, m); break;
    default: hipLaunchKernelGGL(k_attn_wsum_mfma<4>, wgrid, dim3(512), 0, s, m); break;
  }
  return true;
}

}  // namespace det
