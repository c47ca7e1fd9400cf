// HIP kernels of the deterministic integer transformer path for MI355X (gfx950).
//
// All reductions are integer: wrapping i64 MAC sums (any grouping is exact),
// saturating sums of non-negative terms (any grouping gives min(sum, MAX)),
// and (max, first index) selections. Results are therefore bit-identical to
// the reference's serial order regardless of the launch shape.
#include <hip/hip_runtime.h>

#include <stdexcept>

#include <mutex>
#include <type_traits>
#include <vector>

#include <algorithm>

#include "det_arith.h"
#include "kernels.h"
#include "wave.h"

namespace det {

typedef int v4i __attribute__((ext_vector_type(4)));
// the second 16-byte half of a lane's weight operand, in v4i units
constexpr int kHalfV4 = int(kTileHalfBytes / 16);

// ---------------------------------------------------------------------------
// wave / block reductions
// ---------------------------------------------------------------------------
__device__ __forceinline__ int64_t wave_sum_wrap(int64_t v) { return wave_sum_wrap64(v); }
__device__ __forceinline__ int64_t wave_sum_sat(int64_t v) { return wave_sum_sat64(v); }  // non-negative terms
__device__ __forceinline__ int64_t wave_max(int64_t v) { return wave_max64(v); }
// Sortable key for "max value, first index": larger value wins, then smaller index.
__device__ __forceinline__ int64_t argmax_key(int32_t value, uint32_t index) {
  return (int64_t(value) * 4294967296ll) | int64_t(0xffffffffu - index);
}
__device__ __forceinline__ uint32_t key_index(int64_t key) { return 0xffffffffu - uint32_t(uint64_t(key)); }

template <int NW>
__device__ __forceinline__ int64_t block_reduce(int64_t v, int op, int64_t* red) {
  // op 0: wrapping sum, 1: saturating sum of non-negatives, 2: max
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  v = op == 0 ? wave_sum_wrap(v) : (op == 1 ? wave_sum_sat(v) : wave_max(v));
  __syncthreads();
  if (lane == 0) red[wave] = v;
  __syncthreads();
  int64_t r = red[0];
  for (int w = 1; w < NW; ++w) {
    const int64_t x = red[w];
    r = op == 0 ? int64_t(uint64_t(r) + uint64_t(x)) : (op == 1 ? add_sat64(r, x) : (x > r ? x : r));
  }
  return r;
}

// ---------------------------------------------------------------------------
// int8 x Q16.16 GEMV/GEMM via limb-decomposed activations on MFMA
// ---------------------------------------------------------------------------
// a = sum_j c_j 256^j + 8421504 with c_j = int8 byte j of (a ^ 0x00808080),
// so sum_k a_k q_k = sum_j 256^j P_j + 8421504 * S where P_j = sum_k c_{j,k} q_k
// (int8 x int8 -> i32 on the matrix cores) and S = sum_k q_k.
__global__ void k_act_limbs(const int32_t* __restrict__ act, uint64_t m, uint64_t k, uint64_t ld,
                            uint64_t kpad, int8_t* __restrict__ limbs) {
  const uint64_t idx = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t t = blockIdx.y;
  if (t >= m || idx >= kpad) return;
  const uint32_t u = idx < k ? uint32_t(act[t * ld + idx]) ^ 0x00808080u : 0x00808080u;
  int8_t* base = limbs + t * 4 * kpad + idx;
  if (idx < k) {
#pragma unroll
    for (int j = 0; j < 4; ++j) base[j * kpad] = int8_t(uint8_t(u >> (8 * j)));
  } else {
#pragma unroll
    for (int j = 0; j < 4; ++j) base[j * kpad] = 0;
  }
}

// One workgroup = 16 output rows x all of K; NW waves split K in 128-byte
// steps. Lane (g = l/16, i = l%16) loads the 32 bytes [32g, 32g+32) of each
// 128-byte step for weight row 16*tile + i (B operand) and for activation
// limb row i = 4*token + limb (A operand). The 16x16 i32 result tile puts all
// four limb sums of (token g, row i) in the four accumulator registers of
// lane l, so the combine is lane-local.
// planes > 1 (a digit-plane matrix, planes dividing NW): NW / planes waves
// per plane split K; wave 0 combines the planes' partial tiles with shifts.
template <int NW>
__global__ __launch_bounds__(64 * NW) void k_gemv_i8(const int8_t* __restrict__ q,
                                                    const int32_t* __restrict__ scale,
                                                    const int32_t* __restrict__ rowsum,
                                                    const int8_t* __restrict__ limbs, uint64_t n_rows,
                                                    uint64_t kpad, uint32_t m, int32_t* __restrict__ out,
                                                    uint64_t ld_out, int64_t* __restrict__ acc_out, int lp) {
  __shared__ v4i part[NW][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, i = lane & 15;
  const uint64_t row = uint64_t(blockIdx.x) * 16 + i;
  const int at = i >> 2, aj = i & 3;
  const bool a_on = uint32_t(at) < m;
  const bool b_on = row < n_rows;
  const uint64_t nsteps = kpad / 128;
  // lp = log2(planes): NW >> lp waves per plane (shifts, no divisions)
  constexpr int LNW = NW == 16 ? 4 : (NW == 8 ? 3 : (NW == 4 ? 2 : (NW == 2 ? 1 : 0)));
  static_assert((1 << LNW) == NW, "NW is a power of two");
  const int lw = LNW - lp, wpp = 1 << lw, plane = wave >> lw, pw = wave & (wpp - 1);
  const uint64_t per = (nsteps + wpp - 1) >> lw;
  const uint64_t s0 = pw * per < nsteps ? pw * per : nsteps;
  const uint64_t s1 = s0 + per < nsteps ? s0 + per : nsteps;
  const v4i* bp = reinterpret_cast<const v4i*>(
      q + ((uint64_t(blockIdx.x) << lp) + plane) * nsteps * 2048 + lane * 16);
  const v4i* ap = reinterpret_cast<const v4i*>(limbs + (a_on ? (uint64_t(at) * 4 + aj) : 0) * kpad + 32 * g);
  const v4i zero = {0, 0, 0, 0};
  v4i acc = zero;
  uint64_t s = s0;
  for (; s + 4 <= s1; s += 4) {
    v4i b[8], a[8];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      b[2 * u] = __builtin_nontemporal_load(bp + (s + u) * 128);
      b[2 * u + 1] = __builtin_nontemporal_load(bp + (s + u) * 128 + kHalfV4);
      a[2 * u] = a_on ? ap[(s + u) * 8] : zero;
      a[2 * u + 1] = a_on ? ap[(s + u) * 8 + 1] : zero;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[u], b[u], acc, 0, 0, 0);
  }
  for (; s < s1; ++s) {
    const v4i b0 = __builtin_nontemporal_load(bp + s * 128);
    const v4i b1 = __builtin_nontemporal_load(bp + s * 128 + kHalfV4);
    const v4i a0 = a_on ? ap[s * 8] : zero;
    const v4i a1 = a_on ? ap[s * 8 + 1] : zero;
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, acc, 0, 0, 0);
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  // lane (g, i): token g, output row 16*tile + i; limb j in component j.
  int64_t p[4] = {0, 0, 0, 0};
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const v4i v = part[w][lane];
    const int sh = 8 * (w >> lw);
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] += int64_t(uint64_t(int64_t(v[j])) << sh);
  }
  if (uint32_t(g) >= m || !b_on) return;
  const int64_t dot = p[0] + p[1] * 256 + p[2] * 65536 + p[3] * 16777216 + int64_t(8421504) * rowsum[row];
  const int64_t a = int64_t(uint64_t(dot) * uint64_t(int64_t(scale[row])));
  if (acc_out) acc_out[uint64_t(g) * ld_out + row] = a;
  else out[uint64_t(g) * ld_out + row] = requant(a);
}


// Single-kernel variant: the workgroup converts the activation rows into limb
// planes in LDS once, then walks 16-row tiles persistently. KSPLIT waves
// share one tile (split K, partials combined through LDS); 8/KSPLIT tiles run
// side by side per workgroup iteration.
constexpr int kGemvThreads = 512;
constexpr uint64_t kGemvLdsBudget = 64 * 1024;

__device__ __forceinline__ int64_t limb_combine(const int64_t p[4], int32_t rowsum, int32_t scale) {
  const int64_t dot = p[0] + p[1] * 256 + p[2] * 65536 + p[3] * 16777216 + int64_t(8421504) * rowsum;
  return int64_t(uint64_t(dot) * uint64_t(int64_t(scale)));
}

// IN64: the activation rows are wrapped Q32.32 accumulators, requantized on
// load (the attention weighted sums feeding the O projection).
// EPI 0: requantize (or raw accumulators to acc_out). EPI 1: rows are
// interleaved gate/up pairs per tile (rows 0-7 gate f..f+7, rows 8-15 up
// f..f+7); out[f] = mul_sat(gelu(gate_f), up_f). EPI 2: out[row] =
// mul_sat(gelu(requant(acc)), mulv[row]) (a gate projection times a given
// row, as k_gelu_mul after the GEMV; single-chunk launches only).
// kchunks > 1 splits K across workgroups as well (block b takes K chunk
// b % kchunks): each adds its wrapping share of the Q32.32 accumulator to
// acc_out atomically (the sum over chunks is the accumulator exactly, since
// the row scale distributes over wrapping sums); acc_out starts at zero.
// A digit-plane matrix (KSPLIT * planes <= 8) gives each of a tile's planes
// KSPLIT waves; the tile's KSPLIT * planes partial tiles combine through LDS
// with shifts of 8 bits per plane.
template <int KSPLIT, bool IN64, int EPI, bool DG>
__global__ __launch_bounds__(kGemvThreads) void k_gemv_i8_lds(
    const int8_t* __restrict__ q, const int32_t* __restrict__ scale, const int32_t* __restrict__ rowsum,
    const void* __restrict__ act_v, uint64_t ld_act, uint64_t k, uint64_t n_rows, uint64_t kpad, uint32_t m,
    int32_t* __restrict__ out, uint64_t ld_out, int64_t* __restrict__ acc_out, uint32_t kchunks,
    const int32_t* __restrict__ mulv, int lp_arg) {
  const int lp = DG ? lp_arg : 0;  // (single-plane instances fold it to 0)
  extern __shared__ __attribute__((aligned(16))) int8_t lds_limbs[];
  __shared__ v4i part[8][64];
  constexpr int LKS = KSPLIT == 8 ? 3 : (KSPLIT == 4 ? 2 : (KSPLIT == 2 ? 1 : 0));
  const int ls = LKS + lp, S = 1 << ls;  // waves per tile: KSPLIT << lp (lp = log2 of the digit planes)
  const int TPW = 8 >> ls;
  const uint64_t nsteps = kpad / 128;
  const uint32_t kc = blockIdx.x % kchunks;
  const uint64_t cper = (nsteps + kchunks - 1) / kchunks;
  const uint64_t cs0 = kc * cper < nsteps ? kc * cper : nsteps;
  const uint64_t cs1 = cs0 + cper < nsteps ? cs0 + cper : nsteps;
  const uint64_t col0 = cs0 * 128, col1 = cs1 * 128;
  const uint64_t pstride = cper * 128 + 32;
  const uint64_t quads = (col1 - col0) / 4;
  // prologue: limb planes of this K chunk, 4 activations per thread-iteration
  for (uint64_t idx = threadIdx.x; idx < uint64_t(m) * quads; idx += kGemvThreads) {
    const uint64_t t = idx / quads, c = col0 + (idx % quads) * 4;
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int32_t a = 0;
      if (c + e < k)
        a = IN64 ? requant(static_cast<const int64_t*>(act_v)[t * ld_act + c + e])
                 : static_cast<const int32_t*>(act_v)[t * ld_act + c + e];
      w[e] = uint32_t(a) ^ 0x00808080u;
    }
    // padded columns get limb bytes 0 (their weights are zero as well)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t packed = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t b = (c + e < k) ? ((w[e] >> (8 * j)) & 0xffu) : 0u;
        packed |= b << (8 * e);
      }
      *reinterpret_cast<uint32_t*>(lds_limbs + (t * 4 + j) * pstride + (c - col0)) = packed;
    }
  }
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, i = lane & 15;
  const int slot = wave >> ls, within = wave & (S - 1), plane = within >> LKS, kp = within & (KSPLIT - 1);
  const int at = i >> 2, aj = i & 3;
  const bool a_on = uint32_t(at) < m;
  // LDS column (s - cs0) * 128 of this lane's limb plane
  const int8_t* abase = lds_limbs + (a_on ? (uint64_t(at) * 4 + aj) : 0) * pstride + 32 * g;
  const uint64_t per = (cs1 - cs0 + KSPLIT - 1) / KSPLIT;
  const uint64_t s0 = cs0 + kp * per < cs1 ? cs0 + kp * per : cs1;
  const uint64_t s1 = s0 + per < cs1 ? s0 + per : cs1;
  const uint64_t ntiles = (n_rows + 15) / 16;
  const uint64_t groups = gridDim.x / kchunks;
  const v4i zero = {0, 0, 0, 0};
  for (uint64_t base = uint64_t(blockIdx.x / kchunks) * TPW; base < ntiles; base += groups * TPW) {
    const uint64_t tile = base + slot;
    const uint64_t row = tile * 16 + i;
    const bool t_on = tile < ntiles && slot < TPW;
    const bool b_on = t_on && row < n_rows;
    const v4i* bp = reinterpret_cast<const v4i*>(q + (((t_on ? tile : 0) << lp) + plane) * nsteps * 2048 + lane * 16);
    v4i acc = zero;
    uint64_t s = s0;
    for (; s + 4 <= s1; s += 4) {
      v4i b[8], a[8];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        b[2 * u] = t_on ? __builtin_nontemporal_load(bp + (s + u) * 128) : zero;
        b[2 * u + 1] = t_on ? __builtin_nontemporal_load(bp + (s + u) * 128 + kHalfV4) : zero;
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        a[2 * u] = a_on ? *reinterpret_cast<const v4i*>(abase + (s - cs0 + u) * 128) : zero;
        a[2 * u + 1] = a_on ? *reinterpret_cast<const v4i*>(abase + (s - cs0 + u) * 128 + 16) : zero;
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[u], b[u], acc, 0, 0, 0);
    }
    for (; s < s1; ++s) {
      const v4i b0 = t_on ? __builtin_nontemporal_load(bp + s * 128) : zero;
      const v4i b1 = t_on ? __builtin_nontemporal_load(bp + s * 128 + kHalfV4) : zero;
      const v4i a0 = a_on ? *reinterpret_cast<const v4i*>(abase + (s - cs0) * 128) : zero;
      const v4i a1 = a_on ? *reinterpret_cast<const v4i*>(abase + (s - cs0) * 128 + 16) : zero;
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, acc, 0, 0, 0);
    }
    int64_t p[4] = {acc[0], acc[1], acc[2], acc[3]};
    if (S > 1) {
      part[wave][lane] = acc;
      __syncthreads();
      if (within == 0) {
        for (int w = 1; w < S; ++w) {
          const v4i v = part[wave + w][lane];
          const int sh = 8 * (w >> LKS);
#pragma unroll
          for (int j = 0; j < 4; ++j) p[j] += int64_t(uint64_t(int64_t(v[j])) << sh);
        }
      }
      __syncthreads();
    }
    if (within == 0) {
      const bool ok = uint32_t(g) < m && b_on;
      if (kchunks > 1) {
        if (ok) {
          const int64_t a = limb_combine(p, kc == 0 ? rowsum[row] : 0, scale[row]);
          atomicAdd(reinterpret_cast<unsigned long long*>(acc_out + uint64_t(g) * ld_out + row),
                    static_cast<unsigned long long>(a));
        }
        continue;
      }
      const int64_t a = ok ? limb_combine(p, rowsum[row], scale[row]) : 0;
      if (EPI == 1) {
        const int32_t r = requant(a);
        const int32_t up = __shfl(r, (lane & 48) | ((i + 8) & 15), 64);
        if (ok && i < 8) out[uint64_t(g) * ld_out + tile * 8 + i] = mul_sat(gelu_act(r), up);
      } else if (EPI == 2) {
        if (ok) out[uint64_t(g) * ld_out + row] = mul_sat(gelu_act(requant(a)), mulv[uint64_t(g) * ld_out + row]);
      } else if (ok) {
        if (acc_out) acc_out[uint64_t(g) * ld_out + row] = a;
        else out[uint64_t(g) * ld_out + row] = requant(a);
      }
    }
  }
}

// Batch-1 GEMV for matrices of a few thousand tiles or fewer: one workgroup
// per 16-row tile, NW waves splitting K into shares of at most D steps per
// load batch, so that up to NW * D * 128 columns take a single weight round
// trip. Each wave reads the raw activations of its batch, then issues its
// weight loads, and converts the activations into limb planes in a private
// LDS slice while the weights are in flight (no workgroup barrier before the
// MFMAs). The NW partial tiles combine through LDS; acc_out != null receives
// the Q32.32 accumulators (plain stores), else out the requantized rows.
// IN64: the activation row is a wrapped Q32.32 accumulator row, requantized
// on load.
constexpr int kTileD = 5;
// A digit-plane matrix (planes dividing NW) gives NW / planes waves to each
// plane; the partial tiles combine with shifts of 8 bits per plane.
template <int NW, bool IN64, bool DG>
__global__ __launch_bounds__(64 * NW) void k_gemv_tile(const int8_t* __restrict__ q, const int32_t* __restrict__ scale,
                                                       const int32_t* __restrict__ rowsum, const void* __restrict__ act_v,
                                                       uint64_t k, uint64_t n_rows, uint64_t kpad,
                                                       int32_t* __restrict__ out, int64_t* __restrict__ acc_out,
                                                       int lp_arg) {
  const int lp = DG ? lp_arg : 0;  // (single-plane instances fold it to 0)
  constexpr int D = kTileD;
  constexpr int kPass = (D * 32 + 63) / 64;             // activation quads per lane and batch
  constexpr uint32_t kPlane = kPass * 256 + 32;          // limb plane stride of a wave slice
  static_assert(4 * kPlane >= 64 * sizeof(v4i), "a wave slice holds the wave's partial tile");
  __shared__ __attribute__((aligned(16))) uint8_t al[NW][4 * kPlane];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, i = lane & 15;
  const uint64_t tile = blockIdx.x;
  const uint64_t nsteps = kpad / 128;
  // lp = log2(planes): NW >> lp waves per digit plane (shifts, no divisions)
  constexpr int LNW = NW == 16 ? 4 : (NW == 8 ? 3 : 2);
  static_assert((1 << LNW) == NW, "NW is 4, 8 or 16");
  const int lw = LNW - lp, wpp = 1 << lw, plane = wave >> lw, pw = wave & (wpp - 1);
  const uint64_t per = (nsteps + wpp - 1) >> lw;
  const uint64_t s0 = uint64_t(pw) * per < nsteps ? uint64_t(pw) * per : nsteps;
  const uint64_t s1 = s0 + per < nsteps ? s0 + per : nsteps;
  const v4i* bp = reinterpret_cast<const v4i*>(q + ((tile << lp) + plane) * nsteps * 2048 + lane * 16);
  const bool a_on = i < 4;  // A row i = limb i of the one token
  const uint8_t* aread = al[wave] + (i & 3) * kPlane + 32 * g;
  const v4i zero = {0, 0, 0, 0};
  v4i acc = zero;
  for (uint64_t sb = s0; sb < s1; sb += D) {
    const uint64_t c0 = sb * 128, cend = (sb + D < s1 ? sb + D : s1) * 128;
    // raw activations (lane takes columns c0 + 4 (lane + 64 r) .. + 3), read
    // at clamped addresses and masked afterwards so that no load is predicated
    using AT = typename std::conditional<IN64, int64_t, int32_t>::type;
    const AT* act = static_cast<const AT*>(act_v);
    AT av[kPass][4];
#pragma unroll
    for (int r = 0; r < kPass; ++r)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint64_t c = c0 + 4 * (uint64_t(lane) + 64 * r) + e;
        av[r][e] = act[c < k ? c : k - 1];
      }
    // weights of the batch; steps past the share re-read its last step and
    // meet zero A operands
    v4i b[2 * D];
#pragma unroll
    for (int u = 0; u < D; ++u) {
      const uint64_t st = sb + u < s1 ? sb + u : s1 - 1;
      b[2 * u] = __builtin_nontemporal_load(bp + st * 128);
      b[2 * u + 1] = __builtin_nontemporal_load(bp + st * 128 + kHalfV4);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the conversion waits
    // limb planes of the batch: byte j of a ^ 0x00808080, 0 past k (where the
    // weights are 0 too) and past the share
#pragma unroll
    for (int r = 0; r < kPass; ++r) {
      const uint32_t qd = uint32_t(lane) + 64 * r;
      const uint64_t c = c0 + 4 * uint64_t(qd);
      uint32_t w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int32_t a = IN64 ? requant(int64_t(av[r][e])) : int32_t(av[r][e]);
        w[e] = (c + e < k && c + e < cend) ? (uint32_t(a) ^ 0x00808080u) : 0u;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t packed = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) packed |= ((w[e] >> (8 * j)) & 0xffu) << (8 * e);
        *reinterpret_cast<uint32_t*>(al[wave] + j * kPlane + 4 * qd) = packed;
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    v4i a[2 * D];
#pragma unroll
    for (int u = 0; u < D; ++u) {
      a[2 * u] = *reinterpret_cast<const v4i*>(aread + u * 128);
      a[2 * u + 1] = *reinterpret_cast<const v4i*>(aread + u * 128 + 16);
    }
    if (!a_on)
#pragma unroll
      for (int u = 0; u < 2 * D; ++u) a[u] = zero;
#pragma unroll
    for (int u = 0; u < 2 * D; ++u) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[u], b[u], acc, 0, 0, 0);
    // this batch's A reads precede the next batch's plane writes
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
  // each wave's partial tile goes to its own slice (which only it has used)
  reinterpret_cast<v4i*>(al[wave])[lane] = acc;
  __syncthreads();
  if (wave != 0 || g != 0) return;
  // lane i: output row 16 tile + i, limb j in component j
  int64_t p[4] = {0, 0, 0, 0};
#pragma unroll
  for (int w = 0; w < NW; ++w) {
    const v4i v = reinterpret_cast<const v4i*>(al[w])[lane];
    const int sh = 8 * (w >> lw);
#pragma unroll
    for (int j = 0; j < 4; ++j) p[j] += int64_t(uint64_t(int64_t(v[j])) << sh);
  }
  const uint64_t row = tile * 16 + i;
  if (row >= n_rows) return;
  const int64_t r = limb_combine(p, rowsum[row], scale[row]);
  if (acc_out) acc_out[row] = r;
  else out[row] = requant(r);
}

// Decode GEMV reading the activations as limb planes in global memory (token
// t, limb j: plane 4t + j, stride kpad; byte c is byte j of a_c ^ 0x00808080,
// zero past k), so no workgroup prologue: the A operand loads issue with the
// weight loads and hit L2. NG groups of 4 tokens (one 16-row MFMA A tile
// each: row i = limb i % 4 of token 4 tg + i / 4) share every weight tile, so
// up to 4 NG sequences decode for one pass over the weights; tokens >= ntok
// are zero rows. 256 threads = 4 waves; KS waves split a tile's K range (4/KS
// tiles per workgroup and pass); kchunks splits K across workgroups.
// Outputs (token t): acc_out != null: wrapping Q32.32 partial sums added
// atomically to acc_out[t * acc_ld + row] (zero on entry); else EPI 0:
// out[t * out_ld + row] = requant; EPI 1: interleaved gate/up tiles,
// out[t * out_ld + f] = mul_sat(gelu(gate_f), up_f), also written as limb
// planes 4t..4t+3 of out_limbs (plane stride out_kpad) for the next GEMV.
template <int KS, int EPI, int NG, bool DG>
__global__ __launch_bounds__(256, NG == 1 ? 5 : (NG == 2 ? 4 : 3)) void k_gemv_dec(
    const int8_t* __restrict__ q, const int32_t* __restrict__ scale, const int32_t* __restrict__ rowsum,
    const int8_t* __restrict__ limbs, uint64_t n_rows, uint64_t kpad, uint32_t kchunks, uint32_t ntok,
    int32_t* __restrict__ out, uint64_t out_ld, int64_t* __restrict__ acc_out, uint64_t acc_ld,
    int8_t* __restrict__ out_limbs, uint64_t out_kpad, int lp_arg) {
  const int lp = DG ? lp_arg : 0;  // (single-plane instances fold it to 0)
  __shared__ v4i part[4][NG][64];
  constexpr int LKS = KS == 4 ? 2 : (KS == 2 ? 1 : 0);
  const int ls = LKS + lp, S = 1 << ls;  // waves per tile: K shares x digit planes (lp = log2 planes)
  const int TPW = 4 >> ls;
  // K steps per load batch: three for one token group (a wave's 5-step share
  // of K 2560 split four ways takes two load round trips either way), two when
  // the A tiles of several groups share the registers
  constexpr int D = NG == 1 ? 3 : 2;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, i = lane & 15;
  const int slot = wave >> ls, within = wave & (S - 1), plane = within >> LKS, kp = within & (KS - 1);
  const uint64_t nsteps = kpad / 128;
  const uint32_t kc = blockIdx.x % kchunks;
  const uint64_t cper = (nsteps + kchunks - 1) / kchunks;
  const uint64_t cs0 = kc * cper < nsteps ? kc * cper : nsteps;
  const uint64_t cs1 = cs0 + cper < nsteps ? cs0 + cper : nsteps;
  const uint64_t per = (cs1 - cs0 + KS - 1) / KS;
  const uint64_t s0 = cs0 + kp * per < cs1 ? cs0 + kp * per : cs1;
  const uint64_t s1 = s0 + per < cs1 ? s0 + per : cs1;
  const v4i* ap[NG];
  bool a_on[NG];
#pragma unroll
  for (int tg = 0; tg < NG; ++tg) {
    a_on[tg] = uint32_t(4 * tg + (i >> 2)) < ntok;
    ap[tg] = reinterpret_cast<const v4i*>(limbs + (a_on[tg] ? uint64_t(16 * tg + i) * kpad : 0) + 32 * g);
  }
  const uint64_t ntiles = (n_rows + 15) / 16;
  const uint64_t groups = gridDim.x / kchunks;
  const v4i zero = {0, 0, 0, 0};
  for (uint64_t base = uint64_t(blockIdx.x / kchunks) * TPW; base < ntiles; base += groups * TPW) {
    const uint64_t tile = base + slot;
    const uint64_t row = tile * 16 + i;
    const bool t_on = tile < ntiles;
    const v4i* bp = reinterpret_cast<const v4i*>(q + (((t_on ? tile : 0) << lp) + plane) * nsteps * 2048 + lane * 16);
    v4i acc[NG];
#pragma unroll
    for (int tg = 0; tg < NG; ++tg) acc[tg] = zero;
    uint64_t s = s0;
    for (; s + D <= s1; s += D) {
      v4i b[2 * D], a[NG][2 * D];
#pragma unroll
      for (int u = 0; u < D; ++u) {
        b[2 * u] = t_on ? __builtin_nontemporal_load(bp + (s + u) * 128) : zero;
        b[2 * u + 1] = t_on ? __builtin_nontemporal_load(bp + (s + u) * 128 + kHalfV4) : zero;
#pragma unroll
        for (int tg = 0; tg < NG; ++tg) {
          a[tg][2 * u] = a_on[tg] ? ap[tg][(s + u) * 8] : zero;
          a[tg][2 * u + 1] = a_on[tg] ? ap[tg][(s + u) * 8 + 1] : zero;
        }
      }
#pragma unroll
      for (int u = 0; u < 2 * D; ++u)
#pragma unroll
        for (int tg = 0; tg < NG; ++tg) acc[tg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[tg][u], b[u], acc[tg], 0, 0, 0);
    }
    for (; s < s1; ++s) {
      const v4i b0 = t_on ? __builtin_nontemporal_load(bp + s * 128) : zero;
      const v4i b1 = t_on ? __builtin_nontemporal_load(bp + s * 128 + kHalfV4) : zero;
#pragma unroll
      for (int tg = 0; tg < NG; ++tg) {
        const v4i a0 = a_on[tg] ? ap[tg][s * 8] : zero;
        const v4i a1 = a_on[tg] ? ap[tg][s * 8 + 1] : zero;
        acc[tg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, acc[tg], 0, 0, 0);
        acc[tg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, acc[tg], 0, 0, 0);
      }
    }
    int64_t p[NG][4];
#pragma unroll
    for (int tg = 0; tg < NG; ++tg)
#pragma unroll
      for (int e = 0; e < 4; ++e) p[tg][e] = acc[tg][e];
    if (S > 1) {
#pragma unroll
      for (int tg = 0; tg < NG; ++tg) part[wave][tg][lane] = acc[tg];
      __syncthreads();
      if (within == 0) {
        for (int w = 1; w < S; ++w) {
          const int sh = 8 * (w >> LKS);
#pragma unroll
          for (int tg = 0; tg < NG; ++tg) {
            const v4i v = part[wave + w][tg][lane];
#pragma unroll
            for (int j = 0; j < 4; ++j) p[tg][j] += int64_t(uint64_t(int64_t(v[j])) << sh);
          }
        }
      }
      __syncthreads();
    }
    if (within != 0 || !t_on) continue;
    const bool r_on = row < n_rows;
    const int32_t rs = r_on ? rowsum[row] : 0, sc = r_on ? scale[row] : 0;
    // lane 16 g + i of group tg holds the limb sums of token 4 tg + g, row i
#pragma unroll
    for (int tg = 0; tg < NG; ++tg) {
      const uint32_t tok = 4 * tg + g;
      const bool ok = tok < ntok && r_on;
      if (acc_out) {
        if (ok) {
          const int64_t a = limb_combine(p[tg], kc == 0 ? rs : 0, sc);
          atomicAdd(reinterpret_cast<unsigned long long*>(acc_out + tok * acc_ld + row),
                    static_cast<unsigned long long>(a));
        }
      } else if (EPI == 1) {
        const int32_t r = ok ? requant(limb_combine(p[tg], rs, sc)) : 0;
        const int32_t up = __shfl(r, (lane & 48) | ((i + 8) & 15), 64);
        if (ok && i < 8) {
          const uint64_t f = tile * 8 + i;
          const int32_t h = mul_sat(gelu_act(r), up);
          out[tok * out_ld + f] = h;
          const uint32_t u = uint32_t(h) ^ 0x00808080u;
          int8_t* ol = out_limbs + uint64_t(tok) * 4 * out_kpad + f;
#pragma unroll
          for (int j = 0; j < 4; ++j) ol[j * out_kpad] = int8_t(uint8_t(u >> (8 * j)));
        }
      } else if (ok) {
        out[tok * out_ld + row] = requant(limb_combine(p[tg], rs, sc));
      }
    }
  }
}

// Single-token form of k_gemv_dec (same arguments, outputs and K split) for
// K shares of 4-5 steps per wave (E4B's gate/up projection): the four limb
// planes of a wave's share are copied into a private LDS slice with
// global_load_lds, so that they hold no registers while in flight and all
// D = 5 weight steps of the share fit in registers at once, one weight round
// trip (k_gemv_dec holds A and B in registers and takes 3 steps per trip).
// Every load goes to a clamped address (none is predicated); steps past the
// share meet zero A operands.
template <int KS, int EPI, bool DG>
__global__ __launch_bounds__(256, 5) void k_gemv_dec1(
    const int8_t* __restrict__ q, const int32_t* __restrict__ scale, const int32_t* __restrict__ rowsum,
    const int8_t* __restrict__ limbs, uint64_t n_rows, uint64_t kpad, uint32_t kchunks, int32_t* __restrict__ out,
    int64_t* __restrict__ acc_out, int8_t* __restrict__ out_limbs, uint64_t out_kpad, int lp_arg) {
  const int lp = DG ? lp_arg : 0;  // (single-plane instances fold it to 0)
  constexpr int D = 5;
  constexpr int kCopies = (4 * D * 128 + 1023) / 1024;  // 1 KB wave copies of 4 planes x D steps
  __shared__ __attribute__((aligned(16))) int8_t al[4][kCopies * 1024];
  __shared__ v4i part[4][64];
  constexpr int LKS = KS == 4 ? 2 : (KS == 2 ? 1 : 0);
  const int ls = LKS + lp, S = 1 << ls;  // waves per tile: K shares x digit planes (lp = log2 planes)
  const int TPW = 4 >> ls;
  constexpr int kWaitLds = 15 | (7 << 4) | (0 << 8) | (3 << 14);  // lgkmcnt(0)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, i = lane & 15;
  const int slot = wave >> ls, within = wave & (S - 1), plane = within >> LKS, kp = within & (KS - 1);
  const uint64_t nsteps = kpad / 128;
  const uint32_t kc = blockIdx.x % kchunks;
  const uint64_t cper = (nsteps + kchunks - 1) / kchunks;
  const uint64_t cs0 = kc * cper < nsteps ? kc * cper : nsteps;
  const uint64_t cs1 = cs0 + cper < nsteps ? cs0 + cper : nsteps;
  const uint64_t per = (cs1 - cs0 + KS - 1) / KS;
  const uint64_t s0 = cs0 + kp * per < cs1 ? cs0 + kp * per : cs1;
  const uint64_t s1 = s0 + per < cs1 ? s0 + per : cs1;
  // A row i < 4 is limb i of the token: plane i, bytes [32 g, 32 g + 32) of each step
  const bool a_on = i < 4;
  const int8_t* aread = al[wave] + (i & 3) * (D * 128) + 32 * g;
  const uint64_t ntiles = (n_rows + 15) / 16;
  const uint64_t groups = gridDim.x / kchunks;
  const v4i zero = {0, 0, 0, 0};
  for (uint64_t base = uint64_t(blockIdx.x / kchunks) * TPW; base < ntiles; base += groups * TPW) {
    const uint64_t tile = base + slot;
    const uint64_t row = tile * 16 + i;
    const bool t_on = tile < ntiles;
    const v4i* bp = reinterpret_cast<const v4i*>(q + (((t_on ? tile : ntiles - 1) << lp) + plane) * nsteps * 2048 +
                                                 lane * 16);
    v4i acc = zero;
    for (uint64_t sb = s0; sb < s1; sb += D) {
      const uint64_t nu = s1 - sb < uint64_t(D) ? s1 - sb : uint64_t(D);
      // the previous batch's operand reads are done before its slice is overwritten
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt(kWaitLds);
      asm volatile("" ::: "memory");
      // A: copy r, lane l takes the 16-byte piece (64 r + l) % 8 of chunk (64 r + l) / 8 =
      // (plane, step u) at slice offset 128 (D plane + u); chunks past the 4 D real ones
      // re-read the last real one into the slice's slack
#pragma unroll
      for (int r = 0; r < kCopies; ++r) {
        const uint32_t idx = 64 * r + lane, chunk = idx >> 3, piece = idx & 7;
        const uint32_t c = chunk < uint32_t(4 * D) ? chunk : uint32_t(4 * D - 1);
        const uint32_t plane = c / D, u = c % D;
        const uint64_t st = sb + u < s1 ? sb + u : s1 - 1;
        const int8_t* src = limbs + plane * kpad + st * 128 + piece * 16;
        __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)src,
                                         (void __attribute__((address_space(3)))*)(al[wave] + r * 1024), 16, 0, 0);
      }
      asm volatile("" ::: "memory");
      __builtin_amdgcn_sched_barrier(0);
      // B: the share's weight steps (past the share: its last step again)
      v4i b[2 * D];
#pragma unroll
      for (int u = 0; u < D; ++u) {
        const uint64_t st = sb + u < s1 ? sb + u : s1 - 1;
        b[2 * u] = __builtin_nontemporal_load(bp + st * 128);
        b[2 * u + 1] = __builtin_nontemporal_load(bp + st * 128 + kHalfV4);
      }
      // the copies have landed once every load of the batch has (the compiler does not
      // order LDS reads after global_load_lds by itself; waiting for all loads holds
      // whatever order it gives the weight loads)
      asm volatile("" ::: "memory");
      __builtin_amdgcn_s_waitcnt(0);
      asm volatile("" ::: "memory");
#pragma unroll
      for (int u = 0; u < D; ++u) {
        // idle rows and steps past the share: a mask, not a branch, so the reads stay unconditional
        const int m = (a_on && uint64_t(u) < nu) ? -1 : 0;
        const v4i a0 = *reinterpret_cast<const v4i*>(aread + u * 128) & m;
        const v4i a1 = *reinterpret_cast<const v4i*>(aread + u * 128 + 16) & m;
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b[2 * u], acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b[2 * u + 1], acc, 0, 0, 0);
      }
    }
    int64_t p[4] = {acc[0], acc[1], acc[2], acc[3]};
    if (S > 1) {
      part[wave][lane] = acc;
      __syncthreads();
      if (within == 0) {
        for (int w = 1; w < S; ++w) {
          const v4i v = part[wave + w][lane];
          const int sh = 8 * (w >> LKS);
#pragma unroll
          for (int j = 0; j < 4; ++j) p[j] += int64_t(uint64_t(int64_t(v[j])) << sh);
        }
      }
      __syncthreads();
    }
    if (within != 0 || !t_on) continue;
    const bool r_on = row < n_rows;
    const int32_t rs = r_on ? rowsum[row] : 0, sc = r_on ? scale[row] : 0;
    // lanes 0-15 (g = 0) hold the token's four limb sums of row i
    const bool ok = g == 0 && r_on;
    if (acc_out) {
      if (ok) {
        const int64_t a = limb_combine(p, kc == 0 ? rs : 0, sc);
        atomicAdd(reinterpret_cast<unsigned long long*>(acc_out + row), static_cast<unsigned long long>(a));
      }
    } else if (EPI == 1) {
      const int32_t r = ok ? requant(limb_combine(p, rs, sc)) : 0;
      const int32_t up = __shfl(r, (lane & 48) | ((i + 8) & 15), 64);
      if (ok && i < 8) {
        const uint64_t f = tile * 8 + i;
        const int32_t h = mul_sat(gelu_act(r), up);
        out[f] = h;
        const uint32_t u = uint32_t(h) ^ 0x00808080u;
#pragma unroll
        for (int j = 0; j < 4; ++j) out_limbs[j * out_kpad + f] = int8_t(uint8_t(u >> (8 * j)));
      }
    } else if (ok) {
      out[row] = requant(limb_combine(p, rs, sc));
    }
  }
}

// Residual norm + batch-1 decode GEMV in one kernel (the residual-norm row
// kernel between a projection and the next GEMV is gone, with its launch and
// its reads of the projection's output): every workgroup issues its weight
// loads first, computes the whole residual norm of the row while they are in
// flight (the row is 2-4 K values per thread; the two scale chains run once
// per workgroup, on wave 0), builds the limb planes of the normalised row in
// LDS and then runs its MFMAs.
//   x' = add_sat(x_in, mul_sat(mul_sat(requant(src), s1), w_post)) [* scalar]
//   a  = mul_sat(mul_sat(x', s2), w_next)
// with s1, s2 the rms scales of requant(src) and x' (det_kernels.rs:1058-1075,
// 1108-1133; the arithmetic of k_dec_residual_norm). Workgroup 0 writes x'.
// Work: the grid's G workgroups take tiles b, b + G, ...; each of a tile's
// K parts of kNormD steps (one weight round trip) is a job, and wave w takes
// jobs w and w + NW of its workgroup. Partial tiles combine through LDS.
// EPI 0: Q32.32 accumulators to acc_out (plain stores); EPI 1: interleaved
// gate/up tiles, out[f] = mul_sat(gelu(gate_f), up_f) and its limb planes
// (stride out_kpad) to out_limbs.
constexpr int kNormD = 5;
constexpr uint32_t kNormMaxK = 4096;
// rms scale of a row spread over the workgroup from each thread's saturating
// partial sum of squares (ops.rs:406-425). With at most four waves every wave
// reduces the wave totals and runs the scale chain itself (one per SIMD, no
// second barrier); with more, wave 0 does and broadcasts the scale through
// LDS. red holds this call's wave totals (a separate array per call, so that
// one call's reads never meet the next call's writes).
// `between` runs in every wave once all waves have passed their partial sums.
template <int NW, class F>
__device__ __forceinline__ int32_t wg_rms_scale(int64_t ss, uint64_t n, int64_t eps, int64_t* red, int32_t* bc,
                                                int wave, int lane, F&& between) {
  ss = wave_sum_sat(ss);
  if (lane == 0) red[wave] = ss;
  lds_barrier();
  between();
  if constexpr (NW <= 4) {
    int64_t t = lane < NW ? red[lane] : 0;
    t = wave_sum_sat(t);
    return rms_scale_from_sumsq(t, uint32_t(n), eps);
  } else {
    if (wave == 0) {
      int64_t t = lane < NW ? red[lane] : 0;
      t = wave_sum_sat(t);
      if (lane == 0) *bc = rms_scale_from_sumsq(t, uint32_t(n), eps);
    }
    lds_barrier();
    return *bc;
  }
}
template <int NW, int JM, int QPT, int EPI, bool DG>
__global__ __launch_bounds__(64 * NW) void k_gemv_norm(DecNormIn ni, const int8_t* __restrict__ q,
                                                       const int32_t* __restrict__ scale,
                                                       const int32_t* __restrict__ rowsum, uint64_t n_rows,
                                                       uint64_t kpad, int64_t* __restrict__ acc_out,
                                                       int32_t* __restrict__ out, int8_t* __restrict__ out_limbs,
                                                       uint64_t out_kpad, int lp_arg) {
  const int lp = DG ? lp_arg : 0;  // (single-plane instances fold it to 0)
  constexpr int NT = 64 * NW, D = kNormD;
  constexpr uint32_t kPlaneMax = kNormMaxK + 32;
  typedef long long v2l __attribute__((ext_vector_type(2)));
  __shared__ __attribute__((aligned(16))) uint8_t al[4 * kPlaneMax];
  __shared__ v4i part[NW * JM][64];
  __shared__ int64_t red[2][NW];
  __shared__ int32_t bc;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, i = lane & 15;
  // a tile's jobs: its digit planes x K parts of D steps (job pp: plane pp / np,
  // lp = log2 of the planes)
  const uint64_t nsteps = kpad / 128, np = (nsteps + D - 1) / D, npt = np << lp;
  const uint64_t ntiles = (n_rows + 15) / 16, G = gridDim.x;
  const uint64_t tpw = (ntiles + G - 1) / G, njobs = tpw * npt;
  const uint64_t plane = kpad + 32;  // limb plane stride in LDS (planes start 8 banks apart)
  const uint64_t Q = ni.H / 4;      // activation quads (H % 4 == 0, H <= 4 NT QPT)
  // 1. the norm's inputs, quad qd = tid + NT e (clamped addresses, masked
  // below), and the row sum and scale of the tile whose epilogue this wave
  // runs first
  int64_t sv[QPT][4];
  int32_t xv[QPT][4], wp[QPT][4], wn[QPT][4];
#pragma unroll
  for (int e = 0; e < QPT; ++e) {
    const uint64_t qd = threadIdx.x + uint64_t(NT) * e, qc = qd < Q ? qd : Q - 1;
    const v2l s0 = *reinterpret_cast<const v2l*>(ni.src + 4 * qc);
    const v2l s1 = *reinterpret_cast<const v2l*>(ni.src + 4 * qc + 2);
    const v4i x4 = *reinterpret_cast<const v4i*>(ni.x_in + 4 * qc);
    const v4i p4 = *reinterpret_cast<const v4i*>(ni.w_post + 4 * qc);
    const v4i n4 = *reinterpret_cast<const v4i*>(ni.w_next + 4 * qc);
    sv[e][0] = s0.x, sv[e][1] = s0.y, sv[e][2] = s1.x, sv[e][3] = s1.y;
#pragma unroll
    for (int k = 0; k < 4; ++k) xv[e][k] = x4[k], wp[e][k] = p4[k], wn[e][k] = n4[k];
  }
  // first epilogue tile of this lane group (lanes 16 g + i of wave w take tile 4 w + g)
  const uint64_t et = uint64_t(blockIdx.x) + G * (4 * uint64_t(wave) + uint64_t(g));
  const uint64_t erow = (et < ntiles ? et : ntiles - 1) * 16 + i;
  const uint64_t erc = erow < n_rows ? erow : n_rows - 1;
  const int32_t ers = rowsum[erc], esc = scale[erc];
  // 2. this wave's jobs: weight loads of up to D steps each (steps past the
  // part re-read its last step and meet zero A operands). Slots past the
  // workgroup's jobs load one line at q, never combined. They are issued once
  // every wave of the workgroup holds the norm's inputs: the inputs' reads
  // are not queued behind the weight stream (whose bytes stay in flight
  // through the rest of the norm).
  uint64_t js0[JM], jnu[JM];
  v4i b[JM][2 * D];
  // jobs [u0, u1) of this wave
  auto issue_weights = [&](auto u0c, auto u1c) {
    constexpr int u0 = decltype(u0c)::value, u1 = decltype(u1c)::value;
#pragma unroll
    for (int u = u0; u < u1; ++u) {
      const uint64_t jb = uint64_t(wave) + uint64_t(NW) * u;
      const uint64_t jq = jb / np, p = jb - jq * np, tl = jq >> lp, pl = jq & ((uint64_t(1) << lp) - 1);
      const uint64_t tile = uint64_t(blockIdx.x) + G * tl;
      const bool real = jb < njobs && tile < ntiles;  // wave-uniform
      js0[u] = real ? p * D : 0;
      jnu[u] = real ? (nsteps - js0[u] < uint64_t(D) ? nsteps - js0[u] : uint64_t(D)) : 1;
      const v4i* bp = real ? reinterpret_cast<const v4i*>(q + ((tile << lp) + pl) * nsteps * 2048 + lane * 16)
                           : reinterpret_cast<const v4i*>(q);
      const uint64_t sstride = real ? 128 : 0;
#pragma unroll
      for (int d = 0; d < D; ++d) {
        const uint64_t st = js0[u] + (uint64_t(d) < jnu[u] ? uint64_t(d) : jnu[u] - 1);
        b[u][2 * d] = __builtin_nontemporal_load(bp + st * sstride);
        b[u][2 * d + 1] = __builtin_nontemporal_load(bp + st * sstride + (real ? kHalfV4 : 0));
      }
    }
  };
  // 3. residual norm of the whole row
  int64_t ss = 0;
#pragma unroll
  for (int e = 0; e < QPT; ++e) {
    const bool on = threadIdx.x + uint64_t(NT) * e < Q;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int32_t o = on ? requant(sv[e][k]) : 0;
      sv[e][k] = o;
      ss = add_sat64_nn(ss, sq_term(o));
    }
  }
  // the first job's weights go out once the norm inputs are in, the others
  // after the first scale: the first job's loads are in flight while the scale
  // chain and the residual run, instead of every wave waiting to issue all its
  // loads before any of that arithmetic
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using IJ = std::integral_constant<int, JM>;
  const int32_t s1 = wg_rms_scale<NW>(ss, ni.H, ni.eps, red[0], &bc, wave, lane, [&] { issue_weights(I0(), I1()); });
  ss = 0;
#pragma unroll
  for (int e = 0; e < QPT; ++e) {
    const bool on = threadIdx.x + uint64_t(NT) * e < Q;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      int32_t v = add_sat(xv[e][k], mul_sat(mul_sat(int32_t(sv[e][k]), s1), wp[e][k]));
      if (ni.has_scalar) v = mul_sat(v, ni.scalar);
      v = on ? v : 0;
      xv[e][k] = v;
      ss = add_sat64_nn(ss, sq_term(v));
    }
  }
  const int32_t s2 = wg_rms_scale<NW>(ss, ni.H, ni.eps, red[1], &bc, wave, lane, [&] { issue_weights(I1(), IJ()); });
  // limb planes of the normalised row (quads past H are zero, to kpad / 4)
  const uint64_t kq = kpad / 4;
#pragma unroll
  for (int e = 0; e < QPT; ++e) {
    const uint64_t qd = threadIdx.x + uint64_t(NT) * e;
    const bool on = qd < Q;
    if (qd < kq) {
      uint32_t pk[4] = {0, 0, 0, 0};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t u = on ? uint32_t(mul_sat(mul_sat(xv[e][k], s2), wn[e][k])) ^ 0x00808080u : 0u;
#pragma unroll
        for (int j = 0; j < 4; ++j) pk[j] |= ((u >> (8 * j)) & 0xffu) << (8 * k);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) *reinterpret_cast<uint32_t*>(al + j * plane + 4 * qd) = pk[j];
    }
  }
  lds_barrier();
  // 4. MFMAs: A row i < 4 is limb i of the row (plane i, bytes [32 g, 32 g + 32) of each step)
  const bool a_on = i < 4;
  const uint8_t* aread = al + (i & 3) * plane + 32 * g;
  const v4i zero = {0, 0, 0, 0};
#pragma unroll
  for (int u = 0; u < JM; ++u) {
    v4i acc = zero;
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const uint64_t st = js0[u] + (uint64_t(d) < jnu[u] ? uint64_t(d) : jnu[u] - 1);
      const int m = (a_on && uint64_t(d) < jnu[u]) ? -1 : 0;
      const v4i a0 = *reinterpret_cast<const v4i*>(aread + st * 128) & m;
      const v4i a1 = *reinterpret_cast<const v4i*>(aread + st * 128 + 16) & m;
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b[u][2 * d], acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b[u][2 * d + 1], acc, 0, 0, 0);
    }
    part[wave + NW * u][lane] = acc;
  }
  __syncthreads();
  // 5. lanes 16 g + i of wave w take row i of tile 4 w + g (four tiles per
  // wave, so the GELU epilogue runs on every lane group): the row's four limb
  // sums sit in lane i (g = 0) of each of the tile's part slots
  for (uint64_t tl0 = 4 * uint64_t(wave); tl0 < tpw; tl0 += 4 * uint64_t(NW)) {
    const uint64_t tl = tl0 + uint64_t(g);
    const uint64_t tile = uint64_t(blockIdx.x) + G * tl;
    const bool t_ok = tl < tpw && tile < ntiles;
    int64_t p[4] = {0, 0, 0, 0};
    if (t_ok)
      for (int pl = 0; pl < (1 << lp); ++pl)
        for (uint64_t pp = 0; pp < np; ++pp) {
          const v4i v = part[tl * npt + pl * np + pp][i];
#pragma unroll
          for (int j = 0; j < 4; ++j) p[j] += int64_t(uint64_t(int64_t(v[j])) << (8 * pl));
        }
    const uint64_t row = tile * 16 + i;
    const bool ok = t_ok && row < n_rows;
    const bool first = tl0 == 4 * uint64_t(wave);
    const int32_t rs = first ? ers : (ok ? rowsum[row] : 0);
    const int32_t sc = first ? esc : (ok ? scale[row] : 0);
    const int64_t a = ok ? limb_combine(p, rs, sc) : 0;
    if (EPI == 1) {
      const int32_t r = requant(a);
      const int32_t up = __shfl(r, (lane & 48) | ((i + 8) & 15), 64);
      if (ok && i < 8) {
        const uint64_t f = tile * 8 + i;
        const int32_t h = mul_sat(gelu_act(r), up);
        out[f] = h;
        const uint32_t uh = uint32_t(h) ^ 0x00808080u;
#pragma unroll
        for (int j = 0; j < 4; ++j) out_limbs[j * out_kpad + f] = int8_t(uint8_t(uh >> (8 * j)));
      }
    } else if (ok) {
      acc_out[row] = a;
    }
  }
  // 6. the new residual row (workgroup 0) and the cleared buffer
  if (blockIdx.x == 0)
#pragma unroll
    for (int e = 0; e < QPT; ++e) {
      const uint64_t qd = threadIdx.x + uint64_t(NT) * e;
      if (qd < Q) {
        const v4i x4 = {xv[e][0], xv[e][1], xv[e][2], xv[e][3]};
        *reinterpret_cast<v4i*>(ni.x_out + 4 * qd) = x4;
        if (ni.row_out) *reinterpret_cast<v4i*>(ni.row_out + 4 * qd) = x4;
      }
    }
  if (ni.clear)
    for (uint64_t idx = uint64_t(blockIdx.x) * NT + threadIdx.x; idx < ni.clear_n; idx += G * NT) ni.clear[idx] = 0;
}

// Decode GEMV for 5-16 tokens (NG = 2 or 4 groups of 4): the A tiles of a K
// step are as large as the weight tile or larger, so the four waves of a
// workgroup take four consecutive weight tiles over the same K steps and
// share each step's A tiles through LDS (two buffers; the next step's weight
// and A loads are issued before the current step's MFMAs, one barrier per
// step). Outputs as in k_gemv_dec; kchunks splits K across workgroups
// (atomic outputs only).
// IN64: the activation rows are wrapped Q32.32 accumulator rows (row stride
// in_ld, even; K a multiple of 128 and equal to kpad), requantized and split
// into limbs while a step's A tiles are written to LDS: each thread loads
// 2 NG consecutive accumulators of one token (16-byte loads) and writes their
// four limb bytes.
template <int EPI, int NG, bool DG, bool IN64 = false>
__global__ __launch_bounds__(256, 4) void k_gemv_dec_wg(
    const int8_t* __restrict__ q, const int32_t* __restrict__ scale, const int32_t* __restrict__ rowsum,
    const int8_t* __restrict__ limbs, uint64_t n_rows, uint64_t kpad, uint32_t kchunks, uint32_t ntok,
    int32_t* __restrict__ out, uint64_t out_ld, int64_t* __restrict__ acc_out, uint64_t acc_ld,
    int8_t* __restrict__ out_limbs, uint64_t out_kpad, int lp_arg, const int64_t* __restrict__ acc_in = nullptr,
    uint64_t in_ld = 0, int8_t* __restrict__ out_om = nullptr) {
  const int lp = DG ? lp_arg : 0;  // (single-plane instances fold it to 0)
  __shared__ v4i al[2][NG][2][64];  // [buffer][token group][half][lane]
  const int planes = 1 << lp;  // digit planes
  constexpr int CH = IN64 ? NG : (NG * 2 * 64 + 255) / 256;  // A loads (16 bytes) per thread and step
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, i = lane & 15;
  const uint64_t nsteps = kpad / 128;
  const uint32_t kc = blockIdx.x % kchunks;
  const uint64_t cper = (nsteps + kchunks - 1) / kchunks;
  const uint64_t cs0 = kc * cper < nsteps ? kc * cper : nsteps;
  const uint64_t cs1 = cs0 + cper < nsteps ? cs0 + cper : nsteps;
  const uint64_t ntiles = (n_rows + 15) / 16;
  const uint64_t groups = gridDim.x / kchunks;
  const v4i zero = {0, 0, 0, 0};
  static_assert(NG * 128 % 256 == 0, "every thread copies whole A chunks");
  // this thread's share of a step's A tiles: chunk e = tid + 256 c is lane
  // e % 64, half (e / 64) % 2, token group e / 128 of the LDS buffer. Every
  // load below is unconditional (tokens >= ntok read limb row 0 and tiles
  // past the matrix read tile 0, whose products land only in outputs that are
  // never written), so the loads issue back to back without exec-masked
  // branches between them.
  const v4i* asrc[CH];
  // IN64: token itok, columns icol .. icol + 2 NG - 1 of every K step
  constexpr uint32_t VPT = 2 * NG, TPR = 128 / VPT;
  const uint32_t itok = threadIdx.x / TPR, icol = (threadIdx.x % TPR) * VPT;
  if (IN64) {
    const int64_t* row = acc_in + uint64_t(itok < ntok ? itok : 0) * in_ld + icol;
#pragma unroll
    for (int c = 0; c < CH; ++c) asrc[c] = reinterpret_cast<const v4i*>(row + 2 * c);
  } else {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const uint32_t e = threadIdx.x + 256 * c;
      const uint32_t ln = e & 63, h = (e >> 6) & 1, tg = e >> 7;
      const bool on = 4 * tg + ((ln & 15) >> 2) < ntok;
      asrc[c] = reinterpret_cast<const v4i*>(limbs + (on ? uint64_t(16 * tg + (ln & 15)) * kpad : 0) +
                                             32 * (ln >> 4) + 16 * h);
    }
  }
  // a K step's A loads sit 128 columns apart: 8 v4i of limb bytes, 64 of accumulators
  constexpr uint64_t ASTEP = IN64 ? 64 : 8;
  // LDS bytes of limb 0 of this thread's columns (lane 16 g + 4 ti + j of
  // token group tg, half h, byte b; limb j adds 16 j)
  const uint32_t lds_in64 = (((itok >> 2) * 2 + ((icol >> 4) & 1)) * 64 + 16 * (icol >> 5) + 4 * (itok & 3)) * 16 +
                            (icol & 15);
  auto store_a = [&](int buf, const v4i* ar) {
    if (IN64) {
      uint32_t u[VPT];
#pragma unroll
      for (int c = 0; c < CH; ++c) {
        u[2 * c] = uint32_t(requant(int64_t(uint64_t(uint32_t(ar[c][0])) | uint64_t(uint32_t(ar[c][1])) << 32))) ^
                   0x00808080u;
        u[2 * c + 1] =
            uint32_t(requant(int64_t(uint64_t(uint32_t(ar[c][2])) | uint64_t(uint32_t(ar[c][3])) << 32))) ^
            0x00808080u;
      }
      char* dst = reinterpret_cast<char*>(&al[buf][0][0][0]) + lds_in64;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t w[VPT / 4];
#pragma unroll
        for (int v = 0; v < int(VPT / 4); ++v)
          w[v] = ((u[4 * v] >> (8 * j)) & 0xffu) | ((u[4 * v + 1] >> (8 * j)) & 0xffu) << 8 |
                 ((u[4 * v + 2] >> (8 * j)) & 0xffu) << 16 | ((u[4 * v + 3] >> (8 * j)) & 0xffu) << 24;
        if (VPT == 8)
          *reinterpret_cast<uint2*>(dst + 16 * j) = make_uint2(w[0], w[VPT / 4 - 1]);
        else
          *reinterpret_cast<uint32_t*>(dst + 16 * j) = w[0];
      }
    } else {
#pragma unroll
      for (int c = 0; c < CH; ++c) (&al[buf][0][0][0])[threadIdx.x + 256 * c] = ar[c];
    }
  };
  // the four waves take four consecutive virtual tiles (digit plane p of tile
  // t is virtual tile t * planes + p), whole tiles per workgroup pass
  const uint64_t vtiles = ntiles << lp;
  for (uint64_t base = uint64_t(blockIdx.x / kchunks) * 4; base < vtiles; base += groups * 4) {
    const uint64_t vt = base + wave;
    const bool t_on = vt < vtiles;
    const uint64_t tile = vt >> lp;
    const int plane = int(vt & uint64_t(planes - 1));
    const v4i* bp = reinterpret_cast<const v4i*>(q + (t_on ? vt : 0) * nsteps * 2048 + lane * 16);
    v4i acc[NG];
#pragma unroll
    for (int tg = 0; tg < NG; ++tg) acc[tg] = zero;
    v4i b0 = zero, b1 = zero, ar[CH];
    if (cs0 < cs1) {
      b0 = __builtin_nontemporal_load(bp + cs0 * 128);
      b1 = __builtin_nontemporal_load(bp + cs0 * 128 + kHalfV4);
#pragma unroll
      for (int c = 0; c < CH; ++c) ar[c] = asrc[c][cs0 * ASTEP];
    }
    for (uint64_t s = cs0; s < cs1; ++s) {
      const int buf = int((s - cs0) & 1);
      store_a(buf, ar);
      __syncthreads();
      v4i n0 = zero, n1 = zero;
      if (s + 1 < cs1) {
        n0 = __builtin_nontemporal_load(bp + (s + 1) * 128);
        n1 = __builtin_nontemporal_load(bp + (s + 1) * 128 + kHalfV4);
#pragma unroll
        for (int c = 0; c < CH; ++c) ar[c] = asrc[c][(s + 1) * ASTEP];
      }
#pragma unroll
      for (int tg = 0; tg < NG; ++tg) {
        acc[tg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[buf][tg][0][lane], b0, acc[tg], 0, 0, 0);
        acc[tg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[buf][tg][1][lane], b1, acc[tg], 0, 0, 0);
      }
      b0 = n0;
      b1 = n1;
    }
    __syncthreads();  // both buffers are read before the next tile group refills them
    // a tile's digit planes: the plane-0 wave adds the others' partial tiles
    // (through the A buffers, free until the next pass) with shifts
    int64_t pt[NG][4];
#pragma unroll
    for (int tg = 0; tg < NG; ++tg)
#pragma unroll
      for (int j = 0; j < 4; ++j) pt[tg][j] = acc[tg][j];
    if (planes > 1) {
      v4i* xs = &al[0][0][0][0];
#pragma unroll
      for (int tg = 0; tg < NG; ++tg) xs[(wave * NG + tg) * 64 + lane] = acc[tg];
      __syncthreads();
      if (plane == 0)
        for (int w = 1; w < planes; ++w)
#pragma unroll
          for (int tg = 0; tg < NG; ++tg) {
            const v4i v = xs[((wave + w) * NG + tg) * 64 + lane];
#pragma unroll
            for (int j = 0; j < 4; ++j) pt[tg][j] += int64_t(uint64_t(int64_t(v[j])) << (8 * w));
          }
      __syncthreads();
    }
    if (!t_on || plane != 0) continue;
    const uint64_t row = tile * 16 + i;
    const bool r_on = row < n_rows;
    const int32_t rs = r_on ? rowsum[row] : 0, sc = r_on ? scale[row] : 0;
    // lane 16 g + i of group tg holds the limb sums of token 4 tg + g, row i
#pragma unroll
    for (int tg = 0; tg < NG; ++tg) {
      const int64_t p[4] = {pt[tg][0], pt[tg][1], pt[tg][2], pt[tg][3]};
      const uint32_t tok = 4 * tg + g;
      const bool ok = tok < ntok && r_on;
      if (acc_out) {
        if (ok) {
          const int64_t a = limb_combine(p, kc == 0 ? rs : 0, sc);
          atomicAdd(reinterpret_cast<unsigned long long*>(acc_out + tok * acc_ld + row),
                    static_cast<unsigned long long>(a));
        }
      } else if (EPI == 1) {
        const int32_t r = ok ? requant(limb_combine(p, rs, sc)) : 0;
        const int32_t up = __shfl(r, (lane & 48) | ((i + 8) & 15), 64);
        if (ok && i < 8) {
          const uint64_t f = tile * 8 + i;
          const int32_t h = mul_sat(gelu_act(r), up);
          out[tok * out_ld + f] = h;
          const uint32_t u = uint32_t(h) ^ 0x00808080u;
          int8_t* ol = out_limbs + uint64_t(tok) * 4 * out_kpad + f;
#pragma unroll
          for (int j = 0; j < 4; ++j) ol[j * out_kpad] = int8_t(uint8_t(u >> (8 * j)));
          if (out_om)
#pragma unroll
            for (int j = 0; j < 4; ++j) out_om[om_offset(out_kpad, tok, f, j)] = int8_t(uint8_t(u >> (8 * j)));
        }
      } else if (ok) {
        out[tok * out_ld + row] = requant(limb_combine(p, rs, sc));
      }
    }
  }
}

// Decode GEMV for 5-16 tokens (NG = 2 or 4 groups of 4) with the activation
// limbs resident in registers. The NW waves of a workgroup split a K chunk of
// NW * HPW half-steps (64 columns: half h of 128-column step s is half-step
// 2 s + h); each wave loads the A operands of its HPW half-steps for all NG
// token groups once, then streams its K share of the workgroup's weight
// tiles: a tile's half-step operands are HPW contiguous 1 KB blocks, and the
// next tile's are in flight while this tile's MFMAs run (no barrier between
// the K steps). The waves' partial limb sums of a tile
// (int32; a limb times a weight is at most 128 * 127 in magnitude, so K
// chunks up to 130000 columns cannot wrap) are added through LDS, one
// LDS-only barrier per tile, and wave w combines token groups w, w + NW, ...
// as k_gemv_dec_wg does. Workgroup b takes K chunk b % kchunks
// (kchunks > 1: atomic acc_out only) and tiles b / kchunks + groups * j.
// Half-steps past kpad are read clamped to the last one with zero A operands.
// EPI 1 (gate/up rows interleaved per tile, kchunks 1): the combining waves
// stage each tile's requantized values in LDS, and every kStage tiles (and at
// the end) all the workgroup's lanes form the mul_sat(gelu(gate), up)
// products, one product per lane, rather than half the lanes of NG waves
// between two tiles' barriers.
template <int EPI, int NG, int NW, int HPW>
__global__ __launch_bounds__(64 * NW, 1) void k_gemv_rega(
    const int8_t* __restrict__ q, const int32_t* __restrict__ scale, const int32_t* __restrict__ rowsum,
    const int8_t* __restrict__ limbs, uint64_t n_rows, uint64_t kpad, uint32_t kchunks, uint32_t ntok,
    int32_t* __restrict__ out, uint64_t out_ld, int64_t* __restrict__ acc_out, uint64_t acc_ld,
    int8_t* __restrict__ out_limbs, uint64_t out_kpad, const int8_t* __restrict__ a_om = nullptr,
    int8_t* __restrict__ out_om = nullptr) {
  constexpr int kStage = 8;
  __shared__ v4i red[2][NW][NG][64];  // [tile parity][wave][token group][lane]
  __shared__ int32_t stage[EPI == 1 ? kStage : 1][NG][64];
  __shared__ uint64_t stage_tile[kStage];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int g = lane >> 4, i = lane & 15;
  const uint64_t nhs = kpad / 64;
  const uint32_t kc = blockIdx.x % kchunks;
  const uint64_t hs0 = (uint64_t(kc) * NW + uint64_t(wave)) * HPW;
  const uint64_t ntiles = (n_rows + 15) / 16;
  const uint64_t groups = gridDim.x / kchunks;
  const uint64_t t0 = blockIdx.x / kchunks;
  const v4i zero = {0, 0, 0, 0};
  const uint64_t my_tiles = t0 < ntiles ? (ntiles - t0 + groups - 1) / groups : 0;
  // this wave's first half-step operand of tile j (tiles past the end read the last tile)
  const v4i* qw = reinterpret_cast<const v4i*>(q) + lane;
  auto tile_of = [&](uint64_t j) {
    const uint64_t t = t0 + groups * j;
    return t < ntiles ? t : ntiles - 1;
  };
  auto hs_of = [&](int h) { return hs0 + h < nhs ? hs0 + h : nhs - 1; };
  v4i wb[2][HPW];
  int32_t rsr[2], scr[2];
  // the epilogue's row sum and scale of tile j, loaded just ahead of its weights
  auto issue = [&](int r, uint64_t j) {
    const uint64_t t = tile_of(j);
    const uint64_t row = t * 16 + uint64_t(i) < n_rows ? t * 16 + uint64_t(i) : n_rows - 1;
    rsr[r] = rowsum[row];
    scr[r] = scale[row];
#pragma unroll
    for (int h = 0; h < HPW; ++h) wb[r][h] = __builtin_nontemporal_load(qw + (t * nhs + hs_of(h)) * 64);
  };
  // A operand of (half-step hs, token group tg) in lane 16 g + i: limb row
  // 16 tg + i (token 4 tg + i / 4, limb i % 4), columns 128 s + 32 g + 16 h
  // (clamped addresses, masked values: no predicated loads)
  // (from the operand-major copy when given: one contiguous 1 KB per load)
  v4i ar[HPW][NG];
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    const uint64_t hs = hs0 + h;
    const bool k_on = hs < nhs;
    const uint64_t col = k_on ? 128 * (hs >> 1) + 32 * g + 16 * (hs & 1) : 0;
#pragma unroll
    for (int tg = 0; tg < NG; ++tg) {
      const bool on = k_on && uint32_t(4 * tg + (i >> 2)) < ntok;
      const v4i v = a_om ? reinterpret_cast<const v4i*>(a_om)[((k_on ? hs : 0) * 4 + tg) * 64 + lane]
                         : *reinterpret_cast<const v4i*>(limbs + uint64_t(on ? 16 * tg + i : 0) * kpad + col);
      ar[h][tg] = on ? v : zero;
    }
  }
  issue(0, 0);
  issue(1, 1);
  // EPI 1: the staged tiles' products, lane by lane (token-major within a
  // tile: product p = tok * 8 + f of staged tile slot)
  auto flush = [&](uint32_t cnt) {
    lds_barrier();
    for (uint32_t idx = threadIdx.x; idx < cnt * NG * 32; idx += 64 * NW) {
      const uint32_t slot = idx / (NG * 32), rem = idx % (NG * 32);
      const uint32_t tok = rem >> 3, f8 = rem & 7;
      const uint64_t tile = stage_tile[slot];
      const uint32_t ln = 16 * (tok & 3) + f8;
      const int32_t gate = stage[slot][tok >> 2][ln], up = stage[slot][tok >> 2][ln + 8];
      if (tok < ntok && tile * 16 + f8 < n_rows) {
        const uint64_t f = tile * 8 + f8;
        const int32_t hv = mul_sat(gelu_act(gate), up);
        out[tok * out_ld + f] = hv;
        const uint32_t u = uint32_t(hv) ^ 0x00808080u;
        int8_t* ol = out_limbs + uint64_t(tok) * 4 * out_kpad + f;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) ol[jj * out_kpad] = int8_t(uint8_t(u >> (8 * jj)));
        if (out_om)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) out_om[om_offset(out_kpad, tok, f, jj)] = int8_t(uint8_t(u >> (8 * jj)));
      }
    }
    lds_barrier();
  };
  uint32_t nst = 0;
  for (uint64_t j0 = 0; j0 < my_tiles; j0 += 2) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint64_t j = j0 + r;
      if (j < my_tiles) {
        v4i acc[NG];
#pragma unroll
        for (int tg = 0; tg < NG; ++tg) acc[tg] = zero;
#pragma unroll
        for (int h = 0; h < HPW; ++h)
#pragma unroll
          for (int tg = 0; tg < NG; ++tg)
            acc[tg] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ar[h][tg], wb[r][h], acc[tg], 0, 0, 0);
        const int32_t rs = rsr[r], sc = scr[r];
        issue(r, j + 2);
#pragma unroll
        for (int tg = 0; tg < NG; ++tg) red[r][wave][tg][lane] = acc[tg];
        lds_barrier();
        const uint64_t tile = t0 + groups * j;
        if (EPI == 1 && wave == 0 && lane == 0) stage_tile[nst] = tile;
#pragma unroll
        for (int tg = wave; tg < NG; tg += NW) {
          // lane 16 g + i holds the limb sums of token 4 tg + g, row i
          v4i s = red[r][0][tg][lane];
#pragma unroll
          for (int w = 1; w < NW; ++w) s += red[r][w][tg][lane];
          const int64_t p[4] = {s[0], s[1], s[2], s[3]};
          const uint64_t row = tile * 16 + uint64_t(i);
          const uint32_t tok = 4 * uint32_t(tg) + uint32_t(g);
          const bool ok = tok < ntok && row < n_rows;
          if (acc_out) {
            if (ok)
              atomicAdd(reinterpret_cast<unsigned long long*>(acc_out + tok * acc_ld + row),
                        static_cast<unsigned long long>(limb_combine(p, kc == 0 ? rs : 0, sc)));
          } else if (EPI == 1) {
            stage[nst][tg][lane] = ok ? requant(limb_combine(p, rs, sc)) : 0;
          } else if (ok) {
            out[tok * out_ld + row] = requant(limb_combine(p, rs, sc));
          }
        }
        if (EPI == 1 && ++nst == kStage) {
          flush(kStage);
          nst = 0;
        }
      }
    }
  }
  if (EPI == 1 && nst > 0) flush(nst);
}

// ---------------------------------------------------------------------------
// Prefill GEMM (det_linear_slab, det_kernels.rs:180-203): C[m][n] =
// requantize(sum_k act[m][k] * W[n][k]) for a slab of M activation rows.
//
// The activations enter as limb rows: row 4m + j holds byte j of
// act[m][k] ^ 0x00808080 (the four int8 limbs c_j with
// act = sum_j c_j 256^j + 8421504), in tiles like the tile-major weights
// (16-row tiles x 128-column steps of 2 KB; MFMA lane 16g + i of a step takes
// row i, columns [32g, 32g + 32)). A 16x16x64 MFMA of an A tile (4 tokens x
// 4 limbs) with a weight tile leaves the four limb sums of (token g, weight
// row i) in lane 16g + i, which are combined exactly as in the GEMV.
// ---------------------------------------------------------------------------


// Prefill GEMM A operand: activation rows as limb-major token groups. Token
// group T (tokens 16 T .. 16 T + 15) has four limb tiles T 4 + j; tile-step
// (tile, s) is 2048 bytes of 32-byte lane slots (slot 16 g + i: token 16 T + i,
// columns [128 s + 32 g, +32); the weights store the two 16-byte halves of a
// lane's columns 1 KB apart instead, which only the copy addresses see), so an
// MFMA A operand is one
// limb of 16 tokens and the four limb products of (token, row) land in the
// same lane of four accumulators.
// The decomposition is chosen per token group and column part of
// kLimbPartCols: where the part's activations all lie in [-2^23, 2^23), three
// limbs: with u = (a + 2^23) ^ 0x808080, a = sum_{j<3} c_j 256^j + 32896 (c_j
// the signed bytes of u; its top byte is 0, so the fourth limb tile is zero
// and the GEMM skips it); otherwise u = a ^ 0x808080, a = sum_{j<4} c_j 256^j
// + 8421504. flags[T * parts + p] = 1 marks the four-limb parts.
// One workgroup per (16-token group T, part), NT threads (LPT = NT / 16 per
// token): thread (r, l) reads token 16 T + r's columns 4 l + 4 LPT q + [0, 4)
// of the part, so each load instruction covers 64 / LPT rows x 16 LPT
// contiguous bytes (vec: act rows are 16-byte aligned, base and ld, and load
// as 128-bit reads); the workgroup decides the part's decomposition
// (__syncthreads_or); the limb bytes are regrouped in LDS into the tile-step
// layout (limb j, step, lane slot 16 g + i of 32 bytes: token i's columns
// 32 g + [0, 32) of the step) and copied out in whole 16-byte pieces, each
// tile-step a contiguous 2 KB. Tokens past m and columns past k are zero.
// 1024 threads for grids of up to 256 workgroups and 512 for up to 512
// (shorter chains per thread), else 256: at 128 rows 3.1 us on 512 threads
// against 4.3 us for 256 threads and 512-column parts (K = 2560), at 2048 rows
// x 10240 columns 24.6 against 26.1 us.
template <int NT>
__global__ __launch_bounds__(NT) void k_act_limbs_rows(const int32_t* __restrict__ act, uint64_t m, uint64_t k,
                                                      uint64_t ld, uint64_t kpad, int vec,
                                                      uint32_t* __restrict__ flags, int8_t* __restrict__ out) {
  constexpr int PC = int(kLimbPartCols), PS = PC / 128;  // columns and K steps per part
  constexpr int LPT = NT / 16, Q = PC / (4 * LPT);       // threads per token, loads per thread
  static_assert(Q >= 1 && PC % (4 * LPT) == 0, "whole 16-byte loads per thread");
  __shared__ __attribute__((aligned(16))) uint32_t st[4][PS][64][8];
  const uint64_t nsteps = kpad / 128, parts = limb_parts(kpad);
  const uint64_t T = blockIdx.x, part = blockIdx.y;
  const uint32_t r = threadIdx.x / LPT, l = threadIdx.x % LPT;
  const uint64_t t = 16 * T + r;
  const bool row_on = t < m;
  const int32_t* src = act + (row_on ? t : 0) * ld;
  const uint64_t c0 = part * PC + 4 * l;
  uint32_t a[4 * Q];
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const uint64_t c = c0 + 4 * LPT * q;
    if (vec && row_on && c + 4 <= k) {
      const int4 v = *reinterpret_cast<const int4*>(src + c);
      a[4 * q] = uint32_t(v.x), a[4 * q + 1] = uint32_t(v.y), a[4 * q + 2] = uint32_t(v.z), a[4 * q + 3] = uint32_t(v.w);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) a[4 * q + e] = (row_on && c + e < k) ? uint32_t(src[c + e]) : 0u;
    }
  }
  uint32_t wide = 0;
#pragma unroll
  for (int e = 0; e < 4 * Q; ++e) wide |= a[e] + 0x800000u >= 0x1000000u;
  const bool four = __syncthreads_or(int(wide)) != 0 || parts > kLimbMaxParts;
  if (threadIdx.x == 0) flags[T * parts + part] = four ? 1u : 0u;
  const uint32_t off = four ? 0u : 0x800000u;
  // column cp = 4 l + 4 LPT q + e of the part: step cp / 128, lane group
  // g = (cp % 128) / 32, byte cp % 32 of the lane slot (word (cp % 32) / 4)
#pragma unroll
  for (int q = 0; q < Q; ++q) {
    const uint32_t cp = 4 * l + 4 * LPT * q;
    uint32_t u[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) u[e] = (row_on && c0 + 4 * LPT * q + e < k) ? (a[4 * q + e] + off) ^ 0x00808080u : 0u;
    const uint32_t sl = cp / 128, g = (cp % 128) / 32, w = (cp % 32) / 4;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      st[j][sl][16 * g + r][w] = ((u[0] >> (8 * j)) & 0xffu) | ((u[1] >> (8 * j)) & 0xffu) << 8 |
                                 ((u[2] >> (8 * j)) & 0xffu) << 16 | ((u[3] >> (8 * j)) & 0xffu) << 24;
  }
  __syncthreads();
  // 4 PS tile-steps of 2 KB (limb j, step sl of the part), 128 pieces each
  constexpr int PIECES = 4 * PS * 128;
  static_assert(PIECES % NT == 0, "whole pieces per thread");
#pragma unroll
  for (int kq = 0; kq < PIECES / NT; ++kq) {
    const uint32_t p = threadIdx.x + NT * kq, chunk = p >> 7, j = chunk / PS, sl = chunk % PS;
    const uint64_t step = part * PS + sl;
    if (step < nsteps)
      *reinterpret_cast<int4*>(out + ((4 * T + j) * nsteps + step) * 2048 + (p & 127) * 16) =
          reinterpret_cast<const int4*>(&st[j][sl][0][0])[p & 127];
  }
}

// Block: TA A tiles (TA / 4 token groups of 16 tokens, four limb tiles each)
// x TB weight tiles on WM x WN waves, each wave (TA / WM) x (TB / WN) MFMA
// tiles (whole token groups). A block whose token groups all take three limbs
// multiplies no fourth-limb tile, and with two buffers does not copy them
// either (with more, every wave copies a fixed number of tile-step halves per
// step, so that one vmcnt immediate covers the steps in flight). Every
// 128-column K step, the block's
// TA + TB tile-steps (2 KB each) are copied straight from global memory into
// one of NBUF LDS buffers with global_load_lds_dwordx4 (no register staging).
// The 2 (TA + TB) copy halves are dealt out LPW per wave; where they do not
// divide evenly, the slots past them re-copy the block's first weight
// tile-step half into the buffer's spare kilobytes, so that every wave issues
// the same copies per step:
// the copies of the next NBUF - 1 steps are in flight while step s's MFMAs
// run, and one barrier per step hands a buffer over. Copy h of a tile-step
// takes the 16-byte half h of every lane's 32 columns (a weight tile-step's
// contiguous half h; bytes [16 h, 16 h + 16) of each 32-byte slot of an
// activation tile-step), so each 1 KB LDS half holds one MFMA operand of all
// 64 lanes contiguously
// and the 128-bit operand reads do not conflict on LDS banks. The MFMAs of a
// step run as two passes over the wave's tile pairs (first 64 columns, then
// the second 64), so consecutive MFMAs never share an accumulator.
// GELU: W holds tiles of 8 gate rows and the matching 8 up rows (rows
// 16 t + i, i < 8: gate row 8 t + i; rows 16 t + 8 + i: up row 8 t + i) and
// out[token][8 t + i] = mul_sat(gelu(gate), up) (the decode step's gate/up
// epilogue; no other output form).
template <int TA, int TB, int WM, int WN, uint32_t GM, int NBUF, bool SPLIT, bool GELU, bool DG>
__global__ __launch_bounds__(64 * WM * WN) void k_gemm_lds(const int8_t* __restrict__ a, const int8_t* __restrict__ q,
                                                           const int32_t* __restrict__ scale,
                                                           const int32_t* __restrict__ rowsum,
                                                           const int32_t* __restrict__ rowsum_p, uint64_t rowsum_p_ld,
                                                           uint64_t n_rows, uint64_t kpad, uint64_t m_tokens,
                                                           uint64_t a_tiles, const uint32_t* __restrict__ a_flags,
                                                           uint32_t mblocks, int32_t* __restrict__ out,
                                                           uint64_t ld_out, int64_t* __restrict__ acc_out,
                                                           RowSplit split, KSplit ks, int lp_arg) {
  const int lp = DG ? lp_arg : 0;  // (single-plane instances fold it to 0)
  constexpr int NW = WM * WN;                  // waves
  constexpr int TS = TA + TB;                  // tile-steps per K step
  constexpr int LPW = (2 * TS + NW - 1) / NW;  // 1 KB wave copies per wave per K step
  constexpr int SLOTS = LPW * NW;               // 1 KB copy slots per LDS buffer (>= 2 TS)
  constexpr int FA = TA / WM, FB = TB / WN;    // MFMA tiles per wave
  static_assert(FA % 4 == 0 && NBUF >= 2, "whole token groups per wave");
  extern __shared__ __attribute__((aligned(16))) int8_t lds_gemm[];
  // the wave index as a scalar, so that copy addresses and LDS targets stay in SGPRs
  const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Block order: block b runs on XCD b % 8, and each XCD takes a contiguous
  // range of logical blocks; logical blocks go in groups of GM m-blocks x all
  // n-blocks with m fastest, so the blocks resident on one XCD at a time form
  // a compact GM x (resident / GM) patch whose A and weight tiles share its L2.
  // With K split into ks.chunks ranges, chunk c takes logical blocks
  // [c nblk, (c + 1) nblk) and the same ordering inside them.
  const uint32_t nall = gridDim.x, nblk = nall / ks.chunks;
  uint32_t logical = blockIdx.x;
  if (nall % 8 == 0) logical = (blockIdx.x % 8) * (nall / 8) + blockIdx.x / 8;
  const uint32_t chunk = logical / nblk;
  logical -= chunk * nblk;
  const uint32_t nblocks_n = nblk / mblocks;
  const uint32_t wm = wave / WN, wn = wave % WN;
  const uint32_t group = logical / (GM * nblocks_n), first_m = group * GM;
  const uint32_t gm = mblocks - first_m < GM ? mblocks - first_m : GM;
  const uint32_t in_group = logical - group * GM * nblocks_n;
  const uint32_t mb = first_m + in_group % gm, nb = in_group / gm;
  const uint64_t ksteps = kpad / 128, cper = (ksteps + ks.chunks - 1) / ks.chunks;
  const uint64_t k0 = uint64_t(chunk) * cper < ksteps ? uint64_t(chunk) * cper : ksteps;
  const uint64_t nsteps = (k0 + cper < ksteps ? k0 + cper : ksteps) - k0;  // this block's K steps
  // weight tiles are virtual: digit plane p of tile t is tile t * planes + p
  // (a block's FB tiles per wave hold whole tiles' planes)
  const uint64_t ntiles = (n_rows + 15) / 16 << lp;  // (lp = log2 of the digit planes)
  const int planes = 1 << lp;
  const uint64_t at0 = uint64_t(mb) * TA, bt0 = uint64_t(nb) * TB;
  // The block's decomposition flags, one vector load per token group (lane p
  // reads part p's flag, at clamped addresses), issued ahead of the first
  // step's copies so that waiting for them leaves the copies in flight.
  const uint64_t parts = limb_parts(kpad);
  const bool many = parts > kLimbMaxParts;  // (every part of every group takes four limbs)
  constexpr int NG = TA / 4;                // the block's token groups
  const uint64_t ngroups = a_tiles / 4;
  uint32_t flag[NG];
#pragma unroll
  for (int t = 0; t < NG; ++t) {
    const uint64_t grp = at0 / 4 + t < ngroups ? at0 / 4 + t : ngroups - 1;
    flag[t] = a_flags[grp * parts + (lane < parts ? lane : parts - 1)];
  }
  // this wave's copies: chunk c = wave * LPW + u is tile-step c / 2 (A tiles
  // first), half c % 2; tiles past the matrix re-read its last tile (their
  // results are never stored); fourth-limb A tiles are not copied in a
  // three-limb block (the first step copies them before the flags are known)
  const int8_t* src[LPW];
  bool limb3[LPW];
#pragma unroll
  for (int u = 0; u < LPW; ++u) {
    const uint32_t c = wave * LPW + u, ts = c >> 1, h = c & 1;
    const bool is_a = ts < uint32_t(TA);
    uint64_t tile = is_a ? at0 + ts : (ts < uint32_t(TS) ? bt0 + (ts - TA) : bt0);  // (spare slots: bt0)
    if (is_a ? tile >= a_tiles : tile >= ntiles) tile = (is_a ? a_tiles : ntiles) - 1;
    // (weight tile-steps hold each half of the lanes' operands contiguously;
    // the activation limb tiles keep the 32-byte lane slots)
    src[u] = (is_a ? a : q) + (tile * ksteps + k0) * 2048 + (is_a ? lane * 32 + h * 16 : h * kTileHalfBytes + lane * 16);
    limb3[u] = is_a && (ts & 3) == 3;
  }
  bool four = true;
  auto copy_step = [&](uint64_t s, int buf) {
#pragma unroll
    for (int u = 0; u < LPW; ++u) {
      const uint32_t c = wave * LPW + u;
      if (NBUF > 2 || four || !limb3[u])
        __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)(src[u] + s * 2048),
                                         (void __attribute__((address_space(3)))*)(lds_gemm + (buf * SLOTS + c) * 1024),
                                         16, 0, 0);
    }
  };
  const v4i zero = {0, 0, 0, 0};
  v4i acc[FA][FB];
#pragma unroll
  for (int i = 0; i < FA; ++i)
#pragma unroll
    for (int j = 0; j < FB; ++j) acc[i][j] = zero;
  // NBUF - 1 steps in flight ahead of the one being multiplied
#pragma unroll
  for (int p = 0; p < NBUF - 1; ++p)
    if (uint64_t(p) < nsteps) copy_step(p, p);
  // the epilogue's row sums and scales, loaded while the K loop runs
  const uint32_t g = lane >> 4, i = lane & 15;
  int32_t ep_rowsum[FB], ep_scale[FB];
#pragma unroll
  for (int tj = 0; tj < FB; ++tj) {
    const uint64_t row = ((bt0 + wn * FB + tj) >> lp) * 16 + i;
    const uint64_t rc = row < n_rows ? row : n_rows - 1;
    ep_rowsum[tj] = rowsum[rc];
    ep_scale[tj] = scale[rc];
  }
  // per token group, the parts that take four limbs (bit p); the block runs
  // four limbs when any group needs them anywhere (one limb count for the
  // whole K range: a loop that switches between the two forms per part needs
  // more registers than the larger block has)
  uint64_t gmask[NG];
  uint64_t fourmask = many ? 1 : 0;
#pragma unroll
  for (int t = 0; t < NG; ++t) {
    const uint64_t bits = __ballot(lane < parts && flag[t] != 0);
    gmask[t] = !many && at0 / 4 + t < ngroups ? bits : 0;
    fourmask |= gmask[t];
  }
  four = fourmask != 0;
  // vmcnt immediate: wait until at most (NBUF - 2) steps of copies are outstanding
  constexpr int kWait = (NBUF - 2) * LPW;
  static_assert(kWait < 64, "vmcnt range");
  constexpr int kWaitImm = (kWait & 15) | (7 << 4) | (15 << 8) | ((kWait >> 4) << 14);
  // Each wave waits for its own copies of a step (vmcnt, in issue order),
  // then the barrier makes every wave's copies of that step visible. A bare
  // s_barrier (not __syncthreads, whose fence would wait for every copy in
  // flight) between compiler memory barriers keeps the later steps' copies
  // outstanding across it.
  auto step_barrier = [&](bool more) {
    asm volatile("" ::: "memory");
    if (more) __builtin_amdgcn_s_waitcnt(kWaitImm);
    else __builtin_amdgcn_s_waitcnt(0);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
  };
  step_barrier(nsteps >= uint64_t(NBUF - 1));
  // the K loop with L limbs (A tiles with i % 4 >= L are neither read nor multiplied)
  auto kloop = [&](auto Lc) {
    constexpr int L = decltype(Lc)::value;
    for (uint64_t s = 0; s < nsteps; ++s) {
      const int buf = int(s % NBUF);
      const int8_t* base = lds_gemm + buf * SLOTS * 1024 + lane * 16;
      // the first half's operands, the copies, the second half's operands
      // (read while the first half's MFMAs run), then the MFMAs
      v4i ao[2][FA], bo[2][FB];
      auto read_half = [&](int h) {
#pragma unroll
        for (int j = 0; j < FB; ++j) bo[h][j] = *reinterpret_cast<const v4i*>(base + (TA + wn * FB + j) * 2048 + 1024 * h);
#pragma unroll
        for (int i = 0; i < FA; ++i)
          if ((i & 3) < L) ao[h][i] = *reinterpret_cast<const v4i*>(base + (wm * FA + i) * 2048 + 1024 * h);
      };
      read_half(0);
      if (s + NBUF - 1 < nsteps) copy_step(s + NBUF - 1, int((s + NBUF - 1) % NBUF));
      read_half(1);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < FA; ++i)
#pragma unroll
          for (int j = 0; j < FB; ++j)
            if ((i & 3) < L) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ao[h][i], bo[h][j], acc[i][j], 0, 0, 0);
      // step s + 1's copies are complete when no more than the later steps' are outstanding
      step_barrier(s + NBUF - 1 < nsteps);
    }
  };
  if (four) kloop(std::integral_constant<int, 4>());
  else kloop(std::integral_constant<int, 3>());
  // epilogue: lane 16 g + i holds, in component r of the four limb tiles of a
  // token group, the limb sums of token 16 group + 4 g + r and weight row 16 tile + i
#pragma unroll
  for (int tg = 0; tg < FA / 4; ++tg) {
    const uint64_t grp = (at0 + wm * FA) / 4 + tg;
    // this group's four-limb parts (a uniform select among the block's groups)
    uint64_t wmask = 0;
#pragma unroll
    for (int t = 0; t < NG; ++t)
      if (uint32_t(t) == wm * (FA / 4) + tg) wmask = gmask[t];
    // a tile's digit planes are consecutive virtual tiles of this wave: their
    // limb sums accumulate (shifted 8 bits per plane) until the last plane
    int64_t run[4] = {0, 0, 0, 0};
#pragma unroll
    for (int tj = 0; tj < FB; ++tj) {
    const uint64_t vt = bt0 + wn * FB + tj;
    const int plane = int(vt & uint64_t(planes - 1));
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int64_t d = int64_t(acc[4 * tg][tj][r]) + int64_t(acc[4 * tg + 1][tj][r]) * 256 +
                        int64_t(acc[4 * tg + 2][tj][r]) * 65536 + int64_t(acc[4 * tg + 3][tj][r]) * 16777216;
      run[r] = int64_t(uint64_t(run[r]) + (uint64_t(d) << (8 * plane)));
    }
    if (plane != planes - 1) continue;
    int64_t dsum[4] = {run[0], run[1], run[2], run[3]};
    run[0] = run[1] = run[2] = run[3] = 0;
    const uint64_t row = (vt >> lp) * 16 + i;
    const uint64_t rc = row < n_rows ? row : n_rows - 1;
    // the chunk holding column 0 adds the constant term (wrapping i64): the
    // decomposition's sum_p c_p S_p (S_p the row sum of part p), i.e. 32896 S
    // plus 8388608 S_p for every four-limb part p
    uint64_t cterm = 0;
    if (chunk == 0) {
      const bool all4 = many || wmask == (parts >= 64 ? ~uint64_t(0) : (uint64_t(1) << parts) - 1);
      cterm = uint64_t(int64_t(all4 ? 8421504 : 32896) * ep_rowsum[tj]);
      if (!all4)
        for (uint64_t gm = wmask; gm; gm &= gm - 1)
          cterm += uint64_t(int64_t(8388608) * rowsum_p[uint64_t(__builtin_ctzll(gm)) * rowsum_p_ld + rc]);
    }
    const uint64_t sc = uint64_t(int64_t(ep_scale[tj]));
    if constexpr (GELU) {
      int32_t val[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t dot = int64_t(uint64_t(dsum[r]) + cterm);
        val[r] = requant(int64_t(uint64_t(dot) * sc));
      }
      // lane i < 8 holds gate row i, lane i + 8 its up row: the lower lanes
      // take tokens 4 g and 4 g + 1, the upper lanes 4 g + 2 and 4 g + 3, each
      // receiving the other half's values of its tokens
      const bool lo = i < 8;
      const int32_t send0 = lo ? val[2] : val[0], send1 = lo ? val[3] : val[1];
      const int32_t recv0 = __shfl(send0, int(lane ^ 8u), 64), recv1 = __shfl(send1, int(lane ^ 8u), 64);
      const int32_t g0 = lo ? val[0] : recv0, u0 = lo ? recv0 : val[2];
      const int32_t g1 = lo ? val[1] : recv1, u1 = lo ? recv1 : val[3];
      const uint64_t f = (vt >> lp) * 8 + (i & 7);
      const uint64_t t0 = grp * 16 + 4 * g + (lo ? 0 : 2);
      if (row < n_rows) {  // (whole tiles: the up row is there too)
        if (t0 < m_tokens) out[t0 * ld_out + f] = mul_sat(gelu_act(g0), u0);
        if (t0 + 1 < m_tokens) out[(t0 + 1) * ld_out + f] = mul_sat(gelu_act(g1), u1);
      }
      continue;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint64_t token = grp * 16 + 4 * g + r;
      if (token >= m_tokens || row >= n_rows) continue;
      const int64_t dot = int64_t(uint64_t(dsum[r]) + cterm);
      const int64_t v = int64_t(uint64_t(dot) * sc);
      if (ks.chunks > 1) {
        // this K range's wrapping share
        ks.planes[(uint64_t(chunk) * m_tokens + token) * n_rows + row] = v;
        continue;
      }
      if (SPLIT) {
        // rows [0, r1) to out, [r1, r2) to out1, [r2, n_rows) to out2
        int32_t* o = out;
        uint64_t ld = ld_out, rr = row;
        if (row >= split.r2) o = split.out2, ld = split.ld2, rr = row - split.r2;
        else if (row >= split.r1) o = split.out1, ld = split.ld1, rr = row - split.r1;
        o[token * ld + rr] = requant(v);
      } else if (acc_out) {
        acc_out[token * ld_out + row] = v;
      } else {
        out[token * ld_out + row] = requant(v);
      }
    }
    }
  }
}

// Sum of the K-range planes of a split GEMM (wrapping, so exactly the
// accumulator), requantized to out (rows split as in k_gemm_lds) or written
// to acc_out; two outputs per thread.
__global__ __launch_bounds__(256) void k_gemm_reduce(const int64_t* __restrict__ planes, uint32_t chunks,
                                                     uint64_t m_tokens, uint64_t n_rows, int32_t* __restrict__ out,
                                                     uint64_t ld_out, int64_t* __restrict__ acc_out, RowSplit split) {
  const uint64_t total = m_tokens * n_rows;
  const uint64_t e0 = (uint64_t(blockIdx.x) * 256 + threadIdx.x) * 2;
  if (e0 >= total) return;
  const uint64_t plane = total;
  // every plane's two values are requested before the first is added (up to
  // kUnroll planes at clamped addresses, masked; more in a second loop)
  constexpr uint32_t kUnroll = 8;
  const uint64_t e1 = e0 + 1 < total ? e0 + 1 : e0;
  int64_t p0[kUnroll], p1[kUnroll];
#pragma unroll
  for (uint32_t c = 0; c < kUnroll; ++c) {
    const uint64_t cc = c < chunks ? c : 0;
    p0[c] = planes[cc * plane + e0];
    p1[c] = planes[cc * plane + e1];
  }
  uint64_t sum[2] = {0, 0};
#pragma unroll
  for (uint32_t c = 0; c < kUnroll; ++c)
    if (c < chunks) sum[0] += uint64_t(p0[c]), sum[1] += uint64_t(p1[c]);
  for (uint32_t c = kUnroll; c < chunks; ++c) {
    sum[0] += uint64_t(planes[c * plane + e0]);
    sum[1] += uint64_t(planes[c * plane + e1]);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint64_t e = e0 + h;
    if (e >= total) break;
    const uint64_t v = sum[h];
    const uint64_t token = e / n_rows, row = e % n_rows;
    if (acc_out) {
      acc_out[token * ld_out + row] = int64_t(v);
    } else if (split.out1) {
      int32_t* o = out;
      uint64_t ld = ld_out, rr = row;
      if (row >= split.r2) o = split.out2, ld = split.ld2, rr = row - split.r2;
      else if (row >= split.r1) o = split.out1, ld = split.ld1, rr = row - split.r1;
      o[token * ld + rr] = requant(int64_t(v));
    } else {
      out[token * ld_out + row] = requant(int64_t(v));
    }
  }
}

// Wide (i16 / i32 Wgt) GEMV on the vector ALUs: one wave per output row.
template <class T>
__global__ __launch_bounds__(256) void k_gemv_wide(const T* __restrict__ w, uint64_t n_rows, uint64_t k,
                                                   const int32_t* __restrict__ act, uint64_t ld_act,
                                                   uint32_t m, int32_t* __restrict__ out, uint64_t ld_out,
                                                   int64_t* __restrict__ acc_out) {
  const int lane = threadIdx.x & 63;
  const uint64_t row = uint64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  const T* wr = w + row * k;
  for (uint32_t t = 0; t < m; ++t) {
    const int32_t* a = act + t * ld_act;
    int64_t acc = 0;
    for (uint64_t c = lane; c < k; c += 64) acc = mac(acc, a[c], int32_t(wr[c]));
    acc = wave_sum_wrap(acc);
    if (lane == 0) {
      if (acc_out) acc_out[t * ld_out + row] = acc;
      else out[t * ld_out + row] = requant(acc);
    }
  }
}

// ---------------------------------------------------------------------------
// RMSNorm (ops.rs:95-131, 406-425): one wave per row; dst = rmsnorm(src)
// (times the gain w when given), plus res (add_sat) when given.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rmsnorm(const int32_t* src, int32_t* dst, const int32_t* res, uint64_t rows,
                                                 uint64_t cols, uint64_t ld, const int32_t* __restrict__ w,
                                                 int64_t eps) {
  const int lane = threadIdx.x & 63;
  const uint64_t row = uint64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int32_t* xr = src + row * ld;
  int64_t ss = 0;
  for (uint64_t c = lane; c < cols; c += 64) ss = add_sat64_nn(ss, sq_term(xr[c]));
  ss = wave_sum_sat(ss);
  const int32_t scale = rms_scale_from_sumsq(ss, uint32_t(cols), eps);
  // each element is read (src, res) and written (dst) by the same lane, so
  // dst may alias src or res
  for (uint64_t c = lane; c < cols; c += 64) {
    const int32_t y = mul_sat(xr[c], scale);
    const int32_t z = w ? mul_sat(y, w[c]) : y;
    dst[row * ld + c] = res ? add_sat(z, res[row * ld + c]) : z;
  }
}

// Wide rows: one workgroup of NT threads per row, element c = tid + NT * e
// held in registers (e < EPT); every wave reduces its saturating partial sum
// of squares, and after one barrier each wave combines the NT / 64 partials
// and computes the scale itself. src and dst may be the same rows; with res,
// dst = add_sat(rmsnorm(src), res) (the residual add after a sub-block).
template <int NT, int EPT>
__global__ __launch_bounds__(NT) void k_rmsnorm_wide(const int32_t* src, int32_t* dst, uint64_t cols, uint64_t ld,
                                                     const int32_t* __restrict__ w, int64_t eps,
                                                     const int32_t* res) {
  __shared__ int64_t red[NT / 64];
  const uint64_t row = blockIdx.x;
  const int32_t* xr = src + row * ld;
  int32_t v[EPT], g[EPT];
  int64_t ss = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const uint64_t c = threadIdx.x + uint64_t(NT) * e;
    v[e] = c < cols ? xr[c] : 0;
    g[e] = (w && c < cols) ? w[c] : 0;
    ss = add_sat64_nn(ss, sq_term(v[e]));
  }
  ss = wave_sum_sat(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  int64_t tot = 0;
#pragma unroll
  for (int k = 0; k < NT / 64; ++k) tot = add_sat64(tot, red[k]);
  const int32_t scale = rms_scale_from_sumsq(tot, uint32_t(cols), eps);
  int32_t* yr = dst + row * ld;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const uint64_t c = threadIdx.x + uint64_t(NT) * e;
    if (c < cols) {
      const int32_t y = mul_sat(v[e], scale);
      const int32_t z = w ? mul_sat(y, g[e]) : y;
      yr[c] = res ? add_sat(z, res[row * ld + c]) : z;
    }
  }
}

// The residual add after a sub-block and the next input norm in one pass
// over a wide row (the two k_rmsnorm_wide launches it replaces, in order):
// x = add_sat(rmsnorm(src) * w1, x) [then x = mul_sat(x, scalar) with
// has_scalar, the layer scalar between two layers], then normed =
// rmsnorm(x) * w2 (w1, w2 optional). One workgroup of NT threads per row, as
// k_rmsnorm_wide.
template <int NT, int EPT>
__global__ __launch_bounds__(NT) void k_rmsnorm_add_norm(const int32_t* __restrict__ src, int32_t* __restrict__ x,
                                                         int32_t* __restrict__ normed, uint64_t cols, uint64_t ld,
                                                         const int32_t* __restrict__ w1,
                                                         const int32_t* __restrict__ w2, int64_t eps,
                                                         int has_scalar, int32_t scalar) {
  __shared__ int64_t red[2][NT / 64];
  const uint64_t row = blockIdx.x;
  int32_t v[EPT], xv[EPT], g1[EPT], g2[EPT];
  int64_t ss = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const uint64_t c = threadIdx.x + uint64_t(NT) * e;
    const bool in = c < cols;
    v[e] = in ? src[row * ld + c] : 0;
    xv[e] = in ? x[row * ld + c] : 0;
    g1[e] = (w1 && in) ? w1[c] : 0;
    g2[e] = (w2 && in) ? w2[c] : 0;
    ss = add_sat64_nn(ss, sq_term(v[e]));
  }
  auto block_scale = [&](int k, int64_t part) {
    part = wave_sum_sat(part);
    if ((threadIdx.x & 63) == 0) red[k][threadIdx.x >> 6] = part;
    __syncthreads();
    int64_t tot = 0;
#pragma unroll
    for (int j = 0; j < NT / 64; ++j) tot = add_sat64(tot, red[k][j]);
    return rms_scale_from_sumsq(tot, uint32_t(cols), eps);
  };
  const int32_t s1 = block_scale(0, ss);
  ss = 0;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const uint64_t c = threadIdx.x + uint64_t(NT) * e;
    const int32_t y = mul_sat(v[e], s1);
    int32_t nx = add_sat(w1 ? mul_sat(y, g1[e]) : y, xv[e]);
    if (has_scalar) nx = mul_sat(nx, scalar);
    xv[e] = c < cols ? nx : 0;
    if (c < cols) x[row * ld + c] = xv[e];
    ss = add_sat64_nn(ss, sq_term(xv[e]));
  }
  const int32_t s2 = block_scale(1, ss);
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const uint64_t c = threadIdx.x + uint64_t(NT) * e;
    if (c < cols) {
      const int32_t y = mul_sat(xv[e], s2);
      normed[row * ld + c] = w2 ? mul_sat(y, g2[e]) : y;
    }
  }
}

// ---------------------------------------------------------------------------
// RoPE (ops.rs:151-196): one thread per (row, head, pair).
// ---------------------------------------------------------------------------
__global__ void k_rope(int32_t* __restrict__ x, uint64_t rows, uint64_t ld, uint64_t heads, uint64_t hd,
                       uint64_t half, const int64_t* __restrict__ inv_freq, uint64_t pos0, uint64_t pos_step,
                       const uint64_t* __restrict__ positions) {
  const uint64_t idx = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t total = rows * heads * half;
  if (idx >= total) return;
  const uint64_t i = idx % half;
  const uint64_t h = (idx / half) % heads;
  const uint64_t r = idx / (half * heads);
  const uint64_t pos = positions ? positions[r] : pos0 + r * pos_step;
  if (pos == 0) return;  // identity (ops.rs:179-181)
  int32_t c, s;
  sin_cos(rope_angle(pos, inv_freq[i]), &c, &s);
  int32_t* base = x + r * ld + h * hd;
  const int32_t lhs = base[i], rhs = base[i + half];
  base[i] = sub_sat(mul_sat(lhs, c), mul_sat(rhs, s));
  base[i + half] = add_sat(mul_sat(rhs, c), mul_sat(lhs, s));
}

// The head norms of a token's q, k and v rows and the rotation of its q and
// k rows in one pass (the arithmetic of k_rmsnorm over every head row, q rows
// times q_gain, k rows times k_gain, v rows without gain, then k_rope on the
// q and k rows): one workgroup per token computes the token's cos/sin pairs
// once into LDS; each wave loads up to four of the token's head rows at a
// time (rows wave, wave + 4, ...), normalises them, and writes a rotated
// row through its own LDS row so that each pair's two elements meet in one
// lane. E: elements per lane (head dim <= 64 E).
template <int E>
__global__ __launch_bounds__(256) void k_head_norm_rope(HeadNormRope a) {
  constexpr int RPW = 4;  // head rows per wave in flight
  __shared__ int32_t tcs[2][kHeadRopeMaxHalf];
  __shared__ __attribute__((aligned(16))) int32_t rowbuf[4][RPW][64 * E];
  const uint64_t t = blockIdx.x;
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, hd = a.hd, half = a.half;
  const uint32_t nsub = hd / 64;
  // One 16-dim slot of the 1 KB MFMA operand blocks of head row hidx (of the q
  // or k blocks): dims [16 sl, 16 sl + 16) go to limb j's block
  // ((hidx * nt + t / 16) * nsub + sl / 4) * 4 + j, bytes (16 (sl % 4) + t % 16) * 16;
  // returns the slot's sum of x - C4 (src null: a padding row, x = C4)
  auto put_slot = [&](int8_t* limbs, uint64_t nt, uint32_t hidx, uint32_t sl, const int32_t* src) {
    int32_t x16[16];
    if (src) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int4 v = reinterpret_cast<const int4*>(src + 16 * sl)[q];
        x16[4 * q] = v.x, x16[4 * q + 1] = v.y, x16[4 * q + 2] = v.z, x16[4 * q + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int q = 0; q < 16; ++q) x16[q] = int32_t(kAttnC4);
    }
    uint32_t w[4][4];
    const int64_t sm = attn_split16(x16, w);
    int8_t* blk = limbs + ((uint64_t(hidx) * nt + t / 16) * nsub + sl / 4) * 4 * kAttnOp + (16 * (sl % 4) + t % 16) * 16;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<uint4*>(blk + j * kAttnOp) = make_uint4(w[j][0], w[j][1], w[j][2], w[j][3]);
    return sm;
  };
  // sum over the spr lanes of a row's slots (every lane takes part): segments
  // of a power-of-two width share the wave, any other width takes one row per
  // pass and the whole wave (lanes past its slots add zero)
  const uint32_t spr = hd / 16;  // slots per row
  const bool pow2 = (spr & (spr - 1)) == 0;
  const uint32_t rpp = pow2 ? 64 / spr : 1;  // rows per 64-lane pass
  auto seg_sum = [&](int64_t sm) {
    if (!pow2) return wave_sum_wrap64(sm);
    for (uint32_t off = 1; off < spr; off <<= 1) sm += __shfl_xor(sm, int(off), 64);
    return sm;
  };
  auto put_blocks = [&](int8_t* limbs, int64_t* sums, uint64_t nt, uint32_t hidx, const int32_t* src) {
    const int64_t sm = seg_sum(lane < spr ? put_slot(limbs, nt, hidx, lane, src) : 0);
    if (lane == 0) sums[uint64_t(hidx) * nt * 16 + t] = sm;
  };
  if (t >= a.rows) {
    // rows past the tokens up to whole tiles of the MFMA blocks
    for (uint32_t h = wave; h < a.nh; h += 4) put_blocks(a.qlimbs, a.qsum, a.nqt, h, nullptr);
    if (a.klimbs)
      for (uint32_t h = wave; h < a.nkv; h += 4) put_blocks(a.klimbs, a.ksum, a.nkt, h, nullptr);
    return;
  }
  const uint64_t pos = a.positions ? a.positions[t] : a.pos0 + t;
  const bool rot = a.half != 0 && pos != 0;  // position 0 is the identity (ops.rs:179-181)
  if (rot)
    for (uint32_t i = threadIdx.x; i < a.half; i += 256) {
      int32_t c, s;
      sin_cos(rope_angle(pos, a.inv_freq[i]), &c, &s);
      tcs[0][i] = c;
      tcs[1][i] = s;
    }
  __syncthreads();
  const uint32_t nv = a.v ? a.nkv : 0, nrows = a.nh + a.nkv + nv;

  // this lane's q and k gains (every q row shares one gain vector, every k row another)
  int32_t gq[E], gk[E];
#pragma unroll
  for (int k = 0; k < E; ++k) {
    const uint32_t c = lane + 64 * k;
    gq[k] = (a.q_gain && c < hd) ? a.q_gain[c] : 0;
    gk[k] = (a.k_gain && c < hd) ? a.k_gain[c] : 0;
  }
  auto row_of = [&](uint32_t r) {
    return r < a.nh ? a.q + (t * a.nh + r) * hd
                    : (r < a.nh + a.nkv ? a.k + (t * a.nkv + (r - a.nh)) * hd
                                        : a.v + (t * a.nkv + (r - a.nh - a.nkv)) * hd);
  };
  // this token's cache rows (k and v rows also go there)
  const bool cached = a.kc && t >= a.kv_from;
  const uint64_t slot = a.kv_ring ? t % a.kv_cap : t;
  auto cache_of = [&](uint32_t r) -> int32_t* {
    if (!cached || r < a.nh) return nullptr;
    return r < a.nh + a.nkv ? a.kc + (slot * a.nkv + (r - a.nh)) * hd : a.vc + (slot * a.nkv + (r - a.nh - a.nkv)) * hd;
  };
  for (uint32_t r0 = wave; r0 < nrows; r0 += 4 * RPW) {
    uint32_t blk_mask = 0;  // rows of this group whose blocks are written after the group
    int32_t x[RPW][E];
#pragma unroll
    for (int u = 0; u < RPW; ++u) {
      const uint32_t r = r0 + 4 * u;
      const int32_t* row = row_of(r < nrows ? r : r0);
#pragma unroll
      for (int k = 0; k < E; ++k) {
        const uint32_t c = lane + 64 * k;
        x[u][k] = (r < nrows && c < hd) ? row[c] : 0;
      }
    }
#pragma unroll
    for (int u = 0; u < RPW; ++u) {
      const uint32_t r = r0 + 4 * u;
      if (r >= nrows) break;  // (wave-uniform)
      int32_t* row = row_of(r);
      int32_t* crow = cache_of(r);
      int32_t* rb = rowbuf[wave][u];
      const bool is_q = r < a.nh, is_k = !is_q && r < a.nh + a.nkv;
      const bool gained = is_q ? a.q_gain != nullptr : (is_k && a.k_gain != nullptr);
      const bool rotate = rot && (is_q || is_k);
      // the final row also goes to the MFMA attention's operand blocks (through this wave's LDS row)
      const bool blocks = (is_q && a.qlimbs) || (is_k && a.klimbs);
      if (blocks) blk_mask |= 1u << u;
      int64_t ss = 0;
#pragma unroll
      for (int k = 0; k < E; ++k) ss = add_sat64_nn(ss, sq_term(x[u][k]));
      ss = wave_sum_sat(ss);
      const int32_t sc = rms_scale_from_sumsq(ss, hd, a.eps);
#pragma unroll
      for (int k = 0; k < E; ++k) {
        const uint32_t c = lane + 64 * k;
        if (c < hd) {
          const int32_t y = mul_sat(x[u][k], sc);
          const int32_t z = gained ? mul_sat(y, is_q ? gq[k] : gk[k]) : y;
          if (rotate || blocks) rb[c] = z;
          if (!rotate) {
            row[c] = z;
            if (crow) crow[c] = z;
          }
        }
      }
      if (rotate) {
        wave_lds_sync();  // the wave's LDS row is complete before its lanes read each other's elements
        for (uint32_t i = lane; i < half; i += 64) {
          const int32_t c = tcs[0][i], s = tcs[1][i];
          const int32_t lhs = rb[i], rhs = rb[i + half];
          const int32_t y0 = sub_sat(mul_sat(lhs, c), mul_sat(rhs, s));
          const int32_t y1 = add_sat(mul_sat(rhs, c), mul_sat(lhs, s));
          row[i] = y0;
          row[i + half] = y1;
          if (crow) crow[i] = y0, crow[i + half] = y1;
          if (blocks) rb[i] = y0, rb[i + half] = y1;  // (this lane's own pair: read above)
        }
        for (uint32_t c = 2 * half + lane; c < hd; c += 64) {
          row[c] = rb[c];
          if (crow) crow[c] = rb[c];
        }
      }
    }
    // the group's operand blocks, rpp rows per pass of the wave's 64 lanes
    if (blk_mask) {
      wave_lds_sync();  // the final rows are in the wave's LDS rows
      for (uint32_t p0 = 0; p0 < RPW; p0 += rpp) {
        const uint32_t u = p0 + lane / spr, sl = lane % spr;
        const uint32_t r = r0 + 4 * u;
        const bool on = lane < rpp * spr && u < RPW && ((blk_mask >> u) & 1u);
        const bool is_q = r < a.nh;
        int64_t sm = 0;
        if (on) sm = is_q ? put_slot(a.qlimbs, a.nqt, r, sl, rowbuf[wave][u])
                          : put_slot(a.klimbs, a.nkt, r - a.nh, sl, rowbuf[wave][u]);
        sm = seg_sum(sm);
        if (on && sl == 0) {
          if (is_q) a.qsum[uint64_t(r) * a.nqt * 16 + t] = sm;
          else a.ksum[uint64_t(r - a.nh) * a.nkt * 16 + t] = sm;
        }
      }
    }
    wave_lds_sync();  // every read of the group's LDS rows precedes the next group's writes
  }
}

// ---------------------------------------------------------------------------
// Attention for one (head, query): score dots -> integer softmax -> weighted
// sum (det_kernels.rs:340-367, ops.rs:230-258).
// ---------------------------------------------------------------------------
constexpr int kAttnThreads = 256;
constexpr int kAttnWaves = kAttnThreads / 64;
constexpr uint64_t kMaxAttnRows = 16000;  // LDS: one int32 per window row

// Key/value window of query t: window row r sits at physical cache row
// phys(r) = base + r, wrapped once around a ring of `wrap` rows (base < wrap,
// r < count <= wrap).
struct AttnWin {
  global_ptr<const int32_t> k;
  global_ptr<const int32_t> v;
  uint64_t base, wrap, count;
  __device__ uint64_t phys(uint64_t r) const {
    const uint64_t p = base + r;
    return p >= wrap ? p - wrap : p;
  }
};

__device__ inline AttnWin attn_window_of(const AttnArgs& a, uint32_t t) {
  if (a.seqs) {
    // one query per sequence, each over its own cache window
    const AttnSeq sq = a.seqs[t];
    return {to_global(sq.k), to_global(sq.v), sq.base, sq.wrap ? sq.wrap : ~0ull, sq.count};
  }
  uint64_t start, count;
  if (a.causal) {
    uint64_t end = t + 1 + a.causal_offset;
    start = (a.window && end > a.window) ? end - a.window : 0;
    if (start > a.avail) start = a.avail;
    if (end > a.avail) end = a.avail;
    count = end > start ? end - start : 0;
  } else {
    start = a.fix_start;
    count = a.fix_count;
  }
  const uint64_t base = a.ring_cap ? (a.ring_start + start) % a.ring_cap : start;
  return {to_global(a.k), to_global(a.v), base, a.ring_cap ? a.ring_cap : ~0ull, count};
}

__global__ __launch_bounds__(kAttnThreads) void k_attention(AttnArgs a) {
  extern __shared__ int32_t lds_w[];  // one int32 per window row (scores, then weights)
  __shared__ int64_t red[kAttnWaves];
  __shared__ int64_t bcast[2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t h = blockIdx.x, t = blockIdx.y;
  const uint32_t kvh = h / a.groups;
  const AttnWin win = attn_window_of(a, t);
  const uint64_t count = win.count;
  if (count == 0) return;  // host validation makes every window non-empty
  const int32_t* qrow = a.q + uint64_t(t) * a.q_ld + uint64_t(h) * a.hd;
  int32_t* orow = a.out + uint64_t(t) * a.out_ld + uint64_t(h) * a.hd;
  // 1. scores (wave per row, lanes over head dims)
  for (uint64_t r = wave; r < count; r += kAttnWaves) {
    const auto krow = win.k + win.phys(r) * a.kv_ld + uint64_t(kvh) * a.hd;
    int64_t acc = 0;
    for (uint32_t d = lane; d < a.hd; d += 64) acc = mac(acc, qrow[d], krow[d]);
    acc = wave_sum_wrap(acc);
    if (lane == 0) lds_w[r] = requant(acc);
  }
  __syncthreads();
  // 2. first argmax
  int64_t best = INT64_MIN;
  for (uint64_t r = threadIdx.x; r < count; r += kAttnThreads) {
    const int64_t key = argmax_key(lds_w[r], uint32_t(r));
    best = key > best ? key : best;
  }
  best = block_reduce<kAttnWaves>(best, 2, red);
  const uint32_t max_idx = key_index(best);
  const int32_t max_logit = lds_w[max_idx];
  // 3. saturating sum of exp terms
  int64_t sum = 0;
  for (uint64_t r = threadIdx.x; r < count; r += kAttnThreads) sum = add_sat64(sum, softmax_exp(lds_w[r], max_logit));
  sum = block_reduce<kAttnWaves>(sum, 1, red);
  __syncthreads();
  // 4. weights (in place) and their saturating sum
  int64_t wsum = 0;
  for (uint64_t r = threadIdx.x; r < count; r += kAttnThreads) {
    const int32_t wgt = softmax_weight(softmax_exp(lds_w[r], max_logit), sum);
    lds_w[r] = wgt;
    wsum = add_sat64(wsum, int64_t(wgt));
  }
  wsum = block_reduce<kAttnWaves>(wsum, 1, red);
  if (threadIdx.x == 0) {
    const int32_t summed = sat32(wsum);
    const int32_t residual = sub_sat(kOneAct, summed);
    lds_w[max_idx] = add_sat(lds_w[max_idx], residual);
  }
  __syncthreads();
  // 5. weighted sum over value rows
  for (uint32_t d = threadIdx.x; d < a.hd; d += kAttnThreads) {
    int64_t acc = 0;
    for (uint64_t r = 0; r < count; ++r) acc = mac(acc, win.v[win.phys(r) * a.kv_ld + uint64_t(kvh) * a.hd + d], lds_w[r]);
    orow[d] = requant(acc);
  }
  (void)bcast;
}

// ---------------------------------------------------------------------------
// Causal / windowed attention for a slab of queries (det_attention_prefill,
// det_kernels.rs:525-671, and the decode loop :1001-1053): per query head,
// scores = requantize(wrap-dot(q, k_r)), integer softmax with the residual on
// the first argmax row (ops.rs:230-273), out = requantize(sum_r w_r v_r).
// One workgroup (512 threads) per (group of HB query heads sharing a KV
// head, query): the key and value rows are read once for the HB heads.
// Scores: sixteen lanes per key row, U rows per lane group in flight;
// softmax: 8 / HB waves per head; weighted sum: one thread per dimension.
// ---------------------------------------------------------------------------
constexpr int kAttnPThreads = 512;

// Score-row stride of a launch: no window of its queries is longer.
__host__ __device__ inline uint64_t attn_row_stride(const AttnArgs& a) {
  if (a.seqs || !a.causal) return a.fix_count;
  return (a.window && a.window < a.avail) ? a.window : a.avail;
}

template <int KPER, int HB>
__global__ __launch_bounds__(kAttnPThreads) void k_attention_prefill(AttnArgs a) {
  extern __shared__ int32_t sc[];  // [HB][max_count] scores, then weights
  __shared__ int32_t ql[HB * 16 * KPER];
  __shared__ int64_t red[8];
  __shared__ int64_t hkey[HB], hsum[HB];
  __shared__ uint64_t hrec[HB];
  constexpr int U = 64 / KPER;  // key rows per lane group per pass
  const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t hg = blockIdx.x, t = blockIdx.y;
  const uint32_t h0 = hg * HB, kvh = h0 / a.groups;
  const uint32_t hd = a.hd;
  const AttnWin win = attn_window_of(a, t);
  const uint64_t count = win.count;
  if (count == 0) return;  // host validation makes every window non-empty
  const uint64_t cstride = attn_row_stride(a);
  const auto kc = win.k;
  const auto vc = win.v;
  auto phys = [&](uint64_t r) { return win.phys(r); };
  for (uint32_t i = threadIdx.x; i < HB * hd; i += kAttnPThreads)
    ql[i] = a.q[uint64_t(t) * a.q_ld + uint64_t(h0 + i / hd) * hd + i % hd];
  __syncthreads();
  // 1. scores
  const uint32_t grp = threadIdx.x >> 4, li = threadIdx.x & 15;
  for (uint64_t r0 = 0; r0 < count; r0 += 32 * U) {
    int32_t kr[U][KPER];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint64_t r = r0 + grp + 32 * u;
      const bool on = r < count;
      const auto krow = kc + (on ? phys(r) : 0) * a.kv_ld + uint64_t(kvh) * hd;
#pragma unroll
      for (int tt = 0; tt < KPER / 4; ++tt) {
        const uint32_t d = 4 * li + 64 * tt;
        int4 v = make_int4(0, 0, 0, 0);
        if (on && d < hd) v = load_int4(krow + d);
        kr[u][4 * tt] = v.x, kr[u][4 * tt + 1] = v.y, kr[u][4 * tt + 2] = v.z, kr[u][4 * tt + 3] = v.w;
      }
    }
#pragma unroll
    for (int g = 0; g < HB; ++g) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        int64_t acc = 0;
#pragma unroll
        for (int tt = 0; tt < KPER / 4; ++tt) {
          const uint32_t d = 4 * li + 64 * tt;
          if (d < hd) {
            const int4 q = *reinterpret_cast<const int4*>(ql + g * hd + d);
            acc = mac(acc, q.x, kr[u][4 * tt]);
            acc = mac(acc, q.y, kr[u][4 * tt + 1]);
            acc = mac(acc, q.z, kr[u][4 * tt + 2]);
            acc = mac(acc, q.w, kr[u][4 * tt + 3]);
          }
        }
        acc = int64_t(row16_reduce(uint64_t(acc), OpWrapAdd()));
        const uint64_t r = r0 + grp + 32 * u;
        if (li == 0 && r < count) sc[g * cstride + r] = requant(acc);
      }
    }
  }
  __syncthreads();
  // 2. softmax per head: waves wi of head g take rows wi*64 + lane + stride*n
  constexpr uint32_t WPH = 8 / HB;
  const uint32_t g = wave / WPH, wi = wave % WPH;
  const uint64_t stride = 64 * uint64_t(WPH);
  int32_t* sg = sc + g * cstride;
  int64_t best = INT64_MIN;
  for (uint64_t r = wi * 64 + lane; r < count; r += stride) {
    const int64_t k = argmax_key(sg[r], uint32_t(r));
    best = k > best ? k : best;
  }
  best = wave_max64(best);
  if (lane == 0) red[wave] = best;
  __syncthreads();
  if (threadIdx.x < HB) {
    int64_t k = red[threadIdx.x * WPH];
    for (uint32_t w = 1; w < WPH; ++w) k = red[threadIdx.x * WPH + w] > k ? red[threadIdx.x * WPH + w] : k;
    hkey[threadIdx.x] = k;
  }
  __syncthreads();
  const uint32_t mi = key_index(hkey[g]);
  const int32_t mx = sg[mi];
  int64_t s = 0;
  for (uint64_t r = wi * 64 + lane; r < count; r += stride) s += softmax_exp(sg[r], mx);  // below 2^63
  s = wave_sum_wrap64(s);
  __syncthreads();
  if (lane == 0) red[wave] = s;
  __syncthreads();
  if (threadIdx.x < HB) {
    int64_t tsum = 0;
    for (uint32_t w = 0; w < WPH; ++w) tsum += red[threadIdx.x * WPH + w];
    hsum[threadIdx.x] = tsum;
    hrec[threadIdx.x] = tsum < (int64_t(1) << 61) ? softmax_recip(tsum) : 0;
  }
  __syncthreads();
  const int64_t S = hsum[g];
  const uint64_t M = hrec[g];
  int64_t ws = 0;
  for (uint64_t r = wi * 64 + lane; r < count; r += stride) {
    const int64_t e = softmax_exp(sg[r], mx);
    const int32_t w = M ? softmax_weight_r(e, S, M) : softmax_weight(e, S);
    sg[r] = w;  // each row is read and written by the same thread
    ws += w;
  }
  ws = wave_sum_wrap64(ws);
  __syncthreads();
  if (lane == 0) red[wave] = ws;
  __syncthreads();
  if (threadIdx.x < HB) {
    int64_t tsum = 0;
    for (uint32_t w = 0; w < WPH; ++w) tsum += red[threadIdx.x * WPH + w];
    const uint32_t m2 = key_index(hkey[threadIdx.x]);
    int32_t* row = sc + threadIdx.x * cstride;
    row[m2] = add_sat(row[m2], sub_sat(kOneAct, sat32(tsum)));
  }
  __syncthreads();
  // 3. weighted sums: thread d, rows in batches of 8 loads
  for (uint32_t d = threadIdx.x; d < hd; d += kAttnPThreads) {
    int64_t acc[HB];
#pragma unroll
    for (int gg = 0; gg < HB; ++gg) acc[gg] = 0;
    uint64_t r = 0;
    for (; r + 8 <= count; r += 8) {
      int32_t v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = vc[phys(r + u) * a.kv_ld + uint64_t(kvh) * hd + d];
#pragma unroll
      for (int u = 0; u < 8; ++u)
#pragma unroll
        for (int gg = 0; gg < HB; ++gg) acc[gg] = mac(acc[gg], v[u], sc[gg * cstride + r + u]);
    }
    for (; r < count; ++r) {
      const int32_t v = vc[phys(r) * a.kv_ld + uint64_t(kvh) * hd + d];
#pragma unroll
      for (int gg = 0; gg < HB; ++gg) acc[gg] = mac(acc[gg], v, sc[gg * cstride + r]);
    }
#pragma unroll
    for (int gg = 0; gg < HB; ++gg)
      a.out[uint64_t(t) * a.out_ld + uint64_t(h0 + gg) * hd + d] = requant(acc[gg]);
  }
}

// Appends one key and one value row per sequence at its canonical slot:
// dst[i] (key, value) receive rows i of k and v (width w).
__global__ void k_kv_append(const int32_t* __restrict__ k, const int32_t* __restrict__ v, uint64_t w,
                            int32_t* const* __restrict__ kdst, int32_t* const* __restrict__ vdst) {
  const uint64_t i = blockIdx.y, c = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (c >= w) return;
  kdst[i][c] = k[i * w + c];
  vdst[i][c] = v[i * w + c];
}

// First-index argmax of each row of x [rows][n] in two passes: workgroup
// (p, r) reduces columns [p * kArgmaxSpan, (p + 1) * kArgmaxSpan) of row r to
// one argmax key; one workgroup per row then reduces the row's keys.
constexpr uint64_t kArgmaxSpan = 4096;
__global__ __launch_bounds__(256) void k_argmax_rows_part(const int32_t* __restrict__ x, uint64_t n,
                                                          int64_t* __restrict__ keys, uint32_t parts) {
  __shared__ int64_t red[4];
  const int32_t* xr = x + uint64_t(blockIdx.y) * n;
  const uint64_t c0 = uint64_t(blockIdx.x) * kArgmaxSpan;
  const uint64_t c1 = c0 + kArgmaxSpan < n ? c0 + kArgmaxSpan : n;
  int64_t best = INT64_MIN;
  for (uint64_t i = c0 + threadIdx.x; i < c1; i += 256) {
    const int64_t key = argmax_key(xr[i], uint32_t(i));
    best = key > best ? key : best;
  }
  best = block_reduce<4>(best, 2, red);
  if (threadIdx.x == 0) keys[uint64_t(blockIdx.y) * parts + blockIdx.x] = best;
}
__global__ __launch_bounds__(256) void k_argmax_rows_final(const int64_t* __restrict__ keys, uint32_t parts,
                                                           uint32_t* __restrict__ out) {
  __shared__ int64_t red[4];
  int64_t best = INT64_MIN;
  for (uint32_t p = threadIdx.x; p < parts; p += 256) {
    const int64_t k = keys[uint64_t(blockIdx.x) * parts + p];
    best = k > best ? k : best;
  }
  best = block_reduce<4>(best, 2, red);
  if (threadIdx.x == 0) out[blockIdx.x] = key_index(best);
}

// ---------------------------------------------------------------------------
// Elementwise
// ---------------------------------------------------------------------------
__global__ void k_add_sat(int32_t* __restrict__ d, const int32_t* __restrict__ s, uint64_t n) {
  const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) d[i] = add_sat(d[i], s[i]);
}
__global__ void k_gelu_mul(int32_t* __restrict__ g, const int32_t* __restrict__ u, uint64_t n) {
  const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) g[i] = mul_sat(gelu_act(g[i]), u[i]);
}
__global__ void k_scale(int32_t* __restrict__ x, uint64_t n, int32_t s) {
  const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) x[i] = mul_sat(x[i], s);
}
__global__ void k_softcap(int32_t* __restrict__ x, uint64_t n, int32_t cap) {
  const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) x[i] = softcap_act(x[i], cap);
}

__device__ __forceinline__ int32_t wgt_at(const DevMatrix& M, uint64_t r, uint64_t c) {
  if (M.storage == kInt8) {
    uint32_t v = 0;
    for (int p = 0; p < M.planes; ++p) v += uint32_t(int32_t(M.q[tiled_offset(M.kpad, digit_row(r, M.planes, p), c)])) << (8 * p);
    return int32_t(v * uint32_t(M.scale[r]));
  }
  if (M.storage == kI16) return int32_t(static_cast<const int16_t*>(M.w)[r * M.cols + c]);
  return static_cast<const int32_t*>(M.w)[r * M.cols + c];
}
__global__ void k_gather_rows(DevMatrix M, const uint32_t* __restrict__ ids, uint64_t ids_stride, uint64_t m,
                              uint64_t col0, uint64_t ncols, int32_t scale, int32_t* __restrict__ out,
                              uint64_t ld_out) {
  const uint64_t c = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint64_t t = blockIdx.y;
  if (c >= ncols || t >= m) return;
  out[t * ld_out + c] = mul_sat(wgt_at(M, ids[t * ids_stride], col0 + c), scale);
}

__global__ __launch_bounds__(256) void k_argmax_partial(const int32_t* __restrict__ x, uint64_t n,
                                                        int64_t* __restrict__ part) {
  __shared__ int64_t red[4];
  int64_t best = INT64_MIN;
  const uint64_t base = uint64_t(blockIdx.x) * 1024;
  for (uint64_t i = base + threadIdx.x; i < base + 1024 && i < n; i += 256) {
    const int64_t key = argmax_key(x[i], uint32_t(i));
    best = key > best ? key : best;
  }
  best = block_reduce<4>(best, 2, red);
  if (threadIdx.x == 0) part[blockIdx.x] = best;
}
__global__ __launch_bounds__(256) void k_argmax_final(const int64_t* __restrict__ part, uint64_t nparts,
                                                      uint32_t* __restrict__ out) {
  __shared__ int64_t red[4];
  int64_t best = INT64_MIN;
  for (uint64_t i = threadIdx.x; i < nparts; i += 256) best = part[i] > best ? part[i] : best;
  best = block_reduce<4>(best, 2, red);
  if (threadIdx.x == 0) *out = key_index(best);
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
static inline unsigned blocks_for(uint64_t n, unsigned per) { return unsigned((n + per - 1) / per); }
// log2 of a matrix's digit planes (1, 2 or 4), the kernels' shift amount
static inline int plane_log2(const DevMatrix& W) {
  if (W.planes != 1 && W.planes != 2 && W.planes != 4) throw std::invalid_argument("digit planes must be 1, 2 or 4");
  return W.planes >> 1;
}

DevMatrix row_view(const DevMatrix& m, uint64_t r0, uint64_t n) {
  DevMatrix v = m;
  v.rows = n;
  v.owns = false;
  if (m.storage == kInt8) {
    v.q = m.q + (r0 / 16) * uint64_t(m.planes) * (m.kpad / 128) * 2048;  // r0 is tile aligned
    v.scale = m.scale + r0;
    v.rowsum = m.rowsum + r0;
    v.rowsum_p = m.rowsum_p ? m.rowsum_p + r0 : nullptr;  // (rowsum_p_ld is the parent's)
  } else if (m.storage == kI16) {
    v.w = static_cast<int16_t*>(m.w) + r0 * m.cols;
  } else {
    v.w = static_cast<int32_t*>(m.w) + r0 * m.cols;
  }
  return v;
}

void launch_act_limbs(const int32_t* act, uint64_t m, uint64_t k, uint64_t ld, uint64_t kpad, int8_t* limbs,
                      hipStream_t s) {
  dim3 grid(blocks_for(kpad, 256), unsigned(m));
  hipLaunchKernelGGL(k_act_limbs, grid, dim3(256), 0, s, act, m, k, ld, kpad, limbs);
}

// In-workgroup K split: the smallest of 1, 2, 4, 8 that gives at least 512
// workgroups while every wave keeps at least 4 K steps. The grid is capped at
// 1024 workgroups, which then loop over tile groups.
static int pick_ksplit(uint64_t ntiles, uint64_t nsteps) {
  int ks = 1;
  while (ks < 8 && (ntiles * ks + 7) / 8 < 512 && uint64_t(ks) * 2 * 4 <= nsteps) ks *= 2;
  return ks;
}

template <bool IN64, int EPI>
static void launch_lds_gemv(const DevMatrix& W, const void* act, uint64_t ld_act, uint32_t mm, int32_t* o,
                            uint64_t ld_out, int64_t* ao, hipStream_t s, int ks = 0, uint32_t kchunks = 1,
                            const int32_t* mulv = nullptr) {
  const uint64_t ntiles = (W.rows + 15) / 16;
  const uint64_t nsteps = W.kpad / 128;
  const uint64_t cper = (nsteps + kchunks - 1) / kchunks;
  const uint64_t lds = uint64_t(mm) * 4 * (cper * 128 + 32);
  if (ks == 0) ks = pick_ksplit(ntiles, nsteps);
  while (ks * W.planes > 8) ks /= 2;
  const uint64_t tpw = 8 / (uint64_t(ks) * W.planes);
  const uint64_t groups = std::min<uint64_t>((ntiles + tpw - 1) / tpw, std::max<uint64_t>(1024 / kchunks, 1));
  const uint64_t grid = groups * kchunks;
#define DET_GEMV_LAUNCH_DG(KS, DG)                                                                              \
  hipLaunchKernelGGL((k_gemv_i8_lds<KS, IN64, EPI, DG>), dim3(unsigned(grid)), dim3(kGemvThreads), size_t(lds), s, \
                     W.q, W.scale, W.rowsum, act, ld_act, W.cols, W.rows, W.kpad, mm, o, ld_out, ao, kchunks, mulv,   \
                     plane_log2(W))
#define DET_GEMV_LAUNCH(KS)                                                                                     \
  do {                                                                                                          \
    if (W.planes == 1) DET_GEMV_LAUNCH_DG(KS, false);                                                           \
    else DET_GEMV_LAUNCH_DG(KS, true);                                                                          \
  } while (0)
  switch (ks) {
    case 8: DET_GEMV_LAUNCH(8); break;
    case 4: DET_GEMV_LAUNCH(4); break;
    case 2: DET_GEMV_LAUNCH(2); break;
    default: DET_GEMV_LAUNCH(1); break;
  }
#undef DET_GEMV_LAUNCH
#undef DET_GEMV_LAUNCH_DG
}

bool gemv_fits_lds(const DevMatrix& W, uint64_t m) { return m * 4 * (W.kpad + 32) <= kGemvLdsBudget; }

// One-tile-per-workgroup batch-1 GEMV (k_gemv_tile) for int8 matrices of at
// most kTileMaxTiles tiles; larger ones (the lm_head) amortise one activation
// prologue over many tiles in k_gemv_i8_lds.
constexpr uint64_t kTileMaxTiles = 4096;
static bool gemv_tile_fits(const DevMatrix& W) { return W.storage == kInt8 && (W.rows + 15) / 16 <= kTileMaxTiles; }
static void launch_gemv_tile(const DevMatrix& W, const void* act, bool in64, int32_t* o, int64_t* ao, hipStream_t s) {
  const uint64_t ntiles = (W.rows + 15) / 16, nsteps = W.kpad / 128 * uint64_t(W.planes);
  const int nw = nsteps <= 4 * kTileD ? 4 : (nsteps <= 8 * kTileD ? 8 : 16);
#define DET_TILE_LAUNCH_DG(NW, IN, DG)                                                                          \
  hipLaunchKernelGGL((k_gemv_tile<NW, IN, DG>), dim3(unsigned(ntiles)), dim3(64 * NW), 0, s, W.q, W.scale,        \
                     W.rowsum, act, W.cols, W.rows, W.kpad, o, ao, plane_log2(W))
#define DET_TILE_LAUNCH(NW, IN)                                                                                 \
  do {                                                                                                          \
    if (W.planes == 1) DET_TILE_LAUNCH_DG(NW, IN, false);                                                       \
    else DET_TILE_LAUNCH_DG(NW, IN, true);                                                                      \
  } while (0)
  if (in64) {
    if (nw == 4) DET_TILE_LAUNCH(4, true);
    else if (nw == 8) DET_TILE_LAUNCH(8, true);
    else DET_TILE_LAUNCH(16, true);
  } else {
    if (nw == 4) DET_TILE_LAUNCH(4, false);
    else if (nw == 8) DET_TILE_LAUNCH(8, false);
    else DET_TILE_LAUNCH(16, false);
  }
#undef DET_TILE_LAUNCH
#undef DET_TILE_LAUNCH_DG
}

void launch_gemv_decode(const DevMatrix& W, const void* act, bool act_i64, int epilogue, int32_t* out,
                        hipStream_t s, const int32_t* mul) {
  if (act_i64) launch_lds_gemv<true, 0>(W, act, W.cols, 1, out, W.rows, nullptr, s);
  else if (epilogue == 2) launch_lds_gemv<false, 2>(W, act, W.cols, 1, out, W.rows, nullptr, s, 0, 1, mul);
  else if (epilogue == 1) launch_lds_gemv<false, 1>(W, act, W.cols, 1, out, W.rows / 2, nullptr, s);
  else launch_lds_gemv<false, 0>(W, act, W.cols, 1, out, W.rows, nullptr, s);
}

// Decode GEMV into wrapping Q32.32 accumulators that are zero on entry:
// k_gemv_tile where the matrix is small enough (one workgroup per tile, plain
// stores); otherwise eight waves split K inside each workgroup and K is
// further split across workgroups (doubling) until the launch has at least
// 512 workgroups, keeping at least one K step per wave and at most 1024
// workgroups (atomic adds).
bool gemv_decode_acc_plain(const DevMatrix& W) { return gemv_tile_fits(W); }
void launch_gemv_decode_acc(const DevMatrix& W, const void* act, bool act_i64, int64_t* acc, hipStream_t s) {
  if (gemv_tile_fits(W)) return launch_gemv_tile(W, act, act_i64, nullptr, acc, s);
  const uint64_t ntiles = (W.rows + 15) / 16, nsteps = W.kpad / 128;
  int ks = 8;
  while (ks > 1 && uint64_t(ks) > nsteps) ks >>= 1;
  const uint64_t groups = (ntiles * ks + 7) / 8;
  uint32_t kc = 1;
  while (groups * kc < 512 && groups * kc * 2 <= 1024 && uint64_t(kc) * 2 * ks <= nsteps) kc *= 2;
  if (act_i64) launch_lds_gemv<true, 0>(W, act, W.cols, 1, nullptr, W.rows, acc, s, ks, kc);
  else launch_lds_gemv<false, 0>(W, act, W.cols, 1, nullptr, W.rows, acc, s, ks, kc);
}

// Workgroups of a kernel that fit on the device at once (occupancy x CUs),
// queried once per kernel.
static uint64_t resident_blocks(const void* kernel, int threads) {
  static std::mutex mu;
  static std::vector<std::pair<const void*, uint64_t>> cache;
  std::lock_guard<std::mutex> lock(mu);
  for (const auto& e : cache)
    if (e.first == kernel) return e.second;
  int dev = 0, cus = 0, per = 0;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, 0) != hipSuccess || cus <= 0 || per <= 0) {
    cus = 256;
    per = 1;
  }
  const uint64_t n = uint64_t(cus) * uint64_t(per);
  cache.push_back({kernel, n});
  return n;
}

template <int KS, int EPI, int NG>
static void launch_gemv_dec_ks(const DevMatrix& W, const int8_t* limbs, uint32_t ntok, uint32_t kc, uint64_t groups,
                               int32_t* out, uint64_t out_ld, int64_t* acc, uint64_t acc_ld, int8_t* out_limbs,
                               uint64_t out_kpad, hipStream_t s) {
  // k_gemv_dec takes shares of up to 3 K steps in one round trip and is the
  // faster of the two there (measured on E4B's qkv and down projections)
  const uint64_t nsteps = W.kpad / 128, cper = (nsteps + kc - 1) / kc, per = (cper + KS - 1) / KS;
  const bool dg = W.planes > 1;
  if (NG == 1 && ntok == 1 && per > 3) {
    if (dg)
      hipLaunchKernelGGL((k_gemv_dec1<KS, EPI, true>), dim3(unsigned(groups * kc)), dim3(256), 0, s, W.q, W.scale,
                         W.rowsum, limbs, W.rows, W.kpad, kc, out, acc, out_limbs, out_kpad, plane_log2(W));
    else
      hipLaunchKernelGGL((k_gemv_dec1<KS, EPI, false>), dim3(unsigned(groups * kc)), dim3(256), 0, s, W.q, W.scale,
                         W.rowsum, limbs, W.rows, W.kpad, kc, out, acc, out_limbs, out_kpad, 0);
  } else if (dg) {
    hipLaunchKernelGGL((k_gemv_dec<KS, EPI, NG, true>), dim3(unsigned(groups * kc)), dim3(256), 0, s, W.q, W.scale,
                       W.rowsum, limbs, W.rows, W.kpad, kc, ntok, out, out_ld, acc, acc_ld, out_limbs, out_kpad,
                       plane_log2(W));
  } else {
    hipLaunchKernelGGL((k_gemv_dec<KS, EPI, NG, false>), dim3(unsigned(groups * kc)), dim3(256), 0, s, W.q, W.scale,
                       W.rowsum, limbs, W.rows, W.kpad, kc, ntok, out, out_ld, acc, acc_ld, out_limbs, out_kpad, 0);
  }
}

template <int NG>
static void launch_gemv_dec_ng(const DevMatrix& W, const int8_t* limbs, uint32_t ntok, int32_t* out, uint64_t out_ld,
                               int64_t* acc, uint64_t acc_ld, int epilogue, int8_t* out_limbs, uint64_t out_kpad,
                               hipStream_t s) {
  const uint64_t ntiles = (W.rows + 15) / 16, nsteps = W.kpad / 128;
  // (k_gemv_dec1 has the same 5 workgroups per CU as k_gemv_dec<4, 0, 1>)
  const uint64_t cap = resident_blocks(reinterpret_cast<const void*>(&k_gemv_dec<4, 0, NG, false>), 256);
  // a tile's waves: K shares x digit planes, at most the workgroup's four
  const uint64_t P = uint64_t(W.planes);
  auto groups = [&](int ks) { return (ntiles * ks * P + 3) / 4; };
  // in-workgroup K split: smallest that fills the device, keeping >= 4 K steps per wave
  int ks = 1;
  while (uint64_t(ks) * 2 * P <= 4 && groups(ks) < cap && nsteps >= uint64_t(ks) * 2 * 4) ks *= 2;
  // K chunks across workgroups (atomic outputs only) while the launch stays resident
  uint32_t kc = 1;
  if (acc)
    while (groups(ks) * kc * 2 <= cap && nsteps >= uint64_t(ks) * kc * 2) kc *= 2;
  const uint64_t g = std::min<uint64_t>(groups(ks), std::max<uint64_t>(cap / kc, 1));
#define DET_GEMV_DEC(KS, EPI) \
  launch_gemv_dec_ks<KS, EPI, NG>(W, limbs, ntok, kc, g, out, out_ld, acc, acc_ld, out_limbs, out_kpad, s)
  if (epilogue == 1) {
    if (ks == 4) DET_GEMV_DEC(4, 1); else if (ks == 2) DET_GEMV_DEC(2, 1); else DET_GEMV_DEC(1, 1);
  } else {
    if (ks == 4) DET_GEMV_DEC(4, 0); else if (ks == 2) DET_GEMV_DEC(2, 0); else DET_GEMV_DEC(1, 0);
  }
#undef DET_GEMV_DEC
}

static uint64_t device_cus() {
  static const uint64_t n = [] {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    return uint64_t(cus);
  }();
  return n;
}

template <int NG>
static void launch_gemv_dec_wg(const DevMatrix& W, const int8_t* limbs, uint32_t ntok, int32_t* out, uint64_t out_ld,
                               int64_t* acc, uint64_t acc_ld, int epilogue, int8_t* out_limbs, uint64_t out_kpad,
                               hipStream_t s, const int64_t* acc_in = nullptr, uint64_t in_ld = 0,
                               int8_t* out_om = nullptr) {
  const uint64_t ntiles = (W.rows + 15) / 16, nsteps = W.kpad / 128;
  const void* fn = epilogue == 1 ? reinterpret_cast<const void*>(&k_gemv_dec_wg<1, NG, false>)
                                 : reinterpret_cast<const void*>(&k_gemv_dec_wg<0, NG, false>);
  const uint64_t cap = resident_blocks(fn, 256);
  const uint64_t groups = (ntiles * uint64_t(W.planes) + 3) / 4;
  // K chunks across workgroups (atomic outputs only) up to about 2.5
  // workgroups per CU (measured best at E4B shapes), keeping at least two K
  // steps per chunk
  uint32_t kc = 1;
  const uint64_t target = device_cus() * 5 / 2;
  if (acc)
    while (groups * kc * 2 <= target && nsteps >= uint64_t(kc) * 2 * 2) kc *= 2;
  const uint64_t g = std::min<uint64_t>(groups, std::max<uint64_t>(cap / kc, 1));
#define DET_DEC_WG(E, DG, IN)                                                                                    \
  hipLaunchKernelGGL((k_gemv_dec_wg<E, NG, DG, IN>), dim3(unsigned(g * kc)), dim3(256), 0, s, W.q, W.scale,        \
                     W.rowsum, limbs, W.rows, W.kpad, kc, ntok, out, out_ld, acc, acc_ld, out_limbs, out_kpad,      \
                     plane_log2(W), acc_in, in_ld, out_om)
  if (acc_in) {
    if (W.planes == 1) DET_DEC_WG(0, false, true);
    else DET_DEC_WG(0, true, true);
  } else if (epilogue == 1) {
    if (W.planes == 1) DET_DEC_WG(1, false, false);
    else DET_DEC_WG(1, true, false);
  } else {
    if (W.planes == 1) DET_DEC_WG(0, false, false);
    else DET_DEC_WG(0, true, false);
  }
#undef DET_DEC_WG
}

// 5-16 tokens over single-plane weights with K of at least 24 half-steps
// (1536 columns): k_gemv_rega. False where the shape is outside its range
// (digit planes, short K, or a K split without atomic outputs) or where the
// tiles cannot give every workgroup two or more: a workgroup loads its K
// chunk's activation limbs of all tokens once, which only several tiles
// amortise.
// - Atomic outputs: workgroups of 2 waves x HPW half-steps, so K splits into
//   many chunks and each workgroup loads a small share of the activations
//   (HPW from 5, 4, 3, whichever leaves the fewest idle half-steps), about
//   512 workgroups with at least three tiles each. Measured on E4B shapes at
//   16 tokens: down 2560 x 10240 8.9 us in 16 chunks against 12.0 us for
//   k_gemv_dec_wg and 12.0 us with 8 waves x 5 half-steps in 4 chunks;
//   q/k/v 3072 x 2560 5.6 us in 4 chunks against 6.7 us.
// - One K chunk (requantized outputs, the GELU epilogue): 8 waves x up to 5
//   half-steps cover K = 2560 in one workgroup per CU (gate/up 20480 x 2560
//   17.2 us against 25.3 us; lm_head 262144 x 2560 122 us against 185 us).
template <int NG>
static bool launch_gemv_rega(const DevMatrix& W, const int8_t* limbs, uint32_t ntok, int32_t* out, uint64_t out_ld,
                             int64_t* acc, uint64_t acc_ld, int epilogue, int8_t* out_limbs, uint64_t out_kpad,
                             hipStream_t s, const int8_t* a_om, int8_t* out_om) {
  const uint64_t nhs = W.kpad / 64;
  if (W.planes != 1 || nhs < 24) return false;
  const uint64_t ntiles = (W.rows + 15) / 16;
  const uint64_t cus = device_cus();
  if (acc && epilogue == 0) {
    uint64_t hpw = 5, best = ~uint64_t(0);
    for (uint64_t h = 5; h >= 3; --h) {
      const uint64_t idle = (nhs + 2 * h - 1) / (2 * h) * 2 * h - nhs;
      if (idle < best) best = idle, hpw = h;
    }
    const uint64_t kc = (nhs + 2 * hpw - 1) / (2 * hpw);
    if (ntiles * kc < 2 * cus) return false;
    const uint64_t groups =
        std::max<uint64_t>(1, std::min<uint64_t>({ntiles, std::max<uint64_t>(2 * cus / kc, 1), ntiles / 3}));
    const dim3 grid(unsigned(groups * kc)), block(128);
#define DET_REGA2(H)                                                                                              \
    hipLaunchKernelGGL((k_gemv_rega<0, NG, 2, H>), grid, block, 0, s, W.q, W.scale, W.rowsum, limbs, W.rows, W.kpad, \
                       uint32_t(kc), ntok, out, out_ld, acc, acc_ld, out_limbs, out_kpad, a_om, out_om)
    if (hpw == 5) DET_REGA2(5); else if (hpw == 4) DET_REGA2(4); else DET_REGA2(3);
#undef DET_REGA2
    return true;
  }
  if (acc || nhs > 40 || ntiles < 2 * cus) return false;
  const uint64_t hpw = (nhs + 7) / 8;
  const uint64_t groups = std::min<uint64_t>(ntiles, cus);
  const dim3 grid{unsigned(groups)}, block{512};
#define DET_REGA(E, H)                                                                                          \
  hipLaunchKernelGGL((k_gemv_rega<E, NG, 8, H>), grid, block, 0, s, W.q, W.scale, W.rowsum, limbs, W.rows, W.kpad, \
                     1u, ntok, out, out_ld, acc, acc_ld, out_limbs, out_kpad, a_om, out_om)
  if (epilogue == 1) {
    if (hpw == 5) DET_REGA(1, 5); else if (hpw == 4) DET_REGA(1, 4); else DET_REGA(1, 3);
  } else {
    if (hpw == 5) DET_REGA(0, 5); else if (hpw == 4) DET_REGA(0, 4); else DET_REGA(0, 3);
  }
#undef DET_REGA
  return true;
}

bool gemv_dec_batch_in64_ok(const DevMatrix& W, uint32_t ntok, uint64_t in_ld) {
  const uint32_t tail = ntok % 16;
  return W.storage == kInt8 && W.rows > 0 && W.cols == W.kpad && in_ld % 2 == 0 && ntok >= 5 &&
         (tail == 0 || tail >= 5);
}

void launch_gemv_dec_batch_in64(const DevMatrix& W, const int64_t* acc_in, uint64_t in_ld, uint32_t ntok,
                                int64_t* acc, uint64_t acc_ld, hipStream_t s) {
  if (!gemv_dec_batch_in64_ok(W, ntok, in_ld) || !acc)
    throw std::invalid_argument("launch_gemv_dec_batch_in64: shape outside the kernel's range");
  for (uint32_t t0 = 0; t0 < ntok; t0 += 16) {
    const uint32_t nt = ntok - t0 < 16 ? ntok - t0 : 16;
    const int64_t* a_in = acc_in + uint64_t(t0) * in_ld;
    int64_t* a = acc + uint64_t(t0) * acc_ld;
    if (nt <= 8) launch_gemv_dec_wg<2>(W, nullptr, nt, nullptr, 0, a, acc_ld, 0, nullptr, 0, s, a_in, in_ld);
    else launch_gemv_dec_wg<4>(W, nullptr, nt, nullptr, 0, a, acc_ld, 0, nullptr, 0, s, a_in, in_ld);
  }
}

void launch_gemv_dec_batch(const DevMatrix& W, const int8_t* limbs, uint32_t ntok, int32_t* out, uint64_t out_ld,
                           int64_t* acc, uint64_t acc_ld, int epilogue, int8_t* out_limbs, uint64_t out_kpad,
                           hipStream_t s, const int8_t* limbs_om, int8_t* out_om) {
  if (W.rows == 0 || ntok == 0) return;
  // up to 16 tokens per pass over the weights (pass p of the operand-major
  // copies at p * 64 * kpad bytes)
  for (uint32_t t0 = 0; t0 < ntok; t0 += 16) {
    const uint32_t nt = ntok - t0 < 16 ? ntok - t0 : 16;
    const int8_t* l = limbs + uint64_t(t0) * 4 * W.kpad;
    int32_t* o = out ? out + uint64_t(t0) * out_ld : nullptr;
    int64_t* a = acc ? acc + uint64_t(t0) * acc_ld : nullptr;
    int8_t* ol = out_limbs ? out_limbs + uint64_t(t0) * 4 * out_kpad : nullptr;
    const int8_t* lo = limbs_om ? limbs_om + uint64_t(t0) * 4 * W.kpad : nullptr;
    int8_t* oo = (out_om && out_limbs) ? out_om + uint64_t(t0) * 4 * out_kpad : nullptr;
    if (nt <= 4) launch_gemv_dec_ng<1>(W, l, nt, o, out_ld, a, acc_ld, epilogue, ol, out_kpad, s);
    else if (nt <= 8) {
      if (!launch_gemv_rega<2>(W, l, nt, o, out_ld, a, acc_ld, epilogue, ol, out_kpad, s, lo, oo))
        launch_gemv_dec_wg<2>(W, l, nt, o, out_ld, a, acc_ld, epilogue, ol, out_kpad, s, nullptr, 0, oo);
    } else if (!launch_gemv_rega<4>(W, l, nt, o, out_ld, a, acc_ld, epilogue, ol, out_kpad, s, lo, oo)) {
      launch_gemv_dec_wg<4>(W, l, nt, o, out_ld, a, acc_ld, epilogue, ol, out_kpad, s, nullptr, 0, oo);
    }
  }
}

void launch_gemv_dec(const DevMatrix& W, const int8_t* limbs, int32_t* out, int64_t* acc, int epilogue,
                     int8_t* out_limbs, uint64_t out_kpad, hipStream_t s) {
  launch_gemv_dec_ng<1>(W, limbs, 1, out, 0, acc, 0, epilogue, out_limbs, out_kpad, s);
}

// Work split of k_gemv_norm: one workgroup per CU (or per tile when fewer),
// each taking ceil(tiles / G) tiles of ceil(steps / kNormD) jobs.
struct NormSplit {
  uint64_t grid, jobs;
};
static NormSplit norm_split(const DevMatrix& W) {
  const uint64_t ntiles = (W.rows + 15) / 16, nsteps = W.kpad / 128;
  const uint64_t grid = std::min<uint64_t>(ntiles, device_cus());
  const uint64_t tpw = (ntiles + grid - 1) / grid;
  return {grid, tpw * ((nsteps + kNormD - 1) / kNormD) * uint64_t(W.planes)};
}
bool gemv_norm_fits(const DevMatrix& W, uint64_t H) {
  if (W.storage != kInt8 || W.rows == 0 || H == 0 || H % 4 != 0 || W.cols != H || W.kpad > kNormMaxK) return false;
  return norm_split(W).jobs <= 32;
}
void launch_gemv_norm(const DecNormIn& ni, const DevMatrix& W, int epilogue, int64_t* acc_out, int32_t* out,
                      int8_t* out_limbs, uint64_t out_kpad, hipStream_t s) {
  if (!gemv_norm_fits(W, ni.H)) throw std::runtime_error("launch_gemv_norm: shape outside the fused kernel's range");
  const NormSplit sp = norm_split(W);
  // waves: one job each up to 16 jobs, else two, with as few idle job slots
  // as the instances allow; quads per thread: the fewest that cover the
  // kpad / 4 limb quads
  const uint64_t kq = W.kpad / 4;
  auto qpt = [&](int nw) { return (kq + 64 * nw - 1) / (64 * nw); };
#define DET_NORM_LAUNCH_DG(NW, JM, QPT, E, DG)                                                                       \
  hipLaunchKernelGGL((k_gemv_norm<NW, JM, QPT, E, DG>), dim3(unsigned(sp.grid)), dim3(64 * NW), 0, s, ni, W.q,       \
                     W.scale, W.rowsum, W.rows, W.kpad, acc_out, out, out_limbs, out_kpad, plane_log2(W))
#define DET_NORM_LAUNCH(NW, JM, QPT)                                                                                 \
  do {                                                                                                               \
    const bool dg = W.planes > 1;                                                                                    \
    if (epilogue == 1) {                                                                                             \
      if (dg) DET_NORM_LAUNCH_DG(NW, JM, QPT, 1, true);                                                              \
      else DET_NORM_LAUNCH_DG(NW, JM, QPT, 1, false);                                                                \
    } else {                                                                                                         \
      if (dg) DET_NORM_LAUNCH_DG(NW, JM, QPT, 0, true);                                                              \
      else DET_NORM_LAUNCH_DG(NW, JM, QPT, 0, false);                                                                \
    }                                                                                                                \
  } while (0)
  if (sp.jobs <= 4) {
    switch (qpt(4)) {
      case 1: DET_NORM_LAUNCH(4, 1, 1); break;
      case 2: DET_NORM_LAUNCH(4, 1, 2); break;
      case 3: DET_NORM_LAUNCH(4, 1, 3); break;
      default: DET_NORM_LAUNCH(4, 1, 4); break;
    }
  } else if (sp.jobs <= 10) {
    if (qpt(10) == 1) DET_NORM_LAUNCH(10, 1, 1);
    else DET_NORM_LAUNCH(10, 1, 2);
  } else if (sp.jobs <= 16) {
    DET_NORM_LAUNCH(16, 1, 1);
  } else if (sp.jobs <= 20) {
    if (qpt(10) == 1) DET_NORM_LAUNCH(10, 2, 1);
    else DET_NORM_LAUNCH(10, 2, 2);
  } else {
    DET_NORM_LAUNCH(16, 2, 1);
  }
#undef DET_NORM_LAUNCH
#undef DET_NORM_LAUNCH_DG
}

// a_tiled holds the limb tiles of (m rounded up to 64) tokens, then the
// four-limb flag of every (token group, column part).
static uint64_t gemm_tile_bytes(uint64_t m, uint64_t kpad) { return ((m + 63) / 64) * 64 * 4 * kpad; }
static uint32_t* gemm_flags(const int8_t* a_tiled, uint64_t m, uint64_t kpad) {
  return reinterpret_cast<uint32_t*>(const_cast<int8_t*>(a_tiled) + gemm_tile_bytes(m, kpad));
}
uint64_t gemm_act_bytes(uint64_t m, uint64_t kpad) {
  const uint64_t groups = (m + 63) / 64 * 4;
  return gemm_tile_bytes(m, kpad) + 4 * groups * limb_parts(kpad);
}

template <int TA, int TB, int WM, int WN, uint32_t GM, int NBUF, bool SPLIT, bool GELU, bool DG>
static void launch_gemm_lds_dg(const DevMatrix& W, uint64_t m, int32_t* out, uint64_t ld_out, int64_t* acc_out,
                               const int8_t* a_tiled, uint64_t a_tiles, hipStream_t s, RowSplit split, KSplit ks) {
  constexpr int NW = WM * WN;
  constexpr uint32_t lds = uint32_t(NBUF) * uint32_t((2 * (TA + TB) + NW - 1) / NW * NW) * 1024u;
  static_assert(lds <= 160u * 1024u, "LDS of one workgroup");
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&k_gemm_lds<TA, TB, WM, WN, GM, NBUF, SPLIT, GELU, DG>),
      hipFuncAttributeMaxDynamicSharedMemorySize, int(lds));
  (void)attr;
  const uint64_t mblocks = (m + 4 * TA - 1) / (4 * TA);
  const uint64_t nblocks = ((W.rows + 15) / 16 * uint64_t(W.planes) + TB - 1) / TB;
  hipLaunchKernelGGL((k_gemm_lds<TA, TB, WM, WN, GM, NBUF, SPLIT, GELU, DG>),
                     dim3(unsigned(mblocks * nblocks * ks.chunks)), dim3(64 * WM * WN), lds, s, a_tiled, W.q, W.scale,
                     W.rowsum, W.rowsum_p, W.rowsum_p_ld, W.rows, W.kpad, m, a_tiles, gemm_flags(a_tiled, m, W.kpad),
                     uint32_t(mblocks), out, ld_out, acc_out, split, ks, plane_log2(W));
}

template <int TA, int TB, int WM, int WN, uint32_t GM, int NBUF, bool SPLIT = false, bool GELU = false>
static void launch_gemm_lds_shape(const DevMatrix& W, uint64_t m, int32_t* out, uint64_t ld_out, int64_t* acc_out,
                                  const int8_t* a_tiled, uint64_t a_tiles, hipStream_t s, RowSplit split = {},
                                  KSplit ks = {}) {
  static_assert(TB / WN >= 1, "weight tiles per wave");
  if ((TB / WN) % W.planes) throw std::invalid_argument("GEMM block: a wave's weight tiles must hold whole digit-plane tiles");
  if (W.planes == 1)
    launch_gemm_lds_dg<TA, TB, WM, WN, GM, NBUF, SPLIT, GELU, false>(W, m, out, ld_out, acc_out, a_tiled, a_tiles, s,
                                                                     split, ks);
  else
    launch_gemm_lds_dg<TA, TB, WM, WN, GM, NBUF, SPLIT, GELU, true>(W, m, out, ld_out, acc_out, a_tiled, a_tiles, s,
                                                                    split, ks);
}

// K split of a GEMM whose 128 x 128 blocks leave CUs idle: chunks of at least
// four K steps, up to one block per CU (a second block on a CU shares its LDS
// bandwidth, which bounds a block's K step), with their partial planes within
// kGemmPlaneBudget bytes, and only where it saves at least kGemmSplitMinSteps
// K steps per block: the planes' stores and the summing kernel cost about
// that much (measured on E4B's projections at 128 rows).
constexpr uint64_t kGemmPlaneBudget = uint64_t(16) << 20;
constexpr uint64_t kGemmSplitMinSteps = 12;
// Small grids (single-plane matrices of at most 32 K steps whose 128 x 128
// blocks would leave CUs idle: the short prompts' q/k/v/o) take 16-token x
// 64-row blocks on 4 waves: four times the blocks, several per CU, and K split
// only where even those leave CUs idle. (Longer rows keep the larger block
// split in K: at 128 rows the 2560 x 10240 down projection took 40.8 us in
// the small block against 23.3 + 9.9 us split.)
static bool gemm_small(const DevMatrix& W, uint64_t m) {
  if (W.planes != 1 || W.kpad > 32 * 128) return false;
  const uint64_t blocks128 = ((m + 31) / 32) * (((W.rows + 15) / 16 + 7) / 8);
  return blocks128 < device_cus();
}
// One-round block shapes: a grid of one block per CU that fills at least
// nine tenths of the CUs, for single-plane matrices of at most 32 K steps,
// each wave one token group x one or five weight tiles, four LDS buffers
// where they fit (their copy halves per K step need not divide over the
// waves). Tried in this order (cold weights, 128 rows):
//   64 tokens x 160 rows, 8 waves, 2 buffers (112 KB): the 20480-row gate/up
//     37.1 us against 39.7 us in 256 x 256 blocks, with the GELU epilogue
//     41.1 against 51.2 us in 128 x 128 blocks;
//   32 tokens x 48 rows, 6 waves (96 KB): q/k/v 3072 x 2560 11.7 against
//     14.4 us in 384 16 x 64 blocks;
//   16 tokens x 80 rows, 5 waves (80 KB): o 2560 x 2048 8.5 against 9.3 us.
// At 512 and 2048 rows the grids take several rounds and none applies.
enum class PadShape { kNone, k64x160, k32x48, k16x80 };
static PadShape gemm_pad_shape(const DevMatrix& W, uint64_t m) {
  if (W.storage != kInt8 || W.planes != 1 || W.kpad > 32 * 128) return PadShape::kNone;
  const uint64_t tiles = (W.rows + 15) / 16, cus = device_cus();
  auto fills = [&](uint64_t tokens, uint64_t tb) {
    const uint64_t blocks = ((m + tokens - 1) / tokens) * ((tiles + tb - 1) / tb);
    return blocks <= cus && blocks * 10 >= cus * 9;
  };
  if (fills(64, 10)) return PadShape::k64x160;
  if (fills(32, 3)) return PadShape::k32x48;
  if (fills(16, 5)) return PadShape::k16x80;
  return PadShape::kNone;
}
template <bool SPLIT, bool GELU>
static void launch_gemm_pad(PadShape p, const DevMatrix& W, uint64_t m, int32_t* out, uint64_t ld_out,
                            int64_t* acc_out, const int8_t* a_tiled, uint64_t a_tiles, hipStream_t s,
                            RowSplit split) {
  if (p == PadShape::k64x160)
    launch_gemm_lds_dg<16, 10, 4, 2, 8, 2, SPLIT, GELU, false>(W, m, out, ld_out, acc_out, a_tiled, a_tiles, s, split, {});
  else if (p == PadShape::k32x48)
    launch_gemm_lds_dg<8, 3, 2, 3, 8, 4, SPLIT, GELU, false>(W, m, out, ld_out, acc_out, a_tiled, a_tiles, s, split, {});
  else
    launch_gemm_lds_dg<4, 5, 1, 5, 8, 4, SPLIT, GELU, false>(W, m, out, ld_out, acc_out, a_tiled, a_tiles, s, split, {});
}
uint32_t gemm_kchunks(const DevMatrix& W, uint64_t m) {
  if (W.storage != kInt8 || m == 0 || W.rows == 0 || W.planes > 2) return 1;
  if (gemm_pad_shape(W, m) != PadShape::kNone) return 1;  // one-round blocks, no K split
  const bool small = gemm_small(W, m);
  const uint64_t blocks = small ? ((m + 15) / 16) * (((W.rows + 15) / 16 + 3) / 4)
                                : ((m + 31) / 32) * (((W.rows + 15) / 16 * uint64_t(W.planes) + 7) / 8);
  const uint64_t cus = device_cus();
  if (blocks >= cus) return 1;
  const uint64_t nsteps = W.kpad / 128;
  uint64_t kc = std::min<uint64_t>(cus / blocks, nsteps / 4);
  kc = std::min<uint64_t>(kc, kGemmPlaneBudget / (m * W.rows * 8));
  if (kc < 2 || nsteps - (nsteps + kc - 1) / kc < kGemmSplitMinSteps) return 1;
  return uint32_t(kc);
}
uint64_t gemm_plane_bytes(const DevMatrix& W, uint64_t m) {
  const uint32_t kc = gemm_kchunks(W, m);
  return kc > 1 ? uint64_t(kc) * m * W.rows * 8 : 0;
}

void launch_gemm_limbs(const int32_t* act, uint64_t m, uint64_t k, uint64_t ld_act, uint64_t kpad, int8_t* a_tiled,
                       hipStream_t s) {
  if (m == 0) return;
  const uint64_t groups = (m + 63) / 64 * 4;  // the larger block's 4 token groups
  const int vec = (reinterpret_cast<uintptr_t>(act) % 16 == 0 && ld_act % 4 == 0) ? 1 : 0;
  const dim3 grid(unsigned(groups), unsigned(limb_parts(kpad)));
  const uint64_t wgs = uint64_t(grid.x) * grid.y;
  if (wgs <= 256)
    hipLaunchKernelGGL(k_act_limbs_rows<1024>, grid, dim3(1024), 0, s, act, m, k, ld_act, kpad, vec,
                       gemm_flags(a_tiled, m, kpad), a_tiled);
  else if (wgs <= 512)
    hipLaunchKernelGGL(k_act_limbs_rows<512>, grid, dim3(512), 0, s, act, m, k, ld_act, kpad, vec,
                       gemm_flags(a_tiled, m, kpad), a_tiled);
  else
    hipLaunchKernelGGL(k_act_limbs_rows<256>, grid, dim3(256), 0, s, act, m, k, ld_act, kpad, vec,
                       gemm_flags(a_tiled, m, kpad), a_tiled);
}

void launch_gemm_tiled(const DevMatrix& W, uint64_t m, int32_t* out, uint64_t ld_out, int64_t* acc_out,
                       const int8_t* a_tiled, hipStream_t s, const RowSplit* split, int64_t* planes) {
  if (W.rows == 0 || m == 0) return;
  const uint64_t a_tiles = (m + 63) / 64 * 64 / 4;
  const PadShape pad = gemm_pad_shape(W, m);
  if (pad != PadShape::kNone) {
    if (split) return launch_gemm_pad<true, false>(pad, W, m, out, ld_out, nullptr, a_tiled, a_tiles, s, *split);
    return launch_gemm_pad<false, false>(pad, W, m, out, ld_out, acc_out, a_tiled, a_tiles, s, {});
  }
  const uint32_t kc = planes ? gemm_kchunks(W, m) : 1;
  const bool small = gemm_small(W, m);
  // Grids that fit one round at the deeper pipeline's residency (64 KB of LDS
  // per small block, two per CU; 128 KB per 128 x 128 block, one per CU) keep
  // three K steps of copies in flight instead of one: at 128 rows the K loop
  // of a lone block waits on its copies' latency (q/k/v 3072 x 2560 18.4 ->
  // 14.2 us, o 11.8 -> 9.5, down's three K chunks 27.2 -> 20.1 us); larger
  // grids keep two buffers and two blocks per CU.
  const uint64_t cus = device_cus();
  const uint64_t vt = (W.rows + 15) / 16 * uint64_t(W.planes);
  const bool deep = small ? ((m + 15) / 16) * ((vt + 3) / 4) * kc <= 2 * cus : ((m + 31) / 32) * ((vt + 7) / 8) * kc <= cus;
  if (kc > 1) {
    KSplit ks;
    ks.chunks = kc;
    ks.planes = planes;
    if (small && deep) launch_gemm_lds_shape<4, 4, 1, 4, 8, 4>(W, m, nullptr, 0, nullptr, a_tiled, a_tiles, s, {}, ks);
    else if (small) launch_gemm_lds_shape<4, 4, 1, 4, 8, 2>(W, m, nullptr, 0, nullptr, a_tiled, a_tiles, s, {}, ks);
    else if (deep) launch_gemm_lds_shape<8, 8, 2, 4, 8, 4>(W, m, nullptr, 0, nullptr, a_tiled, a_tiles, s, {}, ks);
    else launch_gemm_lds_shape<8, 8, 2, 4, 8, 2>(W, m, nullptr, 0, nullptr, a_tiled, a_tiles, s, {}, ks);
    const uint64_t total = m * W.rows;
    hipLaunchKernelGGL(k_gemm_reduce, dim3(unsigned((total + 511) / 512)), dim3(256), 0, s, planes, kc, m, W.rows,
                       out, ld_out, acc_out, split ? *split : RowSplit{});
    return;
  }
  // row-split outputs take the 128 x 128 blocks only (their epilogue is kept
  // out of the 256 x 256 block's registers)
  if (split) {
    if (W.planes > 2) throw std::invalid_argument("row-split GEMM: at most two digit planes");
    if (small && deep)
      return launch_gemm_lds_shape<4, 4, 1, 4, 8, 4, true>(W, m, out, ld_out, nullptr, a_tiled, a_tiles, s, *split);
    if (small) return launch_gemm_lds_shape<4, 4, 1, 4, 8, 2, true>(W, m, out, ld_out, nullptr, a_tiled, a_tiles, s, *split);
    if (deep) return launch_gemm_lds_shape<8, 8, 2, 4, 8, 4, true>(W, m, out, ld_out, nullptr, a_tiled, a_tiles, s, *split);
    return launch_gemm_lds_shape<8, 8, 2, 4, 8, 2, true>(W, m, out, ld_out, nullptr, a_tiled, a_tiles, s, *split);
  }
  if (small && deep) return launch_gemm_lds_shape<4, 4, 1, 4, 8, 4>(W, m, out, ld_out, acc_out, a_tiled, a_tiles, s);
  if (small) return launch_gemm_lds_shape<4, 4, 1, 4, 8, 2>(W, m, out, ld_out, acc_out, a_tiled, a_tiles, s);
  // 64 tokens x 256 rows on 8 waves (one block per CU) when its blocks fill
  // whole rounds of the device; otherwise 32 tokens x 128 rows on 8 waves
  // (two blocks per CU, so two waves per SIMD hide each other's LDS and
  // MFMA latency), whose finer grid leaves a smaller last round. Four digit
  // planes take the larger block (four weight tiles per wave).
  // A single round of 256 x 256 blocks that fills at least five eighths of
  // the CUs also beats 128 x 128 blocks that need more than one round at two
  // per CU (measured on the 20480-row gate/up slab at 128 rows: 160 blocks,
  // 41 us against 49 us for 640 128 x 128 blocks, cold weights; single-plane
  // matrices of that shape now take the one-round 64 x 160 block above, and
  // this rule serves digit-plane matrices and rows past 4096 columns).
  const uint64_t big = ((m + 63) / 64) * ((vt + 15) / 16);
  const uint64_t rounds = (big + cus - 1) / cus;
  const uint64_t blocks128 = ((m + 31) / 32) * ((vt + 7) / 8);
  const bool one_round = big < cus && big * 8 >= cus * 5 && blocks128 > 2 * cus;
  if (W.planes > 2 || (big >= cus && big * 10 >= rounds * cus * 9) || one_round)
    launch_gemm_lds_shape<16, 16, 2, 4, 4, 2>(W, m, out, ld_out, acc_out, a_tiled, a_tiles, s);
  else if (deep)
    launch_gemm_lds_shape<8, 8, 2, 4, 8, 4>(W, m, out, ld_out, acc_out, a_tiled, a_tiles, s);
  else
    launch_gemm_lds_shape<8, 8, 2, 4, 8, 2>(W, m, out, ld_out, acc_out, a_tiled, a_tiles, s);
}

void launch_gemm_tiled_gelu(const DevMatrix& W, uint64_t m, int32_t* out, uint64_t ld_out, const int8_t* a_tiled,
                            hipStream_t s) {
  if (W.rows == 0 || m == 0) return;
  if (W.rows % 16) throw std::invalid_argument("gate/up GEMM: rows must be whole tiles of 8 gate + 8 up rows");
  if (W.planes > 2) throw std::invalid_argument("gate/up GEMM: at most two digit planes");
  const uint64_t a_tiles = (m + 63) / 64 * 64 / 4;
  // a one-round block shape where one fills the device, else 128 x 128
  // blocks (no K split): with the GELU arithmetic in its epilogue the
  // 256 x 256 block does not fit its registers
  const PadShape pad = gemm_pad_shape(W, m);
  if (pad != PadShape::kNone)
    return launch_gemm_pad<false, true>(pad, W, m, out, ld_out, nullptr, a_tiled, a_tiles, s, {});
  launch_gemm_lds_shape<8, 8, 2, 4, 8, 2, false, true>(W, m, out, ld_out, nullptr, a_tiled, a_tiles, s);
}

void launch_gemm(const DevMatrix& W, const int32_t* act, uint64_t m, uint64_t ld_act, int32_t* out, uint64_t ld_out,
                 int64_t* acc_out, int8_t* a_tiled, hipStream_t s, int64_t* planes) {
  if (W.rows == 0 || m == 0) return;
  launch_gemm_limbs(act, m, W.cols, ld_act, W.kpad, a_tiled, s);
  launch_gemm_tiled(W, m, out, ld_out, acc_out, a_tiled, s, nullptr, planes);
}

void launch_linear(const DevMatrix& W, const int32_t* act, uint64_t m, uint64_t ld_act, int32_t* out,
                   uint64_t ld_out, int64_t* acc_out, int8_t* limbs, hipStream_t s) {
  if (W.rows == 0 || m == 0) return;
  if (W.storage == kInt8) {
    // tokens in groups of 4 (one 16-row MFMA A tile = 4 tokens x 4 limbs)
    for (uint64_t t0 = 0; t0 < m; t0 += 4) {
      const uint32_t mm = uint32_t(m - t0 < 4 ? m - t0 : 4);
      int32_t* o = acc_out ? nullptr : out + t0 * ld_out;
      int64_t* ao = acc_out ? acc_out + t0 * ld_out : nullptr;
      if (mm == 1 && gemv_tile_fits(W)) {
        launch_gemv_tile(W, act + t0 * ld_act, false, o, ao, s);
      } else if (gemv_fits_lds(W, mm)) {
        launch_lds_gemv<false, 0>(W, act + t0 * ld_act, ld_act, mm, o, ld_out, ao, s);
      } else {
        launch_act_limbs(act + t0 * ld_act, mm, W.cols, ld_act, W.kpad, limbs, s);
        hipLaunchKernelGGL(k_gemv_i8<8>, dim3(blocks_for(W.rows, 16)), dim3(512), 0, s, W.q, W.scale, W.rowsum,
                           limbs, W.rows, W.kpad, mm, o, ld_out, ao, plane_log2(W));
      }
    }
  } else if (W.storage == kI16) {
    hipLaunchKernelGGL(k_gemv_wide<int16_t>, dim3(blocks_for(W.rows, 4)), dim3(256), 0, s,
                       static_cast<const int16_t*>(W.w), W.rows, W.cols, act, ld_act, uint32_t(m), out, ld_out,
                       acc_out);
  } else {
    hipLaunchKernelGGL(k_gemv_wide<int32_t>, dim3(blocks_for(W.rows, 4)), dim3(256), 0, s,
                       static_cast<const int32_t*>(W.w), W.rows, W.cols, act, ld_act, uint32_t(m), out, ld_out,
                       acc_out);
  }
}

void launch_rmsnorm_add(int32_t* dst, const int32_t* src, const int32_t* res, uint64_t rows, uint64_t cols,
                        uint64_t ld, const int32_t* w, int64_t eps, hipStream_t s) {
  if (rows == 0) return;
  const dim3 g(static_cast<unsigned>(rows));
  if (cols > 512 && cols <= 2048)
    hipLaunchKernelGGL((k_rmsnorm_wide<256, 8>), g, dim3(256), 0, s, src, dst, cols, ld, w, eps, res);
  else if (cols > 2048 && cols <= 4096)
    hipLaunchKernelGGL((k_rmsnorm_wide<256, 16>), g, dim3(256), 0, s, src, dst, cols, ld, w, eps, res);
  else if (cols > 4096 && cols <= 8192)
    hipLaunchKernelGGL((k_rmsnorm_wide<512, 16>), g, dim3(512), 0, s, src, dst, cols, ld, w, eps, res);
  else if (cols > 8192 && cols <= 16384)
    hipLaunchKernelGGL((k_rmsnorm_wide<1024, 16>), g, dim3(1024), 0, s, src, dst, cols, ld, w, eps, res);
  else
    hipLaunchKernelGGL(k_rmsnorm, dim3(blocks_for(rows, 4)), dim3(256), 0, s, src, dst, res, rows, cols, ld, w, eps);
}

void launch_rmsnorm_add_norm(int32_t* x, const int32_t* src, int32_t* normed, uint64_t rows, uint64_t cols,
                             uint64_t ld, const int32_t* w1, const int32_t* w2, int64_t eps, hipStream_t s,
                             bool has_scalar, int32_t scalar) {
  if (rows == 0) return;
  if (cols > 2048 && cols <= 4096) {
    hipLaunchKernelGGL((k_rmsnorm_add_norm<256, 16>), dim3(unsigned(rows)), dim3(256), 0, s, src, x, normed, cols, ld,
                       w1, w2, eps, has_scalar ? 1 : 0, scalar);
  } else {
    launch_rmsnorm_add(x, src, x, rows, cols, ld, w1, eps, s);
    if (has_scalar) {
      if (ld != cols) throw std::runtime_error("rmsnorm_add_norm: the layer scalar needs contiguous rows");
      launch_scale(x, rows * cols, scalar, s);
    }
    launch_rmsnorm_to(normed, x, rows, cols, ld, w2, eps, s);
  }
}

void launch_rmsnorm_to(int32_t* dst, const int32_t* src, uint64_t rows, uint64_t cols, uint64_t ld, const int32_t* w,
                       int64_t eps, hipStream_t s) {
  launch_rmsnorm_add(dst, src, nullptr, rows, cols, ld, w, eps, s);
}

void launch_rmsnorm(int32_t* x, uint64_t rows, uint64_t cols, uint64_t ld, const int32_t* w, int64_t eps,
                    hipStream_t s) {
  launch_rmsnorm_to(x, x, rows, cols, ld, w, eps, s);
}

void launch_rope(int32_t* x, uint64_t rows, uint64_t ld, uint64_t heads, uint64_t hd, uint64_t half,
                 const int64_t* inv_freq, uint64_t pos0, uint64_t pos_step, hipStream_t s) {
  const uint64_t total = rows * heads * half;
  if (total == 0) return;
  hipLaunchKernelGGL(k_rope, dim3(blocks_for(total, 256)), dim3(256), 0, s, x, rows, ld, heads, hd, half, inv_freq,
                     pos0, pos_step, nullptr);
}

void launch_rope_rows(int32_t* x, uint64_t rows, uint64_t ld, uint64_t heads, uint64_t hd, uint64_t half,
                      const int64_t* inv_freq, const uint64_t* positions, hipStream_t s) {
  const uint64_t total = rows * heads * half;
  if (total == 0) return;
  hipLaunchKernelGGL(k_rope, dim3(blocks_for(total, 256)), dim3(256), 0, s, x, rows, ld, heads, hd, half, inv_freq,
                     0, 0, positions);
}

bool launch_head_norm_rope(const HeadNormRope& a0, uint64_t m, hipStream_t s) {
  if (a0.hd == 0 || a0.hd > 512 || a0.half > kHeadRopeMaxHalf || 2 * uint64_t(a0.half) > a0.hd) return false;
  if ((a0.qlimbs || a0.klimbs) && (a0.hd % 64 != 0 || !a0.qlimbs || a0.nqt * 16 < m || (a0.klimbs && a0.nkt != a0.nqt)))
    return false;
  if (m == 0) return true;
  HeadNormRope a = a0;
  a.rows = m;
  const uint64_t grid = a.qlimbs ? a.nqt * 16 : m;  // (padding rows of the last tile write zero blocks)
  if (a.hd <= 256) hipLaunchKernelGGL(k_head_norm_rope<4>, dim3(unsigned(grid)), dim3(256), 0, s, a);
  else hipLaunchKernelGGL(k_head_norm_rope<8>, dim3(unsigned(grid)), dim3(256), 0, s, a);
  return true;
}

void launch_attention(const AttnArgs& a, hipStream_t s) {
  if (a.n_queries == 0 || a.num_heads == 0) return;
  if (launch_attention_mfma(a, a.work, a.work_bytes, s)) return;
  uint64_t max_rows = a.causal ? (a.avail) : a.fix_count;
  if (max_rows == 0) max_rows = 1;
  // callers validate against kMaxAttentionRows first; a window that still
  // exceeds the LDS score rows fails here instead of leaving `out` stale
  if (max_rows > kMaxAttnRows) throw std::invalid_argument("attention window longer than 16000 rows is not supported");
  // grouped-head kernel: 128-bit row loads need 4-aligned widths and strides
  const uint64_t stride = std::max<uint64_t>(attn_row_stride(a), 1);
  const bool aligned = a.hd % 4 == 0 && a.kv_ld % 4 == 0 && a.hd <= 512;
  if (aligned) {
    int hb = 8;
    while (hb > 1 && (a.groups % hb != 0 || uint64_t(hb) * stride * 4 > 65536)) hb >>= 1;
    if (uint64_t(hb) * stride * 4 <= 65536) {
      const dim3 grid(a.num_heads / hb, a.n_queries);
      const size_t lds = size_t(hb) * stride * 4;
#define DET_ATTN_P(KPER, HB) \
  hipLaunchKernelGGL((k_attention_prefill<KPER, HB>), grid, dim3(kAttnPThreads), lds, s, a)
      if (a.hd <= 256) {
        if (hb == 8) DET_ATTN_P(16, 8); else if (hb == 4) DET_ATTN_P(16, 4); else if (hb == 2) DET_ATTN_P(16, 2); else DET_ATTN_P(16, 1);
      } else {
        if (hb == 8) DET_ATTN_P(32, 8); else if (hb == 4) DET_ATTN_P(32, 4); else if (hb == 2) DET_ATTN_P(32, 2); else DET_ATTN_P(32, 1);
      }
#undef DET_ATTN_P
      return;
    }
  }
  const size_t lds = size_t(max_rows) * sizeof(int32_t);
  hipLaunchKernelGGL(k_attention, dim3(a.num_heads, a.n_queries), dim3(kAttnThreads), lds, s, a);
}

void launch_add_sat(int32_t* d, const int32_t* src, uint64_t n, hipStream_t s) {
  if (n) hipLaunchKernelGGL(k_add_sat, dim3(blocks_for(n, 256)), dim3(256), 0, s, d, src, n);
}
void launch_gelu_mul(int32_t* g, const int32_t* u, uint64_t n, hipStream_t s) {
  if (n) hipLaunchKernelGGL(k_gelu_mul, dim3(blocks_for(n, 256)), dim3(256), 0, s, g, u, n);
}
void launch_scale(int32_t* x, uint64_t n, int32_t sc, hipStream_t s) {
  if (n) hipLaunchKernelGGL(k_scale, dim3(blocks_for(n, 256)), dim3(256), 0, s, x, n, sc);
}
void launch_softcap(int32_t* x, uint64_t n, int32_t cap, hipStream_t s) {
  if (n) hipLaunchKernelGGL(k_softcap, dim3(blocks_for(n, 256)), dim3(256), 0, s, x, n, cap);
}
void launch_gather_rows(const DevMatrix& M, const uint32_t* ids, uint64_t m, uint64_t col0, uint64_t ncols,
                        int32_t scale, int32_t* out, uint64_t ld_out, hipStream_t s, uint64_t ids_stride) {
  if (!m || !ncols) return;
  hipLaunchKernelGGL(k_gather_rows, dim3(blocks_for(ncols, 256), unsigned(m)), dim3(256), 0, s, M, ids, ids_stride, m,
                     col0, ncols, scale, out, ld_out);
}
void launch_kv_append(const int32_t* k, const int32_t* v, uint64_t w, uint64_t n, int32_t* const* kdst,
                      int32_t* const* vdst, hipStream_t s) {
  if (n && w) hipLaunchKernelGGL(k_kv_append, dim3(blocks_for(w, 256), unsigned(n)), dim3(256), 0, s, k, v, w, kdst, vdst);
}
uint64_t argmax_rows_scratch(uint64_t rows, uint64_t n) { return rows * ((n + kArgmaxSpan - 1) / kArgmaxSpan); }
void launch_argmax_rows(const int32_t* x, uint64_t rows, uint64_t n, int64_t* scratch, uint32_t* out, hipStream_t s) {
  if (rows == 0 || n == 0) return;
  const uint32_t parts = uint32_t((n + kArgmaxSpan - 1) / kArgmaxSpan);
  hipLaunchKernelGGL(k_argmax_rows_part, dim3(parts, unsigned(rows)), dim3(256), 0, s, x, n, scratch, parts);
  hipLaunchKernelGGL(k_argmax_rows_final, dim3(unsigned(rows)), dim3(256), 0, s, scratch, parts, out);
}
void launch_argmax(const int32_t* x, uint64_t n, int64_t* scratch, uint32_t* out, hipStream_t s) {
  const uint64_t parts = (n + 1023) / 1024;
  hipLaunchKernelGGL(k_argmax_partial, dim3(unsigned(parts)), dim3(256), 0, s, x, n, scratch);
  hipLaunchKernelGGL(k_argmax_final, dim3(1), dim3(256), 0, s, scratch, parts, out);
}

}  // namespace det
