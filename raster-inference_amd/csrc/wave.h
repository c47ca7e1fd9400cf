// 64-bit cross-lane reductions for 64-wide wavefronts on gfx950, built from
// DPP lane moves (VALU-speed, no LDS round trip):
//   quad_perm [1,0,3,2] (0xb1) and [2,3,0,1] (0x4e) combine lanes within a quad,
//   row_ror:4 (0x124) and row_ror:8 (0x128) rotate within a 16-lane row, so
//   after these four steps every lane holds its row's total;
//   row_bcast:15 (0x142) adds row r-1's last lane into row r and
//   row_bcast:31 (0x143) adds lane 31 into rows 2 and 3, so lane 63 ends with
//   the wavefront total, which is then read back as a wave-uniform value.
// The combining operations used here (wrapping add, saturating add of
// non-negative terms, signed max) are associative and commutative, so the
// results equal any sequential order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace det {

// Pointers typed as addressing global memory. Pointers read out of memory
// (per-sequence cache tables) are not known to be global, and accesses
// through them compile to FLAT instructions, which count against the
// LDS/scalar wait counter as well: a wait for an LDS result then also waits
// for every FLAT load in flight (an HBM round trip). Accesses through a
// global_ptr compile to global loads and stores.
template <class T>
using global_ptr = __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ global_ptr<T> to_global(T* p) {
  return (global_ptr<T>)p;
}
// A 16-byte global load of four int32 (HIP's int4 class cannot be assigned
// from an address-space-qualified object, so the load goes through a vector).
__device__ __forceinline__ int4 load_int4(global_ptr<const int32_t> p) {
  typedef int v4 __attribute__((ext_vector_type(4)));
  const v4 v = *(global_ptr<const v4>)p;
  return make_int4(v.x, v.y, v.z, v.w);
}

// s_waitcnt lgkmcnt(0) with the vector-memory count left open
constexpr int kWaitLdsOnly = 15 | (7 << 4) | (0 << 8) | (3 << 14);
// LDS hand-over inside a workgroup that leaves its global loads in flight (a
// __syncthreads fence would wait for them). Only LDS contents are handed over:
// global memory written by one wave is not made visible to the others.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kWaitLdsOnly);
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}
// LDS hand-over between the lanes of one wave (no other wave involved)
__device__ __forceinline__ void wave_lds_sync() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(kWaitLdsOnly);
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
}

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_move64(uint64_t v) {
  const uint32_t lo = uint32_t(__builtin_amdgcn_mov_dpp(int(uint32_t(v)), CTRL, 0xf, 0xf, false));
  const uint32_t hi = uint32_t(__builtin_amdgcn_mov_dpp(int(uint32_t(v >> 32)), CTRL, 0xf, 0xf, false));
  return (uint64_t(hi) << 32) | lo;
}

__device__ __forceinline__ uint64_t readlane64(uint64_t v, int lane) {
  const uint32_t lo = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(v)), lane));
  const uint32_t hi = uint32_t(__builtin_amdgcn_readlane(int(uint32_t(v >> 32)), lane));
  return (uint64_t(hi) << 32) | lo;
}

struct OpWrapAdd {
  __device__ __forceinline__ uint64_t operator()(uint64_t a, uint64_t b) const { return a + b; }
};
// Saturating add of non-negative int64 values (as uint64): min(a + b, INT64_MAX).
struct OpSatAdd {
  __device__ __forceinline__ uint64_t operator()(uint64_t a, uint64_t b) const {
    const uint64_t s = a + b;
    return s > uint64_t(INT64_MAX) ? uint64_t(INT64_MAX) : s;
  }
};
struct OpMaxI64 {
  __device__ __forceinline__ uint64_t operator()(uint64_t a, uint64_t b) const {
    return int64_t(a) > int64_t(b) ? a : b;
  }
};

// Total of each 16-lane row, in every lane of the row.
template <class Op>
__device__ __forceinline__ uint64_t row16_reduce(uint64_t v, Op op) {
  v = op(v, dpp_move64<0xb1>(v));
  v = op(v, dpp_move64<0x4e>(v));
  v = op(v, dpp_move64<0x124>(v));
  v = op(v, dpp_move64<0x128>(v));
  return v;
}

// Wavefront total, returned to every lane (all 64 lanes must be active).
template <class Op>
__device__ __forceinline__ uint64_t wave_reduce(uint64_t v, Op op) {
  v = row16_reduce(v, op);
  v = op(v, dpp_move64<0x142>(v));
  v = op(v, dpp_move64<0x143>(v));
  return readlane64(v, 63);
}

__device__ __forceinline__ int64_t wave_sum_wrap64(int64_t v) { return int64_t(wave_reduce(uint64_t(v), OpWrapAdd())); }
// v >= 0 in every lane
__device__ __forceinline__ int64_t wave_sum_sat64(int64_t v) { return int64_t(wave_reduce(uint64_t(v), OpSatAdd())); }
__device__ __forceinline__ int64_t wave_max64(int64_t v) { return int64_t(wave_reduce(uint64_t(v), OpMaxI64())); }

}  // namespace det
