// Test-only GPU driver: runs the product's integer arithmetic (det_arith.h)
// in device code on random and edge-case inputs and compares every result
// with the oracle's restatement of det_num/ops.rs on the host. The device
// build takes its own paths where the header has them (the 64x64->128-bit
// products and the reciprocal-square-root estimate of inv_sqrt_acc). Prints
// one line per function ("name checked mismatches") and exits non-zero on a
// mismatch.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

#include "../../oracle/oracle.h"
#include "../../raster-inference_amd/csrc/det_arith.h"

#define CK(x)                                                          \
  do {                                                                 \
    hipError_t e_ = (x);                                               \
    if (e_ != hipSuccess) {                                            \
      printf("%s: %s\n", #x, hipGetErrorString(e_));                   \
      exit(2);                                                         \
    }                                                                  \
  } while (0)

__global__ void k_inv_sqrt(const int64_t* __restrict__ x, int32_t* __restrict__ out, uint64_t n) {
  const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = det::inv_sqrt_acc(x[i]);
}
__global__ void k_div(const int64_t* __restrict__ v, const uint32_t* __restrict__ d, int64_t* __restrict__ out, uint64_t n) {
  const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = int64_t(det::div_rte_nonneg_u32(uint64_t(v[i]), d[i]));
}
__global__ void k_rms_scale(const int64_t* __restrict__ ss, const uint32_t* __restrict__ cnt,
                            const int64_t* __restrict__ eps, int32_t* __restrict__ out, uint64_t n) {
  const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = det::rms_scale_from_sumsq(ss[i], cnt[i], eps[i]);
}

__global__ void k_requant(const int64_t* __restrict__ x, int32_t* __restrict__ out, uint64_t n) {
  const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = det::requant(x[i]);
}
// op 0: mul_sat, 1: add_sat, 2: sub_sat
__global__ void k_binop(const int32_t* __restrict__ a, const int32_t* __restrict__ b, int op, int32_t* __restrict__ out,
                        uint64_t n) {
  const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = op == 0 ? det::mul_sat(a[i], b[i]) : (op == 1 ? det::add_sat(a[i], b[i]) : det::sub_sat(a[i], b[i]));
}
__global__ void k_add_sat64_nn(const int64_t* __restrict__ a, const int64_t* __restrict__ b, int64_t* __restrict__ out,
                               uint64_t n) {
  const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = det::add_sat64_nn(a[i], b[i]);
}

static std::mt19937_64 rng(777);

template <class T>
static T* to_dev(const std::vector<T>& v) {
  T* d = nullptr;
  CK(hipMalloc(&d, std::max<size_t>(v.size(), 1) * sizeof(T)));
  CK(hipMemcpy(d, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice));
  return d;
}

int main(int argc, char** argv) {
  const long N = argc > 1 ? atol(argv[1]) : 1000000;
  int failures = 0;
  // inv_sqrt_acc: every x below 2^16, random x at every magnitude, and x
  // next to the two decision boundaries (c^2 x and (c + 1/2)^2 x near 2^64)
  std::vector<int64_t> xs;
  for (int64_t x = 0; x < (1 << 16); ++x) xs.push_back(x);
  for (long i = 0; i < N; ++i) xs.push_back(int64_t(rng() >> 1) >> (rng() % 63));
  // x next to the floor boundary c^2 x = 2^64 and the rounding boundary
  // (2 c^2 + 2 c + 1) x = 2^65, for c at every magnitude
  for (long i = 0; i < N / 5; ++i) {
    const uint64_t c = 1 + (rng() >> (33 + rng() % 31)) % ((1ull << 31) - 2);
    const unsigned __int128 den = (rng() & 1) ? (unsigned __int128)c * c : 2 * (unsigned __int128)c * c + 2 * c + 1;
    const unsigned __int128 num = (rng() & 1) && den != (unsigned __int128)c * c ? ((unsigned __int128)1 << 65)
                                                                                : ((unsigned __int128)1 << 64);
    const unsigned __int128 x0 = num / den;
    for (int dx = -2; dx <= 2; ++dx) {
      const unsigned __int128 x = x0 + dx;
      if (x0 + 2 >= 2 && x < ((unsigned __int128)1 << 63)) xs.push_back(int64_t(x));
    }
  }
  {
    int64_t* dx = to_dev(xs);
    int32_t* dout = nullptr;
    CK(hipMalloc(&dout, xs.size() * 4));
    hipLaunchKernelGGL(k_inv_sqrt, dim3(unsigned((xs.size() + 255) / 256)), dim3(256), 0, 0, dx, dout, uint64_t(xs.size()));
    CK(hipGetLastError());
    std::vector<int32_t> got(xs.size());
    CK(hipMemcpy(got.data(), dout, xs.size() * 4, hipMemcpyDeviceToHost));
    long bad = 0;
    for (size_t i = 0; i < xs.size(); ++i) {
      int32_t o;
      orc_inv_sqrt_acc(xs[i], &o);
      if (got[i] != o && ++bad < 5) printf("  inv_sqrt x=%lld gpu=%d orc=%d\n", (long long)xs[i], got[i], o);
    }
    printf("gpu_inv_sqrt_acc %zu %ld\n", xs.size(), bad);
    failures += bad != 0;
    CK(hipFree(dx));
    CK(hipFree(dout));
  }
  // div_rte_nonneg_u32: random v and d at every magnitude, exact multiples,
  // halves (ties) and their neighbours
  {
    std::vector<int64_t> vs;
    std::vector<uint32_t> ds;
    for (long i = 0; i < N; ++i) {
      uint32_t d = uint32_t(rng() >> (32 + rng() % 32));
      if (d == 0) d = 1;
      const int kind = int(rng() % 4);
      uint64_t v = (rng() >> 1) >> (rng() % 63);
      if (kind >= 2) {
        const uint64_t q = v / d;
        v = q * d + (kind == 3 ? d / 2 : 0) + (rng() % 3) - 1;
        if (v >> 63) v = (rng() >> 1);
      }
      vs.push_back(int64_t(v));
      ds.push_back(d);
    }
    vs.push_back(INT64_MAX); ds.push_back(1);
    vs.push_back(INT64_MAX); ds.push_back(2);
    vs.push_back(INT64_MAX); ds.push_back(0xffffffffu);
    vs.push_back(0); ds.push_back(7);
    int64_t* dv = to_dev(vs);
    uint32_t* dd = to_dev(ds);
    int64_t* dout = nullptr;
    CK(hipMalloc(&dout, vs.size() * 8));
    hipLaunchKernelGGL(k_div, dim3(unsigned((vs.size() + 255) / 256)), dim3(256), 0, 0, dv, dd, dout, uint64_t(vs.size()));
    CK(hipGetLastError());
    std::vector<int64_t> got(vs.size());
    CK(hipMemcpy(got.data(), dout, vs.size() * 8, hipMemcpyDeviceToHost));
    long bad = 0;
    for (size_t i = 0; i < vs.size(); ++i) {
      int64_t o;
      orc_div_acc_by_u32(vs[i], ds[i], &o);
      if (got[i] != o && ++bad < 5) printf("  div v=%lld d=%u gpu=%lld orc=%lld\n", (long long)vs[i], ds[i], (long long)got[i], (long long)o);
    }
    printf("gpu_div_rte_nonneg_u32 %zu %ld\n", vs.size(), bad);
    failures += bad != 0;
    CK(hipFree(dv));
    CK(hipFree(dd));
    CK(hipFree(dout));
  }
  // rms_scale_from_sumsq on sums of squares of random rows (as the norms see them)
  {
    const long M = N / 20;
    std::vector<int64_t> ss(M), eps(M);
    std::vector<uint32_t> cnt(M);
    std::vector<int32_t> want(M);
    for (long i = 0; i < M; ++i) {
      const uint32_t n = 1 + rng() % 3000;
      std::vector<int32_t> x(n);
      const int sh = rng() % 31;
      for (auto& v : x) v = int32_t(rng()) >> sh;
      eps[i] = (rng() % 3 == 0) ? 0 : int64_t(rng() % (1ull << 40));
      int64_t s = 0;
      for (auto v : x) s = det::add_sat64(s, det::sq_term(v));
      ss[i] = s;
      cnt[i] = n;
      orc_rms_norm_scale(x.data(), n, eps[i], &want[i]);
    }
    int64_t* dss = to_dev(ss);
    int64_t* deps = to_dev(eps);
    uint32_t* dcnt = to_dev(cnt);
    int32_t* dout = nullptr;
    CK(hipMalloc(&dout, M * 4));
    hipLaunchKernelGGL(k_rms_scale, dim3(unsigned((M + 255) / 256)), dim3(256), 0, 0, dss, dcnt, deps, dout, uint64_t(M));
    CK(hipGetLastError());
    std::vector<int32_t> got(M);
    CK(hipMemcpy(got.data(), dout, M * 4, hipMemcpyDeviceToHost));
    long bad = 0;
    for (long i = 0; i < M; ++i)
      if (got[i] != want[i] && ++bad < 5) printf("  rms_scale ss=%lld n=%u gpu=%d orc=%d\n", (long long)ss[i], cnt[i], got[i], want[i]);
    printf("gpu_rms_scale %ld %ld\n", M, bad);
    failures += bad != 0;
  }
  // requant (Q32.32 -> Q16.16, ties to even, saturating): every magnitude, the
  // saturation edges +-2^47 with the rounding offsets around them, exact ties
  // with odd and even quotients, and the i64 extremes
  {
    std::vector<int64_t> xs;
    for (long i = 0; i < N; ++i) xs.push_back(int64_t(rng()) >> (rng() % 64));
    const int64_t edge = int64_t(1) << 47;
    for (int64_t base : {edge, -edge, int64_t(0), INT64_MAX, INT64_MIN, edge - 0x10000, -edge + 0x10000})
      for (int64_t d = -0x18000; d <= 0x18000; d += 0x100) {
        int64_t x;
        if (!__builtin_add_overflow(base, d, &x)) xs.push_back(x);
        for (int64_t e : {-1, 0, 1, 0x7fff, 0x8000, 0x8001})
          if (!__builtin_add_overflow(base, d + e, &x)) xs.push_back(x);
      }
    for (long i = 0; i < N / 10; ++i) {  // ties
      const int64_t q = int64_t(rng()) >> (17 + rng() % 40);
      xs.push_back(q * 65536 + 0x8000);
    }
    int64_t* dx = to_dev(xs);
    int32_t* dout = nullptr;
    CK(hipMalloc(&dout, xs.size() * 4));
    hipLaunchKernelGGL(k_requant, dim3(unsigned((xs.size() + 255) / 256)), dim3(256), 0, 0, dx, dout, uint64_t(xs.size()));
    CK(hipGetLastError());
    std::vector<int32_t> got(xs.size());
    CK(hipMemcpy(got.data(), dout, xs.size() * 4, hipMemcpyDeviceToHost));
    long bad = 0;
    for (size_t i = 0; i < xs.size(); ++i) {
      const int32_t o = orc_requantize(xs[i]);
      if (got[i] != o && ++bad < 5) printf("  requant x=%lld gpu=%d orc=%d\n", (long long)xs[i], got[i], o);
    }
    printf("gpu_requant %zu %ld\n", xs.size(), bad);
    failures += bad != 0;
    CK(hipFree(dx));
    CK(hipFree(dout));
  }
  // mul_sat / add_sat / sub_sat: random operands at every magnitude, the
  // extremes, products next to the saturation edges and exact ties
  {
    std::vector<int32_t> as, bs;
    const int32_t ext[] = {INT32_MIN, INT32_MIN + 1, -65536, -1, 0, 1, 65536, INT32_MAX - 1, INT32_MAX};
    for (int32_t a : ext)
      for (int32_t b : ext) as.push_back(a), bs.push_back(b);
    for (long i = 0; i < N; ++i) {
      as.push_back(int32_t(rng()) >> (rng() % 32));
      bs.push_back(int32_t(rng()) >> (rng() % 32));
    }
    for (long i = 0; i < N / 4; ++i) {  // a b next to +-2^47 and +-2^47 - 2^15
      int32_t a = int32_t(rng()) >> (rng() % 31);
      if (a == 0) a = 3;
      const int64_t t = ((rng() & 1) ? 1 : -1) * ((int64_t(1) << 47) - ((rng() & 1) ? 0x8000 : 0));
      const int64_t b0 = t / a;
      for (int64_t db = -2; db <= 2; ++db) {
        const int64_t b = b0 + db;
        if (b >= INT32_MIN && b <= INT32_MAX) as.push_back(a), bs.push_back(int32_t(b));
      }
    }
    for (long i = 0; i < N / 10; ++i) {  // exact ties: a b = q 2^16 + 2^15 with a = 2^k
      const int k = int(rng() % 16);
      as.push_back(int32_t(1) << k);
      bs.push_back(int32_t((int32_t(rng()) >> (rng() % 20)) | (1 << (15 - k))) & ~((1 << (15 - k)) - 1));
    }
    int32_t* da = to_dev(as);
    int32_t* db = to_dev(bs);
    int32_t* dout = nullptr;
    CK(hipMalloc(&dout, as.size() * 4));
    const char* names[] = {"gpu_mul_sat", "gpu_add_sat", "gpu_sub_sat"};
    for (int op = 0; op < 3; ++op) {
      hipLaunchKernelGGL(k_binop, dim3(unsigned((as.size() + 255) / 256)), dim3(256), 0, 0, da, db, op, dout,
                         uint64_t(as.size()));
      CK(hipGetLastError());
      std::vector<int32_t> got(as.size());
      CK(hipMemcpy(got.data(), dout, as.size() * 4, hipMemcpyDeviceToHost));
      long bad = 0;
      for (size_t i = 0; i < as.size(); ++i) {
        const int32_t o = op == 0 ? orc_mul_sat(as[i], bs[i]) : (op == 1 ? orc_add_sat(as[i], bs[i]) : orc_sub_sat(as[i], bs[i]));
        if (got[i] != o && ++bad < 5) printf("  %s a=%d b=%d gpu=%d orc=%d\n", names[op], as[i], bs[i], got[i], o);
      }
      printf("%s %zu %ld\n", names[op], as.size(), bad);
      failures += bad != 0;
    }
    CK(hipFree(da));
    CK(hipFree(db));
    CK(hipFree(dout));
  }
  // add_sat64_nn: non-negative operands at every magnitude and around i64::MAX
  {
    std::vector<int64_t> as, bs;
    for (long i = 0; i < N; ++i) {
      as.push_back(int64_t(rng() >> 1) >> (rng() % 63));
      bs.push_back(int64_t(rng() >> 1) >> (rng() % 63));
    }
    for (int64_t a : {int64_t(0), int64_t(1), INT64_MAX, INT64_MAX - 1, INT64_MAX / 2, INT64_MAX / 2 + 1, int64_t(1) << 62})
      for (int64_t b : {int64_t(0), int64_t(1), INT64_MAX, INT64_MAX / 2, INT64_MAX / 2 + 1, int64_t(1) << 62})
        as.push_back(a), bs.push_back(b);
    int64_t* da = to_dev(as);
    int64_t* db = to_dev(bs);
    int64_t* dout = nullptr;
    CK(hipMalloc(&dout, as.size() * 8));
    hipLaunchKernelGGL(k_add_sat64_nn, dim3(unsigned((as.size() + 255) / 256)), dim3(256), 0, 0, da, db, dout,
                       uint64_t(as.size()));
    CK(hipGetLastError());
    std::vector<int64_t> got(as.size());
    CK(hipMemcpy(got.data(), dout, as.size() * 8, hipMemcpyDeviceToHost));
    long bad = 0;
    for (size_t i = 0; i < as.size(); ++i) {
      const int64_t o = orc_acc_add_sat(as[i], bs[i]);
      if (got[i] != o && ++bad < 5) printf("  add_sat64_nn a=%lld b=%lld gpu=%lld orc=%lld\n", (long long)as[i], (long long)bs[i], (long long)got[i], (long long)o);
    }
    printf("gpu_add_sat64_nn %zu %ld\n", as.size(), bad);
    failures += bad != 0;
    CK(hipFree(da));
    CK(hipFree(db));
    CK(hipFree(dout));
  }
  return failures ? 1 : 0;
}
