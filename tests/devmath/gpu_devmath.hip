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
  return failures ? 1 : 0;
}
