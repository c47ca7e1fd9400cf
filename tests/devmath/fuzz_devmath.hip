// Test-only fuzz driver: compares the product's integer arithmetic
// (det_arith.h, built for the host) with the oracle's restatement of
// det_num/ops.rs on random and edge-case inputs. Prints one line per function
// ("name checked mismatches") and exits non-zero on any mismatch.
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "../../oracle/oracle.h"
#include "../../raster-inference_amd/csrc/det_arith.h"

static std::mt19937_64 rng(12345);
static int64_t r64() { return int64_t(rng()); }
static int32_t r32() { return int32_t(rng()); }
static int64_t pick64() {
  static const int64_t edges[] = {0, 1, -1, INT64_MAX, INT64_MIN, INT64_MAX - 1, INT64_MIN + 1, 1ll << 32, -(1ll << 32),
                                  0x8000, -0x8000, 0x18000, -0x18000, (1ll << 47), -(1ll << 47)};
  switch (rng() % 4) {
    case 0: return edges[rng() % (sizeof(edges) / 8)];
    case 1: return r64() >> (rng() % 63);
    default: return r64();
  }
}
static int32_t pick32() {
  static const int32_t edges[] = {0, 1, -1, INT32_MAX, INT32_MIN, 65536, -65536, 32768, -32768, 3 << 16, -(3 << 16)};
  switch (rng() % 4) {
    case 0: return edges[rng() % (sizeof(edges) / 4)];
    case 1: return r32() >> (rng() % 31);
    default: return r32();
  }
}

int failures = 0;
static void report(const char* name, long n, long bad) {
  printf("%s %ld %ld\n", name, n, bad);
  if (bad) failures++;
}

int main(int argc, char** argv) {
  const long N = argc > 1 ? atol(argv[1]) : 200000;
  long bad;
  bad = 0; for (long i = 0; i < N; ++i) { int64_t x = pick64(); if (det::requant(x) != orc_requantize(x)) bad++; } report("requant", N, bad);
  bad = 0; for (long i = 0; i < N; ++i) { int32_t a = pick32(), b = pick32(); if (det::mul_sat(a, b) != orc_mul_sat(a, b)) bad++; } report("mul_sat", N, bad);
  bad = 0; for (long i = 0; i < N; ++i) { int64_t a = pick64(), b = pick64(); if (a < 0) a = -(a + 1); if (b < 0) b = -(b + 1); if (det::add_sat64_nn(a, b) != orc_acc_add_sat(a, b)) bad++; } report("add_sat64_nn", N, bad);
  bad = 0; for (long i = 0; i < N; ++i) { int32_t a = pick32(), b = pick32(); if (!b) continue; int32_t o; orc_div_act(a, b, &o); if (det::div_act(a, b) != o) bad++; } report("div_act", N, bad);
  bad = 0; for (long i = 0; i < N; ++i) { int64_t v = pick64(); uint32_t d = uint32_t(rng()) >> (rng() % 32); if (!d) d = 1; int64_t o; orc_div_acc_by_u32(v, d, &o); if (det::div_acc_u32(v, d) != o) bad++; } report("div_acc_u32", N, bad);
  bad = 0; for (long i = 0; i < N; ++i) { int64_t a = pick64(), b = pick64(); if (det::acc_mul(a, b) != orc_acc_mul(a, b)) bad++; } report("acc_mul", N, bad);
  bad = 0; for (long i = 0; i < N; ++i) { int64_t x = pick64(); if (x < 0) x = -(x + 1); int32_t o; orc_inv_sqrt_acc(x, &o); if (det::inv_sqrt_acc(x) != o) { bad++; if (bad < 5) printf("  inv_sqrt x=%lld dev=%d orc=%d\n", (long long)x, det::inv_sqrt_acc(x), o); } } report("inv_sqrt_acc", N, bad);
  // inv_sqrt_acc near the rounding boundaries: x where c^2 x or (c+1/2)^2 x
  // sits next to 2^64, for random c, plus every x below 2^16.
  bad = 0;
  long nis = 0;
  for (int64_t x = 0; x < (1 << 16); ++x, ++nis) { int32_t o; orc_inv_sqrt_acc(x, &o); if (det::inv_sqrt_acc(x) != o) bad++; }
  for (long i = 0; i < N; ++i) {
    const uint64_t c = 2 + rng() % ((1ull << 31) - 3);
    const long double target = 18446744073709551616.0L;
    const long double cc = (rng() & 1) ? (long double)c * c : ((long double)c + 0.5L) * ((long double)c + 0.5L);
    const int64_t x0 = int64_t(target / cc);
    for (int64_t dx = -2; dx <= 2; ++dx, ++nis) {
      const int64_t x = x0 + dx;
      if (x < 0) continue;
      int32_t o;
      orc_inv_sqrt_acc(x, &o);
      if (det::inv_sqrt_acc(x) != o) { bad++; if (bad < 5) printf("  inv_sqrt_edge x=%lld dev=%d orc=%d\n", (long long)x, det::inv_sqrt_acc(x), o); }
    }
  }
  report("inv_sqrt_acc_edges", nis, bad);
  // softmax_exp over every max-shift gap that yields a non-zero term (and past it).
  bad = 0;
  long nexp = 0;
  for (int64_t d = 0; d < (1 << 20) + 64; ++d, ++nexp) {
    const int32_t m = int32_t(rng() % 2000000) - 1000000;
    const int32_t l = int32_t(int64_t(m) - d);
    int64_t o;
    orc_attention_softmax_exp_term(l, m, &o);
    if (det::softmax_exp(l, m) != o) { bad++; if (bad < 5) printf("  softmax_exp d=%lld dev=%lld orc=%lld\n", (long long)d, (long long)det::softmax_exp(l, m), (long long)o); }
    // the decode kernel encodes the d == 0 term 2^32 as 0xffffffff in 32 bits: no other term may reach it
    if (d > 0 && o > int64_t((1ull << 32) - (1ull << 16))) bad++;
  }
  report("softmax_exp_all_gaps", nexp, bad);
  // softmax_weight at exact half-way quotients and near the 2^61 sum boundary.
  bad = 0;
  long nw = 0;
  for (long i = 0; i < N; ++i, ++nw) {
    const uint64_t sum = (1ull << 32) + (rng() % (1ull << (20 + rng() % 40)));
    uint64_t e;
    switch (i % 4) {
      case 0: { const uint64_t q = rng() % (1ull << 32); e = uint64_t(((unsigned __int128)q * sum * 2 + sum) / ((unsigned __int128)1 << 33)); break; }
      case 1: e = sum < (1ull << 32) ? sum : (1ull << 32); break;
      case 2: e = rng() % ((1ull << 32) + 1); break;
      default: e = 1 + rng() % 1024; break;
    }
    if (e > sum) e = sum;
    const uint64_t s2 = (i % 7 == 0) ? (1ull << 61) - 1 - rng() % 3 : ((i % 11 == 0) ? (1ull << 61) + rng() % 3 : sum);
    int64_t q;
    orc_div_acc(int64_t(e), int64_t(s2), &q);
    if (det::softmax_weight(int64_t(e), int64_t(s2)) != orc_requantize(q)) bad++;
  }
  report("softmax_weight_edges", nw, bad);
  // reciprocal-based softmax weight (per-head M) on the same kinds of inputs
  bad = 0;
  nw = 0;
  for (long i = 0; i < N; ++i, ++nw) {
    uint64_t sum = (1ull << 32) + (rng() % (1ull << (rng() % 29)));
    if (i % 5 == 0) sum = (1ull << 32);
    if (i % 7 == 0) sum = (1ull << 61) - 1 - rng() % 1000;
    uint64_t e;
    switch (i % 4) {
      case 0: { const uint64_t q = rng() % (1ull << 32); e = uint64_t(((unsigned __int128)q * sum * 2 + sum) / ((unsigned __int128)1 << 33)); break; }
      case 1: e = 1ull << 32; break;
      case 2: e = rng() % ((1ull << 32) + 1); break;
      default: e = 1 + rng() % 1024; break;
    }
    if (e > sum) e = sum;
    int64_t q;
    orc_div_acc(int64_t(e), int64_t(sum), &q);
    const int32_t w = det::softmax_weight_r(int64_t(e), int64_t(sum), det::softmax_recip(int64_t(sum)));
    if (w != orc_requantize(q)) { bad++; if (bad < 5) printf("  weight_r e=%llu s=%llu dev=%d orc=%d\n", (unsigned long long)e, (unsigned long long)sum, w, orc_requantize(q)); }
  }
  report("softmax_weight_recip", nw, bad);
  // round-half-even division of non-negative values (row-norm means)
  bad = 0;
  for (long i = 0; i < N; ++i) {
    int64_t v = pick64();
    if (v < 0) v = v == INT64_MIN ? INT64_MAX : -v;
    uint32_t d = uint32_t(rng()) >> (rng() % 32);
    if (!d) d = 1;
    if (i % 3 == 0) { const uint64_t q = rng() >> (rng() % 64); d = 1 + uint32_t(rng() % 5000); v = int64_t((q % (uint64_t(INT64_MAX) / d)) * d + d / 2); }
    int64_t o;
    orc_div_acc_by_u32(v, d, &o);
    if (int64_t(det::div_rte_nonneg_u32(uint64_t(v), d)) != o) bad++;
  }
  report("div_rte_nonneg", N, bad);
  bad = 0;
  for (long i = 0; i < N / 20; ++i) {
    const uint32_t n = 1 + rng() % 300;
    std::vector<int32_t> x(n);
    const int sh = rng() % 31;
    for (auto& v : x) v = r32() >> sh;
    const int64_t eps = (rng() % 3 == 0) ? 0 : int64_t(rng() % (1ull << 40));
    int64_t ss = 0;
    for (auto v : x) ss = det::add_sat64(ss, det::sq_term(v));
    int32_t o;
    orc_rms_norm_scale(x.data(), n, eps, &o);
    if (det::rms_scale_from_sumsq(ss, n, eps) != o) bad++;
  }
  report("rms_scale", N / 20, bad);
  bad = 0; for (long i = 0; i < N; ++i) { int32_t m = pick32(), l = pick32(); if (l > m) std::swap(l, m); int64_t o; orc_attention_softmax_exp_term(l, m, &o); if (det::softmax_exp(l, m) != o) bad++; } report("softmax_exp", N, bad);
  bad = 0;
  for (long i = 0; i < N; ++i) {
    int64_t sum = int64_t(rng() % (1ull << 50)) + (1ll << 32);
    if (rng() % 8 == 0) sum = INT64_MAX;
    int64_t e = int64_t(rng() % ((1ull << 32) + 1));
    if (rng() % 16 == 0) e = 1ll << 32;
    if (e > sum) e = sum;
    int64_t q;
    orc_div_acc(e, sum, &q);
    if (det::softmax_weight(e, sum) != orc_requantize(q)) bad++;
  }
  report("softmax_weight", N, bad);
  bad = 0; for (long i = 0; i < N; ++i) { int32_t x = pick32(); if (det::tanh_act(x) != orc_tanh_act(x)) bad++; } report("tanh", N, bad);
  bad = 0; for (long i = 0; i < N; ++i) { int32_t x = pick32(); if (det::gelu_act(x) != orc_gelu_pytorch_tanh_act(x)) bad++; } report("gelu", N, bad);
  bad = 0; for (long i = 0; i < N; ++i) { int32_t x = pick32(), c = pick32(); if (c <= 0) c = c == INT32_MIN ? 1 : -c; if (!c) c = 1; int32_t o; orc_softcap_act(x, c, &o); if (det::softcap_act(x, c) != o) bad++; } report("softcap", N, bad);
  bad = 0; for (long i = 0; i < N; ++i) { int64_t a = pick64(); int32_t c1, s1, c2, s2; det::sin_cos(a, &c1, &s1); orc_sin_cos_acc(a, &c2, &s2); if (c1 != c2 || s1 != s2) bad++; } report("sin_cos", N, bad);
  // RoPE: rotate with the table-driven product form vs the oracle's row rotation.
  bad = 0;
  long nrope = 0;
  const int64_t bases[] = {10000ll << 32, 1000000ll << 32, 16ll << 32, 12345ll << 32, int64_t(3.5 * 4294967296.0)};
  const uint32_t dims[] = {2, 4, 16, 64, 256};
  for (int64_t base : bases)
    for (uint32_t hd : dims)
      for (uint32_t rot : {hd, hd / 2 - (hd / 2) % 2, uint32_t(hd / 4 - (hd / 4) % 2)}) {
        if (rot == 0 || rot > hd) continue;
        std::vector<int64_t> tab(rot / 2);
        det::rope_inv_freq_table(base, hd, rot / 2, tab.data());
        for (uint64_t pos : {uint64_t(0), uint64_t(1), uint64_t(7), uint64_t(511), uint64_t(4096), uint64_t(1) << 20}) {
          std::vector<int32_t> x(hd), y;
          for (auto& v : x) v = r32() >> (8 + rng() % 12);
          y = x;
          orc_rope_rotate_pairs(y.data(), hd, rot, hd, base, pos);
          if (pos) for (uint32_t i = 0; i < rot / 2; ++i) {
            int32_t c, s;
            det::sin_cos(det::rope_angle(pos, tab[i]), &c, &s);
            const int32_t l = x[i], r = x[i + rot / 2];
            x[i] = det::sub_sat(det::mul_sat(l, c), det::mul_sat(r, s));
            x[i + rot / 2] = det::add_sat(det::mul_sat(r, c), det::mul_sat(l, s));
          }
          ++nrope;
          if (x != y) bad++;
        }
      }
  report("rope", nrope, bad);
  bad = 0;
  for (long i = 0; i < N; ++i) {
    uint32_t b = uint32_t(rng());
    float f; memcpy(&f, &b, 4);
    if (!std::isfinite(f)) continue;
    int32_t oa; int64_t oc;
    orc_f32_to_act(f, &oa); orc_f32_to_acc(f, &oc);
    if (det::f32_to_act(f) != oa || det::f32_to_acc(f) != oc) bad++;
  }
  report("f32_to_fixed", N, bad);
  return failures ? 1 : 0;
}
