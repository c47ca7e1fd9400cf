// Canonical Q16.16 / Q32.32 integer arithmetic for the MI355X det path.
//
// Every function here is __host__ __device__ and computes exactly the value
// the reference's det_num contract defines (src/shared/numerics/det_num/ops.rs),
// but in forms that suit 64-wide wavefronts: floor-based round-half-even
// shifts, 64-bit divisions by small constants, one 64x64->128 multiply where
// the reference uses i128, and exact-correction steps instead of 31-step
// binary searches. No 128-bit division is ever emitted (gfx950 has no
// library routine for it).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define DET_HD __host__ __device__ __forceinline__

namespace det {

constexpr int32_t kOneAct = 1 << 16;
constexpr int64_t kOneAcc = int64_t(1) << 32;

typedef __int128 i128;
typedef unsigned __int128 u128;

DET_HD int32_t sat32(int64_t v) {
  return v > INT32_MAX ? INT32_MAX : (v < INT32_MIN ? INT32_MIN : int32_t(v));
}
// (on the GPU: the clamping 32-bit add and subtract)
DET_HD int32_t add_sat(int32_t a, int32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_elementwise_add_sat(a, b);
#else
  return sat32(int64_t(a) + int64_t(b));
#endif
}
DET_HD int32_t sub_sat(int32_t a, int32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_elementwise_sub_sat(a, b);
#else
  return sat32(int64_t(a) - int64_t(b));
#endif
}
DET_HD int32_t neg_sat32(int32_t a) { return a == INT32_MIN ? INT32_MAX : -a; }
DET_HD int64_t neg_sat64(int64_t a) { return a == INT64_MIN ? INT64_MAX : -a; }
DET_HD int64_t add_sat64(int64_t a, int64_t b) {
  int64_t r;
  if (__builtin_add_overflow(a, b, &r)) return a < 0 ? INT64_MIN : INT64_MAX;
  return r;
}
// add_sat64 for a, b >= 0: the unsigned sum stays below 2^64, and a set top
// bit (a sum past i64::MAX) turns the result into i64::MAX.
DET_HD int64_t add_sat64_nn(int64_t a, int64_t b) {
  const uint64_t s = uint64_t(a) + uint64_t(b);
  const uint32_t m = uint32_t(int32_t(uint32_t(s >> 32)) >> 31);  // all ones past i64::MAX
  const uint32_t lo = uint32_t(s) | m, hi = (uint32_t(s >> 32) | m) & 0x7fffffffu;
  return int64_t((uint64_t(hi) << 32) | lo);
}
// Wrapping i64 MAC (ops.rs:14-16).
DET_HD int64_t mac(int64_t acc, int32_t a, int32_t w) {
  return int64_t(uint64_t(acc) + uint64_t(int64_t(a) * int64_t(w)));
}

// Round x / 2^s to nearest, ties to even, for 1 <= s <= 63 (ops.rs:770-800).
// Floor quotient + remainder: identical to the reference's truncate-and-step.
DET_HD int64_t rshift_rte(int64_t x, unsigned s) {
  if (s == 0) return x;
  const int64_t q = x >> s;  // arithmetic: floor
  const uint64_t r = uint64_t(x) & ((uint64_t(1) << s) - 1);
  const uint64_t half = uint64_t(1) << (s - 1);
  return q + int64_t((r > half) | ((r == half) & uint64_t(q & 1)));
}

// requantize: Q32.32 -> Q16.16, ties to even, saturating (ops.rs:445-448).
// On the GPU in 32-bit halves: with b = bit 16 of x (the low bit of the floor
// quotient q), floor((x + 0x7fff + b) / 2^16) is q rounded half to even. For
// x in [-2^47, 2^47) (high word in [-2^15, 2^15)) the sum y does not wrap and
// the quotient is y's bits 16..47, exact when y's high word is in range as
// well; every other x saturates with its sign.
DET_HD int32_t requant(int64_t acc) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint32_t xl = uint32_t(uint64_t(acc)), xh = uint32_t(uint64_t(acc) >> 32);
  const uint64_t y = uint64_t(acc) + (0x7fffu + ((xl >> 16) & 1u));
  const uint32_t yl = uint32_t(y), yh = uint32_t(y >> 32);
  const int32_t q = int32_t(__builtin_amdgcn_alignbit(yh, yl, 16));
  const bool ok = (xh + 0x8000u < 0x10000u) & (yh + 0x8000u < 0x10000u);
  return ok ? q : int32_t((uint32_t(int32_t(xh) >> 31)) ^ 0x7fffffffu);
#else
  return sat32(rshift_rte(acc, 16));
#endif
}
// |a b| <= 2^62, so the rounding sum of requant never wraps and the range
// test needs y's high word only.
DET_HD int32_t mul_sat(int32_t a, int32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  const uint64_t p = uint64_t(int64_t(a) * int64_t(b));
  const uint64_t y = p + (0x7fffu + ((uint32_t(p) >> 16) & 1u));
  const uint32_t yl = uint32_t(y), yh = uint32_t(y >> 32);
  const int32_t q = int32_t(__builtin_amdgcn_alignbit(yh, yl, 16));
  return yh + 0x8000u < 0x10000u ? q : int32_t((uint32_t(int32_t(yh) >> 31)) ^ 0x7fffffffu);
#else
  return requant(int64_t(a) * int64_t(b));
#endif
}

// Round |n| / d to nearest with ties to even on the magnitude, sign restored
// (the reference's round_ties_even_division for |quotient| < 2^63).
DET_HD uint64_t udiv_rte(uint64_t n, uint64_t d) {
  const uint64_t q = n / d, r = n - q * d;
  const uint64_t rem_twice_hi = r >> 63;  // r < d <= 2^64-1; 2r may overflow
  const uint64_t twice = r << 1;
  const bool gt = rem_twice_hi || twice > d;
  const bool eq = !rem_twice_hi && twice == d;
  return (gt || (eq && (q & 1))) ? q + 1 : q;
}

// div_acc_by_u32 (ops.rs:78-85).
DET_HD int64_t div_acc_u32(int64_t v, uint32_t d) {
  const bool neg = v < 0;
  const uint64_t mag = neg ? uint64_t(0) - uint64_t(v) : uint64_t(v);
  const uint64_t q = udiv_rte(mag, d);
  return neg ? int64_t(uint64_t(0) - q) : int64_t(q);
}

// div_act (ops.rs:50-61): round(n * 2^16 / d) ties to even on the magnitude,
// saturating to i32; d != 0. |n 2^16| < 2^47 and |d| < 2^32 are exact doubles,
// so the double quotient is within one of the floor quotient; quotients of
// 2^31 + 2 or more saturate whatever the rounding; below that the exact
// remainder (products below 2^64) fixes and rounds the estimate.
DET_HD int32_t div_act(int32_t n, int32_t d) {
  const int64_t num = int64_t(n) * 65536;
  const bool neg = (num < 0) != (d < 0);
  const uint64_t un = num < 0 ? uint64_t(-num) : uint64_t(num);
  const uint64_t ud = d < 0 ? uint64_t(-int64_t(d)) : uint64_t(d);
  const double qd = double(un) / double(ud);
  if (qd >= 2147483650.0) return neg ? INT32_MIN : INT32_MAX;
  uint64_t q = uint64_t(qd);
  int64_t r = int64_t(un - q * ud);
  if (r < 0) {
    --q;
    r += int64_t(ud);
  } else if (r >= int64_t(ud)) {
    ++q;
    r -= int64_t(ud);
  }
  const uint64_t twice = uint64_t(r) << 1;
  q += uint64_t((twice > ud) | ((twice == ud) & (q & 1)));
  return sat32(neg ? -int64_t(q) : int64_t(q));
}

// acc_mul (ops.rs:682-686): round(lhs * rhs / 2^32), saturating to i64.
DET_HD int64_t acc_mul(int64_t lhs, int64_t rhs) {
  const i128 p = i128(lhs) * i128(rhs);
  const i128 q = p >> 32;  // floor
  const uint64_t r = uint64_t(p) & 0xffffffffull;
  const i128 rq = (r > 0x80000000ull || (r == 0x80000000ull && (int64_t(q) & 1))) ? q + 1 : q;
  if (rq > i128(INT64_MAX)) return INT64_MAX;
  if (rq < i128(INT64_MIN)) return INT64_MIN;
  return int64_t(rq);
}

// inv_sqrt_acc (ops.rs:719-763): the c in [0, 2^31-1] nearest to
// 2^32/sqrt(x) in the sense |c^2 x - 2^64| minimal, ties to even; x == 0 and
// tiny x saturate to i32::MAX.
// For x >= 5 the lower candidate lo = max{c : c^2 x <= 2^64} is below
// 2^31 - 1. An estimate of 2^32/sqrt(x) is moved to lo one step at a time
// with the exact test on the 128-bit product c^2 x, so lo is exact whatever
// the estimate's error (the double estimate is within one of it). Then
// |lo^2 x - 2^64| vs |hi^2 x - 2^64| (hi = lo + 1) is the sign of
// 2^65 - (lo^2 + hi^2) x, again one exact 128-bit product. On the GPU the
// 128-bit products are a 64-bit multiply and multiply-high, and the estimate
// is the hardware reciprocal square root refined by one Newton step.
DET_HD void mul_64x64(uint64_t a, uint64_t b, uint64_t* hi, uint64_t* lo) {
#if defined(__HIP_DEVICE_COMPILE__)
  *hi = __umul64hi(a, b);
  *lo = a * b;
#else
  const u128 p = u128(a) * b;
  *hi = uint64_t(p >> 64);
  *lo = uint64_t(p);
#endif
}
DET_HD bool sq_times_le_2_64(uint64_t c, uint64_t x) {  // c^2 x <= 2^64, c < 2^31
  uint64_t hi, lo;
  mul_64x64(c * c, x, &hi, &lo);
  return hi == 0 || (hi == 1 && lo == 0);
}
DET_HD uint64_t inv_sqrt_estimate(uint64_t ux) {  // about 2^32 / sqrt(ux)
#if defined(__HIP_DEVICE_COMPILE__)
  const double xd = double(ux);
  double r = __builtin_amdgcn_rsq(xd);
  r = r * (1.5 - 0.5 * xd * r * r);
  return uint64_t(4294967296.0 * r);
#else
  return uint64_t(4294967296.0 / __builtin_sqrt(double(ux)));
#endif
}
DET_HD int32_t inv_sqrt_acc(int64_t x) {
  // (2^31-1)^2 * x <= 2^64 exactly for x <= 4
  if (x <= 4) return INT32_MAX;  // includes x == 0 (negative x is rejected upstream)
  const uint64_t ux = uint64_t(x);
#if defined(__HIP_DEVICE_COMPILE__)
  {
    // The result is lo = floor(Y), Y = 2^32 / sqrt(x), or lo + 1 when
    // Y > T = sqrt(lo^2 + lo + 1/2) (the exact rule below: (lo^2 + hi^2) x
    // against 2^65). Y = T is impossible: it needs x (2 lo^2 + 2 lo + 1) =
    // 2^65 with an odd factor above 1 (lo = 0 would need x = 2^65). The
    // estimate y (hardware rsq, two Newton steps; double x within 2^-53)
    // has relative error below 2^-49.5 and y < 2^31.5, so |y - Y| < 2^-18;
    // t is within 2^-20 of T. Both decisions are taken from y only when y
    // is more than 2^-14 from the integer and from t; otherwise the exact
    // integer search runs.
    const double xd = double(ux);
    double r = __builtin_amdgcn_rsq(xd);
    r = r * (1.5 - 0.5 * xd * r * r);
    r = r * (1.5 - 0.5 * xd * r * r);
    const double y = 4294967296.0 * r;
    const double fl = __builtin_floor(y);
    const double fr = y - fl;  // exact
    const double t = __builtin_sqrt(__builtin_fma(fl, fl, fl + 0.5));
    const double gap = y - t;
    const double m = 1.0 / 16384;
    if (fr > m && fr < 1.0 - m && (gap > m || gap < -m)) return int32_t(uint32_t(fl) + (gap > 0 ? 1u : 0u));
  }
#endif
  uint64_t lo = inv_sqrt_estimate(ux);
  if (lo > 2147483646ull) lo = 2147483646ull;
  while (lo > 0 && !sq_times_le_2_64(lo, ux)) --lo;
  while (sq_times_le_2_64(lo + 1, ux)) ++lo;
  const uint64_t hi = lo + 1;
  uint64_t ph, pl;  // (lo^2 + hi^2) x against 2^65 = (2, 0); lo^2 + hi^2 < 2^63
  mul_64x64(lo * lo + hi * hi, ux, &ph, &pl);
  if (ph == 2 && pl == 0) return int32_t((lo & 1) == 0 ? lo : hi);
  return int32_t(ph >= 2 ? lo : hi);
}

// Round-half-even quotient of a non-negative v < 2^63 by 1 <= d < 2^32
// (div_acc_by_u32, ops.rs:78-85, on the non-negative domain): a double
// estimate within two of the floor quotient for quotients below 2^51, then
// the exact remainder; larger quotients use the integer division.
DET_HD uint64_t div_rte_nonneg_u32(uint64_t v, uint32_t d) {
#if defined(__HIP_DEVICE_COMPILE__)
  // Branch-free on the GPU: rd = 1/d within 2^-51 (hardware rcp, two Newton
  // steps), so v rd is within 2^-50 relative of v / d < 2^63 and q0 =
  // trunc(v rd) within 2^13 + 1 of it; the exact remainder r = v - q0 d has
  // |r| < 2^46 (an exact double). r rd is within 2^-36 of r / d, whose
  // fractional part is 0 or at least 1/d > 2^-32, so trunc(r rd) leaves a
  // remainder in [-d, d] that one step each way brings into [0, d); then
  // round half to even.
  const double dd = double(d);
  double rd = __builtin_amdgcn_rcp(dd);
  rd = rd * (2.0 - dd * rd);
  rd = rd * (2.0 - dd * rd);
  uint64_t q = uint64_t(double(v) * rd);
  int64_t r = int64_t(v - q * uint64_t(d));
  const int64_t adj = int64_t(double(r) * rd);
  q += uint64_t(adj);
  r -= adj * int64_t(d);
  const bool neg = r < 0;
  q -= uint64_t(neg);
  r += neg ? int64_t(d) : 0;
  const bool big = r >= int64_t(d);
  q += uint64_t(big);
  r -= big ? int64_t(d) : 0;
  const uint64_t twice2 = uint64_t(r) << 1;
  return q + uint64_t((twice2 > d) | ((twice2 == d) & (q & 1)));
#else
  const double qd = double(v) / double(d);
  if (qd >= 2251799813685248.0) return udiv_rte(v, d);  // 2^51
  uint64_t q = uint64_t(qd);
  int64_t r = int64_t(v - q * d);
  while (r < 0) {
    --q;
    r += d;
  }
  while (r >= int64_t(d)) {
    ++q;
    r -= d;
  }
  const uint64_t twice = uint64_t(r) << 1;
  return (twice > d || (twice == d && (q & 1))) ? q + 1 : q;
#endif
}

// rms_norm_scale from a saturated sum of squares (ops.rs:406-425). The
// saturating sum of non-negative terms is min(true sum, i64::MAX) in any order.
DET_HD int32_t rms_scale_from_sumsq(int64_t sumsq, uint32_t n, int64_t eps) {
  const int64_t mean = int64_t(div_rte_nonneg_u32(uint64_t(sumsq), n));
  return inv_sqrt_acc(add_sat64(mean, eps));
}
DET_HD int64_t sq_term(int32_t v) { return int64_t(v) * int64_t(v); }

// Round-half-even quotient of a non-negative v < 2^32 by a constant d.
template <uint32_t d>
DET_HD uint32_t div_rte_u32(uint32_t v) {
  const uint32_t q = v / d, r2 = 2 * (v - q * d);
  return q + uint32_t((r2 > d) | ((r2 == d) & (q & 1)));
}
// acc_mul of two non-negative values below 2^32: the product fits in 64 bits
// and the rounded quotient stays below 2^32.
DET_HD uint32_t acc_mul_u32(uint32_t a, uint32_t b) {
  const uint64_t p = uint64_t(a) * b;
  const uint32_t q = uint32_t(p >> 32), r = uint32_t(p);
  return q + uint32_t((r > 0x80000000u) | ((r == 0x80000000u) & (q & 1)));
}

// softmax exp term of a max-shifted logit (ops.rs:505-553, 261-263),
// requires logit <= max_logit. With d = max_logit - logit the term is zero
// for d >= 2^20 (delta <= -16 in Q32.32); below that, pos = d * 2^16 < 2^36,
// the ln2 remainder r is below 2^32 and every power of r stays below 2^32, so
// the series runs in 32x32->64-bit products with the reference's rounding.
DET_HD int64_t softmax_exp(int32_t logit, int32_t max_logit) {
  const int64_t dd = int64_t(max_logit) - int64_t(logit);
  if (dd >= (int64_t(1) << 20)) return 0;
  const uint32_t d = uint32_t(dd);
  const int64_t LN2 = 2977044472ll;
  // shift = floor(d 2^16 / LN2) <= 23: a float estimate (relative error
  // below 2^-22, so at most one off) fixed by the remainder's range
  int32_t shift = int32_t(float(d) * (65536.0f / 2977044472.0f));
  int64_t r = (int64_t(d) << 16) - int64_t(shift) * LN2;
  const int32_t lo = r < 0, hi = r >= LN2;
  shift += hi - lo;
  r += int64_t(lo - hi) * LN2;
  const uint32_t r1 = uint32_t(r);
  const uint32_t r2 = acc_mul_u32(r1, r1);
  const uint32_t r3 = acc_mul_u32(r2, r1);
  const uint32_t r4 = acc_mul_u32(r3, r1);
  const uint32_t r5 = acc_mul_u32(r4, r1);
  const int64_t t = kOneAcc - int64_t(r1) + int64_t(div_rte_u32<2>(r2)) - int64_t(div_rte_u32<6>(r3)) +
                    int64_t(div_rte_u32<24>(r4)) - int64_t(div_rte_u32<120>(r5));
  if (t <= 0) return 0;
  return rshift_rte(t, unsigned(shift));  // shift <= 23 here
}

// Softmax raw weight: requantize(div_acc(exp, sum)) (ops.rs:266-268) for the
// softmax domain 0 <= exp <= min(sum, 2^32), sum > 0: round(exp * 2^32 / sum)
// ties to even, then requantize. A double estimate is within one of the floor
// quotient; the remainder e*2^32 - q*sum is exact in wrapping 64-bit
// arithmetic while |remainder| < 2^63, i.e. for sum < 2^61 (softmax over
// fewer than 2^29 rows). Larger sums take 128-bit remainders.
DET_HD int32_t softmax_weight(int64_t e, int64_t sum) {
  const uint64_t ue = uint64_t(e), d = uint64_t(sum);
  uint64_t q = uint64_t(double(e) * 4294967296.0 / double(sum));
  if (d < (uint64_t(1) << 61)) {
    int64_t rem = int64_t((ue << 32) - q * d);
    while (rem < 0) {
      --q;
      rem += int64_t(d);
    }
    while (rem >= int64_t(d)) {
      ++q;
      rem -= int64_t(d);
    }
    const uint64_t twice = uint64_t(rem) << 1;
    if (twice > d || (twice == d && (q & 1))) ++q;
    return requant(int64_t(q));
  }
  const u128 num = u128(ue) << 32;
  while (q > 0 && u128(q) * d > num) --q;
  while (u128(q + 1) * d <= num) ++q;
  const u128 rem = num - u128(q) * d;
  const u128 twice = rem << 1;
  if (twice > u128(d) || (twice == u128(d) && (q & 1))) ++q;
  return requant(int64_t(q));
}

// Reciprocal of a softmax exp sum S (2^32 <= S < 2^61) for softmax_weight_r:
// M = 2^96 / S truncated (relative error below 2^-32), capped at 2^64 - 1.
DET_HD uint64_t softmax_recip(int64_t sum) {
  const double m = 79228162514264337593543950336.0 / double(sum);  // 2^96 / S
  return m >= 18446744073709551615.0 ? UINT64_MAX : uint64_t(m);
}
// softmax_weight for 0 <= e <= min(S, 2^32), 2^32 <= S < 2^61 using M =
// softmax_recip(S): floor(e M / 2^64) is at most two below the floor
// quotient of e 2^32 / S; the exact remainder fixes it.
DET_HD int32_t softmax_weight_r(int64_t e, int64_t sum, uint64_t M) {
  const uint64_t ue = uint64_t(e), d = uint64_t(sum);
  uint64_t q = uint64_t((u128(ue) * M) >> 64);
  int64_t rem = int64_t((ue << 32) - q * d);
  while (rem < 0) {
    --q;
    rem += int64_t(d);
  }
  while (rem >= int64_t(d)) {
    ++q;
    rem -= int64_t(d);
  }
  const uint64_t twice = uint64_t(rem) << 1;
  if (twice > d || (twice == d && (q & 1))) ++q;
  return requant(int64_t(q));
}

// tanh_act (ops.rs:354-374), softcap_act (ops.rs:377-385),
// gelu_pytorch_tanh_act (ops.rs:388-403).
DET_HD int32_t tanh_act(int32_t x) {
  const int32_t LIN = 27 << 16, QUAD = 9 << 16, SAT = 3 << 16;
  if (x >= SAT) return kOneAct;
  if (x <= -SAT) return -kOneAct;
  const int32_t x2 = mul_sat(x, x);
  const int32_t num = mul_sat(x, add_sat(LIN, x2));
  const int32_t den = add_sat(LIN, mul_sat(QUAD, x2));
  return div_act(num, den);
}
DET_HD int32_t softcap_act(int32_t x, int32_t cap) { return mul_sat(cap, tanh_act(div_act(x, cap))); }
DET_HD int32_t gelu_act(int32_t x) {
  const int32_t x2 = mul_sat(x, x);
  const int32_t x3 = mul_sat(x2, x);
  const int32_t inner = add_sat(x, mul_sat(2930, x3));
  const int32_t t = tanh_act(mul_sat(52290, inner));
  return mul_sat(mul_sat(1 << 15, x), add_sat(kOneAct, t));
}

// sin/cos of a Q32.32 angle (ops.rs:619-680).
DET_HD int64_t sin_poly(int64_t x) {
  const int64_t x2 = acc_mul(x, x), x3 = acc_mul(x2, x), x5 = acc_mul(x3, x2), x7 = acc_mul(x5, x2);
  return add_sat64(add_sat64(x, neg_sat64(div_acc_u32(x3, 6))),
                   add_sat64(div_acc_u32(x5, 120), neg_sat64(div_acc_u32(x7, 5040))));
}
DET_HD int64_t cos_poly(int64_t x) {
  const int64_t x2 = acc_mul(x, x), x4 = acc_mul(x2, x2), x6 = acc_mul(x4, x2);
  return add_sat64(add_sat64(kOneAcc, neg_sat64(div_acc_u32(x2, 2))),
                   add_sat64(div_acc_u32(x4, 24), neg_sat64(div_acc_u32(x6, 720))));
}
DET_HD void sin_cos(int64_t angle, int32_t* c, int32_t* s) {
  const int64_t HALF_PI = 6746518852ll, PI = 13493037705ll, THREE_HALF_PI = 20239556557ll,
                TWO_PI = 26986075409ll;
  int64_t red = angle % TWO_PI;
  if (red < 0) red += TWO_PI;
  int64_t q;
  bool sneg, cneg;
  if (red <= HALF_PI) { q = red; sneg = false; cneg = false; }
  else if (red <= PI) { q = PI - red; sneg = false; cneg = true; }
  else if (red <= THREE_HALF_PI) { q = red - PI; sneg = true; cneg = true; }
  else { q = TWO_PI - red; sneg = true; cneg = false; }
  int32_t sv = requant(sin_poly(q)), cv = requant(cos_poly(q));
  *s = sneg ? neg_sat32(sv) : sv;
  *c = cneg ? neg_sat32(cv) : cv;
}
// RoPE angle = position * inv_freq, clamped to i64 (ops.rs:613-617).
DET_HD int64_t rope_angle(uint64_t position, int64_t inv_freq) {
  const i128 p = i128(position) * i128(inv_freq);
  if (p > i128(INT64_MAX)) return INT64_MAX;
  if (p < i128(INT64_MIN)) return INT64_MIN;
  return int64_t(p);
}

// ---------------------------------------------------------------------------
// Host-only helpers (load-time constants)
// ---------------------------------------------------------------------------
// pow_acc_u32 / nth_root_acc / rope_frequency_step (ops.rs:555-611).
inline int64_t pow_acc(int64_t base, uint32_t e) {
  int64_t r = kOneAcc;
  for (uint32_t i = 0; i < e; ++i) r = acc_mul(r, base);
  return r;
}
// Callers reject value == INT64_MAX first: the reference's bisection
// overflows i64 there (ops.rs:578) and never returns a root.
inline int64_t nth_root(int64_t value, uint32_t degree) {
  if (degree == 1 || value == kOneAcc) return value;
  int64_t lo = 0, hi = value > kOneAcc ? value : kOneAcc;
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo + 1) / 2;
    if (pow_acc(mid, degree) <= value) lo = mid; else hi = mid - 1;
  }
  const int64_t up = lo == INT64_MAX ? lo : lo + 1;
  const i128 le = i128(value) - i128(pow_acc(lo, degree));
  const i128 ue = i128(pow_acc(up, degree)) - i128(value);
  const i128 ale = le < 0 ? -le : le, aue = ue < 0 ? -ue : ue;
  if (aue < ale) return up;
  if (ale < aue) return lo;
  return (lo & 1) == 0 ? lo : up;
}
// div_acc(one, d) for d > 0: round(2^64 / d).
inline int64_t recip_acc(int64_t d) {
  const u128 num = u128(1) << 64;
  const u128 q = num / u128(uint64_t(d));
  const u128 r = num - q * u128(uint64_t(d));
  u128 qq = q;
  if (r * 2 > u128(uint64_t(d)) || (r * 2 == u128(uint64_t(d)) && (q & 1))) qq = q + 1;
  if (qq > u128(INT64_MAX)) return INT64_MAX;
  return int64_t(qq);
}
// inv_frequency table: entry i = step^i computed by the sequential rounded
// product chain of ops.rs:184-195.
inline void rope_inv_freq_table(int64_t base, uint32_t freq_base_dim, uint32_t half, int64_t* out) {
  const int64_t step = recip_acc(nth_root(base, freq_base_dim / 2));
  int64_t f = kOneAcc;
  for (uint32_t i = 0; i < half; ++i) { out[i] = f; f = acc_mul(f, step); }
}

// f32 -> Q16.16 / Q32.32 conversions from the IEEE-754 payload
// (convert.rs:82-153): round half to even, saturate.
inline int64_t f32_to_fixed(float x, unsigned frac, bool acc) {
  uint32_t bits;
  __builtin_memcpy(&bits, &x, 4);
  const bool neg = bits >> 31;
  const int eb = int((bits >> 23) & 0xff);
  const uint32_t fb = bits & 0x7fffff;
  const u128 maxpos = acc ? u128(INT64_MAX) : u128(INT32_MAX);
  const u128 maxneg = acc ? (u128(1) << 63) : (u128(1) << 31);
  if (eb == 0 && fb == 0) return 0;
  u128 sig = eb == 0 ? u128(fb) : u128((1u << 23) | fb);
  const int e = (eb == 0 ? -149 : eb - 150) + int(frac);
  const u128 maxm = neg ? maxneg : maxpos;
  u128 mag;
  if (e >= 0) {
    mag = (e >= 128 || sig > (maxm >> e)) ? maxm : (sig << e);
  } else {
    const unsigned s = unsigned(-e);
    if (s >= 128) mag = 0;
    else {
      const u128 q = sig >> s, rem = sig & ((u128(1) << s) - 1), half = u128(1) << (s - 1);
      mag = (rem > half || (rem == half && (q & 1))) ? q + 1 : q;
    }
    if (mag > maxm) mag = maxm;
  }
  if (neg) return mag >= maxneg ? -int64_t(maxneg - 1) - 1 : -int64_t(mag);
  return int64_t(mag);
}
inline int32_t f32_to_act(float x) { return int32_t(f32_to_fixed(x, 16, false)); }
inline int64_t f32_to_acc(float x) { return f32_to_fixed(x, 32, true); }

}  // namespace det
