// ORACLE — test infrastructure only (see det_num.h). CPU restatement of
// src/shared/numerics/det_num/ops.rs and convert.rs.
#include "det_num.h"

#include <cmath>
#include <cstring>
#include <vector>

namespace oracle {

void contract_violation(const std::string& what) { throw ContractViolation(what); }

static i128 abs128(i128 v) { return v < 0 ? -v : v; }

// ops.rs:770-800
int64_t rshift_round_ties_even(int64_t x_bits, unsigned shift) {
  if (shift == 0) return x_bits;
  if (shift >= 64) contract_violation("shift must be less than 64 bits");
  const i128 divisor = i128(1) << shift;
  const i128 x = x_bits;
  const i128 quotient = x / divisor;   // truncating, as Rust i128 `/`
  const i128 remainder = x % divisor;  // sign of dividend, as Rust `%`
  if (remainder == 0) return int64_t(quotient);
  const i128 twice = abs128(remainder) * 2;
  const i128 step = x < 0 ? -1 : 1;
  i128 rounded;
  if (twice < divisor) rounded = quotient;
  else if (twice > divisor) rounded = quotient + step;
  else if ((quotient & 1) == 0) rounded = quotient;
  else rounded = quotient + step;
  return int64_t(rounded);
}

// ops.rs:688-717
i128 round_ties_even_division(i128 dividend, i128 divisor) {
  if (divisor == 0) contract_violation("round_ties_even_division requires a non-zero divisor");
  const i128 quotient = dividend / divisor;
  const i128 remainder = dividend % divisor;
  if (remainder == 0) return quotient;
  const i128 twice = abs128(remainder) * 2;
  const i128 abs_div = abs128(divisor);
  const i128 step = ((dividend < 0) != (divisor < 0)) ? -1 : 1;
  if (twice < abs_div) return quotient;
  if (twice > abs_div) return quotient + step;
  if ((quotient & 1) == 0) return quotient;
  return quotient + step;
}

// ops.rs:50-61
int32_t div_act(int32_t numerator, int32_t denominator) {
  if (denominator == 0) contract_violation("div_act requires a non-zero denominator");
  const i128 dividend = i128(numerator) << kActFrac;
  return clamp_i128_to_i32(round_ties_even_division(dividend, i128(denominator)));
}

// ops.rs:64-75
int64_t div_acc(int64_t numerator, int64_t denominator) {
  if (denominator == 0) contract_violation("div_acc requires a non-zero denominator");
  const i128 dividend = i128(numerator) << kAccFrac;
  return clamp_i128_to_i64(round_ties_even_division(dividend, i128(denominator)));
}

// ops.rs:78-85
int64_t div_acc_by_u32(int64_t value, uint32_t divisor) {
  if (divisor == 0) contract_violation("div_acc_by_u32 requires a non-zero divisor");
  return clamp_i128_to_i64(round_ties_even_division(i128(value), i128(divisor)));
}

// ops.rs:682-686
int64_t acc_mul(int64_t lhs, int64_t rhs) {
  const i128 product = i128(lhs) * i128(rhs);
  return clamp_i128_to_i64(round_ties_even_division(product, i128(1) << kAccFrac));
}

// ops.rs:765-768 (u128 saturating products)
static u128 sat_mul_u128(u128 a, u128 b) {
  u128 r;
  if (__builtin_mul_overflow(a, b, &r)) return ~u128(0);
  return r;
}
static u128 inv_sqrt_product(uint32_t candidate_bits, u128 divisor) {
  const u128 c = candidate_bits;
  return sat_mul_u128(sat_mul_u128(c, c), divisor);
}

// ops.rs:719-763
int32_t inv_sqrt_acc(int64_t x_bits) {
  if (x_bits < 0) contract_violation("inv_sqrt_acc requires a non-negative input");
  if (x_bits == 0) return INT32_MAX;
  const u128 target = u128(1) << 64;
  const u128 divisor = u128(uint64_t(x_bits));
  const uint32_t max_bits = uint32_t(INT32_MAX);
  if (inv_sqrt_product(max_bits, divisor) <= target) return INT32_MAX;
  uint32_t low = 0, high = max_bits;
  while (low < high) {
    const uint32_t mid = low + ((high - low + 1) / 2);
    if (inv_sqrt_product(mid, divisor) <= target) low = mid;
    else high = mid - 1;
  }
  const uint32_t lower_bits = low;
  uint32_t upper_bits = lower_bits == UINT32_MAX ? UINT32_MAX : lower_bits + 1;
  if (upper_bits > max_bits) upper_bits = max_bits;
  const u128 lower_product = inv_sqrt_product(lower_bits, divisor);
  const u128 upper_product = inv_sqrt_product(upper_bits, divisor);
  const u128 lower_error = target - lower_product;
  const u128 upper_error = upper_product > target ? upper_product - target : 0;
  uint32_t rounded;
  if (upper_bits == lower_bits || lower_error < upper_error) rounded = lower_bits;
  else if (upper_error < lower_error) rounded = upper_bits;
  else if ((lower_bits & 1) == 0) rounded = lower_bits;
  else rounded = upper_bits;
  return int32_t(rounded);
}

// ops.rs:406-425
int32_t rms_norm_scale(const int32_t* x, size_t n, int64_t eps) {
  if (n == 0) contract_violation("rms_norm_scale requires a non-empty input slice");
  if (eps < 0) contract_violation("rms_norm_scale requires a non-negative epsilon");
  int64_t sum_squares = 0;
  for (size_t i = 0; i < n; ++i) sum_squares = acc_add_sat(sum_squares, mul_wide(x[i], x[i]));
  if (n > UINT32_MAX) contract_violation("row width should fit in u32");
  const int64_t mean_square = div_acc_by_u32(sum_squares, uint32_t(n));
  const int64_t adjusted = acc_add_sat(mean_square, eps);
  return inv_sqrt_acc(adjusted);
}

// ops.rs:95-111
void rms_norm_in_place(int32_t* x, const int32_t* w, size_t n, int64_t eps) {
  if (n == 0) contract_violation("rms_norm requires a non-empty input slice");
  const int32_t scale = rms_norm_scale(x, n, eps);
  for (size_t i = 0; i < n; ++i) x[i] = mul_sat(mul_sat(x[i], scale), w[i]);
}

// ops.rs:121-131
void value_rms_norm_in_place(int32_t* x, size_t n, int64_t eps) {
  if (n == 0) contract_violation("value_rms_norm requires a non-empty input slice");
  const int32_t scale = rms_norm_scale(x, n, eps);
  for (size_t i = 0; i < n; ++i) x[i] = mul_sat(x[i], scale);
}

// ops.rs:199-217
int32_t attention_score(const int32_t* q, const int32_t* k, size_t n) {
  if (n == 0) contract_violation("attention_score requires a non-empty query slice");
  int64_t acc = 0;
  for (size_t i = 0; i < n; ++i) acc = mac_bits(acc, q[i], k[i]);
  return requantize(acc);
}

// ops.rs:505-553
int64_t softmax_exp_term(int64_t delta) {
  const int64_t LN_2_BITS = 2977044472LL;
  const int64_t MIN_DELTA_BITS = -(int64_t(16) << kAccFrac);
  if (delta > 0) contract_violation("softmax_exp_term requires max-shifted non-positive logits");
  if (delta <= MIN_DELTA_BITS) return 0;
  const int64_t positive = neg_sat64(delta);
  const int64_t shift = positive / LN_2_BITS;
  const int64_t r = positive % LN_2_BITS;
  const int64_t r2 = acc_mul(r, r);
  const int64_t r3 = acc_mul(r2, r);
  const int64_t r4 = acc_mul(r3, r);
  const int64_t r5 = acc_mul(r4, r);
  const int64_t approx = acc_add_sat(
      acc_add_sat(kOneAcc, neg_sat64(r)),
      acc_add_sat(div_acc_by_u32(r2, 2),
                  acc_add_sat(neg_sat64(div_acc_by_u32(r3, 6)),
                              acc_add_sat(div_acc_by_u32(r4, 24), neg_sat64(div_acc_by_u32(r5, 120))))));
  if (approx <= 0) return 0;
  if (shift >= 0 && shift < 64) return rshift_round_ties_even(approx, unsigned(shift));
  return 0;
}

// ops.rs:261-263 (act_to_acc is ops.rs:493-495)
int64_t attention_softmax_exp_term(int32_t logit, int32_t max_logit) {
  return softmax_exp_term(int64_t(sub_sat(logit, max_logit)) << kRequantShift);
}

// ops.rs:230-258 with ops.rs:266-273
void attention_softmax(const int32_t* logits, size_t n, int32_t* weights) {
  if (n == 0) contract_violation("attention_softmax requires a non-empty logits slice");
  const size_t max_index = argmax_first(logits, n);
  const int32_t max_logit = logits[max_index];
  std::vector<int64_t> exp_terms(n);
  for (size_t i = 0; i < n; ++i) exp_terms[i] = attention_softmax_exp_term(logits[i], max_logit);
  int64_t sum_exp = 0;
  for (size_t i = 0; i < n; ++i) sum_exp = acc_add_sat(sum_exp, exp_terms[i]);
  for (size_t i = 0; i < n; ++i) weights[i] = requantize(div_acc(exp_terms[i], sum_exp));
  int32_t summed = 0;
  for (size_t i = 0; i < n; ++i) summed = add_sat(summed, weights[i]);
  const int32_t residual = sub_sat(kOneAct, summed);
  weights[max_index] = add_sat(weights[max_index], residual);
}

// ops.rs:336-351 (canonical column-major MAC order)
void attention_weighted_sum(const int32_t* weights, const int32_t* rows, size_t n_rows,
                            size_t width, int32_t* out) {
  if (n_rows == 0) contract_violation("attention_weighted_sum requires a non-empty weights slice");
  for (size_t d = 0; d < width; ++d) {
    int64_t acc = 0;
    for (size_t r = 0; r < n_rows; ++r) acc = mac_bits(acc, rows[r * width + d], weights[r]);
    out[d] = requantize(acc);
  }
}

// ops.rs:354-374
int32_t tanh_act(int32_t x) {
  const int32_t LIN = 27 << kActFrac;
  const int32_t QUAD = 9 << kActFrac;
  const int32_t SAT = 3 << kActFrac;
  if (x >= SAT) return kOneAct;
  if (x <= -SAT) return neg_sat32(kOneAct);
  const int32_t x2 = mul_sat(x, x);
  const int32_t num_scale = add_sat(LIN, x2);
  const int32_t den_scale = add_sat(LIN, mul_sat(QUAD, x2));
  const int32_t num = mul_sat(x, num_scale);
  return div_act(num, den_scale);
}

// ops.rs:377-385
int32_t softcap_act(int32_t x, int32_t softcap) {
  if (softcap <= 0) contract_violation("softcap_act requires a strictly positive softcap");
  return mul_sat(softcap, tanh_act(div_act(x, softcap)));
}

// ops.rs:388-403
int32_t gelu_pytorch_tanh_act(int32_t x) {
  const int32_t HALF = 1 << (kActFrac - 1);
  const int32_t INNER = 52290;
  const int32_t CUBIC = 2930;
  const int32_t x2 = mul_sat(x, x);
  const int32_t x3 = mul_sat(x2, x);
  const int32_t cubic = mul_sat(CUBIC, x3);
  const int32_t inner = add_sat(x, cubic);
  const int32_t t = tanh_act(mul_sat(INNER, inner));
  return mul_sat(mul_sat(HALF, x), add_sat(kOneAct, t));
}

// ops.rs:605-611
int64_t pow_acc_u32(int64_t base, uint32_t exponent) {
  int64_t result = kOneAcc;
  for (uint32_t i = 0; i < exponent; ++i) result = acc_mul(result, base);
  return result;
}

// ops.rs:561-603
int64_t nth_root_acc(int64_t value, uint32_t degree) {
  if (degree == 0) contract_violation("nth_root_acc requires a positive degree");
  if (value <= 0) contract_violation("nth_root_acc requires a positive input");
  if (degree == 1 || value == kOneAcc) return value;
  // ops.rs:578 evaluates `high_bits - low_bits + 1`, which overflows i64 on the
  // first step when value == i64::MAX: the reference panics there ("attempt to
  // add with overflow") in builds with overflow checks and, without them,
  // wraps into a bisection that never terminates. The oracle reports the panic.
  if (value == INT64_MAX) contract_violation("nth_root_acc: attempt to add with overflow (value i64::MAX)");
  int64_t low = 0;
  int64_t high = value > kOneAcc ? value : kOneAcc;
  while (low < high) {
    const int64_t mid = low + ((high - low + 1) / 2);
    if (pow_acc_u32(mid, degree) <= value) low = mid;
    else high = mid - 1;
  }
  const int64_t lower = low;
  const int64_t upper = lower == INT64_MAX ? INT64_MAX : lower + 1;
  const int64_t lower_value = pow_acc_u32(lower, degree);
  const int64_t upper_value = pow_acc_u32(upper, degree);
  const i128 lower_error = abs128(i128(value) - i128(lower_value));
  const i128 upper_error = abs128(i128(upper_value) - i128(value));
  if (upper_error < lower_error) return upper;
  if (lower_error < upper_error) return lower;
  return (lower & 1) == 0 ? lower : upper;
}

// ops.rs:555-559
int64_t rope_frequency_step(int64_t base, size_t freq_base_dim) {
  const uint32_t degree = uint32_t(freq_base_dim / 2);
  return div_acc(kOneAcc, nth_root_acc(base, degree));
}

// ops.rs:647-663
static int64_t sin_polynomial(int64_t x) {
  const int64_t x2 = acc_mul(x, x);
  const int64_t x3 = acc_mul(x2, x);
  const int64_t x5 = acc_mul(x3, x2);
  const int64_t x7 = acc_mul(x5, x2);
  return acc_add_sat(acc_add_sat(x, neg_sat64(div_acc_by_u32(x3, 6))),
                     acc_add_sat(div_acc_by_u32(x5, 120), neg_sat64(div_acc_by_u32(x7, 5040))));
}

// ops.rs:665-680
static int64_t cos_polynomial(int64_t x) {
  const int64_t x2 = acc_mul(x, x);
  const int64_t x4 = acc_mul(x2, x2);
  const int64_t x6 = acc_mul(x4, x2);
  return acc_add_sat(acc_add_sat(kOneAcc, neg_sat64(div_acc_by_u32(x2, 2))),
                     acc_add_sat(div_acc_by_u32(x4, 24), neg_sat64(div_acc_by_u32(x6, 720))));
}

// ops.rs:619-645
void sin_cos_acc(int64_t angle, int32_t* cos_out, int32_t* sin_out) {
  const int64_t HALF_PI = 6746518852LL;
  const int64_t PI = 13493037705LL;
  const int64_t THREE_HALF_PI = 20239556557LL;
  const int64_t TWO_PI = 26986075409LL;
  int64_t reduced = angle % TWO_PI;  // rem_euclid
  if (reduced < 0) reduced += TWO_PI;
  int64_t q;
  int sin_sign, cos_sign;
  if (reduced <= HALF_PI) { q = reduced; sin_sign = 1; cos_sign = 1; }
  else if (reduced <= PI) { q = PI - reduced; sin_sign = 1; cos_sign = -1; }
  else if (reduced <= THREE_HALF_PI) { q = reduced - PI; sin_sign = -1; cos_sign = -1; }
  else { q = TWO_PI - reduced; sin_sign = -1; cos_sign = 1; }
  int32_t s = requantize(sin_polynomial(q));
  int32_t c = requantize(cos_polynomial(q));
  if (sin_sign < 0) s = neg_sat32(s);
  if (cos_sign < 0) c = neg_sat32(c);
  *cos_out = c;
  *sin_out = s;
}

// ops.rs:613-617
static int64_t mul_usize_by_acc(size_t m, int64_t v) { return clamp_i128_to_i64(i128(m) * i128(v)); }

// ops.rs:151-196
void rope_rotate_pairs_in_place(int32_t* v, size_t n, size_t rotary_dim, size_t freq_base_dim,
                                int64_t base, size_t position) {
  if (rotary_dim == 0) return;
  if (rotary_dim % 2 != 0) contract_violation("rope_rotate_pairs requires an even rotary_dim");
  if (rotary_dim > n) contract_violation("rope_rotate_pairs requires rotary_dim to fit within the input width");
  if (freq_base_dim < 2 || freq_base_dim % 2 != 0)
    contract_violation("rope_rotate_pairs requires an even freq_base_dim of at least 2");
  if (base <= 0) contract_violation("rope_rotate_pairs requires a positive base");
  if (position == 0) return;
  const size_t half = rotary_dim / 2;
  int64_t inv_frequency = kOneAcc;
  const int64_t step = rope_frequency_step(base, freq_base_dim);
  for (size_t i = 0; i < half; ++i) {
    const int64_t angle = mul_usize_by_acc(position, inv_frequency);
    int32_t c, s;
    sin_cos_acc(angle, &c, &s);
    const int32_t lhs = v[i];
    const int32_t rhs = v[i + half];
    v[i] = sub_sat(mul_sat(lhs, c), mul_sat(rhs, s));
    v[i + half] = add_sat(mul_sat(rhs, c), mul_sat(lhs, s));
    inv_frequency = acc_mul(inv_frequency, step);
  }
}

// ops.rs:463-478
size_t argmax_first(const int32_t* x, size_t n) {
  if (n == 0) contract_violation("argmax_first requires a non-empty slice");
  size_t best = 0;
  int32_t best_bits = x[0];
  for (size_t i = 1; i < n; ++i) {
    if (x[i] > best_bits) { best = i; best_bits = x[i]; }
  }
  return best;
}

// convert.rs:155-189
static u128 saturating_shift_left(u128 value, unsigned shift, u128 max_magnitude) {
  if (value == 0) return 0;
  if (shift >= 128) return max_magnitude;
  const u128 threshold = max_magnitude >> shift;
  return value > threshold ? max_magnitude : (value << shift);
}
static u128 round_ties_even_div_pow2(u128 value, unsigned shift) {
  if (shift == 0) return value;
  if (shift >= 128) return 0;
  const u128 quotient = value >> shift;
  const u128 remainder = value & ((u128(1) << shift) - 1);
  const u128 halfway = u128(1) << (shift - 1);
  if (remainder > halfway || (remainder == halfway && (quotient & 1) == 1)) return quotient + 1;
  return quotient;
}

// convert.rs:108-153
static i128 f32_to_fixed_bits(float x, unsigned frac, u128 max_pos, u128 max_neg) {
  uint32_t bits;
  std::memcpy(&bits, &x, 4);
  const bool negative = (bits >> 31) != 0;
  const int exponent_bits = int((bits >> 23) & 0xff);
  const uint32_t fraction_bits = bits & 0x7fffff;
  if (exponent_bits == 0 && fraction_bits == 0) return 0;
  u128 significand;
  int exponent;
  if (exponent_bits == 0) { significand = fraction_bits; exponent = -149; }
  else { significand = (uint32_t(1) << 23) | fraction_bits; exponent = exponent_bits - 127 - 23; }
  const int scaled = exponent + int(frac);
  const u128 max_mag = negative ? max_neg : max_pos;
  u128 magnitude;
  if (scaled >= 0) magnitude = saturating_shift_left(significand, unsigned(scaled), max_mag);
  else {
    magnitude = round_ties_even_div_pow2(significand, unsigned(-scaled));
    if (magnitude > max_mag) magnitude = max_mag;
  }
  if (negative) return magnitude >= max_neg ? -i128(max_neg) : -i128(magnitude);
  return i128(magnitude);
}

// convert.rs:82-93
static int32_t f32_to_q16_16_bits(float x) {
  if (!std::isfinite(x)) contract_violation("f32 conversion requires a finite source value");
  const i128 b = f32_to_fixed_bits(x, kActFrac, u128(INT32_MAX), u128(1) << 31);
  return clamp_i128_to_i32(b);
}
int32_t f32_to_act(float x) { return f32_to_q16_16_bits(x); }  // convert.rs:53-57
int32_t f32_to_wgt(float x) { return f32_to_q16_16_bits(x); }  // convert.rs:77-80

// convert.rs:60-64, 95-106
int64_t f32_to_acc(float x) {
  if (!std::isfinite(x)) contract_violation("f32_to_acc requires a finite source value");
  const i128 b = f32_to_fixed_bits(x, kAccFrac, u128(INT64_MAX), u128(1) << 63);
  return clamp_i128_to_i64(b);
}

}  // namespace oracle
