// ORACLE — test infrastructure only. This file is a CPU restatement of the
// reference's canonical fixed-point arithmetic; it exists to check the HIP
// product path and is never linked into it. Only tests/, the smoke check and
// bench.py's cpu_baseline leg may load it.
//
// Restates src/shared/numerics/det_num/{types,ops,convert,serialize}.rs.
// Value model: Act/Wgt are Q16.16 in i32, Acc is Q32.32 in i64
// (det_num/types.rs:8-25). Every function keeps the reference's operation
// order; wide intermediates use __int128 exactly where the reference uses
// i128/u128.
#pragma once

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

namespace oracle {

using i128 = __int128;
using u128 = unsigned __int128;

constexpr unsigned kActFrac = 16;      // types.rs:23
constexpr unsigned kAccFrac = 32;      // types.rs:24
constexpr unsigned kRequantShift = 16; // types.rs:25

// Contract violations: the reference panics (assert!); the oracle throws so
// that the C ABI can report them as an error status.
struct ContractViolation : std::logic_error {
  using std::logic_error::logic_error;
};
[[noreturn]] void contract_violation(const std::string& what);

// ops.rs:4-7 mul_wide: exact i32 x i32 -> i64.
inline int64_t mul_wide(int32_t a, int32_t w) { return int64_t(a) * int64_t(w); }

// ops.rs:14-16 mac_bits: wrapping i64 accumulate of the exact product.
inline int64_t mac_bits(int64_t acc, int32_t a, int32_t w) {
  return int64_t(uint64_t(acc) + uint64_t(int64_t(a) * int64_t(w)));
}

// ops.rs:28-30 acc_combine: wrapping i64 add.
inline int64_t acc_combine(int64_t a, int64_t b) { return int64_t(uint64_t(a) + uint64_t(b)); }

inline int32_t sat_i64_to_i32(int64_t v) {  // ops.rs:480-483 narrow_act_sat
  if (v > INT32_MAX) return INT32_MAX;
  if (v < INT32_MIN) return INT32_MIN;
  return int32_t(v);
}
inline int32_t clamp_i128_to_i32(i128 v) {  // ops.rs:485-487
  if (v > i128(INT32_MAX)) return INT32_MAX;
  if (v < i128(INT32_MIN)) return INT32_MIN;
  return int32_t(v);
}
inline int64_t clamp_i128_to_i64(i128 v) {  // ops.rs:489-491
  if (v > i128(INT64_MAX)) return INT64_MAX;
  if (v < i128(INT64_MIN)) return INT64_MIN;
  return int64_t(v);
}

// ops.rs:33-35 add_sat, ops.rs:428-430 sub_sat, ops.rs:433-435 acc_add_sat.
inline int32_t add_sat(int32_t a, int32_t b) { return sat_i64_to_i32(int64_t(a) + int64_t(b)); }
inline int32_t sub_sat(int32_t a, int32_t b) { return sat_i64_to_i32(int64_t(a) - int64_t(b)); }
inline int64_t acc_add_sat(int64_t a, int64_t b) { return clamp_i128_to_i64(i128(a) + i128(b)); }
inline int32_t neg_sat32(int32_t a) { return a == INT32_MIN ? INT32_MAX : -a; }  // i32::saturating_neg
inline int64_t neg_sat64(int64_t a) { return a == INT64_MIN ? INT64_MAX : -a; }  // i64::saturating_neg

constexpr int32_t kOneAct = int32_t(1) << kActFrac;  // ops.rs:497-499
constexpr int64_t kOneAcc = int64_t(1) << kAccFrac;  // ops.rs:501-503

// ops.rs:770-800 rshift_round_ties_even_bits (shift < 64).
int64_t rshift_round_ties_even(int64_t x, unsigned shift);
// ops.rs:688-717 round_ties_even_division.
i128 round_ties_even_division(i128 dividend, i128 divisor);

// ops.rs:445-448 requantize (and clip_act, ops.rs:454-458).
inline int32_t requantize(int64_t acc) {
  return sat_i64_to_i32(rshift_round_ties_even(acc, kRequantShift));
}
// ops.rs:38-42 mul_sat; ops.rs:45-47 scale_act.
inline int32_t mul_sat(int32_t a, int32_t b) { return requantize(int64_t(a) * int64_t(b)); }
inline int32_t scale_act(int32_t v, int32_t s) { return mul_sat(v, s); }

int32_t div_act(int32_t numerator, int32_t denominator);        // ops.rs:50-61
int64_t div_acc(int64_t numerator, int64_t denominator);        // ops.rs:64-75
int64_t div_acc_by_u32(int64_t value, uint32_t divisor);        // ops.rs:78-85
int64_t acc_mul(int64_t lhs, int64_t rhs);                      // ops.rs:682-686
int32_t inv_sqrt_acc(int64_t x);                                // ops.rs:719-763

// ops.rs:406-425 rms_norm_scale; ops.rs:95-111 / 121-131 norms in place.
int32_t rms_norm_scale(const int32_t* x, size_t n, int64_t eps);
void rms_norm_in_place(int32_t* x, const int32_t* w, size_t n, int64_t eps);
void value_rms_norm_in_place(int32_t* x, size_t n, int64_t eps);

// ops.rs:199-217 attention_score.
int32_t attention_score(const int32_t* q, const int32_t* k, size_t n);
// ops.rs:505-553 softmax_exp_term, exposed through ops.rs:261-263.
int64_t softmax_exp_term(int64_t delta);
int64_t attention_softmax_exp_term(int32_t logit, int32_t max_logit);
// ops.rs:230-258 attention_softmax_into.
void attention_softmax(const int32_t* logits, size_t n, int32_t* weights);
// ops.rs:336-351 attention_weighted_sum_core (rows are contiguous, `width` wide).
void attention_weighted_sum(const int32_t* weights, const int32_t* rows, size_t n_rows,
                            size_t width, int32_t* out);

int32_t tanh_act(int32_t x);                         // ops.rs:354-374
int32_t softcap_act(int32_t x, int32_t softcap);     // ops.rs:377-385
int32_t gelu_pytorch_tanh_act(int32_t x);            // ops.rs:388-403

// RoPE, ops.rs:151-196 and helpers ops.rs:555-680.
int64_t pow_acc_u32(int64_t base, uint32_t exponent);
int64_t nth_root_acc(int64_t value, uint32_t degree);
int64_t rope_frequency_step(int64_t base, size_t freq_base_dim);
void sin_cos_acc(int64_t angle, int32_t* cos_out, int32_t* sin_out);
void rope_rotate_pairs_in_place(int32_t* v, size_t n, size_t rotary_dim, size_t freq_base_dim,
                                int64_t base, size_t position);

size_t argmax_first(const int32_t* x, size_t n);  // ops.rs:463-478

// convert.rs:53-106 f32 -> fixed conversions (exact from the IEEE payload).
int32_t f32_to_act(float x);
int32_t f32_to_wgt(float x);
int64_t f32_to_acc(float x);

}  // namespace oracle
