// ORACLE — test infrastructure only (see oracle.h). C wrappers over the
// scalar restatement in det_num.cpp, used by the golden-vector tests.
#include <string>

#include "det_num.h"
#include "oracle.h"

using namespace oracle;

namespace {
thread_local std::string g_scalar_error;
template <class F>
int guard(F&& f) {
  try {
    f();
    return 0;
  } catch (const ContractViolation& e) {
    g_scalar_error = e.what();
    return 2;
  } catch (const std::exception& e) {
    g_scalar_error = e.what();
    return 3;
  }
}
}  // namespace

extern "C" {

const char* orc_scalar_last_error(void) { return g_scalar_error.c_str(); }
int64_t orc_mac_bits(int64_t acc, int32_t a, int32_t w) { return mac_bits(acc, a, w); }
int64_t orc_acc_combine(int64_t a, int64_t b) { return acc_combine(a, b); }
int32_t orc_add_sat(int32_t a, int32_t b) { return add_sat(a, b); }
int32_t orc_sub_sat(int32_t a, int32_t b) { return sub_sat(a, b); }
int64_t orc_acc_add_sat(int64_t a, int64_t b) { return acc_add_sat(a, b); }
int32_t orc_mul_sat(int32_t a, int32_t b) { return mul_sat(a, b); }
int32_t orc_requantize(int64_t acc) { return requantize(acc); }
int orc_rshift_round_ties_even(int64_t x, uint32_t s, int64_t* out) {
  return guard([&] { *out = rshift_round_ties_even(x, s); });
}
int orc_div_act(int32_t n, int32_t d, int32_t* out) { return guard([&] { *out = div_act(n, d); }); }
int orc_div_acc(int64_t n, int64_t d, int64_t* out) { return guard([&] { *out = div_acc(n, d); }); }
int orc_div_acc_by_u32(int64_t v, uint32_t d, int64_t* out) {
  return guard([&] { *out = div_acc_by_u32(v, d); });
}
int64_t orc_acc_mul(int64_t a, int64_t b) { return acc_mul(a, b); }
int orc_inv_sqrt_acc(int64_t x, int32_t* out) { return guard([&] { *out = inv_sqrt_acc(x); }); }
int orc_rms_norm_scale(const int32_t* x, size_t n, int64_t eps, int32_t* out) {
  return guard([&] { *out = rms_norm_scale(x, n, eps); });
}
int orc_rms_norm(int32_t* x, const int32_t* w, size_t n, int64_t eps) {
  return guard([&] { rms_norm_in_place(x, w, n, eps); });
}
int orc_value_rms_norm(int32_t* x, size_t n, int64_t eps) {
  return guard([&] { value_rms_norm_in_place(x, n, eps); });
}
int orc_attention_score(const int32_t* q, const int32_t* k, size_t n, int32_t* out) {
  return guard([&] { *out = attention_score(q, k, n); });
}
int orc_attention_softmax_exp_term(int32_t logit, int32_t max_logit, int64_t* out) {
  return guard([&] { *out = attention_softmax_exp_term(logit, max_logit); });
}
int orc_attention_softmax(const int32_t* logits, size_t n, int32_t* weights) {
  return guard([&] { attention_softmax(logits, n, weights); });
}
int orc_attention_weighted_sum(const int32_t* weights, const int32_t* rows, size_t n_rows,
                               size_t width, int32_t* out) {
  return guard([&] { attention_weighted_sum(weights, rows, n_rows, width, out); });
}
int32_t orc_tanh_act(int32_t x) { return tanh_act(x); }
int orc_softcap_act(int32_t x, int32_t softcap, int32_t* out) {
  return guard([&] { *out = softcap_act(x, softcap); });
}
int32_t orc_gelu_pytorch_tanh_act(int32_t x) { return gelu_pytorch_tanh_act(x); }
int orc_nth_root_acc(int64_t v, uint32_t degree, int64_t* out) {
  return guard([&] { *out = nth_root_acc(v, degree); });
}
int orc_rope_frequency_step(int64_t base, size_t fbd, int64_t* out) {
  return guard([&] { *out = rope_frequency_step(base, fbd); });
}
void orc_sin_cos_acc(int64_t angle, int32_t* c, int32_t* s) { sin_cos_acc(angle, c, s); }
int orc_rope_rotate_pairs(int32_t* v, size_t n, size_t rotary_dim, size_t fbd, int64_t base,
                          size_t position) {
  return guard([&] { rope_rotate_pairs_in_place(v, n, rotary_dim, fbd, base, position); });
}
int orc_argmax_first(const int32_t* x, size_t n, size_t* out) {
  return guard([&] { *out = argmax_first(x, n); });
}
int orc_f32_to_act(float x, int32_t* out) { return guard([&] { *out = f32_to_act(x); }); }
int orc_f32_to_wgt(float x, int32_t* out) { return guard([&] { *out = f32_to_wgt(x); }); }
int orc_f32_to_acc(float x, int64_t* out) { return guard([&] { *out = f32_to_acc(x); }); }

}  // extern "C"
