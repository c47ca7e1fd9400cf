// ORACLE — test infrastructure only. C ABI of the CPU restatement of the
// reference's deterministic path, loaded by tests/ (ctypes), the smoke check
// and bench.py's cpu_baseline leg. Never linked into the HIP product.
//
// Status convention: 0 = ok, 1 = invalid argument / shape mismatch,
// 2 = contract violation (the reference would panic), 3 = internal error.
// orc_last_error() returns the message of the last failure on this thread.
#pragma once
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// Raw Gemma text config (mirrors GemmaTextConfigFile, gemma/io.rs:60-83).
// has_* flags mark Option<...> fields that were present in config.json.
typedef struct orc_text_config {
  int32_t enable_moe_block;
  int32_t hidden_activation_is_gelu_pytorch_tanh;
  int32_t has_final_logit_softcapping;
  float final_logit_softcapping;
  int32_t has_global_head_dim;
  uint64_t global_head_dim;
  uint64_t head_dim;
  uint64_t hidden_size;
  int32_t has_hidden_size_per_layer_input;
  uint64_t hidden_size_per_layer_input;
  uint64_t num_layer_types;
  const int32_t* layer_types;  // 1 = "sliding_attention", 0 = anything else
  int32_t has_num_global_key_value_heads;
  uint64_t num_global_key_value_heads;
  uint64_t num_attention_heads;
  uint64_t num_hidden_layers;
  uint64_t num_key_value_heads;
  float rms_norm_eps;
  int32_t has_full_partial_rotary_factor;
  float full_partial_rotary_factor;
  int32_t has_full_rope_theta;
  float full_rope_theta;
  int32_t has_sliding_rope_theta;
  float sliding_rope_theta;
  int32_t has_rope_theta;
  float rope_theta;
  uint64_t sliding_window;
  int32_t has_tie_word_embeddings;
  int32_t tie_word_embeddings;
  uint64_t vocab_size;
  int32_t has_vocab_size_per_layer_input;
  uint64_t vocab_size_per_layer_input;
  int32_t has_attention_k_eq_v;
  int32_t attention_k_eq_v;
  int32_t has_num_kv_shared_layers;
  uint64_t num_kv_shared_layers;
  int32_t bidirectional_all;  // use_bidirectional_attention == "all"
} orc_text_config;

const char* orc_last_error(void);

// ---- scalar arithmetic (det_num/ops.rs, convert.rs) ----
int64_t orc_mac_bits(int64_t acc, int32_t a, int32_t w);
int64_t orc_acc_combine(int64_t a, int64_t b);
int32_t orc_add_sat(int32_t a, int32_t b);
int32_t orc_sub_sat(int32_t a, int32_t b);
int64_t orc_acc_add_sat(int64_t a, int64_t b);
int32_t orc_mul_sat(int32_t a, int32_t b);
int32_t orc_requantize(int64_t acc);
int orc_rshift_round_ties_even(int64_t x, uint32_t shift, int64_t* out);
int orc_div_act(int32_t n, int32_t d, int32_t* out);
int orc_div_acc(int64_t n, int64_t d, int64_t* out);
int orc_div_acc_by_u32(int64_t v, uint32_t d, int64_t* out);
int64_t orc_acc_mul(int64_t a, int64_t b);
int orc_inv_sqrt_acc(int64_t x, int32_t* out);
int orc_rms_norm_scale(const int32_t* x, size_t n, int64_t eps, int32_t* out);
int orc_rms_norm(int32_t* x, const int32_t* w, size_t n, int64_t eps);
int orc_value_rms_norm(int32_t* x, size_t n, int64_t eps);
int orc_attention_score(const int32_t* q, const int32_t* k, size_t n, int32_t* out);
int orc_attention_softmax_exp_term(int32_t logit, int32_t max_logit, int64_t* out);
int orc_attention_softmax(const int32_t* logits, size_t n, int32_t* weights);
int orc_attention_weighted_sum(const int32_t* weights, const int32_t* rows, size_t n_rows,
                               size_t width, int32_t* out);
int32_t orc_tanh_act(int32_t x);
int orc_softcap_act(int32_t x, int32_t softcap, int32_t* out);
int32_t orc_gelu_pytorch_tanh_act(int32_t x);
int orc_nth_root_acc(int64_t v, uint32_t degree, int64_t* out);
int orc_rope_frequency_step(int64_t base, size_t freq_base_dim, int64_t* out);
void orc_sin_cos_acc(int64_t angle, int32_t* cos_out, int32_t* sin_out);
int orc_rope_rotate_pairs(int32_t* v, size_t n, size_t rotary_dim, size_t freq_base_dim,
                          int64_t base, size_t position);
int orc_argmax_first(const int32_t* x, size_t n, size_t* out);
int orc_f32_to_act(float x, int32_t* out);
int orc_f32_to_wgt(float x, int32_t* out);
int orc_f32_to_acc(float x, int64_t* out);

// ---- GEMV / GEMM (det_kernels.rs:108-203) ----
// weight: rows x cols row-major; elem_width 16 or 32 (sign-extended on read).
// threads <= 1: serial reference order; > 1: output-row-parallel schedule of
// det_linear_into_par (identical bits by construction).
int orc_det_linear(size_t rows, size_t cols, int elem_width, const void* weight,
                   const int32_t* act, int32_t* out, int threads);
int orc_det_linear_acc_i64(size_t rows, size_t cols, int elem_width, const void* weight,
                           const int32_t* act, int64_t* acc_out);
// threads > 1: token rows spread over the threads, each one serial GEMV
// (det_linear_slab's parallel schedule).
int orc_det_linear_slab(size_t m, size_t rows, size_t cols, int elem_width, const void* weight,
                        const int32_t* act, int32_t* out, int threads);

// ---- attention / RoPE drivers ----
// det_attention_prefill's (head, query) items without a donor cache
// (det_kernels.rs:584-646): q [nq][nh*hd], k/v [nrows][nkv*hd]; query t attends
// rows [max(0, t+1-window), t+1), window 0 = unbounded; out [nq][nh*hd].
int orc_attention_causal(const int32_t* q, const int32_t* k, const int32_t* v, size_t nq, size_t nrows,
                         size_t nh, size_t nkv, size_t hd, size_t window, int32_t* out, int threads);
// RoPE inverse frequencies before each of `half` pairs (ops.rs:184-195).
int orc_rope_inv_frequencies(int64_t base, size_t freq_base_dim, size_t half, int64_t* out);

// ---- commitments (transformer_kernels.rs:1395-1482) ----
void orc_commit_activation_rows(const int32_t* rows, size_t n_rows, size_t width, char out_hex[65]);
void orc_commit_vector(const int32_t* v, size_t n, char out_hex[65]);

// ---- model + routines ----
typedef struct orc_model orc_model;
int orc_model_create(const orc_text_config* cfg, orc_model** out);
// elem_width 16/32: canonical Wgt bits. elem_width 8: int8 q with per-row
// integer scale (rank 2, or rank 1 treated as one row); expanded to
// q*scale exactly, the way a detwgt v2 converter would store it.
int orc_model_set_tensor(orc_model* m, const char* name, size_t rank, const uint64_t* dims,
                         int elem_width, const void* data, const int32_t* row_scale);
int orc_model_load_detwgt(orc_model* m, const uint8_t* bytes, size_t len);
int orc_model_finalize(orc_model* m);
void orc_model_free(orc_model* m);
void orc_set_threads(int threads);
/* Token rows per slab work item (default 1, the reference's schedule); more
 * read each weight row once per group. Results are identical for any value. */
void orc_set_slab_group(int tokens);

// Runs the det_goldens capture (src/runtime/det_goldens.rs:90-185) for the
// given prompt ids and writes it as compact JSON into `out` (NUL-terminated).
int orc_capture(orc_model* m, const uint32_t* prompt, size_t prompt_len, size_t decode_steps,
                char* out, size_t out_cap);

// The commitments of the native deterministic routines' checkpoints as JSON:
// prefill embedding, per layer its output rows, its token ranges of width
// prefill_width (0 = one range) and the caches up to it; final hidden,
// logits, caches; then per greedy step the token, every layer's output, the
// effective caches at the end of each layer range of width decode_width
// (0 = one range), and the logits.
int orc_trace_capture(orc_model* m, const uint32_t* prompt, size_t prompt_len, size_t decode_steps,
                      size_t prefill_width, size_t decode_width, char* out, size_t out_cap);

// Stateful session for timing / incremental checks.
typedef struct orc_session orc_session;
int orc_session_prefill(orc_model* m, const uint32_t* prompt, size_t prompt_len,
                        orc_session** out, int32_t* logits_out);
int orc_session_decode(orc_session* s, uint32_t token, int32_t* logits_out, int32_t* hidden_out);
/* An independent copy of a session (its caches, position and last logits). */
int orc_session_clone(const orc_session* src, orc_session** out);
void orc_session_free(orc_session* s);

#ifdef __cplusplus
}
#endif
