/*
 * detgpu — C ABI of the MI355X-native deterministic integer transformer path.
 *
 * This is the drop-in boundary for raster-inference's native deterministic
 * executor: a GPU executor beside src/runtime/executors/native.rs binds these
 * entry points through FFI and keeps the reference's routine / checkpoint
 * contract (src/routines/{prefill_range,decode_layer_range,prefill_finalize,
 * decode_transition_finalize}/native) and the detwgt v2 weight format.
 *
 * Conventions
 *  - Every function returns int status: 0 ok, 1 invalid argument / shape
 *    mismatch / missing weight (the reference's anyhow::bail!), 2 contract
 *    violation (the reference's det_num assert! panics), 3 runtime / HIP
 *    error. No C++ exception crosses this boundary; det_ctx_last_error()
 *    returns the message of the last failure on that context.
 *  - Pointers named *_dev are device pointers (allocate with
 *    det_device_alloc or any HIP allocation on the context's device); all
 *    other pointers are host pointers.
 *  - One context owns one HIP stream. Calls on one context are serialized by
 *    the caller; distinct contexts are independent. Work is enqueued on the
 *    context stream; functions that return host data synchronize it.
 *  - Values are canonical det_num bit patterns: Act/Wgt = Q16.16 in int32,
 *    Acc = Q32.32 in int64 (src/shared/numerics/det_num/types.rs:8-25).
 */
#ifndef DETGPU_H
#define DETGPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct det_ctx det_ctx_t;
typedef struct det_matrix det_matrix_t;
typedef struct det_model det_model_t;
typedef struct det_session det_session_t;
typedef struct det_event det_event_t;
typedef struct det_graph det_graph_t;
typedef struct det_kv det_kv_t;
typedef struct det_scratch det_scratch_t;

/* ------------------------------------------------------------------------ */
/* Context, memory, timing                                                   */
/* ------------------------------------------------------------------------ */
int det_ctx_create(int device, det_ctx_t** out);
void det_ctx_destroy(det_ctx_t* ctx);
const char* det_ctx_last_error(const det_ctx_t* ctx);
int det_ctx_synchronize(det_ctx_t* ctx);
/* Library build string (kernel ISA, version). */
const char* det_version(void);

int det_device_alloc(det_ctx_t* ctx, size_t bytes, void** out_dev);
int det_device_free(det_ctx_t* ctx, void* dev);
int det_memcpy_h2d(det_ctx_t* ctx, void* dst_dev, const void* src, size_t bytes);
int det_memcpy_d2h(det_ctx_t* ctx, void* dst, const void* src_dev, size_t bytes);
int det_memcpy_d2d(det_ctx_t* ctx, void* dst_dev, const void* src_dev, size_t bytes);

/* HIP events recorded on the context stream (for timing the hot kernels). */
int det_event_create(det_ctx_t* ctx, det_event_t** out);
int det_event_record(det_ctx_t* ctx, det_event_t* ev);
int det_event_elapsed_ms(det_ctx_t* ctx, det_event_t* start, det_event_t* stop, float* ms);
void det_event_destroy(det_event_t* ev);

/* A fixed sequence of calls on the context stream, recorded once and replayed
   as one HIP graph (no counterpart in the reference: for callers that issue
   the same short kernels repeatedly, where the per-call host launch cost
   would exceed the GPU time). Between begin and end the calls are recorded,
   not run; only calls that allocate nothing and do not synchronize may be
   recorded (run each once beforehand so that their scratch exists; a call
   whose scratch would grow is refused), and the buffers they name must
   outlive the graph. A failed or refused call ends the capture and discards
   what was recorded; det_ctx_capture_end then reports that no capture is in
   progress. */
int det_ctx_capture_begin(det_ctx_t* ctx);
int det_ctx_capture_end(det_ctx_t* ctx, det_graph_t** out);
int det_graph_launch(det_ctx_t* ctx, det_graph_t* g);
void det_graph_destroy(det_graph_t* g);

/* ------------------------------------------------------------------------ */
/* Weights: DetNumMatrix (src/shared/model/transformer.rs:194-198)            */
/* ------------------------------------------------------------------------ */
/* Storage after upload (det_matrix_info): */
#define DET_STORAGE_INT8 8   /* int8 q with per-row integer scale: W = q * s exactly */
#define DET_STORAGE_I16 16   /* Wgt bits of int16 range (detwgt v2 i16) that do not factor */
#define DET_STORAGE_I32 32   /* Wgt bits of int32 range (detwgt v2 i32) that do not factor */

/* Uploads a rows x cols row-major weight matrix.
 *  elem_width 8 : `values` is int8 q, `row_scale` int32[rows] (W = q*s);
 *  elem_width 16/32 : `values` are detwgt v2 Wgt bits (row_scale ignored);
 *                     rows are stored as int8 x scale whenever that
 *                     factorization is exact for the whole matrix. Else
 *                     each row is held as s * sum_p 256^p d_p with int8
 *                     digits d_p (balanced, in [-128, 127]) and s = +1 or -1:
 *                     two digit planes when every row fits them (i16 data
 *                     without rows that hold values near both ends of the
 *                     range), four otherwise. Every GEMV and GEMM then runs
 *                     on the int8 MFMA path (the planes' products combine
 *                     with shifts, exactly). Rows longer than 130000 columns
 *                     are stored as the Wgt bits (vector-ALU path).
 * Rejects matrices whose max row mass sum_c |W[r][c]| >= 2^31
 * (det_num/mod.rs:39-42, gemma/io.rs:327-335). */
int det_matrix_upload(det_ctx_t* ctx, uint64_t rows, uint64_t cols, int elem_width, const void* values,
                      const int32_t* row_scale, det_matrix_t** out);
int det_matrix_info(const det_matrix_t* m, uint64_t* rows, uint64_t* cols, int* storage);
void det_matrix_free(det_matrix_t* m);

/* ------------------------------------------------------------------------ */
/* Primitive ops (device pointers, enqueued on the context stream)           */
/* ------------------------------------------------------------------------ */
/* det_linear_into / det_linear_into_par (det_kernels.rs:108-178):
 * out[r] = requantize(sum_c act[c] * W[r][c]) with wrapping i64 MAC. */
int det_linear(det_ctx_t* ctx, const det_matrix_t* w, const int32_t* act_dev, int32_t* out_dev);
/* Raw wrapped Q32.32 accumulators (before requantize), for split-K
 * combination by wrapping i64 addition (det_num/ops.rs:23-30). */
int det_linear_acc_i64(det_ctx_t* ctx, const det_matrix_t* w, const int32_t* act_dev, int64_t* acc_dev);
/* det_linear_slab (det_kernels.rs:180-203): m token rows, act [m][cols] -> out [m][rows]. */
int det_linear_slab(det_ctx_t* ctx, const det_matrix_t* w, uint64_t m, const int32_t* act_dev, int32_t* out_dev);

/* rms_norm_in_place / value_rms_norm_in_place per row (det_num/ops.rs:95-131);
 * weight_dev NULL selects the value norm. */
int det_rms_norm(det_ctx_t* ctx, int32_t* x_dev, uint64_t rows, uint64_t cols, const int32_t* weight_dev,
                 int64_t eps_acc);
/* rope_rotate_pairs_in_place over rows x heads of head_dim (det_num/ops.rs:151-196);
 * row r uses position pos0 + r * pos_step. */
int det_rope(det_ctx_t* ctx, int32_t* x_dev, uint64_t rows, uint64_t heads, uint64_t head_dim, uint64_t rotary_dim,
             uint64_t freq_base_dim, int64_t base_acc, uint64_t pos0, uint64_t pos_step);
/* attention_output_into for every (head, query) (det_kernels.rs:340-367, 525-651):
 * q [n_queries][num_heads*head_dim], k/v [n_rows][num_kv_heads*head_dim],
 * causal rows [max(0, t+1-window), t+1) (window 0 = unbounded),
 * out [n_queries][num_heads*head_dim]. */
int det_attention_causal(det_ctx_t* ctx, const int32_t* q_dev, const int32_t* k_dev, const int32_t* v_dev,
                         uint64_t n_queries, uint64_t n_rows, uint64_t num_heads, uint64_t num_kv_heads,
                         uint64_t head_dim, uint64_t window, int32_t* out_dev);
/* argmax_first (det_num/ops.rs:463-478); result written to *index (host). */
int det_argmax_first(det_ctx_t* ctx, const int32_t* x_dev, uint64_t n, uint32_t* index);
/* No counterpart in the reference: det_argmax_first for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops). It allocates
 * and frees nothing, does not synchronize, and writes the index to the device
 * word *index_dev. Its partial results live in a fixed per-GPU array sized for
 * n <= 16777216 (larger n is rejected, status 1). All calls on one GPU share
 * that array: calls that overlap on one GPU (other streams, other contexts)
 * race and must be ordered by the caller. */
int det_argmax_first_noalloc(det_ctx_t* ctx, const int32_t* x_dev, uint64_t n, uint32_t* index_dev);
/* Elementwise saturating ops (det_kernels.rs:252-282, det_num/ops.rs:33-47, 377-403). */
#define DET_EW_ADD 0      /* x = add_sat(x, y) */
#define DET_EW_GELU_MUL 1 /* x = mul_sat(gelu_pytorch_tanh(x), y) */
#define DET_EW_SCALE 2    /* x = scale_act(x, scalar) */
#define DET_EW_SOFTCAP 3  /* x = softcap_act(x, scalar) */
int det_elementwise(det_ctx_t* ctx, int op, int32_t* x_dev, const int32_t* y_dev, uint64_t n, int32_t scalar);

/* ------------------------------------------------------------------------ */
/* Model: Gemma4TransformerModel in det mode (gemma/io.rs:1043-1123)         */
/* ------------------------------------------------------------------------ */
/* Raw config.json text_config (GemmaTextConfigFile, gemma/io.rs:60-96);
 * has_* flags mark Option<...> fields that were present. */
typedef struct det_text_config {
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
  const int32_t* layer_types; /* 1 = "sliding_attention", 0 = any other type */
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
  int32_t bidirectional_all; /* use_bidirectional_attention == "all" */
} det_text_config_t;

int det_model_create(det_ctx_t* ctx, const det_text_config_t* cfg, det_model_t** out);
/* Adds one named tensor (names as in gemma/io.rs, e.g.
 * "model.language_model.layers.0.self_attn.q_proj.weight"). rank 1 or 2;
 * elem_width 8 (+row_scale), 16 or 32 as in det_matrix_upload. */
int det_model_set_tensor(det_model_t* model, const char* name, uint64_t rank, const uint64_t* dims, int elem_width,
                         const void* values, const int32_t* row_scale);
/* Parses a whole detwgt v2 artifact with the fail-closed checks of
 * DetNumTensorReader::load_artifact (gemma/io.rs:224-387). Also accepts the
 * int8 variant detwgt-q8 (magic "DNWGTQ8\0", version 1; no reference
 * counterpart): the same records, where a rank >= 2 tensor may be stored at
 * element_width 8 as int8 q followed by a u64 scale count (= rows), a
 * 64-byte aligned int8 payload and a 64-byte aligned i32 scale per row
 * (W = q * s, which must fit i32). Written by rasterdet.detwgt. */
int det_model_load_detwgt(det_model_t* model, const uint8_t* bytes, size_t len);
/* Resolves layers exactly like load_det_num_gemma4_layer_weights (gemma/io.rs:1896-2045). */
int det_model_finalize(det_model_t* model);
/* 1 when the model's decode steps run the graph-captured fused step (int8
 * matrices whose shapes fit its kernels, with or without per-layer inputs),
 * 0 when they run one kernel sequence per operation, -1 before finalize. No
 * counterpart in the reference (its executor has one CPU path); for callers
 * and tests that need to know which GPU schedule a model takes. */
int det_model_fused_decode(const det_model_t* model);
/* Sessions, KV caches and scratches may be freed before or after their model
 * (they keep their own device memory and the context's stream); the context
 * must outlive all of them, and a model must not be freed while a call on one
 * of its sessions, caches or scratches is running. */
void det_model_free(det_model_t* model);

/* ------------------------------------------------------------------------ */
/* Layer-level operators: the reference's det_kernels.rs API                 */
/* ------------------------------------------------------------------------ */
/* These are the functions the routines' native deterministic tiles call per
 * layer (prefill_range/native/deterministic_tiles.rs:69-199,
 * decode_layer_range/native/tiles.rs:133-197), so an executor can run any
 * layer range and emit its own checkpoints between layers. Activations are
 * device buffers of Q16.16 int32 rows of the model's hidden width; work is
 * enqueued on the model context's stream. */

/* Reusable row buffers (DetDecodeScratch, det_kernels.rs:830-864), grown on
 * demand; one scratch serves one caller at a time. det_layer_prefill
 * allocates its scratch per call in the reference and takes one here. */
int det_scratch_create(det_model_t* model, det_scratch_t** out);
void det_scratch_free(det_scratch_t* scratch);

/* LayerKvCache of one layer (shared/model/transformer.rs:278-337) with room
 * for max_tokens appended tokens; a sliding-window layer that owns its cache
 * keeps its last `window` rows. Starts without det data (None). A prefill of
 * more than max_tokens rows, or an append past max_tokens tokens, fails with
 * "KV cache capacity exceeded" (status 1), except on a sliding-window cache
 * created with max_tokens >= window, which keeps taking tokens as the
 * reference's trimmed cache does. */
int det_kv_create(det_model_t* model, uint64_t layer, uint64_t max_tokens, det_kv_t** out);
/* LayerKvCache::clone (e.g. to keep the pre-step caches a decode.layer_range
 * commitment needs). */
int det_kv_clone(const det_kv_t* src, det_kv_t** out);
void det_kv_free(det_kv_t* kv);
/* current_len, head count, head dim, and whether det data is present. */
int det_kv_info(const det_kv_t* kv, uint64_t* len, uint64_t* heads, uint64_t* head_dim, int32_t* has_det);
/* DetKvCacheData's rows in logical order (det_tensor.rs:147-397): keys and
 * values host [heads][len][head_dim]; capacity = values each buffer holds. */
int det_kv_read_logical(const det_kv_t* kv, int32_t* keys, int32_t* values, uint64_t capacity);
/* build_det_kv_cache_commitment (transformer_kernels.rs:1460-1482) over
 * caches[0..n) in order: *is_some = 0 and out = "" when one lacks det data. */
int det_kv_commitment(const det_kv_t* const* caches, uint64_t n, char out[65], int32_t* is_some);

/* decode_embedding_rows_for_token_ids_from_det_num + scale_act_row
 * (gemma/io.rs:2446-2518): out [n][hidden]. */
int det_embed_tokens(det_model_t* model, det_scratch_t* scratch, const uint32_t* ids, uint64_t n, int32_t* out_dev);
/* compute_prefill_ple_inputs_det for one layer
 * (prefill_prepare_aux/native/tiles.rs:111-240): out [n][ple_dim] from the
 * token ids and the embedded rows input [n][hidden]; *produced = 0 (output
 * untouched) when the layer has no per-layer input. */
int det_prefill_ple_inputs(det_model_t* model, det_scratch_t* scratch, uint64_t layer, const uint32_t* ids, uint64_t n,
                           const int32_t* input_dev, int32_t* out_dev, int32_t* produced);
/* det_decode_ple_input (det_kernels.rs:1142-1150): the same for one token. */
int det_decode_ple_input(det_model_t* model, det_scratch_t* scratch, uint32_t token, const int32_t* input_dev,
                         uint64_t layer, int32_t* output_dev, int32_t* produced);
/* det_layer_prefill (det_kernels.rs:678-683): xs [n][hidden] at positions
 * 0..n-1 -> out [n][hidden] (may equal xs). per_layer_input [n][ple_dim] or
 * NULL. With donor == NULL, `cache` (this layer's handle) receives the new
 * cache (DetKvCacheData::from_head_slabs); with a donor, attention reads the
 * donor's cache and `cache` (may be NULL) is left as it was, as the
 * reference returns no cache. */
int det_layer_prefill(det_model_t* model, det_scratch_t* scratch, uint64_t layer, const int32_t* xs_dev, uint64_t n,
                      const int32_t* per_layer_input_dev, const det_kv_t* donor, det_kv_t* cache, int32_t* out_dev);
/* det_layer_decode (det_kernels.rs:866-875): one row at `position`. Without a
 * donor the token's K/V row is appended to `cache` (with the sliding-window
 * trim); with a donor (already updated for this step) attention reads it. */
int det_layer_decode(det_model_t* model, det_scratch_t* scratch, uint64_t layer, const int32_t* input_dev,
                     const int32_t* per_layer_input_dev, det_kv_t* cache, const det_kv_t* donor, uint64_t position,
                     int32_t* output_dev);
/* det_hidden_to_logits (det_kernels.rs:1217-1225): final norm, the lm_head or
 * tied embedding projection, optional softcap; logits [vocab]. */
int det_hidden_to_logits(det_model_t* model, det_scratch_t* scratch, const int32_t* hidden_dev, int32_t* logits_dev);

/* ------------------------------------------------------------------------ */
/* Sessions: the prefill_layer / decode_transition routines on the GPU        */
/* ------------------------------------------------------------------------ */
/* A session owns one sequence's KV caches (LayerKvCache per layer) sized for
 * max_tokens positions, plus device scratch. */
int det_session_create(det_model_t* model, uint64_t max_tokens, det_session_t** out);
int det_session_clone(const det_session_t* src, det_session_t** out);
void det_session_free(det_session_t* s);

/* Commitments are lowercase hex SHA-256 strings (65 bytes incl. NUL) built
 * exactly like build_det_*_commitment (transformer_kernels.rs:1395-1482);
 * kv is "" when the reference would return None (a layer without det data). */
typedef struct det_prefill_result {
  char embedding[65];    /* input.embedding det_activations_sha256 */
  char final_hidden[65]; /* prefill final_hidden_states det commitment */
  char logits[65];       /* det_final_logits_sha256 (vector commitment) */
  char kv[65];           /* build_det_kv_cache_commitment of all layer caches */
  uint32_t next_token;   /* argmax_first of the logits (greedy selection) */
} det_prefill_result_t;

typedef struct det_decode_result {
  char activation[65]; /* decode activation_state det commitment */
  char logits[65];
  char kv[65];
  uint32_t next_token;
} det_decode_result_t;

/* Flags for prefill/decode: which commitments to compute on the host. */
#define DET_COMMIT_NONE 0u
#define DET_COMMIT_ACTIVATIONS 1u /* embedding / hidden / activation / logits */
#define DET_COMMIT_KV 2u          /* KV cache commitment */
#define DET_COMMIT_ALL 3u
/* Decode flag: run the per-operation kernel sequence instead of the fused,
 * graph-captured decode step (both are bit-identical; for cross-checks). */
#define DET_DECODE_PER_OP 0x100u
/* Decode flag: launch the fused step's kernels directly on the stream
 * instead of replaying the captured graph (same kernels, same results). */
#define DET_DECODE_EAGER 0x200u

/* pipeline::run_prefill_pass_with_mode (runtime/pipeline.rs:55-98): embedding,
 * PLE inputs, every prefill_layer, prefill_finalize logits. */
int det_session_prefill(det_session_t* s, const uint32_t* token_ids, uint64_t n, uint32_t flags,
                        det_prefill_result_t* out);
/* pipeline::decode_step_with_mode (runtime/pipeline.rs:165-216): embed token,
 * every decode_transition layer with in-place KV append, finalize logits. */
int det_session_decode(det_session_t* s, uint32_t token, uint32_t flags, det_decode_result_t* out);
/* One decode_step (runtime/pipeline.rs:165-216, as det_session_decode) for
 * each of n distinct sessions of one model, in shared launches: every
 * projection runs once over the n activation rows (M = n) and attention reads
 * each session's own ragged cache window. tokens[i] feeds sessions[i] and
 * out[i] (may be NULL) receives its result. Each session's next token, logits,
 * caches and commitments are bit-identical to det_session_decode of that
 * session alone. The reference decodes one sequence per call; this entry point
 * batches those calls and has no other behaviour. */
int det_session_decode_batch(det_session_t* const* sessions, uint64_t n, const uint32_t* tokens, uint32_t flags,
                             det_decode_result_t* out);
/* Copies the last logits (vocab int32) to host. */
int det_session_logits(det_session_t* s, int32_t* out, uint64_t n);
int det_session_position(const det_session_t* s, uint64_t* position);

/* Runs the det_goldens capture protocol (src/runtime/det_goldens.rs:90-185)
 * and writes it as compact JSON into out (NUL-terminated). */
int det_capture(det_model_t* model, const uint32_t* prompt, uint64_t prompt_len, uint64_t decode_steps, char* out,
                size_t out_cap);

/* ------------------------------------------------------------------------ */
/* Checkpoint trace (runtime/trace.rs, runtime/sequence.rs)                  */
/* ------------------------------------------------------------------------ */
/* SamplingConfig (src/shared/api/input.rs:45-50); has_* = Some(..). */
typedef struct det_sampling {
  int32_t has_max_new_tokens;
  uint64_t max_new_tokens;
  int32_t has_temperature;
  float temperature;
  int32_t has_top_k;
  uint64_t top_k;
  int32_t has_top_p;
  float top_p;
} det_sampling_t;

/* Text of generated token ids (the tokenizer's decode with special tokens
 * skipped, output_finalize/native/tiles.rs:5-13). Writes up to cap bytes of
 * UTF-8 plus a NUL into out and returns the text length; a length >= cap asks
 * for a call with a larger buffer; a negative value is a failure. */
typedef int64_t (*det_detokenize_fn)(const uint32_t* ids, uint64_t n, char* out, size_t cap, void* user);

typedef struct det_trace_request {
  const char* prompt_text;          /* prompt.prepare's decoded prompt text (UTF-8) */
  const uint32_t* prompt_token_ids; /* the rendered prompt's token ids (prompt_prepare::tokenize_prompt) */
  uint64_t prompt_token_count;
  det_sampling_t sampling;          /* max_new_tokens (None = 0); temperature must be 1, no top_k / top_p */
  int32_t prompt_checkpoint;        /* emit prompt.prepare (det runs with an authenticated tokenizer source) */
  const char* terminal_checkpoint;  /* NULL, "checkpoint" or "checkpoint:occurrence" */
  uint64_t prefill_token_range_width; /* 0 = unbounded (InferenceControls default) */
  uint64_t decode_layer_range_width;  /* 0 = unbounded */
  det_detokenize_fn detokenize;     /* needed once a token is generated */
  void* detokenize_user;
} det_trace_request_t;

/* Runs the native deterministic sequence with checkpoint commitment
 * (runtime/sequence.rs; runtime/executors/native.rs:60-450): prompt.prepare,
 * input.embedding, prefill.prepare_aux, prefill.range / prefill.range_finalize
 * per layer, prefill.finalize, then per generated token decode.select_token,
 * decode.layer_range(s) and decode.transition_finalize, and output.finalize.
 * Writes the checkpoint trace artifact (serde_json pretty array of
 * {checkpoint: sha256(payload)}, runtime/trace.rs:262-330, 555-566) plus a
 * NUL into out; *out_len is its length. *paused = 1 when the terminal
 * checkpoint was reached. On an error the artifact of the checkpoints so far is
 * still written (abort_inference_trace) and the status is nonzero. */
int det_trace_run(det_model_t* model, const det_trace_request_t* request, char* out, size_t out_cap, size_t* out_len,
                  int32_t* paused);

/* ------------------------------------------------------------------------ */
/* Challenger audit (runtime/roles/challenger.rs, shared/api/audit.rs)       */
/* ------------------------------------------------------------------------ */
/* Audit outcomes are written as compact JSON plus a NUL into out (*out_len =
 * its length; *diverged = 1 on a divergence):
 *   {"diverged":false}                                  AuditOutcome::NoDivergence
 *   {"diverged":true,"divergence":{...},"detour":S}     AuditOutcome::Diverged
 * The divergence object is CheckpointDivergence (audit.rs:85-110) in its
 * serde form: entry_index, checkpoint_id, occurrence, then whichever of
 * claimed_checkpoint_id, claimed_commitment, replayed_commitment are set. S is
 * the --raster-at spec of the divergent routine occurrence
 * (challenger.rs:185-210) or null for a structural divergence or a routine
 * without a raster detour; running that detour is the raster executor's job.
 * A claimed trace that is not a JSON array of single-key
 * {"checkpoint": "commitment"} objects is an error (ClaimedTrace,
 * audit.rs:34-82). */

/* locate_first_divergence (challenger.rs:136-183) between two serialized
 * trace artifacts. Host only: no device work. */
int det_trace_locate_divergence(const char* claimed, size_t claimed_len, const char* replayed, size_t replayed_len,
                                char* out, size_t out_cap, size_t* out_len, int32_t* diverged);

/* challenger::audit (challenger.rs:55-113): parses the claimed trace, replays
 * the request on the GPU under the claimer policy (claimer.rs:34-61: commitment
 * on, prompt_checkpoint set, no terminal checkpoint, unbounded ranges; other
 * control settings are refused) and locates the first divergence. */
int det_audit_trace(det_model_t* model, const det_trace_request_t* request, const char* claimed, size_t claimed_len,
                    char* out, size_t out_cap, size_t* out_len, int32_t* diverged);

/* ------------------------------------------------------------------------ */
/* Synthetic workloads (no reference counterpart; random-init benchmarks)    */
/* ------------------------------------------------------------------------ */
/* Fills q[rows*cols] and s[rows] with counter-hash weights: q in [-127, 127],
 * s in [1, scale_max]. Host memory; multi-threaded. Same definition as
 * rasterdet.synthetic.fast_int8_matrix. */
int det_synthetic_int8(uint64_t seed, uint64_t rows, uint64_t cols, int32_t scale_max, int8_t* q, int32_t* s);
/* Counter-hash i16 Wgt bits uniform in [-lim, lim] that do not factor into
 * int8 x scale (column 0 holds 1; every 7th row holds 32767 and rows 3 mod 11
 * not among them hold -32768, at hashed columns): the benchmark's i16 model
 * weights, multi-threaded. No reference counterpart (synthetic data). */
int det_synthetic_i16(uint64_t seed, uint64_t rows, uint64_t cols, int32_t lim, int16_t* w);

#ifdef __cplusplus
}
#endif

#endif /* DETGPU_H */
