// ORACLE — test infrastructure only (see oracle.h). CPU restatement of:
//   src/shared/numerics/det_kernels.rs        (GEMV/GEMM, attention, layers, PLE, logits)
//   src/shared/numerics/det_tensor.rs:147-397 (ActHeadBuf / DetKvCacheData)
//   src/shared/numerics/transformer_kernels.rs:1395-1482 (commitments)
//   src/shared/model/gemma/io.rs:60-190, 224-387, 1043-1234, 1896-2045, 2118-2132, 2446-2518
//   src/routines/{prefill_range,decode_layer_range,prefill_prepare_aux,
//                 prefill_finalize,decode_transition_finalize}/native/*
//   src/runtime/det_goldens.rs:90-236 (the capture protocol)
// Serial reference order everywhere; the optional thread count only splits
// GEMV output rows (det_kernels.rs:156-178), which cannot change any bit.
#include <openssl/sha.h>
#include <omp.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <functional>
#include <map>
#include <memory>
#include <optional>
#include <string>
#include <vector>

#include "det_num.h"
#include "oracle.h"

namespace oracle {

static thread_local std::string g_last_error;
static int g_threads = 1;
// Token rows per slab work item: 1 is the reference's schedule (one serial
// GEMV per token row). Tests may take several token rows per item, each
// weight row then read once for the group while it is in cache; every output
// element still adds its terms in column order, so the results are the same.
static int g_slab_group = 1;

struct InvalidArgument : std::runtime_error {
  using std::runtime_error::runtime_error;
};
[[noreturn]] static void bail(const std::string& msg) { throw InvalidArgument(msg); }

// ---------------------------------------------------------------------------
// Weight matrices (DetNumMatrix, shared/model/transformer.rs:194-198)
// ---------------------------------------------------------------------------
struct Matrix {
  size_t rows = 0, cols = 0;
  int width = 32;
  std::vector<int16_t> w16;
  std::vector<int32_t> w32;
  int32_t at(size_t i) const { return width == 16 ? int32_t(w16[i]) : w32[i]; }
};

template <class T>
static void gemv_rows(const T* w, size_t cols, const int32_t* act, size_t r0, size_t r1,
                      int32_t* out) {
  // det_kernels.rs:108-134: one wrapping-MAC reduction + requantize per row.
  for (size_t r = r0; r < r1; ++r) {
    const T* row = w + r * cols;
    int64_t acc = 0;
    for (size_t c = 0; c < cols; ++c) acc = mac_bits(acc, act[c], int32_t(row[c]));
    out[r] = requantize(acc);
  }
}

template <class T>
static void gemv_dispatch(const T* w, size_t rows, size_t cols, const int32_t* act, int32_t* out,
                          int threads) {
  // det_kernels.rs:156-178: serial below 128 rows or with one thread; else
  // contiguous chunks of max(64, ceil(rows/threads)) rows.
  if (threads <= 1 || rows < 128) {
    gemv_rows(w, cols, act, 0, rows, out);
    return;
  }
  const size_t chunk = std::max<size_t>(64, (rows + threads - 1) / threads);
  const long n_chunks = long((rows + chunk - 1) / chunk);
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
  for (long c = 0; c < n_chunks; ++c) {
    const size_t r0 = size_t(c) * chunk;
    gemv_rows(w, cols, act, r0, std::min(rows, r0 + chunk), out);
  }
}

static void det_linear(const Matrix& W, const int32_t* act, size_t act_len, int32_t* out) {
  if (act_len != W.cols)
    bail("deterministic linear input width mismatch: " + std::to_string(act_len) + " vs " +
         std::to_string(W.cols));
  if (W.width == 16) gemv_dispatch(W.w16.data(), W.rows, W.cols, act, out, g_threads);
  else gemv_dispatch(W.w32.data(), W.rows, W.cols, act, out, g_threads);
}

// det_kernels.rs:180-203 det_linear_slab: each token row is an independent
// serial GEMV (det_linear_into); with a thread pool the token rows are spread
// over the threads (par_chunks_mut over output rows), never the matrix rows.
template <class T>
static void slab_group(const T* w, size_t rows, size_t cols, size_t t0, size_t t1, const int32_t* act,
                       int32_t* out) {
  for (size_t r = 0; r < rows; ++r) {
    const T* row = w + r * cols;
    for (size_t t = t0; t < t1; ++t) {
      const int32_t* a = act + t * cols;
      int64_t acc = 0;
      for (size_t c = 0; c < cols; ++c) acc = mac_bits(acc, a[c], int32_t(row[c]));
      out[t * rows + r] = requantize(acc);
    }
  }
}

template <class T>
static void slab_rows(const T* w, size_t rows, size_t cols, size_t m, const int32_t* act, int32_t* out,
                      int threads) {
  if (g_slab_group > 1 && m > 1) {
    const size_t G = size_t(g_slab_group);
    const long groups = long((m + G - 1) / G);
#pragma omp parallel for num_threads(threads > 1 ? threads : 1) schedule(dynamic, 1)
    for (long g = 0; g < groups; ++g)
      slab_group(w, rows, cols, size_t(g) * G, std::min(m, size_t(g + 1) * G), act, out);
    return;
  }
  if (threads <= 1 || m <= 1) {
    for (size_t t = 0; t < m; ++t) gemv_rows(w, cols, act + t * cols, 0, rows, out + t * rows);
    return;
  }
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
  for (long t = 0; t < long(m); ++t) gemv_rows(w, cols, act + size_t(t) * cols, 0, rows, out + size_t(t) * rows);
}

static std::vector<int32_t> det_linear_slab(const std::vector<int32_t>& in, size_t m, size_t k,
                                            const Matrix& W) {
  if (k != W.cols)
    bail("deterministic linear input row 0 has width " + std::to_string(k) + ", expected " +
         std::to_string(W.cols));
  std::vector<int32_t> out(m * W.rows);
  if (W.width == 16) slab_rows(W.w16.data(), W.rows, W.cols, m, in.data(), out.data(), g_threads);
  else slab_rows(W.w32.data(), W.rows, W.cols, m, in.data(), out.data(), g_threads);
  return out;
}

// ---------------------------------------------------------------------------
// KV cache (det_tensor.rs:147-397; LayerKvCache transformer.rs:278-340)
// ---------------------------------------------------------------------------
struct HeadBuf {
  std::vector<int32_t> data;
  size_t cols = 0, start_row = 0, len_rows = 0;
  void push_row(const int32_t* row, size_t n) {
    if (len_rows == 0 && data.empty()) { cols = n; start_row = 0; }
    data.insert(data.end(), row, row + n);
    ++len_rows;
  }
  void pop_front_row() {
    ++start_row;
    --len_rows;
    if (start_row > len_rows) {  // compaction is unobservable; kept for fidelity
      std::memmove(data.data(), data.data() + start_row * cols, len_rows * cols * sizeof(int32_t));
      data.resize(len_rows * cols);
      start_row = 0;
    }
  }
  const int32_t* rows_window(size_t start) const { return data.data() + (start_row + start) * cols; }
};

struct KvData {
  std::vector<HeadBuf> keys, values;
  KvData() = default;
  KvData(size_t heads, size_t head_dim) : keys(heads), values(heads) {
    for (auto& h : keys) h.cols = head_dim;
    for (auto& h : values) h.cols = head_dim;
  }
  size_t len() const { return keys.empty() ? 0 : keys[0].len_rows; }
  void append_rows(const int32_t* k, const int32_t* v, size_t head_dim,
                   std::optional<size_t> window) {
    for (size_t h = 0; h < keys.size(); ++h) {
      keys[h].push_row(k + h * head_dim, head_dim);
      values[h].push_row(v + h * head_dim, head_dim);
      if (window) {
        while (keys[h].len_rows > *window) {
          keys[h].pop_front_row();
          values[h].pop_front_row();
        }
      }
    }
  }
};

struct LayerCache {
  size_t num_kv_heads = 0;
  std::optional<KvData> det;
  size_t current_len() const { return det ? det->len() : 0; }
};

// ---------------------------------------------------------------------------
// Commitments (transformer_kernels.rs:1395-1482)
// ---------------------------------------------------------------------------
struct Hasher {
  SHA256_CTX ctx;
  Hasher() { SHA256_Init(&ctx); }
  void bytes(const void* p, size_t n) { SHA256_Update(&ctx, p, n); }
  void u64(uint64_t v) { uint8_t b[8]; for (int i = 0; i < 8; ++i) b[i] = uint8_t(v >> (8 * i)); bytes(b, 8); }
  // i32 values as little-endian bytes: the host's own layout on x86-64.
  void i32s(const int32_t* v, size_t n) {
    static_assert(__BYTE_ORDER__ == __ORDER_LITTLE_ENDIAN__, "commitments hash little-endian i32 bytes");
    bytes(v, n * 4);
  }
  std::string hex() {
    uint8_t d[32];
    SHA256_Final(d, &ctx);
    static const char* H = "0123456789abcdef";
    std::string s(64, '0');
    for (int i = 0; i < 32; ++i) { s[2 * i] = H[d[i] >> 4]; s[2 * i + 1] = H[d[i] & 15]; }
    return s;
  }
};

static std::string commit_rows(const int32_t* rows, size_t n_rows, size_t width) {
  Hasher h;  // build_det_activation_commitment{,_slab,_row}
  static const char kDom[] = "raster-det-num-act-v1";
  h.bytes(kDom, sizeof(kDom) - 1);
  h.u64(n_rows);
  for (size_t r = 0; r < n_rows; ++r) { h.u64(width); h.i32s(rows + r * width, width); }
  return h.hex();
}
static std::string commit_vector(const int32_t* v, size_t n) {
  Hasher h;  // build_det_vector_commitment
  static const char kDom[] = "raster-det-num-act-vector-v1";
  h.bytes(kDom, sizeof(kDom) - 1);
  h.u64(n);
  h.i32s(v, n);
  return h.hex();
}
static std::optional<std::string> commit_kv(const std::vector<const LayerCache*>& caches) {
  Hasher h;  // build_det_kv_cache_commitment: None when any layer lacks det data
  static const char kDom[] = "raster-det-num-kv-cache-v1";
  h.bytes(kDom, sizeof(kDom) - 1);
  h.u64(caches.size());
  for (const LayerCache* c : caches) {
    if (!c->det) return std::nullopt;
    const KvData& d = *c->det;
    h.u64(d.keys.size());
    const std::vector<HeadBuf>* sides[2] = {&d.keys, &d.values};
    const char kinds[2] = {'k', 'v'};
    for (int s = 0; s < 2; ++s) {
      h.bytes(&kinds[s], 1);
      h.u64(sides[s]->size());
      for (const HeadBuf& hb : *sides[s]) {
        h.u64(hb.len_rows);
        const size_t w = std::max<size_t>(hb.cols, 1);
        for (size_t r = 0; r < hb.len_rows; ++r) { h.u64(w); h.i32s(hb.rows_window(r), w); }
      }
    }
  }
  return h.hex();
}

// ---------------------------------------------------------------------------
// Model (Gemma4LayerWeights / Gemma4TransformerModel in det mode)
// ---------------------------------------------------------------------------
struct Tensor {
  std::vector<uint64_t> shape;
  Matrix m;  // rank-2: rows x cols; rank 1: 1 x n
};

struct Layer {
  bool sliding = false;
  size_t hidden = 0, num_heads = 0, num_kv_heads = 0, head_dim = 0;
  std::optional<size_t> sliding_window, cache_sliding_window, kv_shared_layer_index;
  int64_t eps = 0, rope_base = 0;
  size_t partial_rotary_dim = 0, rope_freq_base_dim = 0;
  bool k_eq_v = false;
  const Matrix *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr, *gate = nullptr,
               *up = nullptr, *down = nullptr;
  std::vector<int32_t> q_norm, k_norm, input_ln, post_attn_ln, pre_ff_ln, post_ff_ln;
  bool has_ple = false;
  const Matrix *ple_gate = nullptr, *ple_proj = nullptr;
  std::vector<int32_t> ple_post_norm;
  std::optional<int32_t> layer_scalar;
};

}  // namespace oracle

struct orc_model {
  orc_text_config cfg;
  std::vector<int32_t> layer_types;
  std::map<std::string, oracle::Tensor> tensors;
  bool finalized = false;
  // derived
  const oracle::Matrix* embedding = nullptr;
  int32_t embed_scale = 0;
  std::vector<oracle::Layer> layers;
  bool has_ple = false;
  size_t ple_dim = 0;
  std::vector<oracle::Matrix> ple_token_emb;  // per layer: ple_vocab x ple_dim
  std::vector<oracle::Matrix> ple_model_proj; // per layer: ple_dim x hidden
  std::vector<int32_t> ple_proj_norm;
  int32_t ple_embedding_scale = 0, ple_projection_scalar = 0, ple_input_scale = 0;
  std::vector<int32_t> final_norm;
  const oracle::Matrix* lm_head = nullptr;
  std::optional<int32_t> softcap;
  int64_t eps = 0;
  size_t hidden = 0;
};

namespace oracle {

static const Tensor& need(orc_model* m, const std::string& name) {
  auto it = m->tensors.find(name);
  if (it == m->tensors.end()) bail("missing tensor `" + name + "`");
  return it->second;
}
static const Matrix& need_matrix(orc_model* m, const std::string& name) {
  const Tensor& t = need(m, name);
  if (t.shape.size() != 2) bail("tensor `" + name + "` is not a matrix");
  return t.m;
}
static std::vector<int32_t> need_vector(orc_model* m, const std::string& name) {
  const Tensor& t = need(m, name);
  if (t.shape.size() != 1) bail("tensor `" + name + "` is not a vector");
  std::vector<int32_t> v(t.m.cols);
  for (size_t i = 0; i < v.size(); ++i) v[i] = t.m.at(i);
  return v;
}
static Matrix slice(const Matrix& src, size_t r0, size_t nr, size_t c0, size_t nc) {
  if (r0 + nr > src.rows || c0 + nc > src.cols) bail("matrix slice out of bounds");
  Matrix out;
  out.rows = nr; out.cols = nc; out.width = src.width;
  if (src.width == 16) out.w16.resize(nr * nc); else out.w32.resize(nr * nc);
  for (size_t r = 0; r < nr; ++r)
    for (size_t c = 0; c < nc; ++c) {
      const size_t si = (r0 + r) * src.cols + c0 + c;
      if (src.width == 16) out.w16[r * nc + c] = src.w16[si]; else out.w32[r * nc + c] = src.w32[si];
    }
  return out;
}

// gemma/io.rs:165-190
static std::optional<size_t> kv_shared_layer_index(const orc_model* m, size_t layer_idx) {
  const uint64_t nshared = m->cfg.has_num_kv_shared_layers ? m->cfg.num_kv_shared_layers : 0;
  const size_t L = m->cfg.num_hidden_layers;
  const size_t first_shared = L > nshared ? L - nshared : 0;
  if (nshared == 0 || layer_idx < first_shared) return std::nullopt;
  const int32_t ty = m->layer_types[layer_idx];
  for (size_t i = first_shared; i-- > 0;)
    if (m->layer_types[i] == ty) return i;
  bail("Gemma layer " + std::to_string(layer_idx) + " is configured to share KV without a prior donor layer");
}

static void finalize_model(orc_model* m) {
  const orc_text_config& c = m->cfg;
  if (c.enable_moe_block) bail("MoE checkpoints are not supported");
  if (!c.hidden_activation_is_gelu_pytorch_tanh) bail("only gelu_pytorch_tanh is supported");
  if (c.num_hidden_layers != m->layer_types.size()) bail("Gemma config layer count mismatch");
  m->hidden = c.hidden_size;
  m->eps = f32_to_acc(c.rms_norm_eps);

  // Embedding source (gemma/io.rs:44-48, 2118-2132).
  const char* embed_names[] = {"model.language_model.embed_tokens.weight",
                               "language_model.embed_tokens.weight", "embed_tokens.weight"};
  for (const char* n : embed_names) {
    auto it = m->tensors.find(n);
    if (it != m->tensors.end()) { m->embedding = &it->second.m; break; }
  }
  if (!m->embedding) bail("missing embedding tensor");
  if (m->embedding->cols != c.hidden_size) bail("embedding tensor width mismatch");
  m->embed_scale = f32_to_act(std::sqrt(float(m->embedding->cols)));

  // KV donors (gemma/io.rs:1071-1079).
  std::vector<bool> is_donor(c.num_hidden_layers, false);
  for (size_t l = 0; l < c.num_hidden_layers; ++l)
    if (auto d = kv_shared_layer_index(m, l)) is_donor[*d] = true;

  const bool k_eq_v_cfg = c.has_attention_k_eq_v && c.attention_k_eq_v;
  const size_t eff_window = c.bidirectional_all ? c.sliding_window / 2 + 1 : c.sliding_window;
  const size_t ple_dim = c.has_hidden_size_per_layer_input ? c.hidden_size_per_layer_input : 0;
  m->layers.resize(c.num_hidden_layers);
  for (size_t l = 0; l < c.num_hidden_layers; ++l) {
    // gemma/io.rs:1896-2045
    Layer& L = m->layers[l];
    const std::string p = "model.language_model.layers." + std::to_string(l);
    L.sliding = m->layer_types[l] == 1;
    L.head_dim = L.sliding ? c.head_dim : (c.has_global_head_dim ? c.global_head_dim : c.head_dim);
    if (L.sliding) L.num_kv_heads = c.num_key_value_heads;
    else if (k_eq_v_cfg)
      L.num_kv_heads = c.has_num_global_key_value_heads ? c.num_global_key_value_heads : c.num_key_value_heads;
    else L.num_kv_heads = c.num_key_value_heads;
    const float factor = c.has_full_partial_rotary_factor ? c.full_partial_rotary_factor : 0.25f;
    L.partial_rotary_dim = L.sliding ? L.head_dim : size_t(float(L.head_dim) * factor);
    L.kv_shared_layer_index = kv_shared_layer_index(m, l);
    if (L.sliding) L.sliding_window = eff_window;
    if (L.sliding && !is_donor[l]) L.cache_sliding_window = eff_window;
    float base;
    if (L.sliding) base = c.has_sliding_rope_theta ? c.sliding_rope_theta : 10000.0f;
    else base = c.has_full_rope_theta ? c.full_rope_theta : (c.has_rope_theta ? c.rope_theta : 1000000.0f);
    L.rope_base = f32_to_acc(base);
    L.rope_freq_base_dim = L.head_dim;
    L.hidden = c.hidden_size;
    L.num_heads = c.num_attention_heads;
    L.eps = m->eps;
    L.k_eq_v = !L.sliding && k_eq_v_cfg;
    L.q = &need_matrix(m, p + ".self_attn.q_proj.weight");
    L.k = &need_matrix(m, p + ".self_attn.k_proj.weight");
    const std::string vname = p + ".self_attn.v_proj.weight";
    if (L.k_eq_v) {
      if (m->tensors.count(vname)) L.v = &need_matrix(m, vname);
    } else {
      L.v = &need_matrix(m, vname);
    }
    L.o = &need_matrix(m, p + ".self_attn.o_proj.weight");
    L.q_norm = need_vector(m, p + ".self_attn.q_norm.weight");
    L.k_norm = need_vector(m, p + ".self_attn.k_norm.weight");
    L.input_ln = need_vector(m, p + ".input_layernorm.weight");
    L.post_attn_ln = need_vector(m, p + ".post_attention_layernorm.weight");
    L.pre_ff_ln = need_vector(m, p + ".pre_feedforward_layernorm.weight");
    L.post_ff_ln = need_vector(m, p + ".post_feedforward_layernorm.weight");
    L.gate = &need_matrix(m, p + ".mlp.gate_proj.weight");
    L.up = &need_matrix(m, p + ".mlp.up_proj.weight");
    L.down = &need_matrix(m, p + ".mlp.down_proj.weight");
    if (ple_dim > 0) {
      L.has_ple = true;
      L.ple_gate = &need_matrix(m, p + ".per_layer_input_gate.weight");
      L.ple_proj = &need_matrix(m, p + ".per_layer_projection.weight");
      L.ple_post_norm = need_vector(m, p + ".post_per_layer_input_norm.weight");
    }
    auto sc = m->tensors.find(p + ".layer_scalar");
    if (sc != m->tensors.end()) {
      if (sc->second.shape != std::vector<uint64_t>{1}) bail("layer_scalar must have shape [1]");
      L.layer_scalar = sc->second.m.at(0);
    }
  }

  // PLE globals (gemma/io.rs:1183-1234).
  if (ple_dim > 0) {
    m->has_ple = true;
    m->ple_dim = ple_dim;
    const size_t ple_vocab = c.has_vocab_size_per_layer_input ? c.vocab_size_per_layer_input : c.vocab_size;
    const Matrix& tok = need_matrix(m, "model.language_model.embed_tokens_per_layer.weight");
    const Matrix& proj = need_matrix(m, "model.language_model.per_layer_model_projection.weight");
    for (size_t l = 0; l < c.num_hidden_layers; ++l) {
      m->ple_token_emb.push_back(slice(tok, 0, ple_vocab, l * ple_dim, ple_dim));
      m->ple_model_proj.push_back(slice(proj, l * ple_dim, ple_dim, 0, c.hidden_size));
    }
    m->ple_proj_norm = need_vector(m, "model.language_model.per_layer_projection_norm.weight");
    m->ple_embedding_scale = f32_to_act(std::sqrt(float(ple_dim)));
    m->ple_projection_scalar = f32_to_act(std::pow(float(c.hidden_size), -0.5f));
    m->ple_input_scale = f32_to_act(std::pow(2.0f, -0.5f));
  }

  m->final_norm = need_vector(m, "model.language_model.norm.weight");
  const bool tied = c.has_tie_word_embeddings ? c.tie_word_embeddings != 0 : true;
  m->lm_head = tied ? m->embedding : &need_matrix(m, "model.language_model.lm_head.weight");
  if (c.has_final_logit_softcapping) m->softcap = f32_to_act(c.final_logit_softcapping);
  m->finalized = true;
}

// ---------------------------------------------------------------------------
// Elementwise drivers (det_kernels.rs:223-282)
// ---------------------------------------------------------------------------
// rms_norm_slab / apply_head_rms_norm_slab / apply_value_rms_norm_slab
// (det_kernels.rs:231-250, 393-428): rows in parallel, each normalised alone.
static void rms_rows(int32_t* x, size_t rows, size_t cols, const std::vector<int32_t>& w, int64_t eps) {
  if (w.size() != cols) bail("rms norm width mismatch: " + std::to_string(cols) + " vs " + std::to_string(w.size()));
  // in parallel only when no row can fail a contract check
  const bool par = g_threads > 1 && rows >= 16 && cols > 0 && cols <= UINT32_MAX && eps >= 0;
#pragma omp parallel for num_threads(g_threads) schedule(static) if (par)
  for (long r = 0; r < long(rows); ++r) rms_norm_in_place(x + size_t(r) * cols, w.data(), cols, eps);
}
static void value_rms_rows(int32_t* x, size_t rows, size_t cols, int64_t eps) {
  const bool par = g_threads > 1 && rows >= 16 && cols > 0 && cols <= UINT32_MAX && eps >= 0;
#pragma omp parallel for num_threads(g_threads) schedule(static) if (par)
  for (long r = 0; r < long(rows); ++r) value_rms_norm_in_place(x + size_t(r) * cols, cols, eps);
}
static void add_into(int32_t* dst, const int32_t* src, size_t n) { for (size_t i = 0; i < n; ++i) dst[i] = add_sat(dst[i], src[i]); }
static void mul_into(int32_t* dst, const int32_t* src, size_t n) { for (size_t i = 0; i < n; ++i) dst[i] = mul_sat(dst[i], src[i]); }
static void gelu_all(int32_t* x, size_t n) { for (size_t i = 0; i < n; ++i) x[i] = gelu_pytorch_tanh_act(x[i]); }
static void scale_all(int32_t* x, size_t n, int32_t s) { for (size_t i = 0; i < n; ++i) x[i] = scale_act(x[i], s); }

// det_kernels.rs:340-367 (score dot -> softmax -> weighted sum).
static void attention_output(const int32_t* q, const int32_t* keys, const int32_t* vals, size_t rows,
                             size_t hd, int32_t* out) {
  std::vector<int32_t> logits(rows), weights(rows);
  for (size_t r = 0; r < rows; ++r) logits[r] = attention_score(q, keys + r * hd, hd);
  attention_softmax(logits.data(), rows, weights.data());
  attention_weighted_sum(weights.data(), vals, rows, hd, out);
}

static size_t kv_groups(const Layer& L) {
  if (L.num_kv_heads == 0) bail("invalid Gemma head configuration");
  const size_t g = L.num_heads / L.num_kv_heads;
  if (g == 0) bail("Gemma layer must have at least one KV group");
  return g;
}

// ---------------------------------------------------------------------------
// Prefill layer (det_kernels.rs:525-821)
// ---------------------------------------------------------------------------
// Activations are seq-major [M x width]; a "head slab" [heads x M x hd] is
// represented by its seq-major twin, indexing (head, row) -> row*width + head*hd.
static std::vector<int32_t> to_heads(const std::vector<int32_t>& x, size_t m, size_t heads, size_t hd) {
  std::vector<int32_t> out(heads * m * hd);
  for (size_t t = 0; t < m; ++t)
    for (size_t h = 0; h < heads; ++h)
      std::memcpy(&out[(h * m + t) * hd], &x[t * heads * hd + h * hd], hd * 4);
  return out;
}

static std::vector<int32_t> layer_prefill(const Layer& L, const std::vector<int32_t>& xs, size_t m,
                                          const std::vector<int32_t>* ple_in, const KvData* donor,
                                          std::optional<KvData>* cache_out) {
  if (m == 0) bail("transformer layer execution requires at least one activation row");
  const size_t H = L.hidden, hd = L.head_dim;
  std::vector<int32_t> normed = xs;
  rms_rows(normed.data(), m, H, L.input_ln, L.eps);
  std::optional<size_t> attn_window = L.sliding ? L.sliding_window : std::nullopt;
  std::optional<size_t> cache_window = L.sliding ? L.cache_sliding_window : std::nullopt;
  const size_t groups = kv_groups(L);

  // project_qkv_slab (det_kernels.rs:499-523)
  std::vector<int32_t> qp = det_linear_slab(normed, m, H, *L.q);
  std::vector<int32_t> kp = det_linear_slab(normed, m, H, *L.k);
  std::vector<int32_t> vp;
  if (L.v) vp = det_linear_slab(normed, m, H, *L.v);
  else if (L.k_eq_v) vp = kp;
  else bail("Gemma layer is missing v_proj without attention_k_eq_v enabled");
  if (qp.size() != m * L.num_heads * hd || kp.size() != m * L.num_kv_heads * hd || vp.size() != kp.size())
    bail("projected attention states have unexpected width");
  std::vector<int32_t> q = to_heads(qp, m, L.num_heads, hd);
  std::vector<int32_t> k = to_heads(kp, m, L.num_kv_heads, hd);
  std::vector<int32_t> v = to_heads(vp, m, L.num_kv_heads, hd);
  rms_rows(q.data(), L.num_heads * m, hd, L.q_norm, L.eps);
  rms_rows(k.data(), L.num_kv_heads * m, hd, L.k_norm, L.eps);
  value_rms_rows(v.data(), L.num_kv_heads * m, hd, L.eps);
  if (L.partial_rotary_dim > 0) {  // apply_rope_slab, det_kernels.rs:430-468: (head, row) items in parallel
#pragma omp parallel for num_threads(g_threads) schedule(dynamic, 4) if (g_threads > 1)
    for (long i = 0; i < long(L.num_heads * m); ++i)
      rope_rotate_pairs_in_place(&q[size_t(i) * hd], hd, L.partial_rotary_dim, L.rope_freq_base_dim, L.rope_base,
                                 size_t(i) % m);
#pragma omp parallel for num_threads(g_threads) schedule(dynamic, 4) if (g_threads > 1)
    for (long i = 0; i < long(L.num_kv_heads * m); ++i)
      rope_rotate_pairs_in_place(&k[size_t(i) * hd], hd, L.partial_rotary_dim, L.rope_freq_base_dim, L.rope_base,
                                 size_t(i) % m);
  }
  if (!donor) {  // DetKvCacheData::from_head_slabs (det_tensor.rs:250-268)
    const size_t retained = cache_window ? (m > *cache_window ? m - *cache_window : 0) : 0;
    KvData d(L.num_kv_heads, hd);
    for (size_t h = 0; h < L.num_kv_heads; ++h) {
      for (size_t t = retained; t < m; ++t) {
        d.keys[h].push_row(&k[(h * m + t) * hd], hd);
        d.values[h].push_row(&v[(h * m + t) * hd], hd);
      }
    }
    *cache_out = std::move(d);
  } else {
    cache_out->reset();
  }
  std::vector<int32_t> combined(m * L.num_heads * hd);
  // det_kernels.rs:584-646: one item per (head, query), head-major; items are
  // independent and each writes its own output row, so the thread pool takes
  // them in any order.
  auto item_window = [&](size_t h, size_t t, const int32_t** kk, const int32_t** vv) -> size_t {
    const size_t kvh = h / groups;
    size_t start = 0;
    if (attn_window) start = (t + 1) > *attn_window ? t + 1 - *attn_window : 0;
    size_t rows = t + 1 - start;
    if (donor) {  // cache_windows (det_kernels.rs:297-311)
      const size_t avail = donor->len();
      start = std::min(start, avail);
      rows = std::min(rows, avail - start);
      *kk = donor->keys[kvh].rows_window(start);
      *vv = donor->values[kvh].rows_window(start);
    } else {
      *kk = &k[(kvh * m + start) * hd];
      *vv = &v[(kvh * m + start) * hd];
    }
    return rows;
  };
  for (size_t h = 0; h < L.num_heads; ++h)
    for (size_t t = 0; t < m; ++t) {
      const int32_t *kk, *vv;
      if (item_window(h, t, &kk, &vv) == 0) contract_violation("attention_softmax requires a non-empty logits slice");
    }
  const long items = long(L.num_heads * m);
#pragma omp parallel for num_threads(g_threads) schedule(dynamic, 8) if (g_threads > 1)
  for (long it = 0; it < items; ++it) {
    const size_t h = size_t(it) / m, t = size_t(it) % m;
    const int32_t *kk, *vv;
    const size_t rows = item_window(h, t, &kk, &vv);
    attention_output(&q[(h * m + t) * hd], kk, vv, rows, hd, &combined[t * L.num_heads * hd + h * hd]);
  }
  std::vector<int32_t> attn = det_linear_slab(combined, m, L.num_heads * hd, *L.o);
  if (L.o->rows != H) bail("o_proj output width mismatch");
  rms_rows(attn.data(), m, H, L.post_attn_ln, L.eps);
  add_into(attn.data(), xs.data(), m * H);
  std::vector<int32_t> x = std::move(attn);

  std::vector<int32_t> n2 = x;
  rms_rows(n2.data(), m, H, L.pre_ff_ln, L.eps);
  std::vector<int32_t> gate = det_linear_slab(n2, m, H, *L.gate);
  std::vector<int32_t> up = det_linear_slab(n2, m, H, *L.up);
  gelu_all(gate.data(), gate.size());
  if (gate.size() != up.size()) bail("row width mismatch");
  mul_into(gate.data(), up.data(), gate.size());
  std::vector<int32_t> ff = det_linear_slab(gate, m, L.gate->rows, *L.down);
  rms_rows(ff.data(), m, H, L.post_ff_ln, L.eps);
  add_into(ff.data(), x.data(), m * H);
  x = std::move(ff);

  if (L.has_ple && ple_in) {
    const size_t P = L.ple_gate->rows;
    std::vector<int32_t> g = det_linear_slab(x, m, H, *L.ple_gate);
    gelu_all(g.data(), g.size());
    if (ple_in->size() != m * P) bail("per-layer inputs width mismatch");
    mul_into(g.data(), ple_in->data(), g.size());
    std::vector<int32_t> pr = det_linear_slab(g, m, P, *L.ple_proj);
    rms_rows(pr.data(), m, H, L.ple_post_norm, L.eps);
    add_into(pr.data(), x.data(), m * H);
    x = std::move(pr);
  }
  if (L.layer_scalar) scale_all(x.data(), x.size(), *L.layer_scalar);
  return x;
}

// ---------------------------------------------------------------------------
// Decode layer (det_kernels.rs:866-1133)
// ---------------------------------------------------------------------------
static std::vector<int32_t> layer_decode(const Layer& L, const std::vector<int32_t>& input,
                                         const std::vector<int32_t>* ple_in, LayerCache& cache,
                                         const LayerCache* donor, size_t position) {
  const size_t H = L.hidden, hd = L.head_dim;
  if (input.size() != H) bail("decode input activation width mismatch");
  const size_t groups = kv_groups(L);
  const LayerCache& validated = donor ? *donor : cache;
  if (validated.num_kv_heads != L.num_kv_heads) bail("layer cache head count mismatch");
  std::optional<size_t> attn_window = L.sliding ? L.sliding_window : std::nullopt;
  std::optional<size_t> cache_window = L.sliding ? L.cache_sliding_window : std::nullopt;

  std::vector<int32_t> normed = input;
  rms_rows(normed.data(), 1, H, L.input_ln, L.eps);
  std::vector<int32_t> q(L.q->rows), k(L.k->rows), v;
  det_linear(*L.q, normed.data(), H, q.data());
  det_linear(*L.k, normed.data(), H, k.data());
  if (L.v) { v.resize(L.v->rows); det_linear(*L.v, normed.data(), H, v.data()); }
  else if (L.k_eq_v) v = k;
  else bail("Gemma layer is missing v_proj without attention_k_eq_v enabled");
  rms_rows(q.data(), q.size() / hd, hd, L.q_norm, L.eps);
  rms_rows(k.data(), k.size() / hd, hd, L.k_norm, L.eps);
  value_rms_rows(v.data(), v.size() / hd, hd, L.eps);
  if (L.partial_rotary_dim > 0) {  // apply_rope_row_heads (det_kernels.rs:470-486)
    for (size_t i = 0; i < q.size() / hd; ++i)
      rope_rotate_pairs_in_place(&q[i * hd], hd, L.partial_rotary_dim, L.rope_freq_base_dim, L.rope_base, position);
    for (size_t i = 0; i < k.size() / hd; ++i)
      rope_rotate_pairs_in_place(&k[i * hd], hd, L.partial_rotary_dim, L.rope_freq_base_dim, L.rope_base, position);
  }
  if (!donor) {
    if (!cache.det) cache.det = KvData(L.num_kv_heads, hd);
    if (k.size() != L.num_kv_heads * hd || v.size() != k.size()) bail("layer cache append head count mismatch");
    cache.det->append_rows(k.data(), v.data(), hd, cache_window);
  }
  const LayerCache& ac = donor ? *donor : cache;
  if (!ac.det) bail("deterministic attention requires canonical key cache rows");
  const size_t cur = ac.current_len();
  const size_t key_start = attn_window ? (cur > *attn_window ? cur - *attn_window : 0) : 0;
  const size_t window_len = ac.det->len() > key_start ? ac.det->len() - key_start : 0;
  std::vector<int32_t> combined(L.num_heads * hd);
  const size_t avail = ac.det->len();
  const size_t start = std::min(key_start, avail);
  const size_t rows = std::min(window_len, avail - start);
  if (rows == 0) contract_violation("attention_softmax requires a non-empty logits slice");
  // det_kernels.rs:1013-1036: heads in parallel, each into its own output chunk.
#pragma omp parallel for num_threads(g_threads) schedule(static, 1) if (g_threads > 1 && L.num_heads > 1)
  for (long h = 0; h < long(L.num_heads); ++h) {
    const size_t kvh = size_t(h) / groups;
    attention_output(&q[size_t(h) * hd], ac.det->keys[kvh].rows_window(start), ac.det->values[kvh].rows_window(start),
                     rows, hd, &combined[size_t(h) * hd]);
  }
  std::vector<int32_t> attn(L.o->rows);
  det_linear(*L.o, combined.data(), combined.size(), attn.data());
  rms_rows(attn.data(), 1, H, L.post_attn_ln, L.eps);
  std::vector<int32_t> xs = input;
  add_into(xs.data(), attn.data(), H);

  std::vector<int32_t> ffn = xs;
  rms_rows(ffn.data(), 1, H, L.pre_ff_ln, L.eps);
  std::vector<int32_t> gate(L.gate->rows), up(L.up->rows);
  det_linear(*L.gate, ffn.data(), H, gate.data());
  gelu_all(gate.data(), gate.size());
  det_linear(*L.up, ffn.data(), H, up.data());
  mul_into(gate.data(), up.data(), gate.size());
  std::vector<int32_t> ff(L.down->rows);
  det_linear(*L.down, gate.data(), gate.size(), ff.data());
  rms_rows(ff.data(), 1, H, L.post_ff_ln, L.eps);
  add_into(xs.data(), ff.data(), H);

  if (L.has_ple && ple_in) {
    std::vector<int32_t> g(L.ple_gate->rows);
    det_linear(*L.ple_gate, xs.data(), H, g.data());
    gelu_all(g.data(), g.size());
    if (ple_in->size() != g.size()) bail("decode per-layer input width mismatch");
    mul_into(g.data(), ple_in->data(), g.size());
    std::vector<int32_t> pr(L.ple_proj->rows);
    det_linear(*L.ple_proj, g.data(), g.size(), pr.data());
    rms_rows(pr.data(), 1, H, L.ple_post_norm, L.eps);
    add_into(xs.data(), pr.data(), H);
  }
  if (L.layer_scalar) scale_all(xs.data(), xs.size(), *L.layer_scalar);
  return xs;
}

// ---------------------------------------------------------------------------
// Embedding, PLE inputs, logits
// ---------------------------------------------------------------------------
static std::vector<int32_t> embed(const orc_model* m, const uint32_t* ids, size_t n) {
  // gemma/io.rs:2446-2518
  const Matrix& E = *m->embedding;
  std::vector<int32_t> out(n * E.cols);
  for (size_t t = 0; t < n; ++t) {
    if (ids[t] >= E.rows) bail("token id " + std::to_string(ids[t]) + " is out of bounds for embedding tensor");
    for (size_t c = 0; c < E.cols; ++c) out[t * E.cols + c] = scale_act(E.at(size_t(ids[t]) * E.cols + c), m->embed_scale);
  }
  return out;
}

// prefill_prepare_aux/native/tiles.rs:111-243 and det_kernels.rs:1142-1208
// (identical arithmetic; add_sat is commutative).
static std::vector<int32_t> ple_input_row(const orc_model* m, size_t layer, uint32_t token,
                                          const int32_t* input_row) {
  const Matrix& tok = m->ple_token_emb[layer];
  if (token >= tok.rows) bail("matrix row is out of bounds for PLE slice");
  std::vector<int32_t> emb(tok.cols);
  for (size_t c = 0; c < tok.cols; ++c) emb[c] = scale_act(tok.at(size_t(token) * tok.cols + c), m->ple_embedding_scale);
  const Matrix& P = m->ple_model_proj[layer];
  std::vector<int32_t> proj(P.rows);
  det_linear(P, input_row, m->hidden, proj.data());
  scale_all(proj.data(), proj.size(), m->ple_projection_scalar);
  rms_rows(proj.data(), 1, proj.size(), m->ple_proj_norm, m->eps);
  if (emb.size() != proj.size()) bail("row width mismatch");
  for (size_t c = 0; c < emb.size(); ++c) emb[c] = add_sat(emb[c], proj[c]);
  scale_all(emb.data(), emb.size(), m->ple_input_scale);
  return emb;
}

static std::vector<int32_t> hidden_to_logits(const orc_model* m, const int32_t* hidden) {
  // det_kernels.rs:1217-1267
  std::vector<int32_t> normed(hidden, hidden + m->hidden);
  rms_rows(normed.data(), 1, m->hidden, m->final_norm, m->eps);
  std::vector<int32_t> logits(m->lm_head->rows);
  det_linear(*m->lm_head, normed.data(), normed.size(), logits.data());
  if (m->softcap)
    for (auto& x : logits) x = softcap_act(x, *m->softcap);
  return logits;
}

}  // namespace oracle

// ---------------------------------------------------------------------------
// Sessions: prefill + decode routines
// ---------------------------------------------------------------------------
struct orc_session {
  orc_model* m = nullptr;
  std::vector<oracle::LayerCache> caches;
  size_t position = 0;
  std::vector<int32_t> logits;
  // capture products
  std::string embedding_commit, final_hidden_commit, logits_commit;
};

namespace oracle {

static std::vector<const LayerCache*> ptrs(const std::vector<LayerCache>& v) {
  std::vector<const LayerCache*> p;
  for (auto& c : v) p.push_back(&c);
  return p;
}

// Observer of each prefill layer: its output rows and the caches so far.
using PrefillObserver = std::function<void(size_t layer, const std::vector<int32_t>& xs,
                                           const std::vector<LayerCache>& caches)>;

// pipeline.rs:70-98 (+ prefill_range deterministic_tiles.rs:69-199, prefill_finalize tiles.rs:11-107)
static std::unique_ptr<orc_session> run_prefill(orc_model* m, const uint32_t* ids, size_t n,
                                                const PrefillObserver* observe = nullptr) {
  if (!m->finalized) bail("model is not finalized");
  if (n == 0) bail("transformer layer execution requires at least one activation row");
  auto s = std::make_unique<orc_session>();
  s->m = m;
  const size_t H = m->hidden;
  std::vector<int32_t> emb = embed(m, ids, n);
  s->embedding_commit = commit_rows(emb.data(), n, H);
  std::vector<std::vector<int32_t>> ple(m->layers.size());
  if (m->has_ple) {
    for (size_t l = 0; l < m->layers.size(); ++l) {
      if (!m->layers[l].has_ple) continue;
      for (size_t t = 0; t < n; ++t) {
        std::vector<int32_t> r = ple_input_row(m, l, ids[t], &emb[t * H]);
        ple[l].insert(ple[l].end(), r.begin(), r.end());
      }
    }
  }
  std::vector<int32_t> xs = emb;
  for (size_t l = 0; l < m->layers.size(); ++l) {
    const Layer& L = m->layers[l];
    const KvData* donor = nullptr;
    if (L.kv_shared_layer_index) {
      const size_t d = *L.kv_shared_layer_index;
      if (d >= l) bail("transformer prefill layer cannot share KV with non-prior donor");
      if (!s->caches[d].det) bail("deterministic attention requires canonical key cache rows");
      donor = &*s->caches[d].det;
    }
    std::optional<KvData> cache;
    xs = layer_prefill(L, xs, n, (m->has_ple && L.has_ple) ? &ple[l] : nullptr, donor, &cache);
    LayerCache lc;
    lc.num_kv_heads = L.num_kv_heads;
    lc.det = std::move(cache);
    s->caches.push_back(std::move(lc));
    if (observe) (*observe)(l, xs, s->caches);
  }
  s->final_hidden_commit = commit_rows(xs.data(), n, H);
  s->logits = hidden_to_logits(m, &xs[(n - 1) * H]);
  s->logits_commit = commit_vector(s->logits.data(), s->logits.size());
  s->position = n;
  return s;
}

struct LayerCapture {
  std::string layer_output;
  bool has_kv = false;  // the effective-cache commitment was taken after this layer
  std::optional<std::string> kv;
};

// decode_layer_range native tiles.rs:133-197 + decode_transition_finalize tiles.rs:9-65.
// per_layer: each layer's output commitment, and the effective caches'
// commitment after every kv_every-th layer and after the last one.
static std::vector<int32_t> run_decode(orc_session* s, uint32_t token, std::vector<LayerCapture>* per_layer,
                                       size_t kv_every = 1) {
  orc_model* m = s->m;
  const size_t H = m->hidden;
  std::vector<int32_t> input = embed(m, &token, 1);
  std::vector<LayerCache> updated;
  updated.reserve(m->layers.size());
  std::vector<int32_t> xs = input;
  for (size_t l = 0; l < m->layers.size(); ++l) {
    const Layer& L = m->layers[l];
    std::vector<int32_t> ple;
    if (m->has_ple && L.has_ple) ple = ple_input_row(m, l, token, input.data());
    const LayerCache* donor = nullptr;
    if (L.kv_shared_layer_index) {
      const size_t d = *L.kv_shared_layer_index;
      if (d >= l) bail("transformer decode layer cannot share KV with non-prior donor");
      donor = &updated[d];
    }
    LayerCache cache = std::move(s->caches[l]);
    xs = layer_decode(L, xs, (m->has_ple && L.has_ple) ? &ple : nullptr, cache, donor, s->position);
    updated.push_back(std::move(cache));
    if (per_layer) {
      LayerCapture c;
      c.layer_output = commit_rows(xs.data(), 1, H);
      if ((l + 1) % std::max<size_t>(kv_every, 1) == 0 || l + 1 == m->layers.size()) {
        // effective_layer_caches (decode_layer_range/mod.rs:497-506)
        std::vector<const LayerCache*> eff;
        for (auto& uc : updated) eff.push_back(&uc);
        for (size_t j = updated.size(); j < s->caches.size(); ++j) eff.push_back(&s->caches[j]);
        c.has_kv = true;
        c.kv = commit_kv(eff);
      }
      per_layer->push_back(std::move(c));
    }
  }
  s->caches = std::move(updated);
  s->position += 1;
  s->logits = hidden_to_logits(m, xs.data());
  return xs;
}

static std::string json_opt(const std::optional<std::string>& v) { return v ? "\"" + *v + "\"" : "null"; }

// det_goldens.rs:90-185
static std::string capture(orc_model* m, const uint32_t* ids, size_t n, size_t steps) {
  std::unique_ptr<orc_session> s = run_prefill(m, ids, n);
  std::string out = "{\"prefill\":{\"embedding\":\"" + s->embedding_commit + "\",\"final_hidden\":\"" +
                    s->final_hidden_commit + "\",\"logits\":\"" + s->logits_commit + "\",\"kv\":" +
                    json_opt(commit_kv(ptrs(s->caches))) + "},";
  // first_step_layers on a copy of the prefill state
  {
    orc_session copy = *s;
    const uint32_t tok = uint32_t(argmax_first(copy.logits.data(), copy.logits.size()));
    std::vector<LayerCapture> layers;
    run_decode(&copy, tok, &layers);
    out += "\"first_step_layers\":[";
    for (size_t i = 0; i < layers.size(); ++i) {
      if (i) out += ",";
      out += "{\"layer_output\":\"" + layers[i].layer_output + "\",\"kv\":" + json_opt(layers[i].kv) + "}";
    }
    out += "],";
  }
  out += "\"decode_steps\":[";
  std::vector<uint32_t> generated;
  for (size_t i = 0; i < steps; ++i) {
    const uint32_t tok = uint32_t(argmax_first(s->logits.data(), s->logits.size()));
    generated.push_back(tok);
    std::vector<int32_t> act = run_decode(s.get(), tok, nullptr);
    if (i) out += ",";
    out += "{\"token\":" + std::to_string(tok) + ",\"activation\":\"" + commit_rows(act.data(), 1, m->hidden) +
           "\",\"logits\":\"" + commit_vector(s->logits.data(), s->logits.size()) + "\",\"kv\":" +
           json_opt(commit_kv(ptrs(s->caches))) + "}";
  }
  std::string ids_json = "[";
  for (size_t i = 0; i < generated.size(); ++i) ids_json += (i ? "," : "") + std::to_string(generated[i]);
  ids_json += "]";
  Hasher h;  // trace.rs:425-430 sha256_hex of the serde_json text
  h.bytes(ids_json.data(), ids_json.size());
  out += "],\"end_to_end\":{\"generated_token_ids\":" + ids_json + ",\"generated_token_ids_sha256\":\"" + h.hex() + "\"}}";
  return out;
}

// The commitments the native deterministic routines put into their
// checkpoints (routines/prefill_range/mod.rs:36-88, prefill_range_finalize/mod.rs:17-73,
// decode_layer_range/mod.rs:553-664): every prefill layer's output rows, its
// token ranges of width `prefill_width` and the caches up to it; then per
// greedy step every layer's output and, at the end of each layer range of
// width `decode_width`, the effective caches.
static std::string trace_capture(orc_model* m, const uint32_t* ids, size_t n, size_t steps, size_t prefill_width,
                                 size_t decode_width) {
  const size_t H = m->hidden, L = m->layers.size();
  const size_t pw = std::min(std::max<size_t>(prefill_width ? prefill_width : SIZE_MAX, 1), n);
  const size_t dw = std::min(std::max<size_t>(decode_width ? decode_width : SIZE_MAX, 1), std::max<size_t>(L, 1));
  std::string layers_json;
  PrefillObserver obs = [&](size_t l, const std::vector<int32_t>& xs, const std::vector<LayerCache>& caches) {
    std::string ranges;
    for (size_t a = 0; a < n; a += pw) {
      const size_t b = std::min(n, a + pw);
      ranges += (a ? ",\"" : "\"") + commit_rows(xs.data() + a * H, b - a, H) + "\"";
    }
    layers_json += std::string(l ? "," : "") + "{\"output\":\"" + commit_rows(xs.data(), n, H) + "\",\"ranges\":[" +
                   ranges + "],\"kv\":" + json_opt(commit_kv(ptrs(caches))) + "}";
  };
  std::unique_ptr<orc_session> s = run_prefill(m, ids, n, &obs);
  std::string out = "{\"prefill\":{\"embedding\":\"" + s->embedding_commit + "\",\"layers\":[" + layers_json +
                    "],\"final_hidden\":\"" + s->final_hidden_commit + "\",\"logits\":\"" + s->logits_commit +
                    "\",\"kv\":" + json_opt(commit_kv(ptrs(s->caches))) + "},\"steps\":[";
  for (size_t i = 0; i < steps; ++i) {
    const uint32_t tok = uint32_t(argmax_first(s->logits.data(), s->logits.size()));
    std::vector<LayerCapture> per_layer;
    run_decode(s.get(), tok, &per_layer, dw);
    out += std::string(i ? "," : "") + "{\"token\":" + std::to_string(tok) + ",\"layers\":[";
    for (size_t l = 0; l < per_layer.size(); ++l) {
      out += std::string(l ? "," : "") + "{\"output\":\"" + per_layer[l].layer_output + "\"";
      if (per_layer[l].has_kv) out += ",\"kv\":" + json_opt(per_layer[l].kv);
      out += "}";
    }
    out += "],\"logits\":\"" + commit_vector(s->logits.data(), s->logits.size()) + "\"}";
  }
  return out + "]}";
}

// ---------------------------------------------------------------------------
// detwgt v2 reader (gemma/io.rs:224-387; DETWGT_V2_FORMAT.md)
// ---------------------------------------------------------------------------
static void load_detwgt(orc_model* m, const uint8_t* b, size_t len) {
  size_t cur = 0;
  auto take = [&](size_t n) -> const uint8_t* {
    if (n > len - cur) bail("artifact ended unexpectedly");
    const uint8_t* p = b + cur;
    cur += n;
    return p;
  };
  auto rd32 = [&]() { const uint8_t* p = take(4); return uint32_t(p[0]) | uint32_t(p[1]) << 8 | uint32_t(p[2]) << 16 | uint32_t(p[3]) << 24; };
  auto rd64 = [&]() { uint64_t lo = rd32(); uint64_t hi = rd32(); return lo | (hi << 32); };
  if (std::memcmp(take(8), "DNWGTV0\0", 8) != 0) bail("unsupported deterministic artifact magic");
  if (rd32() != 2) bail("unsupported deterministic artifact format version");
  if (rd32() != 1) bail("unsupported deterministic artifact det_num spec version");
  const uint64_t count = rd64();
  std::map<std::string, Tensor> tensors;
  for (uint64_t i = 0; i < count; ++i) {
    const uint32_t name_len = rd32();
    const uint8_t* np = take(name_len);
    std::string name(reinterpret_cast<const char*>(np), name_len);
    const uint32_t rank = rd32();
    if (rank > (len - cur) / 8) bail("artifact ended unexpectedly");  // before allocating the dims
    std::vector<uint64_t> shape(rank);
    uint64_t prod = 1;
    for (uint32_t r = 0; r < rank; ++r) {
      shape[r] = rd64();
      if (shape[r] != 0 && prod > UINT64_MAX / shape[r]) bail("tensor shape overflowed");
      prod *= shape[r];
    }
    const uint64_t element_count = rd64();
    if (element_count != prod) bail("tensor `" + name + "` element count mismatch");
    const uint32_t width = rd32();
    if (width != 16 && width != 32) bail("tensor `" + name + "` has an invalid element width");
    const uint64_t payload_len = rd64();
    uint64_t expected_payload_len = 0;  // gemma/io.rs:327-331 checked_mul
    if (__builtin_mul_overflow(element_count, uint64_t(width / 8), &expected_payload_len))
      bail("tensor payload byte count overflowed");
    if (payload_len != expected_payload_len) bail("tensor `" + name + "` payload length mismatch");
    const uint64_t mass = rd64();
    if (rank >= 2 && mass >= (uint64_t(1) << 31)) bail("tensor `" + name + "` max row mass violates the overflow bound");
    const size_t pad = (64 - cur % 64) % 64;
    const uint8_t* pp = take(pad);
    for (size_t k = 0; k < pad; ++k) if (pp[k]) bail("tensor `" + name + "` has non-zero payload alignment padding");
    const uint8_t* payload = take(payload_len);
    Tensor t;
    t.shape = shape;
    t.m.width = int(width);
    t.m.rows = rank >= 2 ? size_t(shape[0]) : 1;
    t.m.cols = rank >= 2 ? size_t(prod / std::max<uint64_t>(shape[0], 1)) : size_t(prod);
    if (rank >= 2 && shape[0] == 0) t.m.cols = 0;
    if (width == 16) { t.m.w16.resize(element_count); std::memcpy(t.m.w16.data(), payload, payload_len); }
    else { t.m.w32.resize(element_count); std::memcpy(t.m.w32.data(), payload, payload_len); }
    if (!tensors.emplace(name, std::move(t)).second) bail("deterministic artifact contains duplicate tensor `" + name + "`");
  }
  if (cur != len) bail("deterministic artifact has trailing bytes after tensor payloads");
  for (auto& kv : tensors) m->tensors[kv.first] = std::move(kv.second);
}

}  // namespace oracle

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
using namespace oracle;

template <class F>
static int guarded(F&& f) {
  try {
    f();
    return 0;
  } catch (const ContractViolation& e) {
    g_last_error = e.what();
    return 2;
  } catch (const InvalidArgument& e) {
    g_last_error = e.what();
    return 1;
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return 3;
  }
}

extern "C" {

const char* orc_last_error(void) { return g_last_error.c_str(); }
void orc_set_threads(int threads) { g_threads = threads < 1 ? 1 : threads; }
void orc_set_slab_group(int tokens) { g_slab_group = tokens < 1 ? 1 : tokens; }

int orc_det_linear(size_t rows, size_t cols, int w, const void* weight, const int32_t* act, int32_t* out, int threads) {
  return guarded([&] {
    if (w == 16) gemv_dispatch(static_cast<const int16_t*>(weight), rows, cols, act, out, threads);
    else if (w == 32) gemv_dispatch(static_cast<const int32_t*>(weight), rows, cols, act, out, threads);
    else bail("unsupported element width");
  });
}

int orc_det_linear_acc_i64(size_t rows, size_t cols, int w, const void* weight, const int32_t* act, int64_t* acc_out) {
  return guarded([&] {
    if (w != 16 && w != 32) bail("unsupported element width");
    for (size_t r = 0; r < rows; ++r) {
      int64_t acc = 0;
      for (size_t c = 0; c < cols; ++c) {
        const int32_t wv = w == 16 ? int32_t(static_cast<const int16_t*>(weight)[r * cols + c])
                                   : static_cast<const int32_t*>(weight)[r * cols + c];
        acc = mac_bits(acc, act[c], wv);
      }
      acc_out[r] = acc;
    }
  });
}

int orc_det_linear_slab(size_t m, size_t rows, size_t cols, int w, const void* weight, const int32_t* act, int32_t* out, int threads) {
  return guarded([&] {
    if (w == 16) slab_rows(static_cast<const int16_t*>(weight), rows, cols, m, act, out, threads);
    else if (w == 32) slab_rows(static_cast<const int32_t*>(weight), rows, cols, m, act, out, threads);
    else bail("unsupported element width");
  });
}

// det_attention_prefill's attention items (det_kernels.rs:584-646) for caller
// buffers: q [nq][nh*hd], k/v [nrows][nkv*hd] seq-major; query t attends key
// rows [max(0, t+1-window), t+1) (window 0 = unbounded) of KV head h/groups.
int orc_attention_causal(const int32_t* q, const int32_t* k, const int32_t* v, size_t nq, size_t nrows, size_t nh,
                         size_t nkv, size_t hd, size_t window, int32_t* out, int threads) {
  return guarded([&] {
    if (nkv == 0 || nh / nkv == 0) bail("invalid Gemma head configuration");
    if (nq == 0 || nh == 0 || hd == 0) bail("empty attention problem");
    if (nrows < nq) contract_violation("attention_softmax requires a non-empty logits slice");
    const size_t groups = nh / nkv;
    if ((nh - 1) / groups >= nkv) contract_violation("query head maps past the last KV head");
    // head-major copies of the key / value rows (HeadSlab layout, det_tensor.rs:12-146)
    std::vector<int32_t> kh(nkv * nrows * hd), vh(nkv * nrows * hd);
    for (size_t h = 0; h < nkv; ++h)
      for (size_t r = 0; r < nrows; ++r) {
        std::memcpy(&kh[(h * nrows + r) * hd], k + r * nkv * hd + h * hd, hd * 4);
        std::memcpy(&vh[(h * nrows + r) * hd], v + r * nkv * hd + h * hd, hd * 4);
      }
    const long items = long(nh * nq);
#pragma omp parallel for num_threads(threads) schedule(dynamic, 8) if (threads > 1)
    for (long it = 0; it < items; ++it) {
      const size_t h = size_t(it) / nq, t = size_t(it) % nq, kvh = h / groups;
      const size_t start = window && t + 1 > window ? t + 1 - window : 0;
      attention_output(q + t * nh * hd + h * hd, &kh[(kvh * nrows + start) * hd], &vh[(kvh * nrows + start) * hd],
                       t + 1 - start, hd, out + t * nh * hd + h * hd);
    }
  });
}

// The inverse-frequency chain of rope_rotate_pairs_in_place (ops.rs:184-195):
// out[i] = inv_frequency before pair i, starting at one and multiplied by
// rope_frequency_step(base, freq_base_dim) with acc_mul after every pair.
int orc_rope_inv_frequencies(int64_t base, size_t freq_base_dim, size_t half, int64_t* out) {
  return guarded([&] {
    if (freq_base_dim < 2 || freq_base_dim % 2) contract_violation("rope_rotate_pairs requires an even freq_base_dim of at least 2");
    if (base <= 0) contract_violation("rope_rotate_pairs requires a positive base");
    int64_t inv_frequency = kOneAcc;
    const int64_t step = rope_frequency_step(base, freq_base_dim);
    for (size_t i = 0; i < half; ++i) {
      out[i] = inv_frequency;
      inv_frequency = acc_mul(inv_frequency, step);
    }
  });
}

void orc_commit_activation_rows(const int32_t* rows, size_t n_rows, size_t width, char out_hex[65]) {
  std::string h = commit_rows(rows, n_rows, width);
  std::memcpy(out_hex, h.c_str(), 65);
}
void orc_commit_vector(const int32_t* v, size_t n, char out_hex[65]) {
  std::string h = commit_vector(v, n);
  std::memcpy(out_hex, h.c_str(), 65);
}

int orc_model_create(const orc_text_config* cfg, orc_model** out) {
  return guarded([&] {
    auto m = std::make_unique<orc_model>();
    m->cfg = *cfg;
    if (cfg->num_layer_types && !cfg->layer_types) bail("layer_types pointer is null");
    m->layer_types.assign(cfg->layer_types, cfg->layer_types + cfg->num_layer_types);
    m->cfg.layer_types = nullptr;
    *out = m.release();
  });
}

int orc_model_set_tensor(orc_model* m, const char* name, size_t rank, const uint64_t* dims, int w,
                         const void* data, const int32_t* row_scale) {
  return guarded([&] {
    if (m->finalized) bail("model is already finalized");
    if (rank == 0 || rank > 2) bail("tensor rank must be 1 or 2");
    Tensor t;
    t.shape.assign(dims, dims + rank);
    const size_t rows = rank == 2 ? dims[0] : 1;
    const size_t cols = rank == 2 ? dims[1] : dims[0];
    const size_t n = rows * cols;
    t.m.rows = rows;
    t.m.cols = cols;
    if (w == 8) {
      // Exact expansion q*s into canonical Wgt bits; i16 iff every value fits
      // (artifact.rs:250-256), as a detwgt v2 converter would store it.
      if (!row_scale) bail("int8 tensors need a row scale");
      const int8_t* q = static_cast<const int8_t*>(data);
      bool fits16 = true, fits32 = true, mass_ok = true;
#pragma omp parallel for schedule(static) reduction(&& : fits16, fits32, mass_ok)
      for (long r = 0; r < long(rows); ++r) {
        uint64_t mass = 0;
        for (size_t c = 0; c < cols; ++c) {
          const int64_t v = int64_t(q[size_t(r) * cols + c]) * int64_t(row_scale[r]);
          fits32 = fits32 && v >= INT32_MIN && v <= INT32_MAX;
          fits16 = fits16 && v >= INT16_MIN && v <= INT16_MAX;
          mass += uint64_t(v < 0 ? -v : v);
        }
        mass_ok = mass_ok && !(rank == 2 && mass >= (uint64_t(1) << 31));
      }
      if (!fits32) bail("int8 x scale does not fit a Q16.16 weight");
      if (!mass_ok) bail("row mass violates the overflow bound");
      // Exact expansion q*s into canonical Wgt bits; i16 iff every value fits
      // (artifact.rs:250-256), as a detwgt v2 converter would store it.
      t.m.width = fits16 ? 16 : 32;
      if (fits16) t.m.w16.resize(n); else t.m.w32.resize(n);
#pragma omp parallel for schedule(static)
      for (long r = 0; r < long(rows); ++r)
        for (size_t c = 0; c < cols; ++c) {
          const size_t i = size_t(r) * cols + c;
          const int32_t v = int32_t(int64_t(q[i]) * int64_t(row_scale[r]));
          if (fits16) t.m.w16[i] = int16_t(v); else t.m.w32[i] = v;
        }
    } else if (w == 16) {
      t.m.width = 16;
      t.m.w16.assign(static_cast<const int16_t*>(data), static_cast<const int16_t*>(data) + n);
    } else if (w == 32) {
      t.m.width = 32;
      t.m.w32.assign(static_cast<const int32_t*>(data), static_cast<const int32_t*>(data) + n);
    } else {
      bail("unsupported element width");
    }
    m->tensors[name] = std::move(t);
  });
}

int orc_model_load_detwgt(orc_model* m, const uint8_t* bytes, size_t len) {
  return guarded([&] {
    if (m->finalized) bail("model is already finalized");
    load_detwgt(m, bytes, len);
  });
}

int orc_model_finalize(orc_model* m) { return guarded([&] { finalize_model(m); }); }
void orc_model_free(orc_model* m) { delete m; }

int orc_capture(orc_model* m, const uint32_t* prompt, size_t n, size_t steps, char* out, size_t cap) {
  return guarded([&] {
    std::string s = capture(m, prompt, n, steps);
    if (s.size() + 1 > cap) bail("capture output buffer too small: need " + std::to_string(s.size() + 1));
    std::memcpy(out, s.c_str(), s.size() + 1);
  });
}

int orc_trace_capture(orc_model* m, const uint32_t* prompt, size_t n, size_t steps, size_t prefill_width,
                      size_t decode_width, char* out, size_t cap) {
  return guarded([&] {
    if (!m->finalized) bail("model is not finalized");
    std::string s = trace_capture(m, prompt, n, steps, prefill_width, decode_width);
    if (s.size() + 1 > cap) bail("capture output buffer too small: need " + std::to_string(s.size() + 1));
    std::memcpy(out, s.c_str(), s.size() + 1);
  });
}

int orc_session_prefill(orc_model* m, const uint32_t* prompt, size_t n, orc_session** out, int32_t* logits_out) {
  return guarded([&] {
    std::unique_ptr<orc_session> s = run_prefill(m, prompt, n);
    if (logits_out) std::memcpy(logits_out, s->logits.data(), s->logits.size() * 4);
    *out = s.release();
  });
}

int orc_session_decode(orc_session* s, uint32_t token, int32_t* logits_out, int32_t* hidden_out) {
  return guarded([&] {
    std::vector<int32_t> xs = run_decode(s, token, nullptr);
    if (logits_out) std::memcpy(logits_out, s->logits.data(), s->logits.size() * 4);
    if (hidden_out) std::memcpy(hidden_out, xs.data(), xs.size() * 4);
  });
}

int orc_session_clone(const orc_session* src, orc_session** out) {
  if (!src || !out) return 1;
  *out = new orc_session(*src);
  return 0;
}
void orc_session_free(orc_session* s) { delete s; }

}  // extern "C"
