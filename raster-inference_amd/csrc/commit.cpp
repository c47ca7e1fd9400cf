// Host-side det commitments, KV mirror and hashing pool (see commit.h).
#include "commit.h"

#include <algorithm>
#include <cstring>

namespace det_commit {

void Sha::u64(uint64_t v) {
  uint8_t b[8];
  for (int i = 0; i < 8; ++i) b[i] = uint8_t(v >> (8 * i));
  put(b, 8);
}

void Sha::hex(char out[65]) {
  uint8_t d[32];
  SHA256_Final(d, &c);
  static const char* H = "0123456789abcdef";
  for (int i = 0; i < 32; ++i) {
    out[2 * i] = H[d[i] >> 4];
    out[2 * i + 1] = H[d[i] & 15];
  }
  out[64] = 0;
}

std::string Sha::hex() {
  char out[65];
  hex(out);
  return out;
}

// transformer_kernels.rs:1395-1430: domain, row count, then per row its
// width and its values.
void commit_rows(const int32_t* rows, uint64_t n, uint64_t width, char out[65]) {
  Sha h;
  static const char kDom[] = "raster-det-num-act-v1";
  h.put(kDom, sizeof(kDom) - 1);
  h.u64(n);
  for (uint64_t r = 0; r < n; ++r) {
    h.u64(width);
    h.i32s(rows + r * width, width);
  }
  h.hex(out);
}

std::string commit_rows(const int32_t* rows, uint64_t n, uint64_t width) {
  char out[65];
  commit_rows(rows, n, width, out);
  return out;
}

// transformer_kernels.rs:1432-1438
void commit_vector(const int32_t* v, uint64_t n, char out[65]) {
  Sha h;
  static const char kDom[] = "raster-det-num-act-vector-v1";
  h.put(kDom, sizeof(kDom) - 1);
  h.u64(n);
  h.i32s(v, n);
  h.hex(out);
}

std::string commit_vector(const int32_t* v, uint64_t n) {
  char out[65];
  commit_vector(v, n, out);
  return out;
}

std::string sha_hex(const std::string& bytes) {
  Sha h;
  h.put(bytes.data(), bytes.size());
  return h.hex();
}

// transformer_kernels.rs:1460-1482: domain, layer count; per layer its head
// count, then "k" and "v" each with the head count and, per head, the row
// count and each row's width and values. None as soon as one layer has no
// det data.
std::string commit_kv(const std::vector<KvLayerView>& layers) {
  for (const KvLayerView& l : layers)
    if (!l.has) return "";
  Sha h;
  static const char kDom[] = "raster-det-num-kv-cache-v1";
  h.put(kDom, sizeof(kDom) - 1);
  h.u64(layers.size());
  for (const KvLayerView& l : layers) {
    h.u64(l.heads);
    for (int side = 0; side < 2; ++side) {
      const char kind = side ? 'v' : 'k';
      h.put(&kind, 1);
      h.u64(l.heads);
      for (uint64_t hh = 0; hh < l.heads; ++hh) {
        h.u64(l.len);
        for (uint64_t r = 0; r < l.len; ++r) {
          h.u64(l.hd);
          h.i32s(l.row(side, r) + hh * l.hd, l.hd);
        }
      }
    }
  }
  return h.hex();
}

void KvMirror::add_layer(bool own, uint64_t heads, uint64_t hd, std::optional<uint64_t> window, uint64_t max_tokens) {
  Layer L;
  L.own = own;
  L.heads = heads;
  L.hd = hd;
  L.width = heads * hd;
  L.window = window;
  if (own) {
    L.cap = std::max<uint64_t>(max_tokens, 1);
    L.k.reset(new int32_t[L.cap * std::max<uint64_t>(L.width, 1)]);
    L.v.reset(new int32_t[L.cap * std::max<uint64_t>(L.width, 1)]);
  }
  layers_.push_back(std::move(L));
}

KvLayerView KvMirror::view(size_t l, uint64_t total) const {
  const Layer& L = layers_[l];
  KvLayerView v;
  v.has = L.own && total > 0;
  v.heads = L.heads;
  v.hd = L.hd;
  if (!v.has) return v;
  v.len = L.window ? std::min(total, *L.window) : total;
  const uint64_t first = total - v.len;
  const int32_t* k = L.k.get();
  const int32_t* vv = L.v.get();
  const uint64_t w = L.width;
  v.row = [k, vv, w, first](int side, uint64_t r) { return (side ? vv : k) + (first + r) * w; };
  return v;
}

HashPool::HashPool(unsigned threads) {
  threads = std::max(1u, threads);
  for (unsigned t = 0; t < threads; ++t)
    workers_.emplace_back([this] {
      for (;;) {
        std::packaged_task<std::string()> task;
        {
          std::unique_lock<std::mutex> lk(mu_);
          cv_.wait(lk, [this] { return stop_ || !queue_.empty(); });
          if (queue_.empty()) return;  // stop_ with nothing left
          task = std::move(queue_.front());
          queue_.pop_front();
        }
        task();
      }
    });
}

HashPool::~HashPool() {
  {
    std::lock_guard<std::mutex> lk(mu_);
    stop_ = true;
  }
  cv_.notify_all();
  for (auto& t : workers_) t.join();
}

std::shared_future<std::string> HashPool::submit(std::function<std::string()> fn) {
  std::packaged_task<std::string()> task(std::move(fn));
  std::shared_future<std::string> f = task.get_future().share();
  {
    std::lock_guard<std::mutex> lk(mu_);
    queue_.push_back(std::move(task));
  }
  cv_.notify_one();
  return f;
}

std::shared_future<std::string> HashPool::ready(std::string v) {
  std::promise<std::string> p;
  p.set_value(std::move(v));
  return p.get_future().share();
}

}  // namespace det_commit
