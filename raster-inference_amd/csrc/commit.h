// Host-side det commitments (transformer_kernels.rs:1395-1482), the
// append-only host mirror of a sequence's KV rows, and the worker pool that
// hashes checkpoint commitments concurrently with the GPU.
#pragma once

#include <openssl/sha.h>
#include <stdint.h>

#include <condition_variable>
#include <deque>
#include <functional>
#include <future>
#include <memory>
#include <mutex>
#include <optional>
#include <string>
#include <thread>
#include <vector>

namespace det_commit {

struct Sha {
  SHA256_CTX c;
  Sha() { SHA256_Init(&c); }
  void put(const void* p, size_t n) { SHA256_Update(&c, p, n); }
  void u64(uint64_t v);
  // int32 values as little-endian bytes: the host's own layout on x86-64.
  void i32s(const int32_t* v, size_t n) {
    static_assert(__BYTE_ORDER__ == __ORDER_LITTLE_ENDIAN__, "commitments hash little-endian i32 bytes");
    put(v, n * 4);
  }
  void hex(char out[65]);
  std::string hex();
};

// build_det_activation_commitment{,_slab,_row}: n rows of `width` Act.
void commit_rows(const int32_t* rows, uint64_t n, uint64_t width, char out[65]);
std::string commit_rows(const int32_t* rows, uint64_t n, uint64_t width);
// build_det_vector_commitment.
void commit_vector(const int32_t* v, uint64_t n, char out[65]);
std::string commit_vector(const int32_t* v, uint64_t n);
std::string sha_hex(const std::string& bytes);

// One layer's cache as build_det_kv_cache_commitment reads it: `heads` heads
// of `hd` values, logical rows oldest to newest. Row r of head h is at
// row(r) + h * hd. has == false: LayerKvCache without det data (the whole
// commitment is then None).
struct KvLayerView {
  bool has = false;
  uint64_t heads = 0, hd = 0, len = 0;
  std::function<const int32_t*(int side, uint64_t r)> row;  // side 0 = keys, 1 = values
};
// build_det_kv_cache_commitment over the layers in order; "" for None.
std::string commit_kv(const std::vector<KvLayerView>& layers);

// Append-only host copy of a sequence's KV rows by absolute token index.
// Layers without their own cache (KV-shared) hold nothing. Rows are written
// once and never moved, so commitments over earlier views can be hashed on
// other threads while later rows are appended.
class KvMirror {
 public:
  struct Layer {
    bool own = false;
    uint64_t heads = 0, hd = 0, width = 0, cap = 0;
    std::optional<uint64_t> window;  // cache_sliding_window: the last `window` rows are kept
    std::unique_ptr<int32_t[]> k, v;  // [cap][width]
  };
  void add_layer(bool own, uint64_t heads, uint64_t hd, std::optional<uint64_t> window, uint64_t max_tokens);
  size_t layers() const { return layers_.size(); }
  Layer& layer(size_t l) { return layers_[l]; }
  // The cache of layer l after `total` tokens were appended: rows
  // [total - min(total, window), total); has == false for a shared layer or
  // before the first token (LayerKvCache without det data).
  KvLayerView view(size_t l, uint64_t total) const;

 private:
  std::vector<Layer> layers_;
};

// Fixed pool of hashing threads; results are futures, work runs in FIFO order.
class HashPool {
 public:
  explicit HashPool(unsigned threads);
  ~HashPool();
  std::shared_future<std::string> submit(std::function<std::string()> fn);
  // A future already holding v.
  static std::shared_future<std::string> ready(std::string v);

 private:
  std::vector<std::thread> workers_;
  std::deque<std::packaged_task<std::string()>> queue_;
  std::mutex mu_;
  std::condition_variable cv_;
  bool stop_ = false;
};

}  // namespace det_commit
