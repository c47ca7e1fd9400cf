// C ABI (include/detgpu.h) and the GPU executor of the deterministic path.
//
// Host side of the MI355X det path: context/stream management, weight upload
// (int8 x row-scale factorization of detwgt v2 matrices), model resolution
// mirroring load_det_num_gemma4_layer_weights (gemma/io.rs:1896-2045), and
// the prefill_layer / decode_transition routines (det_kernels.rs:678-1267,
// routines/*/native) driven as HIP kernel sequences on one stream.
#include <hip/hip_runtime.h>
#include <openssl/sha.h>

#include <algorithm>
#include <cfloat>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <numeric>
#include <optional>
#include <stdexcept>
#include <string>
#include <thread>
#include <initializer_list>
#include <vector>

#include "../../include/detgpu.h"
#include "decode.h"
#include "det_arith.h"
#include "audit.h"
#include "commit.h"
#include "kernels.h"

using det::DevMatrix;

namespace {

struct Status : std::runtime_error {
  int code;
  Status(int c, const std::string& m) : std::runtime_error(m), code(c) {}
};
[[noreturn]] void bail(const std::string& m) { throw Status(1, m); }
[[noreturn]] void contract(const std::string& m) { throw Status(2, m); }
void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw Status(3, std::string(what) + ": " + hipGetErrorString(e));
}
#define HIPC(x) hip_check((x), #x)

thread_local std::string g_error;  // errors before a context exists

}  // namespace

struct det_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  int64_t* noalloc_parts = nullptr;  // this device's address of the allocation-free argmax scratch
  std::string last_error;
  int8_t* limbs = nullptr;  // activation limb scratch for the int8 GEMV
  size_t limbs_bytes = 0;
  int64_t* argmax_scratch = nullptr;
  size_t argmax_parts = 0;
  uint32_t* argmax_out = nullptr;

  int8_t* gemm_a = nullptr;  // tiled activation limb rows for the prefill GEMM
  size_t gemm_a_bytes = 0;
  int64_t* gemm_planes = nullptr;  // K-range partial planes of split GEMMs
  size_t gemm_planes_bytes = 0;
  void* attn_work = nullptr;  // work area of the MFMA form of causal attention
  size_t attn_work_bytes = 0;
  bool capturing = false;  // between det_ctx_capture_begin and _end

  // scratch that has to grow cannot be allocated while the stream records
  void grow_check(const char* what) const {
    if (capturing)
      bail(std::string("det_ctx capture: ") + what +
           " scratch would grow inside the capture; run the call once before capturing");
  }
  void ensure_gemm_a(size_t bytes) {
    if (bytes <= gemm_a_bytes) return;
    grow_check("GEMM activation");
    HIPC(hipStreamSynchronize(stream));
    if (gemm_a) HIPC(hipFree(gemm_a));
    gemm_a = nullptr;
    HIPC(hipMalloc(&gemm_a, bytes));
    gemm_a_bytes = bytes;
  }
  // the partial planes a GEMM of W over m rows splits K into (null: no split)
  int64_t* gemm_planes_for(const det::DevMatrix& W, uint64_t m) {
    const size_t bytes = det::gemm_plane_bytes(W, m);
    if (bytes == 0) return nullptr;
    if (bytes > gemm_planes_bytes) {
      grow_check("GEMM partial-plane");
      HIPC(hipStreamSynchronize(stream));
      if (gemm_planes) HIPC(hipFree(gemm_planes));
      gemm_planes = nullptr;
      HIPC(hipMalloc(&gemm_planes, bytes));
      gemm_planes_bytes = bytes;
    }
    return gemm_planes;
  }
  // The MFMA attention's work area for a (null where that form does not
  // apply or would need more than kAttnWorkMax bytes: the vector-ALU kernel
  // runs then).
  static constexpr uint64_t kAttnWorkMax = uint64_t(512) << 20;
  void attach_attn_work(det::AttnArgs& a) {
    const uint64_t bytes = det::attn_mfma_bytes(a);
    a.work = nullptr;
    a.work_bytes = 0;
    if (bytes == 0 || bytes > kAttnWorkMax) return;
    if (bytes > attn_work_bytes) {
      grow_check("attention");
      HIPC(hipStreamSynchronize(stream));
      if (attn_work) HIPC(hipFree(attn_work));
      attn_work = nullptr;
      HIPC(hipMalloc(&attn_work, bytes));
      attn_work_bytes = bytes;
    }
    a.work = attn_work;
    a.work_bytes = attn_work_bytes;
  }
  // Slab GEMM / GEMV dispatch: int8 weights with at least kGemmMinRows
  // activation rows take the MFMA GEMM, everything else the GEMV kernels.
  static constexpr uint64_t kGemmMinRows = 16;
  void linear(const det::DevMatrix& W, const int32_t* act, uint64_t m, uint64_t ld_act, int32_t* out, uint64_t ld_out,
              int64_t* acc_out) {
    if (W.storage == det::kInt8 && m >= kGemmMinRows) {
      ensure_gemm_a(det::gemm_act_bytes(m, W.kpad));
      int64_t* planes = gemm_planes_for(W, m);
      det::launch_gemm(W, act, m, ld_act, out, ld_out, acc_out, gemm_a, stream, planes);
    } else {
      det::launch_linear(W, act, m, ld_act, out, ld_out, acc_out, limbs, stream);
    }
  }

  // Several matrices applied to the same activation rows: with the GEMM, one
  // limb expansion feeds all of them when their input widths agree.
  void linear_group(std::initializer_list<std::pair<const det::DevMatrix*, int32_t*>> items, const int32_t* act,
                    uint64_t m, uint64_t ld_act) {
    const det::DevMatrix* first = items.begin()->first;
    bool shared = m >= kGemmMinRows;
    for (const auto& it : items)
      shared &= it.first->storage == det::kInt8 && it.first->kpad == first->kpad && it.first->cols == first->cols;
    if (!shared) {
      for (const auto& it : items) linear(*it.first, act, m, ld_act, it.second, it.first->rows, nullptr);
      return;
    }
    ensure_gemm_a(det::gemm_act_bytes(m, first->kpad));
    det::launch_gemm_limbs(act, m, first->cols, ld_act, first->kpad, gemm_a, stream);
    for (const auto& it : items) {
      int64_t* planes = gemm_planes_for(*it.first, m);
      det::launch_gemm_tiled(*it.first, m, it.second, it.first->rows, nullptr, gemm_a, stream, nullptr, planes);
    }
  }

  void ensure_limbs(size_t bytes) {
    if (bytes <= limbs_bytes) return;
    grow_check("GEMV limb");
    HIPC(hipStreamSynchronize(stream));
    if (limbs) HIPC(hipFree(limbs));
    limbs = nullptr;
    HIPC(hipMalloc(&limbs, bytes));
    limbs_bytes = bytes;
  }
  uint32_t argmax(const int32_t* x, uint64_t n) {
    if (capturing) bail("det_ctx capture: the argmax returns its index to the host and cannot be recorded");
    const size_t parts = (n + 1023) / 1024;
    if (parts > argmax_parts) {
      HIPC(hipStreamSynchronize(stream));
      if (argmax_scratch) HIPC(hipFree(argmax_scratch));
      argmax_scratch = nullptr;
      HIPC(hipMalloc(&argmax_scratch, parts * sizeof(int64_t)));
      argmax_parts = parts;
    }
    det::launch_argmax(x, n, argmax_scratch, argmax_out, stream);
    uint32_t r = 0;
    HIPC(hipMemcpyAsync(&r, argmax_out, 4, hipMemcpyDeviceToHost, stream));
    HIPC(hipStreamSynchronize(stream));
    return r;
  }
};

struct det_matrix {
  det_ctx* ctx = nullptr;
  DevMatrix m;
};

struct det_event {
  hipEvent_t ev = nullptr;
};
struct det_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  ~det_graph() {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
  }
};

namespace {

// A call that fails while the context's stream is recording ends the
// capture: the partial recording is discarded and the stream runs again.
void abort_capture(det_ctx* ctx) {
  if (!ctx || !ctx->capturing) return;
  ctx->capturing = false;
  hipGraph_t g = nullptr;
  (void)hipStreamEndCapture(ctx->stream, &g);
  if (g) (void)hipGraphDestroy(g);
}

template <class F>
int guarded(det_ctx* ctx, F&& f) {
  try {
    f();
    return 0;
  } catch (const Status& e) {
    (ctx ? ctx->last_error : g_error) = e.what();
    abort_capture(ctx);
    return e.code;
  } catch (const std::invalid_argument& e) {  // argument checks inside the kernel launchers
    (ctx ? ctx->last_error : g_error) = e.what();
    abort_capture(ctx);
    return 1;
  } catch (const std::exception& e) {
    (ctx ? ctx->last_error : g_error) = e.what();
    abort_capture(ctx);
    return 3;
  }
}

// ---------------------------------------------------------------------------
// weight upload
// ---------------------------------------------------------------------------
uint64_t round_up(uint64_t v, uint64_t a) { return (v + a - 1) / a * a; }

// Runs fn(r0, r1) over [0, n) on up to 16 host threads (load-time work only).
template <class F>
void parallel_rows(uint64_t n, F&& fn) {
  const unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  const uint64_t per = (n + hw - 1) / hw;
  if (n < 4096 || hw == 1) { fn(uint64_t(0), n); return; }
  std::vector<std::thread> th;
  for (unsigned t = 0; t < hw; ++t) {
    const uint64_t r0 = t * per, r1 = std::min(n, r0 + per);
    if (r0 >= r1) break;
    th.emplace_back([&fn, r0, r1] { fn(r0, r1); });
  }
  for (auto& x : th) x.join();
}

void free_matrix(DevMatrix& m) {
  if (!m.owns) return;
  if (m.q) (void)hipFree(m.q);
  if (m.scale) (void)hipFree(m.scale);
  if (m.rowsum) (void)hipFree(m.rowsum);
  if (m.rowsum_p) (void)hipFree(m.rowsum_p);
  if (m.w) (void)hipFree(m.w);
  m = DevMatrix();
}

// Uploads a digit-plane matrix: W[r][c] = scale[r] * sum_p 256^p d[p][r][c]
// (d plane-major [planes][rows][cols]) in the tile-major layout, each tile's
// planes consecutive (virtual rows digit_row(r, planes, p)), rows padded to a
// multiple of 16 and columns to kpad, with the row sums (of sum_p 256^p d_p)
// used by the limb correction, whole and per column part.
DevMatrix upload_digits(det_ctx* ctx, uint64_t rows, uint64_t cols, int planes, const int8_t* d,
                        const int32_t* scale) {
  if (cols > 130000) bail("int8 rows longer than 130000 columns are not supported");
  DevMatrix m;
  m.rows = rows;
  m.cols = cols;
  m.storage = det::kInt8;
  m.planes = planes;
  m.kpad = round_up(std::max<uint64_t>(cols, 1), 128);
  const uint64_t prow = round_up(std::max<uint64_t>(rows, 1), 16);
  std::vector<int8_t> tiled(prow * uint64_t(planes) * m.kpad, 0);
  const uint64_t nparts = det::limb_parts(m.kpad);
  std::vector<int32_t> rowsum(prow, 0), sc(prow, 0), rowsum_p(prow * nparts, 0);
  bool sums_fit = true;
  std::mutex mu;
  parallel_rows(rows, [&](uint64_t r0, uint64_t r1) {
    bool fit = true;
    for (uint64_t r = r0; r < r1; ++r) {
      int64_t s = 0;
      // (16 columns at a time: the run of one row that is contiguous in the tile-step)
      for (uint64_t c0 = 0; c0 < cols; c0 += 16) {
        const uint64_t n = std::min<uint64_t>(16, cols - c0);
        int64_t sp = 0;
        for (int p = 0; p < planes; ++p) {
          const int8_t* src = d + (uint64_t(p) * rows + r) * cols + c0;
          std::memcpy(&tiled[det::tiled_offset(m.kpad, det::digit_row(r, planes, p), c0)], src, n);
          int64_t dp = 0;
          for (uint64_t c = 0; c < n; ++c) dp += src[c];
          sp += dp * (int64_t(1) << (8 * p));
        }
        s += sp;
        const int64_t acc = int64_t(rowsum_p[(c0 / det::kLimbPartCols) * prow + r]) + sp;
        fit &= acc >= INT32_MIN && acc <= INT32_MAX;
        rowsum_p[(c0 / det::kLimbPartCols) * prow + r] = int32_t(acc);
      }
      fit &= s >= INT32_MIN && s <= INT32_MAX;
      rowsum[r] = int32_t(s);
      sc[r] = scale[r];
    }
    if (!fit) {
      std::lock_guard<std::mutex> lock(mu);
      sums_fit = false;
    }
  });
  if (!sums_fit) bail("weight row mass violates the 2^31 overflow bound");
  HIPC(hipMalloc(&m.q, tiled.size()));
  HIPC(hipMalloc(&m.scale, prow * 4));
  HIPC(hipMalloc(&m.rowsum, prow * 4));
  HIPC(hipMalloc(&m.rowsum_p, rowsum_p.size() * 4));
  m.rowsum_p_ld = prow;
  HIPC(hipMemcpyAsync(m.q, tiled.data(), tiled.size(), hipMemcpyHostToDevice, ctx->stream));
  HIPC(hipMemcpyAsync(m.scale, sc.data(), prow * 4, hipMemcpyHostToDevice, ctx->stream));
  HIPC(hipMemcpyAsync(m.rowsum, rowsum.data(), prow * 4, hipMemcpyHostToDevice, ctx->stream));
  HIPC(hipMemcpyAsync(m.rowsum_p, rowsum_p.data(), rowsum_p.size() * 4, hipMemcpyHostToDevice, ctx->stream));
  HIPC(hipStreamSynchronize(ctx->stream));
  ctx->ensure_limbs(4 * 4 * m.kpad);
  return m;
}

// Uploads int8 q (rows x cols) with per-row scales: one digit plane.
DevMatrix upload_int8(det_ctx* ctx, uint64_t rows, uint64_t cols, const int8_t* q, const int32_t* scale) {
  return upload_digits(ctx, rows, cols, 1, q, scale);
}

// A digit-plane matrix on the host: d plane-major [planes][rows][cols].
struct HostDigits {
  uint64_t rows = 0, cols = 0;
  int planes = 1;
  std::vector<int8_t> d;
  std::vector<int32_t> scale;
};

// Downloads a digit-plane matrix back to row-major planes + scales.
HostDigits untile(det_ctx* ctx, const DevMatrix& M) {
  HostDigits h;
  h.rows = M.rows;
  h.cols = M.cols;
  h.planes = M.planes;
  const uint64_t prow = round_up(std::max<uint64_t>(M.rows, 1), 16);
  std::vector<int8_t> tiled(prow * uint64_t(M.planes) * M.kpad);
  HIPC(hipMemcpy(tiled.data(), M.q, tiled.size(), hipMemcpyDeviceToHost));
  h.scale.resize(M.rows);
  HIPC(hipMemcpy(h.scale.data(), M.scale, M.rows * 4, hipMemcpyDeviceToHost));
  h.d.resize(uint64_t(M.planes) * M.rows * M.cols);
  parallel_rows(M.rows, [&](uint64_t r0, uint64_t r1) {
    for (uint64_t r = r0; r < r1; ++r)
      for (int p = 0; p < M.planes; ++p)
        for (uint64_t c0 = 0; c0 < M.cols; c0 += 16)
          std::memcpy(&h.d[(uint64_t(p) * M.rows + r) * M.cols + c0],
                      &tiled[det::tiled_offset(M.kpad, det::digit_row(r, M.planes, p), c0)],
                      std::min<uint64_t>(16, M.cols - c0));
  });
  return h;
}

// Copies rows [r0, r0+n) of a device matrix into a new matrix (host round trip;
// load time only). Used for row slices that are not tile aligned.
DevMatrix extract_rows(det_ctx* ctx, const DevMatrix& src, uint64_t r0, uint64_t n) {
  if (r0 + n > src.rows) bail("matrix row slice out of bounds");
  if (src.storage != det::kInt8) return det::row_view(src, r0, n);
  if (r0 % 16 == 0) return det::row_view(src, r0, n);
  const HostDigits h = untile(ctx, src);
  std::vector<int8_t> d(uint64_t(h.planes) * n * h.cols);
  for (int p = 0; p < h.planes; ++p)
    std::memcpy(&d[uint64_t(p) * n * h.cols], &h.d[(uint64_t(p) * h.rows + r0) * h.cols], n * h.cols);
  DevMatrix m = upload_digits(ctx, n, src.cols, h.planes, d.data(), h.scale.data() + r0);
  m.value_width = src.value_width;
  return m;
}

// Balanced base-256 digits of v, each in [-128, 127]: false when v needs
// more than `planes` of them.
bool balanced_digits(int64_t v, int planes, int8_t* d) {
  for (int p = 0; p < planes; ++p) {
    const int64_t lo = ((v + 128) & 255) - 128;
    d[p] = int8_t(lo);
    v = (v - lo) / 256;
  }
  return v == 0;
}

// Row mass bound (det_num/mod.rs:39-42).
void check_row_mass(uint64_t rows, uint64_t cols, const std::vector<int64_t>& mass) {
  for (uint64_t r = 0; r < rows; ++r)
    if (mass[r] >= (int64_t(1) << 31)) bail("weight row mass violates the 2^31 overflow bound");
  (void)cols;
}

DevMatrix upload_matrix(det_ctx* ctx, uint64_t rows, uint64_t cols, int width, const void* values,
                        const int32_t* row_scale) {
  uint64_t elems = 0;
  if (__builtin_mul_overflow(rows, cols, &elems) || elems > UINT64_MAX / 4) bail("tensor shape overflowed");
  if (elems && !values) bail("matrix values pointer is null");
  if (width == 8) {
    if (!row_scale) bail("int8 matrices need a row scale");
    const int8_t* q = static_cast<const int8_t*>(values);
    std::vector<int64_t> mass(rows, 0);
    parallel_rows(rows, [&](uint64_t r0, uint64_t r1) {
      for (uint64_t r = r0; r < r1; ++r) {
        int64_t s = 0;
        for (uint64_t c = 0; c < cols; ++c) s += std::abs(int64_t(q[r * cols + c]));
        mass[r] = s * std::abs(int64_t(row_scale[r]));
      }
    });
    check_row_mass(rows, cols, mass);
    return upload_int8(ctx, rows, cols, q, row_scale);
  }
  if (width != 16 && width != 32) bail("unsupported element width");
  auto at = [&](uint64_t i) -> int32_t {
    return width == 16 ? int32_t(static_cast<const int16_t*>(values)[i]) : static_cast<const int32_t*>(values)[i];
  };
  // Exact int8 factorization: s_r = gcd_c |W[r][c]|, q = W / s_r, valid when
  // every |q| <= 127. Products q*s reproduce the Wgt bits exactly.
  std::vector<int32_t> scale(rows, 1);
  std::vector<int64_t> mass(rows, 0);
  std::vector<uint8_t> row_factors(rows, 1), row_fits16(rows, 1);
  parallel_rows(rows, [&](uint64_t r0, uint64_t r1) {
    for (uint64_t r = r0; r < r1; ++r) {
      uint64_t g = 0, mx = 0;
      int64_t ms = 0;
      bool f16 = true;
      for (uint64_t c = 0; c < cols; ++c) {
        const int32_t v = at(r * cols + c);
        const uint64_t a = uint64_t(std::abs(int64_t(v)));
        g = std::gcd(g, a);
        mx = std::max(mx, a);
        ms += int64_t(a);
        f16 &= v >= INT16_MIN && v <= INT16_MAX;
      }
      mass[r] = ms;
      if (g == 0) g = 1;
      row_factors[r] = mx / g <= 127;
      row_fits16[r] = f16;
      scale[r] = int32_t(g);
    }
  });
  check_row_mass(rows, cols, mass);
  const bool factor = std::all_of(row_factors.begin(), row_factors.end(), [](uint8_t b) { return b != 0; });
  if (factor) {
    std::vector<int8_t> q(rows * cols);
    parallel_rows(rows, [&](uint64_t r0, uint64_t r1) {
      for (uint64_t r = r0; r < r1; ++r)
        for (uint64_t c = 0; c < cols; ++c) q[r * cols + c] = int8_t(at(r * cols + c) / scale[r]);
    });
    return upload_int8(ctx, rows, cols, q.data(), scale.data());
  }
  const bool fits16 = std::all_of(row_fits16.begin(), row_fits16.end(), [](uint8_t b) { return b != 0; });
  if (cols <= 130000) {
    // Digit planes on the int8 MFMA path: each row as s * sum_p 256^p d_p
    // with balanced digits and s = +1 or -1 (whichever sign the row's values
    // fit). Two planes hold every i16 row unless it has values near both
    // ends of the range; four hold every i32 row within the row-mass bound.
    // The products s * (digits) are the Wgt bits exactly.
    for (int planes : {2, 4}) {
      if (planes == 2 && !fits16) continue;
      std::vector<int8_t> d(uint64_t(planes) * rows * cols);
      std::vector<int32_t> sgn(rows, 1);
      bool ok = true;
      std::mutex mu;
      parallel_rows(rows, [&](uint64_t r0, uint64_t r1) {
        bool all = true;
        int8_t dg[4];
        for (uint64_t r = r0; r < r1 && all; ++r) {
          bool row_ok = false;
          for (int32_t sign : {1, -1}) {
            row_ok = true;
            for (uint64_t c = 0; c < cols && row_ok; ++c) {
              row_ok = balanced_digits(int64_t(sign) * at(r * cols + c), planes, dg);
              for (int p = 0; p < planes && row_ok; ++p) d[(uint64_t(p) * rows + r) * cols + c] = dg[p];
            }
            if (row_ok) {
              sgn[r] = sign;
              break;
            }
          }
          all = row_ok;
        }
        if (!all) {
          std::lock_guard<std::mutex> lock(mu);
          ok = false;
        }
      });
      if (!ok) continue;
      DevMatrix m = upload_digits(ctx, rows, cols, planes, d.data(), sgn.data());
      m.value_width = fits16 ? 16 : 32;
      return m;
    }
    contract("weight row fits no digit-plane form");
  }
  // rows longer than the MFMA path takes: wide storage on the vector ALUs
  DevMatrix m;
  m.rows = rows;
  m.cols = cols;
  m.storage = fits16 ? det::kI16 : det::kI32;
  m.value_width = fits16 ? 16 : 32;
  const size_t esz = fits16 ? 2 : 4;
  HIPC(hipMalloc(&m.w, std::max<size_t>(rows * cols * esz, 4)));
  if ((width == 16) == fits16) {
    HIPC(hipMemcpyAsync(m.w, values, rows * cols * esz, hipMemcpyHostToDevice, ctx->stream));
  } else {
    std::vector<int16_t> n16;
    std::vector<int32_t> n32;
    if (fits16) { n16.resize(rows * cols); for (uint64_t i = 0; i < rows * cols; ++i) n16[i] = int16_t(at(i)); }
    else { n32.resize(rows * cols); for (uint64_t i = 0; i < rows * cols; ++i) n32[i] = at(i); }
    HIPC(hipMemcpyAsync(m.w, fits16 ? (const void*)n16.data() : (const void*)n32.data(), rows * cols * esz,
                        hipMemcpyHostToDevice, ctx->stream));
  }
  HIPC(hipStreamSynchronize(ctx->stream));
  return m;
}

int32_t* upload_vec(det_ctx* ctx, const std::vector<int32_t>& v) {
  int32_t* d = nullptr;
  HIPC(hipMalloc(&d, std::max<size_t>(v.size(), 1) * 4));
  HIPC(hipMemcpyAsync(d, v.data(), v.size() * 4, hipMemcpyHostToDevice, ctx->stream));
  HIPC(hipStreamSynchronize(ctx->stream));
  return d;
}

// SHA-256 commitments (transformer_kernels.rs:1395-1482) live in commit.cpp.
using det_commit::commit_rows;
using det_commit::commit_vector;
using det_commit::Sha;
using det_commit::sha_hex;

}  // namespace

// ---------------------------------------------------------------------------
// model
// ---------------------------------------------------------------------------
namespace {

struct HostTensor {
  std::vector<uint64_t> shape;
  std::vector<int32_t> vec;  // rank-1 tensors (Wgt bits)
  DevMatrix mat;             // rank-2 tensors
  bool is_matrix = false;
};

struct GLayer {
  bool sliding = false;
  uint64_t hidden = 0, num_heads = 0, num_kv_heads = 0, head_dim = 0;
  std::optional<uint64_t> sliding_window, cache_sliding_window, donor;
  int64_t eps = 0, rope_base = 0;
  uint64_t rotary = 0, freq_base_dim = 0;
  bool k_eq_v = false;
  const DevMatrix *q = nullptr, *k = nullptr, *v = nullptr, *o = nullptr, *gate = nullptr, *up = nullptr,
                  *down = nullptr, *ple_gate = nullptr, *ple_proj = nullptr;
  int32_t *q_norm = nullptr, *k_norm = nullptr, *in_ln = nullptr, *post_attn_ln = nullptr, *pre_ff_ln = nullptr,
          *post_ff_ln = nullptr, *ple_post_norm = nullptr;
  bool has_ple = false;
  std::optional<int32_t> layer_scalar;
  int64_t* inv_freq = nullptr;  // rotary/2 entries (shared by layers with the same table)
  uint32_t trig_off = 0;        // first cos/sin pair of this layer's table in the step trig buffer
};

}  // namespace

namespace {
struct BatchWs;
void free_batch(BatchWs* b);
}  // namespace

struct det_model {
  det_ctx* ctx = nullptr;
  det_text_config_t cfg{};
  std::vector<int32_t> layer_types;
  std::map<std::string, HostTensor> tensors;
  bool finalized = false;
  // resolved
  const DevMatrix* embedding = nullptr;
  int32_t embed_scale = 0;
  std::vector<GLayer> layers;
  bool has_ple = false;
  uint64_t ple_dim = 0;
  const DevMatrix* ple_tok = nullptr;  // [ple_vocab x L*ple]
  const DevMatrix* ple_proj_full = nullptr;  // [L*ple x hidden]: every layer's projection rows
  std::vector<DevMatrix> ple_proj_views;
  int32_t* ple_proj_norm = nullptr;
  int32_t ple_embedding_scale = 0, ple_projection_scalar = 0, ple_input_scale = 0;
  int32_t* final_norm = nullptr;
  const DevMatrix* lm_head = nullptr;
  std::optional<int32_t> softcap;
  int64_t eps = 0;
  uint64_t hidden = 0, vocab = 0;
  std::vector<void*> owned_dev;
  // fused decode matrices: [q; k; v] rows and interleaved gate/up blocks of 8
  struct Fused {
    DevMatrix qkv, gateup;
    bool has_v = true;
  };
  std::vector<Fused> fused;
  // distinct RoPE tables (layers with the same base, base dim and pair count share one)
  struct RopeKey {
    int64_t base;
    uint64_t fbd, pairs;
  };
  std::vector<std::pair<RopeKey, det::RopeTable>> rope_tables;
  det::RopeTable* rope_tables_dev = nullptr;
  uint32_t trig_pairs = 0;
  bool fused_ok = false;
  // the fused step applies each residual norm inside the next projection
  // (post-attention norm in gate/up, post-FF norm in the next layer's q/k/v)
  bool norm_fused = false;
  // a RoPE base of i64::MAX (theta >= 2^31): the reference's nth_root_acc
  // overflows on it (ops.rs:578) at the first rotation of a position > 0
  bool rope_overflow = false;
  BatchWs* batch = nullptr;  // row scratch of batched decode steps (grown on demand)

  ~det_model() {
    free_batch(batch);
    for (auto& f : fused) { free_matrix(f.qkv); free_matrix(f.gateup); }
    for (auto& v : ple_proj_views) free_matrix(v);
    for (auto& kv : tensors)
      if (kv.second.is_matrix) free_matrix(kv.second.mat);
    for (void* p : owned_dev) (void)hipFree(p);
  }
  const HostTensor& need(const std::string& n) const {
    auto it = tensors.find(n);
    if (it == tensors.end()) bail("missing tensor `" + n + "`");
    return it->second;
  }
  const DevMatrix* need_matrix(const std::string& n) const {
    const HostTensor& t = need(n);
    if (!t.is_matrix) bail("tensor `" + n + "` is not a matrix");
    return &t.mat;
  }
  int32_t* need_vector(const std::string& n, uint64_t expect) {
    const HostTensor& t = need(n);
    if (t.is_matrix) bail("tensor `" + n + "` is not a vector");
    if (expect && t.vec.size() != expect)
      bail("rms norm width mismatch: " + std::to_string(expect) + " vs " + std::to_string(t.vec.size()));
    int32_t* d = upload_vec(ctx, t.vec);
    owned_dev.push_back(d);
    return d;
  }
};

namespace {

// Stacks digit-plane matrices of equal width row-wise (the result takes the
// largest plane count; a row with fewer planes gets zero digits above its
// own); with interleave8 (two inputs of equal height) rows alternate in
// blocks of 8: a[0..8), b[0..8), a[8..16), ...
DevMatrix fuse_rows(det_ctx* ctx, const std::vector<const DevMatrix*>& ms, bool interleave8) {
  const uint64_t cols = ms[0]->cols;
  uint64_t rows = 0;
  int planes = 1, vw = 8;
  std::vector<HostDigits> hs;
  for (const DevMatrix* m : ms) {
    if (m->cols != cols || m->storage != det::kInt8) bail("cannot fuse matrices of different widths");
    hs.push_back(untile(ctx, *m));
    rows += m->rows;
    planes = std::max(planes, m->planes);
    vw = std::max(vw, m->value_width);
  }
  std::vector<int8_t> d(uint64_t(planes) * rows * cols, 0);
  std::vector<int32_t> sc(rows);
  uint64_t r = 0;
  auto put = [&](size_t i, uint64_t src_row) {
    const HostDigits& h = hs[i];
    for (int p = 0; p < h.planes; ++p)
      std::memcpy(&d[(uint64_t(p) * rows + r) * cols], &h.d[(uint64_t(p) * h.rows + src_row) * cols], cols);
    sc[r] = h.scale[src_row];
    ++r;
  };
  if (interleave8) {
    for (uint64_t b = 0; b < ms[0]->rows; b += 8) {
      for (uint64_t j = 0; j < 8; ++j) put(0, b + j);
      for (uint64_t j = 0; j < 8; ++j) put(1, b + j);
    }
  } else {
    for (size_t i = 0; i < ms.size(); ++i)
      for (uint64_t j = 0; j < ms[i]->rows; ++j) put(i, j);
  }
  DevMatrix m = upload_digits(ctx, rows, cols, planes, d.data(), sc.data());
  m.value_width = vw;
  return m;
}

// gemma/io.rs:165-190
std::optional<uint64_t> kv_shared_layer_index(const det_model* m, uint64_t l) {
  const uint64_t ns = m->cfg.has_num_kv_shared_layers ? m->cfg.num_kv_shared_layers : 0;
  const uint64_t L = m->cfg.num_hidden_layers;
  const uint64_t first = L > ns ? L - ns : 0;
  if (ns == 0 || l < first) return std::nullopt;
  for (uint64_t i = first; i-- > 0;)
    if (m->layer_types[i] == m->layer_types[l]) return i;
  bail("Gemma layer " + std::to_string(l) + " is configured to share KV without a prior donor layer");
}

void finalize(det_model* m) {
  const det_text_config_t& c = m->cfg;
  if (c.enable_moe_block) bail("only dense Gemma 4 layers are supported, not MoE checkpoints");
  if (!c.hidden_activation_is_gelu_pytorch_tanh) bail("only gelu_pytorch_tanh is supported");
  if (c.num_hidden_layers != m->layer_types.size()) bail("Gemma config layer count mismatch");
  m->hidden = c.hidden_size;
  m->eps = det::f32_to_acc(c.rms_norm_eps);
  for (const char* n : {"model.language_model.embed_tokens.weight", "language_model.embed_tokens.weight",
                        "embed_tokens.weight"}) {
    auto it = m->tensors.find(n);
    if (it != m->tensors.end() && it->second.is_matrix) { m->embedding = &it->second.mat; break; }
  }
  if (!m->embedding) bail("missing embedding tensor");
  if (m->embedding->cols != c.hidden_size) bail("embedding tensor width mismatch");
  m->embed_scale = det::f32_to_act(std::sqrt(float(m->embedding->cols)));

  std::vector<bool> is_donor(c.num_hidden_layers, false);
  for (uint64_t l = 0; l < c.num_hidden_layers; ++l)
    if (auto d = kv_shared_layer_index(m, l)) is_donor[*d] = true;
  const bool kev = c.has_attention_k_eq_v && c.attention_k_eq_v;
  const uint64_t win = c.bidirectional_all ? c.sliding_window / 2 + 1 : c.sliding_window;
  const uint64_t ple = c.has_hidden_size_per_layer_input ? c.hidden_size_per_layer_input : 0;
  m->layers.assign(c.num_hidden_layers, GLayer());
  for (uint64_t l = 0; l < c.num_hidden_layers; ++l) {
    GLayer& L = m->layers[l];
    const std::string p = "model.language_model.layers." + std::to_string(l);
    L.sliding = m->layer_types[l] == 1;
    L.head_dim = L.sliding ? c.head_dim : (c.has_global_head_dim ? c.global_head_dim : c.head_dim);
    if (L.sliding) L.num_kv_heads = c.num_key_value_heads;
    else if (kev) L.num_kv_heads = c.has_num_global_key_value_heads ? c.num_global_key_value_heads : c.num_key_value_heads;
    else L.num_kv_heads = c.num_key_value_heads;
    const float factor = c.has_full_partial_rotary_factor ? c.full_partial_rotary_factor : 0.25f;
    L.rotary = L.sliding ? L.head_dim : uint64_t(float(L.head_dim) * factor);
    L.donor = kv_shared_layer_index(m, l);
    if (L.sliding) L.sliding_window = win;
    if (L.sliding && !is_donor[l]) L.cache_sliding_window = win;
    const float base = L.sliding ? (c.has_sliding_rope_theta ? c.sliding_rope_theta : 10000.0f)
                                 : (c.has_full_rope_theta ? c.full_rope_theta
                                                          : (c.has_rope_theta ? c.rope_theta : 1000000.0f));
    L.rope_base = det::f32_to_acc(base);
    L.freq_base_dim = L.head_dim;
    L.hidden = c.hidden_size;
    L.num_heads = c.num_attention_heads;
    L.eps = m->eps;
    L.k_eq_v = !L.sliding && kev;
    L.q = m->need_matrix(p + ".self_attn.q_proj.weight");
    L.k = m->need_matrix(p + ".self_attn.k_proj.weight");
    const std::string vn = p + ".self_attn.v_proj.weight";
    if (!L.k_eq_v || m->tensors.count(vn)) L.v = m->need_matrix(vn);
    L.o = m->need_matrix(p + ".self_attn.o_proj.weight");
    L.q_norm = m->need_vector(p + ".self_attn.q_norm.weight", L.head_dim);
    L.k_norm = m->need_vector(p + ".self_attn.k_norm.weight", L.head_dim);
    L.in_ln = m->need_vector(p + ".input_layernorm.weight", L.hidden);
    L.post_attn_ln = m->need_vector(p + ".post_attention_layernorm.weight", L.hidden);
    L.pre_ff_ln = m->need_vector(p + ".pre_feedforward_layernorm.weight", L.hidden);
    L.post_ff_ln = m->need_vector(p + ".post_feedforward_layernorm.weight", L.hidden);
    L.gate = m->need_matrix(p + ".mlp.gate_proj.weight");
    L.up = m->need_matrix(p + ".mlp.up_proj.weight");
    L.down = m->need_matrix(p + ".mlp.down_proj.weight");
    if (ple > 0) {
      L.has_ple = true;
      L.ple_gate = m->need_matrix(p + ".per_layer_input_gate.weight");
      L.ple_proj = m->need_matrix(p + ".per_layer_projection.weight");
      L.ple_post_norm = m->need_vector(p + ".post_per_layer_input_norm.weight", L.hidden);
    }
    auto sc = m->tensors.find(p + ".layer_scalar");
    if (sc != m->tensors.end()) {
      if (sc->second.shape != std::vector<uint64_t>{1}) bail("layer_scalar must have shape [1]");
      L.layer_scalar = sc->second.vec[0];
    }
    // shape checks the kernels rely on
    if (L.num_kv_heads == 0 || L.num_heads / L.num_kv_heads == 0) bail("invalid Gemma head configuration");
    if ((L.num_heads - 1) / (L.num_heads / L.num_kv_heads) >= L.num_kv_heads)
      contract("query head maps past the last KV head");
    if (L.q->cols != L.hidden || L.k->cols != L.hidden || (L.v && L.v->cols != L.hidden))
      bail("attention projection input width mismatch");
    if (L.q->rows != L.num_heads * L.head_dim) bail("q_proj rows do not match heads x head_dim");
    if (L.k->rows != L.num_kv_heads * L.head_dim || (L.v && L.v->rows != L.k->rows))
      bail("k/v_proj rows do not match kv heads x head_dim");
    if (L.o->cols != L.num_heads * L.head_dim || L.o->rows != L.hidden) bail("o_proj shape mismatch");
    if (L.gate->cols != L.hidden || L.up->cols != L.hidden || L.gate->rows != L.up->rows) bail("gate/up shape mismatch");
    if (L.down->cols != L.gate->rows || L.down->rows != L.hidden) bail("down_proj shape mismatch");
    if (L.has_ple && (L.ple_gate->cols != L.hidden || L.ple_proj->cols != L.ple_gate->rows || L.ple_proj->rows != L.hidden ||
                      L.ple_gate->rows != ple))
      bail("per-layer input projection shape mismatch");
    if (L.rotary) {
      if (L.rotary % 2) contract("rope_rotate_pairs requires an even rotary_dim");
      if (L.rotary > L.head_dim) contract("rope_rotate_pairs requires rotary_dim to fit within the input width");
      if (L.freq_base_dim < 2 || L.freq_base_dim % 2) contract("rope_rotate_pairs requires an even freq_base_dim of at least 2");
      if (L.rope_base <= 0) contract("rope_rotate_pairs requires a positive base");
      const det_model::RopeKey key{L.rope_base, L.freq_base_dim, L.rotary / 2};
      for (const auto& [k, t] : m->rope_tables)
        if (k.base == key.base && k.fbd == key.fbd && k.pairs == key.pairs) {
          L.inv_freq = const_cast<int64_t*>(t.inv_freq);
          L.trig_off = t.offset;
        }
      if (!L.inv_freq) {
        std::vector<int64_t> tab(L.rotary / 2, 0);
        if (L.rope_base == INT64_MAX && L.freq_base_dim / 2 > 1) m->rope_overflow = true;  // table never used
        else det::rope_inv_freq_table(L.rope_base, uint32_t(L.freq_base_dim), uint32_t(L.rotary / 2), tab.data());
        HIPC(hipMalloc(&L.inv_freq, tab.size() * 8));
        HIPC(hipMemcpy(L.inv_freq, tab.data(), tab.size() * 8, hipMemcpyHostToDevice));
        m->owned_dev.push_back(L.inv_freq);
        L.trig_off = m->trig_pairs;
        m->rope_tables.push_back({key, det::RopeTable{L.inv_freq, uint32_t(L.rotary / 2), m->trig_pairs}});
        m->trig_pairs += uint32_t(L.rotary / 2);
      }
    }
  }
  if (ple > 0) {
    m->has_ple = true;
    m->ple_dim = ple;
    const uint64_t pv = c.has_vocab_size_per_layer_input ? c.vocab_size_per_layer_input : c.vocab_size;
    m->ple_tok = m->need_matrix("model.language_model.embed_tokens_per_layer.weight");
    const DevMatrix* proj = m->need_matrix("model.language_model.per_layer_model_projection.weight");
    if (m->ple_tok->rows < pv || m->ple_tok->cols < c.num_hidden_layers * ple) bail("PLE token embedding shape mismatch");
    if (proj->rows < c.num_hidden_layers * ple || proj->cols != c.hidden_size) bail("PLE model projection shape mismatch");
    for (uint64_t l = 0; l < c.num_hidden_layers; ++l) {
      m->ple_proj_views.push_back(extract_rows(m->ctx, *proj, l * ple, ple));
    }
    m->ple_proj_full = proj;
    m->ple_proj_norm = m->need_vector("model.language_model.per_layer_projection_norm.weight", ple);
    m->ple_embedding_scale = det::f32_to_act(std::sqrt(float(ple)));
    m->ple_projection_scalar = det::f32_to_act(std::pow(float(c.hidden_size), -0.5f));
    m->ple_input_scale = det::f32_to_act(std::pow(2.0f, -0.5f));
  }
  m->final_norm = m->need_vector("model.language_model.norm.weight", c.hidden_size);
  const bool tied = c.has_tie_word_embeddings ? c.tie_word_embeddings != 0 : true;
  m->lm_head = tied ? m->embedding : m->need_matrix("model.language_model.lm_head.weight");
  if (m->lm_head->cols != c.hidden_size) bail("logits projection input width mismatch");
  m->vocab = m->lm_head->rows;
  if (c.has_final_logit_softcapping) {
    m->softcap = det::f32_to_act(c.final_logit_softcapping);
    if (*m->softcap <= 0) contract("softcap_act requires a strictly positive softcap");
  }
  // The fused, graph-captured decode step covers int8 models whose shapes
  // fit its kernels, with or without PLE; everything else runs the per-op
  // sequence.
  auto gemv_ok = [](const DevMatrix* w) { return w->storage == det::kInt8 && det::gemv_fits_lds(*w, 1); };
  bool ok = m->hidden <= det::kDecMaxHidden && gemv_ok(m->lm_head);
  if (m->has_ple) {
    ok = ok && gemv_ok(m->ple_proj_full);
    for (const GLayer& L : m->layers)
      if (L.has_ple && (!gemv_ok(L.ple_gate) || !gemv_ok(L.ple_proj))) ok = false;
  }
  for (const GLayer& L : m->layers) {
    for (const DevMatrix* w : {L.q, L.k, L.v, L.o, L.gate, L.up, L.down})
      if (w && (w->storage != det::kInt8 || !det::gemv_fits_lds(*w, 1))) ok = false;
    if (L.head_dim % 4 || L.head_dim > det::kDecMaxHeadDim || L.num_heads % L.num_kv_heads ||
        L.num_heads / L.num_kv_heads > det::kDecMaxGroup || L.gate->rows % 8)
      ok = false;
  }
  if (ok) {
    m->fused.resize(m->layers.size());
    for (size_t l = 0; l < m->layers.size(); ++l) {
      const GLayer& L = m->layers[l];
      auto& F = m->fused[l];
      F.has_v = L.v != nullptr;
      // layers reading a donor's cache need the query rows only
      std::vector<const DevMatrix*> parts = {L.q};
      if (!L.donor) {
        parts.push_back(L.k);
        if (L.v) parts.push_back(L.v);
      }
      F.qkv = fuse_rows(m->ctx, parts, false);
      F.gateup = fuse_rows(m->ctx, {L.gate, L.up}, true);
      if (!det::gemv_fits_lds(F.qkv, 1) || !det::gemv_fits_lds(F.gateup, 1)) ok = false;
      // the normalised row's limb planes feed qkv, gate/up and the logits projection
      if (F.qkv.kpad != m->lm_head->kpad || F.gateup.kpad != m->lm_head->kpad) ok = false;
    }
  }
  if (ok && !m->rope_tables.empty()) {
    std::vector<det::RopeTable> tabs;
    for (const auto& kt : m->rope_tables) tabs.push_back(kt.second);
    HIPC(hipMalloc(&m->rope_tables_dev, tabs.size() * sizeof(det::RopeTable)));
    m->owned_dev.push_back(m->rope_tables_dev);
    HIPC(hipMemcpy(m->rope_tables_dev, tabs.data(), tabs.size() * sizeof(det::RopeTable), hipMemcpyHostToDevice));
  }
  m->fused_ok = ok;
  // the O projection's accumulators are complete rows (plain stores), which
  // the gate/up projection's norm reads from every workgroup
  bool nf = ok;
  if (ok)
    for (size_t l = 0; l < m->layers.size(); ++l)
      if (!det::gemv_norm_fits(m->fused[l].qkv, m->hidden) || !det::gemv_norm_fits(m->fused[l].gateup, m->hidden) ||
          !det::gemv_decode_acc_plain(*m->layers[l].o))
        nf = false;
  m->norm_fused = nf;
  m->finalized = true;
}

// detwgt v2 reader (gemma/io.rs:224-387, DETWGT_V2_FORMAT.md), also reading
// the int8 variant detwgt-q8 written by rasterdet.detwgt.
void load_detwgt(det_model* m, const uint8_t* b, size_t len) {
  size_t cur = 0;
  auto take = [&](size_t n) {
    if (n > len - cur) bail("artifact ended unexpectedly");
    const uint8_t* p = b + cur;
    cur += n;
    return p;
  };
  auto rd32 = [&]() { uint32_t v; std::memcpy(&v, take(4), 4); return v; };
  auto rd64 = [&]() { uint64_t v; std::memcpy(&v, take(8), 8); return v; };
  // detwgt v2, or detwgt-q8 (same records; rank >= 2 tensors may be int8 q
  // plus one i32 scale per row, W = q * s)
  const uint8_t* magic = take(8);
  const bool q8 = std::memcmp(magic, "DNWGTQ8\0", 8) == 0;
  if (!q8 && std::memcmp(magic, "DNWGTV0\0", 8) != 0) bail("unsupported deterministic artifact magic");
  if (rd32() != (q8 ? 1u : 2u))
    bail(q8 ? "unsupported detwgt-q8 format version; expected 1"
            : "unsupported deterministic artifact format version; expected 2");
  if (rd32() != 1) bail("unsupported deterministic artifact det_num spec version; expected 1");
  const uint64_t count = rd64();
  struct Rec { std::string name; std::vector<uint64_t> shape; int width; const uint8_t* data; const int32_t* scale; };
  std::vector<std::vector<int32_t>> scales;
  scales.reserve(count);
  std::vector<Rec> recs;
  std::map<std::string, int> seen;
  for (uint64_t i = 0; i < count; ++i) {
    const uint32_t nl = rd32();
    std::string name(reinterpret_cast<const char*>(take(nl)), nl);
    const uint32_t rank = rd32();
    // every dimension is 8 bytes of the artifact: a rank the remaining bytes
    // cannot hold ends the artifact before any allocation
    if (rank > (len - cur) / 8) bail("artifact ended unexpectedly");
    std::vector<uint64_t> shape(rank);
    uint64_t prod = 1;
    for (auto& d : shape) {
      d = rd64();
      if (__builtin_mul_overflow(prod, d, &prod)) bail("tensor shape overflowed");
    }
    if (rd64() != prod) bail("tensor `" + name + "` element count mismatch");
    const uint32_t width = rd32();
    if (width != 16 && width != 32 && !(q8 && width == 8 && rank >= 2))
      bail("tensor `" + name + "` has an invalid element width");
    // gemma/io.rs:327-331: element_count.checked_mul(byte width)
    uint64_t payload = 0;
    if (__builtin_mul_overflow(prod, uint64_t(width / 8), &payload)) bail("tensor payload byte count overflowed");
    if (rd64() != payload) bail("tensor `" + name + "` payload length mismatch");
    const uint64_t mass = rd64();
    if (rank >= 2 && mass >= (uint64_t(1) << 31)) bail("tensor `" + name + "` max row mass violates the overflow bound");
    const uint64_t rows = (width == 8 && shape.back()) ? prod / shape.back() : 0;
    uint64_t scale_bytes = 0;
    if (__builtin_mul_overflow(rows, uint64_t(4), &scale_bytes)) bail("tensor `" + name + "` scale byte count overflowed");
    if (width == 8 && rd64() != rows) bail("tensor `" + name + "` scale count mismatch");
    auto pad = [&]() {
      const size_t n = (64 - cur % 64) % 64;
      const uint8_t* pp = take(n);
      for (size_t k = 0; k < n; ++k)
        if (pp[k]) bail("tensor `" + name + "` has non-zero payload alignment padding");
    };
    pad();
    const uint8_t* data = take(payload);
    const int32_t* scale = nullptr;
    if (width == 8) {
      pad();
      const uint8_t* sp = take(scale_bytes);
      scales.emplace_back(rows);
      if (rows) std::memcpy(scales.back().data(), sp, scale_bytes);
      scale = scales.back().data();
      // W = q * s must be a canonical (i32) Wgt value
      const uint64_t cols = shape.back();
      for (uint64_t r = 0; r < rows; ++r) {
        int64_t mx = 0;
        for (uint64_t c = 0; c < cols; ++c) mx = std::max<int64_t>(mx, std::abs(int64_t(int8_t(data[r * cols + c]))));
        if (mx * std::abs(int64_t(scale[r])) > INT32_MAX)
          bail("tensor `" + name + "` has q * scale values outside i32");
      }
    }
    if (seen.count(name)) bail("deterministic artifact contains duplicate tensor `" + name + "`");
    seen[name] = 1;
    recs.push_back({name, shape, int(width), data, scale});
  }
  if (cur != len) bail("deterministic artifact has trailing bytes after tensor payloads");
  for (const Rec& r : recs) {
    if (r.shape.size() > 2 || r.shape.empty()) continue;  // only vectors and matrices are used on this path
    uint64_t dims[2] = {r.shape[0], r.shape.size() > 1 ? r.shape[1] : 0};
    const int st = det_model_set_tensor(m, r.name.c_str(), r.shape.size(), dims, r.width, r.data, r.scale);
    if (st) throw Status(st, m->ctx->last_error);
  }
}

// ---------------------------------------------------------------------------
// per-sequence state
// ---------------------------------------------------------------------------
struct GKv {
  bool has = false;  // LayerKvCache::det is Some
  int32_t* k = nullptr;
  int32_t* v = nullptr;
  uint64_t cap = 0, row_w = 0, heads = 0, hd = 0;
  bool ring = false;  // sliding-window cache of capacity == window
  uint64_t start = 0, len = 0;
  uint64_t total = 0;  // tokens appended so far; token t sits at slot t % cap (ring) or t
  // tokens the cache may take in all: a ring smaller than its window (a
  // layer-level cache created for fewer tokens than the window) would
  // otherwise overwrite rows the window still reads
  uint64_t limit = UINT64_MAX;
};

}  // namespace

struct det_session {
  det_model* m = nullptr;
  det_ctx* ctx = nullptr;  // m->ctx, kept so that freeing the session does not read the model
  uint64_t max_tokens = 0, position = 0;
  std::vector<GKv> kv;
  // device scratch (sized for max_tokens rows)
  uint32_t* ids = nullptr;
  int32_t *x = nullptr, *x2 = nullptr, *normed = nullptr, *qb = nullptr, *kb = nullptr, *vb = nullptr,
          *attn = nullptr, *gate = nullptr, *up = nullptr, *ple_all = nullptr, *pe = nullptr, *pp = nullptr,
          *logits = nullptr, *dec_in = nullptr;
  std::vector<void*> owned;
  bool logits_valid = false;
  // fused decode step (HIP graph)
  det::StepState* st_dev = nullptr;
  int32_t *scores = nullptr, *hbuf = nullptr;
  // projection accumulators (wrapping Q32.32); each consumer kernel clears
  // what it reads, so they are zero whenever a step starts
  int64_t *qkv_acc = nullptr, *o_acc = nullptr, *ff_acc = nullptr;
  // the residual row alternates between x and x_alt where a projection
  // applies the residual norm (its workgroups read one while one writes the other)
  int32_t* x_alt = nullptr;
  // limb planes (4 x kpad bytes) of the normalised row and of the MLP hidden row
  int8_t *limbs_x = nullptr, *limbs_ff = nullptr;
  uint64_t kpad_x = 0;
  // PLE of the fused step: every layer's per-layer input of the step token
  // ([L*ple], then the model projection rows), the gate row and the
  // projection accumulators (cleared by their consumer)
  int32_t *ple_in_all = nullptr, *ple_pp = nullptr, *ple_g = nullptr;
  int64_t* ple_acc = nullptr;
  int64_t* attn_acc = nullptr;
  int64_t* attn_keys = nullptr;      // per-chunk argmax keys of the scores
  det::AttnStat* attn_stats = nullptr;  // per-head softmax statistics
  int32_t* trig = nullptr;  // cos/sin pairs of every RoPE table at the step position
  int64_t* am_scratch = nullptr;
  uint32_t* am_out = nullptr;
  uint64_t score_stride = 0;
  // checkpointed decode: every layer's output row of the last step ([layers][hidden])
  bool capture_layers = false;
  int32_t* layer_rows = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;

  ~det_session() {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    for (auto& c : kv) {
      if (c.k) (void)hipFree(c.k);
      if (c.v) (void)hipFree(c.v);
    }
    for (void* p : owned) (void)hipFree(p);
  }
  template <class T>
  T* alloc(uint64_t n) {
    void* p = nullptr;
    HIPC(hipMalloc(&p, std::max<uint64_t>(n, 1) * sizeof(T)));
    owned.push_back(p);
    return static_cast<T*>(p);
  }
};

// A layer's KV cache outside a session (LayerKvCache, shared/model/transformer.rs:278-337),
// for the layer-level entry points.
struct det_kv {
  det_model* m = nullptr;
  det_ctx* ctx = nullptr;  // m->ctx, kept so that freeing the cache does not read the model
  uint64_t layer = 0;
  GKv c;
  ~det_kv() {
    if (c.k) (void)hipFree(c.k);
    if (c.v) (void)hipFree(c.v);
  }
};

// Row buffers reused by the layer-level entry points (DetDecodeScratch,
// det_kernels.rs:830-864), grown on demand to the largest row count seen.
struct det_scratch {
  det_model* m = nullptr;
  det_ctx* ctx = nullptr;  // m->ctx, kept so that freeing the scratch does not read the model
  std::unique_ptr<det_session> ws;
};

namespace {

// Allocates a session's row buffers for max_tokens rows; with_state adds the
// per-layer KV caches and the fused decode step's buffers (a workspace for
// the layer-level entry points has neither).
void session_alloc(det_session* s, bool with_state = true) {
  det_model* m = s->m;
  s->ctx = m->ctx;
  const uint64_t T = s->max_tokens, H = m->hidden;
  uint64_t qw = 0, kw = 0, ffw = 0, plew = m->ple_dim;
  for (const GLayer& L : m->layers) {
    qw = std::max(qw, L.num_heads * L.head_dim);
    kw = std::max(kw, L.num_kv_heads * L.head_dim);
    ffw = std::max(ffw, L.gate->rows);
  }
  s->ids = s->alloc<uint32_t>(T);
  s->x = s->alloc<int32_t>(T * H);
  s->x2 = s->alloc<int32_t>(T * H);
  s->normed = s->alloc<int32_t>(T * std::max(H, qw));
  s->qb = s->alloc<int32_t>(T * qw);
  s->kb = s->alloc<int32_t>(T * kw);
  s->vb = s->alloc<int32_t>(T * kw);
  s->attn = s->alloc<int32_t>(T * std::max(H, qw));
  s->gate = s->alloc<int32_t>(T * std::max(ffw, H));
  s->up = s->alloc<int32_t>(T * std::max(ffw, H));
  s->ple_all = s->alloc<int32_t>(T * m->layers.size() * std::max<uint64_t>(plew, 1));
  s->pe = s->alloc<int32_t>(T * std::max<uint64_t>(plew, 1));
  s->pp = s->alloc<int32_t>(T * std::max<uint64_t>(std::max(plew, H), 1));
  s->logits = s->alloc<int32_t>(m->vocab);
  s->dec_in = s->alloc<int32_t>(H);
  s->kv.assign(m->layers.size(), GKv());
  if (!with_state) return;
  if (s->capture_layers) s->layer_rows = s->alloc<int32_t>(m->layers.size() * H);
  if (m->fused_ok) {
    uint64_t fr = 0, nhd = 0, ff = 0;
    for (size_t l = 0; l < m->layers.size(); ++l) {
      fr = std::max(fr, m->fused[l].qkv.rows);
      nhd = std::max(nhd, m->layers[l].num_heads * m->layers[l].head_dim);
      ff = std::max(ff, m->layers[l].gate->rows);
    }
    uint64_t nh = 0;
    for (const GLayer& L : m->layers) nh = std::max(nh, L.num_heads);
    s->score_stride = T;  // no attention window exceeds the session length
    s->qkv_acc = s->alloc<int64_t>(fr);
    s->o_acc = s->alloc<int64_t>(H);
    s->ff_acc = s->alloc<int64_t>(H);
    s->x_alt = s->alloc<int32_t>(H);
    uint64_t kff = 0;
    for (const GLayer& L : m->layers) kff = std::max(kff, L.down->kpad);
    s->kpad_x = m->fused[0].qkv.kpad;
    s->limbs_x = s->alloc<int8_t>(4 * s->kpad_x);
    s->limbs_ff = s->alloc<int8_t>(4 * kff);
    hipStream_t zst = m->ctx->stream;  // stream-ordered before any step (not inside a graph)
    HIPC(hipMemsetAsync(s->limbs_x, 0, 4 * s->kpad_x, zst));
    HIPC(hipMemsetAsync(s->limbs_ff, 0, 4 * kff, zst));
    HIPC(hipMemsetAsync(s->qkv_acc, 0, fr * 8, zst));
    HIPC(hipMemsetAsync(s->o_acc, 0, H * 8, zst));
    HIPC(hipMemsetAsync(s->ff_acc, 0, H * 8, zst));
    s->scores = s->alloc<int32_t>(nh * T);
    s->attn_keys = s->alloc<int64_t>(nh * ((T + det::kAttnScoreRows - 1) / det::kAttnScoreRows));
    s->attn_stats = s->alloc<det::AttnStat>(nh);
    s->attn_acc = s->alloc<int64_t>(nhd);
    s->hbuf = s->alloc<int32_t>(ff);
    s->am_scratch = s->alloc<int64_t>((m->vocab + 1023) / 1024);
    s->am_out = s->alloc<uint32_t>(1);
    s->st_dev = s->alloc<det::StepState>(1);
    s->trig = s->alloc<int32_t>(2 * uint64_t(std::max<uint32_t>(m->trig_pairs, 1)));
    if (m->has_ple) {
      const uint64_t rows = std::max<uint64_t>(m->ple_proj_full->rows, m->layers.size() * m->ple_dim);
      s->ple_in_all = s->alloc<int32_t>(rows);
      s->ple_pp = s->alloc<int32_t>(rows);
      s->ple_g = s->alloc<int32_t>(m->ple_dim);
      s->ple_acc = s->alloc<int64_t>(H);
      HIPC(hipMemsetAsync(s->ple_acc, 0, H * 8, zst));
    }
  }
  for (size_t l = 0; l < m->layers.size(); ++l) {
    const GLayer& L = m->layers[l];
    GKv& c = s->kv[l];
    c.heads = L.num_kv_heads;
    c.hd = L.head_dim;
    c.row_w = L.num_kv_heads * L.head_dim;
    if (L.donor) continue;  // shared layers never hold det data
    c.ring = L.cache_sliding_window.has_value();
    c.cap = c.ring ? std::min<uint64_t>(*L.cache_sliding_window, T) : T;
    if (c.ring && c.cap == 0) c.cap = 1;
    HIPC(hipMalloc(&c.k, std::max<uint64_t>(c.cap * c.row_w, 1) * 4));
    HIPC(hipMalloc(&c.v, std::max<uint64_t>(c.cap * c.row_w, 1) * 4));
  }
}

// The logical rows of a cache (oldest to newest) copied to the host as
// [len][row_w]: at most two contiguous spans of a ring.
std::vector<int32_t> host_rows(det_ctx* ctx, const GKv& c, int side) {
  std::vector<int32_t> out(std::max<uint64_t>(c.len * c.row_w, 1));
  const int32_t* base = side ? c.v : c.k;
  const uint64_t first = c.ring ? std::min(c.len, c.cap - c.start) : c.len;
  if (first)
    HIPC(hipMemcpyAsync(out.data(), base + c.start * c.row_w, first * c.row_w * 4, hipMemcpyDeviceToHost, ctx->stream));
  if (c.len > first)
    HIPC(hipMemcpyAsync(out.data() + first * c.row_w, base, (c.len - first) * c.row_w * 4, hipMemcpyDeviceToHost,
                        ctx->stream));
  return out;
}

// The rows of the given layers' caches on the host, for one KV commitment:
// the copies are enqueued here and complete at the next stream synchronize.
struct KvHost {
  bool some = true;  // every cache holds det data
  std::vector<const GKv*> caches;
  std::vector<std::vector<int32_t>> keys, vals;
};

KvHost fetch_kv(det_ctx* ctx, const std::vector<const GKv*>& caches) {
  KvHost h;
  for (const GKv* c : caches)
    if (!c->has) {
      h.some = false;
      return h;
    }
  h.caches = caches;
  for (const GKv* c : caches) {
    h.keys.push_back(host_rows(ctx, *c, 0));
    h.vals.push_back(host_rows(ctx, *c, 1));
  }
  return h;
}

// build_det_kv_cache_commitment (transformer_kernels.rs:1460-1482) over
// fetched rows (after the synchronize); false (None) when a cache has no det data.
bool hash_kv(const KvHost& h, char out[65]) {
  if (!h.some) {
    out[0] = 0;
    return false;
  }
  std::vector<det_commit::KvLayerView> views;
  for (size_t i = 0; i < h.caches.size(); ++i) {
    det_commit::KvLayerView v;
    v.has = true;
    v.heads = h.caches[i]->heads;
    v.hd = h.caches[i]->hd;
    v.len = h.caches[i]->len;
    const int32_t* k = h.keys[i].data();
    const int32_t* vv = h.vals[i].data();
    const uint64_t w = h.caches[i]->row_w;
    v.row = [k, vv, w](int side, uint64_t r) { return (side ? vv : k) + r * w; };
    views.push_back(std::move(v));
  }
  const std::string d = det_commit::commit_kv(views);
  std::memcpy(out, d.c_str(), 65);
  return true;
}

bool commit_kv(det_ctx* ctx, const std::vector<const GKv*>& caches, char out[65]) {
  const KvHost h = fetch_kv(ctx, caches);
  HIPC(hipStreamSynchronize(ctx->stream));
  return hash_kv(h, out);
}

// The KV commitments of several sessions' caches: one synchronize for all
// the copies, then one hashing thread per session (at most the host's cores).
void commit_kv_sessions(det_ctx* ctx, const std::vector<std::vector<const GKv*>>& sets, std::vector<char*> outs) {
  std::vector<KvHost> hs;
  for (const auto& set : sets) hs.push_back(fetch_kv(ctx, set));
  HIPC(hipStreamSynchronize(ctx->stream));
  const size_t n = hs.size();
  const size_t nt = std::max<size_t>(1, std::min<size_t>(n, std::max(1u, std::thread::hardware_concurrency())));
  std::vector<std::thread> pool;
  for (size_t t = 0; t < nt; ++t)
    pool.emplace_back([&, t] {
      for (size_t i = t; i < n; i += nt) hash_kv(hs[i], outs[i]);
    });
  for (auto& th : pool) th.join();
}

std::vector<const GKv*> all_caches(det_session* s) {
  std::vector<const GKv*> v;
  for (auto& c : s->kv) v.push_back(&c);
  return v;
}

void linear(det_ctx* ctx, const DevMatrix& W, const int32_t* act, uint64_t m, int32_t* out) {
  ctx->linear(W, act, m, W.cols, out, W.rows, nullptr);
}

void copy_d2d(det_ctx* ctx, void* dst, const void* src, uint64_t bytes) {
  if (bytes) HIPC(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
}

// Q/K/V projections + head norms + RoPE for M rows at positions pos0.. (det_kernels.rs:499-566, 930-985).
// positions: one device position per row (batched decode) instead of pos0 + row.
// With `cache`, the final K/V rows of tokens t >= cache_from are also written
// to their canonical slots (t % cap on a ring, else t) when the head-norm
// kernel takes the shape; returns whether it did.
// With `plan` (the MFMA attention's work area), the head-norm kernel also
// writes the Q operand blocks, and the K blocks with `k_blocks`; *split_done
// receives the blocks it wrote (1: Q, 2: K) for AttnArgs::split_done.
bool qkv_block(det_session* s, const GLayer& L, uint64_t M, uint64_t pos0, const uint64_t* positions = nullptr,
               const GKv* cache = nullptr, uint64_t cache_from = 0, const det::AttnMfmaArgs* plan = nullptr,
               bool k_blocks = false, uint32_t* split_done = nullptr) {
  if (split_done) *split_done = 0;
  det_ctx* ctx = s->m->ctx;
  hipStream_t st = ctx->stream;
  const uint64_t qw = L.num_heads * L.head_dim, kw = L.num_kv_heads * L.head_dim;
  // with the fused [q; k; v] matrix of the decode step, one GEMM writes the
  // three row buffers (its rows split at whole 16-row tiles)
  const det_model* m = s->m;
  const size_t li = size_t(&L - m->layers.data());
  const det::DevMatrix* QKV = (m->fused_ok && li < m->fused.size()) ? &m->fused[li].qkv : nullptr;
  if (L.v && QKV && M >= det_ctx::kGemmMinRows && QKV->storage == det::kInt8 && QKV->planes <= 2 && QKV->rows == qw + 2 * kw &&
      L.q->rows == qw && L.k->rows == kw && L.v->rows == kw && qw % 16 == 0 && kw % 16 == 0) {
    ctx->ensure_gemm_a(det::gemm_act_bytes(M, QKV->kpad));
    det::launch_gemm_limbs(s->normed, M, QKV->cols, L.q->cols, QKV->kpad, ctx->gemm_a, st);
    det::RowSplit sp;
    sp.out1 = s->kb;
    sp.out2 = s->vb;
    sp.ld1 = sp.ld2 = kw;
    sp.r1 = qw;
    sp.r2 = qw + kw;
    det::launch_gemm_tiled(*QKV, M, s->qb, qw, nullptr, ctx->gemm_a, st, &sp, ctx->gemm_planes_for(*QKV, M));
  } else if (L.v) {
    ctx->linear_group({{L.q, s->qb}, {L.k, s->kb}, {L.v, s->vb}}, s->normed, M, L.q->cols);
  } else if (L.k_eq_v) {
    ctx->linear_group({{L.q, s->qb}, {L.k, s->kb}}, s->normed, M, L.q->cols);
    copy_d2d(ctx, s->vb, s->kb, M * kw * 4);
  } else {
    bail("Gemma layer is missing v_proj without attention_k_eq_v enabled");
  }
  // head norms and RoPE in one launch where the shape allows
  det::HeadNormRope hn;
  hn.q = s->qb;
  hn.k = s->kb;
  hn.v = s->vb;
  hn.q_gain = L.q_norm;
  hn.k_gain = L.k_norm;
  hn.nh = uint32_t(L.num_heads);
  hn.nkv = uint32_t(L.num_kv_heads);
  hn.hd = uint32_t(L.head_dim);
  hn.half = uint32_t(L.rotary / 2);
  hn.eps = L.eps;
  hn.inv_freq = L.inv_freq;
  hn.pos0 = pos0;
  hn.positions = positions;
  if (cache) {
    hn.kc = cache->k;
    hn.vc = cache->v;
    hn.kv_from = cache_from;
    hn.kv_cap = cache->cap;
    hn.kv_ring = cache->ring ? 1 : 0;
  }
  if (plan) {
    hn.qlimbs = plan->qlimbs;
    hn.qsum = plan->qsum;
    hn.nqt = plan->nqt;
    if (k_blocks) {
      hn.klimbs = plan->klimbs;
      hn.ksum = plan->ksum;
      hn.nkt = plan->nkt;
    }
  }
  if (det::launch_head_norm_rope(hn, M, st)) {
    if (split_done && plan) *split_done = k_blocks ? 3u : 1u;
    return cache != nullptr;
  }
  det::launch_rmsnorm(s->qb, M * L.num_heads, L.head_dim, L.head_dim, L.q_norm, L.eps, st);
  det::launch_rmsnorm(s->kb, M * L.num_kv_heads, L.head_dim, L.head_dim, L.k_norm, L.eps, st);
  det::launch_rmsnorm(s->vb, M * L.num_kv_heads, L.head_dim, L.head_dim, nullptr, L.eps, st);
  if (L.rotary && positions) {
    det::launch_rope_rows(s->qb, M, qw, L.num_heads, L.head_dim, L.rotary / 2, L.inv_freq, positions, st);
    det::launch_rope_rows(s->kb, M, kw, L.num_kv_heads, L.head_dim, L.rotary / 2, L.inv_freq, positions, st);
  } else if (L.rotary) {
    det::launch_rope(s->qb, M, qw, L.num_heads, L.head_dim, L.rotary / 2, L.inv_freq, pos0, 1, st);
    det::launch_rope(s->kb, M, kw, L.num_kv_heads, L.head_dim, L.rotary / 2, L.inv_freq, pos0, 1, st);
  }
  return false;
}

// Everything after attention: O proj, norms, residuals, MLP, PLE, scalar
// (det_kernels.rs:733-818 / 1054-1128). Input residual in s->x, combined
// attention heads in s->attn; result in s->x.
// With `next`, the last residual norm of the layer, the layer scalar and the
// next layer's input norm run as one pass that also leaves next's normalised
// rows in s->normed; returns whether it did.
bool post_attention(det_session* s, const GLayer& L, uint64_t M, const int32_t* ple_in,
                    const GLayer* next = nullptr) {
  det_ctx* ctx = s->m->ctx;
  hipStream_t st = ctx->stream;
  const uint64_t H = L.hidden;
  linear(ctx, *L.o, s->attn, M, s->x2);
  // x = add_sat(norm(o), x); normed = norm(x) (pre-FF)
  det::launch_rmsnorm_add_norm(s->x, s->x2, s->normed, M, H, H, L.post_attn_ln, L.pre_ff_ln, L.eps, st);
  // with the decode step's interleaved gate/up matrix, one GEMM whose
  // epilogue forms gelu(gate) * up
  const det_model* m = s->m;
  const size_t li = size_t(&L - m->layers.data());
  const det::DevMatrix* GU = (m->fused_ok && li < m->fused.size()) ? &m->fused[li].gateup : nullptr;
  if (GU && M >= det_ctx::kGemmMinRows && GU->storage == det::kInt8 && GU->planes <= 2 && GU->rows == 2 * L.gate->rows &&
      GU->cols == H && L.gate->rows % 8 == 0) {
    ctx->ensure_gemm_a(det::gemm_act_bytes(M, GU->kpad));
    det::launch_gemm_limbs(s->normed, M, H, H, GU->kpad, ctx->gemm_a, st);
    det::launch_gemm_tiled_gelu(*GU, M, s->gate, L.gate->rows, ctx->gemm_a, st);
  } else {
    ctx->linear_group({{L.gate, s->gate}, {L.up, s->up}}, s->normed, M, H);
    det::launch_gelu_mul(s->gate, s->up, M * L.gate->rows, st);
  }
  linear(ctx, *L.down, s->gate, M, s->x2);
  const bool ple = L.has_ple && ple_in;
  const bool fuse_next = next && next->hidden == H && next->eps == L.eps;
  // x = add_sat(norm(x2) * w, x), times the layer scalar; then next's input norm
  auto last_norm = [&](const int32_t* w) {
    if (fuse_next) {
      det::launch_rmsnorm_add_norm(s->x, s->x2, s->normed, M, H, H, w, next->in_ln, L.eps, st,
                                   L.layer_scalar.has_value(), L.layer_scalar.value_or(0));
    } else {
      det::launch_rmsnorm_add(s->x, s->x2, s->x, M, H, H, w, L.eps, st);
      if (L.layer_scalar) det::launch_scale(s->x, M * H, *L.layer_scalar, st);
    }
  };
  if (!ple) {
    last_norm(L.post_ff_ln);
    return fuse_next;
  }
  det::launch_rmsnorm_add(s->x, s->x2, s->x, M, H, H, L.post_ff_ln, L.eps, st);
  const uint64_t P = L.ple_gate->rows;
  linear(ctx, *L.ple_gate, s->x, M, s->gate);
  det::launch_gelu_mul(s->gate, ple_in, M * P, st);
  linear(ctx, *L.ple_proj, s->gate, M, s->x2);
  last_norm(L.ple_post_norm);
  return fuse_next;
}

// PLE inputs for M tokens of one layer into out [M x P]
// (prefill_prepare_aux/native/tiles.rs:111-243, det_kernels.rs:1142-1208).
void ple_inputs(det_session* s, uint64_t l, const uint32_t* ids_dev, const int32_t* input, uint64_t M, int32_t* out) {
  det_model* m = s->m;
  det_ctx* ctx = m->ctx;
  hipStream_t st = ctx->stream;
  const uint64_t P = m->ple_dim;
  det::launch_gather_rows(*m->ple_tok, ids_dev, M, l * P, P, m->ple_embedding_scale, out, P, st);
  ctx->linear(m->ple_proj_views[l], input, M, m->hidden, s->pp, P, nullptr);
  det::launch_scale(s->pp, M * P, m->ple_projection_scalar, st);
  det::launch_rmsnorm(s->pp, M, P, P, m->ple_proj_norm, m->eps, st);
  det::launch_add_sat(out, s->pp, M * P, st);
  det::launch_scale(out, M * P, m->ple_input_scale, st);
}

void check_ids(det_model* m, const uint32_t* ids, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) {
    if (ids[i] >= m->embedding->rows) bail("token id " + std::to_string(ids[i]) + " is out of bounds for embedding tensor");
    if (m->has_ple) {
      const uint64_t pv = m->cfg.has_vocab_size_per_layer_input ? m->cfg.vocab_size_per_layer_input : m->cfg.vocab_size;
      if (ids[i] >= pv) bail("matrix row is out of bounds for PLE slice");
    }
  }
}

// Rotations at positions up to max_position reach the reference's
// nth_root_acc bisection, which overflows for a base of i64::MAX.
void check_rope(const det_model* m, uint64_t max_position) {
  if (m->rope_overflow && max_position > 0)
    contract("nth_root_acc: attempt to add with overflow (RoPE base i64::MAX)");
}

void logits_from(det_session* s, const int32_t* hidden_row) {
  det_model* m = s->m;
  det_ctx* ctx = m->ctx;
  hipStream_t st = ctx->stream;
  det::launch_rmsnorm_to(s->normed, hidden_row, 1, m->hidden, m->hidden, m->final_norm, m->eps, st);
  linear(ctx, *m->lm_head, s->normed, 1, s->logits);
  if (m->softcap) det::launch_softcap(s->logits, m->vocab, *m->softcap, st);
  s->logits_valid = true;
}

// Cache bookkeeping after n tokens with canonical slots (token t at t % cap
// in a ring, t in a linear cache); equals push + trim-front of
// DetKvCacheData::append_rows (det_tensor.rs:308-337).
void kv_advance(GKv& c, uint64_t n) {
  c.len = c.ring ? std::min(n, c.cap) : n;
  c.start = c.ring ? (n - c.len) % c.cap : 0;
  c.total = n;
}

// det_layer_prefill (det_kernels.rs:678-821) on the n activation rows in
// ws->x, in place. With donor == nullptr the layer's own cache `own` receives
// the rows its window keeps (DetKvCacheData::from_head_slabs,
// det_tensor.rs:250-268); with a donor, attention reads the donor's cache and
// `own` is left untouched (the reference returns no cache).
// `normed_ready`: the previous layer's last pass already wrote this layer's
// input norm of ws->x into ws->normed. With `next`, this layer leaves next's
// input norm there (returned true) or not (false).
bool layer_prefill(det_session* ws, const GLayer& L, uint64_t n, GKv* own, const GKv* donor, const int32_t* ple_in,
                   const GLayer* next = nullptr, bool normed_ready = false) {
  det_model* m = ws->m;
  det_ctx* ctx = m->ctx;
  hipStream_t st = ctx->stream;
  const uint64_t H = m->hidden;
  if (n == 0) bail("transformer layer execution requires at least one activation row");
  if (n > ws->max_tokens) bail("activation rows exceed the scratch capacity");
  if (!donor && !own) bail("transformer prefill layer needs its own cache or a donor cache");
  if (!normed_ready) det::launch_rmsnorm_to(ws->normed, ws->x, n, H, H, L.in_ln, L.eps, st);
  const uint64_t kw = L.num_kv_heads * L.head_dim;
  // DetKvCacheData::from_head_slabs: keep the last rows past the window.
  const uint64_t retained = (!donor && own && own->ring) ? (n > own->cap ? n - own->cap : 0) : 0;
  if (!donor && own) {
    if (own->row_w != kw) bail("layer cache head count mismatch");
    if (n - retained > own->cap || n > own->limit) bail("KV cache capacity exceeded");
  }
  // the attention's arguments and work area first: the head-norm kernel then
  // writes the MFMA form's Q (and, with this layer's own K rows, K) operand
  // blocks itself
  det::AttnArgs a{};
  a.q = ws->qb; a.q_ld = L.num_heads * L.head_dim;
  a.out = ws->attn; a.out_ld = L.num_heads * L.head_dim;
  a.hd = uint32_t(L.head_dim); a.num_heads = uint32_t(L.num_heads);
  a.groups = uint32_t(L.num_heads / L.num_kv_heads);
  a.n_queries = uint32_t(n); a.causal = 1;
  a.window = L.sliding ? *L.sliding_window : 0; a.causal_offset = 0;
  if (donor) {
    const GKv& d = *donor;
    if (!d.has) bail("deterministic attention requires canonical key cache rows");
    if (d.row_w != kw) bail("layer cache head count mismatch");
    a.k = d.k; a.v = d.v; a.kv_ld = d.row_w;
    a.ring_start = d.start; a.ring_cap = d.ring ? d.cap : 0; a.avail = d.len;
    if (d.len < n) contract("attention_softmax requires a non-empty logits slice");
  } else {
    a.k = ws->kb; a.v = ws->vb; a.kv_ld = kw; a.ring_start = 0; a.ring_cap = 0; a.avail = n;
  }
  if (a.avail > det::kMaxAttentionRows) bail("attention window longer than 16000 rows is not supported");
  ctx->attach_attn_work(a);
  det::AttnMfmaArgs plan;
  const bool mfma = det::attn_mfma_plan(a, plan);
  uint32_t split = 0;
  const bool cached = qkv_block(ws, L, n, 0, nullptr, donor ? nullptr : own, retained, mfma ? &plan : nullptr,
                                donor == nullptr, &split);
  a.split_done = split;
  if (!donor) {
    GKv& c = *own;
    // canonical slots: token t at t % cap (ring) or t (linear), unless the
    // head-norm kernel wrote them
    for (uint64_t t = cached ? n : retained; t < n;) {
      const uint64_t slot = c.ring ? t % c.cap : t;
      const uint64_t span = std::min<uint64_t>(n - t, c.cap - slot);
      copy_d2d(ctx, c.k + slot * kw, ws->kb + t * kw, span * kw * 4);
      copy_d2d(ctx, c.v + slot * kw, ws->vb + t * kw, span * kw * 4);
      t += span;
    }
    kv_advance(c, n);
    c.has = true;
  }
  det::launch_attention(a, st);
  return post_attention(ws, L, n, ple_in, next);
}

// det_layer_decode (det_kernels.rs:866-1133) on the activation row in ws->x,
// in place, with RoPE at `position`. Without a donor the token's K/V row is
// appended to `own` (DetKvCacheData::append_rows with the sliding-window
// trim, det_tensor.rs:308-337) and attention reads it; with a donor (already
// updated for this step) attention reads the donor's cache.
void layer_decode(det_session* ws, const GLayer& L, uint64_t position, GKv* own, const GKv* donor,
                  const int32_t* ple_in) {
  det_model* m = ws->m;
  det_ctx* ctx = m->ctx;
  hipStream_t st = ctx->stream;
  const uint64_t H = m->hidden;
  if (!donor && !own) bail("transformer decode layer needs its own cache or a donor cache");
  det::launch_rmsnorm_to(ws->normed, ws->x, 1, H, H, L.in_ln, L.eps, st);
  qkv_block(ws, L, 1, position);
  const uint64_t kw = L.num_kv_heads * L.head_dim;
  if (!donor) {
    GKv& c = *own;
    if (c.row_w != kw) bail("layer cache append head count mismatch");
    if ((!c.ring && c.total >= c.cap) || c.total >= c.limit) bail("KV cache capacity exceeded");
    const uint64_t slot = c.ring ? c.total % c.cap : c.total;
    copy_d2d(ctx, c.k + slot * kw, ws->kb, kw * 4);
    copy_d2d(ctx, c.v + slot * kw, ws->vb, kw * 4);
    kv_advance(c, c.total + 1);
    c.has = true;
  }
  const GKv& ac = donor ? *donor : *own;
  if (!ac.has) bail("deterministic attention requires canonical key cache rows");
  if (ac.row_w != kw) bail("layer cache head count mismatch");
  const uint64_t cur = ac.len;
  const uint64_t key_start = L.sliding ? (cur > *L.sliding_window ? cur - *L.sliding_window : 0) : 0;
  const uint64_t count = cur > key_start ? cur - key_start : 0;
  if (count == 0) contract("attention_softmax requires a non-empty logits slice");
  det::AttnArgs a{};
  a.q = ws->qb; a.q_ld = L.num_heads * L.head_dim;
  a.k = ac.k; a.v = ac.v; a.kv_ld = kw;
  a.ring_start = ac.start; a.ring_cap = ac.ring ? ac.cap : 0;
  a.out = ws->attn; a.out_ld = L.num_heads * L.head_dim;
  a.hd = uint32_t(L.head_dim); a.num_heads = uint32_t(L.num_heads);
  a.groups = uint32_t(L.num_heads / L.num_kv_heads);
  a.n_queries = 1; a.causal = 0; a.fix_start = key_start; a.fix_count = count;
  if (count > det::kMaxAttentionRows) bail("attention window longer than 16000 rows is not supported");
  det::launch_attention(a, st);
  post_attention(ws, L, 1, ple_in);
}

// The layer's own cache in a session (nullptr for a layer that reads a
// donor's cache) and the donor cache it reads.
GKv* own_cache(det_session* s, const GLayer& L, uint64_t l) { return L.donor ? nullptr : &s->kv[l]; }
const GKv* donor_cache(det_session* s, const GLayer& L) { return L.donor ? &s->kv[*L.donor] : nullptr; }

// Embeds n token ids (already in s->ids) into s->x.
void embed_ids(det_session* s, uint64_t n) {
  det_model* m = s->m;
  det::launch_gather_rows(*m->embedding, s->ids, n, 0, m->hidden, m->embed_scale, s->x, m->hidden, m->ctx->stream);
}

// pipeline::run_prefill_pass_with_mode (runtime/pipeline.rs:55-98): embedding,
// PLE inputs, every layer's det_layer_prefill, prefill_finalize logits.
void prefill(det_session* s, const uint32_t* ids, uint64_t n, uint32_t flags, det_prefill_result_t* out) {
  det_model* m = s->m;
  det_ctx* ctx = m->ctx;
  hipStream_t st = ctx->stream;
  if (n == 0) bail("transformer layer execution requires at least one activation row");
  if (n > s->max_tokens) bail("prompt longer than the session capacity");
  if (s->position != 0) bail("session already holds a prefilled sequence");
  check_ids(m, ids, n);
  check_rope(m, n - 1);
  const uint64_t H = m->hidden;
  HIPC(hipMemcpyAsync(s->ids, ids, n * 4, hipMemcpyHostToDevice, st));
  embed_ids(s, n);
  std::vector<int32_t> host;
  if (flags & DET_COMMIT_ACTIVATIONS) {
    host.resize(n * H);
    HIPC(hipMemcpyAsync(host.data(), s->x, n * H * 4, hipMemcpyDeviceToHost, st));
    HIPC(hipStreamSynchronize(st));
    commit_rows(host.data(), n, H, out->embedding);
  }
  const uint64_t P = m->ple_dim;
  if (m->has_ple)
    for (uint64_t l = 0; l < m->layers.size(); ++l)
      if (m->layers[l].has_ple) ple_inputs(s, l, s->ids, s->x, n, s->ple_all + l * n * P);
  bool ready = false;  // the layer's input norm was written by the previous layer
  for (uint64_t l = 0; l < m->layers.size(); ++l) {
    const GLayer& L = m->layers[l];
    const GLayer* next = l + 1 < m->layers.size() ? &m->layers[l + 1] : nullptr;
    ready = layer_prefill(s, L, n, own_cache(s, L, l), donor_cache(s, L),
                          (m->has_ple && L.has_ple) ? s->ple_all + l * n * P : nullptr, next, ready);
  }
  if (flags & DET_COMMIT_ACTIVATIONS) {
    host.resize(n * H);
    HIPC(hipMemcpyAsync(host.data(), s->x, n * H * 4, hipMemcpyDeviceToHost, st));
    HIPC(hipStreamSynchronize(st));
    commit_rows(host.data(), n, H, out->final_hidden);
  }
  logits_from(s, s->x + (n - 1) * H);
  s->position = n;
  if (flags & DET_COMMIT_ACTIVATIONS) {
    std::vector<int32_t> lg(m->vocab);
    HIPC(hipMemcpyAsync(lg.data(), s->logits, m->vocab * 4, hipMemcpyDeviceToHost, st));
    HIPC(hipStreamSynchronize(st));
    commit_vector(lg.data(), m->vocab, out->logits);
  }
  out->kv[0] = 0;
  if (flags & DET_COMMIT_KV) commit_kv(s->m->ctx, all_caches(s), out->kv);
  out->next_token = ctx->argmax(s->logits, m->vocab);
}

// Observer of a per-op decode step; after_layer returns true to stop the
// step there.
struct LayerHook {
  virtual bool after_layer(det_session* s, uint64_t l) = 0;
  virtual ~LayerHook() = default;
};

// One decode_step with one kernel sequence per layer. layer_rows (device,
// [layers][hidden]) receives every layer's output row when non-null. Returns
// false when the hook stopped the step early (the session is then left
// mid-step and must not be used further).
bool decode(det_session* s, uint32_t token, uint32_t flags, det_decode_result_t* out, LayerHook* hook,
            int32_t* layer_rows = nullptr) {
  det_model* m = s->m;
  det_ctx* ctx = m->ctx;
  hipStream_t st = ctx->stream;
  if (s->position == 0) bail("decode requires a prefilled session");
  if (s->position >= s->max_tokens) bail("session capacity exhausted");
  check_ids(m, &token, 1);
  check_rope(m, s->position);
  const uint64_t H = m->hidden;
  HIPC(hipMemcpyAsync(s->ids, &token, 4, hipMemcpyHostToDevice, st));
  det::launch_gather_rows(*m->embedding, s->ids, 1, 0, H, m->embed_scale, s->dec_in, H, st);
  copy_d2d(ctx, s->x, s->dec_in, H * 4);
  const uint64_t pos = s->position;
  for (uint64_t l = 0; l < m->layers.size(); ++l) {
    const GLayer& L = m->layers[l];
    if (m->has_ple && L.has_ple) ple_inputs(s, l, s->ids, s->dec_in, 1, s->pe);
    layer_decode(s, L, pos, own_cache(s, L, l), donor_cache(s, L), (m->has_ple && L.has_ple) ? s->pe : nullptr);
    if (layer_rows) copy_d2d(ctx, layer_rows + l * H, s->x, H * 4);
    if (hook && hook->after_layer(s, l)) return false;
  }
  std::vector<int32_t> host;
  if (flags & DET_COMMIT_ACTIVATIONS) {
    host.resize(H);
    HIPC(hipMemcpyAsync(host.data(), s->x, H * 4, hipMemcpyDeviceToHost, st));
    HIPC(hipStreamSynchronize(st));
    commit_rows(host.data(), 1, H, out->activation);
  }
  logits_from(s, s->x);
  s->position += 1;
  if (flags & DET_COMMIT_ACTIVATIONS) {
    std::vector<int32_t> lg(m->vocab);
    HIPC(hipMemcpyAsync(lg.data(), s->logits, m->vocab * 4, hipMemcpyDeviceToHost, st));
    HIPC(hipStreamSynchronize(st));
    commit_vector(lg.data(), m->vocab, out->logits);
  }
  out->kv[0] = 0;
  if (flags & DET_COMMIT_KV) commit_kv(s->m->ctx, all_caches(s), out->kv);
  out->next_token = ctx->argmax(s->logits, m->vocab);
  return true;
}

// ---------------------------------------------------------------------------
// Batched decode: one decode_step (runtime/pipeline.rs:165-216) for each of n
// independent sequences of one model, with every projection run once over the
// n activation rows (the weights stream once for all of them) and attention
// reading each sequence's own cache window. Per row, every operation is the
// single-sequence one, so each sequence's outputs, caches and commitments are
// those of its solo decode.
// ---------------------------------------------------------------------------
struct BatchWs {
  std::unique_ptr<det_session> rows;  // activation scratch sized for cap rows
  uint64_t cap = 0;
  int32_t* logits = nullptr;  // [cap][vocab]
  int32_t* dec_in = nullptr;  // [cap][hidden] token embeddings (PLE input)
  uint32_t* next = nullptr;   // [cap] greedy tokens
  int64_t* am_keys = nullptr;  // argmax partial keys of cap logits rows
  uint8_t* desc = nullptr;    // device: positions, per-layer windows and append targets
  size_t desc_bytes = 0;
  // fused step: the cache and logits-row part of desc as last written (it
  // changes only with the batch's sessions; the step states every step)
  std::vector<uint8_t> desc_tail;
  // fused batched step: per-sequence rows of the fused decode buffers
  bool fused = false;
  uint64_t grid_cap = 0;  // cache rows the captured attention grids cover
  uint64_t qkv_stride = 0, attn_stride = 0, ff_stride = 0, score_heads = 0;
  int32_t *x = nullptr, *normed = nullptr, *trig = nullptr, *hbuf = nullptr, *scores = nullptr;
  int64_t* attn_keys = nullptr;  // [cap][score_heads][grid_cap / kAttnScoreRows]
  det::AttnStat* attn_stats = nullptr;  // [cap][score_heads]
  int64_t *qkv_acc = nullptr, *attn_acc = nullptr, *o_acc = nullptr, *ff_acc = nullptr;
  int8_t *limbs_x = nullptr, *limbs_o = nullptr, *limbs_ff = nullptr;
  // the same activations in the batched GEMV's operand-major layout
  // (det::om_offset, passes of 16 rows), written by every kernel that writes
  // limbs_x / limbs_ff / limbs_p
  int8_t *om_x = nullptr, *om_ff = nullptr, *om_p = nullptr;
  // per-layer inputs (PLE models): every layer's inputs of each sequence's
  // token [cap][L*P], the model projection rows [cap][L*P], the gate rows
  // [cap][P], the projection accumulators [cap][hidden] and the limb planes
  // of the embedded row (model projection) or of the gate (layer projection)
  int32_t *ple_in = nullptr, *ple_pp = nullptr, *ple_g = nullptr;
  int64_t* ple_acc = nullptr;
  int8_t* limbs_p = nullptr;
  std::vector<void*> owned;
  uint32_t graph_n = 0;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  void drop_graph() {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    exec = nullptr;
    graph = nullptr;
    graph_n = 0;
  }
  template <class T>
  T* alloc(uint64_t n) {
    void* p = nullptr;
    HIPC(hipMalloc(&p, std::max<uint64_t>(n, 1) * sizeof(T)));
    owned.push_back(p);
    return static_cast<T*>(p);
  }
  ~BatchWs() {
    drop_graph();
    for (void* p : {static_cast<void*>(logits), static_cast<void*>(dec_in), static_cast<void*>(next),
                    static_cast<void*>(desc), static_cast<void*>(scores), static_cast<void*>(am_keys),
                    static_cast<void*>(attn_keys)})
      if (p) (void)hipFree(p);
    for (void* p : owned) (void)hipFree(p);
  }
};

void free_batch(BatchWs* b) { delete b; }

// Byte layout of the per-step descriptor block for n sequences and L layers:
// positions u64[n] | AttnSeq[L][n] | key rows int32*[L][n] | value rows int32*[L][n].
struct BatchDesc {
  size_t pos = 0, seqs = 0, kdst = 0, vdst = 0, bytes = 0;
  BatchDesc(uint64_t n, uint64_t L) {
    seqs = pos + 8 * n;
    kdst = seqs + sizeof(det::AttnSeq) * L * n;
    vdst = kdst + sizeof(int32_t*) * L * n;
    bytes = vdst + sizeof(int32_t*) * L * n;
  }
};

// Per-step descriptor block of the fused batched step for n sequences and L
// layers: StepState[n] | DecSeqCache[L][n] | logits row pointers int32*[n].
struct FusedDesc {
  size_t st = 0, caches = 0, logit_dst = 0, bytes = 0;
  FusedDesc(uint64_t n, uint64_t L) {
    caches = st + sizeof(det::StepState) * n;
    logit_dst = caches + sizeof(det::DecSeqCache) * L * n;
    bytes = logit_dst + sizeof(int32_t*) * n;
  }
};

BatchWs& ensure_batch(det_model* m, uint64_t n) {
  if (m->batch && m->batch->cap >= n) return *m->batch;
  HIPC(hipStreamSynchronize(m->ctx->stream));
  free_batch(m->batch);
  m->batch = nullptr;
  auto b = std::make_unique<BatchWs>();
  b->cap = std::max<uint64_t>(n, 16);
  b->rows = std::make_unique<det_session>();
  b->rows->m = m;
  b->rows->max_tokens = b->cap;
  session_alloc(b->rows.get());
  HIPC(hipMalloc(&b->logits, b->cap * m->vocab * 4));
  HIPC(hipMalloc(&b->dec_in, b->cap * m->hidden * 4));
  HIPC(hipMalloc(&b->next, b->cap * 4));
  HIPC(hipMalloc(&b->am_keys, det::argmax_rows_scratch(b->cap, m->vocab) * 8));
  b->desc_bytes = std::max(BatchDesc(b->cap, m->layers.size()).bytes, FusedDesc(b->cap, m->layers.size()).bytes);
  HIPC(hipMalloc(&b->desc, b->desc_bytes));
  m->batch = b.release();
  return *m->batch;
}

void check_batch(det_session* const* ss, uint64_t n, const uint32_t* tokens) {
  if (n == 0) bail("batched decode requires at least one session");
  det_model* m = ss[0]->m;
  for (uint64_t i = 0; i < n; ++i) {
    det_session* s = ss[i];
    if (!s) bail("null session in batch");
    if (s->m != m) bail("batched sessions must share one model");
    for (uint64_t j = 0; j < i; ++j)
      if (ss[j] == s) bail("a session appears twice in one batch");
    if (s->position == 0) bail("decode requires a prefilled session");
    if (s->position >= s->max_tokens) bail("session capacity exhausted");
    check_rope(m, s->position);
    for (size_t l = 0; l < m->layers.size(); ++l) {
      const GKv& c = s->kv[l];
      if (m->layers[l].donor) continue;
      if (!c.has) bail("deterministic decode cache append requires canonical key rows");
      if (!c.ring && s->position >= c.cap) bail("KV cache capacity exceeded");
    }
  }
  check_ids(m, tokens, n);
}

void decode_batch(det_session* const* ss, uint64_t n, const uint32_t* tokens, uint32_t flags,
                  det_decode_result_t* out) {
  check_batch(ss, n, tokens);
  det_model* m = ss[0]->m;
  det_ctx* ctx = m->ctx;
  hipStream_t st = ctx->stream;
  const uint64_t H = m->hidden, V = m->vocab, nl = m->layers.size();
  BatchWs& b = ensure_batch(m, n);
  det_session* w = b.rows.get();
  // host bookkeeping: cache state after this step's append, then the windows
  const BatchDesc D(n, nl);
  std::vector<uint8_t> hbv(D.bytes);
  uint8_t* hb = hbv.data();
  auto* pos = reinterpret_cast<uint64_t*>(hb + D.pos);
  auto* seqs = reinterpret_cast<det::AttnSeq*>(hb + D.seqs);
  auto* kdst = reinterpret_cast<int32_t**>(hb + D.kdst);
  auto* vdst = reinterpret_cast<int32_t**>(hb + D.vdst);
  std::vector<std::vector<GKv>> after(n);
  std::vector<uint64_t> longest(nl, 1);
  for (uint64_t i = 0; i < n; ++i) {
    det_session* s = ss[i];
    pos[i] = s->position;
    after[i] = s->kv;
    for (size_t l = 0; l < nl; ++l) {
      const GLayer& L = m->layers[l];
      const uint64_t kw = L.num_kv_heads * L.head_dim;
      if (!L.donor) {
        GKv& own = after[i][l];
        const uint64_t slot = own.ring ? pos[i] % own.cap : pos[i];
        kv_advance(own, pos[i] + 1);
        own.has = true;
        kdst[l * n + i] = own.k + slot * kw;
        vdst[l * n + i] = own.v + slot * kw;
      } else {
        kdst[l * n + i] = vdst[l * n + i] = nullptr;
      }
      const GKv& ac = L.donor ? after[i][*L.donor] : after[i][l];
      if (!ac.has) bail("deterministic attention requires canonical key cache rows");
      if (ac.row_w != kw) bail("layer cache head count mismatch");
      const uint64_t cur = ac.len;
      const uint64_t key_start = L.sliding ? (cur > *L.sliding_window ? cur - *L.sliding_window : 0) : 0;
      const uint64_t count = cur - key_start;
      if (count == 0) contract("attention_softmax requires a non-empty logits slice");
      if (count > det::kMaxAttentionRows) bail("attention window longer than 16000 rows is not supported");
      det::AttnSeq& q = seqs[l * n + i];
      q.k = ac.k;
      q.v = ac.v;
      q.base = ac.ring ? (ac.start + key_start) % ac.cap : key_start;
      q.wrap = ac.ring ? ac.cap : 0;
      q.count = count;
      longest[l] = std::max(longest[l], count);
    }
  }
  uint8_t* dd = b.desc;
  det::launch_set_bytes(dd, hb, D.bytes, st);
  b.desc_tail.clear();  // desc now holds this layout, not the fused step's cache table
  HIPC(hipMemcpyAsync(w->ids, tokens, n * 4, hipMemcpyHostToDevice, st));
  const auto* pos_dev = reinterpret_cast<const uint64_t*>(dd + D.pos);
  det::launch_gather_rows(*m->embedding, w->ids, n, 0, H, m->embed_scale, b.dec_in, H, st);
  copy_d2d(ctx, w->x, b.dec_in, n * H * 4);
  for (size_t l = 0; l < nl; ++l) {
    const GLayer& L = m->layers[l];
    const uint64_t kw = L.num_kv_heads * L.head_dim;
    if (m->has_ple && L.has_ple) ple_inputs(w, l, w->ids, b.dec_in, n, w->pe);
    det::launch_rmsnorm_to(w->normed, w->x, n, H, H, L.in_ln, L.eps, st);
    qkv_block(w, L, n, 0, pos_dev);
    if (!L.donor)
      det::launch_kv_append(w->kb, w->vb, kw, n, reinterpret_cast<int32_t* const*>(dd + D.kdst) + l * n,
                            reinterpret_cast<int32_t* const*>(dd + D.vdst) + l * n, st);
    det::AttnArgs a{};
    a.q = w->qb; a.q_ld = L.num_heads * L.head_dim;
    a.kv_ld = kw;
    a.out = w->attn; a.out_ld = L.num_heads * L.head_dim;
    a.hd = uint32_t(L.head_dim); a.num_heads = uint32_t(L.num_heads);
    a.groups = uint32_t(L.num_heads / L.num_kv_heads);
    a.n_queries = uint32_t(n); a.causal = 0; a.fix_start = 0; a.fix_count = longest[l];
    a.seqs = reinterpret_cast<const det::AttnSeq*>(dd + D.seqs) + l * n;
    det::launch_attention(a, st);
    post_attention(w, L, n, (m->has_ple && L.has_ple) ? w->pe : nullptr);
  }
  // det_hidden_to_logits for every row, then argmax_first per row
  det::launch_rmsnorm_to(w->normed, w->x, n, H, H, m->final_norm, m->eps, st);
  ctx->linear(*m->lm_head, w->normed, n, H, b.logits, V, nullptr);
  if (m->softcap) det::launch_softcap(b.logits, n * V, *m->softcap, st);
  det::launch_argmax_rows(b.logits, n, V, b.am_keys, b.next, st);
  for (uint64_t i = 0; i < n; ++i) copy_d2d(ctx, ss[i]->logits, b.logits + i * V, V * 4);
  std::vector<uint32_t> next(n);
  HIPC(hipMemcpyAsync(next.data(), b.next, n * 4, hipMemcpyDeviceToHost, st));
  HIPC(hipStreamSynchronize(st));
  for (uint64_t i = 0; i < n; ++i) {
    ss[i]->kv = after[i];
    ss[i]->position += 1;
    ss[i]->logits_valid = true;
  }
  if (flags & DET_COMMIT_ACTIVATIONS) {
    std::vector<int32_t> hx(n * H), lg(n * V);
    HIPC(hipMemcpyAsync(hx.data(), w->x, n * H * 4, hipMemcpyDeviceToHost, st));
    HIPC(hipMemcpyAsync(lg.data(), b.logits, n * V * 4, hipMemcpyDeviceToHost, st));
    HIPC(hipStreamSynchronize(st));
    for (uint64_t i = 0; i < n; ++i) {
      commit_rows(hx.data() + i * H, 1, H, out[i].activation);
      commit_vector(lg.data() + i * V, V, out[i].logits);
    }
  }
  for (uint64_t i = 0; i < n; ++i) {
    out[i].kv[0] = 0;
    out[i].next_token = next[i];
  }
  if (flags & DET_COMMIT_KV) {
    std::vector<std::vector<const GKv*>> sets;
    std::vector<char*> outs;
    for (uint64_t i = 0; i < n; ++i) {
      sets.push_back(all_caches(ss[i]));
      outs.push_back(out[i].kv);
    }
    commit_kv_sessions(m->ctx, sets, outs);
  }
}

// Buffers of the fused batched step for b.cap sequences; the attention
// grids and score rows cover caches of up to `need` rows (grown on demand,
// which drops the captured graph).
void ensure_fused_batch(det_model* m, BatchWs& b, uint64_t need) {
  const uint64_t T = b.cap, H = m->hidden;
  if (!b.fused) {
    uint64_t fr = 0, nhd = 0, ff = 0, kpo = 0, kff = 0, nh = 0;
    for (size_t l = 0; l < m->layers.size(); ++l) {
      const GLayer& L = m->layers[l];
      fr = std::max(fr, m->fused[l].qkv.rows);
      nhd = std::max(nhd, L.num_heads * L.head_dim);
      ff = std::max(ff, L.gate->rows);
      kpo = std::max(kpo, L.o->kpad);
      kff = std::max(kff, L.down->kpad);
      nh = std::max(nh, L.num_heads);
    }
    b.qkv_stride = fr;
    b.attn_stride = nhd;
    b.ff_stride = ff;
    b.score_heads = nh;
    b.x = b.alloc<int32_t>(T * H);
    b.normed = b.alloc<int32_t>(T * H);
    b.trig = b.alloc<int32_t>(T * 2 * uint64_t(std::max<uint32_t>(m->trig_pairs, 1)));
    b.hbuf = b.alloc<int32_t>(T * ff);
    b.qkv_acc = b.alloc<int64_t>(T * fr);
    b.attn_acc = b.alloc<int64_t>(T * nhd);
    b.o_acc = b.alloc<int64_t>(T * H);
    b.ff_acc = b.alloc<int64_t>(T * H);
    b.limbs_x = b.alloc<int8_t>(T * 4 * m->fused[0].qkv.kpad);
    b.limbs_o = b.alloc<int8_t>(T * 4 * kpo);
    b.limbs_ff = b.alloc<int8_t>(T * 4 * kff);
    const uint64_t T16 = (T + 15) / 16 * 16;
    b.om_x = b.alloc<int8_t>(T16 * 4 * m->fused[0].qkv.kpad);
    b.om_ff = b.alloc<int8_t>(T16 * 4 * kff);
    b.attn_stats = b.alloc<det::AttnStat>(T * nh);
    // every accumulator is cleared by the kernel that consumes it, so they
    // only need to start at zero (stream-ordered, outside any graph)
    hipStream_t zst = m->ctx->stream;
    HIPC(hipMemsetAsync(b.qkv_acc, 0, T * fr * 8, zst));
    HIPC(hipMemsetAsync(b.attn_acc, 0, T * nhd * 8, zst));
    HIPC(hipMemsetAsync(b.o_acc, 0, T * H * 8, zst));
    HIPC(hipMemsetAsync(b.ff_acc, 0, T * H * 8, zst));
    HIPC(hipMemsetAsync(b.limbs_o, 0, T * 4 * kpo, zst));
    HIPC(hipMemsetAsync(b.limbs_ff, 0, T * 4 * kff, zst));
    HIPC(hipMemsetAsync(b.limbs_x, 0, T * 4 * m->fused[0].qkv.kpad, zst));
    HIPC(hipMemsetAsync(b.om_x, 0, T16 * 4 * m->fused[0].qkv.kpad, zst));
    HIPC(hipMemsetAsync(b.om_ff, 0, T16 * 4 * kff, zst));
    if (m->has_ple) {
      const uint64_t LP = m->layers.size() * m->ple_dim;
      uint64_t kp = m->ple_proj_full->kpad;
      for (const GLayer& L : m->layers)
        if (L.has_ple) kp = std::max(kp, L.ple_proj->kpad);
      b.ple_in = b.alloc<int32_t>(T * LP);
      b.ple_pp = b.alloc<int32_t>(T * LP);
      b.ple_g = b.alloc<int32_t>(T * m->ple_dim);
      b.ple_acc = b.alloc<int64_t>(T * H);
      b.limbs_p = b.alloc<int8_t>(T * 4 * kp);
      b.om_p = b.alloc<int8_t>(T16 * 4 * kp);
      HIPC(hipMemsetAsync(b.ple_acc, 0, T * H * 8, zst));
    }
    b.fused = true;
  }
  if (need > b.grid_cap) {
    const uint64_t rows = (need + 255) / 256 * 256;
    HIPC(hipStreamSynchronize(m->ctx->stream));
    b.drop_graph();
    if (b.scores) HIPC(hipFree(b.scores));
    if (b.attn_keys) HIPC(hipFree(b.attn_keys));
    b.scores = nullptr;
    b.attn_keys = nullptr;
    HIPC(hipMalloc(&b.scores, T * b.score_heads * rows * 4));
    HIPC(hipMalloc(&b.attn_keys, T * b.score_heads * (rows / det::kAttnScoreRows) * 8));
    b.grid_cap = rows;
  }
}

// Attention arguments of layer l for a batched step of n sequences.
det::AttnDecArgs batch_attn_args(det_model* m, BatchWs& b, size_t l, uint32_t n) {
  const GLayer& L = m->layers[l];
  const auto& F = m->fused[l];
  const FusedDesc D(n, m->layers.size());
  det::AttnDecArgs a{};
  a.qkv = b.qkv_acc;
  a.q_norm = L.q_norm;
  a.k_norm = L.k_norm;
  a.trig = b.trig + 2 * uint64_t(L.trig_off);
  a.eps = L.eps;
  a.rotary = L.rotary;
  a.has_v = F.has_v;
  a.own_cache = !L.donor;
  a.st = reinterpret_cast<const det::StepState*>(b.desc + D.st);
  const size_t src = L.donor ? *L.donor : l;
  const bool ring = m->layers[src].cache_sliding_window.has_value();
  // ring caches hold at most the cache window; linear ones the session length
  a.cap = ring ? std::min<uint64_t>(std::max<uint64_t>(*m->layers[src].cache_sliding_window, 1), b.grid_cap) : b.grid_cap;
  a.window = L.sliding ? *L.sliding_window : 0;
  a.max_rows = b.grid_cap;
  a.ring = ring;
  a.hd = uint32_t(L.head_dim);
  a.nh = uint32_t(L.num_heads);
  a.nkv = uint32_t(L.num_kv_heads);
  a.scores = b.scores;
  a.acc = b.attn_acc;
  a.lds_stride = a.cap;
  a.scores_in_lds = (L.num_heads / L.num_kv_heads) * a.cap * 4 <= 32768;
  a.caches = reinterpret_cast<const det::DecSeqCache*>(b.desc + D.caches) + l * n;
  a.trig_stride = 2 * uint64_t(std::max<uint32_t>(m->trig_pairs, 1));
  a.qkv_stride = b.qkv_stride;
  a.scores_stride = b.score_heads * b.grid_cap;
  a.acc_stride = b.attn_stride;
  a.keys = b.attn_keys;
  a.key_chunks = b.grid_cap / det::kAttnScoreRows;
  a.keys_stride = b.score_heads * a.key_chunks;
  a.stats = b.attn_stats;
  a.stats_stride = b.score_heads;
  a.nseq = n;
  return a;
}

// One fused decode step for n sequences: the single-sequence fused step with
// every kernel over the n rows (GEMVs with up to 16 tokens per weight pass).
void enqueue_fused_batch(det_model* m, BatchWs& b, uint32_t n) {
  hipStream_t st = m->ctx->stream;
  const uint64_t H = m->hidden, V = m->vocab;
  const FusedDesc D(n, m->layers.size());
  const auto* st_dev = reinterpret_cast<const det::StepState*>(b.desc + D.st);
  const uint64_t kpad_x = m->fused[0].qkv.kpad;
  det::launch_dec_set_trig(st_dev, n, m->rope_tables_dev, uint32_t(m->rope_tables.size()), m->trig_pairs, b.trig, st);
  det::launch_dec_embed(*m->embedding, st_dev, m->embed_scale, H, b.x, b.dec_in, m->layers[0].in_ln, m->eps, b.normed,
                        b.limbs_x, kpad_x, st, n, b.om_x);
  const uint64_t P = m->ple_dim, LP = m->layers.size() * P;
  if (m->has_ple) {
    // every layer's per-layer input of each sequence's token (det_decode_ple_input,
    // det_kernels.rs:1142-1208), rows [n][L*P] as in the single-sequence step
    const uint64_t id_stride = sizeof(det::StepState) / sizeof(uint32_t);
    det::launch_gather_rows(*m->ple_tok, &st_dev->token, n, 0, LP, m->ple_embedding_scale, b.ple_in, LP, st, id_stride);
    det::launch_dec_row_limbs(b.dec_in, H, H, n, b.limbs_p, m->ple_proj_full->kpad, st, nullptr, 0, b.om_p);
    det::launch_gemv_dec_batch(*m->ple_proj_full, b.limbs_p, n, b.ple_pp, LP, nullptr, 0, 0, nullptr, 0, st, b.om_p);
    det::launch_scale(b.ple_pp, n * LP, m->ple_projection_scalar, st);
    det::launch_rmsnorm(b.ple_pp, n * m->layers.size(), P, P, m->ple_proj_norm, m->eps, st);
    det::launch_add_sat(b.ple_in, b.ple_pp, n * LP, st);
    det::launch_scale(b.ple_in, n * LP, m->ple_input_scale, st);
  }
  for (size_t l = 0; l < m->layers.size(); ++l) {
    const GLayer& L = m->layers[l];
    const auto& F = m->fused[l];
    det::launch_gemv_dec_batch(F.qkv, b.limbs_x, n, nullptr, 0, b.qkv_acc, b.qkv_stride, 0, nullptr, 0, st, b.om_x);
    det::launch_dec_attention(batch_attn_args(m, b, l, n), st);
    // the O projection reads the weighted-sum accumulators directly where
    // its kernel takes them (the scores kernel clears them at the next layer)
    if (det::gemv_dec_batch_in64_ok(*L.o, n, b.attn_stride)) {
      det::launch_gemv_dec_batch_in64(*L.o, b.attn_acc, b.attn_stride, n, b.o_acc, H, st);
    } else {
      det::launch_dec_acc_limbs(b.attn_acc, L.num_heads * L.head_dim, b.attn_stride, n, b.limbs_o, L.o->kpad, st);
      det::launch_gemv_dec_batch(*L.o, b.limbs_o, n, nullptr, 0, b.o_acc, H, 0, nullptr, 0, st);
    }
    det::launch_dec_residual_norm(b.o_acc, b.x, b.normed, L.post_attn_ln, false, 0, L.pre_ff_ln, H, L.eps, b.limbs_x,
                                  kpad_x, st, n, nullptr, nullptr, false, b.om_x);
    det::launch_gemv_dec_batch(F.gateup, b.limbs_x, n, b.hbuf, b.ff_stride, nullptr, 0, 1, b.limbs_ff, L.down->kpad, st,
                               b.om_x, b.om_ff);
    det::launch_gemv_dec_batch(*L.down, b.limbs_ff, n, nullptr, 0, b.ff_acc, H, 0, nullptr, 0, st, b.om_ff);
    const int32_t* w_next = l + 1 < m->layers.size() ? m->layers[l + 1].in_ln : m->final_norm;
    if (m->has_ple && L.has_ple) {
      // x += norm(down) (with x's limb planes); then the per-layer input block
      // (det_kernels.rs:1108-1128): x += norm(proj(gelu(gate(x)) * ple_in)),
      // the layer scalar and the next norm
      det::launch_dec_residual_norm(b.ff_acc, b.x, b.normed, L.post_ff_ln, false, 0, nullptr, H, L.eps, b.limbs_x,
                                    kpad_x, st, n, nullptr, nullptr, true, b.om_x);
      det::launch_gemv_dec_batch(*L.ple_gate, b.limbs_x, n, b.ple_g, P, nullptr, 0, 0, nullptr, 0, st, b.om_x);
      det::launch_dec_row_limbs(b.ple_g, P, P, n, b.limbs_p, L.ple_proj->kpad, st, b.ple_in + l * P, LP, b.om_p);
      det::launch_gemv_dec_batch(*L.ple_proj, b.limbs_p, n, nullptr, 0, b.ple_acc, H, 0, nullptr, 0, st, b.om_p);
      det::launch_dec_residual_norm(b.ple_acc, b.x, b.normed, L.ple_post_norm, L.layer_scalar.has_value(),
                                    L.layer_scalar.value_or(0), w_next, H, L.eps, b.limbs_x, kpad_x, st, n, nullptr,
                                    nullptr, false, b.om_x);
    } else {
      det::launch_dec_residual_norm(b.ff_acc, b.x, b.normed, L.post_ff_ln, L.layer_scalar.has_value(),
                                    L.layer_scalar.value_or(0), w_next, H, L.eps, b.limbs_x, kpad_x, st, n, nullptr,
                                    nullptr, false, b.om_x);
    }
  }
  det::launch_gemv_dec_batch(*m->lm_head, b.limbs_x, n, b.logits, V, nullptr, 0, 0, nullptr, 0, st, b.om_x);
  if (m->softcap) det::launch_dec_softcap(b.logits, n * V, *m->softcap, st);
  det::launch_copy_rows(b.logits, V, n, reinterpret_cast<int32_t* const*>(b.desc + D.logit_dst), st);
  det::launch_argmax_rows(b.logits, n, V, b.am_keys, b.next, st);
}

// Whether a model's batched steps take the fused schedule: the single-sequence
// fused step's conditions, and for per-layer inputs a model projection of
// exactly L*P rows (the per-sequence rows [L*P] of the step's PLE buffers).
bool batch_fused_ok(const det_model* m) {
  if (!m->fused_ok) return false;
  return !m->has_ple || m->ple_proj_full->rows == m->layers.size() * m->ple_dim;
}

void decode_batch_fused(det_session* const* ss, uint64_t n, const uint32_t* tokens, uint32_t flags,
                        det_decode_result_t* out) {
  check_batch(ss, n, tokens);
  det_model* m = ss[0]->m;
  det_ctx* ctx = m->ctx;
  hipStream_t st = ctx->stream;
  const uint64_t H = m->hidden, V = m->vocab, nl = m->layers.size();
  BatchWs& b = ensure_batch(m, n);
  uint64_t need = 1;
  for (uint64_t i = 0; i < n; ++i) need = std::max(need, ss[i]->max_tokens);
  ensure_fused_batch(m, b, need);
  const FusedDesc D(n, nl);
  std::vector<uint8_t> hbv(D.bytes);
  uint8_t* hb = hbv.data();
  auto* sts = reinterpret_cast<det::StepState*>(hb + D.st);
  auto* caches = reinterpret_cast<det::DecSeqCache*>(hb + D.caches);
  auto* dst = reinterpret_cast<int32_t**>(hb + D.logit_dst);
  for (uint64_t i = 0; i < n; ++i) {
    det_session* s = ss[i];
    sts[i].position = s->position;
    sts[i].token = tokens[i];
    sts[i].pad = 0;
    dst[i] = s->logits;
    for (size_t l = 0; l < nl; ++l) {
      const GLayer& L = m->layers[l];
      const GKv& c = L.donor ? s->kv[*L.donor] : s->kv[l];
      if (L.donor && !c.has) bail("deterministic attention requires canonical key cache rows");
      if (c.row_w != L.num_kv_heads * L.head_dim) bail("layer cache head count mismatch");
      caches[l * n + i] = det::DecSeqCache{c.k, c.v, c.cap};
    }
  }
  // descriptors by kernel arguments, stream-ordered before the step: the
  // step states every step, the cache table when the batch changes
  det::launch_set_bytes(b.desc + D.st, hb + D.st, D.caches - D.st, st);
  if (b.desc_tail.size() != D.bytes - D.caches ||
      std::memcmp(b.desc_tail.data(), hb + D.caches, D.bytes - D.caches) != 0) {
    det::launch_set_bytes(b.desc + D.caches, hb + D.caches, D.bytes - D.caches, st);
    b.desc_tail.assign(hb + D.caches, hb + D.bytes);
  }
  HIPC(hipGetLastError());
  const bool eager = flags & DET_DECODE_EAGER;
  if (eager) {
    enqueue_fused_batch(m, b, uint32_t(n));
  } else {
    if (!b.exec || b.graph_n != n) {
      b.drop_graph();
      HIPC(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
      try {
        enqueue_fused_batch(m, b, uint32_t(n));
      } catch (...) {
        hipGraph_t g = nullptr;
        (void)hipStreamEndCapture(st, &g);
        if (g) (void)hipGraphDestroy(g);
        throw;
      }
      HIPC(hipStreamEndCapture(st, &b.graph));
      HIPC(hipGraphInstantiate(&b.exec, b.graph, nullptr, nullptr, 0));
      b.graph_n = uint32_t(n);
    }
    HIPC(hipGraphLaunch(b.exec, st));
  }
  std::vector<uint32_t> next(n);
  HIPC(hipMemcpyAsync(next.data(), b.next, n * 4, hipMemcpyDeviceToHost, st));
  HIPC(hipStreamSynchronize(st));
  for (uint64_t i = 0; i < n; ++i) {
    det_session* s = ss[i];
    for (size_t l = 0; l < nl; ++l)
      if (!m->layers[l].donor) kv_advance(s->kv[l], s->position + 1);
    s->position += 1;
    s->logits_valid = true;
  }
  if (flags & DET_COMMIT_ACTIVATIONS) {
    std::vector<int32_t> hx(n * H), lg(n * V);
    HIPC(hipMemcpyAsync(hx.data(), b.x, n * H * 4, hipMemcpyDeviceToHost, st));
    HIPC(hipMemcpyAsync(lg.data(), b.logits, n * V * 4, hipMemcpyDeviceToHost, st));
    HIPC(hipStreamSynchronize(st));
    for (uint64_t i = 0; i < n; ++i) {
      commit_rows(hx.data() + i * H, 1, H, out[i].activation);
      commit_vector(lg.data() + i * V, V, out[i].logits);
    }
  }
  for (uint64_t i = 0; i < n; ++i) {
    out[i].kv[0] = 0;
    out[i].next_token = next[i];
  }
  if (flags & DET_COMMIT_KV) {
    std::vector<std::vector<const GKv*>> sets;
    std::vector<char*> outs;
    for (uint64_t i = 0; i < n; ++i) {
      sets.push_back(all_caches(ss[i]));
      outs.push_back(out[i].kv);
    }
    commit_kv_sessions(m->ctx, sets, outs);
  }
}

// Attention arguments of layer l for the fused decode step.
det::AttnDecArgs attn_args(det_session* s, size_t l) {
  det_model* m = s->m;
  const GLayer& L = m->layers[l];
  const auto& F = m->fused[l];
  GKv& ac = L.donor ? s->kv[*L.donor] : s->kv[l];
  det::AttnDecArgs a{};
  a.qkv = s->qkv_acc;
  a.q_norm = L.q_norm;
  a.k_norm = L.k_norm;
  a.trig = s->trig + 2 * uint64_t(L.trig_off);
  a.eps = L.eps;
  a.rotary = L.rotary;
  a.has_v = F.has_v;
  a.own_cache = !L.donor;
  a.k = ac.k;
  a.v = ac.v;
  a.st = s->st_dev;
  a.cap = ac.cap;
  a.window = L.sliding ? *L.sliding_window : 0;
  a.max_rows = s->score_stride;
  a.ring = ac.ring;
  a.hd = uint32_t(L.head_dim);
  a.nh = uint32_t(L.num_heads);
  a.nkv = uint32_t(L.num_kv_heads);
  a.scores = s->scores;
  a.acc = s->attn_acc;
  a.scores_in_lds = (L.num_heads / L.num_kv_heads) * ac.cap * 4 <= 32768;
  a.lds_stride = ac.cap;
  a.keys = s->attn_keys;
  a.key_chunks = (s->score_stride + det::kAttnScoreRows - 1) / det::kAttnScoreRows;
  a.stats = s->attn_stats;
  return a;
}

// Enqueues one fused decode step (det_layer_decode for every layer, then
// det_hidden_to_logits and argmax_first) reading position/token from st_dev.
void enqueue_fused_step(det_session* s) {
  det_model* m = s->m;
  hipStream_t st = m->ctx->stream;
  const uint64_t H = m->hidden;
  det::launch_dec_embed(*m->embedding, s->st_dev, m->embed_scale, H, s->x, s->dec_in, m->layers[0].in_ln, m->eps,
                        s->normed, s->limbs_x, s->kpad_x, st);
  const uint64_t P = m->ple_dim, LP = m->layers.size() * P;
  if (m->has_ple) {
    // per-layer inputs of the step token for every layer at once
    // (det_decode_ple_input, det_kernels.rs:1142-1208, one slice per layer)
    det::launch_gather_rows(*m->ple_tok, &s->st_dev->token, 1, 0, LP, m->ple_embedding_scale, s->ple_in_all, LP, st);
    det::launch_gemv_decode(*m->ple_proj_full, s->dec_in, false, 0, s->ple_pp, st);
    det::launch_scale(s->ple_pp, LP, m->ple_projection_scalar, st);
    det::launch_rmsnorm(s->ple_pp, m->layers.size(), P, P, m->ple_proj_norm, m->eps, st);
    det::launch_add_sat(s->ple_in_all, s->ple_pp, LP, st);
    det::launch_scale(s->ple_in_all, LP, m->ple_input_scale, st);
  }
  // The residual row: with norm_fused it alternates between s->x and
  // s->x_alt at every projection that applies a residual norm, and the last
  // layer's norm writes it back to s->x.
  int32_t* xc = s->x;
  auto flip = [&](const int32_t* p) { return p == s->x ? s->x_alt : s->x; };
  const size_t nl = m->layers.size();
  bool limbs_ready = true;  // limbs_x holds the normalised input of the next projection
  for (size_t l = 0; l < nl; ++l) {
    const GLayer& L = m->layers[l];
    const auto& F = m->fused[l];
    if (limbs_ready) {
      det::launch_gemv_dec(F.qkv, s->limbs_x, nullptr, s->qkv_acc, 0, nullptr, 0, st);
    } else {
      // the previous layer's post-FF residual norm (and layer scalar), then this layer's input norm
      const GLayer& Lp = m->layers[l - 1];
      det::DecNormIn ni;
      ni.src = s->ff_acc;
      ni.x_in = xc;
      ni.w_post = Lp.post_ff_ln;
      ni.w_next = L.in_ln;
      ni.x_out = flip(xc);
      ni.row_out = s->layer_rows ? s->layer_rows + (l - 1) * H : nullptr;
      ni.H = H;
      ni.eps = Lp.eps;
      ni.has_scalar = Lp.layer_scalar.has_value();
      ni.scalar = Lp.layer_scalar.value_or(0);
      det::launch_gemv_norm(ni, F.qkv, 0, s->qkv_acc, nullptr, nullptr, 0, st);
      xc = ni.x_out;
    }
    const det::AttnDecArgs aa = attn_args(s, l);
    det::launch_dec_attention(aa, st);
    det::launch_gemv_decode_acc(*L.o, s->attn_acc, true, s->o_acc, st);
    if (m->norm_fused) {
      // post-attention residual norm and pre-FF norm inside the gate/up
      // projection, which also clears the down projection's accumulators
      det::DecNormIn ni;
      ni.src = s->o_acc;
      ni.x_in = xc;
      ni.w_post = L.post_attn_ln;
      ni.w_next = L.pre_ff_ln;
      ni.x_out = flip(xc);
      ni.clear = s->ff_acc;
      ni.clear_n = H;
      ni.H = H;
      ni.eps = L.eps;
      det::launch_gemv_norm(ni, F.gateup, 1, nullptr, s->hbuf, s->limbs_ff, L.down->kpad, st);
      xc = ni.x_out;
    } else {
      det::launch_dec_residual_norm(s->o_acc, xc, s->normed, L.post_attn_ln, false, 0, L.pre_ff_ln, H, L.eps,
                                    s->limbs_x, s->kpad_x, st);
      det::launch_gemv_dec(F.gateup, s->limbs_x, s->hbuf, nullptr, 1, s->limbs_ff, L.down->kpad, st);
    }
    det::launch_gemv_dec(*L.down, s->limbs_ff, nullptr, s->ff_acc, 0, nullptr, 0, st);
    const bool last = l + 1 == nl;
    const int32_t* w_next = !last ? m->layers[l + 1].in_ln : m->final_norm;
    int32_t* row_out = s->layer_rows ? s->layer_rows + l * H : nullptr;
    // the last layer's norm leaves the residual row in s->x
    int32_t* x_dst = last ? s->x : xc;
    if (m->has_ple && L.has_ple) {
      // x += norm(down); then the per-layer input block (det_kernels.rs:1108-1128):
      // x += norm(proj(gelu(gate(x)) * ple_in)), then the layer scalar and the next norm
      // (the first residual norm writes x only: the second writes the next norm)
      det::launch_dec_residual_norm(s->ff_acc, xc, s->normed, L.post_ff_ln, false, 0, nullptr, H, L.eps, s->limbs_x,
                                    s->kpad_x, st);
      det::launch_gemv_decode(*L.ple_gate, xc, false, 2, s->ple_g, st, s->ple_in_all + l * P);
      det::launch_gemv_decode_acc(*L.ple_proj, s->ple_g, false, s->ple_acc, st);
      det::launch_dec_residual_norm(s->ple_acc, x_dst, s->normed, L.ple_post_norm, L.layer_scalar.has_value(),
                                    L.layer_scalar.value_or(0), w_next, H, L.eps, s->limbs_x, s->kpad_x, st, 1,
                                    row_out, xc);
      xc = x_dst;
      limbs_ready = true;
    } else if (last || !m->norm_fused) {
      det::launch_dec_residual_norm(s->ff_acc, x_dst, s->normed, L.post_ff_ln, L.layer_scalar.has_value(),
                                    L.layer_scalar.value_or(0), w_next, H, L.eps, s->limbs_x, s->kpad_x, st, 1,
                                    row_out, xc);
      xc = x_dst;
      limbs_ready = true;
    } else {
      limbs_ready = false;  // the next layer's q/k/v projection applies this norm
    }
  }
  // the vocabulary projection streams best through the 8-wave LDS kernel
  det::launch_gemv_decode(*m->lm_head, s->normed, false, 0, s->logits, st);
  if (m->softcap) det::launch_dec_softcap(s->logits, m->vocab, *m->softcap, st);
  det::launch_argmax(s->logits, m->vocab, s->am_scratch, s->am_out, st);
}

void build_decode_graph(det_session* s) {
  hipStream_t st = s->m->ctx->stream;
  HIPC(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
  try {
    enqueue_fused_step(s);
  } catch (...) {
    hipGraph_t g = nullptr;
    (void)hipStreamEndCapture(st, &g);
    if (g) (void)hipGraphDestroy(g);
    throw;
  }
  HIPC(hipStreamEndCapture(st, &s->graph));
  HIPC(hipGraphInstantiate(&s->exec, s->graph, nullptr, nullptr, 0));
}

void decode_fused(det_session* s, uint32_t token, uint32_t flags, det_decode_result_t* out) {
  det_model* m = s->m;
  det_ctx* ctx = m->ctx;
  hipStream_t st = ctx->stream;
  if (s->position == 0) bail("decode requires a prefilled session");
  if (s->position >= s->max_tokens) bail("session capacity exhausted");
  check_ids(m, &token, 1);
  check_rope(m, s->position);
  for (size_t l = 0; l < m->layers.size(); ++l) {
    const GKv& c = s->kv[l];
    if (!m->layers[l].donor && !c.has) bail("deterministic decode cache append requires canonical key rows");
  }
  const bool eager = flags & DET_DECODE_EAGER;
  if (!eager && !s->exec) build_decode_graph(s);
  const uint64_t pos = s->position;
  det::launch_dec_set_step(s->st_dev, pos, token, m->rope_tables_dev, uint32_t(m->rope_tables.size()), m->trig_pairs,
                           s->trig, st);
  HIPC(hipGetLastError());
  if (eager) enqueue_fused_step(s);
  else HIPC(hipGraphLaunch(s->exec, st));
  uint32_t next = 0;
  HIPC(hipMemcpyAsync(&next, s->am_out, 4, hipMemcpyDeviceToHost, st));
  HIPC(hipStreamSynchronize(st));
  for (size_t l = 0; l < m->layers.size(); ++l)
    if (!m->layers[l].donor) kv_advance(s->kv[l], pos + 1);
  s->position += 1;
  s->logits_valid = true;
  const uint64_t H = m->hidden;
  if (flags & DET_COMMIT_ACTIVATIONS) {
    std::vector<int32_t> host(H), lg(m->vocab);
    HIPC(hipMemcpyAsync(host.data(), s->x, H * 4, hipMemcpyDeviceToHost, st));
    HIPC(hipMemcpyAsync(lg.data(), s->logits, m->vocab * 4, hipMemcpyDeviceToHost, st));
    HIPC(hipStreamSynchronize(st));
    commit_rows(host.data(), 1, H, out->activation);
    commit_vector(lg.data(), m->vocab, out->logits);
  }
  out->kv[0] = 0;
  if (flags & DET_COMMIT_KV) commit_kv(s->m->ctx, all_caches(s), out->kv);
  out->next_token = next;
}

std::unique_ptr<det_session> clone_session(const det_session* src) {
  auto s = std::make_unique<det_session>();
  s->m = src->m;
  s->max_tokens = src->max_tokens;
  session_alloc(s.get());
  s->position = src->position;
  det_ctx* ctx = src->m->ctx;
  for (size_t l = 0; l < src->kv.size(); ++l) {
    const GKv& a = src->kv[l];
    GKv& b = s->kv[l];
    b.has = a.has; b.start = a.start; b.len = a.len; b.total = a.total;
    if (a.k) {
      copy_d2d(ctx, b.k, a.k, a.cap * a.row_w * 4);
      copy_d2d(ctx, b.v, a.v, a.cap * a.row_w * 4);
    }
  }
  copy_d2d(ctx, s->logits, src->logits, src->m->vocab * 4);
  s->logits_valid = src->logits_valid;
  HIPC(hipStreamSynchronize(ctx->stream));
  return s;
}

// First-step per-layer capture (det_goldens.rs:187-236): layer output and the
// effective caches (updated layers 0..=l, original layers above).
struct FirstStepHook : LayerHook {
  det_session* original = nullptr;
  std::string json;
  bool after_layer(det_session* s, uint64_t l) override {
    det_model* m = s->m;
    std::vector<int32_t> host(m->hidden);
    HIPC(hipMemcpyAsync(host.data(), s->x, m->hidden * 4, hipMemcpyDeviceToHost, m->ctx->stream));
    HIPC(hipStreamSynchronize(m->ctx->stream));
    char out[65], kv[65];
    commit_rows(host.data(), 1, m->hidden, out);
    std::vector<const GKv*> eff;
    for (uint64_t j = 0; j < s->kv.size(); ++j) eff.push_back(j <= l ? &s->kv[j] : &original->kv[j]);
    const bool has = commit_kv(m->ctx, eff, kv);
    if (!json.empty()) json += ",";
    json += std::string("{\"layer_output\":\"") + out + "\",\"kv\":" + (has ? "\"" + std::string(kv) + "\"" : "null") + "}";
    return false;
  }
};

std::string capture(det_model* m, const uint32_t* ids, uint64_t n, uint64_t steps) {
  det_session s0;
  s0.m = m;
  s0.max_tokens = n + steps + 1;
  session_alloc(&s0);
  det_prefill_result_t pr{};
  prefill(&s0, ids, n, DET_COMMIT_ALL, &pr);
  auto kvj = [](const char* kv) { return kv[0] ? "\"" + std::string(kv) + "\"" : std::string("null"); };
  std::string out = std::string("{\"prefill\":{\"embedding\":\"") + pr.embedding + "\",\"final_hidden\":\"" +
                    pr.final_hidden + "\",\"logits\":\"" + pr.logits + "\",\"kv\":" + kvj(pr.kv) + "},";
  {
    std::unique_ptr<det_session> copy = clone_session(&s0);
    FirstStepHook hook;
    hook.original = &s0;
    det_decode_result_t dr{};
    decode(copy.get(), pr.next_token, DET_COMMIT_NONE, &dr, &hook);
    out += "\"first_step_layers\":[" + hook.json + "],";
  }
  out += "\"decode_steps\":[";
  uint32_t tok = pr.next_token;
  std::string ids_json = "[";
  for (uint64_t i = 0; i < steps; ++i) {
    det_decode_result_t dr{};
    if (m->fused_ok) decode_fused(&s0, tok, DET_COMMIT_ALL, &dr);
    else decode(&s0, tok, DET_COMMIT_ALL, &dr, nullptr);
    if (i) { out += ","; ids_json += ","; }
    ids_json += std::to_string(tok);
    out += "{\"token\":" + std::to_string(tok) + ",\"activation\":\"" + dr.activation + "\",\"logits\":\"" + dr.logits +
           "\",\"kv\":" + kvj(dr.kv) + "}";
    tok = dr.next_token;
  }
  ids_json += "]";
  Sha h;
  h.put(ids_json.data(), ids_json.size());
  char hx[65];
  h.hex(hx);
  out += "],\"end_to_end\":{\"generated_token_ids\":" + ids_json + ",\"generated_token_ids_sha256\":\"" + hx + "\"}}";
  return out;
}

// ---------------------------------------------------------------------------
// Checkpoint trace: the native deterministic sequence (runtime/sequence.rs,
// runtime/executors/native.rs:60-450) with checkpoint commitment. Every
// committed checkpoint adds {name: sha256(compact JSON payload)}
// (runtime/trace.rs:262-330, 425-430); the artifact is the pretty-printed
// array (trace.rs:555-566). Payloads are serde_json maps, whose keys are
// ordered bytewise, so they are written here from std::map.
// ---------------------------------------------------------------------------
std::string json_str(const std::string& v) { return det_audit::json_quote(v); }

// A finite f32 as serde_json writes it: the shortest digit string that reads
// back as the same f32, in plain notation when the decimal point falls within
// [-5, 13] places (with ".0" for whole numbers), else d.ddde<exp>.
std::string json_f32(float v) {
  if (!std::isfinite(v)) return "null";
  if (v == 0.0f) return std::signbit(v) ? "-0.0" : "0.0";
  char buf[64];
  int p = 1;
  for (; p <= 9; ++p) {
    snprintf(buf, sizeof buf, "%.*e", p - 1, double(v));
    if (strtof(buf, nullptr) == v) break;
  }
  std::string t(buf);
  std::string sign;
  if (t[0] == '-') {
    sign = "-";
    t = t.substr(1);
  }
  const size_t epos = t.find('e');
  const int e = std::atoi(t.c_str() + epos + 1);
  std::string d;
  for (size_t i = 0; i < epos; ++i)
    if (t[i] != '.') d += t[i];
  while (d.size() > 1 && d.back() == '0') d.pop_back();
  const int len = int(d.size()), kk = e + 1;  // decimal point after kk digits
  std::string o;
  if (kk >= len && kk <= 13) {
    o = d + std::string(size_t(kk - len), '0') + ".0";
  } else if (kk > 0 && kk <= 13) {
    o = d.substr(0, size_t(kk)) + "." + d.substr(size_t(kk));
  } else if (kk > -6 && kk <= 0) {
    o = "0." + std::string(size_t(-kk), '0') + d;
  } else {
    o = d.substr(0, 1) + (len > 1 ? "." + d.substr(1) : std::string()) + "e" + std::to_string(kk - 1);
  }
  return sign + o;
}

std::string json_u32s(const std::vector<uint32_t>& v) {
  std::string o = "[";
  for (size_t i = 0; i < v.size(); ++i) o += (i ? "," : "") + std::to_string(v[i]);
  return o + "]";
}

std::string json_obj(const std::map<std::string, std::string>& o) {
  std::string s = "{";
  bool first = true;
  for (const auto& kv : o) {
    if (!first) s += ",";
    first = false;
    s += json_str(kv.first) + ":" + kv.second;
  }
  return s + "}";
}

using Fut = std::shared_future<std::string>;

// A commitment future as a payload value: its quoted hex, or null for None ("").
std::string json_fut(const Fut& f) {
  const std::string v = f.get();
  return v.empty() ? "null" : json_str(v);
}
std::string json_futs(const std::vector<Fut>& v, size_t n) {
  std::string o = "[";
  for (size_t i = 0; i < n; ++i) o += (i ? "," : "") + json_fut(v[i]);
  return o + "]";
}

struct TraceCollector {
  // checkpoint name and the builder of its payload; builders run when the
  // artifact is written, once the commitments they read have been hashed
  std::vector<std::pair<std::string, std::function<std::string()>>> entries;
  bool has_terminal = false, reached = false;
  std::string terminal_id;
  uint64_t occurrence = 1, seen = 0;

  // TerminalCheckpointSpec::parse (trace.rs): "id" or "id:occurrence".
  void set_terminal(const char* spec) {
    if (!spec || !*spec) return;
    std::string s(spec);
    const size_t colon = s.rfind(':');
    if (colon != std::string::npos) {
      const std::string n = s.substr(colon + 1);
      if (n.empty() || n.find_first_not_of("0123456789") != std::string::npos)
        bail("terminal checkpoint occurrence must be a positive integer");
      occurrence = std::stoull(n);
      if (occurrence == 0) bail("terminal checkpoint occurrence must be a positive integer");
      s = s.substr(0, colon);
    }
    if (s.empty()) bail("terminal checkpoint id must not be empty");
    terminal_id = s;
    has_terminal = true;
  }
  // mark_terminal_checkpoint (trace.rs:465-480)
  bool mark(const std::string& name) {
    if (!has_terminal) return false;
    if (reached || name != terminal_id) return reached;
    if (++seen == occurrence) reached = true;
    return reached;
  }
  // trace_checkpoint_lazy (trace.rs:266-288); layer_token checkpoints are
  // never committed (trace.rs:451-454), so their payload is not built. The
  // payload builder must own (copy) everything it reads.
  bool checkpoint(const std::string& name, std::function<std::string()> payload) {
    const bool commit = name.rfind("prefill.layer_token.", 0) != 0 && name.rfind("decode.layer_token.", 0) != 0;
    const bool r = mark(name);
    if (commit) entries.emplace_back(name, std::move(payload));
    return r;
  }
  // {checkpoint: sha256(payload)} for every committed checkpoint, in order
  std::vector<std::pair<std::string, std::string>> committed() const {
    std::vector<std::pair<std::string, std::string>> out;
    for (const auto& e : entries) out.emplace_back(e.first, sha_hex(e.second()));
    return out;
  }
  // serde_json::to_vec_pretty of the array of single-entry maps
  std::string artifact() const {
    const auto c = committed();
    if (c.empty()) return "[]";
    std::string o = "[\n";
    for (size_t i = 0; i < c.size(); ++i) {
      o += "  {\n    " + json_str(c[i].first) + ": " + json_str(c[i].second) + "\n  }";
      o += i + 1 < c.size() ? ",\n" : "\n";
    }
    return o + "]";
  }
};

const char* const kDetMode = "\"deterministic\"";

// SamplingConfig (shared/api/input.rs:45-50) as serialized into prompt.prepare.
std::string sampling_json(const det_sampling_t& sp) {
  return std::string("{\"max_new_tokens\":") + (sp.has_max_new_tokens ? std::to_string(sp.max_new_tokens) : "null") +
         ",\"temperature\":" + (sp.has_temperature ? json_f32(sp.temperature) : "null") +
         ",\"top_k\":" + (sp.has_top_k ? std::to_string(sp.top_k) : "null") +
         ",\"top_p\":" + (sp.has_top_p ? json_f32(sp.top_p) : "null") + "}";
}

// Host buffers of one traced sequence. The hashing pool reads the KV mirror
// and the row copies while the GPU runs ahead, so the pool is declared last
// and drains before anything it reads is destroyed.
struct TraceState {
  det_session sess;
  det_commit::KvMirror mirror;
  int32_t* kv_stage = nullptr;  // device: the step's new K/V rows [own layers x 2][max width]
  int32_t* host_stage = nullptr;  // pinned: layer rows | logits | K/V rows
  uint64_t kv_rows = 0, kv_width = 0;
  std::vector<int> own_layers;
  std::unique_ptr<det_commit::HashPool> pool;
  ~TraceState() {
    pool.reset();  // finishes every queued hash before the buffers go
    if (kv_stage) (void)hipFree(kv_stage);
    if (host_stage) (void)hipHostFree(host_stage);
  }
};

// build_det_kv_cache_commitment over the mirror: layer j after total[j] tokens.
Fut commit_mirror(TraceState& ts, std::vector<uint64_t> totals) {
  const det_commit::KvMirror* mirror = &ts.mirror;
  return ts.pool->submit([mirror, totals] {
    std::vector<det_commit::KvLayerView> views;
    for (size_t j = 0; j < totals.size(); ++j) views.push_back(mirror->view(j, totals[j]));
    return det_commit::commit_kv(views);
  });
}

// Runs the traced sequence; returns true when it paused at the terminal
// checkpoint. On an error the collector keeps the checkpoints so far, as
// abort_inference_trace does.
bool trace_run(det_model* m, const det_trace_request_t* rq, TraceCollector& tc) {
  if (!rq) bail("trace request is required");
  tc.set_terminal(rq->terminal_checkpoint);
  if (!rq->prompt_text || !*rq->prompt_text) bail("input embedding requires a non-empty prompt");
  if (!rq->prompt_token_ids || rq->prompt_token_count == 0)
    bail("transformer layer execution requires at least one activation row");
  const std::vector<uint32_t> ids(rq->prompt_token_ids, rq->prompt_token_ids + rq->prompt_token_count);
  const uint64_t n = ids.size(), H = m->hidden, V = m->vocab, nl = m->layers.size();
  const std::string ids_json = json_u32s(ids), ids_sha = sha_hex(ids_json);
  // prompt.prepare (executors/native.rs:68-90): emitted when an authenticated
  // tokenizer source accompanies a deterministic run
  if (rq->prompt_checkpoint) {
    const std::string text = rq->prompt_text, sampling = sampling_json(rq->sampling);
    if (tc.checkpoint("prompt.prepare", [text, ids_json, ids_sha, sampling] {
          return json_obj({{"prompt_text", json_str(text)},
                           {"prompt_token_ids", ids_json},
                           {"prompt_token_ids_sha256", json_str(ids_sha)},
                           {"sampling", sampling}});
        }))
      return true;
  }
  check_ids(m, ids.data(), n);
  const uint64_t max_new = rq->sampling.has_max_new_tokens ? rq->sampling.max_new_tokens : 0;
  det_ctx* ctx = m->ctx;
  hipStream_t st = ctx->stream;
  TraceState ts;
  det_session& sess = ts.sess;
  sess.m = m;
  sess.max_tokens = n + max_new + 1;
  sess.capture_layers = true;
  session_alloc(&sess);
  for (uint64_t l = 0; l < nl; ++l) {
    const GLayer& L = m->layers[l];
    ts.mirror.add_layer(!L.donor, L.num_kv_heads, L.head_dim, L.cache_sliding_window, sess.max_tokens);
    if (!L.donor) {
      ts.own_layers.push_back(int(l));
      ts.kv_width = std::max(ts.kv_width, L.num_kv_heads * L.head_dim);
    }
  }
  ts.kv_rows = 2 * ts.own_layers.size();
  HIPC(hipMalloc(&ts.kv_stage, std::max<uint64_t>(ts.kv_rows * ts.kv_width, 1) * 4));
  HIPC(hipHostMalloc(reinterpret_cast<void**>(&ts.host_stage), (nl * H + V + ts.kv_rows * ts.kv_width + 1) * 4,
                     hipHostMallocDefault));
  ts.pool.reset(new det_commit::HashPool(std::max(2u, std::min(16u, std::thread::hardware_concurrency()) - 1)));
  det_commit::HashPool& pool = *ts.pool;
  auto copy_rows = [&](const int32_t* dev, uint64_t count) {
    auto h = std::make_shared<std::vector<int32_t>>(count);
    if (count) HIPC(hipMemcpyAsync(h->data(), dev, count * 4, hipMemcpyDeviceToHost, st));
    HIPC(hipStreamSynchronize(st));
    return h;
  };
  auto rows_fut = [&](std::shared_ptr<std::vector<int32_t>> h, uint64_t first, uint64_t count, uint64_t width) {
    return pool.submit([h, first, count, width] { return commit_rows(h->data() + first * width, count, width); });
  };

  // input.embedding / prefill.prepare_aux (routines/input_embedding/mod.rs:88-130,
  // routines/prefill_prepare_aux/mod.rs:175-210)
  HIPC(hipMemcpyAsync(sess.ids, ids.data(), n * 4, hipMemcpyHostToDevice, st));
  embed_ids(&sess, n);
  const Fut emb = rows_fut(copy_rows(sess.x, n * H), 0, n, H);
  if (tc.checkpoint("input.embedding", [emb, ids_json, ids_sha] {
        return json_obj({{"det_embedded_prompt_activations_sha256", json_fut(emb)},
                         {"prompt_token_ids", ids_json},
                         {"prompt_token_ids_sha256", json_str(ids_sha)},
                         {"raster", "null"}});
      }))
    return true;
  if (tc.checkpoint("prefill.prepare_aux", [emb, ids_json, ids_sha] {
        return json_obj({{"det_embedded_prompt_activations_sha256", json_fut(emb)},
                         {"prompt_token_ids", ids_json},
                         {"prompt_token_ids_sha256", json_str(ids_sha)}});
      }))
    return true;
  const uint64_t P = m->ple_dim;
  if (m->has_ple)
    for (uint64_t l = 0; l < nl; ++l)
      if (m->layers[l].has_ple) ple_inputs(&sess, l, sess.ids, sess.x, n, sess.ple_all + l * n * P);
  check_rope(m, n - 1);

  // prefill.range per token range and prefill.range_finalize per layer
  // (routines/prefill_range/mod.rs:25-88, routines/prefill_range_finalize/mod.rs:17-73,
  // routines/prefill_range/native/deterministic_tiles.rs:140-190)
  const uint64_t pw = std::min<uint64_t>(std::max<uint64_t>(rq->prefill_token_range_width ? rq->prefill_token_range_width
                                                                                          : UINT64_MAX, 1), n);
  std::vector<Fut> done;  // each layer's output commitment
  bool ready = false;  // the layer's input norm was written by the previous layer
  for (uint64_t l = 0; l < nl; ++l) {
    const GLayer& L = m->layers[l];
    ready = layer_prefill(&sess, L, n, own_cache(&sess, L, l), donor_cache(&sess, L),
                          (m->has_ple && L.has_ple) ? sess.ple_all + l * n * P : nullptr,
                          l + 1 < nl ? &m->layers[l + 1] : nullptr, ready);
    if (!L.donor) {
      // the rows this layer's cache keeps, from the projection rows (kb / vb
      // hold all n rows until the next layer's projections)
      auto& ml = ts.mirror.layer(l);
      const uint64_t kept = ml.window ? std::min(n, *ml.window) : n, first = n - kept;
      HIPC(hipMemcpyAsync(ml.k.get() + first * ml.width, sess.kb + first * ml.width, kept * ml.width * 4,
                          hipMemcpyDeviceToHost, st));
      HIPC(hipMemcpyAsync(ml.v.get() + first * ml.width, sess.vb + first * ml.width, kept * ml.width * 4,
                          hipMemcpyDeviceToHost, st));
    }
    const auto rows = copy_rows(sess.x, n * H);
    const Fut all = rows_fut(rows, 0, n, H);
    done.push_back(all);
    for (uint64_t a = 0; a < n; a += pw) {
      const uint64_t b = std::min(n, a + pw);
      const Fut rc = (a == 0 && b == n) ? all : rows_fut(rows, a, b - a, H);
      if (tc.checkpoint("prefill.range", [rc, l, a, b, n] {
            return json_obj({{"det_range_activations_sha256", json_fut(rc)},
                             {"execution_mode", kDetMode},
                             {"layer_idx", std::to_string(l)},
                             {"range_end", std::to_string(b)},
                             {"range_start", std::to_string(a)},
                             {"token_count", std::to_string(n)}});
          }))
        return true;
    }
    const Fut kv = commit_mirror(ts, std::vector<uint64_t>(l + 1, n));
    const std::vector<Fut> so_far = done;
    if (tc.checkpoint("prefill.range_finalize", [so_far, all, kv, l] {
          return json_obj({{"completed_layer_output_det_sha256s", json_futs(so_far, so_far.size())},
                           {"det_current_activations_sha256", json_fut(all)},
                           {"det_layer_caches_sha256", json_fut(kv)},
                           {"execution_mode", kDetMode},
                           {"next_layer_idx", std::to_string(l + 1)}});
        }))
      return true;
    for (uint64_t t = 0; t < n; ++t)
      if (tc.mark("prefill.layer_token.layer_" + std::to_string(l) + ".token_" + std::to_string(t))) return true;
  }
  // prefill.finalize (prefill_finalize/native/tiles.rs:68-94): the final
  // hidden states are the last layer's output rows
  logits_from(&sess, sess.x + (n - 1) * H);
  sess.position = n;
  const Fut final_hidden = done.back();
  const Fut kv_all = commit_mirror(ts, std::vector<uint64_t>(nl, n));
  uint32_t next = ctx->argmax(sess.logits, V);
  Fut logits;
  {
    const auto lg = copy_rows(sess.logits, V);
    logits = pool.submit([lg, V] { return commit_vector(lg->data(), V); });
  }
  if (tc.checkpoint("prefill.finalize", [n, final_hidden, kv_all, logits] {
        return json_obj({{"decode_position", std::to_string(n)},
                         {"decode_token_count", std::to_string(n)},
                         {"det_final_hidden_states_sha256", json_fut(final_hidden)},
                         {"det_layer_caches_sha256", json_fut(kv_all)},
                         {"det_prefill_logits_sha256", json_fut(logits)}});
      }))
    return true;
  // validate_sampling_config (runtime/pipeline.rs:22-40)
  if (rq->sampling.has_temperature && std::fabs(rq->sampling.temperature - 1.0f) > FLT_EPSILON)
    bail("output decode only supports deterministic greedy decode; expected temperature 1, got " +
         json_f32(rq->sampling.temperature));
  if (rq->sampling.has_top_k) bail("output decode does not support top_k yet, got " + std::to_string(rq->sampling.top_k));
  if (rq->sampling.has_top_p) bail("output decode does not support top_p yet, got " + json_f32(rq->sampling.top_p));

  // the output decode loop (executors/native.rs:265-450)
  std::vector<uint32_t> full = ids, gen;
  const uint64_t dw = std::min<uint64_t>(std::max<uint64_t>(rq->decode_layer_range_width ? rq->decode_layer_range_width
                                                                                         : UINT64_MAX, 1), std::max<uint64_t>(nl, 1));
  int32_t* h_layers = ts.host_stage;
  int32_t* h_logits = h_layers + nl * H;
  int32_t* h_kv = h_logits + V;
  for (;;) {
    if (gen.size() >= max_new) {
      // output.finalize (output_finalize/mod.rs:18-52)
      std::string text;
      if (!gen.empty()) {
        if (!rq->detokenize) bail("output.finalize requires a detokenize callback");
        std::vector<char> buf(4096);
        for (;;) {
          const int64_t len = rq->detokenize(gen.data(), gen.size(), buf.data(), buf.size(), rq->detokenize_user);
          if (len < 0) bail("detokenize callback failed");
          if (uint64_t(len) < buf.size()) {
            text.assign(buf.data(), size_t(len));
            break;
          }
          buf.resize(size_t(len) + 1);
        }
      }
      const std::string full_json = json_u32s(full), gen_json = json_u32s(gen);
      const uint64_t count = gen.size();
      tc.checkpoint("output.finalize", [full_json, gen_json, text, count] {
        return json_obj({{"full_token_ids", full_json},
                         {"full_token_ids_sha256", json_str(sha_hex(full_json))},
                         {"generated_text", json_str(text)},
                         {"generated_token_count", std::to_string(count)},
                         {"generated_token_ids", gen_json},
                         {"generated_token_ids_sha256", json_str(sha_hex(gen_json))},
                         {"stop_reason", "\"max_new_tokens\""}});
      });
      return tc.reached;
    }
    // decode.select_token (decode_select_token/mod.rs:19-47, 362-390)
    const uint32_t t = next;
    full.push_back(t);
    gen.push_back(t);
    const uint64_t pos = sess.position;
    const std::string full_json = json_u32s(full), gen_json = json_u32s(gen);
    if (tc.checkpoint("decode.select_token", [pos, logits, full_json, gen_json, max_new, t] {
          return json_obj({{"decode_position", std::to_string(pos)},
                           {"decode_token_count", std::to_string(pos)},
                           {"det_current_logits_sha256", json_fut(logits)},
                           {"full_token_ids", full_json},
                           {"full_token_ids_sha256", json_str(sha_hex(full_json))},
                           {"generated_token_ids", gen_json},
                           {"generated_token_ids_sha256", json_str(sha_hex(gen_json))},
                           {"max_new_tokens", std::to_string(max_new)},
                           {"selected_next_token", std::to_string(t)}});
        }))
      return true;
    // one decode step; every layer's output row lands in sess.layer_rows
    det_decode_result_t dr{};
    if (m->fused_ok) decode_fused(&sess, t, DET_COMMIT_NONE, &dr);
    else decode(&sess, t, DET_COMMIT_NONE, &dr, nullptr, sess.layer_rows);
    next = dr.next_token;
    // the token's K/V rows of every layer with its own cache
    for (size_t i0 = 0; i0 < ts.own_layers.size(); i0 += det::kMaxRowPtrs / 2) {
      det::RowPtrs g{};
      const size_t i1 = std::min(ts.own_layers.size(), i0 + det::kMaxRowPtrs / 2);
      for (size_t i = i0; i < i1; ++i) {
        const GKv& c = sess.kv[size_t(ts.own_layers[i])];
        const uint64_t slot = c.ring ? pos % c.cap : pos;
        g.src[g.n] = c.k + slot * c.row_w;
        g.width[g.n++] = uint32_t(c.row_w);
        g.src[g.n] = c.v + slot * c.row_w;
        g.width[g.n++] = uint32_t(c.row_w);
      }
      g.stride = uint32_t(ts.kv_width);
      det::launch_gather_row_ptrs(g, ts.kv_stage + 2 * i0 * ts.kv_width, st);
    }
    HIPC(hipMemcpyAsync(h_layers, sess.layer_rows, nl * H * 4, hipMemcpyDeviceToHost, st));
    HIPC(hipMemcpyAsync(h_logits, sess.logits, V * 4, hipMemcpyDeviceToHost, st));
    if (ts.kv_rows) HIPC(hipMemcpyAsync(h_kv, ts.kv_stage, ts.kv_rows * ts.kv_width * 4, hipMemcpyDeviceToHost, st));
    HIPC(hipStreamSynchronize(st));
    for (size_t i = 0; i < ts.own_layers.size(); ++i) {
      auto& ml = ts.mirror.layer(size_t(ts.own_layers[i]));
      std::memcpy(ml.k.get() + pos * ml.width, h_kv + (2 * i) * ts.kv_width, ml.width * 4);
      std::memcpy(ml.v.get() + pos * ml.width, h_kv + (2 * i + 1) * ts.kv_width, ml.width * 4);
    }
    auto outs = std::make_shared<std::vector<int32_t>>(h_layers, h_layers + nl * H);
    auto lg = std::make_shared<std::vector<int32_t>>(h_logits, h_logits + V);
    std::vector<Fut> layer_out;
    for (uint64_t l = 0; l < nl; ++l) layer_out.push_back(rows_fut(outs, l, 1, H));
    logits = pool.submit([lg, V] { return commit_vector(lg->data(), V); });
    // decode.layer_range per layer range (routines/decode_layer_range/mod.rs:553-664,
    // native/tiles.rs:35-70): the activation after the range, the effective
    // caches (layers below the range end updated, the rest as before the step)
    // and the layer outputs so far
    for (uint64_t a = 0; a < nl; a += dw) {
      const uint64_t b = std::min(nl, a + dw);
      std::vector<uint64_t> totals(nl, pos);
      for (uint64_t j = 0; j < b; ++j) totals[j] = pos + 1;
      const Fut kv = commit_mirror(ts, totals);
      const Fut act = layer_out[b - 1];
      if (tc.checkpoint("decode.layer_range", [layer_out, act, kv, pos, nl, a, b, t] {
            return json_obj({{"completed_layer_output_det_sha256s", json_futs(layer_out, b)},
                             {"decode_position", std::to_string(pos)},
                             {"decode_token_count", std::to_string(pos)},
                             {"det_current_activation_sha256", json_fut(act)},
                             {"det_layer_caches_sha256", json_fut(kv)},
                             {"execution_mode", kDetMode},
                             {"layer_count", std::to_string(nl)},
                             {"layer_end", std::to_string(b)},
                             {"layer_start", std::to_string(a)},
                             {"next_token", std::to_string(t)}});
          }))
        return true;
    }
    // decode.transition_finalize (decode_transition_finalize/mod.rs:67-99)
    if (tc.checkpoint("decode.transition_finalize", [pos, logits, full_json, gen_json] {
          return json_obj({{"decode_position", std::to_string(pos + 1)},
                           {"decode_token_count", std::to_string(pos + 1)},
                           {"det_current_logits_sha256", json_fut(logits)},
                           {"full_token_ids", full_json},
                           {"full_token_ids_sha256", json_str(sha_hex(full_json))},
                           {"generated_token_ids", gen_json},
                           {"generated_token_ids_sha256", json_str(sha_hex(gen_json))}});
        }))
      return true;
  }
}

// ---------------------------------------------------------------------------
// Layer-level operators (the reference's det_kernels.rs API) on caller buffers
// ---------------------------------------------------------------------------
det_session* scratch_rows(det_scratch* sc, uint64_t rows) {
  if (!sc->ws || sc->ws->max_tokens < rows) {
    HIPC(hipStreamSynchronize(sc->m->ctx->stream));
    auto w = std::make_unique<det_session>();
    w->m = sc->m;
    w->max_tokens = std::max<uint64_t>(rows, sc->ws ? 2 * sc->ws->max_tokens : 16);
    session_alloc(w.get(), false);
    sc->ws = std::move(w);
  }
  return sc->ws.get();
}

const GLayer& need_layer(det_model* m, uint64_t layer) {
  if (!m->finalized) bail("model is not finalized");
  if (layer >= m->layers.size())
    bail("layer index " + std::to_string(layer) + " out of range for " + std::to_string(m->layers.size()) + " layers");
  return m->layers[layer];
}

void need_handles(det_model* m, det_scratch* sc, const det_kv* a, const det_kv* b) {
  if (!sc || sc->m != m) bail("scratch belongs to another model");
  if ((a && a->m != m) || (b && b->m != m)) bail("KV cache belongs to another model");
}

}  // namespace

// ---------------------------------------------------------------------------
// Allocation-free argmax scratch: one int64 key per 1024-element part of the
// input, in a file-scope device array (each GPU holds its own copy until the
// process ends) instead of context memory allocated on demand. Every call on a
// GPU shares that GPU's array, so calls that overlap on one GPU race.
// ---------------------------------------------------------------------------
constexpr uint64_t kNoAllocArgmaxMax = uint64_t(1) << 24;  // elements per call
static __device__ __align__(256) int64_t g_argmax_parts[kNoAllocArgmaxMax / 1024];

namespace {

std::mutex g_noalloc_mu;
std::map<int, int64_t*> g_noalloc_parts;  // device -> address of g_argmax_parts on it

// Address of this device's copy of g_argmax_parts (the device must be
// current); looked up once per device. The array's name in host code is not
// a device address, so kernels only ever receive this pointer.
int64_t* noalloc_parts_on(int device) {
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  auto it = g_noalloc_parts.find(device);
  if (it != g_noalloc_parts.end()) return it->second;
  void* p = nullptr;
  HIPC(hipGetSymbolAddress(&p, HIP_SYMBOL(g_argmax_parts)));
  if (!p) throw Status(3, "hipGetSymbolAddress returned no address for the argmax scratch");
  g_noalloc_parts[device] = static_cast<int64_t*>(p);
  return static_cast<int64_t*>(p);
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
namespace {
// Writes s plus a NUL into out when it fits; *out_len = its length.
void put_text(const std::string& s, char* out, size_t out_cap, size_t* out_len, const char* what) {
  if (out_len) *out_len = s.size();
  if (!out || out_cap <= s.size())
    bail(std::string(what) + " buffer too small: need " + std::to_string(s.size() + 1) + " bytes");
  std::memcpy(out, s.data(), s.size());
  out[s.size()] = 0;
}
template <class F>
auto audit_input(F&& f) -> decltype(f()) {
  try {
    return f();
  } catch (const det_audit::Error& e) {
    bail(e.what());
  }
}
}  // namespace

extern "C" {

const char* det_version(void) { return "detgpu 0.1 gfx950 (int8-limb MFMA GEMV, integer softmax attention)"; }

int det_ctx_create(int device, det_ctx_t** out) {
  return guarded(nullptr, [&] {
    if (!out) bail("null output pointer");
    int n = 0;
    HIPC(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) bail("invalid HIP device " + std::to_string(device));
    auto c = std::make_unique<det_ctx>();
    c->device = device;
    HIPC(hipSetDevice(device));
    HIPC(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
    HIPC(hipMalloc(&c->argmax_out, 4));
    c->noalloc_parts = noalloc_parts_on(device);
    *out = c.release();
  });
}

void det_ctx_destroy(det_ctx_t* ctx) {
  if (!ctx) return;
  (void)hipStreamSynchronize(ctx->stream);
  if (ctx->limbs) (void)hipFree(ctx->limbs);
  if (ctx->gemm_a) (void)hipFree(ctx->gemm_a);
  if (ctx->gemm_planes) (void)hipFree(ctx->gemm_planes);
  if (ctx->attn_work) (void)hipFree(ctx->attn_work);
  if (ctx->argmax_scratch) (void)hipFree(ctx->argmax_scratch);
  if (ctx->argmax_out) (void)hipFree(ctx->argmax_out);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

const char* det_ctx_last_error(const det_ctx_t* ctx) { return ctx ? ctx->last_error.c_str() : g_error.c_str(); }

int det_ctx_synchronize(det_ctx_t* ctx) {
  return guarded(ctx, [&] { HIPC(hipStreamSynchronize(ctx->stream)); });
}

int det_device_alloc(det_ctx_t* ctx, size_t bytes, void** out) {
  return guarded(ctx, [&] { HIPC(hipMalloc(out, std::max<size_t>(bytes, 1))); });
}
int det_device_free(det_ctx_t* ctx, void* p) {
  return guarded(ctx, [&] {
    HIPC(hipStreamSynchronize(ctx->stream));
    HIPC(hipFree(p));
  });
}
int det_memcpy_h2d(det_ctx_t* ctx, void* dst, const void* src, size_t bytes) {
  return guarded(ctx, [&] {
    HIPC(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
    HIPC(hipStreamSynchronize(ctx->stream));
  });
}
int det_memcpy_d2h(det_ctx_t* ctx, void* dst, const void* src, size_t bytes) {
  return guarded(ctx, [&] {
    HIPC(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
    HIPC(hipStreamSynchronize(ctx->stream));
  });
}
int det_memcpy_d2d(det_ctx_t* ctx, void* dst, const void* src, size_t bytes) {
  return guarded(ctx, [&] { copy_d2d(ctx, dst, src, bytes); });
}

int det_event_create(det_ctx_t* ctx, det_event_t** out) {
  return guarded(ctx, [&] {
    auto e = std::make_unique<det_event>();
    HIPC(hipEventCreate(&e->ev));
    *out = e.release();
  });
}
int det_event_record(det_ctx_t* ctx, det_event_t* ev) {
  return guarded(ctx, [&] { HIPC(hipEventRecord(ev->ev, ctx->stream)); });
}
int det_ctx_capture_begin(det_ctx_t* ctx) {
  return guarded(ctx, [&] {
    if (ctx->capturing) bail("det_ctx_capture_begin: the context is already capturing");
    HIPC(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
    ctx->capturing = true;
  });
}
int det_ctx_capture_end(det_ctx_t* ctx, det_graph_t** out) {
  return guarded(ctx, [&] {
    if (!out) bail("det_ctx_capture_end requires an output handle");
    *out = nullptr;
    if (!ctx->capturing) bail("det_ctx_capture_end: no capture in progress (a failed call ends it)");
    ctx->capturing = false;
    auto g = std::make_unique<det_graph>();
    HIPC(hipStreamEndCapture(ctx->stream, &g->graph));
    HIPC(hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0));
    *out = g.release();
  });
}
int det_graph_launch(det_ctx_t* ctx, det_graph_t* g) {
  return guarded(ctx, [&] {
    if (!g || !g->exec) bail("det_graph_launch requires an instantiated graph");
    if (ctx->capturing) bail("det_graph_launch: the context is capturing");
    HIPC(hipGraphLaunch(g->exec, ctx->stream));
  });
}
void det_graph_destroy(det_graph_t* g) { delete g; }
int det_event_elapsed_ms(det_ctx_t* ctx, det_event_t* a, det_event_t* b, float* ms) {
  return guarded(ctx, [&] {
    HIPC(hipEventSynchronize(b->ev));
    HIPC(hipEventElapsedTime(ms, a->ev, b->ev));
  });
}
void det_event_destroy(det_event_t* ev) {
  if (!ev) return;
  (void)hipEventDestroy(ev->ev);
  delete ev;
}

int det_matrix_upload(det_ctx_t* ctx, uint64_t rows, uint64_t cols, int width, const void* values,
                      const int32_t* row_scale, det_matrix_t** out) {
  return guarded(ctx, [&] {
    if (!values && rows * cols) bail("null weight values");
    auto m = std::make_unique<det_matrix>();
    m->ctx = ctx;
    m->m = upload_matrix(ctx, rows, cols, width, values, row_scale);
    *out = m.release();
  });
}
int det_matrix_info(const det_matrix_t* m, uint64_t* rows, uint64_t* cols, int* storage) {
  if (!m) return 1;
  if (rows) *rows = m->m.rows;
  if (cols) *cols = m->m.cols;
  // int8 x scale, or the width class of values held as digit planes / wide
  if (storage) *storage = m->m.storage == det::kInt8 && m->m.planes == 1 ? det::kInt8 : m->m.value_width;
  return 0;
}
void det_matrix_free(det_matrix_t* m) {
  if (!m) return;
  (void)hipStreamSynchronize(m->ctx->stream);
  free_matrix(m->m);
  delete m;
}

int det_linear(det_ctx_t* ctx, const det_matrix_t* w, const int32_t* act, int32_t* out) {
  return guarded(ctx, [&] { det::launch_linear(w->m, act, 1, w->m.cols, out, w->m.rows, nullptr, ctx->limbs, ctx->stream); });
}
int det_linear_acc_i64(det_ctx_t* ctx, const det_matrix_t* w, const int32_t* act, int64_t* acc) {
  return guarded(ctx, [&] { det::launch_linear(w->m, act, 1, w->m.cols, nullptr, w->m.rows, acc, ctx->limbs, ctx->stream); });
}
int det_linear_slab(det_ctx_t* ctx, const det_matrix_t* w, uint64_t m, const int32_t* act, int32_t* out) {
  return guarded(ctx, [&] { ctx->linear(w->m, act, m, w->m.cols, out, w->m.rows, nullptr); });
}
int det_rms_norm(det_ctx_t* ctx, int32_t* x, uint64_t rows, uint64_t cols, const int32_t* w, int64_t eps) {
  return guarded(ctx, [&] {
    if (cols == 0) contract("rms_norm requires a non-empty input slice");
    if (eps < 0) contract("rms_norm_scale requires a non-negative epsilon");
    if (cols > UINT32_MAX) bail("row width should fit in u32");
    det::launch_rmsnorm(x, rows, cols, cols, w, eps, ctx->stream);
  });
}
int det_rope(det_ctx_t* ctx, int32_t* x, uint64_t rows, uint64_t heads, uint64_t hd, uint64_t rotary, uint64_t fbd,
             int64_t base, uint64_t pos0, uint64_t pos_step) {
  return guarded(ctx, [&] {
    if (rotary == 0) return;
    if (rotary % 2) contract("rope_rotate_pairs requires an even rotary_dim");
    if (rotary > hd) contract("rope_rotate_pairs requires rotary_dim to fit within the input width");
    if (fbd < 2 || fbd % 2) contract("rope_rotate_pairs requires an even freq_base_dim of at least 2");
    if (base <= 0) contract("rope_rotate_pairs requires a positive base");
    if (base == INT64_MAX && fbd / 2 > 1) {
      // position 0 is the identity and returns before the frequency step;
      // any later position reaches the overflowing bisection (ops.rs:578)
      if (rows > 0 && (pos0 > 0 || (rows > 1 && pos_step > 0)))
        contract("nth_root_acc: attempt to add with overflow (RoPE base i64::MAX)");
      return;
    }
    std::vector<int64_t> tab(rotary / 2);
    det::rope_inv_freq_table(base, uint32_t(fbd), uint32_t(rotary / 2), tab.data());
    int64_t* d = nullptr;
    HIPC(hipMalloc(&d, tab.size() * 8));
    HIPC(hipMemcpyAsync(d, tab.data(), tab.size() * 8, hipMemcpyHostToDevice, ctx->stream));
    det::launch_rope(x, rows, heads * hd, heads, hd, rotary / 2, d, pos0, pos_step, ctx->stream);
    HIPC(hipStreamSynchronize(ctx->stream));
    HIPC(hipFree(d));
  });
}
int det_attention_causal(det_ctx_t* ctx, const int32_t* q, const int32_t* k, const int32_t* v, uint64_t nq,
                         uint64_t nrows, uint64_t nh, uint64_t nkv, uint64_t hd, uint64_t window, int32_t* out) {
  return guarded(ctx, [&] {
    if (nkv == 0 || nh / nkv == 0) bail("invalid Gemma head configuration");
    if ((nh - 1) / (nh / nkv) >= nkv) contract("query head maps past the last KV head");
    if (nq == 0 || nh == 0 || hd == 0) bail("empty attention problem");
    if (nrows < nq) contract("attention_softmax requires a non-empty logits slice");
    if (nrows > det::kMaxAttentionRows) bail("attention window longer than 16000 rows is not supported");
    det::AttnArgs a{};
    a.q = q; a.q_ld = nh * hd; a.k = k; a.v = v; a.kv_ld = nkv * hd;
    a.out = out; a.out_ld = nh * hd; a.hd = uint32_t(hd); a.num_heads = uint32_t(nh);
    a.groups = uint32_t(nh / nkv); a.n_queries = uint32_t(nq); a.causal = 1; a.window = window;
    a.causal_offset = 0; a.avail = nrows;
    ctx->attach_attn_work(a);
    det::launch_attention(a, ctx->stream);
  });
}
int det_argmax_first(det_ctx_t* ctx, const int32_t* x, uint64_t n, uint32_t* index) {
  return guarded(ctx, [&] {
    if (n == 0) contract("argmax_first requires a non-empty slice");
    *index = ctx->argmax(x, n);
  });
}
int det_argmax_first_noalloc(det_ctx_t* ctx, const int32_t* x, uint64_t n, uint32_t* index_dev) {
  return guarded(ctx, [&] {
    if (n == 0) contract("argmax_first requires a non-empty slice");
    if (n > kNoAllocArgmaxMax)
      bail("allocation-free argmax takes at most " + std::to_string(kNoAllocArgmaxMax) + " elements, got " +
           std::to_string(n));
    if (!x || !index_dev) bail("input and index device pointers are required");
    // the same two kernels as det_argmax_first; the part keys go to the static
    // array (every part is written before the final pass reads it, so nothing
    // needs clearing) and nothing is allocated, copied to the host or waited on
    det::launch_argmax(x, n, ctx->noalloc_parts, index_dev, ctx->stream);
    HIPC(hipGetLastError());
  });
}
int det_elementwise(det_ctx_t* ctx, int op, int32_t* x, const int32_t* y, uint64_t n, int32_t scalar) {
  return guarded(ctx, [&] {
    switch (op) {
      case DET_EW_ADD: det::launch_add_sat(x, y, n, ctx->stream); break;
      case DET_EW_GELU_MUL: det::launch_gelu_mul(x, y, n, ctx->stream); break;
      case DET_EW_SCALE: det::launch_scale(x, n, scalar, ctx->stream); break;
      case DET_EW_SOFTCAP:
        if (scalar <= 0) contract("softcap_act requires a strictly positive softcap");
        det::launch_softcap(x, n, scalar, ctx->stream);
        break;
      default: bail("unknown elementwise op");
    }
  });
}

int det_model_create(det_ctx_t* ctx, const det_text_config_t* cfg, det_model_t** out) {
  return guarded(ctx, [&] {
    auto m = std::make_unique<det_model>();
    m->ctx = ctx;
    m->cfg = *cfg;
    if (cfg->num_layer_types && !cfg->layer_types) bail("layer_types pointer is null");
    m->layer_types.assign(cfg->layer_types, cfg->layer_types + cfg->num_layer_types);
    m->cfg.layer_types = nullptr;
    *out = m.release();
  });
}

int det_model_set_tensor(det_model_t* m, const char* name, uint64_t rank, const uint64_t* dims, int width,
                         const void* values, const int32_t* row_scale) {
  return guarded(m->ctx, [&] {
    if (m->finalized) bail("model is already finalized");
    if (rank < 1 || rank > 2) bail("tensor rank must be 1 or 2");
    HostTensor t;
    t.shape.assign(dims, dims + rank);
    const uint64_t rows = rank == 2 ? dims[0] : 1, cols = rank == 2 ? dims[1] : dims[0];
    if (rank == 2) {
      t.is_matrix = true;
      t.mat = upload_matrix(m->ctx, rows, cols, width, values, row_scale);
    } else {
      t.vec.resize(cols);
      for (uint64_t i = 0; i < cols; ++i) {
        int64_t v;
        if (width == 8) v = int64_t(static_cast<const int8_t*>(values)[i]) * (row_scale ? row_scale[0] : 1);
        else if (width == 16) v = static_cast<const int16_t*>(values)[i];
        else if (width == 32) v = static_cast<const int32_t*>(values)[i];
        else bail("unsupported element width");
        if (v < INT32_MIN || v > INT32_MAX) bail("weight value does not fit Q16.16");
        t.vec[i] = int32_t(v);
      }
    }
    auto it = m->tensors.find(name);
    if (it != m->tensors.end() && it->second.is_matrix) free_matrix(it->second.mat);
    m->tensors[name] = std::move(t);
  });
}

int det_model_load_detwgt(det_model_t* m, const uint8_t* bytes, size_t len) {
  return guarded(m->ctx, [&] {
    if (m->finalized) bail("model is already finalized");
    load_detwgt(m, bytes, len);
  });
}
int det_model_finalize(det_model_t* m) { return guarded(m->ctx, [&] { finalize(m); }); }
int det_model_fused_decode(const det_model_t* m) { return !m || !m->finalized ? -1 : (m->fused_ok ? 1 : 0); }
void det_model_free(det_model_t* m) {
  if (!m) return;
  (void)hipStreamSynchronize(m->ctx->stream);
  delete m;
}

int det_session_create(det_model_t* m, uint64_t max_tokens, det_session_t** out) {
  return guarded(m->ctx, [&] {
    if (!m->finalized) bail("model is not finalized");
    if (max_tokens == 0) bail("max_tokens must be positive");
    auto s = std::make_unique<det_session>();
    s->m = m;
    s->max_tokens = max_tokens;
    session_alloc(s.get());
    *out = s.release();
  });
}
int det_session_clone(const det_session_t* src, det_session_t** out) {
  return guarded(src->m->ctx, [&] { *out = clone_session(src).release(); });
}
void det_session_free(det_session_t* s) {
  if (!s) return;
  (void)hipStreamSynchronize(s->ctx->stream);
  delete s;
}
int det_session_prefill(det_session_t* s, const uint32_t* ids, uint64_t n, uint32_t flags, det_prefill_result_t* out) {
  return guarded(s->m->ctx, [&] {
    det_prefill_result_t tmp{};
    prefill(s, ids, n, flags, out ? out : &tmp);
  });
}
int det_session_decode(det_session_t* s, uint32_t token, uint32_t flags, det_decode_result_t* out) {
  return guarded(s->m->ctx, [&] {
    det_decode_result_t tmp{};
    if (s->m->fused_ok && !(flags & DET_DECODE_PER_OP)) decode_fused(s, token, flags, out ? out : &tmp);
    else decode(s, token, flags, out ? out : &tmp, nullptr);
  });
}
int det_session_decode_batch(det_session_t* const* sessions, uint64_t n, const uint32_t* tokens, uint32_t flags,
                             det_decode_result_t* out) {
  if (!sessions || n == 0 || !sessions[0]) {
    g_error = "batched decode requires at least one session";
    return 1;
  }
  return guarded(sessions[0]->m->ctx, [&] {
    std::vector<det_decode_result_t> tmp(out ? 0 : n);
    // (the batched fused step has no PLE stage: PLE models batch per op)
    if (batch_fused_ok(sessions[0]->m) && !(flags & DET_DECODE_PER_OP))
      decode_batch_fused(sessions, n, tokens, flags, out ? out : tmp.data());
    else
      decode_batch(sessions, n, tokens, flags, out ? out : tmp.data());
  });
}
int det_session_logits(det_session_t* s, int32_t* out, uint64_t n) {
  return guarded(s->m->ctx, [&] {
    if (!s->logits_valid) bail("no logits yet");
    if (n != s->m->vocab) bail("logits length mismatch");
    HIPC(hipMemcpyAsync(out, s->logits, n * 4, hipMemcpyDeviceToHost, s->m->ctx->stream));
    HIPC(hipStreamSynchronize(s->m->ctx->stream));
  });
}
int det_session_position(const det_session_t* s, uint64_t* position) {
  *position = s->position;
  return 0;
}
// Counter-hash synthetic int8 weights (splitmix64 finaliser over the byte
// counter, 8 bytes per hash; q = byte % 255 - 127; s = 1 + u32 % scale_max).
static inline uint64_t synth_mix(uint64_t x) {
  x ^= x >> 30; x *= 0xBF58476D1CE4E5B9ull;
  x ^= x >> 27; x *= 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}
int det_synthetic_int8(uint64_t seed, uint64_t rows, uint64_t cols, int32_t scale_max, int8_t* q, int32_t* s) {
  return guarded(nullptr, [&] {
    if (scale_max < 1) bail("scale_max must be positive");
    const uint64_t base = seed * 0x9E3779B97F4A7C15ull;
    const uint64_t nbytes = rows * cols;
    parallel_rows((nbytes + 7) / 8, [&](uint64_t w0, uint64_t w1) {
      for (uint64_t w = w0; w < w1; ++w) {
        const uint64_t h = synth_mix(base + w);
        for (int b = 0; b < 8 && w * 8 + b < nbytes; ++b) q[w * 8 + b] = int8_t(int(uint8_t(h >> (8 * b)) % 255) - 127);
      }
    });
    const uint64_t sbase = (seed ^ 0x5CA1Eull) * 0x9E3779B97F4A7C15ull;
    for (uint64_t r = 0; r < rows; ++r) {
      const uint64_t h = synth_mix(sbase + r / 2);
      const uint32_t u = uint32_t(h >> (32 * (r & 1)));
      s[r] = int32_t(u % uint32_t(scale_max)) + 1;
    }
  });
}

int det_synthetic_i16(uint64_t seed, uint64_t rows, uint64_t cols, int32_t lim, int16_t* w) {
  return guarded(nullptr, [&] {
    if (lim < 1 || lim > 32767) bail("lim must be in [1, 32767]");
    const uint64_t base = seed * 0x9E3779B97F4A7C15ull;
    const uint64_t n = rows * cols;
    const uint32_t span = uint32_t(2 * lim + 1);
    parallel_rows((n + 3) / 4, [&](uint64_t w0, uint64_t w1) {
      for (uint64_t u = w0; u < w1; ++u) {
        const uint64_t h = synth_mix(base + u);
        for (int k = 0; k < 4 && u * 4 + k < n; ++k)
          w[u * 4 + k] = int16_t(int32_t(uint32_t(uint16_t(h >> (16 * k))) % span) - lim);
      }
    });
    for (uint64_t r = 0; r < rows; ++r) w[r * cols] = 1;
    if (cols > 1) {
      const uint64_t cbase = (seed ^ 0xE7ull) * 0x9E3779B97F4A7C15ull;
      for (uint64_t r = 0; r < rows; ++r) {
        const bool hi = r % 7 == 0, lo = r % 11 == 3 && !hi;
        if (!hi && !lo) continue;
        const uint32_t u = uint32_t(synth_mix(cbase + r / 2) >> (32 * (r & 1)));
        const uint64_t c = u % uint32_t(cols - 1) + 1;
        w[r * cols + c] = hi ? int16_t(32767) : int16_t(-32768);
      }
    }
  });
}

int det_capture(det_model_t* m, const uint32_t* prompt, uint64_t n, uint64_t steps, char* out, size_t cap) {
  return guarded(m->ctx, [&] {
    if (!m->finalized) bail("model is not finalized");
    std::string s = capture(m, prompt, n, steps);
    if (s.size() + 1 > cap) bail("capture output buffer too small: need " + std::to_string(s.size() + 1));
    std::memcpy(out, s.c_str(), s.size() + 1);
  });
}

int det_trace_run(det_model_t* m, const det_trace_request_t* request, char* out, size_t out_cap, size_t* out_len,
                  int32_t* paused) {
  if (!m) {
    g_error = "model is required";
    return 1;
  }
  TraceCollector tc;
  bool p = false;
  int st = guarded(m->ctx, [&] {
    if (!m->finalized) bail("model is not finalized");
    p = trace_run(m, request, tc);
  });
  // the payloads of the checkpoints so far (also after an error); trace_run
  // has drained its hashing pool, so every commitment they read is ready
  std::string art;
  const int st_art = guarded(m->ctx, [&] { art = tc.artifact(); });
  if (st == 0) st = st_art;
  if (out_len) *out_len = art.size();
  if (paused) *paused = p ? 1 : 0;
  if (out && out_cap > art.size()) {
    std::memcpy(out, art.data(), art.size());
    out[art.size()] = 0;
  } else if (st == 0) {
    m->ctx->last_error = "trace artifact buffer too small: need " + std::to_string(art.size() + 1) + " bytes";
    st = 1;
  }
  return st;
}

int det_trace_locate_divergence(const char* claimed, size_t claimed_len, const char* replayed, size_t replayed_len,
                                char* out, size_t out_cap, size_t* out_len, int32_t* diverged) {
  return guarded(nullptr, [&] {
    if ((!claimed && claimed_len) || (!replayed && replayed_len)) bail("trace bytes are required");
    const auto c = audit_input([&] { return det_audit::parse_trace(claimed, claimed_len); });
    const auto r = audit_input([&] { return det_audit::parse_trace(replayed, replayed_len); });
    bool d = false;
    const std::string o = det_audit::outcome_json(c, r, &d);
    if (diverged) *diverged = d ? 1 : 0;
    put_text(o, out, out_cap, out_len, "audit outcome");
  });
}

int det_audit_trace(det_model_t* m, const det_trace_request_t* request, const char* claimed, size_t claimed_len,
                    char* out, size_t out_cap, size_t* out_len, int32_t* diverged) {
  if (!m) {
    g_error = "model is required";
    return 1;
  }
  return guarded(m->ctx, [&] {
    if (!m->finalized) bail("model is not finalized");
    if (!request) bail("trace request is required");
    if (!claimed && claimed_len) bail("claimed trace bytes are required");
    // challenger::audit (runtime/roles/challenger.rs:55-113): the claimed
    // trace is parsed first, then the request is replayed under the claimer
    // policy (checkpoint commitment, prompt.prepare, no terminal checkpoint,
    // unbounded ranges) and must run to completion.
    if (!request->prompt_checkpoint || (request->terminal_checkpoint && *request->terminal_checkpoint) ||
        request->prefill_token_range_width || request->decode_layer_range_width)
      bail("challenger audit replays under the claimer policy: prompt_checkpoint must be set and "
           "terminal_checkpoint and the range widths unset");
    const auto c = audit_input([&] { return det_audit::parse_trace(claimed, claimed_len); });
    TraceCollector tc;
    if (trace_run(m, request, tc)) bail("challenger replay paused unexpectedly");
    bool d = false;
    const std::string o = det_audit::outcome_json(c, det_audit::entries_of(tc.committed()), &d);
    if (diverged) *diverged = d ? 1 : 0;
    put_text(o, out, out_cap, out_len, "audit outcome");
  });
}

// ------------------------------------------------------------------------
// Layer-level operators
// ------------------------------------------------------------------------
int det_scratch_create(det_model_t* m, det_scratch_t** out) {
  if (!m || !out) {
    g_error = "model and output pointer are required";
    return 1;
  }
  return guarded(m->ctx, [&] {
    if (!m->finalized) bail("model is not finalized");
    auto sc = std::make_unique<det_scratch>();
    sc->m = m;
    sc->ctx = m->ctx;
    *out = sc.release();
  });
}

void det_scratch_free(det_scratch_t* sc) {
  if (!sc) return;
  (void)hipStreamSynchronize(sc->ctx->stream);
  delete sc;
}

int det_kv_create(det_model_t* m, uint64_t layer, uint64_t max_tokens, det_kv_t** out) {
  if (!m || !out) {
    g_error = "model and output pointer are required";
    return 1;
  }
  return guarded(m->ctx, [&] {
    const GLayer& L = need_layer(m, layer);
    if (max_tokens == 0) bail("a KV cache needs room for at least one token");
    auto kv = std::make_unique<det_kv>();
    kv->m = m;
    kv->ctx = m->ctx;
    kv->layer = layer;
    GKv& c = kv->c;
    c.heads = L.num_kv_heads;
    c.hd = L.head_dim;
    c.row_w = L.num_kv_heads * L.head_dim;
    c.ring = L.cache_sliding_window.has_value();
    c.cap = c.ring ? std::max<uint64_t>(std::min<uint64_t>(*L.cache_sliding_window, max_tokens), 1) : max_tokens;
    if (c.ring && max_tokens < *L.cache_sliding_window) c.limit = max_tokens;
    HIPC(hipMalloc(&c.k, std::max<uint64_t>(c.cap * c.row_w, 1) * 4));
    HIPC(hipMalloc(&c.v, std::max<uint64_t>(c.cap * c.row_w, 1) * 4));
    *out = kv.release();
  });
}

int det_kv_clone(const det_kv_t* src, det_kv_t** out) {
  if (!src || !out) {
    g_error = "source cache and output pointer are required";
    return 1;
  }
  return guarded(src->m->ctx, [&] {
    auto kv = std::make_unique<det_kv>();
    kv->m = src->m;
    kv->ctx = src->ctx;
    kv->layer = src->layer;
    kv->c = src->c;
    kv->c.k = kv->c.v = nullptr;
    const size_t bytes = std::max<uint64_t>(src->c.cap * src->c.row_w, 1) * 4;
    HIPC(hipMalloc(&kv->c.k, bytes));
    HIPC(hipMalloc(&kv->c.v, bytes));
    hipStream_t st = src->m->ctx->stream;
    HIPC(hipMemcpyAsync(kv->c.k, src->c.k, bytes, hipMemcpyDeviceToDevice, st));
    HIPC(hipMemcpyAsync(kv->c.v, src->c.v, bytes, hipMemcpyDeviceToDevice, st));
    *out = kv.release();
  });
}

void det_kv_free(det_kv_t* kv) {
  if (!kv) return;
  (void)hipStreamSynchronize(kv->ctx->stream);
  delete kv;
}

int det_kv_info(const det_kv_t* kv, uint64_t* len, uint64_t* heads, uint64_t* head_dim, int32_t* has_det) {
  if (!kv) {
    g_error = "cache is required";
    return 1;
  }
  if (len) *len = kv->c.has ? kv->c.len : 0;
  if (heads) *heads = kv->c.heads;
  if (head_dim) *head_dim = kv->c.hd;
  if (has_det) *has_det = kv->c.has ? 1 : 0;
  return 0;
}

int det_kv_read_logical(const det_kv_t* kv, int32_t* keys, int32_t* values, uint64_t capacity) {
  if (!kv) {
    g_error = "cache is required";
    return 1;
  }
  return guarded(kv->m->ctx, [&] {
    const GKv& c = kv->c;
    if (!c.has) bail("cache holds no det data");
    if (c.len * c.row_w > capacity) bail("output buffers hold fewer values than the cache");
    const auto k = host_rows(kv->m->ctx, c, 0);
    const auto v = host_rows(kv->m->ctx, c, 1);
    HIPC(hipStreamSynchronize(kv->m->ctx->stream));
    // head-major [heads][len][head_dim], as DetKvCacheData keeps one buffer per head
    for (uint64_t h = 0; h < c.heads; ++h)
      for (uint64_t r = 0; r < c.len; ++r) {
        std::memcpy(keys + (h * c.len + r) * c.hd, k.data() + r * c.row_w + h * c.hd, c.hd * 4);
        std::memcpy(values + (h * c.len + r) * c.hd, v.data() + r * c.row_w + h * c.hd, c.hd * 4);
      }
  });
}

int det_kv_commitment(const det_kv_t* const* caches, uint64_t n, char out[65], int32_t* is_some) {
  if (!caches || !out || n == 0 || !caches[0]) {
    g_error = "at least one cache and an output buffer are required";
    return 1;
  }
  det_model* m = caches[0]->m;
  return guarded(m->ctx, [&] {
    std::vector<const GKv*> list;
    for (uint64_t i = 0; i < n; ++i) {
      if (!caches[i]) bail("null cache in commitment list");
      if (caches[i]->m != m) bail("KV cache belongs to another model");
      list.push_back(&caches[i]->c);
    }
    const bool some = commit_kv(m->ctx, list, out);
    if (!some) out[0] = 0;
    if (is_some) *is_some = some ? 1 : 0;
  });
}

int det_embed_tokens(det_model_t* m, det_scratch_t* sc, const uint32_t* ids, uint64_t n, int32_t* out_dev) {
  if (!m) {
    g_error = "model is required";
    return 1;
  }
  return guarded(m->ctx, [&] {
    if (!m->finalized) bail("model is not finalized");
    need_handles(m, sc, nullptr, nullptr);
    if (n == 0) bail("transformer layer execution requires at least one activation row");
    check_ids(m, ids, n);
    det_session* ws = scratch_rows(sc, n);
    HIPC(hipMemcpyAsync(ws->ids, ids, n * 4, hipMemcpyHostToDevice, m->ctx->stream));
    det::launch_gather_rows(*m->embedding, ws->ids, n, 0, m->hidden, m->embed_scale, out_dev, m->hidden, m->ctx->stream);
  });
}

int det_prefill_ple_inputs(det_model_t* m, det_scratch_t* sc, uint64_t layer, const uint32_t* ids, uint64_t n,
                           const int32_t* input_dev, int32_t* out_dev, int32_t* produced) {
  if (!m) {
    g_error = "model is required";
    return 1;
  }
  return guarded(m->ctx, [&] {
    const GLayer& L = need_layer(m, layer);
    need_handles(m, sc, nullptr, nullptr);
    if (produced) *produced = 0;
    if (!m->has_ple || !L.has_ple) return;
    if (n == 0) bail("transformer layer execution requires at least one activation row");
    check_ids(m, ids, n);
    det_session* ws = scratch_rows(sc, n);
    HIPC(hipMemcpyAsync(ws->ids, ids, n * 4, hipMemcpyHostToDevice, m->ctx->stream));
    ple_inputs(ws, layer, ws->ids, input_dev, n, out_dev);
    if (produced) *produced = 1;
  });
}

int det_decode_ple_input(det_model_t* m, det_scratch_t* sc, uint32_t token, const int32_t* input_dev, uint64_t layer,
                         int32_t* output_dev, int32_t* produced) {
  return det_prefill_ple_inputs(m, sc, layer, &token, 1, input_dev, output_dev, produced);
}

int det_layer_prefill(det_model_t* m, det_scratch_t* sc, uint64_t layer, const int32_t* xs_dev, uint64_t n,
                      const int32_t* per_layer_input_dev, const det_kv_t* donor, det_kv_t* cache, int32_t* out_dev) {
  if (!m) {
    g_error = "model is required";
    return 1;
  }
  return guarded(m->ctx, [&] {
    const GLayer& L = need_layer(m, layer);
    need_handles(m, sc, donor, cache);
    if (!donor && !cache) bail("transformer prefill layer needs its own cache or a donor cache");
    if (cache && cache->layer != layer) bail("KV cache belongs to another layer");
    if (n == 0) bail("transformer layer execution requires at least one activation row");
    check_rope(m, n - 1);
    det_session* ws = scratch_rows(sc, n);
    copy_d2d(m->ctx, ws->x, xs_dev, n * m->hidden * 4);
    layer_prefill(ws, L, n, donor ? nullptr : &cache->c, donor ? &donor->c : nullptr, per_layer_input_dev);
    copy_d2d(m->ctx, out_dev, ws->x, n * m->hidden * 4);
  });
}

int det_layer_decode(det_model_t* m, det_scratch_t* sc, uint64_t layer, const int32_t* input_dev,
                     const int32_t* per_layer_input_dev, det_kv_t* cache, const det_kv_t* donor, uint64_t position,
                     int32_t* output_dev) {
  if (!m) {
    g_error = "model is required";
    return 1;
  }
  return guarded(m->ctx, [&] {
    const GLayer& L = need_layer(m, layer);
    need_handles(m, sc, donor, cache);
    if (!donor && !cache) bail("transformer decode layer needs its own cache or a donor cache");
    if (cache && cache->layer != layer) bail("KV cache belongs to another layer");
    check_rope(m, position);
    det_session* ws = scratch_rows(sc, 1);
    copy_d2d(m->ctx, ws->x, input_dev, m->hidden * 4);
    layer_decode(ws, L, position, donor ? nullptr : &cache->c, donor ? &donor->c : nullptr, per_layer_input_dev);
    copy_d2d(m->ctx, output_dev, ws->x, m->hidden * 4);
  });
}

int det_hidden_to_logits(det_model_t* m, det_scratch_t* sc, const int32_t* hidden_dev, int32_t* logits_dev) {
  if (!m) {
    g_error = "model is required";
    return 1;
  }
  return guarded(m->ctx, [&] {
    if (!m->finalized) bail("model is not finalized");
    need_handles(m, sc, nullptr, nullptr);
    det_session* ws = scratch_rows(sc, 1);
    hipStream_t st = m->ctx->stream;
    det::launch_rmsnorm_to(ws->normed, hidden_dev, 1, m->hidden, m->hidden, m->final_norm, m->eps, st);
    linear(m->ctx, *m->lm_head, ws->normed, 1, logits_dev);
    if (m->softcap) det::launch_softcap(logits_dev, m->vocab, *m->softcap, st);
  });
}

}  // extern "C"
