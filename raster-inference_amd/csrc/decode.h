// Fused batch-1 decode step (graph-captured) kernels for the det path.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.h"

namespace det {

// Per-step values the captured decode graph reads from device memory.
struct StepState {
  uint64_t position;  // index of the token being decoded (number of tokens before it)
  uint32_t token;
  uint32_t pad;
};

struct QkvPostArgs {
  const int32_t* qkv;  // fused projection output: [q heads | k heads | v heads (if has_v)]
  int32_t* qbuf;       // normalised + rotated queries [nh][hd]
  int32_t* kc;         // layer KV cache rows [cap][nkv*hd]
  int32_t* vc;
  const int32_t* q_norm;
  const int32_t* k_norm;
  const int64_t* inv_freq;
  const StepState* st;
  int64_t eps;
  uint64_t cap, rotary;
  uint32_t nh, nkv, hd;
  int ring, has_v;
};

struct AttnDecArgs {
  const int32_t* q;  // [nh][hd]
  const int32_t* k;  // attention cache (own or donor) [cap][nkv*hd]
  const int32_t* v;
  const StepState* st;
  uint64_t cap, window;
  uint64_t max_rows;  // row stride of the scores / weights scratch (>= cap)
  int ring;
  uint32_t hd, nh, nkv;
  int32_t* scores;   // scratch [nh][max_rows]
  int32_t* weights;  // scratch [nh][max_rows]
  int64_t* acc;      // [nh][hd] wrapped weighted sums (requantized by the O projection)
};

// Limits of the fused decode kernels.
constexpr uint32_t kDecMaxHeadDim = 512;
constexpr uint32_t kDecMaxGroup = 8;
constexpr uint64_t kDecMaxHidden = 15360;  // one LDS row of int32 per single-workgroup row kernel

void launch_dec_embed(const DevMatrix& E, const StepState* st, int32_t scale, uint64_t H, int32_t* x, int32_t* dec_in,
                      const int32_t* w_in, int64_t eps, int32_t* normed, hipStream_t s);
void launch_dec_mid(const int32_t* o, int32_t* x, int32_t* normed, const int32_t* w_post, const int32_t* w_pre,
                    uint64_t H, int64_t eps, hipStream_t s);
void launch_dec_end(const int32_t* ff, int32_t* x, int32_t* normed, const int32_t* w_post, bool has_scalar,
                    int32_t scalar, const int32_t* w_next, uint64_t H, int64_t eps, hipStream_t s);
void launch_dec_qkv_post(const QkvPostArgs& a, bool own_cache, hipStream_t s);
void launch_dec_attention(const AttnDecArgs& a, hipStream_t s);
void launch_dec_set_step(StepState* st, uint64_t position, uint32_t token, hipStream_t s);
void launch_dec_softcap(int32_t* x, uint64_t n, int32_t cap, hipStream_t s);

}  // namespace det
