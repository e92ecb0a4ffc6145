// vdx_internal.hpp -- host-side launch entry points shared by the C ABI
// (vdx_api.hip) and the kernels (vdx_kernels.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vdx_device.hpp"

namespace vdx {

// Parameters of one sampling call, resolved by the host.
struct CallParams {
  float *logits;
  int64_t stride;
  int32_t rows;
  int32_t vocab;
  int32_t nchunks;
  bool vec;             // 16-byte aligned rows: float4 loads
  float inv_t;          // fl32(1 / T)
  int32_t top_k;
  float top_p;
  float min_p;
  float penalty;
  const int32_t *hist;  // [max_rows * hist_len]
  int32_t hist_len;
  int32_t fuse_penalty; // the top-K kernel applies the penalty itself
  KernelRng rng;
  KernelOut out;
  // workspace
  ChunkMeta *meta;
  Cand *cand;
  FullMeta *fmeta;
  uint64_t *gpart;
  uint32_t *tickets;
};

// Q4_0 lm_head: logits[r*logit_stride + v] for rows r < rows, v < vocab.
struct LmHeadParams {
  const uint8_t *weights;  // vocab x (in_dim/32) blocks of 18 bytes, 16-byte aligned
  const float *hidden;     // rows x in_dim (row r at hidden + r*hidden_stride)
  int64_t hidden_stride;
  float *logits;
  int64_t logit_stride;
  int32_t rows;
  int32_t in_dim;          // multiple of 256
  int32_t vocab;
  float *scratch;          // >= 16 * in_dim floats when rows > 1 (element-major hidden copy)
};

hipError_t launch_lmhead_q4_0(const LmHeadParams &p, hipStream_t st);
hipError_t launch_penalty(const CallParams &p, hipStream_t st);
hipError_t launch_greedy(const CallParams &p, hipStream_t st);
hipError_t launch_topk(const CallParams &p, hipStream_t st);
hipError_t launch_full(const CallParams &p, hipStream_t st);
hipError_t launch_hist_add(const int32_t *tokens, int32_t tok_const, int32_t row0,
                           int32_t rows, int32_t *hist, int32_t hist_len,
                           RowState *rs, hipStream_t st);
hipError_t launch_row_reset(RowState *rs, int32_t row0, int32_t rows, bool clear_hist,
                            bool reseed, uint64_t seed_base, hipStream_t st);

}  // namespace vdx
