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
  const int32_t *hist;  // [max_rows * hist_len]: row r's ring at hist + r * hist_len
  int32_t hist_len;     // ring stride (>= every row's window)
  int32_t fuse_penalty; // the top-K kernel applies the penalty itself
  int32_t exact_kernel; // rows with Top-P >= 1 are finished by k_topk_exact (K <= kKMax)
  const RowCfg *rcfg;   // per-row parameters (nullptr: the fields above for every row)
  KernelRng rng;
  KernelOut out;
  // workspace
  ChunkMeta *meta;
  Cand *cand;
  int32_t cand_cap;     // candidate slots per chunk: kCandCap, or more when some row has K > 64
  uint8_t *huge_ws;     // rows with K > kKBig: per-row slots and sort space
  int64_t huge_row_bytes;
  FullMeta *fmeta;
  uint64_t *gpart;
  uint32_t *tickets;
};

// lm_head weight formats (GGML tensor type ids, GGUFReader.pas:34-42).
constexpr int kLmF16 = 1, kLmQ4_0 = 2, kLmQ8_0 = 8;

// lm_head: logits[r*logit_stride + v] for rows r < rows, v < vocab.
struct LmHeadParams {
  const uint8_t *weights;  // vocab rows in `format`, 16-byte aligned
  const float *hidden;     // rows x in_dim (row r at hidden + r*hidden_stride)
  int64_t hidden_stride;
  float *logits;
  int64_t logit_stride;
  int32_t rows;
  int32_t in_dim;          // multiple of 256
  int32_t vocab;
  float *scratch;          // >= 16 * in_dim floats when rows > 1 or norm_weight (prepared hidden copy)
  int32_t format;          // kLmQ4_0, kLmQ8_0 or kLmF16
  const float *norm_weight;  // output RMSNorm weight [in_dim] (nullable: no norm)
  float norm_eps;
  int32_t packed;          // weights in the packed layout of launch_lmhead_pack
};

hipError_t launch_lmhead(const LmHeadParams &p, hipStream_t st);
// The lm_head weights repacked for coalesced, line-aligned loads (see
// k_lmhead_pack): lmhead_packed_bytes() bytes at `packed`.
int64_t lmhead_packed_bytes(int format, int in_dim, int vocab);
hipError_t launch_lmhead_pack(const uint8_t *w, int format, int in_dim, int vocab, uint8_t *packed,
                              hipStream_t st);
hipError_t launch_penalty(const CallParams &p, hipStream_t st);
hipError_t launch_greedy(const CallParams &p, hipStream_t st);
hipError_t launch_topk(const CallParams &p, hipStream_t st);
hipError_t launch_full(const CallParams &p, hipStream_t st);
// Rows with K > kKBig (one workgroup per row) and the workspace each needs.
hipError_t launch_topk_huge(const CallParams &p, hipStream_t st);
int64_t topk_huge_row_bytes(int K);
hipError_t launch_hist_gather(const int32_t *hist_row, int32_t slots, const RowState *rs_row, const float *L,
                              int32_t vocab, uint64_t *out, hipStream_t st);
hipError_t launch_hist_add(const int32_t *tokens, int32_t tok_const, int32_t row0,
                           int32_t rows, int32_t *hist, int32_t hist_len,
                           RowState *rs, hipStream_t st);
// Reseeding: xoshiro from seed (+ row when add_row); Philox keyed by pkey,
// counting on prow (< 0: the row itself).
hipError_t launch_row_reset(RowState *rs, int32_t row0, int32_t rows, bool clear_hist, int32_t window,
                            bool reseed, uint64_t seed, bool add_row, hipStream_t st, uint64_t pkey = 0,
                            int32_t prow = -1);
// RowState and tickets of rows [0, rows) for a call without a sampler object:
// history counts from `count` (nullable: empty rings), tickets cleared.
hipError_t launch_rows_prepare(RowState *rs, uint32_t *tickets, int32_t rows, const int32_t *count,
                               int32_t window, hipStream_t st);

}  // namespace vdx
