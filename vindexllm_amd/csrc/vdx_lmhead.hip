// vdx_lmhead.hip -- Q4_0 lm_head (the reference's shaders/matvec_q4_0.comp,
// dispatched by TVdxAttention.DispatchMatVec, src/VindexLLM.Attention.pas:979-1025,
// from TVdxModel.UnembedToLogits, src/VindexLLM.Model.pas:1258-1270) for gfx950.
//
// logits[b][v] = sum_e (nibble(v,e) - 8) * d(v, e/32) * hidden[b][e] for a batch
// of up to 16 hidden rows, so the 377 MB of Gemma-3-4B lm_head weights
// (262144 x 2560 in Q4_0) stream from HBM once per step whatever the batch.
//
// Q4_0 row layout (GGUFReader.pas:264-281, matvec_q4_0.comp:7-15): blocks of
// 18 bytes, an fp16 scale d then 16 bytes qs; qs[j] & 0xF is element j and
// qs[j] >> 4 is element j + 16 of the block.
//
// Arithmetic (fixed, so the oracle restates it bit for bit): per (row, batch
// row) and per block k in order, s = 0; s = fma(q_i - 8, x[32k + i], s) for
// i = 0..31; acc = fma(d_k, s, acc).  Each product (q - 8) * x is exact
// before its single rounding, as in the shader; the shader's own summation
// order (64 strided lanes, then a tree) differs only at fp32 rounding level.
//
// Mapping: one thread per vocabulary row, one wave (64 rows) per workgroup.
// The K dimension is streamed in slices of 8 blocks (144 bytes per row): the
// wave loads its 64 rows' slice with coalesced 16-byte loads (piece P of the
// 9 KB slice tile goes to lane P mod 64), stages it in LDS (144-byte row
// stride: each lane's 16-byte reads of its own row are bank-conflict free)
// and prefetches the next slice into registers while computing.  The hidden
// values are the same for every lane, so they are read with scalar loads and
// enter the FMAs as SGPR operands; with more than one batch row they are read
// from a transposed copy (element-major, 16 batch rows per 64-byte line), so
// one scalar load feeds the 16 independent accumulation chains of an element.
// The weights are turned into f16 (q - 8) pairs (v_perm_b32 + one packed f16
// subtract per two weights) that v_fma_mix_f32 consumes directly, so a
// weight costs ~1.5 VALU ops of dequantisation plus one FMA per batch row.
#include "vdx_internal.hpp"

namespace vdx {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr int kLmPieces = 9;    // 16-byte pieces of one row per slice
static_assert(kLmPieces * 16 == 8 * 18, "a slice is 8 Q4_0 blocks");

// Two weights (q - 8) as f16 from bytes of `nib` (each 0..15): the selector
// places one nibble byte under a 0x64 byte per half (f16 1024 + q), and the
// subtraction of 1032 is exact.
__device__ __forceinline__ f16x2 q4_pair(uint32_t nib, uint32_t sel) {
  const uint32_t bits = __builtin_amdgcn_perm(0x64646464u, nib, sel);
  return __builtin_bit_cast(f16x2, bits) - (f16x2){(_Float16)1032.0f, (_Float16)1032.0f};
}

// One block (qs dwords q[0..3], fp16 scale bits `dbits`) for NB batch rows;
// x points at the block's first hidden value in the element-major layout
// x[e * NB + b] (for NB == 1 the hidden row itself).
template <int NB>
__device__ __forceinline__ void q4_block(const uint32_t (&q)[4], uint32_t dbits,
                                         const float *__restrict__ x, float (&acc)[NB]) {
  f16x2 w[16];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t lo = q[j] & 0x0F0F0F0Fu;
    const uint32_t hi = (q[j] >> 4) & 0x0F0F0F0Fu;
    w[2 * j] = q4_pair(lo, 0x04010400u);      // elements 4j, 4j+1
    w[2 * j + 1] = q4_pair(lo, 0x04030402u);  // elements 4j+2, 4j+3
    w[8 + 2 * j] = q4_pair(hi, 0x04010400u);  // elements 16+4j, 16+4j+1
    w[9 + 2 * j] = q4_pair(hi, 0x04030402u);  // elements 16+4j+2, 16+4j+3
  }
  const float d = (float)__builtin_bit_cast(_Float16, (uint16_t)(dbits & 0xFFFFu));
  float s[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) s[b] = 0.0f;
#pragma unroll
  for (int e = 0; e < 32; ++e)
#pragma unroll
    for (int b = 0; b < NB; ++b) s[b] = __builtin_fmaf((float)w[e >> 1][e & 1], x[e * NB + b], s[b]);
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = __builtin_fmaf(d, s[b], acc[b]);
}

// One slice (8 blocks = 4 block pairs of 9 dwords) of a row.
template <int NB>
__device__ __forceinline__ void q4_slice(const uint32_t (&r)[4 * kLmPieces], const float *__restrict__ x,
                                         float (&acc)[NB]) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t *pr = r + 9 * m;
    // even block: scale in bytes 0-1, qs in bytes 2-17 (straddling dwords)
    const uint32_t qa[4] = {__builtin_amdgcn_alignbyte(pr[1], pr[0], 2),
                            __builtin_amdgcn_alignbyte(pr[2], pr[1], 2),
                            __builtin_amdgcn_alignbyte(pr[3], pr[2], 2),
                            __builtin_amdgcn_alignbyte(pr[4], pr[3], 2)};
    q4_block<NB>(qa, pr[0], x + 64 * m * NB, acc);
    // odd block: scale in bytes 18-19, qs in bytes 20-35 (dword aligned)
    const uint32_t qb[4] = {pr[5], pr[6], pr[7], pr[8]};
    q4_block<NB>(qb, pr[4] >> 16, x + (64 * m + 32) * NB, acc);
  }
}

// x: hidden row (NB == 1) or the element-major copy [in_dim][NB].
template <int NB>
__global__ __launch_bounds__(64) void k_lmhead_q4_0(const uint8_t *__restrict__ wq,
                                                    const float *__restrict__ x,
                                                    float *__restrict__ logits, int64_t ls,
                                                    int32_t in_dim, int32_t vocab, int32_t B) {
  __shared__ u32x4 tile[64 * kLmPieces];
  const int t = threadIdx.x;
  const int v0 = blockIdx.x * 64;
  const int nrows = min(64, vocab - v0);
  const int rowbytes = (in_dim >> 5) * 18;
  const int nslices = in_dim >> 8;
  const uint8_t *wt = wq + (int64_t)v0 * rowbytes;

  // piece P = t + 64 i of a slice tile is piece j = P % 9 of row P / 9; rows
  // past the vocabulary read the tile's first row (their results are not
  // stored)
  int goff[kLmPieces];
#pragma unroll
  for (int i = 0; i < kLmPieces; ++i) {
    const int P = t + 64 * i;
    const int r = P / kLmPieces, j = P - r * kLmPieces;
    goff[i] = (r < nrows) ? r * rowbytes + 16 * j : 0;
  }
  u32x4 pre[kLmPieces];
  auto load_slice = [&](int s) {
#pragma unroll
    for (int i = 0; i < kLmPieces; ++i)
      pre[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wt + goff[i] + 144 * s));
  };
  load_slice(0);

  float acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
  for (int s = 0; s < nslices; ++s) {
    __syncthreads();  // the previous slice has been read (one wave: no-op ordering)
#pragma unroll
    for (int i = 0; i < kLmPieces; ++i) tile[t + 64 * i] = pre[i];
    __syncthreads();
    if (s + 1 < nslices) load_slice(s + 1);
    uint32_t r[4 * kLmPieces];
#pragma unroll
    for (int j = 0; j < kLmPieces; ++j) {
      const u32x4 v = tile[t * kLmPieces + j];
      r[4 * j] = v[0];
      r[4 * j + 1] = v[1];
      r[4 * j + 2] = v[2];
      r[4 * j + 3] = v[3];
    }
    q4_slice<NB>(r, x + 256 * NB * s, acc);
  }
  if (t < nrows) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
      if (b < B) logits[(int64_t)b * ls + v0 + t] = acc[b];
  }
}

// Element-major copy of up to 16 hidden rows: xt[e * NB + b] = hidden[b][e]
// (rows b >= B are zero).
__global__ __launch_bounds__(256) void k_lmhead_xt(const float *__restrict__ hidden, int64_t hs,
                                                   int32_t in_dim, int32_t B, int32_t NB,
                                                   float *__restrict__ xt) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= in_dim * NB) return;
  const int e = i / NB, b = i - e * NB;
  xt[i] = (b < B) ? hidden[(int64_t)b * hs + e] : 0.0f;
}

hipError_t launch_lmhead_q4_0(const LmHeadParams &p, hipStream_t st) {
  const dim3 grid((unsigned)((p.vocab + 63) / 64));
  for (int b0 = 0; b0 < p.rows; b0 += 16) {
    const int B = min(16, p.rows - b0);
    const float *x = p.hidden + (int64_t)b0 * p.hidden_stride;
    float *l = p.logits + (int64_t)b0 * p.logit_stride;
    const int NB = (B == 1) ? 1 : (B == 2) ? 2 : (B <= 4) ? 4 : (B <= 8) ? 8 : 16;
    if (NB > 1) {
      hipLaunchKernelGGL(k_lmhead_xt, dim3((unsigned)((p.in_dim * NB + 255) / 256)), dim3(256), 0,
                         st, x, p.hidden_stride, p.in_dim, B, NB, p.scratch);
      x = p.scratch;
    }
#define VDX_LM(N)                                                                           \
  hipLaunchKernelGGL(k_lmhead_q4_0<N>, grid, dim3(64), 0, st, p.weights, x, l, p.logit_stride, \
                     p.in_dim, p.vocab, B)
    if (NB == 1)
      VDX_LM(1);
    else if (NB == 2)
      VDX_LM(2);
    else if (NB == 4)
      VDX_LM(4);
    else if (NB == 8)
      VDX_LM(8);
    else
      VDX_LM(16);
#undef VDX_LM
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace vdx
