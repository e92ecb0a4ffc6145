// vdx_lmhead.hip -- the lm_head of TVdxModel.UnembedToLogits
// (src/VindexLLM.Model.pas:1258-1270) for gfx950: the output RMSNorm
// (shaders/rmsnorm_copy.comp via TVdxLayerNorm.ApplyCopy,
// src/VindexLLM.LayerNorm.pas:395-417) followed by the matrix-vector product in
// the embedding tensor's own GGUF format, as TVdxAttention.DispatchMatVec
// selects it (src/VindexLLM.Attention.pas:979-1025): shaders/matvec_q4_0.comp,
// matvec_q8_0.comp or matvec_f16.comp.
//
// logits[b][v] = sum_e W(v, e) * xn[b][e] for a batch of up to 16 hidden rows,
// so the lm_head weights (377 MB for Gemma-3-4B's 262144 x 2560 in Q4_0) stream
// from HBM once per step whatever the batch.
//
// Row layouts (GGUFReader.pas:264-281 and the shaders' headers):
//   Q4_0: blocks of 18 bytes, fp16 scale d then 16 bytes qs; qs[j] & 0xF is
//         element j and qs[j] >> 4 element j + 16 of the block; W = (q - 8) d.
//   Q8_0: blocks of 34 bytes, fp16 scale d then 32 int8 q; W = q d.
//   F16:  in_dim fp16 values.
//
// Arithmetic (fixed, so the oracle restates it bit for bit): per (row, batch
// row) and per block k of 32 elements in order, s = 0; s = fma(w_i, x[32k + i],
// s) for i = 0..31 with w_i = q_i - 8 (Q4_0), q_i (Q8_0) or the fp16 value
// (F16), each product exact before its single rounding; then acc = fma(d_k, s,
// acc) (d_k = 1 for F16).  For Q4_0 the chain runs on t = 16 s, with weights
// 16 (q_i - 8), and acc = fma(d_k / 16, t, acc): scaling by a power of two
// commutes with every rounding, so this is the same sum bit for bit wherever
// no partial sum is subnormal (or above 2^124); the oracle restates the
// scaled form, so it agrees everywhere.  The shaders' own summation orders
// (256 or 64 strided lanes, then a tree) differ only at fp32 rounding level.
//
// Output RMSNorm (optional, before the product), in the shader's order:
// thread t of 256 sums h[e]^2 for e = t, t + 256, ... (product then sum),
// the 256 partials reduce as a tree (stride 128, 64, ..., 1), inv_rms =
// 1 / sqrt(ss / dim + eps) with IEEE division and square root, and
// xn[e] = (h[e] * inv_rms) * w[e].
//
// Mapping: one thread per vocabulary row, one wave (64 rows) per workgroup.
// The K dimension is streamed in slices (Q4_0: 8 blocks, 144 bytes per row;
// Q8_0: 4 blocks, 136 bytes; F16: 64 values, 128 bytes): the wave loads its
// 64 rows' slice with coalesced loads (piece P of the slice tile goes to lane
// P mod 64), stages it in LDS (each lane then reads its own row) and
// prefetches the next slice into registers while computing.  The hidden
// values are the same for every lane, so they are read with scalar loads and
// enter the FMAs as SGPR operands; with more than one batch row (or the norm)
// they are read from a prepared copy, element-major with 16 batch rows per
// 64-byte line, so one scalar load feeds the independent accumulation chains
// of an element.  Quantised weights become f16 pairs exactly, which
// v_fma_mix_f32 consumes directly: a Q4_0 nibble pair is one v_and_or_b32
// (the nibbles of bytes 0 and 2 of a dword, or of bytes 1 and 3 after one
// shift, under a 0x64 byte: f16 1024 + q, or 1024 + 16 q for the high
// nibbles, left in place) and one packed f16 fma or subtract to 16 (q - 8); a
// Q8_0 byte pair is one v_perm_b32 (each byte under a 0x64 byte) and one
// packed subtract.
#include "vdx_internal.hpp"

namespace vdx {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// Per-format slice geometry: a slice holds NBLK blocks of 32 elements of a
// row, moved as PIECES loads of PIECE_DW dwords.
template <int FMT> struct LmFmt;
template <> struct LmFmt<kLmQ4_0> {
  static constexpr int kBlockBytes = 18, kNBlk = 8, kPieceDw = 4, kPieces = 9;
};
template <> struct LmFmt<kLmQ8_0> {
  static constexpr int kBlockBytes = 34, kNBlk = 4, kPieceDw = 2, kPieces = 17;
};
template <> struct LmFmt<kLmF16> {
  static constexpr int kBlockBytes = 64, kNBlk = 2, kPieceDw = 4, kPieces = 8;
};
template <int FMT> constexpr int slice_dw() { return LmFmt<FMT>::kPieces * LmFmt<FMT>::kPieceDw; }
static_assert(9 * 16 == 8 * 18 && 17 * 8 == 4 * 34 && 8 * 16 == 2 * 64, "slices are whole blocks");

// Two (byte + 128) values of `u` as f16 1024 + (byte + 128) (the selector
// puts one byte of u under a 0x64 byte per half), minus `off`: exact.
template <int OFF>
__device__ __forceinline__ f16x2 byte_pair(uint32_t u, uint32_t sel) {
  const uint32_t bits = __builtin_amdgcn_perm(0x64646464u, u, sel);
  return __builtin_bit_cast(f16x2, bits) - (f16x2){(_Float16)OFF, (_Float16)OFF};
}

// One block of 32 weights (as 16 f16 pairs) for NB batch rows; x points at
// the block's first hidden value in the element-major layout x[e * NB + b]
// (for NB == 1 the hidden row itself).
template <int NB>
__device__ __forceinline__ void block_fma(const f16x2 (&w)[16], float d, const float *__restrict__ x,
                                          float (&acc)[NB]) {
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

__device__ __forceinline__ float half_bits(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xFFFFu));
}

// The Q4_0 nibble masks and the f16 exponent byte pair, in VGPRs: gfx950's
// VOP3 encoding takes no literal, and with all three in registers each
// (u & mask) | 0x64006400 is one v_and_or_b32 (with literals the compiler
// emits an AND and an OR).
struct Q4K {
  uint32_t lo, hi, c;
};
__device__ __forceinline__ Q4K q4_consts() {
  Q4K k;
  asm("v_mov_b32 %0, 0x000F000F" : "=v"(k.lo));
  asm("v_mov_b32 %0, 0x00F000F0" : "=v"(k.hi));
  asm("v_mov_b32 %0, 0x64006400" : "=v"(k.c));
  return k;
}

// Q4_0 block: qs dwords q[0..3] (byte b of dword j is qs[4j + b]: low nibble
// element 4j + b, high nibble element 16 + 4j + b), scale bits dbits.  Every
// weight enters as 16 (q - 8): a low-nibble pair as 16 (1024 + q) - 16512 (one
// packed f16 fma), a high-nibble pair, left in place, as 1024 + 16 q - 1152
// (one packed f16 subtract), all exact; so the chain runs on t = 16 s and the
// scale enters as d / 16 (exact for an fp16 d).
template <int NB>
__device__ __forceinline__ void q4_block(const uint32_t (&q)[4], uint32_t dbits, const float *__restrict__ x,
                                         float (&acc)[NB], const Q4K &K) {
  const f16x2 m16 = {(_Float16)16, (_Float16)16}, o16 = {(_Float16)-16512, (_Float16)-16512};
  const f16x2 o8 = {(_Float16)1152, (_Float16)1152};
  // w[2j], w[2j + 1]: bytes 0 and 2, 1 and 3 (after the shift) of dword j;
  // low nibbles in w[0..7], high nibbles in w[8..15]
  f16x2 w[16];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t u = q[j], u8 = q[j] >> 8;
    w[2 * j] = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, (u & K.lo) | K.c), m16, o16);
    w[2 * j + 1] = __builtin_elementwise_fma(__builtin_bit_cast(f16x2, (u8 & K.lo) | K.c), m16, o16);
    w[8 + 2 * j] = __builtin_bit_cast(f16x2, (u & K.hi) | K.c) - o8;
    w[9 + 2 * j] = __builtin_bit_cast(f16x2, (u8 & K.hi) | K.c) - o8;
  }
  float t[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) t[b] = 0.0f;
#pragma unroll
  for (int e = 0; e < 32; ++e) {  // element e = 16 h + 4 j + k: pair 8 h + 2 j + (k & 1), half k >> 1
    const float we = (float)w[8 * (e >> 4) + 2 * ((e >> 2) & 3) + (e & 1)][(e >> 1) & 1];
#pragma unroll
    for (int b = 0; b < NB; ++b) t[b] = __builtin_fmaf(we, x[e * NB + b], t[b]);
  }
  const float d16 = half_bits(dbits) * 0.0625f;
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = __builtin_fmaf(d16, t[b], acc[b]);
}

// Q8_0 block: qs dwords q[0..7] (four int8 each), scale bits dbits.
template <int NB>
__device__ __forceinline__ void q8_block(const uint32_t (&q)[8], uint32_t dbits, const float *__restrict__ x,
                                         float (&acc)[NB]) {
  f16x2 w[16];
#pragma unroll
  for (int j = 0; j < 8; ++j) {  // offset 1024 + 128
    const uint32_t u = q[j] ^ 0x80808080u;  // signed byte + 128
    w[2 * j] = byte_pair<1152>(u, 0x04010400u);
    w[2 * j + 1] = byte_pair<1152>(u, 0x04030402u);
  }
  block_fma<NB>(w, half_bits(dbits), x, acc);
}

// One slice of a row (dwords r[]), element-major hidden values x.
template <int FMT, int NB>
__device__ __forceinline__ void lm_slice(const uint32_t (&r)[slice_dw<FMT>()], const float *__restrict__ x,
                                         float (&acc)[NB], const Q4K &K) {
  if constexpr (FMT == kLmQ4_0) {
    // 4 block pairs of 9 dwords: the even block's scale in bytes 0-1 and qs in
    // bytes 2-17 (straddling dwords), the odd block's scale in bytes 18-19 and
    // qs in bytes 20-35 (dword aligned)
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const uint32_t *pr = r + 9 * m;
      const uint32_t qa[4] = {__builtin_amdgcn_alignbyte(pr[1], pr[0], 2),
                              __builtin_amdgcn_alignbyte(pr[2], pr[1], 2),
                              __builtin_amdgcn_alignbyte(pr[3], pr[2], 2),
                              __builtin_amdgcn_alignbyte(pr[4], pr[3], 2)};
      q4_block<NB>(qa, pr[0], x + 64 * m * NB, acc, K);
      const uint32_t qb[4] = {pr[5], pr[6], pr[7], pr[8]};
      q4_block<NB>(qb, pr[4] >> 16, x + (64 * m + 32) * NB, acc, K);
    }
  } else if constexpr (FMT == kLmQ8_0) {
    // 2 block pairs of 17 dwords: the even block's scale in bytes 0-1 and qs
    // in bytes 2-33, the odd block's scale in bytes 34-35 and qs in 36-67
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const uint32_t *pr = r + 17 * m;
      uint32_t qa[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) qa[k] = __builtin_amdgcn_alignbyte(pr[k + 1], pr[k], 2);
      q8_block<NB>(qa, pr[0], x + 64 * m * NB, acc);
      uint32_t qb[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) qb[k] = pr[9 + k];
      q8_block<NB>(qb, pr[8] >> 16, x + (64 * m + 32) * NB, acc);
    }
  } else {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      f16x2 w[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) w[k] = __builtin_bit_cast(f16x2, r[16 * m + k]);
      block_fma<NB>(w, 1.0f, x + 32 * m * NB, acc);
    }
  }
}

// One block of a row's tail (the blocks after its last whole slice, when
// in_dim is not a multiple of the slice length), read from a 2-byte aligned
// address (F16 blocks: 4-byte aligned); x points at the block's first hidden
// value.  The arithmetic is the slices' (block_fma), so the block order of
// the sum is unchanged.
template <int FMT, int NB>
__device__ __forceinline__ void lm_tail_block(const uint8_t *__restrict__ p, const float *__restrict__ x,
                                              float (&acc)[NB], const Q4K &K) {
  if constexpr (FMT == kLmQ4_0) {
    const uint16_t *h = reinterpret_cast<const uint16_t *>(p);
    uint32_t q[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) q[j] = (uint32_t)h[1 + 2 * j] | ((uint32_t)h[2 + 2 * j] << 16);
    q4_block<NB>(q, (uint32_t)h[0], x, acc, K);
  } else if constexpr (FMT == kLmQ8_0) {
    const uint16_t *h = reinterpret_cast<const uint16_t *>(p);
    uint32_t q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = (uint32_t)h[1 + 2 * j] | ((uint32_t)h[2 + 2 * j] << 16);
    q8_block<NB>(q, (uint32_t)h[0], x, acc);
  } else {
    const uint32_t *d = reinterpret_cast<const uint32_t *>(p);
    f16x2 w[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) w[k] = __builtin_bit_cast(f16x2, d[k]);
    block_fma<NB>(w, 1.0f, x, acc);
  }
}

template <int FMT> struct PieceT;
template <> struct PieceT<kLmQ4_0> { typedef u32x4 T; };
template <> struct PieceT<kLmQ8_0> { typedef u32x2 T; };
template <> struct PieceT<kLmF16> { typedef u32x4 T; };

// x: hidden row (NB == 1, no norm) or the prepared copy [in_dim][NB].
template <int FMT, int NB, bool PACKED>
__global__ __launch_bounds__(64) void k_lmhead(const uint8_t *__restrict__ wq, const float *__restrict__ x,
                                               float *__restrict__ logits, int64_t ls, int32_t in_dim,
                                               int32_t vocab, int32_t B) {
  typedef LmFmt<FMT> F;
  typedef typename PieceT<FMT>::T Piece;
  constexpr int P = F::kPieces, PD = F::kPieceDw, PB = 4 * PD;  // pieces, dwords and bytes per piece
  constexpr int SE = 32 * F::kNBlk;                              // elements per slice
  const int t = threadIdx.x;
  const int v0 = blockIdx.x * 64;
  const int nrows = min(64, vocab - v0);
  // unsigned arithmetic: in_dim > 0 (the signed forms cost registers here)
  const int rowbytes = (int)(((uint32_t)in_dim >> 5) * (uint32_t)F::kBlockBytes);
  // Whole slices, then the tail blocks.  In the GGUF layout a Q4_0 / Q8_0
  // row whose length is not a whole number of slices does not start on a
  // piece boundary, so there every block takes the tail path (2-byte loads).
  const int nslices = (PACKED || FMT == kLmF16 || (uint32_t)in_dim % (uint32_t)SE == 0u)
                          ? (int)((uint32_t)in_dim / (uint32_t)SE)
                          : 0;
  const int nmain = nslices * F::kNBlk;                    // blocks in whole slices
  const int ntail = (int)((uint32_t)in_dim >> 5) - nmain;  // blocks after them
  float acc[NB];
#pragma unroll
  for (int b = 0; b < NB; ++b) acc[b] = 0.0f;
  Q4K K{};
  if constexpr (FMT == kLmQ4_0) K = q4_consts();

  if constexpr (PACKED) {
    // packed layout (k_lmhead_pack): piece k of slice s of the wave's row t
    // at ((s * P + k) * 64 + t) * PB from the wave's base, so each load
    // instruction reads 64 consecutive pieces and every cache line is fetched
    // once; the lane receives its own row's slice, with no transpose
    // the group's 64 rows: whole slices as above, then each row's tail blocks
    // row after row
    const uint8_t *wg = wq + (int64_t)blockIdx.x * 64 * rowbytes;
    const uint8_t *wp = wg + t * PB;
    Piece ca[P], cb[P];
    auto load = [&](Piece (&dst)[P], int sl) {
#pragma unroll
      for (int k = 0; k < P; ++k)
        dst[k] = __builtin_nontemporal_load(reinterpret_cast<const Piece *>(wp + (sl * P + k) * (64 * PB)));
    };
    auto compute = [&](const Piece (&src)[P], int sl) {
      uint32_t r[P * PD];
#pragma unroll
      for (int j = 0; j < P; ++j)
#pragma unroll
        for (int k = 0; k < PD; ++k) r[PD * j + k] = src[j][k];
      lm_slice<FMT, NB>(r, x + SE * NB * sl, acc, K);
    };
    if (nslices > 0) load(ca, 0);  // (a row shorter than one slice is all tail)
    for (int s = 0; s < nslices; s += 2) {
      if (s + 1 < nslices) load(cb, s + 1);
      compute(ca, s);
      if (s + 1 < nslices) {
        if (s + 2 < nslices) load(ca, s + 2);
        compute(cb, s + 1);
      }
    }
    if (ntail > 0) {  // fewer than kNBlk blocks: uniform branches, no loop-carried state
      const uint8_t *tp = wg + (int64_t)nslices * (P * 64 * PB) + t * (ntail * F::kBlockBytes);
#pragma unroll
      for (int j = 0; j < F::kNBlk - 1; ++j)
        if (j < ntail) lm_tail_block<FMT, NB>(tp + j * F::kBlockBytes, x + 32 * NB * (nmain + j), acc, K);
    }
    if (t < nrows) {
#pragma unroll
      for (int b = 0; b < NB; ++b)
        if (b < B) logits[(int64_t)b * ls + v0 + t] = acc[b];
    }
    return;
  }

  __shared__ Piece tile[64 * P];
  const uint8_t *wt = wq + (int64_t)v0 * rowbytes;

  // piece Q = t + 64 i of a slice tile is piece j = Q % P of row Q / P; rows
  // past the vocabulary read the tile's first row (their results are not
  // stored)
  int goff[P];
#pragma unroll
  for (int i = 0; i < P; ++i) {
    const int Q = t + 64 * i;
    const int r = Q / P, j = Q - r * P;
    goff[i] = (r < nrows) ? r * rowbytes + PB * j : 0;
  }
  Piece pre[P];
  auto load_slice = [&](int s) {
#pragma unroll
    for (int i = 0; i < P; ++i)
      pre[i] = __builtin_nontemporal_load(reinterpret_cast<const Piece *>(wt + goff[i] + P * PB * s));
  };
  if (nslices > 0) load_slice(0);  // (no whole slice: every block is a tail block)

  for (int s = 0; s < nslices; ++s) {
    __syncthreads();  // the previous slice has been read (one wave: no-op ordering)
#pragma unroll
    for (int i = 0; i < P; ++i) tile[t + 64 * i] = pre[i];
    __syncthreads();
    if (s + 1 < nslices) load_slice(s + 1);
    uint32_t r[P * PD];
#pragma unroll
    for (int j = 0; j < P; ++j) {
      const Piece v = tile[t * P + j];
#pragma unroll
      for (int k = 0; k < PD; ++k) r[PD * j + k] = v[k];
    }
    lm_slice<FMT, NB>(r, x + SE * NB * s, acc, K);
  }
  if (ntail > 0 && t < nrows) {  // rows past the vocabulary read nothing here
    const uint8_t *tp = wt + (int64_t)t * rowbytes + nmain * F::kBlockBytes;
    for (int j = 0; j < ntail; ++j)
      lm_tail_block<FMT, NB>(tp + j * F::kBlockBytes, x + 32 * NB * (nmain + j), acc, K);
  }
  if (t < nrows) {
#pragma unroll
    for (int b = 0; b < NB; ++b)
      if (b < B) logits[(int64_t)b * ls + v0 + t] = acc[b];
  }
}

// The prepared hidden copy: xt[e * NB + b] = hidden[b][e], or with the norm
// weight w the output RMSNorm of that row; rows b >= B are zero.  One
// workgroup per b < NB.
__global__ __launch_bounds__(256) void k_lmhead_prep(const float *__restrict__ hidden, int64_t hs,
                                                     const float *__restrict__ w, float eps, int32_t in_dim,
                                                     int32_t B, int32_t NB, float *__restrict__ xt) {
  __shared__ float part[256];
  const int b = blockIdx.x, t = threadIdx.x;
  if (b >= B) {
    for (int e = t; e < in_dim; e += 256) xt[(int64_t)e * NB + b] = 0.0f;
    return;
  }
  const float *h = hidden + (int64_t)b * hs;
  if (!w) {
    for (int e = t; e < in_dim; e += 256) xt[(int64_t)e * NB + b] = h[e];
    return;
  }
  float ss = 0.0f;
  for (int e = t; e < in_dim; e += 256) {
    const float v = h[e];
    ss = ss + v * v;  // product, then sum (-ffp-contract=off: no fused multiply-add)
  }
  part[t] = ss;
  __syncthreads();
  for (int stride = 128; stride > 0; stride >>= 1) {
    if (t < stride) part[t] = part[t] + part[t + stride];
    __syncthreads();
  }
  // fl32(sqrt(q)) and fl32(1 / s) through double operations: both double
  // roundings are innocuous (53 >= 2 * 24 + 2 bits), so these are the
  // correctly rounded fp32 square root and reciprocal
  const float q = part[0] / (float)in_dim + eps;
  const float sq = (float)__builtin_sqrt((double)q);
  const float inv_rms = (float)(1.0 / (double)sq);
  for (int e = t; e < in_dim; e += 256) xt[(int64_t)e * NB + b] = (h[e] * inv_rms) * w[e];
}

// The packed layout of a weight tensor (vocab rows of in_dim elements in
// format FMT): for each group of 64 rows (the last padded with zero rows),
// each whole slice s and each piece k, the 64 rows' pieces in row order; then
// the rows' tail blocks (in_dim not a multiple of the slice length), row
// after row.  One thread per destination piece; rows past the vocabulary are
// zero.
template <int FMT>
__global__ __launch_bounds__(256) void k_lmhead_pack(const uint8_t *__restrict__ wq, uint8_t *__restrict__ out,
                                                      int32_t in_dim, int32_t vocab, int64_t npieces) {
  typedef LmFmt<FMT> F;
  typedef typename PieceT<FMT>::T Piece;
  constexpr int P = F::kPieces, PB = 4 * F::kPieceDw, SE = 32 * F::kNBlk, BB = F::kBlockBytes;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= npieces) return;
  const int64_t nslices = in_dim / SE;
  const int64_t nblocks = in_dim / 32, ntail = nblocks - nslices * F::kNBlk;
  const int64_t rowbytes = nblocks * BB;
  const int64_t per_group = 64 * rowbytes / PB;  // pieces per group of 64 rows
  const int64_t w = i / per_group, ig = i - w * per_group;
  const int64_t nmainp = nslices * P * 64;
  if (ig < nmainp) {
    const int t = (int)(ig & 63);
    const int64_t q = ig >> 6;  // s * P + k
    const int k = (int)(q % P);
    const int64_t s = q / P;
    const int64_t row = w * 64 + t;
    Piece v;
    if (row < vocab)
      v = *reinterpret_cast<const Piece *>(wq + row * rowbytes + (s * P + k) * PB);
    else
      v = Piece{};
    *reinterpret_cast<Piece *>(out + i * PB) = v;
    return;
  }
  // tail region: row t's ntail blocks at t * ntail * BB; a piece may span two rows
  const int64_t tbytes = ntail * BB;
  const int64_t o0 = (ig - nmainp) * PB;
  for (int b = 0; b < PB; ++b) {
    const int64_t o = o0 + b;
    const int64_t row = w * 64 + o / tbytes;
    out[i * PB + b] = (row < vocab) ? wq[row * rowbytes + nslices * F::kNBlk * BB + o % tbytes] : (uint8_t)0;
  }
}

int64_t lmhead_packed_bytes(int format, int in_dim, int vocab) {
  const int bb = format == kLmQ4_0 ? 18 : format == kLmQ8_0 ? 34 : 64;
  return (int64_t)((vocab + 63) / 64) * 64 * (int64_t)(in_dim / 32) * bb;
}

hipError_t launch_lmhead_pack(const uint8_t *w, int format, int in_dim, int vocab, uint8_t *packed,
                              hipStream_t st) {
  const int pb = format == kLmQ8_0 ? 8 : 16;
  const int64_t npieces = lmhead_packed_bytes(format, in_dim, vocab) / pb;
  const dim3 grid((unsigned)((npieces + 255) / 256));
  if (format == kLmQ4_0)
    hipLaunchKernelGGL(k_lmhead_pack<kLmQ4_0>, grid, dim3(256), 0, st, w, packed, in_dim, vocab, npieces);
  else if (format == kLmQ8_0)
    hipLaunchKernelGGL(k_lmhead_pack<kLmQ8_0>, grid, dim3(256), 0, st, w, packed, in_dim, vocab, npieces);
  else
    hipLaunchKernelGGL(k_lmhead_pack<kLmF16>, grid, dim3(256), 0, st, w, packed, in_dim, vocab, npieces);
  return hipGetLastError();
}

template <int FMT, bool PACKED>
static void launch_fmt(int NB, dim3 grid, hipStream_t st, const uint8_t *w, const float *x, float *l,
                       int64_t ls, int32_t in_dim, int32_t vocab, int32_t B) {
#define VDX_LM(N) \
  hipLaunchKernelGGL((k_lmhead<FMT, N, PACKED>), grid, dim3(64), 0, st, w, x, l, ls, in_dim, vocab, B)
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
}

hipError_t launch_lmhead(const LmHeadParams &p, hipStream_t st) {
  const dim3 grid((unsigned)((p.vocab + 63) / 64));
  for (int b0 = 0; b0 < p.rows; b0 += 16) {
    const int B = min(16, p.rows - b0);
    const float *x = p.hidden + (int64_t)b0 * p.hidden_stride;
    float *l = p.logits + (int64_t)b0 * p.logit_stride;
    const int NB = (B == 1) ? 1 : (B == 2) ? 2 : (B <= 4) ? 4 : (B <= 8) ? 8 : 16;
    if (NB > 1 || p.norm_weight) {
      hipLaunchKernelGGL(k_lmhead_prep, dim3((unsigned)NB), dim3(256), 0, st, x, p.hidden_stride,
                         p.norm_weight, p.norm_eps, p.in_dim, B, NB, p.scratch);
      x = p.scratch;
    }
#define VDX_FMT(FM)                                                                          \
  (p.packed ? launch_fmt<FM, true>(NB, grid, st, p.weights, x, l, p.logit_stride, p.in_dim, p.vocab, B) \
            : launch_fmt<FM, false>(NB, grid, st, p.weights, x, l, p.logit_stride, p.in_dim, p.vocab, B))
    if (p.format == kLmQ4_0)
      VDX_FMT(kLmQ4_0);
    else if (p.format == kLmQ8_0)
      VDX_FMT(kLmQ8_0);
    else
      VDX_FMT(kLmF16);
#undef VDX_FMT
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace vdx
