// vdx_device.hpp -- device-side building blocks of the gfx950 sampler:
// order-preserving float keys, wave64 reductions and scans, the two RNGs,
// and the workspace records the kernels exchange through HBM.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vdx {

// ---- launch geometry --------------------------------------------------------
constexpr int kBlock = 256;                    // threads per workgroup (4 waves)
constexpr int kWaves = kBlock / 64;
constexpr int kPerThread = 64;                 // logits per thread per chunk
constexpr int kChunk = kBlock * kPerThread;    // 16384 logits (64 KiB) per chunk
constexpr int kWaveSpan = 64 * kPerThread;     // 4096 contiguous logits per wave
constexpr int kKMax = 64;                      // top-K held one slot per lane
constexpr int kCandCap = 128;                  // candidates stored per chunk
constexpr int kMaxChunks = 256;                // V <= 4 Mi logits
constexpr int kMergeCap = 2048;                // merge-phase LDS candidates
constexpr int kPenMax = 256;                   // history ids handled inside the top-K kernel
constexpr int kKBig = 1024;                    // largest K of the large-K top-K kernel
constexpr int kBigCandCap = 1024;              // its largest candidate slots per chunk

// ---- per-row state kept in HBM -------------------------------------------------
struct RowState {
  uint64_t rng[4];      // xoshiro256** state (Sampler.pas:41-45)
  uint64_t step;        // Philox block counter
  uint64_t key;         // Philox key (the resolved seed)
  int32_t hist_pos;     // ring write position (Sampler.pas:49)
  int32_t hist_count;   // ring fill (Sampler.pas:50)
  int32_t window;       // ring length, RepeatWindow (Sampler.pas:47); <= 0: no history
  int32_t ctr_row;      // Philox counter word 1: the row the stream was seeded on
};
static_assert(sizeof(RowState) == 64, "RowState is 64 bytes");

// Per-row sampling parameters, when rows of one sampler carry their own
// configs: the values of a TVdxSamplerConfig (Sampler.pas:26-34) as the
// kernels use them.
struct RowCfg {
  float inv_t;          // fl32(1 / T) (Sampler.pas:325); 0 when T = 0
  int32_t top_k;
  float top_p;
  float min_p;
  float penalty;
  int32_t window;
  int32_t greedy;       // T = 0 (Sampler.pas:305)
  int32_t pad;
};

// Sampling path of a row over V logits (Sampler.pas:305, 327, 461):
// 0 greedy, 1 top-K with K <= kKBig, 2 full softmax, 3 top-K with K > kKBig
// (one workgroup per row, exact replay only).
constexpr int kPathGreedy = 0, kPathTopk = 1, kPathFull = 2, kPathTopkHuge = 3;
__host__ __device__ __forceinline__ int row_path(const RowCfg &c, int V) {
  if (c.greedy) return kPathGreedy;
  if (c.top_k > 0 && c.top_k < V) return c.top_k <= kKBig ? kPathTopk : kPathTopkHuge;
  return kPathFull;
}
// The sampling kernel applies this row's penalty itself (its window fits the
// kernels' history table); rows with longer windows, and rows of the K > kKBig
// kernel (which has no stream phase), take the separate kernel.
__host__ __device__ __forceinline__ bool row_fuses_penalty(const RowCfg &c, int V) {
  return c.penalty != 1.0f && c.window <= kPenMax && row_path(c, V) != kPathTopkHuge;
}

// Per-chunk candidate quota of the top-K stream phase.  A chunk stores every
// logit >= tau_c, where tau_c guarantees >= Kq stored logits.  The merge
// proves afterwards that the stored set holds the row's top K (theta = K-th
// largest stored value >= every tau_c) or re-reads the chunks for which that
// fails, so Kq may be far below K: the row's top K holds about K/S logits of
// each of its S chunks (3K/S: 12 at K = 64, S = 16, three knock-out rounds
// per wave).  Rows whose draw walks the buffer's slots (`slots`) store four
// more per chunk: their replay feeds a chunk from its stored keys only when
// those include every logit above the buffer's minimum, so more stored keys
// mean fewer chunks re-read.
__host__ __device__ __forceinline__ int chunk_quota(int K, int S, bool slots = false) {
  if (S <= 1) return K;
  const int q = (3 * K + S - 1) / S + (slots ? 4 : 0);
  return q < 8 ? (K < 8 ? K : 8) : (q < K ? q : K);
}
// The large-K kernel's quota: the row's top K holds about K/S logits of a
// chunk, with a spread of about sqrt(K/S); four of those plus 8 leave the
// re-read of a chunk rare while keeping the keys the merge selects from
// (about S times the quota) within its LDS.
__host__ __device__ __forceinline__ int big_chunk_quota(int K, int S) {
  if (S <= 1) return K;
  const int m = (K + S - 1) / S;
  int r = 1;
  while (r * r < m) ++r;  // ceil(sqrt(m))
  const int q = m + 4 * r + 8;
  return q < K ? q : K;
}
// Candidate slots per chunk of the large-K kernel: about three times the
// quota (the stream phase's threshold stores up to ~2-3x it), at least 256.
__host__ __device__ __forceinline__ int big_cand_cap(int K, int S) {
  const int q = big_chunk_quota(K, S);
  int cap = 256;
  while (cap < 3 * q && cap < kBigCandCap) cap <<= 1;
  return cap;
}

// Top-K stream phase: one record per (row, chunk):
//   w    = tau_key | flags << 32  (every logit with key >= tau_key is stored;
//                                  flags bit 0: a NaN or +inf logit was seen)
//   n[w] = candidates wave w found (more than its region holds: overflow)
// The chunk's kCandCap candidate slots are split among the waves that hold
// logits (wave_cap), so each wave stores without a block-wide count.
struct ChunkMeta {
  uint64_t w;
  uint32_t n[kWaves];
  uint32_t pad[2];
};
// Chunks are read in the interleaved layout (position j*1024 + wave*256 + ...),
// so a short chunk of <= 256 logits lives in wave 0 and one of <= 512 in waves
// 0 and 1.
__device__ __forceinline__ int wave_cap(int clen, int cap = kCandCap) {
  return clen <= 256 ? cap : (clen <= 512 ? cap / 2 : cap / kWaves);
}

// A stored candidate: ord_key(value) << 32 | ~index (larger = better, unique).
typedef uint64_t Cand;

// Full-softmax path: one record per (row, chunk):
//   w[0] = bits(m) | flags << 32  (m = chunk max of s = fl32(L * invT))
//   w[1] = bits(d)                (sum of weights relative to m or the row max)
//   w[2+w] = bits(dw[w])          (the same per 4096-logit wave segment)
struct FullMeta {
  uint64_t w[2 + kWaves];
};

// ---- exchange between the workgroups of one launch ------------------------------
// The records above cross workgroups (and XCDs, each with its own L2) inside
// one kernel.  They are written and read with system-scope relaxed accesses
// (sc0 sc1: the L2 of the writer's XCD is written through and the reader's is
// bypassed); a writer waits for its stores to be acknowledged
// (s_waitcnt vmcnt(0)) before taking the row's ticket, so the workgroup that
// takes the last ticket reads complete records without an L2 writeback or
// invalidate.
__device__ __forceinline__ void xstore(uint64_t *p, uint64_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void xstore32(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint64_t xload(const uint64_t *p) {
  return __hip_atomic_load(const_cast<uint64_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
// Logits written in place by the fused penalty are stored with xstoref and
// re-read (replay, chunk re-read) with xloadf.
__device__ __forceinline__ void xstoref(float *p, float v) {
  __hip_atomic_store(reinterpret_cast<uint32_t *>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ float xloadf(const float *p) {
  return __uint_as_float(__hip_atomic_load(reinterpret_cast<uint32_t *>(const_cast<float *>(p)),
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM));
}

struct KernelRng {
  const float *uniforms;  // injected per-row u (nullable)
  RowState *rows;
  int32_t kind;           // 0 xoshiro, 1 philox (key: RowState::key)
  float *u_out;           // optional copy of the consumed u
};

struct KernelOut {
  int32_t *tokens;
  int32_t *topk_idx;
  float *topk_prob;
  int32_t topk_stride;
  uint32_t *flags;
};

constexpr uint32_t kRowGreedy = 0x1, kRowTopkFast = 0x2, kRowTopkReplay = 0x4,
                   kRowFull = 0x8, kRowNan = 0x10, kRowFallback = 0x20;

// ---- float keys ------------------------------------------------------------------
// Order-preserving map of a non-NaN float to uint32 in which -0 and +0 share a
// key (the reference compares them equal).  -inf -> 0x007FFFFF, +inf ->
// 0xFF800000; key 0 is below every float and marks "no value".
__device__ __forceinline__ uint32_t ord_key(float x) {
  uint32_t b = __float_as_uint(x);
  b = (b == 0x80000000u) ? 0u : b;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float key_float(uint32_t k) {
  uint32_t b = (k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k;
  return __uint_as_float(b);
}
// Key used by the reference's min-buffer replay: NaN never becomes the
// minimum, so it maps above +inf.
__device__ __forceinline__ uint32_t slot_key(float x) {
  return (x != x) ? 0xFFFFFFFFu : ord_key(x);
}

// ---- wave64 primitives --------------------------------------------------------------
// Cross-lane steps use DPP (row_shr within 16-lane rows, then row_bcast:15 /
// row_bcast:31 across rows), which run on the VALU without a trip through the
// LDS crossbar.  Every primitive here must be called with all 64 lanes
// active: the results are read from lane 63.
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

template <int CTRL, int ROWMASK>
__device__ __forceinline__ uint32_t dpp32(uint32_t old, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)v, CTRL, ROWMASK, 0xF, false);
}
template <int CTRL, int ROWMASK>
__device__ __forceinline__ uint64_t dpp64(uint64_t old, uint64_t v) {
  const uint32_t lo = dpp32<CTRL, ROWMASK>((uint32_t)old, (uint32_t)v);
  const uint32_t hi = dpp32<CTRL, ROWMASK>((uint32_t)(old >> 32), (uint32_t)(v >> 32));
  return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint32_t readlane32(uint32_t v, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)v, l);
}
__device__ __forceinline__ uint64_t readlane64(uint64_t v, int l) {
  return ((uint64_t)readlane32((uint32_t)(v >> 32), l) << 32) | readlane32((uint32_t)v, l);
}

// Inclusive prefix (lane 0 first) of an associative operation with identity
// `id`: Hillis-Steele over shifts 1, 2, 4, 8 inside each row, then the row
// totals of rows 0 / 2 into rows 1 / 3 and of rows 0-1 into rows 2-3.
template <typename T, typename Op>
__device__ __forceinline__ T wave_scan(T v, T id, Op op) {
  if constexpr (sizeof(T) == 4) {
    v = op(v, dpp32<0x111, 0xF>(id, v));
    v = op(v, dpp32<0x112, 0xF>(id, v));
    v = op(v, dpp32<0x114, 0xF>(id, v));
    v = op(v, dpp32<0x118, 0xF>(id, v));
    v = op(v, dpp32<0x142, 0xA>(id, v));
    v = op(v, dpp32<0x143, 0xC>(id, v));
  } else {
    v = op(v, dpp64<0x111, 0xF>(id, v));
    v = op(v, dpp64<0x112, 0xF>(id, v));
    v = op(v, dpp64<0x114, 0xF>(id, v));
    v = op(v, dpp64<0x118, 0xF>(id, v));
    v = op(v, dpp64<0x142, 0xA>(id, v));
    v = op(v, dpp64<0x143, 0xC>(id, v));
  }
  return v;
}
struct OpMaxU32 { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a > b ? a : b; } };
struct OpMinU32 { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a < b ? a : b; } };
struct OpAddU32 { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a + b; } };
struct OpOrU32 { __device__ uint32_t operator()(uint32_t a, uint32_t b) const { return a | b; } };
struct OpAddU64 { __device__ uint64_t operator()(uint64_t a, uint64_t b) const { return a + b; } };
struct OpMaxU64 { __device__ uint64_t operator()(uint64_t a, uint64_t b) const { return a > b ? a : b; } };
struct OpMinU64 { __device__ uint64_t operator()(uint64_t a, uint64_t b) const { return a < b ? a : b; } };
struct OpAddF64 {
  __device__ uint64_t operator()(uint64_t a, uint64_t b) const {
    return (uint64_t)__double_as_longlong(__longlong_as_double((long long)a) + __longlong_as_double((long long)b));
  }
};

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  return readlane32(wave_scan<uint32_t>(v, 0u, OpMaxU32()), 63);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  return readlane32(wave_scan<uint32_t>(v, 0xFFFFFFFFu, OpMinU32()), 63);
}
__device__ __forceinline__ uint32_t wave_or_u32(uint32_t v) {
  return readlane32(wave_scan<uint32_t>(v, 0u, OpOrU32()), 63);
}
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
  return readlane64(wave_scan<uint64_t>(v, 0ull, OpMaxU64()), 63);
}
__device__ __forceinline__ uint64_t wave_min_u64(uint64_t v) {
  return readlane64(wave_scan<uint64_t>(v, ~0ull, OpMinU64()), 63);
}
// Maximum ignoring NaN (fmaxf): the ordered keys of non-NaN values, NaN as
// the lowest key; an all-NaN wave yields NaN.
__device__ __forceinline__ float wave_max_f32(float v) {
  const uint32_t b = __float_as_uint(v);
  uint32_t k = (v != v) ? 0u : ((b & 0x80000000u) ? ~b : (b | 0x80000000u));
  k = wave_max_u32(k);
  if (k == 0u) return __uint_as_float(0x7FC00000u);
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v) {
  return readlane32(wave_scan<uint32_t>(v, 0u, OpAddU32()), 63);
}
__device__ __forceinline__ uint32_t wave_incl_scan_u32(uint32_t v) {
  return wave_scan<uint32_t>(v, 0u, OpAddU32());
}
// Double sums: exact whenever every partial sum is representable (the
// callers rely on this only where all addends share a 2^-52-relative grid),
// otherwise rounded in the scan's association order.
__device__ __forceinline__ double wave_incl_scan_f64(double v) {
  return __longlong_as_double((long long)wave_scan<uint64_t>((uint64_t)__double_as_longlong(v), 0ull, OpAddF64()));
}
__device__ __forceinline__ double wave_sum_f64(double v) {
  return __longlong_as_double((long long)readlane64((uint64_t)__double_as_longlong(wave_incl_scan_f64(v)), 63));
}
// Number of set bits of `mask` below this lane.
__device__ __forceinline__ uint32_t lane_rank(uint64_t mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}
__device__ __forceinline__ uint64_t lanemask_lt() {
  const int l = lane_id();
  return l == 0 ? 0ull : (~0ull >> (64 - l));
}

// ---- RNG -------------------------------------------------------------------------------
__device__ __forceinline__ uint64_t rotl64(uint64_t x, int k) {
  return (x << k) | (x >> (64 - k));
}
// xoshiro256** step (Sampler.pas:208-222); returns the output word.
__device__ __forceinline__ uint64_t xoshiro_next(uint64_t s[4]) {
  const uint64_t r = rotl64(s[1] * 5ull, 7) * 9ull;
  const uint64_t t = s[1] << 17;
  s[2] ^= s[0];
  s[3] ^= s[1];
  s[1] ^= s[2];
  s[0] ^= s[3];
  s[2] ^= t;
  s[3] = rotl64(s[3], 45);
  return r;
}
// Philox4x64-10 (Salmon et al., SC'11), word 0 only.
__device__ __forceinline__ uint64_t philox4x64_10_w0(uint64_t c0, uint64_t c1,
                                                     uint64_t c2, uint64_t c3,
                                                     uint64_t k0, uint64_t k1) {
  const uint64_t M0 = 0xD2E7470EE14C6C93ull, M1 = 0xCA5A826395121157ull;
  const uint64_t W0 = 0x9E3779B97F4A7C15ull, W1 = 0xBB67AE8584CAA73Bull;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    if (r > 0) {
      k0 += W0;
      k1 += W1;
    }
    const uint64_t hi0 = __umul64hi(M0, c0), lo0 = M0 * c0;
    const uint64_t hi1 = __umul64hi(M1, c2), lo1 = M1 * c2;
    const uint64_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
  }
  return c0;
}
// (x >> 40) / 2^24 (Sampler.pas:247).
__device__ __forceinline__ float u24(uint64_t x) {
  return (float)(x >> 40) * (1.0f / 16777216.0f);
}
// The state one draw for `row` needs (the injected uniform, or the row's RNG
// state), loaded by every workgroup of the row when it starts, so the one that
// finishes the row draws without a further round trip to memory.  The state
// was last written by an earlier launch, never by this one.  It is one vector
// load into one register (lane l < 16 holds dword l of the row's RowState,
// lane 16 the injected uniform), not scalar loads: a wave waits for all of
// its outstanding scalar loads at once, so a scalar load of the state (a miss
// that queues behind the chunk loads of the workgroups already running) would
// hold back the kernel-argument waits before this workgroup's own chunk loads.
struct RngPre {
  uint32_t w;
};
static_assert(offsetof(RowState, step) == 32 && offsetof(RowState, key) == 40 &&
                  offsetof(RowState, ctr_row) == 60,
              "RowState dwords read back by rng_draw");
__device__ __forceinline__ RngPre rng_prefetch(const KernelRng &g, int row) {
  const int l = (int)(threadIdx.x & 63u);
  const uint32_t *a = reinterpret_cast<const uint32_t *>(&g.rows[row]) + (l & 15);
  if (l == 16 && g.uniforms) a = reinterpret_cast<const uint32_t *>(g.uniforms + row);
  RngPre r;
  r.w = *a;
  return r;
}
// The prefetched state read out of its register with v_readlane.  Called
// where every lane of the wave is active (never under a per-lane condition),
// so the load is never moved under one either: v_readlane ignores the
// execution mask, but a lane that skipped the load holds no state.
struct RngVals {
  uint64_t s[4];
  uint64_t step;
  uint64_t key;
  uint32_t ctr_row;
  float u;
};
__device__ __forceinline__ uint64_t rng_pre64(const RngPre &r, int l) {
  return (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)r.w, l) |
         ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)r.w, l + 1) << 32);
}
__device__ __forceinline__ RngVals rng_unpack(const RngPre &r) {
  RngVals v;
  v.s[0] = rng_pre64(r, 0);
  v.s[1] = rng_pre64(r, 2);
  v.s[2] = rng_pre64(r, 4);
  v.s[3] = rng_pre64(r, 6);
  v.step = rng_pre64(r, 8);
  v.key = rng_pre64(r, 10);
  v.ctr_row = (uint32_t)__builtin_amdgcn_readlane((int)r.w, 15);
  v.u = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)r.w, 16));
  return v;
}
// One uniform for `row` from prefetched state: injected, or drawn (advancing
// and storing that row's RNG).  Called by exactly one thread per row.
__device__ __forceinline__ float rng_draw(const KernelRng &g, int row, RngVals &r) {
  float u;
  if (g.uniforms) {
    u = r.u;
  } else if (g.kind == 1) {
    u = u24(philox4x64_10_w0(r.step, (uint64_t)r.ctr_row, 0, 0, r.key, 0));
    g.rows[row].step = r.step + 1;
  } else {
    u = u24(xoshiro_next(r.s));
    g.rows[row].rng[0] = r.s[0];
    g.rows[row].rng[1] = r.s[1];
    g.rows[row].rng[2] = r.s[2];
    g.rows[row].rng[3] = r.s[3];
  }
  if (g.u_out) g.u_out[row] = u;
  return u;
}

// Maps a workgroup id to (row, chunk) so that the chunks of one row run on
// one XCD (workgroups are dealt round-robin over the 8 XCDs).
__device__ __forceinline__ void block_row_chunk(int nchunks, int rows, int &row, int &chunk) {
  const int bid = blockIdx.x;
  const int nb = rows * nchunks;
  int logical = bid;
  if ((nb & 7) == 0) logical = (bid & 7) * (nb >> 3) + (bid >> 3);
  row = logical / nchunks;
  chunk = logical - row * nchunks;
}

}  // namespace vdx
