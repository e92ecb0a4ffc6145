// vdx_kernels.hip -- gfx950 kernels of the token sampler.
//
// The reference runs TVdxSampler.Process (src/VindexLLM.Sampler.pas:265-528)
// on the host after downloading each logit row.  Here every stage runs on the
// GPU over rows that stay in HBM:
//   k_penalty  repetition penalty, once per history occurrence (:285-303)
//   k_greedy   first index of the maximum (:306-322)
//   k_topk     top-K select + softmax / Min-P / Top-P / draw (:327-460)
//   k_full     full-vocabulary softmax + draw, K = 0 or K >= V (:461-527)
// Rows are split into 16384-logit chunks, one 256-thread workgroup per chunk;
// the last workgroup of a row (atomic ticket) merges the chunk results and
// finishes the row, so a sampling call is one kernel launch per stage.
#include <math.h>

#include "vdx_internal.hpp"

namespace vdx {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Four logits read past the caches (see xloadf); p is 16-byte aligned.
__device__ __forceinline__ f32x4 xload4(const float *p) {
  const uint64_t a = xload(reinterpret_cast<const uint64_t *>(p));
  const uint64_t b = xload(reinterpret_cast<const uint64_t *>(p) + 1);
  f32x4 r;
  r[0] = __uint_as_float((uint32_t)a);
  r[1] = __uint_as_float((uint32_t)(a >> 32));
  r[2] = __uint_as_float((uint32_t)b);
  r[3] = __uint_as_float((uint32_t)(b >> 32));
  return r;
}

// Rows with their own configs (p.rcfg): whether `row` takes path `path` in
// this launch (the kernels of the other paths skip it), and the call's
// parameters as the row sees them.  Without per-row configs every row takes
// the launch's path with the call's parameters.
__device__ __forceinline__ bool row_on_path(const CallParams &p, int row, int path) {
  return !p.rcfg || row_path(p.rcfg[row], p.vocab) == path;
}
__device__ __forceinline__ CallParams for_row(const CallParams &p, int row) {
  CallParams q = p;
  if (p.rcfg) {
    const RowCfg c = p.rcfg[row];
    q.inv_t = c.inv_t;
    q.top_k = c.top_k;
    q.top_p = c.top_p;
    q.min_p = c.min_p;
    q.penalty = c.penalty;
    q.fuse_penalty = (p.fuse_penalty && row_fuses_penalty(c, p.vocab)) ? 1 : 0;
  }
  return q;
}

// Block-wide exclusive scan of one double per thread (kBlock threads).
__device__ __forceinline__ double block_excl_scan_f64(double x, double *wtot, double &total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const double incl = wave_incl_scan_f64(x);
  if (lane == 63) wtot[wv] = incl;
  __syncthreads();
  double base = 0.0;
  total = 0.0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    if (w < wv) base += wtot[w];
    total += wtot[w];
  }
  __syncthreads();
  return base + (incl - x);
}

// Chunk layouts.  Thread (wave wv, lane) owns 16 float4 groups j of a chunk:
//   interleaved (default):  j*1024 + wv*256 + lane*4 + e
//     the workgroup's j-th load instruction reads one contiguous 4 KiB piece,
//     which spreads the four waves' requests over HBM channels better than
//     four pieces 16 KiB apart (measured: ~2 us less per 64 MiB);
//   span (SPAN = true):     wv*4096 + j*256 + lane*4 + e
//     each wave owns a contiguous 4096-logit span (the full-softmax path
//     locates its draw inside one such span).
template <bool SPAN = false>
__device__ __forceinline__ int chunk_pos(int wv, int lane, int i) {
  return SPAN ? wv * kWaveSpan + (i >> 2) * 256 + lane * 4 + (i & 3)
              : (i >> 2) * 1024 + wv * 256 + lane * 4 + (i & 3);
}
// Positions at or beyond `clen` read as `fill`.  With VEC (16-byte aligned
// rows whose length is a multiple of 4) every float4 group is either wholly
// inside the row or wholly past it, so the loads are unconditional (a group
// past the end re-reads the chunk's first group and is replaced by `fill`):
// no branch separates them, and the compiler waits for each group on its own
// (in-order vmcnt) instead of for all loads at once.
template <bool VEC, bool SPAN = false>
__device__ __forceinline__ void load_chunk(const float *__restrict__ base, int clen, int wv,
                                           int lane, float (&v)[kPerThread], float fill) {
  if (VEC) {
#pragma unroll
    for (int j = 0; j < kPerThread / 4; ++j) {
      const int local = chunk_pos<SPAN>(wv, lane, 4 * j);
      const f32x4 f = __builtin_nontemporal_load(
          reinterpret_cast<const f32x4 *>(base + (local < clen ? local : 0)));
      v[4 * j + 0] = f[0];
      v[4 * j + 1] = f[1];
      v[4 * j + 2] = f[2];
      v[4 * j + 3] = f[3];
    }
    if (clen < kChunk) {  // uniform; after every load has been issued
#pragma unroll
      for (int j = 0; j < kPerThread / 4; ++j) {
        if (chunk_pos<SPAN>(wv, lane, 4 * j) >= clen) {
          v[4 * j + 0] = fill;
          v[4 * j + 1] = fill;
          v[4 * j + 2] = fill;
          v[4 * j + 3] = fill;
        }
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      const int local = chunk_pos<SPAN>(wv, lane, i);
      v[i] = (local < clen) ? base[local] : fill;
    }
  }
}

// Last-workgroup election for a row: returns true in every thread of the
// workgroup that finished the row last.  Records written with xstore() before
// the call by any workgroup of the row are complete when the winner reads them
// with xload(): each wave waits for its stores to be acknowledged before the
// workgroup takes its ticket.  `meanwhile()` runs (in every thread) while the
// ticket is in flight.
template <typename F>
__device__ __forceinline__ bool last_of_row(uint32_t *tickets, int row, int nchunks, int *flag,
                                            F &&meanwhile) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  uint32_t t = 0u;
  if (threadIdx.x == 0)
    t = __hip_atomic_fetch_add(&tickets[row], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  meanwhile();
  if (threadIdx.x == 0) *flag = (t == (uint32_t)(nchunks - 1));
  __syncthreads();
  if (!*flag) return false;
  if (threadIdx.x == 0)  // every other chunk has arrived: reset for the next launch
    __hip_atomic_store(&tickets[row], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  return true;
}

// =============================================================================
// Repetition penalty (Sampler.pas:285-303).  One workgroup per row; the first
// occurrence of each in-range id applies the reference's sign test and
// divide / multiply once per occurrence, in order, with IEEE fp32 arithmetic.
// =============================================================================
constexpr int kPenStage = 4096;

__device__ __forceinline__ float penalise(float x, int k, float pen) {
  for (int r = 0; r < k; ++r) {
    if (x > 0.0f)
      x = x / pen;
    else if (x < 0.0f)
      x = x * pen;
  }
  return x;
}

// The same k steps with the division as a double product: for fp32 x and p
// (normal, p > 0) with ip = RN64(1/p), RN32(RN64(x * ip)) = RN32(x / p)
// whenever that quotient is normal.  RN64(x * ip) is within 2^-52 (relative)
// of x / p, while x / p is never within 2^-49 of a midpoint of two fp32 values
// (with x = A 2^a, p = B 2^b, A, B < 2^24, and a midpoint m = M 2^c, M odd,
// 2^24 <= M < 2^25: x - m p is a non-zero multiple of 2^min(a, b + c), as M B
// has more than 24 significant bits), so both round to the same fp32 value.
// Quotients below 2^-125 (subnormal or close to it) take the IEEE division.
__device__ __forceinline__ float penalise_fast(float x, int k, float pen, double ip) {
  for (int r = 0; r < k; ++r) {
    const double q = (double)x * ip;
    float d = (float)q;
    if (x > 0.0f && !(q >= 0x1p-125)) d = x / pen;  // rare: tiny quotients
    x = (x > 0.0f) ? d : ((x < 0.0f) ? x * pen : x);
  }
  return x;
}

// With per-row configs, a row runs here when its penalty is not 1 and the
// top-K kernel does not apply it.
__global__ __launch_bounds__(kBlock) void k_penalty(CallParams p0) {
  __shared__ __align__(16) int32_t sh[kPenStage];
  const int row = blockIdx.x;
  const CallParams p = for_row(p0, row);
  if (p.penalty == 1.0f || p.fuse_penalty) return;
  const int V = p.vocab, W = p.hist_len;
  const float pen = p.penalty;
  const int cnt = min(p.rng.rows[row].hist_count, W);
  if (cnt <= 0) return;
  const int32_t *h = p.hist + (int64_t)row * W;
  float *L = p.logits + (int64_t)row * p.stride;
  if (cnt > kPenStage) {
    // long windows: the same rule with the ids read from HBM
    for (int j = threadIdx.x; j < cnt; j += kBlock) {
      const int id = h[j];
      if (id < 0 || id >= V) continue;
      int k = 0;
      bool first = true;
      for (int jj = 0; jj < cnt; ++jj) {
        if (h[jj] == id) {
          if (jj < j) {
            first = false;
            break;
          }
          ++k;
        }
      }
      if (first) L[id] = penalise(L[id], k, pen);
    }
    return;
  }
  const int cnt4 = (cnt + 3) & ~3;
  for (int j = threadIdx.x; j < cnt4; j += kBlock) sh[j] = (j < cnt) ? h[j] : -1;
  __syncthreads();
  const int4 *s4 = reinterpret_cast<const int4 *>(sh);
  for (int j = threadIdx.x; j < cnt; j += kBlock) {
    const int id = sh[j];
    if (id < 0 || id >= V) continue;  // padding (-1) never matches an in-range id
    int total = 0, before = 0;
    for (int q = 0; q < cnt4 / 4; ++q) {
      const int4 w = s4[q];  // every lane reads the same word: LDS broadcast
      const int b = 4 * q;
      total += (w.x == id) + (w.y == id) + (w.z == id) + (w.w == id);
      before += (w.x == id && b < j) + (w.y == id && b + 1 < j) + (w.z == id && b + 2 < j) +
                (w.w == id && b + 3 < j);
    }
    if (before == 0) L[id] = penalise(L[id], total, pen);  // first occurrence applies all
  }
}

// =============================================================================
// Top-K path (Sampler.pas:327-460).
//
// Stream phase (every 16384-logit chunk): 64 logits per thread in registers;
// a threshold tau_c that >= Kq logits of the chunk reach (the smallest of the
// four waves' R-th largest thread maxima); every logit >= tau_c is stored as a
// candidate key (value, then lower index) in the storing wave's region.
//
// Merge (the workgroup that takes the row's last ticket): a logit that was
// not stored is < tau_c <= T = max_c tau_c, so every logit >= T is stored; if
// at least K are, the row's top K is the K largest of them.  Those keys are
// compacted into LDS and the top K found by in-wave bitonic sorts and merges.
// Otherwise (or when a region overflowed) the slower general merge runs: a
// radix select of theta = the K-th largest stored key, and a re-read of every
// chunk whose tau_c exceeds theta.  A K-th value tied with a logit outside the
// set sends the row to the exact replay, as the reference's min-buffer keeps
// the tied logits that arrived first in its own slot order.
//
// Finish: see topk_fast and topk_exact.
// =============================================================================
constexpr int kMergeSpec = 8;   // candidate slots loaded per thread per round
constexpr int kMergeTop = 512;  // keys >= T handled by the bitonic merge

constexpr int kPenHash = 4 * kPenMax;  // open-addressing table of the fused penalty

struct TopkSmem {
  uint32_t thr[64];
  uint32_t cnt[kWaves][64];
  uint32_t wmax[kWaves];
  uint32_t wflag[kWaves];
  uint32_t wtot[kWaves];
  int32_t last;
  uint32_t ccount[kMaxChunks];
  uint32_t ctau[kMaxChunks];
  uint32_t n;
  uint32_t hist[256];
  uint32_t rbin, rneed, rcnt;
  uint32_t ngt;
  int32_t ntop;
  int32_t mres;
  uint64_t topsel[kKMax];
  uint64_t topkey[kKMax];
  float uval;
  int32_t token;
  uint32_t rowflags;
  int32_t replay;
  uint32_t xw[kWaves];   // exact path: candidates per wave in the current group
  uint64_t xw64[kWaves][4];  // exact path, whole chunk: per wave, 16 group counts in 16-bit fields
  uint32_t xmkey;        // exact path: key of the buffer's minimum
  int32_t xfrozen;       // exact path: L[0] is NaN, nothing enters
  int32_t xdone;         // exact path: the slot-order finish ran in wave 0
  int32_t qnan;
  float wfmax[kWaves];
  double S;
  float slot_v[kKMax];
  int32_t slot_i[kKMax];
  float q[kKMax];
  float q_ord[kKMax];
  int32_t i_ord[kKMax];
  float v_ord[kKMax];
  // fused penalty: one entry per distinct history id, id | occurrences << 22
  uint32_t ptab[kPenHash];
  uint32_t pcnt[8 * kBlock];  // history counts of each thread's 64 logits, 4 bits each (word-major)
  union {
    uint64_t sk[kMergeCap];
  } buf;
};

__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }
// Maximum of float4 group j of a thread's logits (NaN-propagating).
__device__ __forceinline__ float gmax4(const float (&v)[kPerThread], int j) {
  return vmax(vmax(vmax(v[4 * j], v[4 * j + 1]), v[4 * j + 2]), v[4 * j + 3]);
}

// Repetition penalty fused into the top-K kernel (Sampler.pas:285-303): each
// workgroup penalises the history ids that fall in its own chunk, in its
// registers, before it selects anything, and stores those logits in place
// (the reference mutates its input).  The ids are prefetched before the
// chunk; while the chunk is in flight the in-chunk ids are counted in an LDS
// open-addressing table (entry = id | occurrences << 22 over the whole
// history) and each count is written, 4 bits wide, next to the logit's
// owner thread.  Everything after (thread maxima, threshold, candidates, merge,
// finish) then runs on penalised values, exactly as without a penalty, and
// the stores are acknowledged before the workgroup takes its ticket, so the
// row's last workgroup reads penalised logits wherever it re-reads the row.
constexpr int kPenPerThread = kPenMax / kBlock;
static_assert(kPenPerThread == 1, "one history id per thread");
constexpr uint32_t kPenEmpty = 0xFFFFFFFFu;
constexpr uint32_t kPenIdMask = (1u << 22) - 1u;  // ids < 4 Mi; count in the top 10 bits
static_assert(kMaxChunks * kChunk <= (1 << 22) && kPenMax < 1024, "packed penalty table entries");
static_assert(kPerThread == 64, "eight 32-bit count words of 4-bit fields per thread");

struct PenaltyPrefetch {
  int cnt;
  int32_t id[kPenPerThread];
};

__device__ __forceinline__ void penalty_prefetch(const CallParams &p, int row, PenaltyPrefetch &pf) {
  const int W = p.hist_len;
  const int32_t *h = p.hist + (int64_t)row * W;
  // a vector load (an atomic is never a scalar load): see rng_prefetch
  pf.cnt = __hip_atomic_load(&p.rng.rows[row].hist_count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  // Unconditional load (index clamped; a position past the count is ignored
  // where the id is used), and no arithmetic on it here: the chunk's loads
  // are issued before anything waits for the id.
  pf.id[0] = h[min((int)threadIdx.x, W - 1)];
}

__device__ __forceinline__ uint32_t pen_hash(uint32_t id) {
  return (id * 2654435761u) >> (32 - 10);  // kPenHash = 1024 slots
}
static_assert(kPenHash == 1024, "pen_hash yields 10 bits");

// The table and the count map live in each kernel's shared-memory record (SM
// has members ptab[kPenHash] and pcnt[8 * kBlock]).
struct PenaltySmem {
  uint32_t ptab[kPenHash];
  // history occurrences of each thread's 64 logits, 4 bits each (15: 15 or
  // more, looked up in ptab): word w of thread t at pcnt[w * kBlock + t],
  // logit i of the thread in bits 4 (i & 7) of word i >> 3
  uint32_t pcnt[8 * kBlock];
};

// Empties the table and the count map (before a barrier).
template <class SM>
__device__ __forceinline__ void penalty_clear(SM &sm) {
#pragma unroll
  for (int i = 0; i < kPenHash / kBlock; ++i) sm.ptab[threadIdx.x + i * kBlock] = kPenEmpty;
#pragma unroll
  for (int w = 0; w < 8; ++w) sm.pcnt[w * kBlock + threadIdx.x] = 0u;
}

// Occurrences of `id` in the history (the id is in the table).
template <class SM>
__device__ __forceinline__ uint32_t pen_count(const SM &sm, uint32_t id) {
  uint32_t h = pen_hash(id);
  for (;;) {
    const uint32_t e = sm.ptab[h];
    if (e == kPenEmpty) return 0u;
    if ((e & kPenIdMask) == id) return e >> 22;
    h = (h + 1u) & (uint32_t)(kPenHash - 1);
  }
}

// The fused penalty for one chunk whose logits are in flight into v (the
// table was cleared at kernel start).  While the chunk is in flight: the
// history ids of the chunk are counted in the open-addressing table (at most
// kPenMax distinct ids in kPenHash slots, so a free slot always exists), and
// the thread that inserted each id writes its count into the count map at
// the logit's owner (position pos is logit 4j + e of its thread:
// j*1024 + wv*256 + lane*4 + e in the interleaved layout, wv*4096 + j*256 +
// lane*4 + e in the wave-span layout).  Once the chunk is in, each thread
// reads its own counts (eight words) and penalises those logits in registers
// and in place (Sampler.pas:285-303), with no table lookup on the way.
// Everything after runs on penalised values; the stores are acknowledged
// before the workgroup's ticket.
template <bool SPAN, class SM>
__device__ __forceinline__ void penalty_pass(const CallParams &p, int row, int c0, int clen,
                                             const PenaltyPrefetch &pf, float (&v)[kPerThread], SM &sm) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  constexpr int kG = kPerThread / 4;
  __syncthreads();
  int hs = -1;  // the table slot this thread inserted (its id's first occurrence)
  uint32_t ow = 0u, ob = 0u;  // the logit's count word and bit
  {
    // opaque from here on: a test of the prefetched values hoisted above the
    // chunk's loads would make the wave wait for them before issuing those
    int32_t id = pf.id[0], cnt = pf.cnt;
    asm volatile("" : "+v"(id), "+v"(cnt));
    if (tid < min(cnt, p.hist_len) && id >= c0 && id < c0 + clen) {
      const uint32_t uid = (uint32_t)id;
      uint32_t h = pen_hash(uid);
      for (;;) {
        const uint32_t old = atomicCAS(&sm.ptab[h], kPenEmpty, uid | (1u << 22));
        if (old == kPenEmpty) {
          hs = (int)h;
          break;
        }
        if ((old & kPenIdMask) == uid) {
          atomicAdd(&sm.ptab[h], 1u << 22);
          break;
        }
        h = (h + 1u) & (uint32_t)(kPenHash - 1);
      }
      const int pos = id - c0;
      const uint32_t t = SPAN ? (uint32_t)((pos >> 12) * 64 + ((pos >> 2) & 63))
                              : (uint32_t)(((pos >> 8) & 3) * 64 + ((pos >> 2) & 63));
      const uint32_t i = SPAN ? (uint32_t)((((pos >> 8) & 15) << 2) | (pos & 3))
                              : (uint32_t)(((pos >> 10) << 2) | (pos & 3));
      ow = (i >> 3) * kBlock + t;
      ob = 4u * (i & 7u);
    }
  }
  __syncthreads();  // the counts are final
  if (hs >= 0) {
    const uint32_t c = sm.ptab[hs] >> 22;
    atomicOr(&sm.pcnt[ow], (c < 15u ? c : 15u) << ob);
  }
  __syncthreads();
  uint32_t cw[8];
#pragma unroll
  for (int w = 0; w < 8; ++w) cw[w] = sm.pcnt[w * kBlock + tid];
  const uint32_t any = cw[0] | cw[1] | cw[2] | cw[3] | cw[4] | cw[5] | cw[6] | cw[7];
  __builtin_amdgcn_sched_barrier(0);
  if (__ballot(any != 0u)) {
    float *Lw = p.logits + (int64_t)row * p.stride;  // written in place: not restrict
    const double ip = 1.0 / (double)p.penalty;
#pragma unroll
    for (int j = 0; j < kG; ++j) {
      const uint32_t n4 = (cw[j >> 1] >> (16 * (j & 1))) & 0xFFFFu;
      if (__ballot(n4 != 0u)) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t c = (n4 >> (4 * e)) & 15u;
          if (c) {
            const int idx = c0 + chunk_pos<SPAN>(wv, lane, 4 * j + e);
            const uint32_t k = (c == 15u) ? pen_count(sm, (uint32_t)idx) : c;
            const float x = penalise_fast(v[4 * j + e], (int)k, p.penalty, ip);
            v[4 * j + e] = x;
            xstoref(&Lw[idx], x);
          }
        }
      }
    }
  }
}

// =============================================================================
// Greedy argmax (Sampler.pas:306-322): the reference's strict '>' scan returns
// the lowest index of the maximum; a NaN at index 0 absorbs the scan (-> 0),
// NaNs elsewhere are never chosen.  Key = (ordered value << 32) | ~index.
// A penalty with a window of up to kPenMax ids is applied here first.
// =============================================================================
template <bool VEC>
__global__ __launch_bounds__(kBlock) void k_greedy(CallParams p0) {
  __shared__ uint64_t s_w[kWaves];
  __shared__ int s_last;
  __shared__ PenaltySmem ps;
  int row, chunk;
  block_row_chunk(p0.nchunks, p0.rows, row, chunk);
  if (!row_on_path(p0, row, kPathGreedy)) return;
  const CallParams p = for_row(p0, row);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const float *L = p.logits + (int64_t)row * p.stride;
  const int c0 = chunk * kChunk;
  const int clen = min(kChunk, p.vocab - c0);
  PenaltyPrefetch pf;
  if (p.fuse_penalty) {
    penalty_prefetch(p, row, pf);
    penalty_clear(ps);
  }
  float v[kPerThread];
  load_chunk<VEC>(L + c0, clen, wv, lane, v, __builtin_nanf(""));
  if (p.fuse_penalty) penalty_pass<false>(p, row, c0, clen, pf, v, ps);
  float m = v[0];
#pragma unroll
  for (int i = 1; i < kPerThread; ++i) m = fmaxf(m, v[i]);  // NaN-ignoring
  int first = -1;
#pragma unroll
  for (int i = kPerThread - 1; i >= 0; --i)
    if (v[i] == m) first = i;  // this thread's lowest position of its max
  uint64_t key = 0;
  if (first >= 0)
    key = ((uint64_t)ord_key(m) << 32) |
          (uint32_t)(~(uint32_t)(c0 + chunk_pos(wv, lane, first)));
  key = wave_max_u64(key);
  if (lane == 0) s_w[wv] = key;
  __syncthreads();
  if (tid == 0) {
    uint64_t k = s_w[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) k = s_w[w] > k ? s_w[w] : k;
    xstore(&p.gpart[(int64_t)row * p.nchunks + chunk], k);
  }
  if (!last_of_row(p.tickets, row, p.nchunks, &s_last, [] {})) return;
  uint64_t k = 0;
  for (int c = tid; c < p.nchunks; c += kBlock) {
    const uint64_t x = xload(&p.gpart[(int64_t)row * p.nchunks + c]);
    k = x > k ? x : k;
  }
  k = wave_max_u64(k);
  __syncthreads();
  if (lane == 0) s_w[wv] = k;
  __syncthreads();
  if (tid == 0) {
#pragma unroll
    for (int w = 0; w < kWaves; ++w) k = s_w[w] > k ? s_w[w] : k;
    int32_t tok = k ? (int32_t)(~(uint32_t)k) : 0;
    if (L[0] != L[0]) tok = 0;
    p.out.tokens[row] = tok;
    if (p.out.flags) p.out.flags[row] = kRowGreedy;
    if (p.rng.u_out) p.rng.u_out[row] = 0.0f;
  }
}

// `ccap`: candidate slots of a full chunk (kCandCap, or more for large K).
// FASTQ: the largest quota the knock-out threshold takes (R = Kq / kWaves
// rounds per wave, rounded up); a larger one samples thread maxima instead.
template <bool VEC, int FASTQ = 4 * kWaves, class SM>
__device__ __forceinline__ void topk_stream(const CallParams &p, int row, const float *__restrict__ L,
                                            int c0, int clen, int Kq, Cand *__restrict__ cand,
                                            ChunkMeta *__restrict__ meta, const PenaltyPrefetch &pf,
                                            SM &sm, int ccap = kCandCap) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  constexpr int kG = kPerThread / 4;
  float v[kPerThread];
  load_chunk<VEC>(L + c0, clen, wv, lane, v, -INFINITY);
  if (p.fuse_penalty) penalty_pass<false>(p, row, c0, clen, pf, v, sm);

  // group (float4) maxima and the thread maximum; v_maximum3 propagates NaN,
  // so a NaN or +inf anywhere in the thread's logits shows in `m`
  // (group maxima are recomputed where they are tested, which keeps 16 fewer
  // registers live across the threshold search)
  float m = gmax4(v, 0);
#pragma unroll
  for (int j = 1; j < kG; ++j) m = vmax(m, gmax4(v, j));
  const bool hasv = chunk_pos(wv, lane, 0) < clen;
  const bool bad = hasv && !(m <= 3.4028235e38f);
  const uint32_t mk = hasv ? ord_key(m) : 0u;
  const uint64_t badw = __ballot(bad);
  // Full chunks with a quota of at most FASTQ: every wave finds its R-th
  // largest thread maximum (R knock-out rounds of a wave max); tau = the
  // smallest of the four, so >= 4R >= Kq thread maxima (distinct logits)
  // reach tau.
  const bool fastthr = (clen == kChunk) && Kq <= FASTQ;
  if (fastthr) {
    const int R = (Kq + kWaves - 1) / kWaves;
    uint32_t key = mk, rth = 0u;
    for (int r = 0; r < R; ++r) {
      const uint32_t mx = wave_max_u32(key);
      rth = mx;
      const uint64_t who = __ballot(key == mx);
      if (lane == __ffsll((unsigned long long)who) - 1) key = 0u;
    }
    if (lane == 0) sm.wmax[wv] = rth;
  } else if (wv == 0) {
    sm.thr[lane] = mk;
  }
  if (lane == 0) sm.wflag[wv] = badw != 0ull;
  __syncthreads();

  // tau: 0 stores every logit of a short chunk
  uint32_t tau = 0u;
  if (fastthr) {
    tau = min(min(sm.wmax[0], sm.wmax[1]), min(sm.wmax[2], sm.wmax[3]));
  } else if (clen > ccap) {
    // the largest of 64 sampled thread maxima (wave 0's) that >= Kq reach
    uint32_t mycnt = 0u;
#pragma unroll 4
    for (int j = 0; j < 64; ++j) {
      const uint32_t tj = sm.thr[j];
      const uint32_t c = (uint32_t)__popcll(__ballot(mk >= tj));
      mycnt = (lane == j) ? c : mycnt;
    }
    sm.cnt[wv][lane] = mycnt;
    __syncthreads();
    const uint32_t tot = sm.cnt[0][lane] + sm.cnt[1][lane] + sm.cnt[2][lane] + sm.cnt[3][lane];
    const uint32_t tk = sm.thr[lane];
    tau = wave_max_u32((tot >= (uint32_t)Kq && tk != 0u) ? tk : 0u);
  }
  const float tf = key_float(tau);

  // Candidates: each wave stores into its own region of the chunk's slots
  // (wave_cap), at a running wave count plus the lane's rank in the ballot,
  // so no block-wide count or barrier is needed.  Full chunks test one float4
  // group maximum per compare and branch (wave-uniform) only into groups in
  // which some lane passes.
  const bool all = (tau == 0u);
  const int cap = wave_cap(clen, ccap);
  Cand *wreg = cand + wv * cap;
  uint32_t wc = 0u;  // wave-uniform
  if (clen == kChunk && !all) {
#pragma unroll
    for (int j = 0; j < kG; ++j) {
      if (__ballot(gmax4(v, j) >= tf)) {
        const int l0 = chunk_pos(wv, lane, 4 * j);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool hit = v[4 * j + e] >= tf;
          const uint64_t hb = __ballot(hit);
          if (hb) {
            const uint32_t q = wc + lane_rank(hb);
            if (hit && q < (uint32_t)cap) {
              const int idx = c0 + l0 + e;
              xstore(&wreg[q], ((uint64_t)ord_key(v[4 * j + e]) << 32) | (uint32_t)(~(uint32_t)idx));
            }
            wc += (uint32_t)__popcll(hb);
          }
        }
      }
    }
  } else if (chunk_pos(wv, 0, 0) < clen) {  // short chunk, or tau = 0: test positions too
#pragma unroll
    for (int j = 0; j < kG; ++j) {
      const int l0 = chunk_pos(wv, lane, 4 * j);
      const bool gp = (l0 < clen) && (all || gmax4(v, j) >= tf);
      if (__ballot(gp)) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const bool hit = gp && (l0 + e < clen) && (all || v[4 * j + e] >= tf);
          const uint64_t hb = __ballot(hit);
          if (hb) {
            const uint32_t q = wc + lane_rank(hb);
            if (hit && q < (uint32_t)cap) {
              const int idx = c0 + l0 + e;
              xstore(&wreg[q], ((uint64_t)ord_key(v[4 * j + e]) << 32) | (uint32_t)(~(uint32_t)idx));
            }
            wc += (uint32_t)__popcll(hb);
          }
        }
      }
    }
  }
  if (lane == 0) xstore32(&meta->n[wv], wc);
  if (tid == 0) {
    const uint32_t fl = sm.wflag[0] | sm.wflag[1] | sm.wflag[2] | sm.wflag[3];
    xstore(&meta->w, (uint64_t)tau | ((uint64_t)fl << 32));
  }
}

// Radix select (8 bits per pass, most significant first) of the K-th largest
// value key among the n keys in sm.buf.sk.  Returns that value key; sm.rcnt
// logits share it and sm.rneed of them are in the top K.
// Bytes above the highest byte in which kmin and kmax (bounds of the keys)
// differ are common to every key and are not scanned.
template <class SM>
__device__ __forceinline__ uint32_t radix_kth(uint32_t n, int K, SM &sm, uint32_t kmin, uint32_t kmax) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t d = kmin ^ kmax;
  if (d == 0u) {  // every key shares one value
    if (tid == 0) {
      sm.rcnt = n;
      sm.rneed = (uint32_t)K;
    }
    __syncthreads();
    return kmax;
  }
  const int top = (31 - __clz((int)d)) & ~7;  // first byte that varies
  uint32_t pmask = (top == 24) ? 0u : (0xFFFFFFFFu << (top + 8));
  uint32_t prefix = kmax & pmask, need = (uint32_t)K;
  for (int shift = top; shift >= 0; shift -= 8) {
    sm.hist[tid] = 0u;
    __syncthreads();
    for (uint32_t i = tid; i < n; i += kBlock) {
      const uint32_t k = (uint32_t)(sm.buf.sk[i] >> 32);
      if ((k & pmask) == prefix) atomicAdd(&sm.hist[(k >> shift) & 255u], 1u);
    }
    __syncthreads();
    if (wv == 0) {
      // lane l holds bins 255-4l .. 252-4l (descending values)
      const int b0 = 255 - 4 * lane;
      const uint32_t h0 = sm.hist[b0], h1 = sm.hist[b0 - 1], h2 = sm.hist[b0 - 2],
                     h3 = sm.hist[b0 - 3];
      const uint32_t sum = h0 + h1 + h2 + h3;
      const uint32_t incl = wave_incl_scan_u32(sum);
      const uint32_t excl = incl - sum;
      if (excl < need && incl >= need) {
        uint32_t above = excl, bin, cnt;
        if (above + h0 >= need) {
          bin = b0;
          cnt = h0;
        } else if (above + h0 + h1 >= need) {
          above += h0;
          bin = b0 - 1;
          cnt = h1;
        } else if (above + h0 + h1 + h2 >= need) {
          above += h0 + h1;
          bin = b0 - 2;
          cnt = h2;
        } else {
          above += h0 + h1 + h2;
          bin = b0 - 3;
          cnt = h3;
        }
        sm.rbin = bin;
        sm.rneed = need - above;
        sm.rcnt = cnt;
      }
    }
    __syncthreads();
    prefix |= sm.rbin << shift;
    pmask |= 255u << shift;
    need = sm.rneed;
  }
  return prefix;
}

// ---- in-wave bitonic network: 64 keys, one per lane ------------------------------------
// Every lane exchange stays on the VALU: DPP quad_perm (xor 1, 2), DPP row
// shifts by 4 in both directions (xor 4), DPP row_ror:8 (xor 8), and gfx950's
// v_permlane16_swap / v_permlane32_swap (xor 16, 32), so a compare-exchange
// step never waits on the LDS crossbar.
// Lane-mask constants as per-lane conditions: the mask stays in an SGPR pair
// and feeds v_cndmask directly (no per-lane compare).
__device__ __forceinline__ bool lanes_in(uint64_t mask) { return __builtin_amdgcn_inverse_ballot_w64(mask); }

template <int J>
__device__ __forceinline__ uint32_t xor_lane32(uint32_t v) {
  if constexpr (J == 1) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
  } else if constexpr (J == 2) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
  } else if constexpr (J == 4) {
    const uint32_t up = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x104, 0xF, 0xF, false);  // lane + 4
    const uint32_t dn = (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x114, 0xF, 0xF, false);  // lane - 4
    return lanes_in(0xF0F0F0F0F0F0F0F0ull) ? dn : up;  // lanes with bit 4 set
  } else if constexpr (J == 8) {
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, false);
  } else if constexpr (J == 16) {
    // swap(v, v): first = rows {0,0,2,2}, second = rows {1,1,3,3}
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return lanes_in(0xFFFF0000FFFF0000ull) ? r[0] : r[1];  // lanes with bit 16 set
  } else {
    // swap(v, v): first = halves {lo,lo}, second = halves {hi,hi}
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return lanes_in(0xFFFFFFFF00000000ull) ? r[0] : r[1];  // lanes with bit 32 set
  }
}
template <int J>
__device__ __forceinline__ uint64_t xor_lane64(uint64_t v) {
  return ((uint64_t)xor_lane32<J>((uint32_t)(v >> 32)) << 32) | xor_lane32<J>((uint32_t)v);
}
__device__ __forceinline__ uint64_t reverse_lanes64(uint64_t v) {
  const int a = (63 - lane_id()) << 2;
  return ((uint64_t)(uint32_t)__builtin_amdgcn_ds_bpermute(a, (int)(uint32_t)(v >> 32)) << 32) |
         (uint32_t)__builtin_amdgcn_ds_bpermute(a, (int)(uint32_t)v);
}
// One compare-exchange step of the network: blocks of size K sorted in
// alternating directions (all in the final direction at K = 64), partners J
// lanes apart; ASC = ascending final order (lower lane keeps the smaller key).
// Lanes that keep the larger key of their pair in step (K, J).
constexpr uint64_t keep_max_lanes(int K, int J, bool ASC) {
  uint64_t m = 0;
  for (int l = 0; l < 64; ++l)
    if ((((l & J) == 0) == ((K >= 64) || ((l & K) == 0))) != ASC) m |= 1ull << l;
  return m;
}
// x stays where (x > partner) agrees with the lane's direction: the compare's
// lane mask XOR the constant mask of the keep-min lanes (one scalar XOR).
template <int K, int J, bool ASC>
__device__ __forceinline__ uint64_t cex(uint64_t x, uint64_t y) {
  constexpr uint64_t kmin = ~keep_max_lanes(K, J, ASC);
  return lanes_in(__builtin_amdgcn_ballot_w64(x > y) ^ kmin) ? x : y;
}
template <int K, int J, bool ASC = false>
__device__ __forceinline__ uint64_t bitonic_step(uint64_t x) {
  return cex<K, J, ASC>(x, xor_lane64<J>(x));
}
template <bool ASC = false>
__device__ __forceinline__ uint64_t wave_sort(uint64_t x) {
  x = bitonic_step<2, 1, ASC>(x);
  x = bitonic_step<4, 2, ASC>(x);  x = bitonic_step<4, 1, ASC>(x);
  x = bitonic_step<8, 4, ASC>(x);  x = bitonic_step<8, 2, ASC>(x);  x = bitonic_step<8, 1, ASC>(x);
  x = bitonic_step<16, 8, ASC>(x); x = bitonic_step<16, 4, ASC>(x); x = bitonic_step<16, 2, ASC>(x);
  x = bitonic_step<16, 1, ASC>(x);
  x = bitonic_step<32, 16, ASC>(x); x = bitonic_step<32, 8, ASC>(x); x = bitonic_step<32, 4, ASC>(x);
  x = bitonic_step<32, 2, ASC>(x);  x = bitonic_step<32, 1, ASC>(x);
  x = bitonic_step<64, 32, ASC>(x); x = bitonic_step<64, 16, ASC>(x); x = bitonic_step<64, 8, ASC>(x);
  x = bitonic_step<64, 4, ASC>(x);  x = bitonic_step<64, 2, ASC>(x);  x = bitonic_step<64, 1, ASC>(x);
  return x;
}
// A bitonic sequence of 64 keys to sorted order.
template <bool ASC = false>
__device__ __forceinline__ uint64_t wave_merge(uint64_t x) {
  x = bitonic_step<64, 32, ASC>(x); x = bitonic_step<64, 16, ASC>(x); x = bitonic_step<64, 8, ASC>(x);
  x = bitonic_step<64, 4, ASC>(x);  x = bitonic_step<64, 2, ASC>(x);  x = bitonic_step<64, 1, ASC>(x);
  return x;
}
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t x) { return wave_sort<false>(x); }
// Top 64 of two sorted 64-key lists held by one wave, one descending and one
// ascending: their lane-wise maximum is bitonic and holds the 64 largest.
template <bool ASC = false>
__device__ __forceinline__ uint64_t wave_top64(uint64_t a, uint64_t b_opposite) {
  return wave_merge<ASC>(a > b_opposite ? a : b_opposite);
}

// Two independent sorts interleaved step by step (x descending, y
// ascending): the second network's instructions fill the first one's
// latency, so both take about the time of one.
template <int K, int J>
__device__ __forceinline__ void bitonic_step2(uint64_t &x, uint64_t &y) {
  const uint64_t xo = xor_lane64<J>(x);
  const uint64_t yo = xor_lane64<J>(y);
  x = cex<K, J, false>(x, xo);
  y = cex<K, J, true>(y, yo);
}
__device__ __forceinline__ void wave_sort2(uint64_t &x, uint64_t &y) {
  bitonic_step2<2, 1>(x, y);
  bitonic_step2<4, 2>(x, y);  bitonic_step2<4, 1>(x, y);
  bitonic_step2<8, 4>(x, y);  bitonic_step2<8, 2>(x, y);  bitonic_step2<8, 1>(x, y);
  bitonic_step2<16, 8>(x, y); bitonic_step2<16, 4>(x, y); bitonic_step2<16, 2>(x, y);
  bitonic_step2<16, 1>(x, y);
  bitonic_step2<32, 16>(x, y); bitonic_step2<32, 8>(x, y); bitonic_step2<32, 4>(x, y);
  bitonic_step2<32, 2>(x, y);  bitonic_step2<32, 1>(x, y);
  bitonic_step2<64, 32>(x, y); bitonic_step2<64, 16>(x, y); bitonic_step2<64, 8>(x, y);
  bitonic_step2<64, 4>(x, y);  bitonic_step2<64, 2>(x, y);  bitonic_step2<64, 1>(x, y);
}

// Candidate slot i of the row (chunk i / kCandCap) holds a stored key.  Only
// the row's last chunk can be short, so every other chunk has regions of
// kCandCap / kWaves slots; `last_sh` is log2 of the last chunk's region size.
__device__ __forceinline__ bool slot_valid(int i, int S, int last_sh, const TopkSmem &sm) {
  const int c = i / kCandCap, e = i - c * kCandCap;
  const int sh = (c == S - 1) ? last_sh : 5;
  static_assert(kCandCap / kWaves == 32, "full-chunk regions hold 32 slots");
  return (uint32_t)(e & ((1 << sh) - 1)) < ((sm.ccount[c] >> (8 * (e >> sh))) & 0xFFu);
}
__device__ __forceinline__ int last_region_sh(int V, int S) {
  const int cap = wave_cap(V - (S - 1) * kChunk);
  return cap == 128 ? 7 : (cap == 64 ? 6 : 5);
}

// General merge: every stored candidate goes to LDS; theta = the K-th largest
// (radix select).  The stored set holds the row's top K (and every logit tied
// with theta) when theta >= tau_c for every chunk, since a logit that was not
// stored is < tau_c.  Chunks where that fails (or whose region overflowed)
// are re-read from HBM against theta, a lower bound of the row's K-th value,
// and theta is recomputed.  Returns false when the row must be replayed: LDS
// capacity exceeded, or the K-th value tied with a logit outside the set.
template <bool VEC>
__device__ __forceinline__ bool topk_merge_general(const CallParams &p, const float *__restrict__ L, int S,
                                                   const Cand *__restrict__ cand_row, TopkSmem &sm,
                                                   uint64_t (&kk)[kMergeSpec], bool reload) {
  const int V = p.vocab, K = p.top_k;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int nslots = S * kCandCap;
  const int last_sh = last_region_sh(V, S);
  if (tid == 0) sm.n = 0u;
  __syncthreads();
  uint32_t kmin = 0xFFFFFFFFu, kmax = 0u;
  for (int base = 0; base < nslots; base += kMergeSpec * kBlock) {
    if (base > 0 || reload) {
#pragma unroll
      for (int r = 0; r < kMergeSpec; ++r) {
        const int i = base + tid + r * kBlock;
        kk[r] = (i < nslots) ? xload(&cand_row[i]) : 0ull;
      }
    }
    uint32_t vm = 0u;
#pragma unroll
    for (int r = 0; r < kMergeSpec; ++r) {
      const int i = base + tid + r * kBlock;
      vm |= (i < nslots && slot_valid(i, S, last_sh, sm)) ? (1u << r) : 0u;
    }
#pragma unroll
    for (int r = 0; r < kMergeSpec; ++r) {
      if ((vm >> r) & 1u) {
        const uint32_t q = atomicAdd(&sm.n, 1u);
        if (q < (uint32_t)kMergeCap) sm.buf.sk[q] = kk[r];
        kmin = min(kmin, (uint32_t)(kk[r] >> 32));
        kmax = max(kmax, (uint32_t)(kk[r] >> 32));
      }
    }
  }
  kmin = wave_min_u32(kmin);
  kmax = wave_max_u32(kmax);
  if (lane == 0) {
    sm.cnt[2][wv] = kmin;
    sm.cnt[3][wv] = kmax;
  }
  __syncthreads();
  kmin = min(min(sm.cnt[2][0], sm.cnt[2][1]), min(sm.cnt[2][2], sm.cnt[2][3]));
  kmax = max(max(sm.cnt[3][0], sm.cnt[3][1]), max(sm.cnt[3][2], sm.cnt[3][3]));
  uint32_t n = sm.n;
  if (n > (uint32_t)kMergeCap) return false;
  uint32_t theta = (n >= (uint32_t)K) ? radix_kth(n, K, sm, kmin, kmax) : 0u;

  // chunks whose unstored logits could still reach theta
  for (int round = 0; round < 2; ++round) {
    int open = 0;
    for (int c = tid; c < S; c += kBlock) open |= (sm.ctau[c] > theta) ? 1 : 0;
    open = __syncthreads_or(open);
    if (!open) break;
    if (round == 1) return false;  // cannot happen: re-read chunks are closed
    // keep stored keys >= theta of closed chunks, then re-read open chunks
    uint64_t keep[kMergeCap / kBlock];
#pragma unroll
    for (int r = 0; r < kMergeCap / kBlock; ++r) {
      const uint32_t i = (uint32_t)(tid + r * kBlock);
      keep[r] = 0ull;
      if (i < n) {
        const uint64_t k = sm.buf.sk[i];
        const int c = (int)((~(uint32_t)k) / (uint32_t)kChunk);
        if ((uint32_t)(k >> 32) >= theta && sm.ctau[c] <= theta) keep[r] = k;
      }
    }
    __syncthreads();
    if (tid == 0) sm.n = 0u;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kMergeCap / kBlock; ++r) {
      if (keep[r]) {
        const uint32_t q = atomicAdd(&sm.n, 1u);
        sm.buf.sk[q] = keep[r];  // at most the previous n entries
      }
    }
    for (int c = 0; c < S; ++c) {
      if (sm.ctau[c] <= theta) continue;  // uniform
      const int c0 = c * kChunk, clen = min(kChunk, V - c0);
      if (VEC && clen == kChunk) {
#pragma nounroll
        for (int jb = 0; jb < kPerThread / 4; jb += 4) {  // four float4 loads in flight
          const int l0 = wv * kWaveSpan + jb * 256 + lane * 4;
          const f32x4 f0 = xload4(L + c0 + l0);
          const f32x4 f1 = xload4(L + c0 + l0 + 256);
          const f32x4 f2 = xload4(L + c0 + l0 + 512);
          const f32x4 f3 = xload4(L + c0 + l0 + 768);
          const f32x4 fs[4] = {f0, f1, f2, f3};
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float x = fs[jj][e];
              if (ord_key(x) >= theta) {
                const uint32_t q = atomicAdd(&sm.n, 1u);
                if (q < (uint32_t)kMergeCap)
                  sm.buf.sk[q] = ((uint64_t)ord_key(x) << 32) |
                                 (uint32_t)(~(uint32_t)(c0 + l0 + jj * 256 + e));
              }
            }
          }
        }
      } else {
#pragma nounroll
        for (int i = 0; i < kPerThread; ++i) {
          const int local = chunk_pos(wv, lane, i);
          if (local < clen) {
            const float x = xloadf(&L[c0 + local]);
            if (ord_key(x) >= theta) {
              const uint32_t q = atomicAdd(&sm.n, 1u);
              if (q < (uint32_t)kMergeCap)
                sm.buf.sk[q] = ((uint64_t)ord_key(x) << 32) | (uint32_t)(~(uint32_t)(c0 + local));
            }
          }
        }
      }
    }
    __syncthreads();
    for (int c = tid; c < S; c += kBlock)
      if (sm.ctau[c] > theta) sm.ctau[c] = theta;  // now closed
    n = sm.n;
    if (n > (uint32_t)kMergeCap) return false;
    theta = radix_kth(n, K, sm, 0u, 0xFFFFFFFFu);
  }
  if (n < (uint32_t)K) return false;
  // `need` of the rcnt logits valued theta are in the top K
  if (sm.rcnt > sm.rneed) return false;  // the K-th value is tied outside the set
  if (tid == 0) sm.ngt = 0u;
  __syncthreads();
  for (uint32_t i = tid; i < n; i += kBlock) {
    const uint64_t k = sm.buf.sk[i];
    if ((uint32_t)(k >> 32) >= theta) {
      const uint32_t q = atomicAdd(&sm.ngt, 1u);
      if (q < (uint32_t)kKMax) sm.topsel[q] = k;
    }
  }
  __syncthreads();
  if (tid < K) {  // exactly K selected: rank by (value desc, index asc)
    const uint64_t key = sm.topsel[tid];
    int rank = 0;
    for (int j = 0; j < K; ++j) rank += (sm.topsel[j] > key) ? 1 : 0;
    sm.topkey[rank] = key;
  }
  if (tid == 0) sm.ntop = K;
  __syncthreads();
  return true;
}


// Fast merge for rows of at most kFastChunks chunks, with no block-wide
// compaction: every wave reads the chunk records itself (T = max tau_c) and
// filters the candidate slots of chunks wv, wv+4, ... (loaded in the same round
// trip as the records) against T into its own LDS list.  Wave 0 then narrows
// the lists with one 8-bit radix digit to the at most 128 keys that can be in
// the top K, sorts them with two interleaved in-register networks and one
// bitonic merge.  With the fused penalty the table of history ids is built
// while the loads are in flight and the keys are penalised before the filter.
// Before the filter barrier every wave returns the same code: 0 when the row
// must be replayed (NaN/+inf), -1 when the general merge must run (a region
// overflowed).  After it, waves 1-3 return 2 (they learn wave 0's result
// through LDS after the caller's barrier) and wave 0 returns 1 when
// sm.topkey holds the row's top K (sm.ntop = -1 when the K-th value is tied
// with a stored key outside the set: replay) or -2 when the general merge
// must run (fewer than K keys reach T, a wave list would exceed kWaveCand, or
// more than 128 keys survive the digit).
constexpr int kFastChunks = 16;
constexpr int kWaveCand = 256;
static_assert(kFastChunks / kWaves * 2 <= 8 && kWaves * kWaveCand + 128 <= kMergeCap && kBlock == 256 &&
                  kWaveCand >= 128,
              "fast merge buffers");

__device__ __forceinline__ int topk_merge_waves(const CallParams &p, int S, const ChunkMeta *__restrict__ cm,
                                                const Cand *__restrict__ cand_row, TopkSmem &sm) {
  const int V = p.vocab, K = p.top_k;
  const int lane = lane_id(), wv = threadIdx.x >> 6;
  // one round trip: the records (lane c < S) and this wave's candidate slots
  const int lc = min(lane, S - 1);
  const uint64_t w0 = xload(&cm[lc].w);
  const uint64_t n01 = xload(reinterpret_cast<const uint64_t *>(&cm[lc].n[0]));
  const uint64_t n23 = xload(reinterpret_cast<const uint64_t *>(&cm[lc].n[2]));
  uint64_t kk[2 * (kFastChunks / kWaves)];
#pragma unroll
  for (int j = 0; j < kFastChunks / kWaves; ++j) {  // unconditional (clamped): precise waits
    const int c = min(wv + kWaves * j, S - 1);
    kk[2 * j] = xload(&cand_row[c * kCandCap + 2 * lane]);
    kk[2 * j + 1] = xload(&cand_row[c * kCandCap + 2 * lane + 1]);
  }
  const uint32_t cap = (lane < S) ? (uint32_t)wave_cap(min(kChunk, V - lane * kChunk)) : 0u;
  const uint32_t n0 = (uint32_t)n01, n1 = (uint32_t)(n01 >> 32), n2 = (uint32_t)n23,
                 n3 = (uint32_t)(n23 >> 32);
  const bool ovf = n0 > cap || n1 > cap || n2 > cap || n3 > cap;
  const uint32_t counts = min(n0, cap) | (min(n1, cap) << 8) | (min(n2, cap) << 16) | (min(n3, cap) << 24);
  const uint32_t tau = (lane < S) ? (ovf ? 0xFFFFFFFFu : (uint32_t)w0) : 0u;
  const uint32_t T = wave_max_u32(tau);
  const uint32_t fl = wave_or_u32((lane < S) ? (uint32_t)(w0 >> 32) : 0u);
  if (fl) return 0;                  // the same in every wave
  if (T == 0xFFFFFFFFu) return -1;

  // keys >= T of this wave's chunks, compacted by ballot into its LDS list
  const uint64_t thr = (uint64_t)T << 32;
  uint32_t okm = 0u;  // bit 2j+e: slot holds a stored key >= T
#pragma unroll
  for (int j = 0; j < kFastChunks / kWaves; ++j) {
    const int c = wv + kWaves * j;
    if (c < S) {  // uniform
      const uint32_t cnt = readlane32(counts, c);
      const uint32_t ccap = (uint32_t)wave_cap(min(kChunk, V - c * kChunk));
      const int sh = ccap == 128u ? 7 : (ccap == 64u ? 6 : 5);
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint32_t slot = 2u * (uint32_t)lane + (uint32_t)e;
        const uint32_t have = (cnt >> (8 * (slot >> sh))) & 0xFFu;
        okm |= ((slot & (ccap - 1u)) < have && kk[2 * j + e] >= thr) ? (1u << (2 * j + e)) : 0u;
      }
    }
  }
  uint64_t *wl = sm.buf.sk + wv * kWaveCand;
  uint32_t nw = 0u;
#pragma unroll
  for (int j = 0; j < kFastChunks / kWaves; ++j) {
    if (wv + kWaves * j >= S) break;  // uniform
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const bool ok = (okm >> (2 * j + e)) & 1u;
      const uint64_t b = __ballot(ok);
      const uint32_t q = nw + lane_rank(b);
      if (ok && q < (uint32_t)kWaveCand) wl[q] = kk[2 * j + e];
      nw += (uint32_t)__popcll(b);
    }
  }
  // The wave's list back in registers, entry lane and 64 + lane (the same
  // wave wrote it: LDS order suffices).  With the penalty, a key whose index
  // is a history id gets its penalised value; one that falls below T is no
  // longer live (it cannot be in the top K: at least K keys stay >= T, or the
  // general merge runs).
  const uint32_t nl = min(nw, 128u);
  const uint64_t e0 = ((uint32_t)lane < nl) ? wl[lane] : 0ull;
  const uint64_t e1 = (64u + (uint32_t)lane < nl) ? wl[64 + lane] : 0ull;
  const bool live0 = (uint32_t)lane < nl && e0 >= thr;
  const bool live1 = 64u + (uint32_t)lane < nl && e1 >= thr;
  const uint32_t vmax_k = wave_max_u32(max(live0 ? (uint32_t)(e0 >> 32) : 0u, live1 ? (uint32_t)(e1 >> 32) : 0u));
  const uint32_t live = (uint32_t)__popcll(__ballot(live0)) + (uint32_t)__popcll(__ballot(live1));
  if (lane == 0) {
    sm.cnt[0][wv] = nw;
    sm.cnt[1][wv] = vmax_k;
    sm.cnt[2][wv] = live;
  }
  sm.hist[threadIdx.x] = 0u;  // kBlock == 256 bins
  if (threadIdx.x == 0) sm.n = 0u;
  __syncthreads();
  // Every wave from here (same values, same branches): one radix digit (the
  // highest bits in which T and the largest key differ; the bits above are
  // common to every key >= T) narrows the nf keys to the m that can be in the
  // top K: every key in bins above the bin holding the K-th key, and that bin.
  uint32_t nf = 0u, kmax = 0u;
  bool big = false;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    nf += sm.cnt[2][w];
    kmax = max(kmax, sm.cnt[1][w]);
    big = big || sm.cnt[0][w] > 128u;
  }
  if (big || nf < (uint32_t)K || kmax == T) return -1;
  const int shift = (31 - __clz((int)(T ^ kmax))) & ~7;
  const uint32_t d0 = (uint32_t)(e0 >> (32 + shift)) & 255u, d1 = (uint32_t)(e1 >> (32 + shift)) & 255u;
  if (live0) atomicAdd(&sm.hist[d0], 1u);
  if (live1) atomicAdd(&sm.hist[d1], 1u);
  __syncthreads();
  // bins from the top: lane l holds bins 255-4l .. 252-4l
  const int b0 = 255 - 4 * lane;
  const uint32_t h0 = sm.hist[b0], h1 = sm.hist[b0 - 1], h2 = sm.hist[b0 - 2], h3 = sm.hist[b0 - 3];
  const uint32_t incl = wave_incl_scan_u32(h0 + h1 + h2 + h3);
  const uint32_t excl = incl - (h0 + h1 + h2 + h3);
  // first lane whose running count reaches K, then the bin inside it
  const uint64_t reach = __ballot(incl >= (uint32_t)K);
  const int ls = __ffsll((unsigned long long)reach) - 1;  // reach != 0: nf >= K
  uint32_t bstar = 0u, m = 0u;
  {
    const uint32_t e0s = readlane32(excl, ls);
    const uint32_t g0 = readlane32(h0, ls), g1 = readlane32(h1, ls), g2 = readlane32(h2, ls),
                   g3 = readlane32(h3, ls);
    const uint32_t bb = 255u - 4u * (uint32_t)ls;
    if (e0s + g0 >= (uint32_t)K) { bstar = bb; m = e0s + g0; }
    else if (e0s + g0 + g1 >= (uint32_t)K) { bstar = bb - 1u; m = e0s + g0 + g1; }
    else if (e0s + g0 + g1 + g2 >= (uint32_t)K) { bstar = bb - 2u; m = e0s + g0 + g1 + g2; }
    else { bstar = bb - 3u; m = e0s + g0 + g1 + g2 + g3; }
  }
  if (m > 128u) return -1;
  // each wave's keys with digit >= bstar go to sel (offset by an LDS counter);
  // the largest value key below them is kept per wave
  uint64_t *sel = sm.buf.sk + kWaves * kWaveCand;
  const bool in0 = live0 && d0 >= bstar, in1 = live1 && d1 >= bstar;
  const uint64_t bm0 = __ballot(in0), bm1 = __ballot(in1);
  const uint32_t cw0 = (uint32_t)__popcll(bm0);
  uint32_t off = 0u;
  if (lane == 0) off = atomicAdd(&sm.n, cw0 + (uint32_t)__popcll(bm1));
  off = readlane32(off, 0);
  if (in0) sel[off + lane_rank(bm0)] = e0;
  if (in1) sel[off + cw0 + lane_rank(bm1)] = e1;
  const uint32_t bw = wave_max_u32(max((live0 && !in0) ? (uint32_t)(e0 >> 32) : 0u,
                                       (live1 && !in1) ? (uint32_t)(e1 >> 32) : 0u));
  if (lane == 0) sm.cnt[3][wv] = bw;
  __syncthreads();
  // wave 0 sorts sel[0, 64) descending, wave 1 sorts sel[64, 128) ascending
  // (back into place)
  uint64_t x = 0ull;
  if (wv == 0) {
    x = wave_sort<false>(((uint32_t)lane < m) ? sel[lane] : 0ull);
  } else if (wv == 1) {
    const uint64_t y = wave_sort<true>((64u + (uint32_t)lane < m) ? sel[64 + lane] : 0ull);
    sel[64 + lane] = y;
  }
  __syncthreads();
  if (wv != 0) return 2;  // waves 1..3 wait at the final barrier of the caller
  const uint32_t below = max(max(sm.cnt[3][0], sm.cnt[3][1]), max(sm.cnt[3][2], sm.cnt[3][3]));
  const uint64_t y = sel[64 + lane];
  const uint64_t lo = x > y ? y : x;
  x = wave_merge<false>(x > y ? x : y);
  // The reference keeps the top K; if the K-th value is shared by a stored
  // key outside them (the (K+1)-th largest), which tied logits it keeps
  // depends on its slot order.
  const uint32_t vk = (uint32_t)(readlane64(x, K - 1) >> 32);
  uint32_t nextv;
  if ((uint32_t)K < m)
    nextv = (K < 64) ? (uint32_t)(readlane64(x, K) >> 32) : (uint32_t)(wave_max_u64(lo) >> 32);
  else
    nextv = below;
  if (lane < K) sm.topkey[lane] = x;
  if (lane == 0) sm.ntop = (nextv == vk) ? -1 : K;
  return 1;
}


// Merge (the last workgroup of the row).  One round trip loads the chunk
// records and, speculatively, the first kMergeSpec * kBlock candidate slots.
// Rows holding NaN or +inf are replayed.  With T = max_c tau_c: every logit
// >= T was stored (a logit that was not is < tau_c <= T), so when at least K
// of the stored keys reach T -- and at most 512, which holds for all but
// pathological rows -- the top K are the K largest of them: each wave
// bitonic-sorts 64 (or 2 x 64) of them, and the four sorted lists are merged
// pairwise.  Otherwise, or when a wave's region overflowed, the general merge
// runs.  Returns false when the row must be replayed.
template <bool VEC>
__device__ __forceinline__ bool topk_merge(const CallParams &p, const float *__restrict__ L, int S,
                                           const ChunkMeta *__restrict__ cm,
                                           const Cand *__restrict__ cand_row, TopkSmem &sm) {
  const int V = p.vocab, K = p.top_k;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int nslots = S * kCandCap;
  uint32_t fl = 0u, tmx = 0u;
  for (int c = tid; c < S; c += kBlock) {
    const uint64_t w0 = xload(&cm[c].w);
    const uint64_t n01 = xload(reinterpret_cast<const uint64_t *>(&cm[c].n[0]));
    const uint64_t n23 = xload(reinterpret_cast<const uint64_t *>(&cm[c].n[2]));
    const uint32_t cap = (uint32_t)wave_cap(min(kChunk, V - c * kChunk));
    const uint32_t n0 = (uint32_t)n01, n1 = (uint32_t)(n01 >> 32), n2 = (uint32_t)n23,
                   n3 = (uint32_t)(n23 >> 32);
    const bool ovf = n0 > cap || n1 > cap || n2 > cap || n3 > cap;
    sm.ccount[c] = min(n0, cap) | (min(n1, cap) << 8) | (min(n2, cap) << 16) | (min(n3, cap) << 24);
    const uint32_t tau = ovf ? 0xFFFFFFFFu : (uint32_t)w0;  // an overflowed chunk is "open"
    sm.ctau[c] = tau;
    tmx = max(tmx, tau);
    fl |= (uint32_t)(w0 >> 32);
  }
  uint64_t kk[kMergeSpec];
#pragma unroll
  for (int r = 0; r < kMergeSpec; ++r) {
    const int i = tid + r * kBlock;
    kk[r] = (i < nslots) ? xload(&cand_row[i]) : 0ull;
  }
  fl = wave_or_u32(fl);
  tmx = wave_max_u32(tmx);
  if (lane == 0) {
    sm.cnt[1][wv] = fl;
    sm.cnt[2][wv] = tmx;
  }
  __syncthreads();
  fl = sm.cnt[1][0] | sm.cnt[1][1] | sm.cnt[1][2] | sm.cnt[1][3];
  tmx = max(max(sm.cnt[2][0], sm.cnt[2][1]), max(sm.cnt[2][2], sm.cnt[2][3]));
  if (fl) return false;
  if (tmx == 0xFFFFFFFFu) return topk_merge_general<VEC>(p, L, S, cand_row, sm, kk, false);

  // keys >= T, compacted by a block-wide exclusive scan
  const uint64_t thr = (uint64_t)tmx << 32;
  const int last_sh = last_region_sh(V, S);
  uint32_t nf = 0u;
  for (int base = 0; base < nslots; base += kMergeSpec * kBlock) {
    if (base > 0) {
#pragma unroll
      for (int r = 0; r < kMergeSpec; ++r) {
        const int i = base + tid + r * kBlock;
        kk[r] = (i < nslots) ? xload(&cand_row[i]) : 0ull;
      }
    }
    uint32_t vb = 0u, m = 0u;
#pragma unroll
    for (int r = 0; r < kMergeSpec; ++r) {
      const int i = base + tid + r * kBlock;
      vb |= (i < nslots && kk[r] >= thr && slot_valid(i, S, last_sh, sm)) ? (1u << r) : 0u;
    }
    m = (uint32_t)__popc(vb);
    const uint32_t incl = wave_incl_scan_u32(m);
    if (lane == 63) sm.wtot[wv] = incl;
    __syncthreads();
    uint32_t off = nf + incl - m, total = 0u;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      if (w < wv) off += sm.wtot[w];
      total += sm.wtot[w];
    }
#pragma unroll
    for (int r = 0; r < kMergeSpec; ++r) {
      if ((vb >> r) & 1u) {
        if (off < (uint32_t)kMergeTop) sm.buf.sk[off] = kk[r];
        ++off;
      }
    }
    nf += total;
    __syncthreads();
  }
  if (nf < (uint32_t)K || nf > (uint32_t)kMergeTop)
    return topk_merge_general<VEC>(p, L, S, cand_row, sm, kk, nslots > kMergeSpec * kBlock);

  // top 64 of the nf <= 512 keys
  uint64_t *R = sm.buf.sk + kMergeTop;  // four sorted lists of 64
  const uint32_t i0 = (uint32_t)(wv * 64 + lane);
  uint64_t a = wave_sort_desc(i0 < nf ? sm.buf.sk[i0] : 0ull);
  if (nf > 256u) {
    const uint64_t b = wave_sort_desc(i0 + 256u < nf ? sm.buf.sk[i0 + 256u] : 0ull);
    a = wave_top64(a, reverse_lanes64(b));
  }
  R[i0] = a;
  __syncthreads();
  if (wv == 0 || wv == 2) {
    a = wave_top64(a, R[(wv + 1) * 64 + 63 - lane]);
    R[i0] = a;
  }
  __syncthreads();
  if (wv == 0) {
    a = wave_top64(a, R[2 * 64 + 63 - lane]);
    // The reference keeps the top K; if the K-th value is shared by a stored
    // key outside them, which tied logits it keeps depends on its slot order.
    const uint32_t vk = (uint32_t)(readlane64(a, K - 1) >> 32);
    const uint32_t inset = (uint32_t)__popcll(__ballot(lane < K && (uint32_t)(a >> 32) == vk));
    uint32_t tied = 0u;
    for (uint32_t j0 = 0u; j0 < nf; j0 += 64u) {
      const uint32_t j = j0 + (uint32_t)lane;
      tied += (uint32_t)__popcll(__ballot(j < nf && (uint32_t)(sm.buf.sk[j] >> 32) == vk));
    }
    if (lane < K) sm.topkey[lane] = a;
    if (lane == 0) sm.ntop = (tied > inset) ? -1 : K;
  }
  __syncthreads();
  return sm.ntop == K;
}

// Fast finish over the sorted top-K.  With Top-P < 1 the reference draws in
// the stable descending order of q (Sampler.pas:412-459); sorting by value
// gives that order up to permutations inside groups of equal q, which only
// matter if the Top-P cut splits such a group or the draw lands in one -- those
// rows (and Top-P >= 1, NaN/inf, non-positive invT) are replayed.  When every
// non-zero q is within 2^22 of the largest, every fp64 partial sum of q is
// exact, so wave-parallel scans give the reference's sums bit for bit;
// otherwise the sums are accumulated sequentially in the draw order as the
// reference does, with the initial sum S (slot order in the reference) taken
// in value order (equal up to a few ulp).
__device__ __forceinline__ void topk_fast(const CallParams &p, int row, TopkSmem &sm) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int K = p.top_k;
  if (tid < 64) {
    bool elig = (p.top_p < 1.0f) && (p.inv_t > 0.0f) && (p.inv_t <= 3.4028235e38f) && (sm.ntop == K);
    const bool act = lane < K;
    const uint64_t sk = act ? sm.topkey[lane] : 0ull;
    const float val = key_float((uint32_t)(sk >> 32));
    const int32_t idx = (int32_t)(~(uint32_t)sk);
    const float M = key_float((uint32_t)(sm.topkey[0] >> 32));
    float q = 0.0f;
    if (act) q = (float)exp(((double)val - (double)M) * (double)p.inv_t);
    const bool bad = act && !(q <= 3.4028235e38f);
    elig = elig && (__ballot(bad) == 0ull);
    const float qmax = __uint_as_float(readlane32(__float_as_uint(q), 0));
    const float qfloor = ldexpf(qmax, -22);
    const bool exact = __ballot(act && !(q == 0.0f || q >= qfloor)) == 0ull;
    if (elig && exact) {
      if (p.min_p > 0.0f) {  // Min-P (:393-410): Qmax = q[0]
        const float thr = qmax * p.min_p;
        if (q < thr) q = 0.0f;
      }
      const double incl = wave_incl_scan_f64((double)q);
      const double S = __longlong_as_double((long long)readlane64((uint64_t)__double_as_longlong(incl), 63));
      const double target = (double)p.top_p * S;
      const bool kept = act && ((incl - (double)q) < target) && q > 0.0f;  // Top-P (:431-444)
      const float qk = kept ? q : 0.0f;
      const double c2 = wave_incl_scan_f64((double)qk);
      const double S2 = __longlong_as_double((long long)readlane64((uint64_t)__double_as_longlong(c2), 63));
      const double t = (double)sm.uval * S2;  // draw (:447-459)
      const uint64_t hit = __ballot(act && c2 > t);
      const int pos = hit ? (__ffsll((unsigned long long)hit) - 1) : -1;
      const uint64_t dropm = __ballot(act && !kept);
      const int cut = dropm ? (__ffsll((unsigned long long)dropm) - 1) : K;
      const float qprev = __shfl_up(q, 1), qnext = __shfl_down(q, 1);
      const bool split = (lane == cut) && cut > 0 && q > 0.0f && q == qprev;
      const bool tie = (lane == pos) && ((lane > 0 && qprev == q) || (lane + 1 < K && qnext == q));
      const bool amb = (pos < 0) || (__ballot(split || tie) != 0ull);
      const int32_t tok = (int32_t)readlane32((uint32_t)idx, pos < 0 ? 0 : pos);
      if (!amb) {
        if (lane == 0) {
          sm.token = tok;
          sm.rowflags = kRowTopkFast;
          sm.replay = 0;
        }
        if (act) {
          const int64_t o = (int64_t)row * p.out.topk_stride + lane;
          if (p.out.topk_idx) p.out.topk_idx[o] = idx;
          if (p.out.topk_prob) p.out.topk_prob[o] = (float)((double)qk / S2);
        }
      } else if (lane == 0) {
        sm.replay = 1;
      }
      if (lane == 0) sm.qnan = 0;  // parallel finish done
    } else {
      if (act) {
        sm.q[lane] = q;
        sm.i_ord[lane] = idx;
      }
      if (lane == 0) {
        sm.replay = elig ? 0 : 1;
        sm.qnan = 1;  // sequential finish pending
      }
    }
  }
  __syncthreads();
  if (!sm.qnan) return;
  if (tid == 0 && !sm.replay) {
    // Min-P (:393-410): Qmax is q[0]; zero q < fl32(Qmax * MinP)
    double S = 0.0;
    for (int k = 0; k < K; ++k) S = S + (double)sm.q[k];
    if (p.min_p > 0.0f) {
      const float thr = sm.q[0] * p.min_p;
      S = 0.0;
      for (int k = 0; k < K; ++k) {
        if (sm.q[k] < thr)
          sm.q[k] = 0.0f;
        else
          S = S + (double)sm.q[k];
      }
    }
    // Top-P (:431-444).  S was summed in value order; the reference sums in
    // slot order.  Each order's rounded sum of K non-negative terms is within
    // (K-1) 2^-53 S of the exact sum, so the two targets differ by at most
    // tol; a running sum C (summed in the draw order, as the reference does)
    // within tol of the target could fall on either side of the reference's:
    // such rows take the exact path.
    const double target = (double)p.top_p * S;
    const double tol = (double)p.top_p * (double)(2 * K) * 0x1p-53 * S + 0x1p-51 * target;
    bool near_cut = false;
    double C = 0.0, S2 = 0.0;
    int cut = K;
    for (int k = 0; k < K; ++k) {
      const float qk = sm.q[k];
      if (qk > 0.0f && fabs(C - target) <= tol) near_cut = true;
      if (C < target && qk > 0.0f) {
        C = C + (double)qk;
        S2 = S2 + (double)qk;
        sm.q_ord[k] = qk;
      } else {
        if (cut == K) cut = k;
        sm.q_ord[k] = 0.0f;
      }
    }
    bool amb = near_cut || ((cut > 0 && cut < K) && sm.q[cut] > 0.0f && sm.q[cut] == sm.q[cut - 1]);
    // draw (:447-459)
    const double t = (double)sm.uval * S2;
    C = 0.0;
    int pos = -1;
    for (int k = 0; k < K; ++k) {
      C = C + (double)sm.q_ord[k];
      if (C > t) {
        pos = k;
        break;
      }
    }
    if (pos < 0) {
      amb = true;  // S' = 0: the fallback picks by slot order
    } else {
      const float qp = sm.q[pos];
      amb = amb || (pos > 0 && sm.q[pos - 1] == qp) || (pos + 1 < K && sm.q[pos + 1] == qp);
    }
    if (amb) {
      sm.replay = 1;
    } else {
      sm.token = sm.i_ord[pos];
      sm.rowflags = kRowTopkFast;
      sm.S = S2;
    }
  }
  __syncthreads();
  if (!sm.replay && tid < K) {
    const int64_t o = (int64_t)row * p.out.topk_stride + tid;
    if (p.out.topk_idx) p.out.topk_idx[o] = sm.i_ord[tid];
    if (p.out.topk_prob) p.out.topk_prob[o] = (float)((double)sm.q_ord[tid] / sm.S);
  }
}

// ---- Exact path: the reference's min-buffer (Sampler.pas:341-383) replayed over
// the logits that can enter it, then the slot-order finish (:385-459).
//
// The buffer (K <= 64) lives in wave 0, one entry per lane, sorted ascending:
//   entry = slot_key(value) << 32 | slot << 22 | index
// so lane 0 holds the reference's "first strict minimum" (smallest value,
// then lowest slot; NaN sorts above +inf and is never the minimum).  A logit
// x enters iff x > that minimum: it takes the minimum's slot, the minimum
// leaves (lane 0), and x is inserted at its rank among the rest (lanes
// shift down by one): lane l takes entry l + 1 if that is below x, else x if
// its own entry is, else keeps its own (a DPP lane shift and two 64-bit
// compares, no trip through the scalar unit).
//
// Only logits above the current minimum can enter, and the minimum only
// rises, so the chunks are walked in index order: a chunk whose stored
// candidates include every logit above the current minimum (its threshold
// tau_c is at most one key above it and no region overflowed) feeds those,
// sorted by index; any other chunk (always chunk 0) is re-read and fed one
// 1024-logit group at a time, each group filtered against the minimum left
// by the previous one.
__device__ __forceinline__ uint64_t wave_shl1_64(uint64_t v) {  // lane l <- lane l + 1, lane 63 <- ~0
  const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)(uint32_t)v, 0x130, 0xF, 0xF, false);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(-1, (int)(uint32_t)(v >> 32), 0x130, 0xF, 0xF, false);
  return ((uint64_t)hi << 32) | lo;
}
constexpr uint32_t kXbIdxMask = (1u << 22) - 1u;
static_assert(kMaxChunks * kChunk <= (1 << 22) && kKMax <= 64, "buffer entry packing");

struct MinBuf {
  uint64_t b;      // lane l < K: the l-th smallest entry; lanes >= K: ~0
  uint32_t mkey;   // slot_key of the minimum (lane 0)
  uint32_t mslot;  // its slot
};
__device__ __forceinline__ void mb_refresh(MinBuf &m) {
  const uint64_t b0 = readlane64(m.b, 0);
  m.mkey = (uint32_t)(b0 >> 32);
  m.mslot = ((uint32_t)b0 >> 22) & 63u;
}
// Logit (key xk, index xi) enters: it replaces the minimum in the minimum's slot.
__device__ __forceinline__ void mb_enter(MinBuf &m, uint32_t xk, uint32_t xi) {
  // entries are distinct (each holds its slot) and nk is above lane 0's
  const uint64_t sh = wave_shl1_64(m.b);
  const uint64_t nk = ((uint64_t)xk << 32) | ((uint64_t)m.mslot << 22) | xi;
  m.b = (sh < nk) ? sh : ((m.b < nk) ? nk : m.b);
  mb_refresh(m);
}
// One logit per lane, lane order = index order; `has` marks real entries.
// Keys are ord_key of non-NaN logits (NaN never enters: Sampler.pas:369).
__device__ __forceinline__ void mb_feed(MinBuf &m, bool has, uint32_t ck, uint32_t ci) {
  uint64_t pend = __ballot(has && ck > m.mkey);
  while (pend) {
    const int src = __ffsll((unsigned long long)pend) - 1;
    mb_enter(m, readlane32(ck, src), readlane32(ci, src));
    pend &= ~(1ull << src);
    pend &= __ballot(ck > m.mkey);
  }
}

// Re-reads chunk [c0, c0 + clen) of L into v (interleaved layout); rows the
// fused penalty wrote in place are read past the caches.
template <bool VEC>
__device__ __forceinline__ void reload_chunk(const float *L, int c0, int clen, bool penalised,
                                             float (&v)[kPerThread]) {
  const int lane = lane_id(), wv = threadIdx.x >> 6;
  if (VEC) {
#pragma unroll
    for (int j = 0; j < kPerThread / 4; ++j) {
      const int local = chunk_pos(wv, lane, 4 * j);
      const float *q = L + c0 + (local < clen ? local : 0);
      const f32x4 f = penalised ? xload4(q) : __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(q));
      v[4 * j + 0] = f[0];
      v[4 * j + 1] = f[1];
      v[4 * j + 2] = f[2];
      v[4 * j + 3] = f[3];
    }
  } else {
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      const int local = chunk_pos(wv, lane, i);
      const float *q = L + c0 + (local < clen ? local : 0);
      v[i] = penalised ? xloadf(q) : *q;
    }
  }
}

// WHOLE (the launch of its own): the row's uniform is drawn from `rp` once
// the buffer is final, so the state's load is in flight during the replay.
template <bool VEC, bool WHOLE = false>
__device__ __forceinline__ void topk_exact(const CallParams &p, int row, const ChunkMeta *__restrict__ cm,
                                           const Cand *__restrict__ cand_row, TopkSmem &sm, RngPre rp = {}) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int K = p.top_k, V = p.vocab, S = p.nchunks;
  const float *L = p.logits + (int64_t)row * p.stride;
  const bool pen = p.fuse_penalty != 0;
  float v[kPerThread];
  // WHOLE and VEC: the chunk whose logits v holds or has in flight: chunk 0
  // (always re-read) goes out with the records, and the next chunk is loaded
  // while wave 0 feeds the current one's list (v is free by then); the
  // scalar form would keep 64 loads in flight and spill
  constexpr bool kAhead = WHOLE && VEC;
  int vc = -1;
  if (kAhead) {
    reload_chunk<VEC>(L, 0, min(kChunk, V), pen, v);
    vc = 0;
  }

  // chunk records: stored counts and thresholds (an overflowed chunk is "open")
  for (int c = tid; c < S; c += kBlock) {
    const uint64_t w0 = xload(&cm[c].w);
    const uint64_t n01 = xload(reinterpret_cast<const uint64_t *>(&cm[c].n[0]));
    const uint64_t n23 = xload(reinterpret_cast<const uint64_t *>(&cm[c].n[2]));
    const uint32_t cap = (uint32_t)wave_cap(min(kChunk, V - c * kChunk));
    const uint32_t n0 = (uint32_t)n01, n1 = (uint32_t)(n01 >> 32), n2 = (uint32_t)n23,
                   n3 = (uint32_t)(n23 >> 32);
    const bool ovf = n0 > cap || n1 > cap || n2 > cap || n3 > cap;
    sm.ccount[c] = min(n0, cap) | (min(n1, cap) << 8) | (min(n2, cap) << 16) | (min(n3, cap) << 24);
    sm.ctau[c] = ovf ? 0xFFFFFFFFu : (uint32_t)w0;
  }
  MinBuf mb{~0ull, 0xFFFFFFFFu, 0u};
  uint64_t *list = sm.buf.sk;  // one group's candidates in index order: ord_key << 32 | index
  uint64_t pk0 = 0ull, pk1 = 0ull;  // wave 0: the next chunk's candidate slots, loaded ahead
  int pc = -1;                      // the chunk they belong to
  for (int c = 0; c < S; ++c) {
    const int c0 = c * kChunk, clen = min(kChunk, V - c0);
    __syncthreads();  // sm.ctau / the previous chunk's list and sm.xmkey
    const uint32_t mk = (c == 0) ? 0u : sm.xmkey;
    if (c > 0 && (sm.xfrozen || mk == 0xFFFFFFFFu)) break;  // nothing can enter any more
    const uint32_t tc = sm.ctau[c];
    if (WHOLE && c > 0 && tc <= mk + 1u) {
      // a run of chunks whose stored candidates hold every logit above the
      // minimum: all of theirs above it in one index-sorted list (the minimum
      // only rises, so a logit at or below it now never enters later)
      int ce = c;
      while (ce + 1 < S && ce + 1 < c + 12 && sm.ctau[ce + 1] <= mk + 1u) ++ce;  // uniform
      if (ce > c) {
        if (tid == 0) sm.n = 0u;
        __syncthreads();
        const int nitems = (ce - c + 1) * kCandCap;
        uint64_t kk[6];
        bool okk[6];
#pragma unroll
        for (int i = 0; i < 6; ++i) {  // every load in flight before any is used
          const int it = tid + kBlock * i;
          okk[i] = false;
          kk[i] = 0ull;
          if (it < nitems) {
            const int cc = c + it / kCandCap, sl = it % kCandCap;
            const uint32_t cap = (uint32_t)wave_cap(min(kChunk, V - cc * kChunk));
            const int sh = cap == 128u ? 7 : (cap == 64u ? 6 : 5);
            if (((uint32_t)sl & (cap - 1u)) < ((sm.ccount[cc] >> (8 * (sl >> sh))) & 0xFFu)) {
              kk[i] = xload(&cand_row[(int64_t)cc * kCandCap + sl]);
              okk[i] = true;
            }
          }
        }
#pragma unroll
        for (int i = 0; i < 6; ++i) {
          if (okk[i] && (uint32_t)(kk[i] >> 32) > mk) {
            const uint32_t q = atomicAdd(&sm.n, 1u);
            if (q < 128u) list[q] = ((uint64_t)(~(uint32_t)kk[i]) << 32) | (kk[i] >> 32);  // index << 32 | key
          }
        }
        __syncthreads();
        const uint32_t n = sm.n;
        if (n <= 128u) {  // uniform
          if (wv == 0) {
            uint64_t x[2] = {(uint32_t)lane < n ? list[lane] : ~0ull, (uint32_t)lane + 64u < n ? list[lane + 64] : ~0ull};
            wave_sort2(x[1], x[0]);  // x[1] descending, x[0] ascending
            const uint64_t lo = x[0] < x[1] ? x[0] : x[1], hi = x[0] < x[1] ? x[1] : x[0];
            x[0] = wave_merge<true>(lo);
            x[1] = wave_merge<true>(hi);
#pragma unroll
            for (int e = 0; e < 2; ++e) mb_feed(mb, x[e] != ~0ull, (uint32_t)x[e], (uint32_t)(x[e] >> 32));
            if (lane == 0) sm.xmkey = mb.mkey;
          }
          c = ce;
          continue;
        }
        // more than one list holds: chunk c alone, below
      }
    }
    if (c > 0 && tc <= mk + 1u) {
      // every logit above the minimum was stored: wave 0 feeds them by index
      if (wv == 0) {
        const Cand *cc = cand_row + (int64_t)c * kCandCap;
        const uint32_t cap = (uint32_t)wave_cap(clen);
        const int sh = cap == 128u ? 7 : (cap == 64u ? 6 : 5);
        const uint32_t cnt = sm.ccount[c];
        uint64_t raw[2];
        if (pc == c) {
          raw[0] = pk0;
          raw[1] = pk1;
        } else {
          raw[0] = xload(&cc[2 * lane]);
          raw[1] = xload(&cc[2 * lane + 1]);
        }
        if (c + 1 < S) {  // the next chunk's slots, in flight while this one is fed
          const Cand *cn = cand_row + (int64_t)(c + 1) * kCandCap;
          pk0 = xload(&cn[2 * lane]);
          pk1 = xload(&cn[2 * lane + 1]);
          pc = c + 1;
        }
        uint64_t x[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const uint32_t slot = 2u * (uint32_t)lane + (uint32_t)e;
          const uint64_t k = raw[e];
          const bool ok = (slot & (cap - 1u)) < ((cnt >> (8 * (slot >> sh))) & 0xFFu) &&
                          (uint32_t)(k >> 32) > mk;
          // sorted by index: index << 32 | key
          x[e] = ok ? (((uint64_t)(~(uint32_t)k) << 32) | (k >> 32)) : ~0ull;
        }
        if (__ballot(x[0] != ~0ull || x[1] != ~0ull)) {
          wave_sort2(x[1], x[0]);  // x[1] descending, x[0] ascending
          const uint64_t lo = x[0] < x[1] ? x[0] : x[1], hi = x[0] < x[1] ? x[1] : x[0];
          x[0] = wave_merge<true>(lo);
          x[1] = wave_merge<true>(hi);
#pragma unroll
          for (int e = 0; e < 2; ++e)
            mb_feed(mb, x[e] != ~0ull, (uint32_t)x[e], (uint32_t)(x[e] >> 32));
        }
        if (lane == 0) sm.xmkey = mb.mkey;
      }
      continue;
    }
    // re-read the chunk and feed it one 1024-logit group at a time
    if (vc != c) reload_chunk<VEC>(L, c0, clen, pen, v);
    if (WHOLE && c > 0) {
      // after chunk 0 the minimum rises slowly: the whole chunk in one list,
      // every logit above the minimum when the chunk starts, in index order
      // (per-thread counts of the 16 groups, four 16-bit fields per wave
      // scan), fed in index order
      const uint32_t m = mk;
      uint64_t hb = 0ull;  // bit 4j + e: logit e of the thread's group j passes
#pragma unroll
      for (int j = 0; j < kPerThread / 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int loc = j * 1024 + wv * 256 + lane * 4 + e;
          const float x = v[4 * j + e];
          if (loc < clen && x == x && ord_key(x) > m) hb |= 1ull << (4 * j + e);
        }
      uint64_t incl[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint64_t w = 0ull;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) w |= (uint64_t)__popcll((hb >> (16 * q + 4 * jj)) & 15ull) << (16 * jj);
        incl[q] = wave_scan<uint64_t>(w, 0ull, OpAddU64());
        if (lane == 63) sm.xw64[wv][q] = incl[q];
      }
      __syncthreads();
      uint32_t gbase = 0u;
      uint32_t off[kPerThread / 4];
#pragma unroll
      for (int j = 0; j < kPerThread / 4; ++j) {  // group j's offset: earlier groups, then earlier waves
        const int q = j >> 2, sh = 16 * (j & 3);
        uint32_t before = 0u, gt = 0u;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          const uint32_t f = (uint32_t)(sm.xw64[w][q] >> sh) & 0xFFFFu;
          before += (w < wv) ? f : 0u;
          gt += f;
        }
        off[j] = gbase + before + ((uint32_t)(incl[q] >> sh) & 0xFFFFu) - (uint32_t)__popcll((hb >> (4 * j)) & 15ull);
        gbase += gt;
      }
      const uint32_t total = gbase;
      if (total <= (uint32_t)kMergeCap) {  // uniform; a longer list goes group by group, below
#pragma unroll
        for (int j = 0; j < kPerThread / 4; ++j) {
          uint32_t o = off[j];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if ((hb >> (4 * j + e)) & 1ull)
              list[o++] = ((uint64_t)ord_key(v[4 * j + e]) << 32) | (uint32_t)(c0 + j * 1024 + wv * 256 + lane * 4 + e);
        }
        __syncthreads();
        if (kAhead && c + 1 < S && sm.ctau[c + 1] > mk + 1u) {  // likely re-read next
          reload_chunk<VEC>(L, c0 + kChunk, min(kChunk, V - c0 - kChunk), pen, v);
          vc = c + 1;
        }
        if (wv == 0) {
          for (uint32_t g = 0u; g < total; g += 64u) {
            const bool has = g + (uint32_t)lane < total;
            const uint64_t en = has ? list[g + lane] : 0ull;
            mb_feed(mb, has, (uint32_t)(en >> 32), (uint32_t)en);
          }
          if (lane == 0) sm.xmkey = mb.mkey;
        }
        continue;
      }
    }
    if (c == 0) {
      // the first K logits fill slots 0..K-1 (Sampler.pas:352-366); a NaN at
      // index 0 stays the minimum and nothing ever enters (:369)
      if (wv == 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (lane * 4 + e < kKMax) sm.q[lane * 4 + e] = v[e];
      }
      __syncthreads();
      if (wv == 0) {
        const float x = sm.q[lane];
        mb.b = (lane < K) ? (((uint64_t)slot_key(x) << 32) | ((uint64_t)lane << 22) | (uint32_t)lane) : ~0ull;
        mb.b = wave_sort<true>(mb.b);
        mb_refresh(mb);
        const float l0 = sm.q[0];
        if (lane == 0) {
          sm.xfrozen = (l0 != l0) ? 1 : 0;
          sm.xmkey = mb.mkey;
        }
      }
    }
    // unrolled: a register array indexed by a loop variable would live in scratch
#pragma unroll
    for (int j = 0; j < kPerThread / 4; ++j) {
      __syncthreads();  // sm.xmkey of the previous group; the list is free
      if (sm.xfrozen) break;
      const uint32_t m = sm.xmkey;
      if (m == 0xFFFFFFFFu) break;  // uniform
      const int base = j * 1024 + wv * 256 + lane * 4;
      float g4[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) g4[e] = v[4 * j + e];
      uint32_t bits = 0u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = g4[e];
        const int loc = base + e;
        const bool ok = loc < clen && (c0 + loc) >= K && x == x && ord_key(x) > m;
        bits |= ok ? (1u << e) : 0u;
      }
      const uint32_t cnt = (uint32_t)__popc(bits);
      const uint32_t incl = wave_incl_scan_u32(cnt);
      if (lane == 63) sm.xw[wv] = incl;
      __syncthreads();
      uint32_t off = incl - cnt, total = 0u;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        off += (w < wv) ? sm.xw[w] : 0u;
        total += sm.xw[w];
      }
      if (total == 0u) continue;  // uniform
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if ((bits >> e) & 1u) {
          list[off++] = ((uint64_t)ord_key(g4[e]) << 32) | (uint32_t)(c0 + base + e);
        }
      }
      __syncthreads();
      if (kAhead && j == kPerThread / 4 - 1 && c + 1 < S && sm.ctau[c + 1] > m + 1u) {  // likely re-read next
        reload_chunk<VEC>(L, c0 + kChunk, min(kChunk, V - c0 - kChunk), pen, v);
        vc = c + 1;
      }
      if (wv == 0) {
        for (uint32_t g = 0u; g < total; g += 64u) {
          const bool has = g + (uint32_t)lane < total;
          const uint64_t en = has ? list[g + lane] : 0ull;
          mb_feed(mb, has, (uint32_t)(en >> 32), (uint32_t)en);
        }
        if (lane == 0) sm.xmkey = mb.mkey;
      }
    }
  }
  __syncthreads();
  // slot order; the running maximum M (strict '>' from L[0]): NaN when L[0]
  // is NaN, else the largest non-NaN logit, which is in the buffer
  if (wv == 0) {
    const uint32_t key = (uint32_t)(mb.b >> 32);
    const float x = (key == 0xFFFFFFFFu) ? __builtin_nanf("") : key_float(key);
    if (lane < K) {
      const int s = (int)(((uint32_t)mb.b >> 22) & 63u);
      sm.slot_v[s] = x;
      sm.slot_i[s] = (int32_t)((uint32_t)mb.b & kXbIdxMask);
    }
    const float wm = wave_max_f32(lane < K ? x : __builtin_nanf(""));
    if (lane == 0) sm.wfmax[0] = wm;
    if (WHOLE) {
      RngVals rv = rng_unpack(rp);  // wave 0, every lane
      if (lane == 0) sm.uval = rng_draw(p.rng, row, rv);
    }
  }
  __syncthreads();
  const bool frozen = sm.xfrozen != 0;
  const float M = frozen ? __builtin_nanf("") : sm.wfmax[0];

  // softmax over the slots (:385-391)
  if (wv == 0) {
    float q = 0.0f;
    if (lane < K) {
      q = (float)exp(((double)sm.slot_v[lane] - (double)M) * (double)p.inv_t);
      sm.q[lane] = q;
    }
    const uint64_t nanm = __ballot(lane < K && q != q);
    if (lane == 0) {
      sm.qnan = nanm != 0ull;
      sm.xdone = 0;
    }
    // Top-P >= 1 (the draw walks the slots) with finite weights: when every
    // non-zero q is within 2^22 of the largest, every fp64 partial sum of
    // the <= 64 q is exact in any order, so wave scans give the slot-order
    // sums of :386-410 and :447-459 bit for bit (else lane 0 below)
    if (!(p.top_p < 1.0f) && nanm == 0ull) {
      const float qmax = wave_max_f32(lane < K ? q : 0.0f);
      if (p.min_p > 0.0f && lane < K && q < qmax * p.min_p) q = 0.0f;  // Min-P: Qmax = the largest q
      const float qfloor = ldexpf(qmax, -22);
      if (__ballot(lane < K && !(q == 0.0f || q >= qfloor)) == 0ull) {
        const double incl = wave_incl_scan_f64(lane < K ? (double)q : 0.0);
        const double S = __longlong_as_double((long long)readlane64((uint64_t)__double_as_longlong(incl), 63));
        const double t = (double)sm.uval * S;
        const uint64_t hit = __ballot(lane < K && incl > t);
        const int pos = hit ? (__ffsll((unsigned long long)hit) - 1) : K - 1;
        if (lane < K) {
          sm.q_ord[lane] = q;
          sm.i_ord[lane] = sm.slot_i[lane];
          sm.v_ord[lane] = sm.slot_v[lane];
        }
        if (lane == 0) {
          sm.token = sm.slot_i[pos];
          sm.rowflags = kRowTopkReplay | (hit ? 0u : kRowFallback);
          sm.S = S;
          sm.xdone = 1;
        }
      }
    }
  }
  __syncthreads();
  const bool xdone = sm.xdone != 0;
  // sums and Min-P in slot order (:386-410)
  if (tid == 0 && !xdone) {
    double S = 0.0;
    for (int k = 0; k < K; ++k) S = S + (double)sm.q[k];
    if (p.min_p > 0.0f) {
      float best = sm.q[0];
      for (int k = 1; k < K; ++k)
        if (sm.q[k] > best) best = sm.q[k];
      const float thr = best * p.min_p;
      S = 0.0;
      for (int k = 0; k < K; ++k) {
        if (sm.q[k] < thr)
          sm.q[k] = 0.0f;
        else
          S = S + (double)sm.q[k];
      }
    }
    sm.S = S;
  }
  __syncthreads();
  // draw order: stable descending sort when Top-P runs (:412-429)
  if (xdone) {
  } else if (p.top_p < 1.0f) {
    if (!sm.qnan) {
      if (wv == 0 && lane < K) {
        const float qk = sm.q[lane];
        int rank = 0;
        for (int j = 0; j < K; ++j) {
          const float qj = sm.q[j];
          rank += (qj > qk || (qj == qk && j < lane)) ? 1 : 0;
        }
        sm.q_ord[rank] = qk;
        sm.i_ord[rank] = sm.slot_i[lane];
        sm.v_ord[rank] = sm.slot_v[lane];
      }
    } else if (tid == 0) {
      for (int k = 0; k < K; ++k) {
        sm.q_ord[k] = sm.q[k];
        sm.i_ord[k] = sm.slot_i[k];
        sm.v_ord[k] = sm.slot_v[k];
      }
      for (int i = 1; i < K; ++i) {  // the reference's insertion sort, literally
        const float qv = sm.q_ord[i];
        const int32_t ti = sm.i_ord[i];
        const float tv = sm.v_ord[i];
        int j = i - 1;
        while (j >= 0 && sm.q_ord[j] < qv) {
          sm.q_ord[j + 1] = sm.q_ord[j];
          sm.i_ord[j + 1] = sm.i_ord[j];
          sm.v_ord[j + 1] = sm.v_ord[j];
          --j;
        }
        sm.q_ord[j + 1] = qv;
        sm.i_ord[j + 1] = ti;
        sm.v_ord[j + 1] = tv;
      }
    }
  } else if (wv == 0 && lane < K) {
    sm.q_ord[lane] = sm.q[lane];
    sm.i_ord[lane] = sm.slot_i[lane];
    sm.v_ord[lane] = sm.slot_v[lane];
  }
  __syncthreads();
  // Top-P cut (:431-444) and draw (:447-459)
  if (tid == 0 && !xdone) {
    double S = sm.S;
    if (p.top_p < 1.0f) {
      const double target = (double)p.top_p * S;
      double C = 0.0;
      S = 0.0;
      for (int k = 0; k < K; ++k) {
        if (C < target && sm.q_ord[k] > 0.0f) {
          C = C + (double)sm.q_ord[k];
          S = S + (double)sm.q_ord[k];
        } else {
          sm.q_ord[k] = 0.0f;
        }
      }
    }
    const double t = (double)sm.uval * S;
    double C = 0.0;
    int32_t tok = sm.i_ord[K - 1];
    uint32_t fl = kRowTopkReplay | kRowFallback;
    for (int k = 0; k < K; ++k) {
      C = C + (double)sm.q_ord[k];
      if (C > t) {
        tok = sm.i_ord[k];
        fl = kRowTopkReplay;
        break;
      }
    }
    if (sm.qnan || !(M == M)) fl |= kRowNan;
    sm.token = tok;
    sm.rowflags = fl;
    sm.S = S;
  }
  __syncthreads();
  if (wv == 0 && lane < K && (p.out.topk_idx || p.out.topk_prob)) {
    const uint32_t kk = slot_key(sm.v_ord[lane]);
    const int32_t ii = sm.i_ord[lane];
    int rank = 0;
    for (int j = 0; j < K; ++j) {
      const uint32_t kj = slot_key(sm.v_ord[j]);
      const int32_t ij = sm.i_ord[j];
      rank += (kj > kk || (kj == kk && ij < ii)) ? 1 : 0;
    }
    const int64_t o = (int64_t)row * p.out.topk_stride + rank;
    if (p.out.topk_idx) p.out.topk_idx[o] = ii;
    if (p.out.topk_prob)
      p.out.topk_prob[o] = (sm.S > 0.0) ? (float)((double)sm.q_ord[lane] / sm.S) : 0.0f;
  }
}

template <bool VEC>
__device__ __forceinline__ void topk_body(const CallParams &p0) {
  __shared__ TopkSmem sm;
  int row, chunk;
  block_row_chunk(p0.nchunks, p0.rows, row, chunk);
  if (!row_on_path(p0, row, kPathTopk)) return;
  const CallParams p = for_row(p0, row);
  const int S = p.nchunks, K = p.top_k;
  const float *L = p.logits + (int64_t)row * p.stride;
  const int c0 = chunk * kChunk;
  const int clen = min(kChunk, p.vocab - c0);
  ChunkMeta *cm = p.meta + (int64_t)row * S;
  Cand *cr = p.cand + (int64_t)row * S * kCandCap;
  RngPre rp = rng_prefetch(p.rng, row);  // one vector load, in flight with the chunk
  PenaltyPrefetch pf;
  if (p.fuse_penalty) {
    penalty_prefetch(p, row, pf);  // issued before the chunk
    penalty_clear(sm);             // ordered before the table by the stream phase's barrier
    // the history ids in hand before the chunk's loads go out (issued
    // together, they come back with the chunk under the other workgroups'
    // loads)
    __builtin_amdgcn_s_waitcnt(0);
  }
  topk_stream<VEC>(p, row, L, c0, clen, chunk_quota(K, S, p.exact_kernel && !(p.top_p < 1.0f)), cr + (int64_t)chunk * kCandCap,
                        cm + chunk, pf, sm);
  if (!last_of_row(p.tickets, row, S, &sm.last, [] {})) return;
  if (p.exact_kernel && !(p.top_p < 1.0f)) return;  // k_topk_exact draws and finishes this row
  RngVals rv = rng_unpack(rp);
  if (threadIdx.x == 0) {
    sm.uval = rng_draw(p.rng, row, rv);
    sm.replay = 1;
  }
  __syncthreads();
  int mr = -1;
  if (S <= kFastChunks) {
    // waves 0-3 narrow the candidates, waves 0 and 1 sort; the verdict is
    // shared at the barrier
    const int r = topk_merge_waves(p, S, cm, cr, sm);
    if (threadIdx.x == 0) sm.mres = r;
    __syncthreads();
    const int m0 = sm.mres;
    mr = (m0 == 1) ? ((sm.ntop == K) ? 1 : 0) : (m0 == 0 ? 0 : -1);
  }
  if (mr < 0) mr = topk_merge<VEC>(p, L, S, cm, cr, sm) ? 1 : 0;
  if (mr > 0) topk_fast(p, row, sm);
  if (sm.replay) topk_exact<VEC>(p, row, cm, cr, sm);
  if (threadIdx.x == 0) {
    p.out.tokens[row] = sm.token;
    if (p.out.flags) p.out.flags[row] = sm.rowflags;
  }
}

// Rows with Top-P >= 1 (the draw walks the min-buffer's slots, Sampler.pas:
// 412-413, 447-459) when the call launches k_topk_exact after the top-K
// kernel: that kernel streams their chunks (thresholds, stored candidates,
// the fused penalty) and stops at the ticket; here one workgroup per row,
// with the register budget of one workgroup per CU, draws u, replays the
// buffer (a re-read chunk after chunk 0 in one index-ordered list instead of
// 16 groups) and finishes in slot order.
template <bool VEC>
__device__ __forceinline__ void topk_exact_body(const CallParams &p0) {
  __shared__ TopkSmem sm;
  const int row = blockIdx.x;
  if (!row_on_path(p0, row, kPathTopk)) return;
  const CallParams p = for_row(p0, row);
  if (p.top_p < 1.0f) return;  // finished by the top-K kernel
  const RngPre rp = rng_prefetch(p.rng, row);  // drawn once the buffer is final
  const int S = p.nchunks;
  const ChunkMeta *cm = p.meta + (int64_t)row * S;
  const Cand *cr = p.cand + (int64_t)row * S * kCandCap;
  if (threadIdx.x == 0) sm.replay = 1;
  __syncthreads();
  topk_exact<VEC, true>(p, row, cm, cr, sm, rp);
  if (threadIdx.x == 0) {
    p.out.tokens[row] = sm.token;
    if (p.out.flags) p.out.flags[row] = sm.rowflags;
  }
}
__global__ __launch_bounds__(kBlock) void k_topk_exact_vec(CallParams p) { topk_exact_body<true>(p); }
__global__ __launch_bounds__(kBlock) void k_topk_exact_scalar(CallParams p) { topk_exact_body<false>(p); }

// =============================================================================
// Top-K for 64 < K <= kKBig (Sampler.pas:327-460).
//
// The stream phase is the one above with more candidate slots per chunk
// (ccap, sized from the chunk quota).  The merge (the row's last workgroup)
// gathers the stored keys into LDS -- only those >= T = max_c tau_c when no
// chunk overflowed, since every logit >= T was stored -- selects theta = the
// K-th largest by radix, re-reads any chunk whose unstored logits could reach
// theta, and sorts the K keys >= theta across the workgroup.  The finish runs
// over them, four per thread; rows it cannot settle exactly take the exact
// path, whose buffer is a two-level tournament in LDS.
// =============================================================================
constexpr int kBigCap = 4096;  // merge-phase LDS keys
static_assert(kKBig <= 1024 && kKBig % kBlock == 0, "large-K layout: 4 sorted keys per thread");

struct TopkBigSmem {
  // stream phase (the fields topk_stream and the fused penalty use)
  uint32_t thr[64];
  uint32_t cnt[kWaves][64];
  uint32_t wmax[kWaves];
  uint32_t wflag[kWaves];
  int32_t last;
  uint32_t ptab[kPenHash];
  uint32_t pcnt[8 * kBlock];
  // merge
  uint32_t ctau[kMaxChunks];
  uint64_t ccnt[kMaxChunks];  // stored keys per wave region, 16 bits each
  uint32_t hist[256];
  uint32_t rbin, rneed, rcnt;
  uint32_t n;
  int32_t ntop;
  int32_t flag;
  // finish
  float uval;
  int32_t token;
  uint32_t rowflags;
  int32_t replay;
  float qmax;
  int32_t pos;
  int32_t amb;
  double wtot[kWaves];
  double S;
  // exact path
  uint64_t xw64[kWaves][4];  // exact path: per-wave group counts of a whole chunk
  uint32_t xw[kWaves];
  uint32_t xmkey;
  int32_t xfrozen;
  int32_t qnan;
  float wfmax[kWaves];
  uint64_t topkey[kKBig];  // the top K, descending (value, then lower index)
  union {
    uint64_t sk[kBigCap];
    struct {
      uint64_t list[1024];   // one group's candidates / sort keys
      uint64_t leaf[kKBig];  // buffer slot s: slot_key << 32 | index
      float q[kKBig];
      float q_ord[kKBig];
      int32_t i_ord[kKBig];
      float v_ord[kKBig];
    } x;
  } buf;
};

// Stored keys of region r (0..3) of a chunk record.
__device__ __forceinline__ uint32_t big_count(uint64_t ccnt, int r) { return (uint32_t)(ccnt >> (16 * r)) & 0xFFFFu; }

// Descending bitonic sort of a[0, N) in LDS (N a power of two, whole workgroup).
__device__ __forceinline__ void block_sort_desc(uint64_t *a, int N) {
  for (int k2 = 2; k2 <= N; k2 <<= 1) {
    for (int j = k2 >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < N; i += kBlock) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const uint64_t x = a[i], y = a[ixj];
          const bool desc = (i & k2) == 0;
          if ((x < y) == desc) {
            a[i] = y;
            a[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
}

// Appends the stored keys >= lo of every chunk (all slots of each wave region
// below its count) to sm.buf.sk and returns how many there were (more than
// kBigCap: not all were kept).  Thread t takes a contiguous run of the
// concatenated regions; it locates each item (binary search over the
// per-chunk offsets, then the chunk's four regions) before issuing its loads,
// so they are in flight together.
__device__ __forceinline__ uint32_t big_gather(const Cand *__restrict__ cand_row, int S, int V, int ccap,
                                               uint32_t lo, TopkBigSmem &sm) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  uint32_t *off = sm.hist;  // per-chunk start in the concatenation (S <= 256)
  uint32_t tot = 0u;
  if (tid < S) {
    const uint64_t cc = sm.ccnt[tid];
    tot = big_count(cc, 0) + big_count(cc, 1) + big_count(cc, 2) + big_count(cc, 3);
  }
  const uint32_t incl = wave_incl_scan_u32(tot);
  if (lane == 63) sm.xw[wv] = incl;
  if (tid == 0) sm.n = 0u;
  __syncthreads();
  uint32_t base = 0u, all = 0u;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    base += (w < wv) ? sm.xw[w] : 0u;
    all += sm.xw[w];
  }
  if (tid < S) off[tid] = base + incl - tot;
  __syncthreads();
  const uint32_t per = (all + kBlock - 1) / kBlock;
  for (uint32_t g0 = 0u; g0 < per; g0 += 16u) {
    uint64_t kk[16];
    const Cand *addr[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t g = (uint32_t)tid * per + g0 + (uint32_t)i;
      addr[i] = nullptr;
      if (g0 + (uint32_t)i < per && g < all) {
        int a = 0, b = S - 1;  // the last chunk whose offset is <= g
        while (a < b) {
          const int mid = (a + b + 1) >> 1;
          if (off[mid] <= g) a = mid; else b = mid - 1;
        }
        const uint64_t cc = sm.ccnt[a];
        uint32_t rel = g - off[a];
        int r = 0;
        while (r < kWaves - 1 && rel >= big_count(cc, r)) rel -= big_count(cc, r++);
        const uint32_t rcap = (uint32_t)wave_cap(min(kChunk, V - a * kChunk), ccap);
        addr[i] = cand_row + (int64_t)a * ccap + (int64_t)r * rcap + rel;
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) kk[i] = addr[i] ? xload(addr[i]) : 0ull;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      if (addr[i] && (uint32_t)(kk[i] >> 32) >= lo) {
        const uint32_t q = atomicAdd(&sm.n, 1u);
        if (q < (uint32_t)kBigCap) sm.buf.sk[q] = kk[i];
      }
    }
  }
  __syncthreads();
  return sm.n;
}

// Block-wide OR / max of one value per thread (through sm.xw).
__device__ __forceinline__ uint32_t block_or_u32(uint32_t v, TopkBigSmem &sm) {
  v = wave_or_u32(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sm.xw[threadIdx.x >> 6] = v;
  __syncthreads();
  return sm.xw[0] | sm.xw[1] | sm.xw[2] | sm.xw[3];
}
__device__ __forceinline__ uint32_t block_max_u32(uint32_t v, TopkBigSmem &sm) {
  v = wave_max_u32(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) sm.xw[threadIdx.x >> 6] = v;
  __syncthreads();
  return max(max(sm.xw[0], sm.xw[1]), max(sm.xw[2], sm.xw[3]));
}

// Merge for large K.  Returns true when sm.topkey[0, K) holds the row's top K
// (descending value, then lower index); false when the exact path must run:
// a NaN or +inf logit, the K-th value tied with a logit outside the set (the
// reference's slot order decides which tied logits it keeps), or more keys
// than the merge's LDS holds.
template <bool VEC>
__device__ __forceinline__ bool topk_merge_big(const CallParams &p, const float *__restrict__ L, int S,
                                               const ChunkMeta *__restrict__ cm, const Cand *__restrict__ cand_row,
                                               int ccap, TopkBigSmem &sm) {
  const int V = p.vocab, K = p.top_k;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  uint32_t fl = 0u, tmx = 0u;
  for (int c = tid; c < S; c += kBlock) {
    const uint64_t w0 = xload(&cm[c].w);
    const uint64_t n01 = xload(reinterpret_cast<const uint64_t *>(&cm[c].n[0]));
    const uint64_t n23 = xload(reinterpret_cast<const uint64_t *>(&cm[c].n[2]));
    const uint32_t rcap = (uint32_t)wave_cap(min(kChunk, V - c * kChunk), ccap);
    const uint32_t n0 = (uint32_t)n01, n1 = (uint32_t)(n01 >> 32), n2 = (uint32_t)n23,
                   n3 = (uint32_t)(n23 >> 32);
    const bool ovf = n0 > rcap || n1 > rcap || n2 > rcap || n3 > rcap;
    sm.ccnt[c] = (uint64_t)min(n0, rcap) | ((uint64_t)min(n1, rcap) << 16) | ((uint64_t)min(n2, rcap) << 32) |
                 ((uint64_t)min(n3, rcap) << 48);
    const uint32_t tau = ovf ? 0xFFFFFFFFu : (uint32_t)w0;
    sm.ctau[c] = tau;
    tmx = max(tmx, tau);
    fl |= (uint32_t)(w0 >> 32);
  }
  fl = block_or_u32(fl, sm);
  tmx = block_max_u32(tmx, sm);
  if (fl) return false;
  // Every logit >= T = max tau_c was stored when no chunk overflowed, so if
  // at least K stored keys reach T the top K is among them.
  uint32_t n = 0u, theta = 0u;
  bool done = false;
  if (tmx != 0xFFFFFFFFu) {
    n = big_gather(cand_row, S, V, ccap, tmx, sm);
    if (n >= (uint32_t)K && n <= (uint32_t)kBigCap) {
      theta = radix_kth(n, K, sm, tmx, 0xFFFFFFFFu);
      done = true;
    }
  }
  if (!done) {
    // every stored key; theta = the K-th largest (a lower bound of the row's
    // K-th value); chunks whose unstored logits could reach it are re-read
    n = big_gather(cand_row, S, V, ccap, 0u, sm);
    if (n > (uint32_t)kBigCap) return false;
    theta = (n >= (uint32_t)K) ? radix_kth(n, K, sm, 0u, 0xFFFFFFFFu) : 0u;
    for (int round = 0; round < 2; ++round) {
      int open = 0;
      for (int c = tid; c < S; c += kBlock) open |= (sm.ctau[c] > theta) ? 1 : 0;
      open = __syncthreads_or(open);
      if (!open) break;
      if (round == 1) return false;  // re-read chunks are closed: not reached
      // keep the stored keys >= theta of closed chunks, then append every
      // logit >= theta of the open ones
      uint64_t keep[kBigCap / kBlock];
#pragma unroll
      for (int r = 0; r < kBigCap / kBlock; ++r) {
        const uint32_t i = (uint32_t)(tid + r * kBlock);
        keep[r] = 0ull;
        if (i < n) {
          const uint64_t k = sm.buf.sk[i];
          const int c = (int)((~(uint32_t)k) / (uint32_t)kChunk);
          if ((uint32_t)(k >> 32) >= theta && sm.ctau[c] <= theta) keep[r] = k;
        }
      }
      __syncthreads();
      if (tid == 0) sm.n = 0u;
      __syncthreads();
#pragma unroll
      for (int r = 0; r < kBigCap / kBlock; ++r) {
        if (keep[r]) {
          const uint32_t q = atomicAdd(&sm.n, 1u);
          sm.buf.sk[q] = keep[r];
        }
      }
      for (int c = 0; c < S; ++c) {
        if (sm.ctau[c] <= theta) continue;  // uniform
        const int c0 = c * kChunk, clen = min(kChunk, V - c0);
        float v[kPerThread];
        reload_chunk<VEC>(L, c0, clen, p.fuse_penalty != 0, v);
#pragma unroll
        for (int i = 0; i < kPerThread; ++i) {
          const int local = chunk_pos(wv, lane, i);
          const float x = v[i];
          if (local < clen && x == x && ord_key(x) >= theta) {
            const uint32_t q = atomicAdd(&sm.n, 1u);
            if (q < (uint32_t)kBigCap) sm.buf.sk[q] = ((uint64_t)ord_key(x) << 32) | (uint32_t)(~(uint32_t)(c0 + local));
          }
        }
      }
      __syncthreads();
      for (int c = tid; c < S; c += kBlock)
        if (sm.ctau[c] > theta) sm.ctau[c] = theta;  // now closed
      n = sm.n;
      if (n > (uint32_t)kBigCap || n < (uint32_t)K) return false;
      theta = radix_kth(n, K, sm, 0u, 0xFFFFFFFFu);
    }
    if (n < (uint32_t)K) return false;
  }
  if (sm.rcnt > sm.rneed) return false;  // the K-th value is tied outside the set
  // the K keys >= theta, sorted descending (padded to a power of two with 0)
  int N = 1;
  while (N < K) N <<= 1;
  for (int i = tid; i < N; i += kBlock) sm.topkey[i] = 0ull;
  __syncthreads();
  if (tid == 0) sm.n = 0u;
  __syncthreads();
  for (uint32_t i = tid; i < n; i += kBlock) {
    const uint64_t k = sm.buf.sk[i];
    if ((uint32_t)(k >> 32) >= theta) {
      const uint32_t q = atomicAdd(&sm.n, 1u);
      if (q < (uint32_t)kKBig) sm.topkey[q] = k;
    }
  }
  __syncthreads();
  block_sort_desc(sm.topkey, N);
  return true;
}

// Block-wide exclusive scan of one double per thread; returns the prefix and
// sets `total` (every thread).
__device__ __forceinline__ double big_excl_scan(double x, double &total, TopkBigSmem &sm) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const double incl = wave_incl_scan_f64(x);
  __syncthreads();
  if (lane == 63) sm.wtot[wv] = incl;
  __syncthreads();
  double base = 0.0;
  total = 0.0;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    if (w < wv) base += sm.wtot[w];
    total += sm.wtot[w];
  }
  return base + (incl - x);
}

// Finish over the sorted top K (Sampler.pas:385-459), thread t holding
// entries 4t..4t+3.  q = fl32(exp((v - M) invT)) as the reference computes
// it; Min-P, the Top-P cut and the draw follow :393-459 in value order,
// which is the reference's sorted order except inside groups of equal q.
// Sums are block scans.  When every non-zero q is within 2^f of the largest
// (f = 29 - ceil(log2 K)), each q is a multiple of 2^(e-f-23) (e the
// exponent of q_max) and any sum of K of them has at most 53 bits, so every
// partial sum is exact in any order and equals the reference's.  Otherwise
// each sum of K non-negative terms is within 2 K 2^-53 of the exact one in
// any order, so a comparison of a running sum with the Top-P target or the
// draw threshold that falls within the combined bound could go either way
// in the reference's order: such rows, a Top-P cut or a draw inside a group
// of equal q, Top-P >= 1 (the draw walks the reference's slot order), and the
// fallback (no running sum exceeds the threshold) take the exact path.
__device__ __forceinline__ void topk_finish_big(const CallParams &p, int row, TopkBigSmem &sm) {
  const int tid = threadIdx.x;
  const int K = p.top_k;
  const float M = key_float((uint32_t)(sm.topkey[0] >> 32));
  bool elig = (p.top_p < 1.0f) && (p.inv_t > 0.0f) && (p.inv_t <= 3.4028235e38f);
  float q[4];
  int32_t id[4];
  bool act[4];
  bool bad = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int k = 4 * tid + i;
    act[i] = k < K;
    const uint64_t key = act[i] ? sm.topkey[k] : 0ull;
    id[i] = (int32_t)(~(uint32_t)key);
    q[i] = act[i] ? (float)exp(((double)key_float((uint32_t)(key >> 32)) - (double)M) * (double)p.inv_t) : 0.0f;
    bad = bad || (act[i] && !(q[i] <= 3.4028235e38f));
  }
  if (tid == 0) sm.qmax = q[0];
  __syncthreads();
  const float qmax = sm.qmax;
  int lk = 0;
  while ((1 << lk) < K) ++lk;
  const float qfloor = ldexpf(qmax, -(29 - lk));
  bool inexact = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) inexact = inexact || (act[i] && q[i] != 0.0f && q[i] < qfloor);
  const uint32_t badm = block_or_u32((bad ? 1u : 0u) | (inexact ? 2u : 0u), sm);
  elig = elig && !(badm & 1u);
  const bool exact = !(badm & 2u);
  if (elig && p.min_p > 0.0f) {  // Min-P (:393-410): Qmax = q[0]
    const float thr = qmax * p.min_p;
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = (q[i] < thr) ? 0.0f : q[i];
  }
  // running sums in value order
  double loc[4], s = 0.0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    loc[i] = s;
    s = s + (double)q[i];
  }
  double S1;
  const double base = big_excl_scan(s, S1, sm);
  const double target = (double)p.top_p * S1;
  const double Kd = (double)K;
  const double err1 = exact ? 0.0 : (4.0 * Kd * 0x1p-53 * S1 * (1.0 + (double)p.top_p) + 0x1p-50 * target);
  bool kept[4], near = false;
  double s2 = 0.0;
  float qk[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const double C = base + loc[i];
    kept[i] = act[i] && q[i] > 0.0f && C < target;  // Top-P (:431-444)
    near = near || (act[i] && q[i] > 0.0f && err1 > 0.0 && fabs(C - target) <= err1);
    qk[i] = kept[i] ? q[i] : 0.0f;
  }
  // the cut must not split a group of equal q (the reference keeps the members
  // that come first in its slot order): the first dropped entry vs the last
  // kept one (kept entries form a prefix)
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (act[i]) {
      sm.buf.x.q[4 * tid + i] = q[i];
      sm.buf.x.i_ord[4 * tid + i] = kept[i] ? 1 : 0;
    }
  __syncthreads();
  bool split = false;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int k = 4 * tid + i;
    if (act[i] && !kept[i] && q[i] > 0.0f && k > 0)
      split = split || (sm.buf.x.i_ord[k - 1] != 0 && sm.buf.x.q[k - 1] == q[i]);
  }
  double s2loc[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s2loc[i] = s2;
    s2 = s2 + (double)qk[i];
  }
  double S2;
  const double base2 = big_excl_scan(s2, S2, sm);
  const double t = (double)sm.uval * S2;  // draw (:447-459)
  const double err2 = exact ? 0.0 : (8.0 * Kd * 0x1p-53 * S2 + 0x1p-50 * t);
  int pos = 0x7FFFFFFF;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const double C2 = base2 + s2loc[i] + (double)qk[i];
    if (kept[i] && C2 > t && pos == 0x7FFFFFFF) pos = 4 * tid + i;
    near = near || (kept[i] && err2 > 0.0 && fabs(C2 - t) <= err2);
  }
  if (tid == 0) sm.pos = 0x7FFFFFFF;
  __syncthreads();
  if (pos != 0x7FFFFFFF) atomicMin(&sm.pos, pos);
  const uint32_t ambm = block_or_u32((near ? 1u : 0u) | (split ? 2u : 0u), sm);
  const int ps = sm.pos;
  bool amb = !elig || ambm != 0u || ps == 0x7FFFFFFF;
  if (!amb) {  // the draw must not land inside a group of equal q
    const float qp = sm.buf.x.q[ps];
    amb = (ps > 0 && sm.buf.x.q[ps - 1] == qp) || (ps + 1 < K && sm.buf.x.q[ps + 1] == qp);
  }
  if (amb) {
    if (tid == 0) sm.replay = 1;
    __syncthreads();
    return;
  }
  if (tid == 0) {
    sm.token = (int32_t)(~(uint32_t)sm.topkey[ps]);
    sm.rowflags = kRowTopkFast;
    sm.replay = 0;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (act[i]) {
      const int64_t o = (int64_t)row * p.out.topk_stride + 4 * tid + i;
      if (p.out.topk_idx) p.out.topk_idx[o] = id[i];
      if (p.out.topk_prob) p.out.topk_prob[o] = (float)((double)qk[i] / S2);
    }
  }
  __syncthreads();
}

// ---- exact path for large K ----------------------------------------------------
// The min-buffer (Sampler.pas:341-383) as a two-level tournament: leaf[s]
// (LDS) is slot s's entry, slot_key << 32 | index; wave 0's lane g holds the
// smallest (key << 32 | slot) of leaves 64g .. 64g + 63, so the smallest of
// the lanes is the reference's first strict minimum (smallest value, then
// lowest slot; NaN sorts above +inf).  An entering logit replaces that leaf,
// and its group and the top are reduced again.
struct TourBuf {
  uint64_t g;
  uint32_t mkey;
  uint32_t mslot;
};
__device__ __forceinline__ uint64_t tb_group_min(const TopkBigSmem &sm, int K, int gi) {
  const int s = gi * 64 + lane_id();
  const uint64_t e = (s < K) ? ((sm.buf.x.leaf[s] & 0xFFFFFFFF00000000ull) | (uint32_t)s) : ~0ull;
  return wave_min_u64(e);
}
__device__ __forceinline__ void tb_refresh(TourBuf &t, int G) {
  const uint64_t m = wave_min_u64(lane_id() < G ? t.g : ~0ull);
  t.mkey = (uint32_t)(m >> 32);
  t.mslot = (uint32_t)m;
}
__device__ __forceinline__ void tb_enter(TourBuf &t, TopkBigSmem &sm, int K, int G, uint32_t xk, uint32_t xi) {
  const int s = (int)t.mslot;
  if (lane_id() == 0) sm.buf.x.leaf[s] = ((uint64_t)xk << 32) | xi;  // read back below by the same wave
  const int gi = s >> 6;
  const uint64_t gm = tb_group_min(sm, K, gi);
  if (lane_id() == gi) t.g = gm;
  tb_refresh(t, G);
}
// K <= 128: the minimum from the slots' (key << 32 | slot) sorted ascending
// over two registers of wave 0 (lanes 0-63, then 64-127; ~0 past K), an
// entry as in the K <= 64 buffer (each position takes the next one if that is
// below the new entry, else the new entry if its own is, else its own), the
// shift carried from the high register's lane 0 into the low one's lane 63.
struct SortBuf2 {
  uint64_t lo, hi;
};
__device__ __forceinline__ void sb2_refresh(const SortBuf2 &b, TourBuf &t) {
  const uint64_t m = readlane64(b.lo, 0);
  t.mkey = (uint32_t)(m >> 32);
  t.mslot = (uint32_t)m;
}
__device__ __forceinline__ void sb2_enter(SortBuf2 &b, TourBuf &t, TopkBigSmem &sm, uint32_t xk, uint32_t xi) {
  const uint32_t s = t.mslot;
  if (lane_id() == 0) sm.buf.x.leaf[s] = ((uint64_t)xk << 32) | xi;
  const uint64_t nk = ((uint64_t)xk << 32) | s;
  const uint64_t h0 = readlane64(b.hi, 0);
  const uint64_t shl = ((uint64_t)(uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)(h0 >> 32), (int)(uint32_t)(b.lo >> 32), 0x130, 0xF, 0xF, false) << 32) |
                       (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)h0, (int)(uint32_t)b.lo, 0x130, 0xF, 0xF, false);
  const uint64_t shh = wave_shl1_64(b.hi);
  b.lo = (shl < nk) ? shl : ((b.lo < nk) ? nk : b.lo);
  b.hi = (shh < nk) ? shh : ((b.hi < nk) ? nk : b.hi);
  sb2_refresh(b, t);
}
// 128 < K <= 256: the same over four registers (positions 64i + lane of
// register i), each register's lane 63 taking the next one's lane 0.
struct SortBuf4 {
  uint64_t r[4];
};
__device__ __forceinline__ uint64_t shl1_from(uint64_t v, uint64_t in63) {  // lane l <- lane l + 1, lane 63 <- in63
  return ((uint64_t)(uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)(in63 >> 32), (int)(uint32_t)(v >> 32), 0x130, 0xF, 0xF, false) << 32) |
         (uint32_t)__builtin_amdgcn_update_dpp((int)(uint32_t)in63, (int)(uint32_t)v, 0x130, 0xF, 0xF, false);
}
__device__ __forceinline__ void sb4_enter(SortBuf4 &b, TourBuf &t, TopkBigSmem &sm, uint32_t xk, uint32_t xi) {
  const uint32_t s = t.mslot;
  if (lane_id() == 0) sm.buf.x.leaf[s] = ((uint64_t)xk << 32) | xi;
  const uint64_t nk = ((uint64_t)xk << 32) | s;
  const uint64_t c0 = readlane64(b.r[1], 0), c1 = readlane64(b.r[2], 0), c2 = readlane64(b.r[3], 0);
  const uint64_t s0 = shl1_from(b.r[0], c0), s1 = shl1_from(b.r[1], c1), s2 = shl1_from(b.r[2], c2),
                 s3 = shl1_from(b.r[3], ~0ull);
  b.r[0] = (s0 < nk) ? s0 : ((b.r[0] < nk) ? nk : b.r[0]);
  b.r[1] = (s1 < nk) ? s1 : ((b.r[1] < nk) ? nk : b.r[1]);
  b.r[2] = (s2 < nk) ? s2 : ((b.r[2] < nk) ? nk : b.r[2]);
  b.r[3] = (s3 < nk) ? s3 : ((b.r[3] < nk) ? nk : b.r[3]);
  const uint64_t m = readlane64(b.r[0], 0);
  t.mkey = (uint32_t)(m >> 32);
  t.mslot = (uint32_t)m;
}
template <int MODE>
__device__ __forceinline__ void tb_feed(TourBuf &t, SortBuf2 &b, SortBuf4 &b4, TopkBigSmem &sm, int K, int G,
                                        bool has, uint32_t ck, uint32_t ci) {
  uint64_t pend = __ballot(has && ck > t.mkey);
  while (pend) {
    const int src = __ffsll((unsigned long long)pend) - 1;
    if constexpr (MODE == 2)
      sb2_enter(b, t, sm, readlane32(ck, src), readlane32(ci, src));
    else if constexpr (MODE == 4)
      sb4_enter(b4, t, sm, readlane32(ck, src), readlane32(ci, src));
    else
      tb_enter(t, sm, K, G, readlane32(ck, src), readlane32(ci, src));
    pend &= ~(1ull << src);
    pend &= __ballot(ck > t.mkey);
  }
}

// MODE: the buffer's minimum from 2 or 4 sorted registers (K <= 128, <= 256)
// or the tournament (0); one instantiation each, so each keeps its registers
template <bool VEC, int MODE>
__device__ __forceinline__ void topk_exact_big(const CallParams &p, int row, TopkBigSmem &sm) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int K = p.top_k, V = p.vocab, S = p.nchunks;
  const int G = (K + 63) >> 6;
  const float *L = p.logits + (int64_t)row * p.stride;
  const bool pen = p.fuse_penalty != 0;
  TourBuf tb{~0ull, 0xFFFFFFFFu, 0u};
  SortBuf2 sb{~0ull, ~0ull};
  SortBuf4 sb4{{~0ull, ~0ull, ~0ull, ~0ull}};
  constexpr bool small = MODE == 2;
  constexpr int mode = MODE;
  uint64_t *list = sm.buf.x.list;
  float v[kPerThread];
  for (int c = 0; c < S; ++c) {
    const int c0 = c * kChunk, clen = min(kChunk, V - c0);
    __syncthreads();
    if (c > 0 && sm.xfrozen) break;
    reload_chunk<VEC>(L, c0, clen, pen, v);
    if (c == 0) {
      // the first K logits fill slots 0..K-1 (Sampler.pas:352-366); all lie in
      // the chunk's first 1024-logit group (K <= 1024)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int s = wv * 256 + lane * 4 + e;
        if (s < K) sm.buf.x.leaf[s] = ((uint64_t)slot_key(v[e]) << 32) | (uint32_t)s;
      }
      __syncthreads();
      if (wv == 0 && small) {
        // x[1] descending, x[0] ascending; lane-wise min / max are bitonic
        uint64_t x0 = lane < K ? ((sm.buf.x.leaf[lane] & 0xFFFFFFFF00000000ull) | (uint32_t)lane) : ~0ull;
        uint64_t x1 = lane + 64 < K ? ((sm.buf.x.leaf[lane + 64] & 0xFFFFFFFF00000000ull) | (uint32_t)(lane + 64)) : ~0ull;
        wave_sort2(x1, x0);
        sb.lo = wave_merge<true>(x0 < x1 ? x0 : x1);
        sb.hi = wave_merge<true>(x0 < x1 ? x1 : x0);
        sb2_refresh(sb, tb);
      } else if (mode == 4) {
        // entry (key << 32 | slot) of slot s at its rank among the K
        if (tid < K) {
          const uint64_t e = (sm.buf.x.leaf[tid] & 0xFFFFFFFF00000000ull) | (uint32_t)tid;
          uint32_t rk = 0u;
          for (int t2 = 0; t2 < K; ++t2)
            rk += (((sm.buf.x.leaf[t2] & 0xFFFFFFFF00000000ull) | (uint32_t)t2) < e) ? 1u : 0u;
          list[rk] = e;
        }
        __syncthreads();
        if (wv == 0) {
#pragma unroll
          for (int i = 0; i < 4; ++i) sb4.r[i] = (64 * i + lane < K) ? list[64 * i + lane] : ~0ull;
          const uint64_t m = readlane64(sb4.r[0], 0);
          tb.mkey = (uint32_t)(m >> 32);
          tb.mslot = (uint32_t)m;
        }
      } else if (wv == 0) {
        for (int gi = 0; gi < G; ++gi) {
          const uint64_t gm = tb_group_min(sm, K, gi);
          if (lane == gi) tb.g = gm;
        }
        tb_refresh(tb, G);
      }
      if (wv == 0) {
        const float l0 = __uint_as_float(readlane32(__float_as_uint(v[0]), 0));
        if (lane == 0) {
          sm.xfrozen = (l0 != l0) ? 1 : 0;
          sm.xmkey = tb.mkey;
        }
      }
    }
    if (c > 0) {
      // after chunk 0 the minimum rises slowly: every logit above it when the
      // chunk starts in one index-ordered list (per-thread counts of the 16
      // groups, four 16-bit fields per wave scan), fed in index order; a
      // longer list goes group by group, below
      const uint32_t m = sm.xmkey;
      uint64_t hb = 0ull;  // bit 4j + e: logit e of the thread's group j passes
#pragma unroll
      for (int j = 0; j < kPerThread / 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int loc = j * 1024 + wv * 256 + lane * 4 + e;
          const float x = v[4 * j + e];
          if (loc < clen && x == x && ord_key(x) > m) hb |= 1ull << (4 * j + e);
        }
      uint64_t incl[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint64_t w = 0ull;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) w |= (uint64_t)__popcll((hb >> (16 * q + 4 * jj)) & 15ull) << (16 * jj);
        incl[q] = wave_scan<uint64_t>(w, 0ull, OpAddU64());
        if (lane == 63) sm.xw64[wv][q] = incl[q];
      }
      __syncthreads();
      uint32_t gbase = 0u;
      uint32_t off[kPerThread / 4];
#pragma unroll
      for (int j = 0; j < kPerThread / 4; ++j) {  // group j's offset: earlier groups, then earlier waves
        const int q = j >> 2, sh = 16 * (j & 3);
        uint32_t before = 0u, gt = 0u;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
          const uint32_t f = (uint32_t)(sm.xw64[w][q] >> sh) & 0xFFFFu;
          before += (w < wv) ? f : 0u;
          gt += f;
        }
        off[j] = gbase + before + ((uint32_t)(incl[q] >> sh) & 0xFFFFu) - (uint32_t)__popcll((hb >> (4 * j)) & 15ull);
        gbase += gt;
      }
      const uint32_t total = gbase;
      if (total <= 1024u) {  // uniform
#pragma unroll
        for (int j = 0; j < kPerThread / 4; ++j) {
          uint32_t o = off[j];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if ((hb >> (4 * j + e)) & 1ull)
              list[o++] = ((uint64_t)ord_key(v[4 * j + e]) << 32) | (uint32_t)(c0 + j * 1024 + wv * 256 + lane * 4 + e);
        }
        __syncthreads();
        if (wv == 0) {
          for (uint32_t g = 0u; g < total; g += 64u) {
            const bool has = g + (uint32_t)lane < total;
            const uint64_t en = has ? list[g + lane] : 0ull;
            tb_feed<MODE>(tb, sb, sb4, sm, K, G, has, (uint32_t)(en >> 32), (uint32_t)en);
          }
          if (lane == 0) sm.xmkey = tb.mkey;
        }
        continue;
      }
    }
#pragma unroll
    for (int j = 0; j < kPerThread / 4; ++j) {
      __syncthreads();
      if (sm.xfrozen) break;
      const uint32_t m = sm.xmkey;
      const int base = j * 1024 + wv * 256 + lane * 4;
      uint32_t bits = 0u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = v[4 * j + e];
        const int loc = base + e;
        const bool ok = loc < clen && (c0 + loc) >= K && x == x && ord_key(x) > m;
        bits |= ok ? (1u << e) : 0u;
      }
      const uint32_t cnt = (uint32_t)__popc(bits);
      const uint32_t incl = wave_incl_scan_u32(cnt);
      if (lane == 63) sm.xw[wv] = incl;
      __syncthreads();
      uint32_t off = incl - cnt, total = 0u;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        off += (w < wv) ? sm.xw[w] : 0u;
        total += sm.xw[w];
      }
      if (total == 0u) continue;  // uniform
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if ((bits >> e) & 1u) list[off++] = ((uint64_t)ord_key(v[4 * j + e]) << 32) | (uint32_t)(c0 + base + e);
      __syncthreads();
      if (wv == 0) {
        for (uint32_t g = 0u; g < total; g += 64u) {
          const bool has = g + (uint32_t)lane < total;
          const uint64_t en = has ? list[g + lane] : 0ull;
          tb_feed<MODE>(tb, sb, sb4, sm, K, G, has, (uint32_t)(en >> 32), (uint32_t)en);
        }
        if (lane == 0) sm.xmkey = tb.mkey;
      }
    }
  }
  __syncthreads();

  // ---- slot-order finish (Sampler.pas:385-459), literally ----
  const bool frozen = sm.xfrozen != 0;
  float mloc = __builtin_nanf("");
  for (int s = tid; s < K; s += kBlock) {  // v_ord[] holds the buffer's values by slot
    const uint32_t key = (uint32_t)(sm.buf.x.leaf[s] >> 32);
    const float x = (key == 0xFFFFFFFFu) ? __builtin_nanf("") : key_float(key);
    sm.buf.x.v_ord[s] = x;
    mloc = fmaxf(mloc, x);  // NaN-ignoring
  }
  mloc = wave_max_f32(mloc);
  __syncthreads();
  if (lane == 0) sm.wfmax[wv] = mloc;
  __syncthreads();
  // M (strict '>' from L[0]): NaN when L[0] is NaN, else the largest
  // non-NaN logit, which is in the buffer
  const float M = frozen ? __builtin_nanf("")
                         : fmaxf(fmaxf(sm.wfmax[0], sm.wfmax[1]), fmaxf(sm.wfmax[2], sm.wfmax[3]));
  uint32_t qn = 0u;
  for (int s = tid; s < K; s += kBlock) {
    const float q = (float)exp(((double)sm.buf.x.v_ord[s] - (double)M) * (double)p.inv_t);
    sm.buf.x.q[s] = q;
    qn |= (q != q) ? 1u : 0u;
  }
  const bool qnan = block_or_u32(qn, sm) != 0u;
  // sums and Min-P in slot order (:386-410)
  if (tid == 0) {
    double S = 0.0;
    for (int k = 0; k < K; ++k) S = S + (double)sm.buf.x.q[k];
    if (p.min_p > 0.0f) {
      float best = sm.buf.x.q[0];
      for (int k = 1; k < K; ++k)
        if (sm.buf.x.q[k] > best) best = sm.buf.x.q[k];
      const float thr = best * p.min_p;
      S = 0.0;
      for (int k = 0; k < K; ++k) {
        if (sm.buf.x.q[k] < thr)
          sm.buf.x.q[k] = 0.0f;
        else
          S = S + (double)sm.buf.x.q[k];
      }
    }
    sm.S = S;
  }
  __syncthreads();
  // draw order: the stable descending sort of Top-P (:412-429), else slot order;
  // list[] then holds, per position, the slot it draws from
  int N = 1;
  while (N < K) N <<= 1;
  if (p.top_p < 1.0f && !qnan) {
    for (int s = tid; s < N; s += kBlock)
      list[s] = (s < K) ? (((uint64_t)__float_as_uint(sm.buf.x.q[s]) << 32) | (0xFFFFFFFFu - (uint32_t)s)) : 0ull;
    __syncthreads();
    block_sort_desc(list, N);  // q descending, equal q in slot order (q >= 0: its bits order it)
    for (int r = tid; r < K; r += kBlock) list[r] = 0xFFFFFFFFu - (uint32_t)list[r];
    __syncthreads();
  } else if (p.top_p < 1.0f) {
    if (tid == 0) {  // NaN among q: the reference's insertion sort, literally
      for (int r = 0; r < K; ++r) list[r] = (uint64_t)r;
      for (int i = 1; i < K; ++i) {
        const uint64_t si = list[i];
        const float qv = sm.buf.x.q[si];
        int j = i - 1;
        while (j >= 0 && sm.buf.x.q[list[j]] < qv) {
          list[j + 1] = list[j];
          --j;
        }
        list[j + 1] = si;
      }
    }
    __syncthreads();
  } else {
    for (int r = tid; r < K; r += kBlock) list[r] = (uint64_t)r;
    __syncthreads();
  }
  for (int r = tid; r < K; r += kBlock) {
    const int s = (int)list[r];
    sm.buf.x.q_ord[r] = sm.buf.x.q[s];
    sm.buf.x.i_ord[r] = (int32_t)((uint32_t)sm.buf.x.leaf[s] & kXbIdxMask);
  }
  __syncthreads();
  if (tid == 0) {
    double S = sm.S;
    if (p.top_p < 1.0f) {  // Top-P cut (:431-444)
      const double target = (double)p.top_p * S;
      double C = 0.0;
      S = 0.0;
      for (int r = 0; r < K; ++r) {
        if (C < target && sm.buf.x.q_ord[r] > 0.0f) {
          C = C + (double)sm.buf.x.q_ord[r];
          S = S + (double)sm.buf.x.q_ord[r];
        } else {
          sm.buf.x.q_ord[r] = 0.0f;
        }
      }
    }
    const double t = (double)sm.uval * S;  // draw (:447-459)
    double C = 0.0;
    int32_t tok = sm.buf.x.i_ord[K - 1];
    uint32_t fl = kRowTopkReplay | kRowFallback;
    for (int r = 0; r < K; ++r) {
      C = C + (double)sm.buf.x.q_ord[r];
      if (C > t) {
        tok = sm.buf.x.i_ord[r];
        fl = kRowTopkReplay;
        break;
      }
    }
    if (qnan || !(M == M)) fl |= kRowNan;
    sm.token = tok;
    sm.rowflags = fl;
    sm.S = S;
  }
  __syncthreads();
  if (p.out.topk_idx || p.out.topk_prob) {
    // canonical order: value descending, then lower index (NaN first)
    for (int r = tid; r < N; r += kBlock) {
      uint64_t key = 0ull;
      if (r < K) {
        const int s = (int)list[r];
        key = ((uint64_t)slot_key(sm.buf.x.v_ord[s]) << 32) |
              ((uint64_t)(kXbIdxMask - (uint32_t)sm.buf.x.i_ord[r]) << 10) | (uint32_t)r;
      }
      sm.buf.x.leaf[r] = key;  // the buffer's leaves are no longer read
    }
    __syncthreads();
    block_sort_desc(sm.buf.x.leaf, N);
    for (int j = tid; j < K; j += kBlock) {
      const int r = (int)(sm.buf.x.leaf[j] & 1023u);
      const int64_t o = (int64_t)row * p.out.topk_stride + j;
      if (p.out.topk_idx) p.out.topk_idx[o] = sm.buf.x.i_ord[r];
      if (p.out.topk_prob)
        p.out.topk_prob[o] = (sm.S > 0.0) ? (float)((double)sm.buf.x.q_ord[r] / sm.S) : 0.0f;
    }
  }
}

// Large K runs in two launches: the stream phase over every (row, chunk)
// within the K <= 64 kernel's register and LDS budget (four workgroups per CU,
// every chunk of a 64-row batch resident at once), then one workgroup per row
// for the merge, the finish and the exact path, whose registers would
// otherwise halve the stream phase's occupancy.  The launch boundary orders
// the chunk records before the merge, so no ticket is taken.
template <bool VEC>
__device__ __forceinline__ void topk_big_stream_body(const CallParams &p0) {
  __shared__ TopkSmem sm;
  int row, chunk;
  block_row_chunk(p0.nchunks, p0.rows, row, chunk);
  if (!row_on_path(p0, row, kPathTopk)) return;
  const CallParams p = for_row(p0, row);
  const int S = p.nchunks, K = p.top_k, ccap = p.cand_cap;
  const float *L = p.logits + (int64_t)row * p.stride;
  const int c0 = chunk * kChunk;
  const int clen = min(kChunk, p.vocab - c0);
  ChunkMeta *cm = p.meta + (int64_t)row * S;
  Cand *cr = p.cand + (int64_t)row * S * ccap;
  PenaltyPrefetch pf;
  if (p.fuse_penalty) {
    penalty_prefetch(p, row, pf);
    penalty_clear(sm);
  }
  topk_stream<VEC, 8 * kWaves>(p, row, L, c0, clen, big_chunk_quota(K, S), cr + (int64_t)chunk * ccap, cm + chunk, pf, sm,
                   ccap);
}

template <bool VEC>
__device__ __forceinline__ void topk_big_finish_body(const CallParams &p0) {
  __shared__ TopkBigSmem sm;
  const int row = blockIdx.x;
  if (!row_on_path(p0, row, kPathTopk)) return;
  const CallParams p = for_row(p0, row);
  const int S = p.nchunks, ccap = p.cand_cap;
  const float *L = p.logits + (int64_t)row * p.stride;
  const ChunkMeta *cm = p.meta + (int64_t)row * S;
  const Cand *cr = p.cand + (int64_t)row * S * ccap;
  const RngPre rp = rng_prefetch(p.rng, row);  // in flight during the merge
  if (threadIdx.x == 0) sm.replay = 1;
  __syncthreads();
  const bool merged = topk_merge_big<VEC>(p, L, S, cm, cr, ccap, sm);
  {
    RngVals rv = rng_unpack(rp);
    if (threadIdx.x == 0) sm.uval = rng_draw(p.rng, row, rv);
  }
  __syncthreads();
  if (merged) topk_finish_big(p, row, sm);
  __syncthreads();
  if (sm.replay) {
    if (p.top_k <= 128)
      topk_exact_big<VEC, 2>(p, row, sm);
    else if (p.top_k <= 256)
      topk_exact_big<VEC, 4>(p, row, sm);
    else
      topk_exact_big<VEC, 0>(p, row, sm);
  }
  if (threadIdx.x == 0) {
    p.out.tokens[row] = sm.token;
    if (p.out.flags) p.out.flags[row] = sm.rowflags;
  }
}

__global__ __launch_bounds__(kBlock, 4) void k_topk_big_stream_vec(CallParams p) { topk_big_stream_body<true>(p); }
__global__ __launch_bounds__(kBlock) void k_topk_big_stream_scalar(CallParams p) { topk_big_stream_body<false>(p); }
__global__ __launch_bounds__(kBlock) void k_topk_big_finish_vec(CallParams p) { topk_big_finish_body<true>(p); }
__global__ __launch_bounds__(kBlock) void k_topk_big_finish_scalar(CallParams p) { topk_big_finish_body<false>(p); }

// =============================================================================
// Top-K for K > kKBig (Sampler.pas:327-460): one workgroup per row replays
// the min-buffer exactly -- every chunk re-read, only logits above the
// buffer's minimum fed, the K slots in a per-row HBM workspace under a
// three-level tournament -- and finishes in slot order literally, with the
// Top-P order and the canonical output order sorted in HBM.  Slow but exact;
// the reference's own scan costs K per entering logit.
// =============================================================================
struct HugeView {
  uint64_t *leaf;   // [K] slot s: slot_key << 32 | index
  uint64_t *l1;     // [ceil(K/64)] minimum (key << 32 | slot) of 64 leaves
  float *q;         // [K] by slot
  float *q_ord;     // [K] by draw position
  int32_t *i_ord;   // [K] by draw position
  uint64_t *keys;   // [N] sort keys (N = the power of two >= K)
  uint32_t *vals;   // [N] sort payloads
};
__host__ __device__ __forceinline__ int64_t huge_align(int64_t x) { return (x + 255) & ~(int64_t)255; }
__host__ __device__ __forceinline__ int64_t huge_row_bytes(int K) {
  int64_t N = 1;
  while (N < K) N <<= 1;
  const int64_t G1 = (K + 63) / 64;
  return huge_align(8 * (int64_t)K) + huge_align(8 * G1) + 2 * huge_align(4 * (int64_t)K) +
         huge_align(4 * (int64_t)K) + huge_align(8 * N) + huge_align(4 * N);
}
__device__ __forceinline__ HugeView huge_view(const CallParams &p, int row, int K) {
  uint8_t *b = p.huge_ws + (int64_t)row * p.huge_row_bytes;
  int64_t N = 1;
  while (N < K) N <<= 1;
  const int64_t G1 = (K + 63) / 64;
  HugeView h;
  h.leaf = reinterpret_cast<uint64_t *>(b);
  b += huge_align(8 * (int64_t)K);
  h.l1 = reinterpret_cast<uint64_t *>(b);
  b += huge_align(8 * G1);
  h.q = reinterpret_cast<float *>(b);
  b += huge_align(4 * (int64_t)K);
  h.q_ord = reinterpret_cast<float *>(b);
  b += huge_align(4 * (int64_t)K);
  h.i_ord = reinterpret_cast<int32_t *>(b);
  b += huge_align(4 * (int64_t)K);
  h.keys = reinterpret_cast<uint64_t *>(b);
  b += huge_align(8 * N);
  h.vals = reinterpret_cast<uint32_t *>(b);
  return h;
}

constexpr int kHugeL2 = 1024;  // 64-group minima of the 64-leaf group minima: K <= 4 Mi
struct TopkHugeSmem {
  uint64_t l2[kHugeL2];
  uint64_t list[1024];
  uint32_t xw[kWaves];
  uint32_t xmkey;
  int32_t xfrozen;
  float wfmax[kWaves];
  double S;
  float uval;
  int32_t token;
  uint32_t rowflags;
};

// Descending bitonic sort of keys[0, N) (HBM) carrying vals[], whole workgroup.
__device__ __forceinline__ void hbm_sort_desc(uint64_t *keys, uint32_t *vals, int64_t N) {
  for (int64_t k2 = 2; k2 <= N; k2 <<= 1) {
    for (int64_t j = k2 >> 1; j > 0; j >>= 1) {
      for (int64_t i = threadIdx.x; i < N; i += kBlock) {
        const int64_t ixj = i ^ j;
        if (ixj > i) {
          const uint64_t x = keys[i], y = keys[ixj];
          const bool desc = (i & k2) == 0;
          if ((x < y) == desc) {
            keys[i] = y;
            keys[ixj] = x;
            if (vals) {
              const uint32_t a = vals[i];
              vals[i] = vals[ixj];
              vals[ixj] = a;
            }
          }
        }
      }
      __syncthreads();
    }
  }
}

// Wave 0: the minimum (key << 32 | slot) of leaves 64g .. 64g+63, with leaf
// s = `ps` read as `pv` (just written by this wave).
__device__ __forceinline__ uint64_t hg_group(const HugeView &h, int K, int g, int ps, uint64_t pv) {
  const int s = 64 * g + lane_id();
  uint64_t e = ~0ull;
  if (s < K) e = (((s == ps) ? pv : h.leaf[s]) & 0xFFFFFFFF00000000ull) | (uint32_t)s;
  return wave_min_u64(e);
}
__device__ __forceinline__ uint64_t hg_super(const HugeView &h, int G1, int hh, int pg, uint64_t pv) {
  const int g = 64 * hh + lane_id();
  uint64_t e = ~0ull;
  if (g < G1) e = (g == pg) ? pv : h.l1[g];
  return wave_min_u64(e);
}
__device__ __forceinline__ void hg_top(const TopkHugeSmem &sm, int G2, uint32_t &mkey, uint32_t &mslot) {
  uint64_t m = ~0ull;
  for (int i = lane_id(); i < G2; i += 64) m = sm.l2[i] < m ? sm.l2[i] : m;
  m = wave_min_u64(m);
  mkey = (uint32_t)(m >> 32);
  mslot = (uint32_t)m;
}

template <bool VEC>
__device__ __forceinline__ void topk_body_huge(const CallParams &p0) {
  __shared__ TopkHugeSmem sm;
  const int row = blockIdx.x;
  if (!row_on_path(p0, row, kPathTopkHuge)) return;
  const CallParams p = for_row(p0, row);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int K = p.top_k, V = p.vocab, S = p.nchunks;
  const int G1 = (K + 63) / 64, G2 = (G1 + 63) / 64;
  const float *L = p.logits + (int64_t)row * p.stride;
  const HugeView h = huge_view(p, row, K);
  RngVals rv = rng_unpack(rng_prefetch(p.rng, row));
  if (tid == 0) sm.uval = rng_draw(p.rng, row, rv);
  uint32_t mkey = 0u, mslot = 0u;  // wave 0
  float v[kPerThread];
  const int cK = (K - 1) / kChunk;  // the chunk holding slot K-1
  // the first K logits fill slots 0..K-1 (Sampler.pas:352-366)
  for (int c = 0; c <= cK; ++c) {
    const int c0 = c * kChunk, clen = min(kChunk, V - c0);
    reload_chunk<VEC>(L, c0, clen, false, v);
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      const int loc = chunk_pos(wv, lane, i), s = c0 + loc;
      if (loc < clen && s < K) h.leaf[s] = ((uint64_t)slot_key(v[i]) << 32) | (uint32_t)s;
    }
  }
  __syncthreads();
  // the tournament: level 1 in HBM (each wave a share of the groups), level 2 in LDS
  for (int g = wv; g < G1; g += kWaves) {
    const uint64_t m = hg_group(h, K, g, -1, 0ull);
    if (lane == 0) h.l1[g] = m;
  }
  __syncthreads();
  for (int hh = wv; hh < G2; hh += kWaves) {
    const uint64_t m = hg_super(h, G1, hh, -1, 0ull);
    if (lane == 0) sm.l2[hh] = m;
  }
  __syncthreads();
  if (wv == 0) {
    hg_top(sm, G2, mkey, mslot);
    const float l0 = xloadf(&L[0]);
    if (lane == 0) {
      sm.xfrozen = (l0 != l0) ? 1 : 0;  // a NaN at index 0 stays the minimum (:369)
      sm.xmkey = mkey;
    }
  }
  // the walk: chunk cK onwards, logits above the minimum in index order
  for (int c = cK; c < S; ++c) {
    const int c0 = c * kChunk, clen = min(kChunk, V - c0);
    __syncthreads();
    if (sm.xfrozen) break;
    reload_chunk<VEC>(L, c0, clen, false, v);
#pragma unroll
    for (int j = 0; j < kPerThread / 4; ++j) {
      __syncthreads();
      const uint32_t m = sm.xmkey;
      const int base = j * 1024 + wv * 256 + lane * 4;
      uint32_t bits = 0u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = v[4 * j + e];
        const int loc = base + e;
        bits |= (loc < clen && (c0 + loc) >= K && x == x && ord_key(x) > m) ? (1u << e) : 0u;
      }
      const uint32_t cnt = (uint32_t)__popc(bits);
      const uint32_t incl = wave_incl_scan_u32(cnt);
      if (lane == 63) sm.xw[wv] = incl;
      __syncthreads();
      uint32_t off = incl - cnt, total = 0u;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) {
        off += (w < wv) ? sm.xw[w] : 0u;
        total += sm.xw[w];
      }
      if (total == 0u) continue;  // uniform
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if ((bits >> e) & 1u) sm.list[off++] = ((uint64_t)ord_key(v[4 * j + e]) << 32) | (uint32_t)(c0 + base + e);
      __syncthreads();
      if (wv == 0) {
        for (uint32_t g0 = 0u; g0 < total; g0 += 64u) {
          const bool has = g0 + (uint32_t)lane < total;
          const uint64_t en = has ? sm.list[g0 + lane] : 0ull;
          const uint32_t ck = (uint32_t)(en >> 32), ci = (uint32_t)en;
          uint64_t pend = __ballot(has && ck > mkey);
          while (pend) {
            const int src = __ffsll((unsigned long long)pend) - 1;
            // the logit takes the minimum's slot; its group, super-group and the top are reduced again
            const int s = (int)mslot;
            const uint64_t nv = ((uint64_t)readlane32(ck, src) << 32) | readlane32(ci, src);
            if (lane == 0) h.leaf[s] = nv;
            const int g = s >> 6;
            const uint64_t gm = hg_group(h, K, g, s, nv);
            if (lane == 0) h.l1[g] = gm;
            const uint64_t sm2 = hg_super(h, G1, g >> 6, g, gm);
            if (lane == 0) sm.l2[g >> 6] = sm2;
            __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "workgroup");  // HBM stores before later reads
            hg_top(sm, G2, mkey, mslot);
            pend &= ~(1ull << src);
            pend &= __ballot(ck > mkey);
          }
        }
        if (lane == 0) sm.xmkey = mkey;
      }
    }
  }
  __syncthreads();

  // ---- slot-order finish (Sampler.pas:385-459), literally ----
  const bool frozen = sm.xfrozen != 0;
  float mloc = __builtin_nanf("");
  for (int s = tid; s < K; s += kBlock) {
    const uint32_t key = (uint32_t)(h.leaf[s] >> 32);
    mloc = fmaxf(mloc, (key == 0xFFFFFFFFu) ? __builtin_nanf("") : key_float(key));
  }
  mloc = wave_max_f32(mloc);
  if (lane == 0) sm.wfmax[wv] = mloc;
  __syncthreads();
  const float M = frozen ? __builtin_nanf("")
                         : fmaxf(fmaxf(sm.wfmax[0], sm.wfmax[1]), fmaxf(sm.wfmax[2], sm.wfmax[3]));
  uint32_t qn = 0u;
  for (int s = tid; s < K; s += kBlock) {
    const uint32_t key = (uint32_t)(h.leaf[s] >> 32);
    const float x = (key == 0xFFFFFFFFu) ? __builtin_nanf("") : key_float(key);
    const float q = (float)exp(((double)x - (double)M) * (double)p.inv_t);
    h.q[s] = q;
    qn |= (q != q) ? 1u : 0u;
  }
  qn = wave_or_u32(qn);
  __syncthreads();
  if (lane == 0) sm.xw[wv] = qn;
  __syncthreads();
  const bool qnan = (sm.xw[0] | sm.xw[1] | sm.xw[2] | sm.xw[3]) != 0u;
  if (tid == 0) {  // sums and Min-P in slot order (:386-410)
    double Sv = 0.0;
    for (int k = 0; k < K; ++k) Sv = Sv + (double)h.q[k];
    if (p.min_p > 0.0f) {
      float best = h.q[0];
      for (int k = 1; k < K; ++k)
        if (h.q[k] > best) best = h.q[k];
      const float thr = best * p.min_p;
      Sv = 0.0;
      for (int k = 0; k < K; ++k) {
        if (h.q[k] < thr)
          h.q[k] = 0.0f;
        else
          Sv = Sv + (double)h.q[k];
      }
    }
    sm.S = Sv;
  }
  __syncthreads();
  int64_t N = 1;
  while (N < K) N <<= 1;
  // draw order in vals[]: the stable descending sort of Top-P (:412-429), else slot order
  if (p.top_p < 1.0f && !qnan) {
    for (int64_t s = tid; s < N; s += kBlock)
      h.keys[s] = (s < K) ? (((uint64_t)__float_as_uint(h.q[s]) << 32) | (0xFFFFFFFFu - (uint32_t)s)) : 0ull;
    __syncthreads();
    hbm_sort_desc(h.keys, nullptr, N);
    for (int r = tid; r < K; r += kBlock) h.vals[r] = 0xFFFFFFFFu - (uint32_t)h.keys[r];
  } else if (p.top_p < 1.0f) {
    if (tid == 0) {  // NaN among q: the reference's insertion sort, literally
      for (int r = 0; r < K; ++r) h.vals[r] = (uint32_t)r;
      for (int i = 1; i < K; ++i) {
        const uint32_t si = h.vals[i];
        const float qv = h.q[si];
        int j = i - 1;
        while (j >= 0 && h.q[h.vals[j]] < qv) {
          h.vals[j + 1] = h.vals[j];
          --j;
        }
        h.vals[j + 1] = si;
      }
    }
  } else {
    for (int r = tid; r < K; r += kBlock) h.vals[r] = (uint32_t)r;
  }
  __syncthreads();
  for (int r = tid; r < K; r += kBlock) {
    const uint32_t s = h.vals[r];
    h.q_ord[r] = h.q[s];
    h.i_ord[r] = (int32_t)((uint32_t)h.leaf[s] & kXbIdxMask);
  }
  __syncthreads();
  if (tid == 0) {
    double Sv = sm.S;
    if (p.top_p < 1.0f) {  // Top-P cut (:431-444)
      const double target = (double)p.top_p * Sv;
      double C = 0.0;
      Sv = 0.0;
      for (int r = 0; r < K; ++r) {
        if (C < target && h.q_ord[r] > 0.0f) {
          C = C + (double)h.q_ord[r];
          Sv = Sv + (double)h.q_ord[r];
        } else {
          h.q_ord[r] = 0.0f;
        }
      }
    }
    const double t = (double)sm.uval * Sv;  // draw (:447-459)
    double C = 0.0;
    int32_t tok = h.i_ord[K - 1];
    uint32_t fl = kRowTopkReplay | kRowFallback;
    for (int r = 0; r < K; ++r) {
      C = C + (double)h.q_ord[r];
      if (C > t) {
        tok = h.i_ord[r];
        fl = kRowTopkReplay;
        break;
      }
    }
    if (qnan || !(M == M)) fl |= kRowNan;
    p.out.tokens[row] = tok;
    if (p.out.flags) p.out.flags[row] = fl;
    sm.S = Sv;
  }
  __syncthreads();
  if (p.out.topk_idx || p.out.topk_prob) {
    // canonical order: value descending, then lower index (NaN first)
    for (int64_t r = tid; r < N; r += kBlock) {
      uint64_t key = 0ull;
      if (r < K) {
        const uint32_t s = h.vals[r];
        const uint32_t vk = (uint32_t)(h.leaf[s] >> 32);
        key = ((uint64_t)vk << 32) | (kXbIdxMask - (uint32_t)h.i_ord[r]);
      }
      h.keys[r] = key;
    }
    __syncthreads();
    for (int64_t r = tid; r < N; r += kBlock) h.vals[r] = (uint32_t)r;
    __syncthreads();
    hbm_sort_desc(h.keys, h.vals, N);
    for (int j = tid; j < K; j += kBlock) {
      const uint32_t r = h.vals[j];
      const int64_t o = (int64_t)row * p.out.topk_stride + j;
      if (p.out.topk_idx) p.out.topk_idx[o] = h.i_ord[r];
      if (p.out.topk_prob) p.out.topk_prob[o] = (sm.S > 0.0) ? (float)((double)h.q_ord[r] / sm.S) : 0.0f;
    }
  }
}

__global__ __launch_bounds__(kBlock) void k_topk_huge_vec(CallParams p) { topk_body_huge<true>(p); }
__global__ __launch_bounds__(kBlock) void k_topk_huge_scalar(CallParams p) { topk_body_huge<false>(p); }

// 16-byte aligned rows: four workgroups per CU (<= 128 VGPRs, no spills).
__global__ __launch_bounds__(kBlock, 4) void k_topk_vec(CallParams p) { topk_body<true>(p); }
__global__ __launch_bounds__(kBlock) void k_topk_scalar(CallParams p) { topk_body<false>(p); }

// =============================================================================
// Full-softmax path (Sampler.pas:461-527): s = fl32(L*invT), M = max s,
// q = fl32(exp(s - M)), S = sum q, first index whose running sum exceeds
// u*S (index order); any NaN (or +inf, or an all -inf row) makes S NaN and
// the reference falls back to V-1.  TopP is not applied here (:461-527).
//
// Single pass (Min-P off): each chunk reduces its weights exp(s - m_c)
// relative to its own maximum m_c, per 4096-logit wave segment; the last
// workgroup rescales by exp(m_c - M), finds the target chunk and segment,
// and rescans that one segment.  With Min-P on, k_full_max first finds M and
// the weights are the reference's q with q < MinP zeroed (Qmax = 1).
// =============================================================================
// e^x for the single pass's weights, x = s - m <= 0 (or -inf): the hardware
// 2^y (v_exp_f32, 1 ulp) of y = fl32(x log2 e).  The product's rounding
// shifts y by at most 2^-25 |y|, so a weight is within (|y| 2^-25 ln 2 +
// 2^-23) of e^x relative, and e^x |x| <= 1/e bounds what any weight adds to
// a running sum's error: far inside the draw's 1e-6 boundary tolerance.
// Weights below 2^-126 may come out as 0.  (The exact pass, with Min-P,
// computes the reference's fl32(exp(double)) instead.)
__device__ __forceinline__ float exp_nonpos(float x) {
  return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

struct FullSmem {
  PenaltySmem pen;  // stream phase: the fused penalty's table
  float wm[kWaves];
  uint32_t wf[kWaves];
  double wd[kWaves];
  double wtot[kWaves];
  int32_t last;
  int32_t cstar;  // finish: -1 when the row's weights are not finite
  int32_t whit[kWaves];
  int32_t wlast[kWaves];
  float whitw[kWaves];  // the weight at whit / wlast
  float wlastw[kWaves];
  // the target segment, set by wave 0 for the rescan
  int32_t seg0;
  float tcm;
  float M;
  double before;
  double scale;
  double total;
  double tval;
};

template <bool VEC>
__global__ __launch_bounds__(kBlock) void k_full_max(CallParams p0) {
  __shared__ float s_m[kWaves];
  __shared__ uint32_t s_f[kWaves];
  __shared__ PenaltySmem ps;
  int row, chunk;
  block_row_chunk(p0.nchunks, p0.rows, row, chunk);
  if (!row_on_path(p0, row, kPathFull)) return;
  const CallParams p = for_row(p0, row);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const float *L = p.logits + (int64_t)row * p.stride;
  const int c0 = chunk * kChunk;
  const int clen = min(kChunk, p.vocab - c0);
  PenaltyPrefetch pf;
  if (p.fuse_penalty) {
    penalty_prefetch(p, row, pf);
    penalty_clear(ps);
  }
  float v[kPerThread];
  load_chunk<VEC>(L + c0, clen, wv, lane, v, -INFINITY);
  // the fused penalty of an exact (Min-P) full pass: applied here, in place,
  // so k_full reads the penalised row
  if (p.fuse_penalty) penalty_pass<false>(p, row, c0, clen, pf, v, ps);
  float m = -INFINITY;
  bool bad = false;
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    if (chunk_pos(wv, lane, i) < clen) {
      const float s = v[i] * p.inv_t;
      m = fmaxf(m, s);
      bad = bad || (s != s);
    }
  }
  m = wave_max_f32(m);
  const uint64_t b = __ballot(bad);
  if (lane == 0) {
    s_m[wv] = m;
    s_f[wv] = b != 0ull;
  }
  __syncthreads();
  if (tid == 0) {
    FullMeta *fm = p.fmeta + (int64_t)row * p.nchunks + chunk;
    const float mc = fmaxf(fmaxf(s_m[0], s_m[1]), fmaxf(s_m[2], s_m[3]));
    const uint32_t fc = s_f[0] | s_f[1] | s_f[2] | s_f[3];
    xstore(&fm->w[0], (uint64_t)__float_as_uint(mc) | ((uint64_t)fc << 32));
  }
}

template <bool VEC, bool EXACT>
__global__ __launch_bounds__(kBlock) void k_full(CallParams p0) {
  __shared__ FullSmem sm;
  int row, chunk;
  block_row_chunk(p0.nchunks, p0.rows, row, chunk);
  if (!row_on_path(p0, row, kPathFull)) return;
  const CallParams p = for_row(p0, row);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int S = p.nchunks, V = p.vocab;
  const float *L = p.logits + (int64_t)row * p.stride;
  FullMeta *fm = p.fmeta + (int64_t)row * S;
  const int c0 = chunk * kChunk;
  const int clen = min(kChunk, V - c0);
  RngPre rp = rng_prefetch(p.rng, row);  // one vector load, in flight with the chunk
  // the fused penalty (without Min-P; with it, k_full_max applied it)
  const bool pen = !EXACT && p.fuse_penalty;
  PenaltyPrefetch pf;
  if (pen) {
    penalty_prefetch(p, row, pf);
    penalty_clear(sm.pen);
  }
  float v[kPerThread];
  load_chunk<VEC, true>(L + c0, clen, wv, lane, v, -INFINITY);
  if (pen) penalty_pass<true>(p, row, c0, clen, pf, v, sm.pen);

  // s = fl32(L * invT); positions past the row end (loaded as -inf) weigh
  // nothing.  v_maximum propagates NaN, so one test of the thread maximum
  // finds a NaN anywhere in its logits.  Only with invT = 0 (T = +inf) would
  // a padding position turn into NaN (-inf * 0): the short last chunk then
  // resets those positions.
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) v[i] = v[i] * p.inv_t;
  if (clen < kChunk && !(p.inv_t > 0.0f)) {
#pragma unroll
    for (int i = 0; i < kPerThread; ++i)
      if (chunk_pos<true>(wv, lane, i) >= clen) v[i] = -INFINITY;
  }
  float m = v[0];
#pragma unroll
  for (int i = 1; i < kPerThread; ++i) m = vmax(m, v[i]);
  const bool bad = (m != m);
  float base;
  if (EXACT) {
    // row maximum from the k_full_max records of this row
    float mm = -INFINITY;
    for (int c = tid; c < S; c += kBlock) mm = fmaxf(mm, __uint_as_float((uint32_t)xload(&fm[c].w[0])));
    mm = wave_max_f32(mm);
    if (lane == 0) sm.wm[wv] = mm;
    __syncthreads();
    base = fmaxf(fmaxf(sm.wm[0], sm.wm[1]), fmaxf(sm.wm[2], sm.wm[3]));
  } else {
    m = wave_max_f32(m);
    const uint64_t b = __ballot(bad);
    if (lane == 0) {
      sm.wm[wv] = m;
      sm.wf[wv] = b != 0ull;
    }
    __syncthreads();
    base = fmaxf(fmaxf(sm.wm[0], sm.wm[1]), fmaxf(sm.wm[2], sm.wm[3]));
  }
  double acc = 0.0;
  if (base > -INFINITY && base < INFINITY) {
    if (EXACT) {
#pragma unroll
      for (int i = 0; i < kPerThread; ++i) {
        const float q = (float)exp((double)v[i] - (double)base);
        acc += (double)((q < p.min_p) ? 0.0f : q);
      }
    } else {
      // a pairwise fp32 tree (no serial chain of fp64 adds): the sum of 64
      // non-negative weights is within 6 * 2^-24 (relative) of the exact one,
      // inside the single pass's draw tolerance; the target segment is
      // rescanned in fp64 by the finish
#pragma unroll
      for (int i = 0; i < kPerThread; ++i) v[i] = exp_nonpos(v[i] - base);
#pragma unroll
      for (int h = kPerThread / 2; h >= 1; h >>= 1) {
#pragma unroll
        for (int i = 0; i < h; ++i) v[i] = v[i] + v[i + h];
      }
      acc = (double)v[0];
    }
  }
  const double ws = wave_sum_f64(acc);
  if (lane == 0) sm.wd[wv] = ws;
  __syncthreads();
  if (tid == 0) {
    FullMeta *me = fm + chunk;
    double d = 0.0;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      xstore(&me->w[2 + w], (uint64_t)__double_as_longlong(sm.wd[w]));
      d = d + sm.wd[w];
    }
    xstore(&me->w[1], (uint64_t)__double_as_longlong(d));
    if (!EXACT) {
      const uint32_t fc = sm.wf[0] | sm.wf[1] | sm.wf[2] | sm.wf[3];
      xstore(&me->w[0], (uint64_t)__float_as_uint(base) | ((uint64_t)fc << 32));
    }
  }
  if (!last_of_row(p.tickets, row, S, &sm.last, [] {})) return;

  // ---- finish (last workgroup of the row) ----
  // Wave 0 reads the chunk records and finds the row maximum M, the chunk
  // weights exp(m_c - M) D_c and their running sums in chunk order, the
  // target chunk (the first whose running sum exceeds t = u S) and, in it,
  // the target 4096-logit segment; the workgroup meets at one barrier and
  // rescans that segment.
  if (wv == 0) {
    float u = 0.0f;
    RngVals rv = rng_unpack(rp);  // wave 0, every lane
    if (lane == 0) u = rng_draw(p.rng, row, rv);
    u = __shfl(u, 0);
    // lane l holds chunks [l * per, l * per + per); each record comes in one
    // round trip
    constexpr int kPer = kMaxChunks / 64;
    const int per = (S + 63) >> 6;
    float mc[kPer];
    double dc[kPer], cw[kPer][kWaves];
    uint32_t fl = 0u;
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int c = lane * per + k;
      mc[k] = -INFINITY;
      dc[k] = 0.0;
#pragma unroll
      for (int w = 0; w < kWaves; ++w) cw[k][w] = 0.0;
      if (k < per && c < S) {
        uint64_t r[2 + kWaves];
#pragma unroll
        for (int j = 0; j < 2 + kWaves; ++j) r[j] = xload(&fm[c].w[j]);
        mc[k] = __uint_as_float((uint32_t)r[0]);
        fl |= (uint32_t)(r[0] >> 32);
        dc[k] = __longlong_as_double((long long)r[1]);
#pragma unroll
        for (int w = 0; w < kWaves; ++w) cw[k][w] = __longlong_as_double((long long)r[2 + w]);
        mx = fmaxf(mx, mc[k]);
      }
    }
    const float M = EXACT ? base : wave_max_f32(mx);
    const bool rowbad = wave_or_u32(fl) != 0u || !(M > -INFINITY && M < INFINITY);
    if (rowbad) {
      if (lane == 0) {
        p.out.tokens[row] = V - 1;
        if (p.out.flags) p.out.flags[row] = kRowFull | kRowNan | kRowFallback;
        const int64_t o = (int64_t)row * p.out.topk_stride;
        if (p.out.topk_idx) p.out.topk_idx[o] = V - 1;
        if (p.out.topk_prob) p.out.topk_prob[o] = 0.0f;  // the weights are not finite
        sm.cstar = -1;
      }
    } else {
      double wc[kPer], part[kPer], acc = 0.0;
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        wc[k] = 0.0;
        if (k < per && lane * per + k < S) wc[k] = EXACT ? dc[k] : dc[k] * exp((double)mc[k] - (double)M);
        acc = acc + wc[k];
        part[k] = acc;
      }
      const double lincl = wave_incl_scan_f64(acc);
      const double total = __longlong_as_double((long long)readlane64((uint64_t)__double_as_longlong(lincl), 63));
      const double t = (double)u * total;
      // incl[k]: the running sum through chunk lane * per + k; prv[k]: through
      // the chunk before it (for k = 0 the previous lane's last, 0 on lane 0)
      const double lexcl = lincl - acc;
      double incl[kPer], prv[kPer];
#pragma unroll
      for (int k = 0; k < kPer; ++k) incl[k] = lexcl + part[k];
      double lastincl = incl[0];
#pragma unroll
      for (int k = 1; k < kPer; ++k)
        if (k < per) lastincl = incl[k];
      const double up = __longlong_as_double((long long)__shfl_up((long long)__double_as_longlong(lastincl), 1));
      prv[0] = lane ? up : 0.0;
#pragma unroll
      for (int k = 1; k < kPer; ++k) prv[k] = incl[k - 1];
      // the first chunk whose running sum exceeds t; if rounding put t at or
      // past the total, the last chunk that weighs (its running sum grows)
      int hk = -1, nk = -1;
#pragma unroll
      for (int k = kPer - 1; k >= 0; --k) {
        const bool real = k < per && lane * per + k < S;
        if (real && incl[k] > t) hk = k;
        if (real && nk < 0 && incl[k] > prv[k]) nk = k;
      }
      const uint64_t hb = __ballot(hk >= 0), nb = __ballot(nk >= 0);
      int sl, sk;
      if (hb) {
        sl = __ffsll((unsigned long long)hb) - 1;
        sk = __shfl(hk, sl);
      } else if (nb) {
        sl = 63 - __clzll((long long)nb);
        sk = __shfl(nk, sl);
      } else {
        sl = (S - 1) / per;
        sk = (S - 1) - sl * per;
      }
      if (lane == sl) {
        // the target chunk's record, selected without indexing the
        // register arrays by a run-time value
        float tcm = mc[0];
        double tdw[kWaves], before = prv[0];
#pragma unroll
        for (int w = 0; w < kWaves; ++w) tdw[w] = cw[0][w];
#pragma unroll
        for (int k = 1; k < kPer; ++k)
          if (k == sk) {
            tcm = mc[k];
            before = prv[k];
#pragma unroll
            for (int w = 0; w < kWaves; ++w) tdw[w] = cw[k][w];
          }
        const double scale = EXACT ? 1.0 : exp((double)tcm - (double)M);
        const double b0 = before;
        int ws_ = -1;
        for (int w = 0; w < kWaves; ++w) {
          const double ww = tdw[w] * scale;
          if (before + ww > t) {
            ws_ = w;
            break;
          }
          before = before + ww;
        }
        if (ws_ < 0) {
          ws_ = kWaves - 1;
          before = b0;
          for (int w = 0; w < kWaves - 1; ++w) before = before + tdw[w] * scale;
          while (ws_ > 0 && tdw[ws_] == 0.0) {
            --ws_;
            before = before - tdw[ws_] * scale;
          }
        }
        sm.seg0 = (sl * per + sk) * kChunk + ws_ * kWaveSpan;
        sm.before = before;
        sm.scale = scale;
        sm.total = total;
        sm.tval = t;
        sm.tcm = tcm;
        sm.M = M;
        sm.cstar = 0;
      }
    }
  }
  __syncthreads();
  if (sm.cstar < 0) return;
  // rescan the target segment: thread tid takes 16 consecutive logits (the
  // wave's four loads cover its 4 KiB; penalised values written by the row's
  // other workgroups are read past the caches)
  const int seg0 = sm.seg0;
  const double scale = sm.scale, total = sm.total, t = sm.tval;
  const float tcm = sm.tcm, M = sm.M;
  const int e0 = seg0 + tid * 16;
  float w16[16];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int e = e0 + 4 * q;
    float x[4];
    if (VEC && e < V) {  // 16-byte aligned rows, V % 4 = 0: the float4 lies in the row
      const f32x4 f = p.fuse_penalty ? xload4(&L[e]) : *reinterpret_cast<const f32x4 *>(&L[e]);
      x[0] = f[0];
      x[1] = f[1];
      x[2] = f[2];
      x[3] = f[3];
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        x[i] = (e + i < V) ? (p.fuse_penalty ? xloadf(&L[e + i]) : L[e + i]) : 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float w = 0.0f;
      if (e + i < V) {
        const float s = x[i] * p.inv_t;
        if (EXACT) {
          const float q = (float)exp((double)s - (double)M);
          w = (q < p.min_p) ? 0.0f : q;
        } else {
          w = exp_nonpos(s - tcm);
        }
      }
      w16[4 * q + i] = w;
    }
  }
  double tsum = 0.0;
#pragma unroll
  for (int i = 0; i < 16; ++i) tsum += (double)w16[i];
  double segtot;
  const double tb = block_excl_scan_f64(tsum * scale, sm.wtot, segtot);
  double run = sm.before + tb;
  int hit = -1, lastnz = -1;
  float hitw = 0.0f, lastw = 0.0f;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const double w = (double)w16[i] * scale;
    if (w16[i] > 0.0f) {
      lastnz = e0 + i;
      lastw = w16[i];
    }
    run = run + w;
    if (hit < 0 && w16[i] > 0.0f && run > t) {
      hit = e0 + i;
      hitw = w16[i];
    }
  }
  // thread order is index order here: the first hit is the lowest thread's,
  // the last non-zero weight the highest thread's (per wave by ballot; LDS
  // atomics with a different value per lane would run a scalar loop per wave)
  const uint64_t hb = __ballot(hit >= 0), nb = __ballot(lastnz >= 0);
  const int hl = hb ? __ffsll((unsigned long long)hb) - 1 : 0, nl = nb ? 63 - __clzll((long long)nb) : 0;
  const int hv = __shfl(hit, hl);  // every lane active
  const int nv = __shfl(lastnz, nl);
  const float hw = __shfl(hitw, hl), nw = __shfl(lastw, nl);
  if (lane == 0) {
    sm.whit[wv] = hb ? hv : 0x7FFFFFFF;
    sm.wlast[wv] = nb ? nv : -1;
    sm.whitw[wv] = hw;
    sm.wlastw[wv] = nw;
  }
  __syncthreads();
  if (tid == 0) {
    int32_t tok;
    uint32_t fl2 = kRowFull;
    int32_t h = 0x7FFFFFFF, ln = -1;
    float hw2 = 0.0f, lw2 = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      if (h == 0x7FFFFFFF) {
        h = sm.whit[w];
        hw2 = sm.whitw[w];
      }
      if (sm.wlast[w] >= 0) {
        ln = sm.wlast[w];
        lw2 = sm.wlastw[w];
      }
    }
    float wt = 0.0f;
    if (h != 0x7FFFFFFF) {
      tok = h;
      wt = hw2;
    } else if (ln >= 0) {
      tok = ln;
      wt = lw2;
    } else {
      tok = V - 1;
      fl2 |= kRowFallback;
    }
    p.out.tokens[row] = tok;
    if (p.out.flags) p.out.flags[row] = fl2;
    // entry 0 of the top-K outputs: the drawn token and its probability q / S
    const int64_t o = (int64_t)row * p.out.topk_stride;
    if (p.out.topk_idx) p.out.topk_idx[o] = tok;
    if (p.out.topk_prob) p.out.topk_prob[o] = (total > 0.0) ? (float)((double)wt * scale / total) : 0.0f;
  }
}

// =============================================================================
// History ring (Sampler.pas:530-549) and RNG seeding (Sampler.pas:194-241).
// =============================================================================
// AddToHistory (Sampler.pas:530-539) for rows [row0, row0 + rows): the ring of
// row r holds its own window's ids at hist + r * stride.
// The history positions of one row after the penalty, for the host entry
// point to mirror the in-place penalty into the caller's buffer: slot j < the
// row's count holds id << 32 | bits(L[id]) for an in-range history id, every
// other slot ~0.  Only history positions are ever penalised, so writing these
// back reproduces the whole penalised row.
__global__ void k_hist_gather(const int32_t *__restrict__ hist_row, int32_t slots,
                              const RowState *__restrict__ rs_row, const float *__restrict__ L, int32_t vocab,
                              uint64_t *__restrict__ out) {
  const int cnt = min(rs_row->hist_count, slots);
  for (int j = threadIdx.x; j < slots; j += blockDim.x) {
    uint64_t e = ~0ull;
    if (j < cnt) {
      const int32_t id = hist_row[j];
      if (id >= 0 && id < vocab) e = ((uint64_t)(uint32_t)id << 32) | __float_as_uint(L[id]);
    }
    out[j] = e;
  }
}

__global__ void k_hist_add(const int32_t *__restrict__ tokens, int32_t tok_const, int32_t row0,
                           int32_t rows, int32_t *__restrict__ hist, int32_t stride,
                           RowState *__restrict__ rs) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int row = row0 + r;
  RowState &s = rs[row];
  const int W = min(s.window, stride);
  if (W <= 0) return;
  const int32_t tok = tokens ? tokens[r] : tok_const;
  hist[(int64_t)row * stride + s.hist_pos] = tok;
  s.hist_pos = (s.hist_pos + 1) % W;
  if (s.hist_count < W) s.hist_count = s.hist_count + 1;
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t &s) {
  s += 0x9E3779B97F4A7C15ull;
  uint64_t z = s;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// Clears the rings of rows [row0, row0 + rows) (and sets their window when
// window >= 0) and/or reseeds them (SeedPRNG, Sampler.pas:224-241): xoshiro
// from seed + row (rows of the sampler-wide config behave as samplers with
// Seed + r), or from `seed` itself (a row with its own config or a restored
// checkpoint).  The Philox stream of a row is keyed by `pkey` and counts on
// (step, prow), prow < 0 standing for the row itself.
__global__ void k_row_reset(RowState *__restrict__ rs, int32_t row0, int32_t rows, int clear_hist,
                            int32_t window, int reseed, uint64_t seed, int add_row, uint64_t pkey,
                            int32_t prow) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const int row = row0 + r;
  RowState &s = rs[row];
  if (clear_hist) {
    s.hist_pos = 0;
    s.hist_count = 0;
    if (window >= 0) s.window = window;
  }
  if (reseed) {
    uint64_t st = seed + (add_row ? (uint64_t)row : 0ull);
    s.key = pkey;
    s.ctr_row = prow < 0 ? row : prow;
    s.rng[0] = splitmix64(st);
    s.rng[1] = splitmix64(st);
    s.rng[2] = splitmix64(st);
    s.rng[3] = splitmix64(st);
    s.step = 0;
  }
}

// State of rows [0, rows) for a call that brings its own history and uniforms
// (no sampler object): each row's ring is the caller's `count[r]` ids (clamped
// to [0, window]), its RNG words are zero (the uniforms are injected), and its
// arrival ticket is cleared.  A kernel rather than a memset, so that a
// captured call replays it.
__global__ void k_rows_prepare(RowState *__restrict__ rs, uint32_t *__restrict__ tickets, int32_t rows,
                               const int32_t *__restrict__ count, int32_t window) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  RowState s{};
  const int32_t c = count ? count[r] : 0;
  s.hist_count = window > 0 ? min(max(c, 0), window) : 0;
  s.window = window;
  s.ctr_row = r;
  rs[r] = s;
  tickets[r] = 0u;
}

// =============================================================================
// Host launchers
// =============================================================================
static inline dim3 grid_rows_chunks(const CallParams &p) {
  return dim3((unsigned)(p.rows * p.nchunks));
}

hipError_t launch_penalty(const CallParams &p, hipStream_t st) {
  hipLaunchKernelGGL(k_penalty, dim3(p.rows), dim3(kBlock), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_greedy(const CallParams &p, hipStream_t st) {
  if (p.vec)
    hipLaunchKernelGGL(k_greedy<true>, grid_rows_chunks(p), dim3(kBlock), 0, st, p);
  else
    hipLaunchKernelGGL(k_greedy<false>, grid_rows_chunks(p), dim3(kBlock), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_topk(const CallParams &p, hipStream_t st) {
  if (p.cand_cap > kCandCap) {  // some row has 64 < K <= kKBig: stream phase, then one workgroup per row
    if (p.vec) {
      hipLaunchKernelGGL(k_topk_big_stream_vec, grid_rows_chunks(p), dim3(kBlock), 0, st, p);
      hipLaunchKernelGGL(k_topk_big_finish_vec, dim3(p.rows), dim3(kBlock), 0, st, p);
    } else {
      hipLaunchKernelGGL(k_topk_big_stream_scalar, grid_rows_chunks(p), dim3(kBlock), 0, st, p);
      hipLaunchKernelGGL(k_topk_big_finish_scalar, dim3(p.rows), dim3(kBlock), 0, st, p);
    }
  } else if (p.vec) {
    hipLaunchKernelGGL(k_topk_vec, grid_rows_chunks(p), dim3(kBlock), 0, st, p);
    if (p.exact_kernel) hipLaunchKernelGGL(k_topk_exact_vec, dim3(p.rows), dim3(kBlock), 0, st, p);
  } else {
    hipLaunchKernelGGL(k_topk_scalar, grid_rows_chunks(p), dim3(kBlock), 0, st, p);
    if (p.exact_kernel) hipLaunchKernelGGL(k_topk_exact_scalar, dim3(p.rows), dim3(kBlock), 0, st, p);
  }
  return hipGetLastError();
}

hipError_t launch_topk_huge(const CallParams &p, hipStream_t st) {
  if (p.vec)
    hipLaunchKernelGGL(k_topk_huge_vec, dim3(p.rows), dim3(kBlock), 0, st, p);
  else
    hipLaunchKernelGGL(k_topk_huge_scalar, dim3(p.rows), dim3(kBlock), 0, st, p);
  return hipGetLastError();
}

int64_t topk_huge_row_bytes(int K) { return huge_row_bytes(K); }

hipError_t launch_full(const CallParams &p, hipStream_t st) {
  const dim3 g = grid_rows_chunks(p);
  if (p.min_p > 0.0f) {
    if (p.vec) {
      hipLaunchKernelGGL(k_full_max<true>, g, dim3(kBlock), 0, st, p);
      hipLaunchKernelGGL((k_full<true, true>), g, dim3(kBlock), 0, st, p);
    } else {
      hipLaunchKernelGGL(k_full_max<false>, g, dim3(kBlock), 0, st, p);
      hipLaunchKernelGGL((k_full<false, true>), g, dim3(kBlock), 0, st, p);
    }
  } else {
    if (p.vec)
      hipLaunchKernelGGL((k_full<true, false>), g, dim3(kBlock), 0, st, p);
    else
      hipLaunchKernelGGL((k_full<false, false>), g, dim3(kBlock), 0, st, p);
  }
  return hipGetLastError();
}

hipError_t launch_hist_add(const int32_t *tokens, int32_t tok_const, int32_t row0, int32_t rows,
                           int32_t *hist, int32_t hist_len, RowState *rs, hipStream_t st) {
  const int nb = (rows + 255) / 256;
  hipLaunchKernelGGL(k_hist_add, dim3(nb), dim3(256), 0, st, tokens, tok_const, row0, rows, hist,
                     hist_len, rs);
  return hipGetLastError();
}

hipError_t launch_hist_gather(const int32_t *hist_row, int32_t slots, const RowState *rs_row, const float *L,
                              int32_t vocab, uint64_t *out, hipStream_t st) {
  hipLaunchKernelGGL(k_hist_gather, dim3(1), dim3(256), 0, st, hist_row, slots, rs_row, L, vocab, out);
  return hipGetLastError();
}

hipError_t launch_row_reset(RowState *rs, int32_t row0, int32_t rows, bool clear_hist, int32_t window,
                            bool reseed, uint64_t seed, bool add_row, hipStream_t st, uint64_t pkey,
                            int32_t prow) {
  const int nb = (rows + 255) / 256;
  hipLaunchKernelGGL(k_row_reset, dim3(nb), dim3(256), 0, st, rs, row0, rows, clear_hist ? 1 : 0,
                     window, reseed ? 1 : 0, seed, add_row ? 1 : 0, pkey, prow);
  return hipGetLastError();
}

hipError_t launch_rows_prepare(RowState *rs, uint32_t *tickets, int32_t rows, const int32_t *count,
                               int32_t window, hipStream_t st) {
  const int nb = (rows + 255) / 256;
  hipLaunchKernelGGL(k_rows_prepare, dim3(nb), dim3(256), 0, st, rs, tickets, rows, count, window);
  return hipGetLastError();
}

}  // namespace vdx
