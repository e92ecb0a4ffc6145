// vdx_api.hip -- C ABI of libvdxsampler.so (declared in include/vdx_sampler.h).
//
// Host half of the drop-in for TVdxSampler (src/VindexLLM.Sampler.pas:37-91):
// configuration, per-row history rings and RNG state in HBM, workspace
// management, and the launches of the kernels in vdx_kernels.hip.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <time.h>

#include <mutex>
#include <string>
#include <vector>

#include "vdx_sampler.h"
#include "vdx_internal.hpp"

using namespace vdx;

struct vdx_sampler {
  int32_t device = 0;
  int32_t max_rows = 0;
  vdx_sampler_config cfg{};
  int32_t rng_kind = VDX_RNG_XOSHIRO;
  uint64_t seed_base = 0;  // resolved seed: Seed, or a timer value when Seed = 0
  bool hist_maybe = false; // some row may hold history ids (host Process write-back)
  hipStream_t stream = nullptr;
  RowState *d_rows = nullptr;
  int32_t *d_hist = nullptr;
  int32_t hist_len = 0;     // ring stride: >= every row's window
  // rows with their own configs (vdx_sampler_set_row_config)
  bool per_row = false;
  std::vector<vdx_sampler_config> row_cfg;  // every row's config (= cfg without per-row configs)
  std::vector<uint8_t> own_seed;            // row seeded from its own Seed (else seed_base + row)
  std::vector<uint64_t> own_seed_val;       // that seed, resolved (timer value for Seed = 0): the xoshiro seed
  std::vector<uint64_t> own_pkey;           // the row's Philox key (its own seed, or a restored stream's)
  std::vector<int32_t> own_prow;            // the row's Philox counter row (-1: the row itself)
  RowCfg *d_rcfg = nullptr;
  // a call whose rows take several paths runs their kernels side by side:
  // forked onto these streams after the penalty, joined before returning
  hipStream_t aux[2] = {nullptr, nullptr};
  hipEvent_t ev_fork = nullptr;
  hipEvent_t ev_join[2] = {nullptr, nullptr};
  // workspace (sized for ws_chunks chunks per row, ws_cap candidate slots per chunk)
  int32_t ws_chunks = 0;
  int32_t ws_cap = 0;
  // rows with K > kKBig: huge_rows rows of huge_rb bytes (slots and sort space)
  uint8_t *d_huge = nullptr;
  int32_t huge_rows = 0;
  int64_t huge_rb = 0;
  ChunkMeta *d_meta = nullptr;
  Cand *d_cand = nullptr;
  FullMeta *d_fmeta = nullptr;
  uint64_t *d_gpart = nullptr;
  uint32_t *d_tickets = nullptr;
  // lm_head logits workspace (rows x vocab, row stride lm_stride)
  float *d_lm = nullptr;
  size_t lm_cap = 0;  // floats
  float *d_xt = nullptr;  // element-major hidden copy (16 x in_dim)
  int32_t xt_dim = 0;
  // host-pointer Process
  float *d_row = nullptr;
  int32_t row_cap = 0;
  int32_t *d_tok = nullptr;
  uint64_t *d_pairs = nullptr;  // penalised history positions of row 0 (id, value)
  uint64_t *h_pairs = nullptr;  // pinned host copy
  int32_t pairs_cap = 0;
  // instrumentation: three events per timed call
  bool timing = false;
  std::vector<hipEvent_t> ev;
  int32_t n_timed = 0;
  std::string err;
};

constexpr int32_t kTimedCalls = 4096;

static std::string g_create_err;
static thread_local std::string g_call_err;  // sampler-less entry points

static int fail(vdx_sampler *s, int code, const std::string &msg) {
  if (s) s->err = msg;
  return code;
}

static int hip_fail(vdx_sampler *s, hipError_t e, const char *where) {
  std::string m = std::string(where) + ": " + hipGetErrorString(e);
  return fail(s, VDX_E_HIP, m);
}

#define HIP_TRY(s, expr)                                   \
  do {                                                     \
    hipError_t _e = (expr);                                \
    if (_e != hipSuccess) return hip_fail((s), _e, #expr); \
  } while (0)

static uint64_t timer_seed() {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

static int32_t chunks_for(int32_t vocab) { return (vocab + kChunk - 1) / kChunk; }

// Reseeds row `row` the way its config says: from its own resolved Seed (or
// the stream a restored checkpoint was taken from), or as row `row` of the
// sampler-wide config (xoshiro from seed_base + row, Philox keyed by seed_base).
static int reseed_row(vdx_sampler *s, int32_t row) {
  if (s->own_seed[row])
    HIP_TRY(s, launch_row_reset(s->d_rows, row, 1, false, -1, true, s->own_seed_val[row], false, s->stream,
                                s->own_pkey[row], s->own_prow[row]));
  else
    HIP_TRY(s, launch_row_reset(s->d_rows, row, 1, false, -1, true, s->seed_base, true, s->stream,
                                s->seed_base, -1));
  return VDX_OK;
}

// Reseeds rows [0, max_rows): SeedPRNG (Sampler.pas:224-241) with Seed + row,
// or a row's own Seed.
static int reseed_all(vdx_sampler *s) {
  s->seed_base = (s->cfg.seed == 0) ? timer_seed() : (uint64_t)s->cfg.seed;
  HIP_TRY(s, launch_row_reset(s->d_rows, 0, s->max_rows, false, -1, true, s->seed_base, true, s->stream,
                              s->seed_base, -1));
  for (int32_t r = 0; r < s->max_rows; ++r)
    if (s->own_seed[r]) {
      int rc = reseed_row(s, r);
      if (rc != VDX_OK) return rc;
    }
  HIP_TRY(s, hipStreamSynchronize(s->stream));
  return VDX_OK;
}

static int32_t window_of(const vdx_sampler_config &c) { return c.repeat_window > 0 ? c.repeat_window : 0; }

// Every row gets `window`; the rings are cleared (SetConfig, Sampler.pas:137-142).
static int alloc_history(vdx_sampler *s, int32_t window) {
  if (s->d_hist) {
    (void)hipFree(s->d_hist);
    s->d_hist = nullptr;
  }
  s->hist_len = window > 0 ? window : 0;
  if (s->hist_len > 0) {
    const size_t bytes = (size_t)s->max_rows * s->hist_len * sizeof(int32_t);
    HIP_TRY(s, hipMalloc(&s->d_hist, bytes));
    HIP_TRY(s, hipMemsetAsync(s->d_hist, 0, bytes, s->stream));
  }
  HIP_TRY(s, launch_row_reset(s->d_rows, 0, s->max_rows, true, s->hist_len, false, 0, false, s->stream));
  HIP_TRY(s, hipStreamSynchronize(s->stream));
  s->hist_maybe = false;
  return VDX_OK;
}

// Widens the ring stride to `stride`, keeping every row's ids in place.
// The device must be idle.
static int grow_history(vdx_sampler *s, int32_t stride) {
  if (stride <= s->hist_len) return VDX_OK;
  int32_t *nh = nullptr;
  const size_t bytes = (size_t)s->max_rows * stride * sizeof(int32_t);
  HIP_TRY(s, hipMalloc(&nh, bytes));
  HIP_TRY(s, hipMemset(nh, 0, bytes));
  if (s->d_hist && s->hist_len > 0)
    HIP_TRY(s, hipMemcpy2D(nh, sizeof(int32_t) * stride, s->d_hist, sizeof(int32_t) * s->hist_len,
                           sizeof(int32_t) * s->hist_len, s->max_rows, hipMemcpyDeviceToDevice));
  HIP_TRY(s, hipDeviceSynchronize());
  (void)hipFree(s->d_hist);
  s->d_hist = nh;
  s->hist_len = stride;
  return VDX_OK;
}

// The fork/join streams and events of mixed-path calls (created once, on the
// first per-row config, never during a call that may be captured).
static int ensure_aux(vdx_sampler *s) {
  if (s->aux[0]) return VDX_OK;
  HIP_TRY(s, hipEventCreateWithFlags(&s->ev_fork, hipEventDisableTiming));
  for (int i = 0; i < 2; ++i) {
    HIP_TRY(s, hipStreamCreateWithFlags(&s->aux[i], hipStreamNonBlocking));
    HIP_TRY(s, hipEventCreateWithFlags(&s->ev_join[i], hipEventDisableTiming));
  }
  return VDX_OK;
}

static RowCfg row_params(const vdx_sampler_config &c) {
  RowCfg r{};
  r.greedy = c.temperature == 0.0f;
  r.inv_t = r.greedy ? 0.0f : 1.0f / c.temperature;  // Sampler.pas:325
  r.top_k = c.top_k;
  r.top_p = c.top_p;
  r.min_p = c.min_p;
  r.penalty = c.repeat_penalty;
  r.window = window_of(c);
  return r;
}

// Copies every row's parameters to the device (the device is idle).
static int upload_row_params(vdx_sampler *s) {
  std::vector<RowCfg> h((size_t)s->max_rows);
  for (int32_t r = 0; r < s->max_rows; ++r) h[r] = row_params(s->row_cfg[r]);
  HIP_TRY(s, hipMemcpy(s->d_rcfg, h.data(), sizeof(RowCfg) * h.size(), hipMemcpyHostToDevice));
  return VDX_OK;
}

// EnsureWorkspace (Sampler.pas:250-263) for the device path: grows the
// per-row chunk records when a larger vocabulary (or a TopK needing more
// candidate slots per chunk) is first seen.
static int ensure_workspace(vdx_sampler *s, int32_t vocab, int32_t cap = kCandCap) {
  const int32_t S0 = chunks_for(vocab);
  if (S0 <= s->ws_chunks && cap <= s->ws_cap) return VDX_OK;
  const int32_t S = S0 > s->ws_chunks ? S0 : s->ws_chunks;
  if (cap < s->ws_cap) cap = s->ws_cap;
  HIP_TRY(s, hipStreamSynchronize(s->stream));
  (void)hipFree(s->d_meta);
  (void)hipFree(s->d_cand);
  (void)hipFree(s->d_fmeta);
  (void)hipFree(s->d_gpart);
  s->d_meta = nullptr;
  s->d_cand = nullptr;
  s->d_fmeta = nullptr;
  s->d_gpart = nullptr;
  s->ws_chunks = 0;
  const size_t rc = (size_t)s->max_rows * S;
  HIP_TRY(s, hipMalloc(&s->d_meta, rc * sizeof(ChunkMeta)));
  HIP_TRY(s, hipMalloc(&s->d_cand, rc * (size_t)cap * sizeof(Cand)));
  HIP_TRY(s, hipMalloc(&s->d_fmeta, rc * sizeof(FullMeta)));
  HIP_TRY(s, hipMalloc(&s->d_gpart, rc * sizeof(uint64_t)));
  // every record is written by its chunk before the row's last workgroup reads it
  s->ws_chunks = S;
  s->ws_cap = cap;
  return VDX_OK;
}

// ---- allocation-free sampling ------------------------------------------------
// vdx_sample_device_noalloc keeps its workspace (row states, arrival tickets,
// chunk records, candidate slots) in one file-scope device array instead of
// memory the library allocates.  In host code the array's name is only a
// stand-in: its device address is looked up once per device
// (hipGetSymbolAddress, with that device current) and that address is what
// the kernels receive.  Every call on a device shares the device's copy.
constexpr int32_t kNoAllocRows = 1024;        // rows per call
constexpr int32_t kNoAllocRowChunks = 4096;   // rows * ceil(vocab / 16384) per call
constexpr size_t na_align(size_t x) { return (x + 255) & ~(size_t)255; }
constexpr size_t kNaRows = 0;
constexpr size_t kNaTickets = kNaRows + na_align(sizeof(RowState) * kNoAllocRows);
constexpr size_t kNaMeta = kNaTickets + na_align(sizeof(uint32_t) * kNoAllocRows);
constexpr size_t kNaCand = kNaMeta + na_align(sizeof(ChunkMeta) * kNoAllocRowChunks);
constexpr size_t kNaFullMeta = kNaCand + na_align(sizeof(Cand) * kCandCap * kNoAllocRowChunks);
constexpr size_t kNaGpart = kNaFullMeta + na_align(sizeof(FullMeta) * kNoAllocRowChunks);
constexpr size_t kNoAllocBytes = kNaGpart + na_align(sizeof(uint64_t) * kNoAllocRowChunks);
static_assert(kNoAllocBytes <= (size_t)5 << 20, "the allocation-free workspace stays under 5 MiB per device");

static __device__ __align__(256) unsigned char scratch[kNoAllocBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static unsigned char *g_scratch_ptr[kMaxDevices];  // device address of `scratch`, per device

// The device address of the current device's `scratch` (looked up on the
// first call on that device); nullptr with the message in g_call_err.
static unsigned char *scratch_on_current_device() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    g_call_err = std::string("noalloc: no current HIP device (") + hipGetErrorString(e) + ")";
    return nullptr;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    unsigned char *ptr = nullptr;
    e = hipGetSymbolAddress((void **)&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      g_call_err = std::string("noalloc: hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
      return nullptr;
    }
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

// The per-row workspace of rows with K > kKBig, grown (outside the sampling
// call's kernels) when more rows or a larger K are first seen.
static int ensure_huge(vdx_sampler *s, int32_t rows, int32_t K) {
  const int64_t rb = topk_huge_row_bytes(K);
  if (rows <= s->huge_rows && rb <= s->huge_rb) return VDX_OK;
  HIP_TRY(s, hipStreamSynchronize(s->stream));
  HIP_TRY(s, hipDeviceSynchronize());
  (void)hipFree(s->d_huge);
  s->d_huge = nullptr;
  const int32_t nr = rows > s->huge_rows ? rows : s->huge_rows;
  const int64_t nb = rb > s->huge_rb ? rb : s->huge_rb;
  s->huge_rows = 0;
  s->huge_rb = 0;
  HIP_TRY(s, hipMalloc(&s->d_huge, (size_t)nr * (size_t)nb));
  s->huge_rows = nr;
  s->huge_rb = nb;
  return VDX_OK;
}

extern "C" {

const char *vdx_sampler_version(void) { return "vdxsampler 0.1.0 (gfx950)"; }

void vdx_sampler_default_config(vdx_sampler_config *c) {
  if (!c) return;
  c->temperature = 0.0f;
  c->top_k = 0;
  c->top_p = 1.0f;
  c->min_p = 0.0f;
  c->repeat_penalty = 1.0f;
  c->repeat_window = 64;
  c->seed = 0;
}

const char *vdx_sampler_last_error(const vdx_sampler *s) {
  if (s) return s->err.c_str();
  return g_call_err.empty() ? g_create_err.c_str() : g_call_err.c_str();
}

void vdx_sampler_destroy(vdx_sampler *s) {
  if (!s) return;
  int cur = 0;
  (void)hipGetDevice(&cur);
  (void)hipSetDevice(s->device);
  if (s->stream) (void)hipStreamSynchronize(s->stream);
  (void)hipFree(s->d_rows);
  (void)hipFree(s->d_rcfg);
  (void)hipFree(s->d_hist);
  (void)hipFree(s->d_meta);
  (void)hipFree(s->d_cand);
  (void)hipFree(s->d_fmeta);
  (void)hipFree(s->d_gpart);
  (void)hipFree(s->d_huge);
  (void)hipFree(s->d_tickets);
  (void)hipFree(s->d_row);
  (void)hipFree(s->d_lm);
  (void)hipFree(s->d_xt);
  (void)hipFree(s->d_tok);
  (void)hipFree(s->d_pairs);
  if (s->h_pairs) (void)hipHostFree(s->h_pairs);
  for (hipEvent_t e : s->ev) (void)hipEventDestroy(e);
  if (s->ev_fork) (void)hipEventDestroy(s->ev_fork);
  for (int i = 0; i < 2; ++i) {
    if (s->ev_join[i]) (void)hipEventDestroy(s->ev_join[i]);
    if (s->aux[i]) (void)hipStreamDestroy(s->aux[i]);
  }
  if (s->stream) (void)hipStreamDestroy(s->stream);
  (void)hipSetDevice(cur);
  delete s;
}

int vdx_sampler_create(vdx_sampler **out, int32_t device, int32_t max_rows) {
  if (!out || max_rows <= 0) {
    g_create_err = "vdx_sampler_create: out must be non-NULL and max_rows > 0";
    return VDX_E_INVALID_ARG;
  }
  *out = nullptr;
  int ndev = 0;
  hipError_t e = hipGetDeviceCount(&ndev);
  if (e != hipSuccess || device < 0 || device >= ndev) {
    g_create_err = std::string("vdx_sampler_create: no HIP device ") + std::to_string(device) +
                   (e != hipSuccess ? std::string(" (") + hipGetErrorString(e) + ")" : "");
    return VDX_E_HIP;
  }
  vdx_sampler *s = new vdx_sampler();
  s->device = device;
  s->max_rows = max_rows;
  vdx_sampler_default_config(&s->cfg);
  s->row_cfg.assign((size_t)max_rows, s->cfg);
  s->own_seed.assign((size_t)max_rows, 0);
  s->own_seed_val.assign((size_t)max_rows, 0);
  s->own_pkey.assign((size_t)max_rows, 0);
  s->own_prow.assign((size_t)max_rows, -1);
  int rc = VDX_OK;
  do {
    if ((e = hipSetDevice(device)) != hipSuccess) { rc = hip_fail(s, e, "hipSetDevice"); break; }
    if ((e = hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking)) != hipSuccess) {
      rc = hip_fail(s, e, "hipStreamCreate");
      break;
    }
    if ((e = hipMalloc(&s->d_rows, sizeof(RowState) * max_rows)) != hipSuccess) {
      rc = hip_fail(s, e, "hipMalloc(rows)");
      break;
    }
    if ((e = hipMemset(s->d_rows, 0, sizeof(RowState) * max_rows)) != hipSuccess) {
      rc = hip_fail(s, e, "hipMemset(rows)");
      break;
    }
    if ((e = hipMalloc(&s->d_rcfg, sizeof(RowCfg) * max_rows)) != hipSuccess) {
      rc = hip_fail(s, e, "hipMalloc(row configs)");
      break;
    }
    if ((e = hipMalloc(&s->d_tickets, sizeof(uint32_t) * max_rows)) != hipSuccess) {
      rc = hip_fail(s, e, "hipMalloc(tickets)");
      break;
    }
    if ((e = hipMemset(s->d_tickets, 0, sizeof(uint32_t) * max_rows)) != hipSuccess) {
      rc = hip_fail(s, e, "hipMemset(tickets)");
      break;
    }
    if ((e = hipMalloc(&s->d_tok, sizeof(int32_t) * 4)) != hipSuccess) {
      rc = hip_fail(s, e, "hipMalloc(tok)");
      break;
    }
    if ((rc = alloc_history(s, s->cfg.repeat_window)) != VDX_OK) break;
    if ((rc = reseed_all(s)) != VDX_OK) break;  // Create seeds from the timer (Seed = 0)
    if ((e = hipDeviceSynchronize()) != hipSuccess) { rc = hip_fail(s, e, "hipDeviceSynchronize"); break; }
  } while (0);
  if (rc != VDX_OK) {
    g_create_err = s->err;
    vdx_sampler_destroy(s);
    return rc;
  }
  *out = s;
  return VDX_OK;
}

int vdx_sampler_set_config(vdx_sampler *s, const vdx_sampler_config *c) {
  if (!s || !c) return VDX_E_INVALID_ARG;
  HIP_TRY(s, hipSetDevice(s->device));
  const bool seed_changed = c->seed != s->cfg.seed;
  const int32_t want = window_of(*c);
  int rc = VDX_OK;
  if (!s->per_row) {
    // a RepeatWindow change resizes and clears the history (Sampler.pas:137-142);
    // the ring stride may exceed the window (widened by earlier per-row configs)
    if (want != window_of(s->cfg) && (rc = alloc_history(s, want)) != VDX_OK) return rc;
  } else {
    // every row takes the sampler-wide config again: rows whose window
    // changes lose their history, rows with their own seed are reseeded
    HIP_TRY(s, hipDeviceSynchronize());
    if ((rc = grow_history(s, want)) != VDX_OK) return rc;
    for (int32_t r = 0; r < s->max_rows; ++r)
      if (window_of(s->row_cfg[r]) != want)
        HIP_TRY(s, launch_row_reset(s->d_rows, r, 1, true, want, false, 0, false, s->stream));
  }
  const bool reseed_own = s->per_row && !seed_changed;
  s->cfg = *c;
  s->row_cfg.assign((size_t)s->max_rows, *c);
  s->per_row = false;
  if (reseed_own) {
    for (int32_t r = 0; r < s->max_rows; ++r)
      if (s->own_seed[r]) {
        s->own_seed[r] = 0;
        if ((rc = reseed_row(s, r)) != VDX_OK) return rc;
      }
    HIP_TRY(s, hipStreamSynchronize(s->stream));
  }
  s->own_seed.assign((size_t)s->max_rows, 0);
  if (seed_changed) return reseed_all(s);
  HIP_TRY(s, hipStreamSynchronize(s->stream));
  return VDX_OK;
}

int vdx_sampler_get_config(const vdx_sampler *s, vdx_sampler_config *out) {
  if (!s || !out) return VDX_E_INVALID_ARG;
  *out = s->cfg;
  return VDX_OK;
}

int vdx_sampler_set_row_config(vdx_sampler *s, int32_t row, const vdx_sampler_config *c) {
  if (!s || !c || row < 0 || row >= s->max_rows)
    return fail(s, VDX_E_INVALID_ARG, "set_row_config: need a config and 0 <= row < max_rows");
  HIP_TRY(s, hipSetDevice(s->device));
  HIP_TRY(s, hipDeviceSynchronize());  // no call in flight reads the row's state
  int rc = ensure_aux(s);
  if (rc != VDX_OK) return rc;
  const vdx_sampler_config old = s->row_cfg[row];
  s->row_cfg[row] = *c;
  s->per_row = true;
  const int32_t w = window_of(*c);
  if (window_of(old) != w) {  // SetConfig: a new window clears the history (Sampler.pas:137-142)
    if ((rc = grow_history(s, w)) != VDX_OK) return rc;
    HIP_TRY(s, launch_row_reset(s->d_rows, row, 1, true, w, false, 0, false, s->stream));
  }
  if (old.seed != c->seed) {  // a new Seed reseeds the row from it (Sampler.pas:144-150)
    s->own_seed[row] = 1;
    s->own_seed_val[row] = c->seed == 0 ? timer_seed() : (uint64_t)c->seed;
    s->own_pkey[row] = s->own_seed_val[row];
    s->own_prow[row] = -1;
    if ((rc = reseed_row(s, row)) != VDX_OK) return rc;
  }
  HIP_TRY(s, hipStreamSynchronize(s->stream));
  return upload_row_params(s);
}

int vdx_sampler_get_row_config(const vdx_sampler *s, int32_t row, vdx_sampler_config *out) {
  if (!s || !out || row < 0 || row >= s->max_rows) return VDX_E_INVALID_ARG;
  *out = s->row_cfg[row];
  return VDX_OK;
}

int vdx_sampler_set_rng(vdx_sampler *s, int32_t kind) {
  if (!s || (kind != VDX_RNG_XOSHIRO && kind != VDX_RNG_PHILOX)) return VDX_E_INVALID_ARG;
  HIP_TRY(s, hipSetDevice(s->device));
  s->rng_kind = kind;
  return reseed_all(s);
}

int vdx_sampler_process_device(vdx_sampler *s, float *logits, int32_t rows, int32_t vocab,
                               int64_t row_stride, const float *uniforms,
                               const vdx_sample_outputs *out, void *stream) {
  if (!s) return VDX_E_INVALID_ARG;
  if (!logits || !out || !out->tokens)
    return fail(s, VDX_E_INVALID_ARG, "process_device: logits and out->tokens are required");
  if (rows <= 0 || rows > s->max_rows)
    return fail(s, VDX_E_INVALID_ARG, "process_device: rows must be in [1, max_rows]");
  if (vocab <= 0 || row_stride < vocab)
    return fail(s, VDX_E_INVALID_ARG, "process_device: need vocab > 0 and row_stride >= vocab");
  const vdx_sampler_config &c = s->cfg;
  // the paths this call takes (with per-row configs: any of the rows')
  bool path_any[4] = {false, false, false, false};
  bool pen_fused = false, pen_sep = false, full_minp = false, slot_draw = false;
  int32_t kmax = 0, kmax_huge = 0;
  if (!s->per_row) {
    const RowCfg rc = row_params(c);
    const int path = row_path(rc, vocab);
    path_any[path] = true;
    if (path == kPathTopk) kmax = rc.top_k;
    if (path == kPathTopk && !(rc.top_p < 1.0f)) slot_draw = true;
    if (path == kPathTopkHuge) kmax_huge = rc.top_k;
    pen_fused = row_fuses_penalty(rc, vocab);
    pen_sep = rc.penalty != 1.0f && !pen_fused;
    full_minp = rc.min_p > 0.0f;
  } else {
    for (int32_t r = 0; r < rows; ++r) {
      const RowCfg rc = row_params(s->row_cfg[r]);
      const int path = row_path(rc, vocab);
      path_any[path] = true;
      if (path == kPathTopk && rc.top_k > kmax) kmax = rc.top_k;
      if (path == kPathTopk && !(rc.top_p < 1.0f)) slot_draw = true;
      if (path == kPathTopkHuge && rc.top_k > kmax_huge) kmax_huge = rc.top_k;
      if (rc.penalty != 1.0f) (row_fuses_penalty(rc, vocab) ? pen_fused : pen_sep) = true;
      if (path == 2 && rc.min_p > 0.0f) full_minp = true;
    }
  }
  const bool topk = path_any[kPathTopk], huge = path_any[kPathTopkHuge];
  if ((out->topk_idx || out->topk_prob) && (topk || huge) && out->topk_stride < (kmax > kmax_huge ? kmax : kmax_huge))
    return fail(s, VDX_E_INVALID_ARG, "process_device: topk_stride must be >= TopK");
  if ((out->topk_idx || out->topk_prob) && path_any[kPathFull] && out->topk_stride < 1)
    return fail(s, VDX_E_INVALID_ARG, "process_device: topk_stride must be >= 1");
  if (chunks_for(vocab) > kMaxChunks)
    return fail(s, VDX_E_UNSUPPORTED, "process_device: vocab > 4194304 is not supported");
  // TopK > 64 runs the large-K kernel, with more candidate slots per chunk
  const int32_t cap = (topk && kmax > kKMax) ? big_cand_cap(kmax, chunks_for(vocab)) : kCandCap;
  HIP_TRY(s, hipSetDevice(s->device));
  int rc = ensure_workspace(s, vocab, cap);
  if (rc != VDX_OK) return rc;
  if (huge && (rc = ensure_huge(s, rows, kmax_huge)) != VDX_OK) return rc;
  hipStream_t st = (hipStream_t)stream;

  CallParams p{};
  p.logits = logits;
  p.stride = row_stride;
  p.rows = rows;
  p.vocab = vocab;
  p.nchunks = chunks_for(vocab);
  p.vec = ((uintptr_t)logits % 16 == 0) && (row_stride % 4 == 0) && (vocab % 4 == 0);
  const RowCfg cp = row_params(c);
  p.inv_t = cp.inv_t;
  p.top_k = c.top_k;
  p.top_p = c.top_p;
  p.min_p = full_minp ? (s->per_row ? 1.0f : c.min_p) : 0.0f;  // per-row: selects the exact full path
  p.penalty = c.repeat_penalty;
  p.hist = s->d_hist;
  p.hist_len = s->hist_len;
  p.rcfg = s->per_row ? s->d_rcfg : nullptr;
  p.rng.uniforms = uniforms;
  p.rng.rows = s->d_rows;
  p.rng.kind = s->rng_kind;
  p.rng.u_out = out->uniforms;
  p.out.tokens = out->tokens;
  p.out.topk_idx = out->topk_idx;
  p.out.topk_prob = out->topk_prob;
  p.out.topk_stride = out->topk_stride;
  p.out.flags = out->flags;
  p.meta = s->d_meta;
  p.cand = s->d_cand;
  p.cand_cap = cap;
  p.huge_ws = s->d_huge;
  p.huge_row_bytes = s->huge_rb;
  p.fmeta = s->d_fmeta;
  p.gpart = s->d_gpart;
  p.tickets = s->d_tickets;

  // Step 0: repetition penalty (Sampler.pas:287); the sampling kernels apply
  // it themselves for windows of up to kPenMax ids; otherwise a separate
  // kernel runs first (for the rows that need it).  Whether it runs depends
  // on the configs only (each kernel reads the row's ring count and skips an
  // empty ring), so a captured call applies it once the device fills rings.
  const bool hist = s->hist_len > 0;
  p.fuse_penalty = (hist && pen_fused) ? 1 : 0;
  // Top-P >= 1 rows with K <= 64: slots and slot-order draw in k_topk_exact
  p.exact_kernel = (slot_draw && cap == kCandCap) ? 1 : 0;
  const bool timed = s->timing && s->n_timed < kTimedCalls;
  hipEvent_t *ev = timed ? &s->ev[3 * s->n_timed] : nullptr;
  if (timed) HIP_TRY(s, hipEventRecord(ev[0], st));
  if (hist && pen_sep) HIP_TRY(s, launch_penalty(p, st));
  if (timed) HIP_TRY(s, hipEventRecord(ev[1], st));
  // rows with K > kKBig: one workgroup each, on the call's stream
  if (huge) HIP_TRY(s, launch_topk_huge(p, st));
  const int npaths = (int)path_any[0] + (int)path_any[1] + (int)path_any[2];
  if (npaths <= 1 || !s->aux[0]) {
    if (path_any[0]) HIP_TRY(s, launch_greedy(p, st));
    if (path_any[1]) HIP_TRY(s, launch_topk(p, st));
    if (path_any[2]) HIP_TRY(s, launch_full(p, st));
  } else {
    // rows of different paths: each path's kernel on its own stream, forked
    // from the call's stream after the penalty and joined back (the kernels
    // touch disjoint rows of the logits and of the workspace)
    HIP_TRY(s, hipEventRecord(s->ev_fork, st));
    int k = 0;
    for (int path = 0; path < 3; ++path) {
      if (!path_any[path] || path == (path_any[1] ? 1 : 2)) continue;  // that one stays on st
      hipStream_t a = s->aux[k];
      HIP_TRY(s, hipStreamWaitEvent(a, s->ev_fork, 0));
      HIP_TRY(s, path == 0 ? launch_greedy(p, a) : launch_full(p, a));
      HIP_TRY(s, hipEventRecord(s->ev_join[k], a));
      ++k;
    }
    HIP_TRY(s, path_any[1] ? launch_topk(p, st) : launch_full(p, st));
    for (int i = 0; i < k; ++i) HIP_TRY(s, hipStreamWaitEvent(st, s->ev_join[i], 0));
  }
  if (timed) {
    HIP_TRY(s, hipEventRecord(ev[2], st));
    ++s->n_timed;
  }
  return VDX_OK;
}

int vdx_sample_device_noalloc(const vdx_sampler_config *cfg, float *logits, int32_t rows, int32_t vocab,
                              int64_t row_stride, const float *uniforms, const int32_t *history,
                              int32_t history_stride, const int32_t *history_count,
                              const vdx_sample_outputs *out, void *stream) {
  auto bad = [](int code, const char *m) {
    g_call_err = m;
    return code;
  };
  if (!cfg || !logits || !uniforms || !out || !out->tokens)
    return bad(VDX_E_INVALID_ARG, "noalloc: cfg, logits, uniforms and out->tokens are required");
  if (rows <= 0 || vocab <= 0 || row_stride < vocab)
    return bad(VDX_E_INVALID_ARG, "noalloc: need rows > 0, vocab > 0 and row_stride >= vocab");
  const RowCfg rc = row_params(*cfg);
  const int path = row_path(rc, vocab);
  const int32_t S = chunks_for(vocab);
  if (rows > kNoAllocRows || (int64_t)rows * S > kNoAllocRowChunks)
    return bad(VDX_E_UNSUPPORTED, "noalloc: rows * ceil(vocab / 16384) must be <= 4096 and rows <= 1024 "
                                  "(the fixed workspace)");
  if (S > kMaxChunks) return bad(VDX_E_UNSUPPORTED, "noalloc: vocab > 4194304 is not supported");
  if ((path == kPathTopk && rc.top_k > kKMax) || path == kPathTopkHuge)
    return bad(VDX_E_UNSUPPORTED, "noalloc: TopK > 64 is not supported by this entry point");
  if ((out->topk_idx || out->topk_prob) && path == 1 && out->topk_stride < rc.top_k)
    return bad(VDX_E_INVALID_ARG, "noalloc: topk_stride must be >= TopK");
  const int32_t window = rc.window;
  const bool pen = rc.penalty != 1.0f && window > 0 && history != nullptr;
  if (pen && history_stride <= 0) return bad(VDX_E_INVALID_ARG, "noalloc: history_stride must be > 0");
  unsigned char *ws = scratch_on_current_device();
  if (!ws) return VDX_E_HIP;
  hipStream_t st = (hipStream_t)stream;

  CallParams p{};
  p.logits = logits;
  p.stride = row_stride;
  p.rows = rows;
  p.vocab = vocab;
  p.nchunks = S;
  p.vec = ((uintptr_t)logits % 16 == 0) && (row_stride % 4 == 0) && (vocab % 4 == 0);
  p.inv_t = rc.inv_t;
  p.top_k = rc.top_k;
  p.top_p = rc.top_p;
  p.min_p = rc.min_p;
  p.penalty = rc.penalty;
  p.hist = pen ? history : nullptr;
  p.hist_len = pen ? history_stride : 0;
  p.fuse_penalty = (pen && row_fuses_penalty(rc, vocab)) ? 1 : 0;
  p.exact_kernel = (path == kPathTopk && !(rc.top_p < 1.0f)) ? 1 : 0;
  p.rcfg = nullptr;
  p.rng.uniforms = uniforms;
  p.rng.rows = reinterpret_cast<RowState *>(ws + kNaRows);
  p.rng.kind = VDX_RNG_XOSHIRO;
  p.rng.u_out = out->uniforms;
  p.out.tokens = out->tokens;
  p.out.topk_idx = path != kPathGreedy ? out->topk_idx : nullptr;
  p.out.topk_prob = path != kPathGreedy ? out->topk_prob : nullptr;
  p.out.topk_stride = out->topk_stride;
  p.out.flags = out->flags;
  p.meta = reinterpret_cast<ChunkMeta *>(ws + kNaMeta);
  p.cand = reinterpret_cast<Cand *>(ws + kNaCand);
  p.cand_cap = kCandCap;
  p.fmeta = reinterpret_cast<FullMeta *>(ws + kNaFullMeta);
  p.gpart = reinterpret_cast<uint64_t *>(ws + kNaGpart);
  p.tickets = reinterpret_cast<uint32_t *>(ws + kNaTickets);
  // a row's count is clamped to its window and to the row's stride
  hipError_t e = launch_rows_prepare(p.rng.rows, p.tickets, rows, pen ? history_count : nullptr,
                                     pen ? (window < history_stride ? window : history_stride) : 0, st);
  if (e == hipSuccess && pen && !p.fuse_penalty) e = launch_penalty(p, st);
  if (e == hipSuccess) e = path == 0 ? launch_greedy(p, st) : (path == 1 ? launch_topk(p, st) : launch_full(p, st));
  if (e != hipSuccess) {
    g_call_err = std::string("noalloc launch: ") + hipGetErrorString(e);
    return VDX_E_HIP;
  }
  g_call_err.clear();
  return VDX_OK;
}

int vdx_sampler_set_timing(vdx_sampler *s, int32_t enable) {
  if (!s) return VDX_E_INVALID_ARG;
  HIP_TRY(s, hipSetDevice(s->device));
  if (enable && s->ev.empty()) {
    s->ev.resize(3 * kTimedCalls);
    for (auto &e : s->ev) HIP_TRY(s, hipEventCreate(&e));
  }
  s->timing = enable != 0;
  s->n_timed = 0;
  return VDX_OK;
}

int vdx_sampler_get_timing(vdx_sampler *s, int32_t which, double *total_ms, int64_t *count) {
  if (!s || !total_ms || !count || which < 0 || which > 2) return VDX_E_INVALID_ARG;
  HIP_TRY(s, hipSetDevice(s->device));
  double tot = 0.0;
  const int a = (which == 1) ? 0 : (which == 0 ? 1 : 0);
  const int b = (which == 1) ? 1 : 2;
  for (int32_t i = 0; i < s->n_timed; ++i) {
    HIP_TRY(s, hipEventSynchronize(s->ev[3 * i + 2]));
    float ms = 0.0f;
    HIP_TRY(s, hipEventElapsedTime(&ms, s->ev[3 * i + a], s->ev[3 * i + b]));
    tot += ms;
  }
  *total_ms = tot;
  *count = s->n_timed;
  s->n_timed = 0;
  return VDX_OK;
}

int32_t vdx_sampler_process(vdx_sampler *s, float *logits, int32_t vocab) {
  if (!s) return VDX_E_INVALID_ARG;
  if (!logits || vocab <= 0) return fail(s, VDX_E_INVALID_ARG, "process: bad logits / vocab");
  HIP_TRY(s, hipSetDevice(s->device));
  if (vocab > s->row_cap) {
    HIP_TRY(s, hipStreamSynchronize(s->stream));
    (void)hipFree(s->d_row);
    s->d_row = nullptr;
    s->row_cap = 0;
    HIP_TRY(s, hipMalloc(&s->d_row, sizeof(float) * (size_t)vocab));
    s->row_cap = vocab;
  }
  HIP_TRY(s, hipMemcpyAsync(s->d_row, logits, sizeof(float) * (size_t)vocab,
                            hipMemcpyHostToDevice, s->stream));
  vdx_sample_outputs o{};
  o.tokens = s->d_tok;
  int rc = vdx_sampler_process_device(s, s->d_row, 1, vocab, vocab, nullptr, &o, s->stream);
  if (rc != VDX_OK) return rc;
  int32_t tok = -1;
  HIP_TRY(s, hipMemcpyAsync(&tok, s->d_tok, sizeof(int32_t), hipMemcpyDeviceToHost, s->stream));
  // The reference penalises the caller's buffer in place (Sampler.pas:285-303):
  // only history positions change, so their penalised values are gathered on
  // the device and written into the caller's row (hist_len pairs, not the row).
  const bool pen = s->row_cfg[0].repeat_penalty != 1.0f && s->hist_maybe && s->hist_len > 0;
  if (pen) {
    if (s->pairs_cap < s->hist_len) {
      HIP_TRY(s, hipStreamSynchronize(s->stream));
      (void)hipFree(s->d_pairs);
      if (s->h_pairs) (void)hipHostFree(s->h_pairs);
      s->d_pairs = nullptr;
      s->h_pairs = nullptr;
      s->pairs_cap = 0;
      HIP_TRY(s, hipMalloc(&s->d_pairs, sizeof(uint64_t) * (size_t)s->hist_len));
      HIP_TRY(s, hipHostMalloc(&s->h_pairs, sizeof(uint64_t) * (size_t)s->hist_len, hipHostMallocDefault));
      s->pairs_cap = s->hist_len;
    }
    HIP_TRY(s, launch_hist_gather(s->d_hist, s->hist_len, s->d_rows, s->d_row, vocab, s->d_pairs, s->stream));
    HIP_TRY(s, hipMemcpyAsync(s->h_pairs, s->d_pairs, sizeof(uint64_t) * (size_t)s->hist_len,
                              hipMemcpyDeviceToHost, s->stream));
  }
  HIP_TRY(s, hipStreamSynchronize(s->stream));
  if (pen) {
    for (int32_t j = 0; j < s->hist_len; ++j) {
      const uint64_t e = s->h_pairs[j];
      if (e == ~0ull) continue;
      const uint32_t bits = (uint32_t)e;
      memcpy(&logits[(uint32_t)(e >> 32)], &bits, sizeof(bits));
    }
  }
  return tok;
}

// wtype = a VDX_TENSOR_* format, optionally | VDX_LMHEAD_PACKED
static int lm_format(int32_t wtype) { return wtype & ~VDX_LMHEAD_PACKED; }
static int lm_block_bytes(int32_t wtype) {
  const int f = lm_format(wtype);
  return f == kLmQ4_0 ? 18 : f == kLmQ8_0 ? 34 : f == kLmF16 ? 64 : 0;
}

// nullptr when the arguments are valid; *rc is set to the error code otherwise
static const char *lmhead_check(const void *weights, int32_t wtype, const float *hidden, int32_t rows,
                                int32_t in_dim, int32_t vocab, int *rc) {
  *rc = VDX_E_INVALID_ARG;
  if (!weights || !hidden) return "lm_head: weights and hidden are required";
  if (rows <= 0 || vocab <= 0) return "lm_head: need rows > 0 and vocab > 0";
  if (lm_block_bytes(wtype) == 0) {
    *rc = VDX_E_UNSUPPORTED;
    return "lm_head: weight type must be VDX_TENSOR_Q4_0, VDX_TENSOR_Q8_0 or VDX_TENSOR_F16";
  }
  if (in_dim <= 0 || in_dim % 32 != 0) return "lm_head: in_dim must be a positive multiple of 32";
  if ((uintptr_t)weights % 16 != 0) return "lm_head: weights must be 16-byte aligned";
  if ((int64_t)(in_dim / 32) * lm_block_bytes(wtype) * 64 > (int64_t)0x7FFFFFFF)
    return "lm_head: in_dim too large";
  *rc = VDX_OK;
  return nullptr;
}

int vdx_lmhead(const void *weights, int32_t wtype, const float *hidden, const float *norm_weight,
               float norm_eps, int32_t rows, int32_t in_dim, int32_t vocab, float *logits,
               int64_t logit_stride, float *scratch, void *stream) {
  int rc = VDX_OK;
  if (const char *m = lmhead_check(weights, wtype, hidden, rows, in_dim, vocab, &rc)) {
    g_call_err = m;
    return rc;
  }
  if (!logits || logit_stride < vocab) {
    g_call_err = "lm_head: logits required, logit_stride >= vocab";
    return VDX_E_INVALID_ARG;
  }
  if ((rows > 1 || norm_weight) && !scratch) {
    g_call_err = "lm_head: scratch (16*in_dim floats) is required when rows > 1 or with the norm";
    return VDX_E_INVALID_ARG;
  }
  LmHeadParams lp{(const uint8_t *)weights, hidden, in_dim, logits, logit_stride, rows, in_dim,
                  vocab, scratch, lm_format(wtype), norm_weight, norm_eps,
                  (wtype & VDX_LMHEAD_PACKED) ? 1 : 0};
  const hipError_t e = launch_lmhead(lp, (hipStream_t)stream);
  if (e != hipSuccess) {
    g_call_err = std::string("lm_head launch: ") + hipGetErrorString(e);
    return VDX_E_HIP;
  }
  g_call_err.clear();
  return VDX_OK;
}

int64_t vdx_lmhead_packed_bytes(int32_t wtype, int32_t in_dim, int32_t vocab) {
  if (lm_block_bytes(wtype) == 0 || in_dim <= 0 || in_dim % 32 != 0 || vocab <= 0) return VDX_E_INVALID_ARG;
  return lmhead_packed_bytes(lm_format(wtype), in_dim, vocab);
}

int vdx_lmhead_pack(const void *weights, int32_t wtype, int32_t in_dim, int32_t vocab, void *packed,
                    int64_t packed_bytes, void *stream) {
  const int64_t need = vdx_lmhead_packed_bytes(wtype, in_dim, vocab);
  if (need < 0 || !weights || !packed || packed_bytes < need || (uintptr_t)weights % 16 != 0 ||
      (uintptr_t)packed % 16 != 0 || (wtype & VDX_LMHEAD_PACKED)) {
    g_call_err = "lm_head pack: need a VDX_TENSOR_* format, in_dim % 32 == 0, 16-byte aligned buffers "
                 "and packed_bytes >= vdx_lmhead_packed_bytes()";
    return VDX_E_INVALID_ARG;
  }
  const hipError_t e = launch_lmhead_pack((const uint8_t *)weights, lm_format(wtype), in_dim, vocab,
                                          (uint8_t *)packed, (hipStream_t)stream);
  if (e != hipSuccess) {
    g_call_err = std::string("lm_head pack launch: ") + hipGetErrorString(e);
    return VDX_E_HIP;
  }
  g_call_err.clear();
  return VDX_OK;
}

int vdx_lmhead_q4_0(const void *weights, const float *hidden, int32_t rows, int32_t in_dim,
                    int32_t vocab, float *logits, int64_t logit_stride, float *scratch,
                    void *stream) {
  return vdx_lmhead(weights, kLmQ4_0, hidden, nullptr, 0.0f, rows, in_dim, vocab, logits, logit_stride,
                    scratch, stream);
}

int vdx_sampler_lmhead_device(vdx_sampler *s, const void *weights, int32_t wtype, const float *hidden,
                              const float *norm_weight, float norm_eps, int32_t rows, int32_t in_dim,
                              int32_t vocab, float *logits, int64_t logit_stride, const float *uniforms,
                              const vdx_sample_outputs *out, void *stream) {
  if (!s) return VDX_E_INVALID_ARG;
  int rc = VDX_OK;
  if (const char *m = lmhead_check(weights, wtype, hidden, rows, in_dim, vocab, &rc))
    return fail(s, rc, m);
  if (rows > s->max_rows) return fail(s, VDX_E_INVALID_ARG, "lm_head: rows must be <= max_rows");
  if (!out || !out->tokens) return fail(s, VDX_E_INVALID_ARG, "lm_head: out->tokens is required");
  HIP_TRY(s, hipSetDevice(s->device));
  int64_t ls = logit_stride;
  if (!logits) {
    ls = ((int64_t)vocab + 3) & ~(int64_t)3;  // 16-byte aligned rows
    const size_t need = (size_t)rows * (size_t)ls;
    if (need > s->lm_cap) {
      HIP_TRY(s, hipStreamSynchronize(s->stream));
      HIP_TRY(s, hipDeviceSynchronize());
      (void)hipFree(s->d_lm);
      s->d_lm = nullptr;
      s->lm_cap = 0;
      HIP_TRY(s, hipMalloc(&s->d_lm, need * sizeof(float)));
      s->lm_cap = need;
    }
    logits = s->d_lm;
  } else if (ls < vocab) {
    return fail(s, VDX_E_INVALID_ARG, "lm_head: logit_stride must be >= vocab");
  }
  if ((rows > 1 || norm_weight) && in_dim > s->xt_dim) {
    HIP_TRY(s, hipStreamSynchronize(s->stream));
    HIP_TRY(s, hipDeviceSynchronize());
    (void)hipFree(s->d_xt);
    s->d_xt = nullptr;
    s->xt_dim = 0;
    HIP_TRY(s, hipMalloc(&s->d_xt, sizeof(float) * 16 * (size_t)in_dim));
    s->xt_dim = in_dim;
  }
  LmHeadParams lp{(const uint8_t *)weights, hidden, in_dim, logits, ls, rows, in_dim, vocab, s->d_xt,
                  lm_format(wtype), norm_weight, norm_eps, (wtype & VDX_LMHEAD_PACKED) ? 1 : 0};
  HIP_TRY(s, launch_lmhead(lp, (hipStream_t)stream));
  return vdx_sampler_process_device(s, logits, rows, vocab, ls, uniforms, out, stream);
}

int vdx_sampler_lmhead_q4_0_device(vdx_sampler *s, const void *weights, const float *hidden,
                                   int32_t rows, int32_t in_dim, int32_t vocab, float *logits,
                                   int64_t logit_stride, const float *uniforms,
                                   const vdx_sample_outputs *out, void *stream) {
  return vdx_sampler_lmhead_device(s, weights, kLmQ4_0, hidden, nullptr, 0.0f, rows, in_dim, vocab, logits,
                                   logit_stride, uniforms, out, stream);
}

int vdx_sampler_add_to_history(vdx_sampler *s, int32_t row, int32_t token) {
  if (!s || row < 0 || row >= s->max_rows) return VDX_E_INVALID_ARG;
  if (window_of(s->row_cfg[row]) <= 0 || s->hist_len <= 0) return VDX_OK;  // Sampler.pas:532-533
  HIP_TRY(s, hipSetDevice(s->device));
  HIP_TRY(s, launch_hist_add(nullptr, token, row, 1, s->d_hist, s->hist_len, s->d_rows, s->stream));
  HIP_TRY(s, hipStreamSynchronize(s->stream));
  s->hist_maybe = true;
  return VDX_OK;
}

int vdx_sampler_add_to_history_device(vdx_sampler *s, const int32_t *tokens, int32_t rows,
                                      void *stream) {
  if (!s || !tokens || rows <= 0 || rows > s->max_rows) return VDX_E_INVALID_ARG;
  if (s->hist_len <= 0) return VDX_OK;  // rows with no window are skipped by the kernel
  HIP_TRY(s, hipSetDevice(s->device));
  HIP_TRY(s, launch_hist_add(tokens, 0, 0, rows, s->d_hist, s->hist_len, s->d_rows,
                             (hipStream_t)stream));
  s->hist_maybe = true;
  return VDX_OK;
}

int vdx_sampler_reset_history(vdx_sampler *s, int32_t row) {
  if (!s || row >= s->max_rows) return VDX_E_INVALID_ARG;
  HIP_TRY(s, hipSetDevice(s->device));
  const int32_t r0 = row < 0 ? 0 : row;
  const int32_t n = row < 0 ? s->max_rows : 1;
  // ResetHistory (Sampler.pas:541-549): reseed only when Seed > 0
  if (!s->per_row) {
    const bool reseed = s->cfg.seed > 0;
    HIP_TRY(s, launch_row_reset(s->d_rows, r0, n, true, -1, reseed, s->seed_base, true, s->stream,
                                s->seed_base, -1));
  } else {
    HIP_TRY(s, launch_row_reset(s->d_rows, r0, n, true, -1, false, 0, false, s->stream));
    for (int32_t r = r0; r < r0 + n; ++r)
      if (s->row_cfg[r].seed > 0) {
        int rc = reseed_row(s, r);
        if (rc != VDX_OK) return rc;
      }
  }
  HIP_TRY(s, hipStreamSynchronize(s->stream));
  if (row < 0) s->hist_maybe = false;
  return VDX_OK;
}

int vdx_sampler_set_history(vdx_sampler *s, int32_t row, const int32_t *ids, int32_t count,
                            int32_t pos) {
  if (!s || row < 0 || row >= s->max_rows) return VDX_E_INVALID_ARG;
  const int32_t w = window_of(s->row_cfg[row]);
  if (count < 0 || count > w || (count > 0 && !ids) || pos < 0 || (w > 0 && pos >= w) || (w == 0 && pos != 0))
    return fail(s, VDX_E_INVALID_ARG, "set_history: need 0 <= count <= window, 0 <= pos < window");
  HIP_TRY(s, hipSetDevice(s->device));
  HIP_TRY(s, hipStreamSynchronize(s->stream));
  if (count > 0)
    HIP_TRY(s, hipMemcpy(s->d_hist + (int64_t)row * s->hist_len, ids, sizeof(int32_t) * count,
                         hipMemcpyHostToDevice));
  RowState rs;
  HIP_TRY(s, hipMemcpy(&rs, s->d_rows + row, sizeof(RowState), hipMemcpyDeviceToHost));
  rs.hist_pos = pos;
  rs.hist_count = count;
  HIP_TRY(s, hipMemcpy(s->d_rows + row, &rs, sizeof(RowState), hipMemcpyHostToDevice));
  if (count > 0) s->hist_maybe = true;
  return VDX_OK;
}

int32_t vdx_sampler_get_history(vdx_sampler *s, int32_t row, int32_t *ids, int32_t cap,
                                int32_t *pos) {
  if (!s || row < 0 || row >= s->max_rows || cap < 0 || (cap > 0 && !ids))
    return VDX_E_INVALID_ARG;
  HIP_TRY(s, hipSetDevice(s->device));
  HIP_TRY(s, hipStreamSynchronize(s->stream));
  RowState rs;
  HIP_TRY(s, hipMemcpy(&rs, s->d_rows + row, sizeof(RowState), hipMemcpyDeviceToHost));
  const int32_t n = rs.hist_count < cap ? rs.hist_count : cap;
  if (n > 0)
    HIP_TRY(s, hipMemcpy(ids, s->d_hist + (int64_t)row * s->hist_len, sizeof(int32_t) * n,
                         hipMemcpyDeviceToHost));
  if (pos) *pos = rs.hist_pos;
  return rs.hist_count;
}

// ---- row checkpoints ---------------------------------------------------------
// Blob layout (little endian): RowCkpt, then `window` int32 ring slots.
struct RowCkpt {
  char magic[4];            // "VDXR"
  uint32_t version;         // 1
  vdx_sampler_config cfg;   // the row's config
  int32_t rng_kind;
  int32_t own_seed;         // seeded from its own Seed (else as row r of the sampler-wide Seed + r)
  uint64_t own_seed_val;    // the xoshiro seed of the row's stream (resolved)
  RowState state;           // RNG words, Philox counter and key, ring position / fill / window
};
static_assert(sizeof(RowCkpt) == 120, "checkpoint header layout");

int64_t vdx_sampler_save_row_state(vdx_sampler *s, int32_t row, void *buf, int64_t cap) {
  if (!s || row < 0 || row >= s->max_rows || cap < 0) return VDX_E_INVALID_ARG;
  HIP_TRY(s, hipSetDevice(s->device));
  HIP_TRY(s, hipDeviceSynchronize());  // the calls issued so far have updated the row
  RowCkpt h{};
  memcpy(h.magic, "VDXR", 4);
  h.version = 1;
  h.cfg = s->row_cfg[row];
  h.rng_kind = s->rng_kind;
  h.own_seed = s->own_seed[row];
  h.own_seed_val = s->own_seed[row] ? s->own_seed_val[row] : s->seed_base + (uint64_t)row;
  HIP_TRY(s, hipMemcpy(&h.state, s->d_rows + row, sizeof(RowState), hipMemcpyDeviceToHost));
  const int32_t w = h.state.window > 0 ? (h.state.window < s->hist_len ? h.state.window : s->hist_len) : 0;
  h.state.window = w;
  const int64_t need = (int64_t)sizeof(RowCkpt) + (int64_t)w * (int64_t)sizeof(int32_t);
  if (!buf || cap < need) return need;
  memcpy(buf, &h, sizeof(h));
  if (w > 0)
    HIP_TRY(s, hipMemcpy((char *)buf + sizeof(h), s->d_hist + (int64_t)row * s->hist_len,
                         sizeof(int32_t) * (size_t)w, hipMemcpyDeviceToHost));
  return need;
}

int vdx_sampler_load_row_state(vdx_sampler *s, int32_t row, const void *buf, int64_t size) {
  if (!s || row < 0 || row >= s->max_rows || !buf || size < (int64_t)sizeof(RowCkpt))
    return fail(s, VDX_E_INVALID_ARG, "load_row_state: need a blob and 0 <= row < max_rows");
  RowCkpt h;
  memcpy(&h, buf, sizeof(h));
  if (memcmp(h.magic, "VDXR", 4) != 0 || h.version != 1)
    return fail(s, VDX_E_INVALID_ARG, "load_row_state: not a row checkpoint (magic / version)");
  const int32_t w = h.state.window;
  if (w < 0 || w != window_of(h.cfg) || size != (int64_t)sizeof(RowCkpt) + (int64_t)w * 4 ||
      h.state.hist_count < 0 || h.state.hist_count > w || h.state.hist_pos < 0 ||
      (w > 0 ? h.state.hist_pos >= w : h.state.hist_pos != 0))
    return fail(s, VDX_E_INVALID_ARG, "load_row_state: inconsistent checkpoint");
  if (h.rng_kind != s->rng_kind)
    return fail(s, VDX_E_INVALID_ARG, "load_row_state: the checkpoint was taken with another RNG kind");
  HIP_TRY(s, hipSetDevice(s->device));
  HIP_TRY(s, hipDeviceSynchronize());
  int rc = ensure_aux(s);
  if (rc != VDX_OK) return rc;
  if ((rc = grow_history(s, w)) != VDX_OK) return rc;
  s->row_cfg[row] = h.cfg;
  s->per_row = true;
  // the restored state carries its own seed: later reseeds of this row
  // (ResetHistory with Seed > 0, set_rng) start the stream it was taken from
  // (xoshiro from its seed; Philox under its key and counter row)
  s->own_seed[row] = 1;
  s->own_seed_val[row] = h.own_seed_val;
  s->own_pkey[row] = h.state.key;
  s->own_prow[row] = h.state.ctr_row;
  HIP_TRY(s, hipMemcpy(s->d_rows + row, &h.state, sizeof(RowState), hipMemcpyHostToDevice));
  if (w > 0)
    HIP_TRY(s, hipMemcpy(s->d_hist + (int64_t)row * s->hist_len, (const char *)buf + sizeof(h),
                         sizeof(int32_t) * (size_t)w, hipMemcpyHostToDevice));
  if (h.state.hist_count > 0) s->hist_maybe = true;
  return upload_row_params(s);
}

}  // extern "C"
