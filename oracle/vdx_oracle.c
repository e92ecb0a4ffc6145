/*
 * vdx_oracle.c -- CPU oracle: plain-C restatement of TVdxSampler.
 *
 * TEST INFRASTRUCTURE ONLY (see vdx_oracle.h).  Restates
 * src/VindexLLM.Sampler.pas op for op; each function cites the lines it
 * follows.  Build: gcc -O2 -fno-fast-math -ffp-contract=off (no FMA
 * contraction, binary32 SSE arithmetic for Single, binary64 for Double).
 */
#define _POSIX_C_SOURCE 200809L
#include "vdx_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ------------------------------------------------------------------------ */
/* PRNG                                                                     */
/* ------------------------------------------------------------------------ */

/* WrapAdd (Sampler.pas:160-167): modular add written without overflow. */
uint64_t vdxo_wrap_add(uint64_t a, uint64_t b) {
  if (b <= UINT64_MAX - a) return a + b;
  return b - (UINT64_MAX - a) - 1u;
}

/* WrapMul (Sampler.pas:169-190): low 64 bits of a*b from 32-bit halves. */
uint64_t vdxo_wrap_mul(uint64_t a, uint64_t b) {
  uint64_t alo = a & 0xFFFFFFFFu, ahi = a >> 32;
  uint64_t blo = b & 0xFFFFFFFFu, bhi = b >> 32;
  uint64_t r = alo * blo;
  uint64_t c1 = alo * bhi, c2 = ahi * blo;
  r = vdxo_wrap_add(r, (c1 & 0xFFFFFFFFu) << 32);
  r = vdxo_wrap_add(r, (c2 & 0xFFFFFFFFu) << 32);
  return r;
}

/* SplitMix64 (Sampler.pas:194-201). */
uint64_t vdxo_splitmix64(uint64_t *state) {
  *state = vdxo_wrap_add(*state, 0x9E3779B97F4A7C15ull);
  uint64_t z = *state;
  z = vdxo_wrap_mul(z ^ (z >> 30), 0xBF58476D1CE4E5B9ull);
  z = vdxo_wrap_mul(z ^ (z >> 27), 0x94D049BB133111EBull);
  return z ^ (z >> 31);
}

/* SeedPRNG (Sampler.pas:224-241): four successive SplitMix64 outputs.  The
 * caller resolves Seed = 0 to a timer value before calling. */
void vdxo_seed(uint64_t st[4], uint64_t seed_state) {
  uint64_t s = seed_state;
  st[0] = vdxo_splitmix64(&s);
  st[1] = vdxo_splitmix64(&s);
  st[2] = vdxo_splitmix64(&s);
  st[3] = vdxo_splitmix64(&s);
}

static uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

/* NextUInt64, xoshiro256** (Sampler.pas:208-222). */
uint64_t vdxo_next_u64(uint64_t st[4]) {
  uint64_t result = vdxo_wrap_mul(rotl64(vdxo_wrap_mul(st[1], 5), 7), 9);
  uint64_t t = st[1] << 17;
  st[2] ^= st[0];
  st[3] ^= st[1];
  st[1] ^= st[2];
  st[0] ^= st[3];
  st[2] ^= t;
  st[3] = rotl64(st[3], 45);
  return result;
}

/* (x shr 40) / 16777216.0 (Sampler.pas:247), exact in binary32. */
float vdxo_u24(uint64_t x) { return (float)((double)(x >> 40) / 16777216.0); }

/* NextFloat (Sampler.pas:243-248). */
float vdxo_next_float(uint64_t st[4]) { return vdxo_u24(vdxo_next_u64(st)); }

/* Philox4x64-10: round function and key schedule of Salmon, Moraes, Dror and
 * Shaw, "Parallel random numbers: as easy as 1, 2, 3" (SC'11). */
static void mulhilo64(uint64_t a, uint64_t b, uint64_t *hi, uint64_t *lo) {
  unsigned __int128 p = (unsigned __int128)a * b;
  *hi = (uint64_t)(p >> 64);
  *lo = (uint64_t)p;
}

void vdxo_philox4x64_10(const uint64_t ctr[4], const uint64_t key[2],
                        uint64_t out[4]) {
  const uint64_t M0 = 0xD2E7470EE14C6C93ull, M1 = 0xCA5A826395121157ull;
  const uint64_t W0 = 0x9E3779B97F4A7C15ull, W1 = 0xBB67AE8584CAA73Bull;
  uint64_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
  uint64_t k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; ++r) {
    if (r > 0) { k0 += W0; k1 += W1; }
    uint64_t hi0, lo0, hi1, lo1;
    mulhilo64(M0, c0, &hi0, &lo0);
    mulhilo64(M1, c2, &hi1, &lo1);
    uint64_t n0 = hi1 ^ c1 ^ k0, n1 = lo1, n2 = hi0 ^ c3 ^ k1, n3 = lo0;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
  }
  out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

float vdxo_philox_uniform(uint64_t seed, uint64_t row, uint64_t step) {
  uint64_t ctr[4] = {step, row, 0, 0}, key[2] = {seed, 0}, out[4];
  vdxo_philox4x64_10(ctr, key, out);
  return vdxo_u24(out[0]);
}

/* ------------------------------------------------------------------------ */
/* Process()                                                                */
/* ------------------------------------------------------------------------ */

/* Step 0 (Sampler.pas:285-303): for every history slot in array order, an
 * in-range id has its logit divided (if > 0) or multiplied (if < 0) by the
 * penalty, in place, once per occurrence. */
void vdxo_apply_penalty(float *logits, int32_t vocab, const int32_t *hist,
                        int32_t hist_count, float penalty) {
  if (penalty == 1.0f || hist_count <= 0) return;
  for (int32_t j = 0; j < hist_count; ++j) {
    int32_t id = hist[j];
    if (id >= 0 && id < vocab) {
      float v = logits[id];
      if (v > 0.0f)
        logits[id] = v / penalty;
      else if (v < 0.0f)
        logits[id] = v * penalty;
    }
  }
}

static int32_t process_greedy(const float *L, int32_t vocab) {
  /* Sampler.pas:306-322: strict '>' scan from index 0. */
  int32_t best = 0;
  float bv = L[0];
  for (int32_t i = 1; i < vocab; ++i)
    if (L[i] > bv) { best = i; bv = L[i]; }
  return best;
}

static void trace_draw(vdxo_trace *tr, double lo, double hi, int fb) {
  if (!tr) return;
  tr->cdf_lo = lo;
  tr->cdf_hi = hi;
  tr->fallback = fb;
}

/* Top-K path (Sampler.pas:327-460). */
static int32_t process_topk(const float *L, int32_t vocab, const vdxo_config *cfg,
                            float inv_t, float u, vdxo_trace *tr) {
  const int32_t K = cfg->top_k;
  float *buf = (float *)malloc(sizeof(float) * (size_t)K);
  int32_t *idx = (int32_t *)malloc(sizeof(int32_t) * (size_t)K);
  int32_t nrep = 0;

  /* Pass 1 (:341-383): running max and K-slot min-buffer. */
  float M = L[0];
  int32_t mi = 0;
  float mv = -1e30f;
  for (int32_t i = 0; i < vocab; ++i) {
    float v = L[i];
    if (v > M) M = v;
    if (i < K) {
      buf[i] = v;
      idx[i] = i;
      if (i == K - 1) {
        mi = 0;
        mv = buf[0];
        for (int32_t j = 1; j < K; ++j)
          if (buf[j] < mv) { mi = j; mv = buf[j]; }
      }
    } else if (v > mv) {
      buf[mi] = v;
      idx[mi] = i;
      ++nrep;
      mi = 0;
      mv = buf[0];
      for (int32_t j = 1; j < K; ++j)
        if (buf[j] < mv) { mi = j; mv = buf[j]; }
    }
  }
  if (tr) {
    tr->k = K;
    tr->max_logit = M;
    tr->n_replacements = nrep;
    for (int32_t k = 0; k < K && k < VDXO_KMAX; ++k) {
      tr->slot_idx[k] = idx[k];
      tr->slot_val[k] = buf[k];
    }
  }

  /* Pass 2 (:385-391): q = fl32(Exp((v - M) * invT)), argument in double. */
  double S = 0.0;
  for (int32_t k = 0; k < K; ++k) {
    buf[k] = (float)exp(((double)buf[k] - (double)M) * (double)inv_t);
    S = S + (double)buf[k];
  }
  if (tr) tr->sum_initial = S;

  /* Min-P (:393-410). */
  if (cfg->min_p > 0.0f) {
    float best = buf[0];
    for (int32_t k = 1; k < K; ++k)
      if (buf[k] > best) best = buf[k];
    float thr = best * cfg->min_p;
    S = 0.0;
    for (int32_t k = 0; k < K; ++k) {
      if (buf[k] < thr)
        buf[k] = 0.0f;
      else
        S = S + (double)buf[k];
    }
  }

  /* Top-P (:412-445): stable insertion sort descending, then keep while the
   * running sum is below TopP * S. */
  if (cfg->top_p < 1.0f) {
    for (int32_t i = 1; i < K; ++i) {
      float v = buf[i];
      int32_t ti = idx[i];
      int32_t j = i - 1;
      while (j >= 0 && buf[j] < v) {
        buf[j + 1] = buf[j];
        idx[j + 1] = idx[j];
        --j;
      }
      buf[j + 1] = v;
      idx[j + 1] = ti;
    }
    double target = (double)cfg->top_p * S;
    double C = 0.0;
    S = 0.0;
    for (int32_t k = 0; k < K; ++k) {
      if (C < target && buf[k] > 0.0f) {
        C = C + (double)buf[k];
        S = S + (double)buf[k];
      } else {
        buf[k] = 0.0f;
      }
    }
  }
  if (tr) {
    for (int32_t k = 0; k < K && k < VDXO_KMAX; ++k) {
      tr->order_idx[k] = idx[k];
      tr->order_q[k] = buf[k];
    }
    tr->sum_final = S;
  }

  /* Draw (:447-459). */
  double t = (double)u * S;
  if (tr) tr->target = t;
  double C = 0.0;
  int32_t result = idx[K - 1];
  int found = 0;
  for (int32_t k = 0; k < K; ++k) {
    double prev = C;
    C = C + (double)buf[k];
    if (C > t) {
      result = idx[k];
      trace_draw(tr, prev, C, 0);
      found = 1;
      break;
    }
  }
  if (!found) trace_draw(tr, C, C, 1);
  free(buf);
  free(idx);
  return result;
}

/* Full-softmax path (Sampler.pas:461-527). */
static int32_t process_full(const float *L, int32_t vocab, const vdxo_config *cfg,
                            float inv_t, float u, vdxo_trace *tr) {
  float *P = (float *)malloc(sizeof(float) * (size_t)vocab);
  /* Pass 1 (:467-476). */
  float M = L[0] * inv_t;
  for (int32_t i = 0; i < vocab; ++i) {
    float v = L[i] * inv_t;
    P[i] = v;
    if (v > M) M = v;
  }
  /* Pass 2 (:478-486). */
  double S = 0.0;
  for (int32_t i = 0; i < vocab; ++i) {
    float q = (float)exp((double)P[i] - (double)M);
    P[i] = q;
    S = S + (double)q;
  }
  if (tr) {
    tr->k = 0;
    tr->max_logit = M;
    tr->sum_initial = S;
  }
  /* Min-P (:488-511). */
  if (cfg->min_p > 0.0f) {
    float best = P[0];
    for (int32_t i = 1; i < vocab; ++i)
      if (P[i] > best) best = P[i];
    float thr = best * cfg->min_p;
    S = 0.0;
    for (int32_t i = 0; i < vocab; ++i) {
      if (P[i] < thr)
        P[i] = 0.0f;
      else
        S = S + (double)P[i];
    }
  }
  if (tr) tr->sum_final = S;
  /* Pass 3 (:513-526). */
  double t = (double)u * S;
  if (tr) tr->target = t;
  double C = 0.0;
  int32_t result = vocab - 1;
  int found = 0;
  for (int32_t i = 0; i < vocab; ++i) {
    double prev = C;
    C = C + (double)P[i];
    if (C > t) {
      result = i;
      trace_draw(tr, prev, C, 0);
      found = 1;
      break;
    }
  }
  if (!found) trace_draw(tr, C, C, 1);
  free(P);
  return result;
}

int32_t vdxo_process_row(float *logits, int32_t vocab, const vdxo_config *cfg,
                         const int32_t *hist, int32_t hist_count, float u,
                         vdxo_trace *tr) {
  int32_t tok;
  if (tr) memset(tr, 0, sizeof(*tr));
  /* Step 0 (:287-303). */
  if (cfg->repeat_penalty != 1.0f && hist_count > 0)
    vdxo_apply_penalty(logits, vocab, hist, hist_count, cfg->repeat_penalty);
  /* Greedy (:306-322). */
  if (cfg->temperature == 0.0f) {
    tok = process_greedy(logits, vocab);
    if (tr) { tr->path = VDXO_PATH_GREEDY; tr->token = tok; }
    return tok;
  }
  /* invT (:325): 1.0 / T stored into a Single. */
  float inv_t = 1.0f / cfg->temperature;
  if (tr) tr->inv_temp = inv_t;
  if (cfg->top_k > 0 && cfg->top_k < vocab) {
    tok = process_topk(logits, vocab, cfg, inv_t, u, tr);
    if (tr) tr->path = VDXO_PATH_TOPK;
  } else {
    tok = process_full(logits, vocab, cfg, inv_t, u, tr);
    if (tr) tr->path = VDXO_PATH_FULL;
  }
  if (tr) tr->token = tok;
  return tok;
}

void vdxo_process_batch(float *logits, int32_t rows, int32_t vocab,
                        int64_t row_stride, const vdxo_config *cfg,
                        const int32_t *hist, int32_t hist_stride,
                        const int32_t *hcount, const float *u,
                        int32_t *tokens) {
  for (int32_t r = 0; r < rows; ++r) {
    const int32_t *h = hist ? hist + (int64_t)r * hist_stride : NULL;
    int32_t hc = (hist && hcount) ? hcount[r] : 0;
    tokens[r] = vdxo_process_row(logits + (int64_t)r * row_stride, vocab, cfg,
                                 h, hc, u[r], NULL);
  }
}

typedef struct batch_job {
  float *logits;
  int32_t r0, r1, vocab, hist_stride;
  int64_t row_stride;
  const vdxo_config *cfg;
  const int32_t *hist, *hcount;
  const float *u;
  int32_t *tokens;
} batch_job;

static void *batch_worker(void *arg) {
  batch_job *j = (batch_job *)arg;
  for (int32_t r = j->r0; r < j->r1; ++r) {
    const int32_t *h = j->hist ? j->hist + (int64_t)r * j->hist_stride : NULL;
    int32_t hc = (j->hist && j->hcount) ? j->hcount[r] : 0;
    j->tokens[r] = vdxo_process_row(j->logits + (int64_t)r * j->row_stride,
                                    j->vocab, j->cfg, h, hc, j->u[r], NULL);
  }
  return NULL;
}

void vdxo_process_batch_mt(float *logits, int32_t rows, int32_t vocab,
                           int64_t row_stride, const vdxo_config *cfg,
                           const int32_t *hist, int32_t hist_stride,
                           const int32_t *hcount, const float *u,
                           int32_t *tokens, int32_t threads) {
  if (threads <= 1 || rows <= 1) {
    vdxo_process_batch(logits, rows, vocab, row_stride, cfg, hist, hist_stride,
                       hcount, u, tokens);
    return;
  }
  if (threads > rows) threads = rows;
  pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
  batch_job *jobs = (batch_job *)malloc(sizeof(batch_job) * (size_t)threads);
  for (int32_t t = 0; t < threads; ++t) {
    batch_job *j = &jobs[t];
    j->logits = logits;
    j->r0 = (int32_t)((int64_t)rows * t / threads);
    j->r1 = (int32_t)((int64_t)rows * (t + 1) / threads);
    j->vocab = vocab;
    j->row_stride = row_stride;
    j->cfg = cfg;
    j->hist = hist;
    j->hist_stride = hist_stride;
    j->hcount = hcount;
    j->u = u;
    j->tokens = tokens;
    pthread_create(&tid[t], NULL, batch_worker, j);
  }
  for (int32_t t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
  free(tid);
  free(jobs);
}

/* ------------------------------------------------------------------------ */
/* Stateful sampler (the TVdxSampler object)                                */
/* ------------------------------------------------------------------------ */

struct vdxo_sampler {
  vdxo_config cfg;
  uint64_t st[4];
  int32_t *hist;
  int32_t hist_len;
  int32_t hist_pos;
  int32_t hist_count;
};

static uint64_t timer_value(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

/* DefaultConfig (Sampler.pas:100-109). */
void vdxo_default_config(vdxo_config *c) {
  c->temperature = 0.0f;
  c->top_k = 0;
  c->top_p = 1.0f;
  c->min_p = 0.0f;
  c->repeat_penalty = 1.0f;
  c->repeat_window = 64;
  c->seed = 0;
}

static void resize_history(vdxo_sampler *s, int32_t n) {
  free(s->hist);
  s->hist = NULL;
  s->hist_len = n > 0 ? n : 0;
  if (s->hist_len > 0) s->hist = (int32_t *)calloc((size_t)s->hist_len, sizeof(int32_t));
}

/* Create (Sampler.pas:111-122). */
vdxo_sampler *vdxo_sampler_create(void) {
  vdxo_sampler *s = (vdxo_sampler *)calloc(1, sizeof(vdxo_sampler));
  vdxo_default_config(&s->cfg);
  resize_history(s, s->cfg.repeat_window);
  vdxo_seed(s->st, timer_value());
  return s;
}

void vdxo_sampler_destroy(vdxo_sampler *s) {
  if (!s) return;
  free(s->hist);
  free(s);
}

/* SetConfig (Sampler.pas:132-150). */
void vdxo_sampler_set_config(vdxo_sampler *s, const vdxo_config *c,
                             uint64_t timer_seed) {
  int seed_changed = c->seed != s->cfg.seed;
  s->cfg = *c;
  if (s->hist_len != (c->repeat_window > 0 ? c->repeat_window : 0)) {
    resize_history(s, c->repeat_window);
    s->hist_pos = 0;
    s->hist_count = 0;
  }
  if (seed_changed)
    vdxo_seed(s->st, s->cfg.seed == 0 ? timer_seed : (uint64_t)s->cfg.seed);
}

void vdxo_sampler_get_config(const vdxo_sampler *s, vdxo_config *c) { *c = s->cfg; }

/* Process (Sampler.pas:265-528) with the object's own PRNG: exactly one draw
 * per non-greedy call. */
int32_t vdxo_sampler_process(vdxo_sampler *s, float *logits, int32_t vocab,
                             vdxo_trace *tr) {
  float u = 0.0f;
  /* The draw happens after the scan in the reference; its value does not
   * depend on the logits, so drawing first is equivalent.  Greedy calls
   * draw nothing (:306-322 exits before NextFloat). */
  if (s->cfg.temperature != 0.0f) u = vdxo_next_float(s->st);
  return vdxo_process_row(logits, vocab, &s->cfg, s->hist, s->hist_count, u, tr);
}

/* AddToHistory (Sampler.pas:530-539). */
void vdxo_sampler_add_to_history(vdxo_sampler *s, int32_t id) {
  if (s->cfg.repeat_window <= 0) return;
  s->hist[s->hist_pos] = id;
  s->hist_pos = (s->hist_pos + 1) % s->cfg.repeat_window;
  if (s->hist_count < s->cfg.repeat_window) s->hist_count++;
}

/* ResetHistory (Sampler.pas:541-549): reseed only when Seed > 0. */
void vdxo_sampler_reset_history(vdxo_sampler *s) {
  s->hist_pos = 0;
  s->hist_count = 0;
  if (s->cfg.seed > 0) vdxo_seed(s->st, (uint64_t)s->cfg.seed);
}

int32_t vdxo_sampler_history(const vdxo_sampler *s, int32_t *out, int32_t cap,
                             int32_t *pos) {
  int32_t n = s->hist_count < cap ? s->hist_count : cap;
  for (int32_t i = 0; i < n; ++i) out[i] = s->hist[i];
  if (pos) *pos = s->hist_pos;
  return s->hist_count;
}

void vdxo_sampler_rng_state(const vdxo_sampler *s, uint64_t st[4]) {
  memcpy(st, s->st, sizeof(s->st));
}

/* ------------------------------------------------------------------------ */
/* Q4_0 lm_head (shaders/matvec_q4_0.comp)                                  */
/* ------------------------------------------------------------------------ */

float vdxo_half_to_float(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) & 1u;
  uint32_t exp = (uint32_t)(h >> 10) & 0x1Fu;
  uint32_t man = (uint32_t)h & 0x3FFu;
  float f;
  if (exp == 0)
    f = ldexpf((float)man, -24); /* zero / subnormal */
  else if (exp == 31)
    f = man ? NAN : INFINITY;
  else
    f = ldexpf((float)(man | 0x400u), (int)exp - 25);
  return sign ? -f : f;
}

/* matvec_q4_0.comp:45-88: block layout :7-15 (18 bytes: f16 d, 16 bytes qs;
 * qs[j] & 0xF -> element j, qs[j] >> 4 -> element j+16); per-lane strided
 * accumulation :57-73; LDS tree reduction :75-83. */
void vdxo_matvec_q4_0(const uint8_t *w, const float *x, int32_t in_dim,
                      int32_t rows, float *logits) {
  const int32_t bpr = in_dim >> 5;
  for (int32_t r = 0; r < rows; ++r) {
    const uint8_t *row = w + (int64_t)r * bpr * 18;
    float partial[64];
    for (int32_t tid = 0; tid < 64; ++tid) {
      float acc = 0.0f;
      for (int32_t e = tid; e < in_dim; e += 64) {
        int32_t blk = e >> 5, inb = e & 31, bi = inb & 15, hi = inb >> 4;
        const uint8_t *b = row + (int64_t)blk * 18;
        float scale = vdxo_half_to_float((uint16_t)(b[0] | (b[1] << 8)));
        uint32_t raw = b[2 + bi];
        uint32_t nib = (raw >> (hi * 4)) & 0xFu;
        float qv = (float)((int32_t)nib - 8);
        float t = qv * scale;
        t = t * x[e];
        acc = acc + t;
      }
      partial[tid] = acc;
    }
    for (int32_t stride = 32; stride > 0; stride >>= 1)
      for (int32_t tid = 0; tid < stride; ++tid)
        partial[tid] = partial[tid] + partial[tid + stride];
    logits[r] = partial[0];
  }
}

/* The same matvec in the accumulation order of the library's fused lm_head
 * kernel (not the shader's): per row, blocks k = 0.. in order, t = 0,
 * t = fmaf(16 (q_i - 8), x[32k+i], t) for i = 0..31 (element order: low
 * nibbles of qs[0..15], then high nibbles), acc = fmaf(d_k / 16, t, acc).
 * The power-of-two scaling is exact, so this is the plain chain
 * s = fmaf(q_i - 8, x, s), acc = fmaf(d_k, s, acc) wherever no partial sum is
 * subnormal; the kernel computes the scaled form, restated here as computed.
 * Mathematically the same sum as matvec_q4_0.comp:57-83; only the fp32
 * rounding points differ (the shader's own are unpinned under GLSL
 * contraction). */
void vdxo_matvec_q4_0_blocked(const uint8_t *w, const float *x, int32_t in_dim,
                              int32_t rows, float *logits) {
  const int32_t bpr = in_dim >> 5;
  for (int32_t r = 0; r < rows; ++r) {
    const uint8_t *row = w + (int64_t)r * bpr * 18;
    float acc = 0.0f;
    for (int32_t k = 0; k < bpr; ++k) {
      const uint8_t *b = row + (int64_t)k * 18;
      const float d = vdxo_half_to_float((uint16_t)(b[0] | (b[1] << 8)));
      float t = 0.0f;
      for (int32_t i = 0; i < 32; ++i) {
        const uint32_t raw = b[2 + (i & 15)];
        const int32_t q = (int32_t)((raw >> ((i >> 4) * 4)) & 0xFu) - 8;
        t = fmaf((float)(16 * q), x[32 * k + i], t);
      }
      acc = fmaf(d * 0.0625f, t, acc);
    }
    logits[r] = acc;
  }
}

/* matvec_q8_0.comp:53-93: block layout :5-9 (34 bytes: f16 d, 32 int8);
 * 256 lanes, lane t sums elements t, t+256, ... as acc += (q * d) * x
 * (:74-78), then the LDS tree (:83-89). */
void vdxo_matvec_q8_0(const uint8_t *w, const float *x, int32_t in_dim, int32_t rows,
                      float *logits) {
  const int32_t bpr = in_dim >> 5;
  for (int32_t r = 0; r < rows; ++r) {
    const uint8_t *row = w + (int64_t)r * bpr * 34;
    float partial[256];
    for (int32_t tid = 0; tid < 256; ++tid) {
      float acc = 0.0f;
      for (int32_t e = tid; e < in_dim; e += 256) {
        const uint8_t *b = row + (int64_t)(e >> 5) * 34;
        const float d = vdxo_half_to_float((uint16_t)(b[0] | (b[1] << 8)));
        const float q = (float)(int8_t)b[2 + (e & 31)];
        float t = q * d;
        t = t * x[e];
        acc = acc + t;
      }
      partial[tid] = acc;
    }
    for (int32_t stride = 128; stride > 0; stride >>= 1)
      for (int32_t tid = 0; tid < stride; ++tid) partial[tid] = partial[tid] + partial[tid + stride];
    logits[r] = partial[0];
  }
}

/* The library kernel's order for Q8_0: per block k, s = fmaf(q_i, x, s) for
 * i = 0..31, acc = fmaf(d_k, s, acc). */
void vdxo_matvec_q8_0_blocked(const uint8_t *w, const float *x, int32_t in_dim, int32_t rows,
                              float *logits) {
  const int32_t bpr = in_dim >> 5;
  for (int32_t r = 0; r < rows; ++r) {
    const uint8_t *row = w + (int64_t)r * bpr * 34;
    float acc = 0.0f;
    for (int32_t k = 0; k < bpr; ++k) {
      const uint8_t *b = row + (int64_t)k * 34;
      const float d = vdxo_half_to_float((uint16_t)(b[0] | (b[1] << 8)));
      float s = 0.0f;
      for (int32_t i = 0; i < 32; ++i) s = fmaf((float)(int8_t)b[2 + i], x[32 * k + i], s);
      acc = fmaf(d, s, acc);
    }
    logits[r] = acc;
  }
}

/* matvec_f16.comp:43-80: packed f16 pairs, 256 lanes, lane t takes pairs
 * t, t+256, ... as acc += w.x * x[2d]; acc += w.y * x[2d+1] (:56-63), then
 * the LDS tree (:68-74). */
void vdxo_matvec_f16(const uint8_t *w, const float *x, int32_t in_dim, int32_t rows,
                     float *logits) {
  for (int32_t r = 0; r < rows; ++r) {
    const uint8_t *row = w + (int64_t)r * in_dim * 2;
    float partial[256];
    for (int32_t tid = 0; tid < 256; ++tid) {
      float acc = 0.0f;
      for (int32_t d = tid; d < in_dim / 2; d += 256) {
        const uint8_t *p = row + 4 * (int64_t)d;
        const float w0 = vdxo_half_to_float((uint16_t)(p[0] | (p[1] << 8)));
        const float w1 = vdxo_half_to_float((uint16_t)(p[2] | (p[3] << 8)));
        float t = w0 * x[2 * d];
        acc = acc + t;
        t = w1 * x[2 * d + 1];
        acc = acc + t;
      }
      partial[tid] = acc;
    }
    for (int32_t stride = 128; stride > 0; stride >>= 1)
      for (int32_t tid = 0; tid < stride; ++tid) partial[tid] = partial[tid] + partial[tid + stride];
    logits[r] = partial[0];
  }
}

/* The library kernel's order for F16: per 32-element block k, s = fmaf(w_i,
 * x, s) for i = 0..31, acc = acc + s. */
void vdxo_matvec_f16_blocked(const uint8_t *w, const float *x, int32_t in_dim, int32_t rows,
                             float *logits) {
  for (int32_t r = 0; r < rows; ++r) {
    const uint8_t *row = w + (int64_t)r * in_dim * 2;
    float acc = 0.0f;
    for (int32_t k = 0; k < in_dim / 32; ++k) {
      float s = 0.0f;
      for (int32_t i = 0; i < 32; ++i) {
        const uint8_t *p = row + 2 * (int64_t)(32 * k + i);
        s = fmaf(vdxo_half_to_float((uint16_t)(p[0] | (p[1] << 8))), x[32 * k + i], s);
      }
      acc = acc + s;
    }
    logits[r] = acc;
  }
}

/* rmsnorm_copy.comp:40-74 (TVdxLayerNorm.ApplyCopy, LayerNorm.pas:395-417):
 * 256 lanes sum source[i]^2 strided (:45-50), the LDS tree (:55-60),
 * inv_rms = 1 / sqrt(ss / dim + eps) (:63-65), dest[i] = (source[i] *
 * inv_rms) * weight[i] (:70-73); IEEE division and square root. */
void vdxo_rmsnorm(const float *h, const float *wt, float eps, int32_t dim, float *out) {
  float part[256];
  for (int32_t t = 0; t < 256; ++t) {
    float ss = 0.0f;
    for (int32_t i = t; i < dim; i += 256) {
      const float sq = h[i] * h[i];
      ss = ss + sq;
    }
    part[t] = ss;
  }
  for (int32_t stride = 128; stride > 0; stride >>= 1)
    for (int32_t t = 0; t < stride; ++t) part[t] = part[t] + part[t + stride];
  const float inv = 1.0f / sqrtf(part[0] / (float)dim + eps);
  for (int32_t i = 0; i < dim; ++i) {
    const float a = h[i] * inv;
    out[i] = a * wt[i];
  }
}

typedef void (*mv_fn)(const uint8_t *, const float *, int32_t, int32_t, float *);

static int64_t mv_row_bytes(int32_t wtype, int32_t in_dim) {
  return wtype == 2 ? (int64_t)(in_dim >> 5) * 18 : wtype == 8 ? (int64_t)(in_dim >> 5) * 34
                                                               : (int64_t)in_dim * 2;
}

static mv_fn mv_pick(int32_t wtype, int32_t blocked) {
  if (wtype == 2) return blocked ? vdxo_matvec_q4_0_blocked : vdxo_matvec_q4_0;
  if (wtype == 8) return blocked ? vdxo_matvec_q8_0_blocked : vdxo_matvec_q8_0;
  return blocked ? vdxo_matvec_f16_blocked : vdxo_matvec_f16;
}

typedef struct {
  const uint8_t *w;
  const float *x;
  int32_t in_dim, r0, r1, blocked, wtype;
  float *out;
} mv_job;

static void *mv_worker(void *arg) {
  const mv_job *j = (const mv_job *)arg;
  const int64_t rb = mv_row_bytes(j->wtype, j->in_dim);
  if (j->r1 > j->r0)
    mv_pick(j->wtype, j->blocked)(j->w + rb * j->r0, j->x, j->in_dim, j->r1 - j->r0, j->out + j->r0);
  return NULL;
}

void vdxo_matvec_q4_0_mt(const uint8_t *w, const float *x, int32_t in_dim, int32_t rows,
                         float *logits, int32_t blocked, int32_t threads) {
  vdxo_matvec_mt(w, 2, x, in_dim, rows, logits, blocked, threads);
}

void vdxo_matvec_mt(const uint8_t *w, int32_t wtype, const float *x, int32_t in_dim, int32_t rows,
                    float *logits, int32_t blocked, int32_t threads) {
  if (threads < 1) threads = 1;
  pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)threads);
  mv_job *jobs = (mv_job *)malloc(sizeof(mv_job) * (size_t)threads);
  for (int32_t t = 0; t < threads; ++t) {
    mv_job *j = &jobs[t];
    j->w = w;
    j->x = x;
    j->in_dim = in_dim;
    j->r0 = (int32_t)((int64_t)rows * t / threads);
    j->r1 = (int32_t)((int64_t)rows * (t + 1) / threads);
    j->blocked = blocked;
    j->wtype = wtype;
    j->out = logits;
    pthread_create(&tid[t], NULL, mv_worker, j);
  }
  for (int32_t t = 0; t < threads; ++t) pthread_join(tid[t], NULL);
  free(tid);
  free(jobs);
}
