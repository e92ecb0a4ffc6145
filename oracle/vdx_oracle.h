/*
 * vdx_oracle.h -- CPU oracle for the token-sampling path of VindexLLM.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference
 * sampler TVdxSampler (src/VindexLLM.Sampler.pas) that the HIP library's
 * results are compared with, and the CPU baseline timed by bench.py.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product library (libvdxsampler.so) never links or calls it.
 *
 * Every function cites the reference lines it restates.  Floating-point
 * semantics follow the reference compiled for Win64 with Delphi's default
 * excess precision: Single sub-expressions feeding Exp() are evaluated in
 * double; every value stored into a Single is rounded to binary32.
 *
 * Pinning (tests/test_oracle_pins.py): the PRNG by published known answers
 * and an independent numpy restatement, Philox by numpy's bit generator,
 * penalty / greedy / top-K slots by brute force, the softmax tail and the
 * full path by an independent numpy restatement and closed forms, the
 * stateful object by the reference's own testbed invariants.  Parity
 * unpinned: the last-ulp bits of Delphi's System.Exp (this file uses the C
 * library's exp), the excess-precision choice for (v - M) * invT, and the
 * Seed = 0 timer stream (taken as an argument here).
 */
#ifndef VDX_ORACLE_H
#define VDX_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* TVdxSamplerConfig, src/VindexLLM.Sampler.pas:26-34, laid out as the Pascal
 * record under {$A8} (src/VindexLLM.Defines.inc:13): 32 bytes. */
typedef struct vdxo_config {
  float temperature;     /* 0 = greedy argmax                         */
  int32_t top_k;         /* 0 = disabled                              */
  float top_p;           /* 1 = disabled                              */
  float min_p;           /* 0 = disabled                              */
  float repeat_penalty;  /* 1 = disabled                              */
  int32_t repeat_window; /* history ring length                       */
  int64_t seed;          /* 0 = timer seed                            */
} vdxo_config;

/* Which branch of Process() produced the token. */
enum { VDXO_PATH_GREEDY = 0, VDXO_PATH_TOPK = 1, VDXO_PATH_FULL = 2 };

#define VDXO_KMAX 1024

/* Diagnostics of one Process() call, for parity tests. */
typedef struct vdxo_trace {
  int32_t path;          /* VDXO_PATH_*                                       */
  int32_t k;             /* K used by the top-K path                          */
  float max_logit;       /* M (top-K path: raw logits; full path: scaled)     */
  float inv_temp;        /* fl32(1/T)                                         */
  int32_t slot_idx[VDXO_KMAX];  /* top-K min-buffer indices, slot order       */
  float slot_val[VDXO_KMAX];    /* top-K min-buffer values, slot order        */
  int32_t order_idx[VDXO_KMAX]; /* final draw order (sorted if top-p ran)     */
  float order_q[VDXO_KMAX];     /* weights in final draw order (0 = dropped)  */
  int32_t n_replacements;       /* min-buffer replacements during the scan    */
  double sum_initial;    /* S after softmax (slot / index order)              */
  double sum_final;      /* S used for the draw                               */
  double target;         /* t = double(u) * S                                 */
  double cdf_lo;         /* cumulative weight before the chosen entry         */
  double cdf_hi;         /* cumulative weight after the chosen entry          */
  int32_t fallback;      /* 1 if no cumulative weight exceeded t              */
  int32_t token;
} vdxo_trace;

/* ---- PRNG (src/VindexLLM.Sampler.pas:157-248) -------------------------- */
uint64_t vdxo_splitmix64(uint64_t *state);                  /* :194-201 */
void vdxo_seed(uint64_t st[4], uint64_t seed_state);        /* :224-241 */
uint64_t vdxo_next_u64(uint64_t st[4]);                     /* :208-222 */
float vdxo_next_float(uint64_t st[4]);                      /* :243-248 */
uint64_t vdxo_wrap_mul(uint64_t a, uint64_t b);             /* :169-190 */
uint64_t vdxo_wrap_add(uint64_t a, uint64_t b);             /* :160-167 */

/* Counter-based Philox4x64-10 (Salmon et al., SC'11), the RNG of the HIP
 * library's Philox mode; not in the reference. */
void vdxo_philox4x64_10(const uint64_t ctr[4], const uint64_t key[2],
                        uint64_t out[4]);
/* Uniform in [0,1) with the reference's 24-bit resolution drawn from
 * Philox4x64-10 at counter {step,row,0,0}, key {seed,0}. */
float vdxo_philox_uniform(uint64_t seed, uint64_t row, uint64_t step);
/* 24-bit uniform from a raw 64-bit word: (x >> 40) / 2^24 (:247). */
float vdxo_u24(uint64_t x);

/* ---- Process() stages --------------------------------------------------- */
/* Step 0, repetition penalty, in place (:285-303). */
void vdxo_apply_penalty(float *logits, int32_t vocab, const int32_t *hist,
                        int32_t hist_count, float penalty);

/* One Process() call on one row with the PRNG draw replaced by `u`
 * (:265-528).  `logits` is mutated by the penalty exactly as the reference
 * does.  `hist` may be NULL when hist_count == 0.  `trace` may be NULL. */
int32_t vdxo_process_row(float *logits, int32_t vocab, const vdxo_config *cfg,
                         const int32_t *hist, int32_t hist_count, float u,
                         vdxo_trace *trace);

/* Rows processed serially (the reference's single-threaded loop), each row
 * with its own history slice (hist + r*hist_stride, count hcount[r]) and its
 * own uniform u[r].  Used as the CPU baseline.  `hcount` may be NULL. */
void vdxo_process_batch(float *logits, int32_t rows, int32_t vocab,
                        int64_t row_stride, const vdxo_config *cfg,
                        const int32_t *hist, int32_t hist_stride,
                        const int32_t *hcount, const float *u,
                        int32_t *tokens);
/* Same, split over `threads` POSIX threads (rows divided evenly). */
void vdxo_process_batch_mt(float *logits, int32_t rows, int32_t vocab,
                           int64_t row_stride, const vdxo_config *cfg,
                           const int32_t *hist, int32_t hist_stride,
                           const int32_t *hcount, const float *u,
                           int32_t *tokens, int32_t threads);

/* ---- Stateful sampler mirroring the TVdxSampler object ------------------- */
typedef struct vdxo_sampler vdxo_sampler;
vdxo_sampler *vdxo_sampler_create(void);                          /* :111-122 */
void vdxo_sampler_destroy(vdxo_sampler *s);                        /* :124-130 */
void vdxo_default_config(vdxo_config *cfg);                        /* :100-109 */
/* `timer_seed` is used in place of QueryPerformanceCounter when Seed = 0. */
void vdxo_sampler_set_config(vdxo_sampler *s, const vdxo_config *cfg,
                             uint64_t timer_seed);                 /* :132-150 */
void vdxo_sampler_get_config(const vdxo_sampler *s, vdxo_config *cfg);
int32_t vdxo_sampler_process(vdxo_sampler *s, float *logits, int32_t vocab,
                             vdxo_trace *trace);                   /* :265-528 */
void vdxo_sampler_add_to_history(vdxo_sampler *s, int32_t id);     /* :530-539 */
void vdxo_sampler_reset_history(vdxo_sampler *s);                  /* :541-549 */
int32_t vdxo_sampler_history(const vdxo_sampler *s, int32_t *out, int32_t cap,
                             int32_t *pos);
void vdxo_sampler_rng_state(const vdxo_sampler *s, uint64_t st[4]);

/* ---- Q4_0 lm_head (shaders/matvec_q4_0.comp) ----------------------------- */
/* logits[r] for r in [0, rows): the shader's per-lane strided fp32 partial
 * sums (lane = e mod 64) followed by its LDS tree reduction (strides
 * 32..1).  `w` holds rows x (in_dim/32) blocks of 18 bytes. */
void vdxo_matvec_q4_0(const uint8_t *w, const float *x, int32_t in_dim,
                      int32_t rows, float *logits);
/* The same products summed in the library kernel's order: per row, per
 * block k in order: s = 0; s = fmaf(q_i - 8, x[32k+i], s) for i = 0..31;
 * acc = fmaf(d_k, s, acc). */
void vdxo_matvec_q4_0_blocked(const uint8_t *w, const float *x, int32_t in_dim,
                              int32_t rows, float *logits);
/* Either order (blocked != 0: the kernel's) over `threads` POSIX threads,
 * rows split evenly. */
void vdxo_matvec_q4_0_mt(const uint8_t *w, const float *x, int32_t in_dim, int32_t rows,
                         float *logits, int32_t blocked, int32_t threads);
/* ---- Q8_0 / F16 lm_head and the output RMSNorm ---------------------------- */
/* shaders/matvec_q8_0.comp: 256 strided lanes, acc += (q * d) * x, LDS tree. */
void vdxo_matvec_q8_0(const uint8_t *w, const float *x, int32_t in_dim, int32_t rows,
                      float *logits);
/* The library kernel's Q8_0 order: per block s = fmaf(q_i, x, s), acc = fmaf(d, s, acc). */
void vdxo_matvec_q8_0_blocked(const uint8_t *w, const float *x, int32_t in_dim, int32_t rows,
                              float *logits);
/* shaders/matvec_f16.comp: 256 strided lanes over f16 pairs, LDS tree. */
void vdxo_matvec_f16(const uint8_t *w, const float *x, int32_t in_dim, int32_t rows,
                     float *logits);
/* The library kernel's F16 order: per 32 elements s = fmaf(w_i, x, s), acc = acc + s. */
void vdxo_matvec_f16_blocked(const uint8_t *w, const float *x, int32_t in_dim, int32_t rows,
                             float *logits);
/* Any of the three formats (wtype: GGML id 1 F16, 2 Q4_0, 8 Q8_0), either
 * order, over `threads` POSIX threads. */
void vdxo_matvec_mt(const uint8_t *w, int32_t wtype, const float *x, int32_t in_dim, int32_t rows,
                    float *logits, int32_t blocked, int32_t threads);
/* shaders/rmsnorm_copy.comp (TVdxLayerNorm.ApplyCopy). */
void vdxo_rmsnorm(const float *h, const float *w, float eps, int32_t dim, float *out);
/* fp16 -> fp32 (IEEE binary16), as unpackHalf2x16. */
float vdxo_half_to_float(uint16_t h);

#ifdef __cplusplus
}
#endif
#endif
