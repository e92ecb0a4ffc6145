/*
 * vdx_sampler.h -- C ABI of libvdxsampler.so, the MI355X (gfx950) token
 * sampler of VindexLLM.
 *
 * Drop-in boundary for TVdxSampler (src/VindexLLM.Sampler.pas:37-91 in the
 * reference).  Logits stay in HBM: the batched entry point samples B rows of
 * device-resident fp32 logits with hand-written HIP kernels and writes B
 * token ids, without a host round trip.  Every type is plain C (pointers,
 * fixed-width integers); `stream` is a hipStream_t passed as void*.
 *
 * Return codes: 0 = OK, negative = error (see VDX_E_*); the message is in
 * vdx_sampler_last_error().  No entry point falls back to the CPU.
 */
#ifndef VDX_SAMPLER_H
#define VDX_SAMPLER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VDX_OK 0
#define VDX_E_INVALID_ARG (-1)
#define VDX_E_HIP (-2)            /* HIP runtime / device error            */
#define VDX_E_UNSUPPORTED (-3)    /* configuration outside the GPU kernels */
#define VDX_E_NO_MEMORY (-4)

/* RNG used for the one uniform each non-greedy row consumes per call. */
#define VDX_RNG_XOSHIRO 0  /* reference stream (Sampler.pas:192-248); row r is
                              seeded as a reference sampler with Seed + r    */
#define VDX_RNG_PHILOX 1   /* counter-based Philox4x64-10: word 0 of block
                              {step,row,0,0} under key {Seed,0}; (x>>40)/2^24 */

/* Per-row diagnostic flags written to vdx_sample_outputs.flags. */
#define VDX_ROW_GREEDY 0x1
#define VDX_ROW_TOPK_FAST 0x2     /* exact top-K without slot-order replay   */
#define VDX_ROW_TOPK_REPLAY 0x4   /* exact path: the reference's min-buffer
                                     replayed over the logits that enter it */
#define VDX_ROW_FULL 0x8          /* K <= 0 or K >= V full-softmax path      */
#define VDX_ROW_NAN 0x10          /* row held NaN (or inf) handled literally */
#define VDX_ROW_FALLBACK 0x20     /* no cumulative weight exceeded t         */

/* TVdxSamplerConfig (src/VindexLLM.Sampler.pas:26-34), bit-identical to the
 * Pascal record under {$A8} (src/VindexLLM.Defines.inc:13): 32 bytes,
 * offsets 0,4,8,12,16,20,24. */
typedef struct vdx_sampler_config {
  float temperature;     /* 0 = greedy argmax, > 0 = divide logits by it     */
  int32_t top_k;         /* 0 = disabled (full softmax), > 0 = keep top K     */
  float top_p;           /* 1 = disabled, < 1 = nucleus (top-K path only)     */
  float min_p;           /* 0 = disabled, > 0 = floor relative to top prob    */
  float repeat_penalty;  /* 1 = disabled                                      */
  int32_t repeat_window; /* history ring length per row                       */
  int64_t seed;          /* 0 = timer seed, > 0 deterministic                 */
} vdx_sampler_config;

typedef struct vdx_sampler vdx_sampler;

/* Optional outputs of vdx_sampler_process_device.  Every pointer is device
 * memory and may be NULL.  topk_* hold `topk_stride` entries per row (>= K)
 * in descending (value, then lower index) order; topk_prob is the final
 * normalised probability (0 for entries cut by Min-P / Top-P).  A row of the
 * full-softmax path (K <= 0 or K >= V) writes entry 0 only: the drawn token
 * and its probability q / S (0 when the row's weights are not finite). */
typedef struct vdx_sample_outputs {
  int32_t *tokens;     /* [rows]                    */
  int32_t *topk_idx;   /* [rows * topk_stride]      */
  float *topk_prob;    /* [rows * topk_stride]      */
  int32_t topk_stride;
  uint32_t *flags;     /* [rows] VDX_ROW_*          */
  float *uniforms;     /* [rows] the uniform each row consumed (0 if greedy) */
} vdx_sample_outputs;

/* TVdxSampler.DefaultConfig (Sampler.pas:100-109). */
void vdx_sampler_default_config(vdx_sampler_config *out);

/* TVdxSampler.Create (Sampler.pas:111-122): default config, a RepeatWindow
 * ring per row, PRNG seeded from the timer (Seed = 0).  `max_rows` bounds
 * the batch of every later call; device memory is allocated here and grown
 * (outside the sampling call) when a larger vocabulary is first seen. */
int vdx_sampler_create(vdx_sampler **out, int32_t device, int32_t max_rows);

/* TVdxSampler.Destroy (Sampler.pas:124-130). */
void vdx_sampler_destroy(vdx_sampler *s);

/* TVdxSampler.SetConfig (Sampler.pas:132-150): a RepeatWindow change resizes
 * and clears every row's history; a Seed change reseeds every row (row r as a
 * sampler with Seed + r).  Rows given their own configs take this one again:
 * those whose window differs lose their history, those with their own seed
 * are reseeded as row r. */
int vdx_sampler_set_config(vdx_sampler *s, const vdx_sampler_config *cfg);

/* TVdxSampler.GetConfig (Sampler.pas:152-155): the sampler-wide config. */
int vdx_sampler_get_config(const vdx_sampler *s, vdx_sampler_config *out);

/* SetConfig for one row (Sampler.pas:132-150 applied to that row): a batch
 * of independent sequences in one sampler, each with its own temperature,
 * Top-K/Top-P/Min-P, penalty, window and seed (the reference holds one
 * sequence per sampler, Sampler.pas:37-91).  A changed RepeatWindow clears the
 * row's history; a changed Seed reseeds the row from Seed itself (a timer
 * value for 0), so it draws what a reference sampler with this config draws.
 * One call samples rows of different paths (greedy, top-K, full) together.
 * Waits for the device to be idle. */
int vdx_sampler_set_row_config(vdx_sampler *s, int32_t row, const vdx_sampler_config *cfg);
int vdx_sampler_get_row_config(const vdx_sampler *s, int32_t row, vdx_sampler_config *out);

/* TVdxSampler.Process (Sampler.pas:265-528) for one host-resident row, as
 * called by TVdxInference.RunUnembedding (Inference.pas:327-339): uploads the
 * row, samples it on the GPU (row 0's history and RNG), writes the
 * penalised logits back into `logits` (the reference mutates its input) and
 * returns the token id (>= 0) or a negative error code. */
int32_t vdx_sampler_process(vdx_sampler *s, float *logits, int32_t vocab);

/* Batched, device-resident Process: row r of `logits` starts at
 * logits + r*row_stride (fp32, device memory, mutated in place by the
 * repetition penalty exactly as Sampler.pas:285-303).  `uniforms` (device,
 * nullable) injects the per-row uniform in [0,1) that replaces the RNG draw
 * (the RNG is then not advanced); NULL draws from the sampler's RNG.
 * Every 0 < TopK < V takes the reference's top-K path (Sampler.pas:327-460);
 * TopK > 1024 runs one workgroup per row and is much slower.
 * Stream-ordered and asynchronous; allocates nothing once the workspace
 * covers `vocab` and TopK.  Rows must not alias. */
int vdx_sampler_process_device(vdx_sampler *s, float *logits, int32_t rows,
                               int32_t vocab, int64_t row_stride,
                               const float *uniforms,
                               const vdx_sample_outputs *out, void *stream);

/* Allocation-free sampling.  No counterpart in the reference: this entry
 * point is for callers that cannot allocate device memory -- code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc.  It
 * needs no sampler object and calls no hipMalloc, hipFree or allocating
 * library routine: its workspace is a fixed device array inside the library
 * (about 4.4 MiB per device, held until the process ends), whose device
 * address is looked up once per device on the first call made with that
 * device current.
 *
 * It samples `rows` device-resident rows exactly as vdx_sampler_process_device
 * does for a sampler whose config is *cfg, whose row r holds the ring of
 * history_count[r] ids at history + r*history_stride (the repetition penalty
 * is applied in place, as Sampler.pas:285-303 does; a count is clamped to
 * [0, min(RepeatWindow, history_stride)]), and whose draws are the injected
 * `uniforms` (device, one per row, required: there is no RNG state).
 * history/history_count may be NULL (no penalty).  Limits: rows <= 1024 and
 * rows * ceil(vocab / 16384) <= 4096 (e.g. 256 rows of 262144 logits), else
 * VDX_E_UNSUPPORTED.  Every call on one device shares that workspace and
 * overwrites it: calls that overlap on one device (concurrent streams or
 * threads) race and must be serialised by the caller.  Stream-ordered,
 * asynchronous; the message of a failure is vdx_sampler_last_error(NULL). */
int vdx_sample_device_noalloc(const vdx_sampler_config *cfg, float *logits, int32_t rows,
                              int32_t vocab, int64_t row_stride, const float *uniforms,
                              const int32_t *history, int32_t history_stride,
                              const int32_t *history_count, const vdx_sample_outputs *out,
                              void *stream);

/* The Q4_0 lm_head alone: shaders/matvec_q4_0.comp as
 * TVdxAttention.DispatchMatVec issues it for ATensorType = gtQ4_0
 * (Attention.pas:979-1025) from TVdxModel.UnembedToLogits (Model.pas:1258-1270),
 * batched over `rows` hidden vectors:
 *   logits[r*logit_stride + v] = sum_e dequant(W[v][e]) * hidden[r*in_dim + e].
 * `weights`: vocab rows of in_dim/32 Q4_0 blocks (18 bytes: fp16 scale, then
 * 16 bytes of nibbles; GGUFReader.pas:264-281), 16-byte aligned; in_dim must
 * be a multiple of 32 (one block), as matvec_q4_0.comp takes it; rows whose
 * length is not a multiple of 256 read their last blocks with 2-byte loads,
 * and in the GGUF layout every block of such rows does (the packed layout
 * keeps whole slices fast).  `scratch` holds an element-major copy of up to 16
 * hidden rows: at least 16*in_dim floats when rows > 1 (may be NULL when
 * rows == 1).  Every pointer is device memory.  Stream-ordered,
 * asynchronous, allocates nothing; the message of a failure is
 * vdx_sampler_last_error(NULL). */
int vdx_lmhead_q4_0(const void *weights, const float *hidden, int32_t rows, int32_t in_dim,
                    int32_t vocab, float *logits, int64_t logit_stride, float *scratch,
                    void *stream);

/* lm_head weight formats: the GGML tensor type ids (GGUFReader.pas:34-42)
 * that TVdxAttention.DispatchMatVec selects a shader by (Attention.pas:994-1014). */
#define VDX_TENSOR_F16 1   /* in_dim fp16 values per row (matvec_f16.comp)          */
#define VDX_TENSOR_Q4_0 2  /* 18-byte blocks: fp16 d, 16 bytes of nibbles          */
#define VDX_TENSOR_Q8_0 8  /* 34-byte blocks: fp16 d, 32 int8 (matvec_q8_0.comp)   */
/* OR-ed into wtype: `weights` are in the packed layout of vdx_lmhead_pack. */
#define VDX_LMHEAD_PACKED 0x100

/* TVdxModel.UnembedToLogits (Model.pas:1258-1270) batched over `rows` hidden
 * vectors: the output RMSNorm as TVdxLayerNorm.ApplyCopy issues it
 * (LayerNorm.pas:395-417, shaders/rmsnorm_copy.comp:
 *   xn[e] = (h[e] * inv_rms) * norm_weight[e],
 *   inv_rms = 1 / sqrt(sum_e h[e]^2 / in_dim + norm_eps)),
 * skipped when `norm_weight` is NULL, then the lm_head in the weight tensor's
 * own format `wtype` (VDX_TENSOR_*), as TVdxAttention.DispatchMatVec issues it
 * (Attention.pas:979-1025): logits[r*logit_stride + v] = sum_e W(v,e) * xn_r[e].
 * `weights` is 16-byte aligned; in_dim is a multiple of 32; `scratch` (at
 * least 16*in_dim floats) holds the prepared hidden rows and is required when
 * rows > 1 or with the norm.  Every pointer is device memory.  Stream-ordered,
 * asynchronous, allocates nothing; a failure's message is
 * vdx_sampler_last_error(NULL); an unknown wtype is VDX_E_UNSUPPORTED. */
int vdx_lmhead(const void *weights, int32_t wtype, const float *hidden, const float *norm_weight,
               float norm_eps, int32_t rows, int32_t in_dim, int32_t vocab, float *logits,
               int64_t logit_stride, float *scratch, void *stream);

/* The lm_head weights repacked for MI355X, once, when the model is loaded (no
 * counterpart in the reference, whose UploadWeightTensor, Model.pas:549-600,
 * uploads the GGUF bytes as they are): the same bytes permuted so that, for
 * each group of 64 rows (the last padded with zero rows), each K slice and
 * each 16-byte (Q8_0: 8-byte) piece, the 64 rows' pieces are consecutive.  A
 * row of a Q4_0 or Q8_0 tensor is not a whole number of 128-byte cache
 * lines, so reading K slices of rows from the GGUF layout fetches the lines
 * at slice boundaries twice; in the packed layout every line is read once, by
 * one coalesced load.  vdx_lmhead and vdx_sampler_lmhead_device read it when
 * wtype carries VDX_LMHEAD_PACKED and give bit-identical logits.
 * vdx_lmhead_packed_bytes returns the packed size (or VDX_E_INVALID_ARG);
 * vdx_lmhead_pack writes it (device buffers, 16-byte aligned; stream-ordered,
 * allocates nothing). */
int64_t vdx_lmhead_packed_bytes(int32_t wtype, int32_t in_dim, int32_t vocab);
int vdx_lmhead_pack(const void *weights, int32_t wtype, int32_t in_dim, int32_t vocab, void *packed,
                    int64_t packed_bytes, void *stream);

/* RunUnembedding followed by Process (Inference.pas:327-339) with the logits
 * kept in HBM: UnembedToLogits (as vdx_lmhead, the sampler's own workspace as
 * scratch) writes rows x vocab logits into `logits` (device, row stride
 * logit_stride >= vocab) or, when `logits` is NULL, into the sampler's own
 * workspace (allocated on the first call with a larger rows*vocab); the rows
 * are then sampled exactly as by vdx_sampler_process_device. */
int vdx_sampler_lmhead_device(vdx_sampler *s, const void *weights, int32_t wtype, const float *hidden,
                              const float *norm_weight, float norm_eps, int32_t rows, int32_t in_dim,
                              int32_t vocab, float *logits, int64_t logit_stride,
                              const float *uniforms, const vdx_sample_outputs *out, void *stream);

/* RunUnembedding followed by Process (Inference.pas:327-339) with the logits
 * kept in HBM: the Q4_0 lm_head (as vdx_lmhead_q4_0) writes rows x vocab
 * logits into `logits` (device, row stride logit_stride >= vocab) or, when
 * `logits` is NULL, into the sampler's own workspace (allocated on the first
 * call with a larger rows*vocab); the rows are then sampled exactly as by
 * vdx_sampler_process_device (penalty in place, per-row RNG or injected
 * uniforms, same outputs). */
int vdx_sampler_lmhead_q4_0_device(vdx_sampler *s, const void *weights, const float *hidden,
                                   int32_t rows, int32_t in_dim, int32_t vocab, float *logits,
                                   int64_t logit_stride, const float *uniforms,
                                   const vdx_sample_outputs *out, void *stream);

/* ---- GGUF model files (TVdxGGUFReader, GGUFReader.pas) ---------------------
 * The lm_head's inputs come from the model file: `token_embd.weight` (the
 * tied lm_head, Model.Gemma3.pas:180-198, in its GGUF layout as vdx_lmhead
 * reads it), `output_norm.weight` (:174) and the dimensions.  The file is
 * memory-mapped read-only and parsed as the reader does (header, metadata,
 * tensor directory, aligned data section: GGUFReader.pas:605-745); a
 * malformed file is an error (message in vdx_gguf_last_error), never a fault. */
typedef struct vdx_gguf vdx_gguf;
typedef struct vdx_gguf_tensor {
  int32_t type;          /* GGML type id (VDX_TENSOR_* among them)          */
  int32_t n_dims;
  uint64_t dims[4];      /* dims[0] varies fastest (the row length)          */
  uint64_t nbytes;       /* VdxGGMLTensorBytes (GGUFReader.pas:264-318); 0
                            for types it does not size                      */
  uint64_t file_offset;
  const void *data;      /* host pointer into the mapping, valid until close */
} vdx_gguf_tensor;

typedef struct vdx_gguf_info {
  uint32_t version;        /* GetVersion (GGUFReader.pas:747)                 */
  uint32_t alignment;      /* GetAlignment (:762); general.alignment or 32    */
  uint64_t tensor_count;   /* GetTensorCount (:752)                           */
  uint64_t metadata_count; /* GetMetadataCount (:757), as the header states   */
  uint64_t file_size;      /* GetFileSize (:767)                              */
  uint64_t data_offset;    /* file offset of the tensor data (:727-745)       */
} vdx_gguf_info;

/* TVdxGGUFReader.Open (GGUFReader.pas:376-430): map and parse; *out is NULL
 * on failure, with the message in vdx_gguf_last_error(NULL). */
int vdx_gguf_open(vdx_gguf **out, const char *path);
/* TVdxGGUFReader.Close (:360): unmaps; every data pointer becomes invalid. */
void vdx_gguf_close(vdx_gguf *g);
const char *vdx_gguf_last_error(const vdx_gguf *g);
int vdx_gguf_get_info(const vdx_gguf *g, vdx_gguf_info *out);
/* GetTensorList (:878): name of tensor `index` in directory order into buf
 * (NUL-terminated, truncated to cap-1); returns the full length. */
int vdx_gguf_tensor_name(const vdx_gguf *g, int64_t index, char *buf, int32_t cap);
/* GetTensorInfo + GetTensorDataPtr (:847-876) for `name`: VDX_E_INVALID_ARG
 * when absent; VDX_E_UNSUPPORTED when its bytes would run past the end of the
 * file (type, dims and file_offset filled, data NULL). */
int vdx_gguf_find_tensor(vdx_gguf *g, const char *name, vdx_gguf_tensor *out);
/* GetMetadataKeys (:826): distinct key `index` in file order into buf;
 * returns the full length. */
int vdx_gguf_meta_key(const vdx_gguf *g, int64_t index, char *buf, int32_t cap);
/* HasMetadata (:774) / TVdxGGUFMetaValue.ValueType: the GGUF value type
 * (0..12) of `key`, or VDX_E_INVALID_ARG when absent. */
int vdx_gguf_meta_type(const vdx_gguf *g, const char *key);
/* Metadata values (GetMetadata, :779): integers of any width and bools as
 * int64, floats of either width as double, strings copied into buf
 * (NUL-terminated; returns the full length), arrays as element type and
 * length (tokenizer.ggml.tokens gives the vocabulary size, Tokenizer.pas:124).
 * A key of another type is VDX_E_INVALID_ARG. */
int vdx_gguf_meta_int(vdx_gguf *g, const char *key, int64_t *out);
int vdx_gguf_meta_float(vdx_gguf *g, const char *key, double *out);
int vdx_gguf_meta_string(vdx_gguf *g, const char *key, char *buf, int32_t cap);
int vdx_gguf_meta_array(vdx_gguf *g, const char *key, int32_t *elem_type, int64_t *length);

/* TVdxSampler.AddToHistory (Sampler.pas:530-539) for one row. */
int vdx_sampler_add_to_history(vdx_sampler *s, int32_t row, int32_t token);

/* AddToHistory for rows [0, rows) from device-resident token ids, as the
 * generation loop does after each step (Inference.pas:653). */
int vdx_sampler_add_to_history_device(vdx_sampler *s, const int32_t *tokens,
                                      int32_t rows, void *stream);

/* TVdxSampler.ResetHistory (Sampler.pas:541-549) for one row (row < 0: all
 * rows): clears the ring and reseeds that row only when Seed > 0. */
int vdx_sampler_reset_history(vdx_sampler *s, int32_t row);

/* Replaces a row's history ring (count ids in array order, next write
 * position `pos`); the reference has no bulk setter -- this restores a saved
 * ring (sampler-state checkpoint). */
int vdx_sampler_set_history(vdx_sampler *s, int32_t row, const int32_t *ids,
                            int32_t count, int32_t pos);

/* Reads a row's history ring back (up to `cap` ids); returns the count. */
int32_t vdx_sampler_get_history(vdx_sampler *s, int32_t row, int32_t *ids,
                                int32_t cap, int32_t *pos);

/* Sampler-state checkpoint of one row: its config, RNG state (xoshiro256**
 * words, Philox counter and key) and history ring as one self-contained blob
 * (the reference's SaveKVCache / LoadKVCache, Inference.pas:750-900, keep no
 * sampler state, so a restored session draws a different stream).  Waits for
 * the calls issued so far.  Returns the blob's size; nothing is written when
 * buf is NULL or cap is smaller. */
int64_t vdx_sampler_save_row_state(vdx_sampler *s, int32_t row, void *buf, int64_t cap);

/* Restores a blob from vdx_sampler_save_row_state into `row` of this or
 * another sampler with the same RNG kind: the row then continues exactly as
 * the saved one would have (its config becomes the row's own). */
int vdx_sampler_load_row_state(vdx_sampler *s, int32_t row, const void *buf, int64_t size);

/* Selects VDX_RNG_XOSHIRO (default) or VDX_RNG_PHILOX; reseeds all rows. */
int vdx_sampler_set_rng(vdx_sampler *s, int32_t kind);

/* Instrumentation; no counterpart in the reference.  When enabled, every
 * vdx_sampler_process_device call records HIP events on its stream before the
 * penalty kernel, between the penalty and the sampling kernel, and after the
 * sampling kernel (events are created here, not in the sampling call). */
int vdx_sampler_set_timing(vdx_sampler *s, int32_t enable);

/* Sum (ms) and count of the recorded durations since the last query:
 * which = 0 the sampling kernel(s), 1 the penalty kernel, 2 the whole call.
 * Waits for the recorded events, then clears the record. */
int vdx_sampler_get_timing(vdx_sampler *s, int32_t which, double *total_ms,
                           int64_t *count);

/* Last error message of `s` (or of the last failed create when s is NULL). */
const char *vdx_sampler_last_error(const vdx_sampler *s);

/* Library version string. */
const char *vdx_sampler_version(void);

#ifdef __cplusplus
}
#endif
#endif
