// vdx_sampler.hpp -- C++ mirror of the reference's sampler class over the C ABI
// of libvdxsampler.so (vdx_sampler.h).
//
// TVdxSampler and TVdxSamplerConfig keep the names, argument meaning and
// defaults of src/VindexLLM.Sampler.pas:26-91 (Create / Destroy / SetConfig /
// GetConfig / DefaultConfig / Process / AddToHistory / ResetHistory), and the
// error list of TVdxBaseObject (GetErrors, src/VindexLLM.Utils.pas): no call
// throws; a failure is recorded (severity, code, message) and the call returns
// a negative VDX_E_* code where the Pascal method would return a value.
// Sampling always runs in the library's GPU kernels; there is no CPU fallback
// (without a GPU, construction records a fatal error and every call fails).
//
// Beyond the reference: ProcessDevice (a batch of device-resident rows),
// per-row configs and row checkpoints, history access.
#pragma once

#include <stdint.h>

#include <string>
#include <utility>
#include <vector>

#include "vdx_sampler.h"

namespace vdx {

// TVdxSamplerConfig (Sampler.pas:26-34): the C record, same layout.
typedef vdx_sampler_config TVdxSamplerConfig;

enum class TVdxErrorSeverity { esError, esFatal };

struct TVdxError {
  TVdxErrorSeverity Severity;
  std::string Code;     // "SAMPLER"
  std::string Message;  // vdx_sampler_last_error
};

// TVdxErrors (Utils.pas): the object's error list.
class TVdxErrors {
 public:
  bool HasErrors() const { return !items_.empty(); }
  bool HasFatal() const {
    for (const TVdxError &e : items_)
      if (e.Severity == TVdxErrorSeverity::esFatal) return true;
    return false;
  }
  int Count() const { return (int)items_.size(); }
  const std::vector<TVdxError> &GetItems() const { return items_; }
  void Clear() { items_.clear(); }
  void Add(TVdxErrorSeverity s, std::string code, std::string msg) {
    items_.push_back(TVdxError{s, std::move(code), std::move(msg)});
  }

 private:
  std::vector<TVdxError> items_;
};

class TVdxSampler {
 public:
  // Create (Sampler.pas:111-122): the default (greedy) config, timer seed.
  // `max_rows` bounds ProcessDevice batches; Process samples row 0.
  explicit TVdxSampler(int32_t device = 0, int32_t max_rows = 1) {
    const int rc = vdx_sampler_create(&h_, device, max_rows);
    if (rc != VDX_OK) {
      h_ = nullptr;
      fail(TVdxErrorSeverity::esFatal, rc);
    }
  }
  // Destroy (Sampler.pas:124-130).
  ~TVdxSampler() {
    if (h_) vdx_sampler_destroy(h_);
  }
  TVdxSampler(const TVdxSampler &) = delete;
  TVdxSampler &operator=(const TVdxSampler &) = delete;

  TVdxErrors &GetErrors() { return errors_; }
  bool Ok() const { return h_ != nullptr; }

  // DefaultConfig (Sampler.pas:100-109).
  static TVdxSamplerConfig DefaultConfig() {
    TVdxSamplerConfig c;
    vdx_sampler_default_config(&c);
    return c;
  }
  // SetConfig / GetConfig (Sampler.pas:132-155): a RepeatWindow change clears
  // the history, a Seed change reseeds.
  int SetConfig(const TVdxSamplerConfig &c) { return check(vdx_sampler_set_config(h_, &c)); }
  TVdxSamplerConfig GetConfig() const {
    TVdxSamplerConfig c = DefaultConfig();
    if (h_) vdx_sampler_get_config(h_, &c);
    return c;
  }

  // Process (Sampler.pas:265-528): one host row of AVocabSize logits,
  // penalised in place as the reference does; returns the token id (or a
  // negative VDX_E_* code, recorded in GetErrors()).
  int32_t Process(float *ALogits, int32_t AVocabSize) {
    if (!h_) return missing();
    const int32_t r = vdx_sampler_process(h_, ALogits, AVocabSize);
    if (r < 0) fail(TVdxErrorSeverity::esError, r);
    return r;
  }

  // AddToHistory / ResetHistory (Sampler.pas:530-549).
  int AddToHistory(int32_t ATokenId, int32_t row = 0) {
    return check(vdx_sampler_add_to_history(h_, row, ATokenId));
  }
  int ResetHistory(int32_t row = -1) { return check(vdx_sampler_reset_history(h_, row)); }

  // ---- beyond the reference ------------------------------------------------
  // `rows` device-resident rows (device pointers), see vdx_sampler_process_device.
  int ProcessDevice(float *logits, int32_t rows, int32_t vocab, int64_t row_stride, const float *uniforms,
                    const vdx_sample_outputs &out, void *stream = nullptr) {
    return check(vdx_sampler_process_device(h_, logits, rows, vocab, row_stride, uniforms, &out, stream));
  }
  int SetRowConfig(int32_t row, const TVdxSamplerConfig &c) {
    return check(vdx_sampler_set_row_config(h_, row, &c));
  }
  TVdxSamplerConfig GetRowConfig(int32_t row) const {
    TVdxSamplerConfig c = DefaultConfig();
    if (h_) vdx_sampler_get_row_config(h_, row, &c);
    return c;
  }
  std::vector<int32_t> GetHistory(int32_t row, int32_t *pos = nullptr) {
    const int32_t w = GetRowConfig(row).repeat_window;
    std::vector<int32_t> ids(w > 0 ? (size_t)w : 1u);
    int32_t p = 0;
    const int32_t n = h_ ? vdx_sampler_get_history(h_, row, ids.data(), (int32_t)ids.size(), &p) : missing();
    if (n < 0) {
      fail(TVdxErrorSeverity::esError, n);
      return {};
    }
    ids.resize(w > 0 && n < w ? (size_t)n : (w > 0 ? (size_t)w : 0u));
    if (pos) *pos = p;
    return ids;
  }
  std::vector<uint8_t> SaveRowState(int32_t row) {
    if (!h_) return (missing(), std::vector<uint8_t>());
    const int64_t n = vdx_sampler_save_row_state(h_, row, nullptr, 0);
    if (n < 0) return (fail(TVdxErrorSeverity::esError, (int)n), std::vector<uint8_t>());
    std::vector<uint8_t> b((size_t)n);
    if (vdx_sampler_save_row_state(h_, row, b.data(), n) != n) fail(TVdxErrorSeverity::esError, VDX_E_HIP);
    return b;
  }
  int LoadRowState(int32_t row, const std::vector<uint8_t> &b) {
    return check(vdx_sampler_load_row_state(h_, row, b.data(), (int64_t)b.size()));
  }
  vdx_sampler *Handle() const { return h_; }

 private:
  int missing() {
    errors_.Add(TVdxErrorSeverity::esError, "SAMPLER", "sampler was not created");
    return VDX_E_INVALID_ARG;
  }
  int check(int rc) {
    if (!h_) return missing();
    if (rc < 0) fail(TVdxErrorSeverity::esError, rc);
    return rc;
  }
  void fail(TVdxErrorSeverity s, int rc) {
    const char *m = vdx_sampler_last_error(h_);
    errors_.Add(s, "SAMPLER", std::string(m ? m : "") + " (code " + std::to_string(rc) + ")");
  }

  vdx_sampler *h_ = nullptr;
  TVdxErrors errors_;
};

}  // namespace vdx
