// The reference's sampler testbed (testbed/UTest.Sampler.pas:53-327) run
// against the GPU library through the C++ mirror of the Pascal class
// (include/vdx_sampler.hpp): the same sections, logits and checks, with a
// Section / Check / FlushErrors harness shaped like TVdxTestCase
// (src/VindexLLM.TestCase.pas).  A few checks beyond the reference follow:
// per-row configs, row checkpoints and the no-GPU error path.
//
// Exit status: 0 when every check passes, 77 when no GPU is present (the
// constructor's fatal error is checked and reported), else the number of
// failed checks.
#include <stdio.h>
#include <string.h>

#include <string>
#include <vector>

#include "vdx_sampler.hpp"

using vdx::TVdxSampler;
using vdx::TVdxSamplerConfig;

static int g_fail = 0, g_pass = 0;

static void Section(const char *name) { printf("== %s\n", name); }
static void Check(bool ok, const char *what) {
  printf("  [%s] %s\n", ok ? "PASS" : "FAIL", what);
  (ok ? g_pass : g_fail)++;
}
static void FlushErrors(vdx::TVdxErrors &e) {
  for (const vdx::TVdxError &x : e.GetItems()) printf("  error %s: %s\n", x.Code.c_str(), x.Message.c_str());
  Check(!e.HasErrors(), "no errors recorded");
  e.Clear();
}

static const int CVocabSize = 10;  // UTest.Sampler.pas: CVocabSize

static void SecCreateDestroy() {
  Section("Create / Destroy + default config");
  TVdxSampler s;
  Check(s.Ok(), "Create returned a usable instance");
  const TVdxSamplerConfig c = s.GetConfig();
  Check(c.temperature == 0.0f, "Default Temperature = 0.0");
  Check(c.top_k == 0, "Default TopK = 0");
  Check(c.top_p == 1.0f, "Default TopP = 1.0");
  Check(c.min_p == 0.0f, "Default MinP = 0.0");
  Check(c.repeat_penalty == 1.0f, "Default RepeatPenalty = 1.0");
  Check(c.repeat_window == 64, "Default RepeatWindow = 64");
  Check(c.seed == 0, "Default Seed = 0");
  FlushErrors(s.GetErrors());
}

static void SecGreedyArgmax() {
  Section("Greedy argmax (Temperature = 0)");
  float L[CVocabSize];
  for (int i = 0; i < CVocabSize; ++i) L[i] = 0.1f;
  L[7] = 5.0f;
  TVdxSampler s;
  TVdxSamplerConfig c = TVdxSampler::DefaultConfig();
  c.temperature = 0.0f;
  s.SetConfig(c);
  Check(s.Process(L, CVocabSize) == 7, "Argmax returns index 7");
  L[7] = 0.1f;
  L[2] = 9.9f;
  Check(s.Process(L, CVocabSize) == 2, "Argmax tracks new max at index 2");
  FlushErrors(s.GetErrors());
}

static void SecDeterministicReseed() {
  Section("Deterministic re-seed (seed = 42)");
  const int CIters = 50;
  float L[CVocabSize];
  for (int i = 0; i < CVocabSize; ++i) L[i] = i * 0.25f;
  TVdxSamplerConfig c = TVdxSampler::DefaultConfig();
  c.temperature = 1.0f;
  c.seed = 42;
  std::vector<int> a, b;
  {
    TVdxSampler s;
    s.SetConfig(c);
    for (int i = 0; i < CIters; ++i) a.push_back(s.Process(L, CVocabSize));
  }
  {
    TVdxSampler s;
    s.SetConfig(c);
    for (int i = 0; i < CIters; ++i) b.push_back(s.Process(L, CVocabSize));
  }
  Check(a == b, "Two seed=42 samplers produce byte-identical 50-token sequences");
}

static void SecTopKBound() {
  Section("Top-K bound (K = 3 over 10 logits)");
  float L[CVocabSize] = {0};
  L[1] = L[4] = L[8] = 10.0f;
  TVdxSamplerConfig c = TVdxSampler::DefaultConfig();
  c.temperature = 1.0f;
  c.top_k = 3;
  c.seed = 42;
  TVdxSampler s;
  s.SetConfig(c);
  bool in = true;
  for (int i = 0; i < 200 && in; ++i) {
    const int r = s.Process(L, CVocabSize);
    in = (r == 1 || r == 4 || r == 8);
  }
  Check(in, "All 200 samples fall within top-3 index set {1, 4, 8}");
  FlushErrors(s.GetErrors());
}

static void SecRepeatPenalty() {
  Section("Repeat penalty reduces frequency of penalized token");
  float L[CVocabSize], Lc[CVocabSize];
  for (int i = 0; i < CVocabSize; ++i) L[i] = 1.0f;
  TVdxSamplerConfig c = TVdxSampler::DefaultConfig();
  c.temperature = 1.0f;
  c.repeat_penalty = 1.0f;
  c.seed = 42;
  int plain = 0, pen = 0;
  {
    TVdxSampler s;
    s.SetConfig(c);
    for (int i = 0; i < 200; ++i) {
      memcpy(Lc, L, sizeof(L));
      plain += s.Process(Lc, CVocabSize) == 3;
    }
  }
  c.repeat_penalty = 2.0f;
  {
    TVdxSampler s;
    s.SetConfig(c);
    s.AddToHistory(3);
    for (int i = 0; i < 200; ++i) {
      memcpy(Lc, L, sizeof(L));
      pen += s.Process(Lc, CVocabSize) == 3;
    }
    FlushErrors(s.GetErrors());
  }
  Check(pen < plain, "Penalized token 3 sampled less often with RepeatPenalty = 2.0");
  Check(plain >= 5, "Baseline frequency of token 3 is plausible (>= 5 of 200)");
}

// ---- beyond the reference --------------------------------------------------
static void SecRowConfigsAndCheckpoint() {
  Section("Per-row configs and a row checkpoint (beyond the reference)");
  float L[CVocabSize];
  for (int i = 0; i < CVocabSize; ++i) L[i] = i * 0.25f;
  TVdxSamplerConfig c = TVdxSampler::DefaultConfig();
  c.temperature = 1.0f;
  c.seed = 42;
  std::vector<int> want;
  {
    TVdxSampler s;
    s.SetConfig(c);
    for (int i = 0; i < 20; ++i) want.push_back(s.Process(L, CVocabSize));
  }
  // row 0 of a two-row sampler given the same config as its own draws the
  // same stream; a checkpoint after 8 draws replays the last 12
  TVdxSampler s(0, 2);
  TVdxSamplerConfig g = TVdxSampler::DefaultConfig();
  g.temperature = 0.7f;
  g.seed = 5;
  s.SetConfig(g);
  s.SetRowConfig(0, c);
  Check(s.GetRowConfig(0).seed == 42 && s.GetConfig().seed == 5, "row 0 holds its own config");
  std::vector<int> got;
  std::vector<uint8_t> blob;
  for (int i = 0; i < 20; ++i) {
    if (i == 8) blob = s.SaveRowState(0);
    got.push_back(s.Process(L, CVocabSize));
  }
  Check(got == want, "row 0 with Seed 42 draws the reference sampler's stream");
  s.LoadRowState(0, blob);
  std::vector<int> again;
  for (int i = 8; i < 20; ++i) again.push_back(s.Process(L, CVocabSize));
  Check(again == std::vector<int>(want.begin() + 8, want.end()), "restored row repeats its last 12 draws");
  FlushErrors(s.GetErrors());
}

int main() {
  {
    TVdxSampler probe;
    if (!probe.Ok()) {
      // no GPU: Create records a fatal error and the calls fail loudly
      Section("No GPU: Create records a fatal error, Process fails");
      Check(probe.GetErrors().HasFatal(), "Create recorded a fatal error");
      float L[CVocabSize] = {0};
      Check(probe.Process(L, CVocabSize) < 0, "Process returns a negative code");
      printf("%d passed, %d failed (no GPU)\n", g_pass, g_fail);
      return g_fail ? g_fail : 77;
    }
  }
  SecCreateDestroy();
  SecGreedyArgmax();
  SecDeterministicReseed();
  SecTopKBound();
  SecRepeatPenalty();
  SecRowConfigsAndCheckpoint();
  printf("%d passed, %d failed\n", g_pass, g_fail);
  return g_fail;
}
