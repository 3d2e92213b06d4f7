// Host-side helpers shared by the runtime translation units (not part of the public C ABI).
#pragma once

#include <stdint.h>

#include <vector>

#include "../../include/w4h.h"

namespace w4h {
int fail(int code, const char* fmt, ...);
float half_to_float(uint16_t h);
uint16_t float_to_half(float f);
int session_rows(const w4h_session* s);
w4h_dims session_dims(const w4h_session* s);

// Beam search run on the device by a batched-engine session (rows = beams): the first beams come
// from the host (prompt step), then up to max_steps device steps, each ending with the device beam
// step.  Returns the finished hypotheses and the last live beams.
bool session_device_beam(const w4h_session* s);
struct BeamSearchIn {
  int beam, eot, timestamp_begin, max_steps;
  const int32_t* suppress;
  int n_suppress;
  const int32_t* first_tokens;  // [beam]
  const double* first_lps;      // [beam]
  const uint32_t* first_mask;   // [beam][(n_vocab + 31) / 32] suppression mask of the first device step
};
struct BeamSearchOut {
  std::vector<std::vector<int32_t>> fin, toks;
  std::vector<double> fin_lp, lps;
};
int device_beam_search(w4h_session* s, const BeamSearchIn& in, BeamSearchOut* out);

// Greedy steps with the decode rules (n-gram repeats, timestamp rules) applied on the device from
// the generated tokens, for one-row sessions on the persistent step kernel.  The run starts with
// the last generated token, feeds back each argmax and ends after the step that selects eot.
struct RulesRun {
  const int32_t* hist;  // tokens generated so far (the last one is the run's first input)
  int nhist, eot, tsb;
};
constexpr int kMaxDecodeTokens = 1024;  // w4h_decode_opts.max_tokens at most
bool session_device_rules(const w4h_session* s);
int session_max_ctx(const w4h_session* s);
int device_greedy_run(w4h_session* s, const RulesRun& r, int n_steps, const uint32_t* mask2, w4h_step_out* out,
                      int* steps_done);

// Sampled decode steps (temperature > 0) on the device for persistent sessions: the run starts with
// the last generated token; after every step the sampling kernel applies the suppress mask `sup`
// and the history rules to row 0, draws the next token from the SplitMix64 generator in state `rng`
// (the run's step k takes its (k + 1)-th output) and feeds it to every row; the run ends after the
// end token or n_steps steps.
struct SampleRun {
  const int32_t* hist;  // tokens generated so far (the last one is the run's first input)
  int nhist, eot, tsb;
  float temperature;
  uint64_t rng;
};
struct SampleRunOut {
  int steps = 0;      // steps run (each sampled one token and appended one self-KV row)
  bool ended = false; // the last sampled token is the end token
  std::vector<int32_t> tokens;
  std::vector<double> lps;
};
bool session_device_sample(const w4h_session* s);
int device_sampled_run(w4h_session* s, const SampleRun& r, int n_steps, const uint32_t* sup, SampleRunOut* out);
}  // namespace w4h
