// Decode drivers over a session: WhisperDecoder.decode / decodeBeam / decodeWithFallback
// (main/nn/WhisperDecoder.java:110-394) with the reference's logit rules (:442-626).
//
// The rules depend only on the token history, so they are evaluated on the host as a per-row
// suppression bitmask; the device applies it inside the logits pass and returns argmax,
// logsumexp and top-k, so no logits row crosses PCIe on greedy or beam steps.  Sampling (T > 0)
// runs on the device for persistent sessions after the first step (w4h_sample.hip); the host loop
// below samples only the first step and the steps of batched sessions, from the fetched row.

#include <zlib.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <random>
#include <vector>

#include "w4h_host.h"

namespace {

struct Mask {
  int V, mw;
  std::vector<uint32_t> bits;
  Mask(int V_, int rows) : V(V_), mw((V_ + 31) / 32), bits((size_t)rows * ((V_ + 31) / 32), 0u) {}
  void clear() { std::fill(bits.begin(), bits.end(), 0u); }
  void set(int r, int t) {
    if (t >= 0 && t < V) bits[(size_t)r * mw + (t >> 5)] |= 1u << (t & 31);
  }
  void range(int r, int lo, int hi) {  // [lo, hi), whole words where the range covers them
    lo = std::max(lo, 0);
    hi = std::min(hi, V);
    for (int t = lo; t < hi;) {
      if ((t & 31) == 0 && t + 32 <= hi) {
        bits[(size_t)r * mw + (t >> 5)] = 0xffffffffu;
        t += 32;
      } else {
        set(r, t);
        ++t;
      }
    }
  }
  bool get(int r, int t) const { return (bits[(size_t)r * mw + (t >> 5)] >> (t & 31)) & 1u; }
};

// suppressBlank: :450-455
void suppress_blank(Mask& m, int r, int eot) {
  m.set(r, eot);
  m.set(r, 220);
}
// applySuppress: :457-466
void apply_suppress(Mask& m, int r, const int32_t* s, int n) {
  for (int i = 0; i < n; i++) m.set(r, s[i]);
}
// applyNgramBlock: :543-564 (n = 3 and 4 via applyRepetitionPenalty :472-476)
void ngram_block(Mask& m, int r, const std::vector<int32_t>& g, int nn) {
  const int cnt = (int)g.size();
  if (cnt < nn - 1) return;
  for (int i = 0; i <= cnt - nn; i++) {
    bool match = true;
    for (int j = 0; j < nn - 1; j++)
      if (g[i + j] != g[cnt - (nn - 1) + j]) {
        match = false;
        break;
      }
    if (match) m.set(r, g[i + nn - 1]);
  }
}
void repetition_penalty(Mask& m, int r, const std::vector<int32_t>& g) {
  ngram_block(m, r, g, 3);
  ngram_block(m, r, g, 4);
}
// applyTimestampRules: :484-541
void timestamp_rules(Mask& m, int r, const std::vector<int32_t>& g, int tsb, int eot, bool first) {
  if (tsb > 0) m.set(r, tsb - 1);
  if (first) {
    m.range(r, 0, tsb);
    m.range(r, tsb + 51, m.V);
    return;
  }
  const int cnt = (int)g.size();
  if (cnt == 0) return;
  const bool lastWasTs = g[cnt - 1] >= tsb;
  const bool penultimateWasTs = cnt < 2 || g[cnt - 2] >= tsb;
  if (lastWasTs) {
    if (penultimateWasTs)
      m.range(r, tsb, m.V);
    else
      m.range(r, 0, eot);
  }
  int lastTs = -1;
  for (int i = cnt - 1; i >= 0; i--)
    if (g[i] >= tsb) {
      lastTs = g[i];
      break;
    }
  if (lastTs >= 0) m.range(r, tsb, (lastWasTs && !penultimateWasTs) ? lastTs + 1 : lastTs);
}

float compression_ratio(const int32_t* t, int n) {
  if (n == 0) return 0.0f;
  std::vector<unsigned char> b((size_t)n * 2);
  for (int i = 0; i < n; i++) {
    b[2 * i] = (unsigned char)(t[i] & 0xff);
    b[2 * i + 1] = (unsigned char)((t[i] >> 8) & 0xff);
  }
  uLongf cl = compressBound(b.size());
  std::vector<unsigned char> c(cl);
  compress2(c.data(), &cl, b.data(), b.size(), Z_DEFAULT_COMPRESSION);
  return (float)b.size() / (float)std::max<uLongf>(1, cl);
}

// Splitmix64 -> [0, 1): the reference's Math.random() is unseeded; a seeded draw makes runs repeat.
struct Rng {
  uint64_t s;
  double next() {
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
    return (double)(z >> 11) * (1.0 / 9007199254740992.0);
  }
};

// sample(): :576-598 (mutates the row into exp values, as the reference does)
int sample_row(std::vector<float>& l, float temperature, Rng& rng) {
  float max = -INFINITY;
  for (float v : l) max = std::max(max, v);
  double sum = 0;
  for (auto& v : l) {
    const double p = std::exp((double)((v - max) / temperature));
    v = (float)p;
    sum += p;
  }
  const double r = rng.next() * sum;
  double cum = 0;
  for (size_t i = 0; i < l.size(); i++) {
    cum += l[i];
    if (cum >= r) return (int)i;
  }
  return (int)l.size() - 1;
}

double log_softmax_at(const std::vector<float>& l, int index) {  // :614-626
  float max = -INFINITY;
  for (float v : l) max = std::max(max, v);
  double s = 0;
  for (float v : l) s += std::exp((double)(v - max));
  return (double)(l[index] - max) - std::log(s);
}

int check_opts(w4h_session* s, const w4h_decode_opts* o, w4h_decode_result* r) {
  if (!s || !o || !r) return w4h::fail(W4H_ERR_INVALID, "null argument");
  const w4h_dims D = w4h::session_dims(s);
  if (!o->prompt || o->n_prompt < 1) return w4h::fail(W4H_ERR_INVALID, "empty prompt");
  if (o->max_tokens < 1 || o->max_tokens > w4h::kMaxDecodeTokens)
    return w4h::fail(W4H_ERR_INVALID, "max_tokens outside [1, %d]", w4h::kMaxDecodeTokens);
  if (o->eot < 0 || o->eot >= D.n_vocab) return w4h::fail(W4H_ERR_INVALID, "eot out of range");
  return W4H_OK;
}

// Prefill the prompt (all rows fed the same tokens).  Returns the last prompt step's outputs in
// `last` (computed with `last_mask`) and the no-speech probability from the first prompt row.
int prefill(w4h_session* s, const w4h_decode_opts* o, const uint32_t* last_mask, int topk, w4h_step_out* last,
            float* logits_last, float* no_speech) {
  const int S = w4h::session_rows(s);
  int rc = w4h_session_reset(s, 0);
  if (rc) return rc;
  const w4h_dims D = w4h::session_dims(s);
  rc = w4h_session_set_probe(s, (o->no_speech >= 0 && o->no_speech < D.n_vocab) ? o->no_speech : -1);
  if (rc) return rc;
  std::vector<int32_t> tok(S);
  std::vector<w4h_step_out> first(S);
  const int n = o->n_prompt;
  if (n > 1) {
    std::vector<int32_t> forced((size_t)(n - 2) * S);
    for (int i = 1; i < n - 1; i++)
      for (int r = 0; r < S; r++) forced[(size_t)(i - 1) * S + r] = o->prompt[i];
    std::vector<w4h_step_out> outs((size_t)(n - 1) * S);
    std::fill(tok.begin(), tok.end(), o->prompt[0]);
    if ((rc = w4h_session_run(s, tok.data(), n > 2 ? forced.data() : nullptr, n - 1, 0, outs.data()))) return rc;
    first.assign(outs.begin(), outs.begin() + S);
  }
  std::fill(tok.begin(), tok.end(), o->prompt[n - 1]);
  std::vector<w4h_step_out> lo(S);
  if ((rc = w4h_session_step(s, tok.data(), last_mask, topk, lo.data(), logits_last))) return rc;
  if (n == 1) first = lo;
  *last = lo[0];
  *no_speech = (o->no_speech >= 0 && o->no_speech < D.n_vocab)
                   ? (float)std::exp((double)first[0].probe_logit - (double)first[0].raw_logsumexp)
                   : 0.0f;
  (void)w4h_session_set_probe(s, -1);
  return W4H_OK;
}

}  // namespace

extern "C" {

int w4h_compression_ratio(const int32_t* tokens, int32_t n, float* ratio) {
  if ((!tokens && n > 0) || n < 0 || !ratio) return w4h::fail(W4H_ERR_INVALID, "bad argument");
  *ratio = compression_ratio(tokens, n);
  return W4H_OK;
}

// WhisperDecoder.decode: main/nn/WhisperDecoder.java:161-204 (row 0 of the session).
int w4h_decode(w4h_session* s, const w4h_decode_opts* o, w4h_decode_result* r) {
  int rc = check_opts(s, o, r);
  if (rc) return rc;
  const w4h_dims D = w4h::session_dims(s);
  const int S = w4h::session_rows(s), V = D.n_vocab;
  const bool greedy = o->temperature == 0.0f;
  Mask mask(V, S);
  std::vector<int32_t> gen;
  double sumLogprob = 0;
  float noSpeech = 0;
  Rng rng{o->seed};
  std::vector<float> logits(greedy ? 0 : (size_t)S * V);
  std::vector<int32_t> tok(S);
  w4h_step_out out0{};
  std::vector<w4h_step_out> outs(S);
  // After the first step a one-row greedy decode runs on the device: the same rules, applied by the
  // step kernel from the generated tokens, for as many steps as the self-KV holds (the host loop
  // below takes over if the decode has not ended by then).
  const bool on_device = greedy && w4h::session_device_rules(s);
  // A sampled decode (T > 0) runs its steps after the first on the device as well: each step's
  // logits stay in device memory, where the sampling kernel applies the rules and draws the token
  // with the same generator, continued from the host's state.
  const bool sample_on_device = !greedy && w4h::session_device_sample(s);
  for (int step = 0; step < o->max_tokens; step++) {
    if (sample_on_device && step == 1) {
      int32_t kv = 0;
      if ((rc = w4h_session_kv_len(s, &kv))) return rc;
      const int n = std::min(o->max_tokens - 1, (int)(w4h::session_max_ctx(s) - kv));
      if (n > 0) {
        Mask sup(V, 1);
        apply_suppress(sup, 0, o->suppress, o->n_suppress);
        const w4h::SampleRun sr{gen.data(), (int)gen.size(), o->eot, o->timestamp_begin > 0 ? o->timestamp_begin : 0,
                                o->temperature, rng.s};
        w4h::SampleRunOut so;
        if ((rc = w4h::device_sampled_run(s, sr, n, sup.bits.data(), &so))) return rc;
        rng.s += (uint64_t)so.steps * 0x9e3779b97f4a7c15ull;  // the draws the device took
        for (int i = 0; i < so.steps; i++) {
          sumLogprob += so.lps[i];
          if (so.tokens[i] != o->eot) gen.push_back(so.tokens[i]);
        }
        step = 1 + so.steps;
        if (so.ended || step >= o->max_tokens) break;
      }
    }
    if (on_device && step == 1) {
      int32_t kv = 0;
      if ((rc = w4h_session_kv_len(s, &kv))) return rc;
      const int n = std::min(o->max_tokens - 1, (int)(w4h::session_max_ctx(s) - kv));
      if (n > 0) {
        Mask sup(V, 1);
        apply_suppress(sup, 0, o->suppress, o->n_suppress);
        std::vector<w4h_step_out> dev(n);
        int done = 0;
        const w4h::RulesRun rr{gen.data(), (int)gen.size(), o->eot, o->timestamp_begin > 0 ? o->timestamp_begin : 0};
        if ((rc = w4h::device_greedy_run(s, rr, n, sup.bits.data(), dev.data(), &done))) return rc;
        bool ended = false;
        for (int i = 0; i < done && !ended; i++) {
          sumLogprob += (double)dev[i].max_logit - (double)dev[i].logsumexp;
          if (dev[i].argmax == o->eot)
            ended = true;
          else
            gen.push_back(dev[i].argmax);
        }
        step = 1 + done;
        if (ended || step >= o->max_tokens) break;
      }
    }
    mask.clear();
    if (step == 0) suppress_blank(mask, 0, o->eot);
    apply_suppress(mask, 0, o->suppress, o->n_suppress);
    repetition_penalty(mask, 0, gen);
    if (o->timestamp_begin > 0) timestamp_rules(mask, 0, gen, o->timestamp_begin, o->eot, step == 0);
    for (int q = 1; q < S; q++) std::copy(mask.bits.begin(), mask.bits.begin() + mask.mw, mask.bits.begin() + (size_t)q * mask.mw);
    if (step == 0) {
      rc = prefill(s, o, mask.bits.data(), 1, &out0, greedy ? nullptr : logits.data(), &noSpeech);
    } else {
      std::fill(tok.begin(), tok.end(), gen.back());
      rc = w4h_session_step(s, tok.data(), mask.bits.data(), 1, outs.data(), greedy ? nullptr : logits.data());
      out0 = outs[0];
    }
    if (rc) return rc;
    int best;
    if (greedy) {
      best = out0.argmax;
      sumLogprob += (double)out0.max_logit - (double)out0.logsumexp;
    } else {
      std::vector<float> row(logits.begin(), logits.begin() + V);
      for (int t = 0; t < V; t++)
        if (mask.get(0, t)) row[t] = -INFINITY;
      best = sample_row(row, o->temperature, rng);
      sumLogprob += log_softmax_at(row, best);
    }
    if (best == o->eot) break;
    gen.push_back(best);
  }
  r->n_tokens = (int32_t)gen.size();
  std::copy(gen.begin(), gen.end(), r->tokens);
  r->avg_logprob = gen.empty() ? 0.0f : (float)(sumLogprob / gen.size());
  r->compression_ratio = compression_ratio(gen.data(), (int)gen.size());
  r->no_speech_prob = noSpeech;
  r->temperature = o->temperature;
  return W4H_OK;
}

// WhisperDecoder.decodeBeam: main/nn/WhisperDecoder.java:214-394.  Rows are beams; the device
// computes all beams in one batched step and the KV rearrangement is a row-history remap.
int w4h_decode_beam(w4h_session* s, const w4h_decode_opts* o, w4h_decode_result* r) {
  int rc = check_opts(s, o, r);
  if (rc) return rc;
  const w4h_dims D = w4h::session_dims(s);
  const int B = o->beam_size, V = D.n_vocab;
  if (B < 1 || B + 1 > W4H_TOPK_MAX) return w4h::fail(W4H_ERR_INVALID, "beam_size %d outside [1, %d]", B, W4H_TOPK_MAX - 1);
  if (w4h::session_rows(s) != B) return w4h::fail(W4H_ERR_INVALID, "session has %d rows, beam_size is %d", w4h::session_rows(s), B);
  Mask mask(V, B);
  suppress_blank(mask, 0, o->eot);
  apply_suppress(mask, 0, o->suppress, o->n_suppress);
  for (int q = 1; q < B; q++) std::copy(mask.bits.begin(), mask.bits.begin() + mask.mw, mask.bits.begin() + (size_t)q * mask.mw);
  w4h_step_out first{};
  float noSpeech = 0;
  if ((rc = prefill(s, o, mask.bits.data(), B, &first, nullptr, &noSpeech))) return rc;
  std::vector<std::vector<int32_t>> toks(B);
  std::vector<double> lps(B);
  const float lse0 = first.logsumexp;
  for (int b = 0; b < B; b++) {
    const bool ok = first.topk_logits[b] > -INFINITY;
    toks[b] = {ok ? first.topk_ids[b] : 0};
    lps[b] = ok ? (double)(first.topk_logits[b] - lse0) : -INFINITY;
  }
  std::vector<std::vector<int32_t>> fin_t;
  std::vector<double> fin_lp;
  std::vector<int32_t> tok(B), parent(B);
  std::vector<w4h_step_out> outs(B);
  struct Cand {
    double score;
    int beam, tok;
  };
  if (w4h::session_device_beam(s) && o->max_tokens > 1) {
    // batched session: the whole search runs on the device (k_w_beam after every step), the host
    // supplies the first beams and the first step's mask (the same rules as below)
    mask.clear();
    for (int b = 0; b < B; b++) {
      tok[b] = toks[b].back();
      apply_suppress(mask, b, o->suppress, o->n_suppress);
      repetition_penalty(mask, b, toks[b]);
      if (o->timestamp_begin > 0) timestamp_rules(mask, b, toks[b], o->timestamp_begin, o->eot, false);
    }
    w4h::BeamSearchIn in{};
    in.beam = B;
    in.eot = o->eot;
    in.timestamp_begin = o->timestamp_begin;
    in.max_steps = o->max_tokens - 1;
    in.suppress = o->suppress;
    in.n_suppress = o->n_suppress;
    in.first_tokens = tok.data();
    in.first_lps = lps.data();
    in.first_mask = mask.bits.data();
    w4h::BeamSearchOut res;
    if ((rc = w4h::device_beam_search(s, in, &res))) return rc;
    fin_t = res.fin;
    fin_lp = res.fin_lp;
    toks = res.toks;
    lps = res.lps;
  }
  for (int step = w4h::session_device_beam(s) ? o->max_tokens : 1; step < o->max_tokens; step++) {
    mask.clear();
    std::vector<bool> live(B);
    for (int b = 0; b < B; b++) {
      live[b] = toks[b].back() != o->eot;
      tok[b] = toks[b].back();
      apply_suppress(mask, b, o->suppress, o->n_suppress);
      repetition_penalty(mask, b, toks[b]);
      if (o->timestamp_begin > 0) timestamp_rules(mask, b, toks[b], o->timestamp_begin, o->eot, false);
    }
    if ((rc = w4h_session_step(s, tok.data(), mask.bits.data(), B + 1, outs.data(), nullptr))) return rc;
    std::vector<Cand> cands;
    for (int b = 0; b < B; b++) {
      if (!live[b]) continue;
      const float lse = outs[b].logsumexp;
      for (int k = 0; k < B + 1; k++) {
        const bool ok = outs[b].topk_logits[k] > -INFINITY;
        const float lp = ok ? outs[b].topk_logits[k] - lse : -INFINITY;
        cands.push_back({lps[b] + (double)lp, b, ok ? outs[b].topk_ids[k] : 0});
      }
    }
    if (cands.empty()) break;
    std::stable_sort(cands.begin(), cands.end(), [](const Cand& a, const Cand& c) { return a.score > c.score; });
    std::vector<std::vector<int32_t>> ntoks(B);
    std::vector<double> nlps(B);
    std::vector<int> src(B, 0);
    int saved = 0;
    for (const Cand& c : cands) {
      if (c.tok == o->eot) {
        fin_t.push_back(toks[c.beam]);
        fin_lp.push_back(c.score);
        if ((int)fin_t.size() >= B) break;
        continue;
      }
      if (saved >= B) continue;
      ntoks[saved] = toks[c.beam];
      ntoks[saved].push_back(c.tok);
      nlps[saved] = c.score;
      src[saved] = c.beam;
      saved++;
    }
    if (saved == 0 || (int)fin_t.size() >= B) break;
    for (int b = saved; b < B; b++) {  // leftover beams continue from beam 0 (:356-361)
      ntoks[b] = ntoks[0];
      nlps[b] = nlps[0];
      src[b] = src[0];
    }
    for (int b = 0; b < B; b++) parent[b] = src[b];
    if ((rc = w4h_session_reorder(s, parent.data()))) return rc;
    toks = ntoks;
    lps = nlps;
  }
  for (int b = 0; b < B && (int)fin_t.size() < B; b++) {
    fin_t.push_back(toks[b]);
    fin_lp.push_back(lps[b]);
  }
  int bestIdx = 0;
  double bestScore = -INFINITY;
  for (size_t i = 0; i < fin_t.size(); i++) {
    const double sc = fin_lp[i] / (double)std::max<size_t>(1, fin_t[i].size());
    if (sc > bestScore) {
      bestScore = sc;
      bestIdx = (int)i;
    }
  }
  const auto& bt = fin_t[bestIdx];
  r->n_tokens = (int32_t)std::min<size_t>(bt.size(), 1024);
  std::copy(bt.begin(), bt.begin() + r->n_tokens, r->tokens);
  r->avg_logprob = bt.empty() ? 0.0f : (float)(fin_lp[bestIdx] / bt.size());
  r->compression_ratio = compression_ratio(bt.data(), (int)bt.size());
  r->no_speech_prob = noSpeech;
  r->temperature = 0.0f;
  return W4H_OK;
}

// WhisperDecoder.decodeWithFallback: main/nn/WhisperDecoder.java:119-149 (needsFallback :435-440).
int w4h_decode_with_fallback(w4h_session* s, const w4h_decode_opts* o, w4h_decode_result* r) {
  int rc = check_opts(s, o, r);
  if (rc) return rc;
  const float temps[6] = {0.0f, 0.2f, 0.4f, 0.6f, 0.8f, 1.0f};
  auto needs_fallback = [](const w4h_decode_result& x) {
    if (x.compression_ratio > 2.4f) return !(x.no_speech_prob > 0.6f && x.avg_logprob < -1.0f);
    return x.avg_logprob < -1.0f && !(x.no_speech_prob > 0.6f);
  };
  w4h_decode_result cur{}, best{};
  bool have = false;
  for (int i = 0; i < 6; i++) {
    w4h_decode_opts oo = *o;
    oo.temperature = temps[i];
    oo.seed = o->seed + (uint64_t)i;
    rc = (o->beam_size > 1 && temps[i] == 0.0f) ? w4h_decode_beam(s, &oo, &cur) : w4h_decode(s, &oo, &cur);
    if (rc) return rc;
    if (!needs_fallback(cur)) {
      *r = cur;
      return W4H_OK;
    }
    if (!have || cur.avg_logprob > best.avg_logprob) {
      best = cur;
      have = true;
    }
    if (temps[i] == 0.0f && cur.compression_ratio <= 2.4f) break;
    if (temps[i] > 0.0f && cur.avg_logprob < best.avg_logprob - 1.0f) break;
  }
  *r = best;
  return W4H_OK;
}

}  // extern "C"
