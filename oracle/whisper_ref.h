/*
 * whisper_ref.h -- the oracle: a CPU restatement of whisper4j's Linux decode path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's CPU
 * baseline leg may load this library, and only as the parity reference (or as the timed CPU
 * baseline).  The product (whisper4j_amd) never links, loads or calls it.
 *
 * Every function states the reference file:line it restates (paths are relative to the
 * whisper4j source tree, "main/" = src/main/java/com/sparrowlogic/whisper4j/,
 * "java26/" = src/main/java26/com/sparrowlogic/whisper4j/).
 *
 * Numerics contract (what makes this a restatement rather than a re-design):
 *   - fp32 weights dequantized at load (main/model/GgmlLoader.java:186-201, 224-300);
 *   - Linear = transposed fp32 weight, M==1 axpy GEMV in strict k order, no FMA
 *     (main/nn/Linear.java:16-26, main/tensor/Tensor.java:383-398, java26/.../VectorSimdOps.java:114-133);
 *     M>1 = sequential-k tiled matmul (main/tensor/Tensor.java:460-489);
 *   - dot = lane-strided partial sums over ORC_LANES lanes, lanes reduced 0..L-1 in order,
 *     scalar tail (java26/.../VectorSimdOps.java:20-39).  The reference's lane count is
 *     SPECIES_PREFERRED (8 on AVX2, 16 on AVX-512) and its reduceLanes order is unspecified:
 *     that choice is documented, not pinned;
 *   - LayerNorm two-pass sequential fp32 (main/tensor/Tensor.java:592-619);
 *   - GELU = 65536-entry table indexed by the f16 bits of x (main/tensor/Tensor.java:493-538);
 *   - single-query fused attention head (java26/.../VectorSimdOps.java:137-203);
 *   - decode drivers and logit rules (main/nn/WhisperDecoder.java:161-626).
 * Compile with -ffp-contract=off (Java never fuses a*b+c).
 */
#ifndef WHISPER_REF_H
#define WHISPER_REF_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_LANES 8
#define ORC_TYPE_F32 0
#define ORC_TYPE_F16 1
#define ORC_TYPE_Q8_0 8

typedef struct {
  const char* name;
  int32_t type;     /* ORC_TYPE_* (GGML type id) */
  int32_t n_dims;
  int64_t ne[4];    /* GGML order: ne[0] is the contiguous dimension */
  const void* data; /* raw GGML bytes */
} orc_tensor;

typedef struct {
  int32_t n_vocab, n_text_ctx, n_text_state, n_text_head, n_text_layer, n_audio_ctx;
} orc_dims;

typedef struct orc_model orc_model;
typedef struct orc_cache orc_cache;

typedef struct {
  int32_t n_tokens;
  int32_t tokens[1024];
  float avg_logprob;
  float compression_ratio;
  float no_speech_prob;
  float temperature;
} orc_result;

/* ---- elementary ops (each restates one reference op) ---- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
void orc_gelu_table(float* table65536);
float orc_dot(const float* a, const float* b, int n);
void orc_layernorm(const float* x, int rows, int n, const float* g, const float* b, float eps, float* out);
void orc_linear(const float* x, int m, int k, const float* wt /*[k][n]*/, int n, const float* bias, float* y);
void orc_gelu(float* x, int n);
void orc_attention_head(const float* q, const float* k, const float* v, int kv_len, int hd, float scale,
                        float* out);
void orc_softmax_rows(float* x, int rows, int n);
int orc_argmax(const float* a, int n);
void orc_log_softmax(const float* logits, int n, float* out);
void orc_topk(const float* values, int n, int k, int32_t* idx);
float orc_compression_ratio(const int32_t* tokens, int n);
void orc_dequant_q8_0(const void* src, int64_t n, float* dst);

/* ---- model / cache ---- */
orc_model* orc_model_create(const orc_dims* dims, const orc_tensor* tensors, int n_tensors, char* err, int errlen);
void orc_model_destroy(orc_model* m);
orc_cache* orc_cache_create(const orc_model* m);
void orc_cache_destroy(orc_cache* c);
int orc_cache_len(const orc_cache* c);
/* forward(tokens, xa, cache) -> logits [n][V]   (main/nn/WhisperDecoder.java:59-104) */
int orc_forward(const orc_model* m, const int32_t* tokens, int n, const float* xa, orc_cache* cache,
                float* logits);

/* ---- audio encoder (main/nn/WhisperEncoder.java:27-76) ---- */
typedef struct {
  int32_t n_mels, n_audio_ctx, n_audio_state, n_audio_head, n_audio_layer;
} orc_enc_dims;
typedef struct orc_encoder orc_encoder;
orc_encoder* orc_encoder_create(const orc_enc_dims* dims, const orc_tensor* tensors, int n_tensors, char* err, int errlen);
void orc_encoder_destroy(orc_encoder* e);
/* forward(mel): mel [n_mels][2 * n_audio_ctx] -> out [n_audio_ctx][n_audio_state] */
int orc_encoder_forward(const orc_encoder* e, const float* mel, float* out);
/* Conv1d.forward (main/nn/Conv1d.java:38-80): w [out][in][k], in [in][len] -> out [out][out_len] */
void orc_conv1d(const float* w, const float* bias, int out_ch, int in_ch, int ksize, int stride, int pad,
                const float* in, int len, float* out);

/* Fixed logit bias [V] added to every logits row after the tied projection (NULL: none).  Not a
 * reference feature: the seeded bias of the beam-search workload. */
void orc_model_set_logit_bias(orc_model* m, const float* bias);

/* ---- logit rules (main/nn/WhisperDecoder.java:435-598), each sets -inf in place ---- */
void orc_suppress_blank(float* logits, int n, int eot);                                   /* :450-455 */
void orc_apply_suppress(float* logits, const int32_t* ids, int n_ids, int n);             /* :457-466 */
void orc_ngram_block(float* logits, const int32_t* gen, int cnt, int ngram, int n);       /* :543-564 */
void orc_timestamp_rules(float* logits, const int32_t* gen, int cnt, int ts_begin, int eot, int n,
                         int first_step);                                                  /* :484-541 */
int orc_needs_fallback(float compression_ratio, float avg_logprob, float no_speech_prob); /* :435-440 */
/* sample (:576-598) with the uniform draw u in [0,1) given; overwrites logits with exp weights */
int orc_sample_u(float* logits, int n, float temperature, double u);
/* logSoftmax (:614-626) of one entry: (l[index] - max) - log(sum exp(l - max)), exp and sum in double */
double orc_log_softmax_at(const float* l, int n, int index);
/* SplitMix64 (the seeded stand-in for Math.random): next 64-bit output, and a double in [0,1) */
uint64_t orc_splitmix64_next(uint64_t* state);
double orc_rng_uniform(uint64_t* state);

/* ---- decode drivers over a logits source (main/nn/WhisperDecoder.java) ---- */
typedef struct {
  void* ctx;
  /* the prompt: logits rows of its first position (no-speech probe) and its last position */
  int (*prefill)(void* ctx, float* first_row, float* last_row);
  /* one token appended to hypothesis `beam` (0 when greedy): its logits row */
  int (*step)(void* ctx, int beam, int32_t token, float* row);
  /* beam rearrangement: hypothesis b continues src[b] for b < saved; src[b] = -1 for b >= saved
   * (those continue new hypothesis 0) */
  int (*rearrange)(void* ctx, const int32_t* src, int saved, int beam);
} orc_ops;
int orc_greedy_drive(const orc_ops* ops, int n_vocab, int eot, int max_tokens, const int32_t* suppress, int n_suppress,
                     int no_speech, float temperature, int ts_begin, uint64_t seed, orc_result* out);
/* gaps (nullable, [max_tokens]): gaps[i] for search step i = the score of the last hypothesis kept
 * minus that of the first non-end candidate left out (+inf when none was left out); gaps[0] = the
 * final pick's margin over the runner-up.  Decisions with a gap above the parity tolerance cannot
 * flip under a logit error below it (test instrumentation, not part of the reference). */
int orc_beam_drive(const orc_ops* ops, int n_vocab, int eot, int max_tokens, const int32_t* suppress, int n_suppress,
                   int no_speech, int ts_begin, int beam, orc_result* out, double* gaps);
/* decodeWithFallback's choice over results already decoded at temperatures 0, 0.2, .., 1.0: the
 * index it returns; *n_used = how many of the decodes it would have run. */
int orc_fallback_pick(const orc_result* per_temp /*[6]*/, int* n_used);

/* ---- decode drivers on the model (main/nn/WhisperDecoder.java) ---- */
int orc_decode(const orc_model* m, const float* xa, const int32_t* prompt, int n_prompt, int eot,
               int max_tokens, const int32_t* suppress, int n_suppress, int no_speech, float temperature,
               int ts_begin, uint64_t seed, orc_result* out);
int orc_decode_beam(const orc_model* m, const float* xa, const int32_t* prompt, int n_prompt, int eot,
                    int max_tokens, const int32_t* suppress, int n_suppress, int no_speech, int ts_begin,
                    int beam, orc_result* out);
/* decode_beam that also records the decision gaps of orc_beam_drive */
int orc_decode_beam_gaps(const orc_model* m, const float* xa, const int32_t* prompt, int n_prompt, int eot,
                         int max_tokens, const int32_t* suppress, int n_suppress, int no_speech, int ts_begin, int beam,
                         orc_result* out, double* gaps);
int orc_decode_with_fallback(const orc_model* m, const float* xa, const int32_t* prompt, int n_prompt, int eot,
                             int max_tokens, const int32_t* suppress, int n_suppress, int no_speech,
                             int ts_begin, int beam, uint64_t seed, orc_result* out);

/* Teacher-forced greedy sweep used by parity tests and the CPU baseline: prefill `prompt`,
 * then run n_steps single-token forwards on forced[0..n_steps).  For every logits row that is
 * produced (prefill last row first, then one per step) record argmax, max, logsumexp (double
 * accumulate), the second-largest logit, and optionally the full row. */
int orc_forced(const orc_model* m, const float* xa, const int32_t* prompt, int n_prompt, const int32_t* forced,
               int n_steps, int32_t* argmax_out, float* max_out, float* second_out, float* lse_out,
               float* logits_out);

/* Beam search over precomputed per-step logits rows is not part of the reference; beam tests
 * drive orc_decode_beam directly. */

#ifdef __cplusplus
}
#endif
#endif
