/*
 * w4h.h -- C ABI of whisper4j_amd: an MI355X (gfx950) implementation of whisper4j's
 * autoregressive text-decoder token loop.
 *
 * Plain C types only (pointers, sizes, ints).  Every call returns 0 on success or a negative
 * W4H_ERR_* code; w4h_last_error() returns a thread-local message for the last failure on the
 * calling thread.  No C++ exception or longjmp crosses this boundary.
 *
 * Reference interfaces each entry point replaces (paths relative to the whisper4j source tree,
 * main/ = src/main/java/com/sparrowlogic/whisper4j/):
 *   model       GgmlLoader.load + WhisperDecoder(WeightStore, ModelDimensions)
 *               main/model/GgmlLoader.java:50-70, 95-220; main/nn/WhisperDecoder.java:36-56
 *   session     the per-decode-call kvCache HashMap (main/nn/WhisperDecoder.java:165, 223-229)
 *   step        WhisperDecoder.forward(int[] tokens, Tensor xa, Map kvCache) for one token per row,
 *               with the argmax / logsumexp / top-k the callers compute on the returned row
 *               (main/nn/WhisperDecoder.java:59-104, 174-191, 278-291, 397-431)
 *   reorder     the beam KV-cache rearrangement (main/nn/WhisperDecoder.java:342-361)
 *   decode*     WhisperDecoder.decode / decodeBeam / decodeWithFallback
 *               (main/nn/WhisperDecoder.java:110-204, 214-394)
 *   w4h_op_*    the CPU kernel plugin seam SimdOps.VectorOpsDelegate and the Tensor ops the decoder
 *               uses (main/tensor/SimdOps.java:233-250; main/tensor/Tensor.java:383-422, 493-538,
 *               592-619; src/main/java26/.../VectorSimdOps.java:20-39, 114-203)
 *
 * Threading: a model is read-only after creation and may be shared by sessions on any thread.
 * A session must be used by one thread at a time (it owns its HIP stream and device buffers).
 */
#ifndef W4H_H
#define W4H_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- return codes ---- */
#define W4H_OK 0
#define W4H_ERR_INVALID -1   /* bad argument (IllegalArgumentException in the reference)  */
#define W4H_ERR_NOT_FOUND -2 /* missing tensor (WeightStore.get, main/model/WeightStore.java:28-34) */
#define W4H_ERR_SHAPE -3     /* tensor shape mismatch (main/tensor/Tensor.java:32-36) */
#define W4H_ERR_FORMAT -4    /* not a GGML file / truncated / unsupported type (GgmlLoader) */
#define W4H_ERR_DEVICE -5    /* HIP error or no usable GPU */
#define W4H_ERR_OOM -6       /* device or host allocation failed */
#define W4H_ERR_CLOSED -7    /* handle already destroyed (IllegalStateException, WhisperModel.java:81-91) */
#define W4H_ERR_CAPACITY -8  /* KV context full */
#define W4H_ERR_TIMEOUT -9   /* a bounded device-side wait expired (the step is aborted, never hangs) */
#define W4H_ERR_IO -10       /* file could not be read */
#define W4H_ERR_CANCELLED -11 /* the session was cancelled (w4h_session_cancel) */

/* ---- GGML tensor types accepted by model creation (GgmlLoader type ids) ---- */
#define W4H_TYPE_F32 0
#define W4H_TYPE_F16 1
#define W4H_TYPE_Q8_0 8

#define W4H_TOPK_MAX 8 /* top-k returned per row by a step: beam + 1 <= W4H_TOPK_MAX */

const char* w4h_last_error(void);

/* Number of HIP devices visible (0 on a machine without a GPU; never an error). */
int w4h_device_count(int32_t* n);

/* ================================ model ================================= */

typedef struct w4h_model w4h_model;

typedef struct {
  const char* name;  /* whisper.cpp tensor name, e.g. "decoder.blocks.0.attn.query.weight" */
  int32_t type;      /* W4H_TYPE_* */
  int32_t n_dims;    /* 1..4 */
  int64_t ne[4];     /* GGML order: ne[0] is the contiguous dimension */
  const void* data;  /* raw GGML bytes; read during the call, not retained */
} w4h_tensor;

typedef struct {
  int32_t n_vocab, n_text_ctx, n_text_state, n_text_head, n_text_layer, n_audio_ctx;
} w4h_dims;

/* Upload a text decoder from a tensor table (names as whisper.cpp GGML files).  f16 and q8_0
 * matrices stay in their storage type on the device (q8_0 is repacked into 16-byte-aligned int8
 * rows plus f16 block scales); f32 matrices are converted to f16. */
int w4h_model_create(const w4h_dims* dims, const w4h_tensor* tensors, int32_t n_tensors, int32_t device,
                     w4h_model** out);
/* Parse a whisper.cpp GGML file (mmap) and upload its decoder. */
int w4h_model_load_ggml(const char* path, int32_t device, w4h_model** out);
int w4h_model_dims(const w4h_model* m, w4h_dims* out);
int w4h_model_destroy(w4h_model* m);

/* GGML file parsing without a device (the loader's format checks, testable on any host). */
int w4h_ggml_inspect(const char* path, w4h_dims* dims, int32_t* n_tensors, int64_t* data_bytes);
/* Copy the raw bytes of one named tensor of a GGML file (returns its type and ne). */
int w4h_ggml_read_tensor(const char* path, const char* name, int32_t* type, int32_t* n_dims, int64_t ne[4],
                         void* dst, int64_t dst_bytes);

/* ================================ encoder ================================ */
/* The audio encoder (WhisperEncoder, main/nn/WhisperEncoder.java:27-76): conv1 + GELU, conv2 (stride
 * 2) + GELU, + positional embedding, n_audio_layer pre-LN blocks of self-attention over the frames and
 * a GELU MLP, ln_post.  Its output is the decoder's xa (w4h_session_set_encoder[_device]). */

typedef struct w4h_encoder w4h_encoder;

typedef struct {
  int32_t n_mels, n_audio_ctx, n_audio_state, n_audio_head, n_audio_layer;
} w4h_encoder_dims;

/* Upload an encoder from a tensor table ("encoder.conv1.weight", "encoder.blocks.i.attn.query.weight",
 * ... as whisper.cpp GGML files name them): WhisperEncoder(WeightStore, ModelDimensions),
 * main/nn/WhisperEncoder.java:27-38, 86-105.  Matrices f16 / f32 (rounded to f16) or q8_0, conv
 * weights f16 / f32; the key projection has no bias.  A handle must not be used after destroy. */
int w4h_encoder_create(const w4h_encoder_dims* dims, const w4h_tensor* tensors, int32_t n_tensors, int32_t device,
                       w4h_encoder** out);
/* Parse a whisper.cpp GGML file (mmap) and upload its encoder (hparams n_audio_*, n_mels). */
int w4h_encoder_load_ggml(const char* path, int32_t device, w4h_encoder** out);
int w4h_encoder_get_dims(const w4h_encoder* e, w4h_encoder_dims* out);
/* WhisperEncoder.forward (main/nn/WhisperEncoder.java:42-76): mel [n_mels][2 * n_audio_ctx] fp32 (host
 * memory) -> out [n_audio_ctx][n_audio_state] fp32 (host memory). */
int w4h_encoder_forward(w4h_encoder* e, const float* mel, float* out);
/* The same with mel and out in device memory of the encoder's device, enqueued on `stream` (a
 * hipStream_t) and not waited for; NULL runs on the encoder's own stream and returns when done.  out
 * can go straight to w4h_session_set_encoder_device.  One forward at a time per encoder. */
int w4h_encoder_forward_device(w4h_encoder* e, const float* mel_dev, float* out_dev, void* stream);
int w4h_encoder_destroy(w4h_encoder* e);

/* =============================== session ================================ */

typedef struct w4h_session w4h_session;

typedef struct {
  int32_t n_rows;     /* S: rows decoded in lockstep (1 greedy, beam size, or independent streams), 1..32;
                         from 5 rows (3 when n_text_state >= 768) every projection is one MFMA GEMM over
                         all rows, fewer rows run on the persistent single-launch step kernel */
  int32_t n_encoders; /* 1 (rows share one encoder output: greedy, beam) or n_rows (independent streams) */
  int32_t max_ctx;    /* self-KV capacity in positions (>= n_text_ctx is typical) */
} w4h_session_desc;

/* Per-row result of a step (row = beam / stream). */
typedef struct {
  int32_t argmax;      /* first index of the maximum over the masked logits */
  float max_logit;     /* logits[argmax] */
  float logsumexp;     /* log sum exp over the masked logits */
  float probe_logit;   /* raw (unmasked) logit of the probe token, or 0 */
  float raw_logsumexp; /* logsumexp over the unmasked logits */
  int32_t topk_ids[W4H_TOPK_MAX]; /* masked logits, descending, ties -> lower index */
  float topk_logits[W4H_TOPK_MAX];
} w4h_step_out;

int w4h_session_create(w4h_model* m, const w4h_session_desc* desc, w4h_session** out);
int w4h_session_destroy(w4h_session* s);
/* Encoder output xa [n_audio_ctx][n_text_state] fp32 (host memory) for encoder `enc`: projects the
 * cross-attention K/V of every layer on the device (MultiHeadAttention.forward, cross branch,
 * main/nn/MultiHeadAttention.java:65-75). */
int w4h_session_set_encoder(w4h_session* s, int32_t enc, const float* xa);
/* The same with xa [n_audio_ctx][n_text_state] fp32 already in memory of the session's device (an
 * encoder that ran on the GPU): no host copy.  The projection is ordered only after earlier work on
 * the session's own stream, so the producer of xa must have finished writing it.  Returns when the
 * K/V are ready; xa may then be reused.  Replaces the same call site as w4h_session_set_encoder. */
int w4h_session_set_encoder_device(w4h_session* s, int32_t enc, const float* xa_device);
/* Rewind the self-KV of every row to kv_len positions (0 = empty, as a fresh decode call). */
int w4h_session_reset(w4h_session* s, int32_t kv_len);
int w4h_session_kv_len(const w4h_session* s, int32_t* kv_len);
/* Tokens set to -inf before selection on every following step (static suppress list). */
int w4h_session_set_suppress(w4h_session* s, const int32_t* ids, int32_t n);
/* A fixed bias [n_vocab] added to every row's raw logits before any mask or selection, on every
 * following step (NULL switches it off).  The reference has no counterpart: it serves the beam-search
 * workload whose selection is made deterministic by a seeded logit bias.  step_out, logits and the
 * decode drivers all see the biased logits. */
int w4h_session_set_logit_bias(w4h_session* s, const float* bias);
/* Cancel the session's work (TranscriptionHandle.cancel, main/WhisperModel.java:620-633; the reference
 * checks it between segments): on = 1 may be called from ANY thread, also while another thread is
 * inside a call on this session.  The call in flight returns W4H_ERR_CANCELLED: a one-launch greedy
 * decode stops at its next step, a sampled decode at its next launch, other launches when they end;
 * every later call returns W4H_ERR_CANCELLED too.  on = 0 (from the session's own thread, with no call
 * in flight) clears it; the self-KV is then undefined until w4h_session_reset (the decode drivers
 * reset it themselves). */
int w4h_session_cancel(w4h_session* s, int32_t on);
/* Token whose raw logit is reported in w4h_step_out.probe_logit (e.g. <|nospeech|>), -1 for none. */
int w4h_session_set_probe(w4h_session* s, int32_t token);

/* One decoder step: tokens[n_rows] at the next position of every row.  extra_mask (nullable) is a
 * per-row bitmask [n_rows][ceil(n_vocab/32)] of further tokens to suppress on this step only
 * (history-dependent rules).  out[n_rows] receives the selection results; logits (nullable)
 * receives the raw fp32 logits [n_rows][n_vocab]. */
int w4h_session_step(w4h_session* s, const int32_t* tokens, const uint32_t* extra_mask, int32_t topk,
                     w4h_step_out* out, float* logits);
/* Run n_steps steps inside one device launch.  Step 0 consumes tokens[n_rows]; every later step
 * consumes the previous step's argmax (greedy) or, when forced != NULL, forced[(i-1)*n_rows + r].
 * out (nullable) receives n_steps * n_rows results.  No host round trip between steps. */
int w4h_session_run(w4h_session* s, const int32_t* tokens, const int32_t* forced, int32_t n_steps, int32_t topk,
                    w4h_step_out* out);
/* Beam rearrangement: row r continues from row parent[r]'s history. */
int w4h_session_reorder(w4h_session* s, const int32_t* parent);

/* Time n_repeats runs of n_steps teacher-forced steps starting from the current kv_len (restored
 * after every repeat), with HIP events on the session stream around each run.  ms_out[n_repeats]
 * receives each run's duration.  Results of the last repeat go to out (nullable). */
int w4h_session_time_run(w4h_session* s, const int32_t* tokens, const int32_t* forced, int32_t n_steps,
                         int32_t n_repeats, float* ms_out, w4h_step_out* out);

/* Diagnostics: run n_steps teacher-forced steps (kv_len restored afterwards) and record, for every
 * step, phase, point and workgroup the device wall-clock (100 MHz) tick: points are 0 phase entered,
 * 1 inputs arrived, 2 work computed, 3 phase left (0 where a workgroup had no work):
 * trace[((step * (6 * n_text_layer + 2) + phase) * 4 + point) * n_workgroups + workgroup].  Phases per
 * layer: self-attention (with the q/k/v projection), self out-proj, cross-attention (with the q
 * projection), cross out-proj, mlp1, mlp2; then logits and selection. */
int w4h_session_trace_run(w4h_session* s, const int32_t* tokens, const int32_t* forced, int32_t n_steps,
                          uint64_t* trace, int64_t trace_len, int32_t* n_workgroups);

/* ============================ decode drivers ============================ */

typedef struct {
  const int32_t* prompt;
  int32_t n_prompt;
  int32_t eot;
  int32_t max_tokens;
  const int32_t* suppress;
  int32_t n_suppress;
  int32_t no_speech;      /* -1: none */
  float temperature;      /* 0: greedy / beam */
  int32_t timestamp_begin;/* <= 0: timestamps off */
  int32_t beam_size;      /* 1: greedy */
  uint64_t seed;          /* sampling draws (the reference uses an unseeded Math.random) */
} w4h_decode_opts;

typedef struct {
  int32_t n_tokens;
  int32_t tokens[1024];
  float avg_logprob;
  float compression_ratio;
  float no_speech_prob;
  float temperature;
} w4h_decode_result;

/* WhisperDecoder.decode (temperature == 0: argmax; > 0: sampling) on a session with n_rows >= 1
 * (row 0 is used). */
int w4h_decode(w4h_session* s, const w4h_decode_opts* o, w4h_decode_result* r);
/* WhisperDecoder.decodeBeam on a session with n_rows == beam_size. */
int w4h_decode_beam(w4h_session* s, const w4h_decode_opts* o, w4h_decode_result* r);
/* WhisperDecoder.decodeWithFallback: temperatures 0, 0.2 .. 1.0. */
int w4h_decode_with_fallback(w4h_session* s, const w4h_decode_opts* o, w4h_decode_result* r);
/* compressionRatio of a token list (zlib default level over 2-byte little-endian tokens). */
int w4h_compression_ratio(const int32_t* tokens, int32_t n, float* ratio);

/* ====================== kernel-level entry points ======================= */
/* Host pointers in and out; the library stages them through device memory.  Each runs the same
 * device code the decoder step uses. */

/* y[m][n] = x[m][k] . W^T + bias, W [n][k] in w_type (W4H_TYPE_F16 raw halves, or W4H_TYPE_Q8_0 raw
 * 34-byte GGML blocks along k).  bias nullable.  m <= 8. */
int w4h_op_linear(const void* w, int32_t w_type, int32_t n, int32_t k, const float* bias, const float* x, int32_t m,
                  float* y);
/* LayerNorm over rows of n (eps 1e-5). */
int w4h_op_layernorm(const float* x, int32_t rows, int32_t n, const float* gamma, const float* beta, float* y);
/* GELU through the 65536-entry f16-indexed table. */
int w4h_op_gelu(const float* x, int32_t n, float* y);
/* Single-query attention for n_heads heads: q [n_heads][64] fp32, k/v [n_heads][kv_len][64] as f16
 * bit patterns, out [n_heads][64]; scale applied to q.k. */
int w4h_op_attention(const float* q, const uint16_t* k, const uint16_t* v, int32_t n_heads, int32_t kv_len,
                     float scale, float* out);
/* Selection over rows of logits [rows][n]: mask (nullable bitmask [rows][ceil(n/32)]) -> argmax,
 * logsumexp and top-k (k <= W4H_TOPK_MAX). */
int w4h_op_select(const float* logits, int32_t rows, int32_t n, const uint32_t* mask, int32_t k, w4h_step_out* out);

/* The sampling step of a decode at temperature > 0 on one logits row [n] (n <= 65536), as the
 * device-sampled decode runs it: the suppress bitmask (nullable, [ceil(n/32)]), the n-gram repeats of
 * history[n_history] and the timestamp rules after the first step (timestamp_begin <= 0: none) set
 * tokens to -inf; then WhisperDecoder.sample with the first SplitMix64 draw after rng_state picks
 * *token, and *logprob is the log-probability the decode loop adds for it (logSoftmax over the
 * weights sample leaves in the row).  main/nn/WhisperDecoder.java:176-195, 457-466, 484-564,
 * 576-598, 614-626. */
int w4h_op_sample(const float* logits, int32_t n, const uint32_t* suppress_mask, const int32_t* history,
                  int32_t n_history, int32_t eot, int32_t timestamp_begin, float temperature, uint64_t rng_state,
                  int32_t* token, double* logprob);

/* No counterpart in the reference: w4h_op_select for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  logits [rows][n],
 * mask (nullable) [rows][ceil(n/32)] and out [rows] are DEVICE pointers on the calling thread's
 * current device; the work is enqueued on `stream` (a hipStream_t, NULL for the default stream) and
 * not waited for.  It allocates nothing: the per-row partials live in a fixed device array of the
 * library (W4H_SELECT_MAX_ROWS rows, 360 KiB, held on each device it runs on until the process
 * ends).  Every call on a device shares that array, so calls that overlap on one device race:
 * issue them on one stream or wait between them.  rows > W4H_SELECT_MAX_ROWS -> W4H_ERR_INVALID. */
#define W4H_SELECT_MAX_ROWS 64
int w4h_op_select_noalloc(const float* logits, int32_t rows, int32_t n, const uint32_t* mask, int32_t k,
                          w4h_step_out* out, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* W4H_H */
