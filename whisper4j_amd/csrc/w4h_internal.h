// Internal interface between the host runtime (w4h_api.cpp, w4h_decode.cpp) and the device code
// (w4h_device.hip).  Not part of the public C ABI.
#pragma once

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include "../../include/w4h.h"

namespace w4h {

constexpr int kHeadDim = 64;
constexpr int kThreads = 256;  // threads per workgroup of every kernel
constexpr int kMaxRows = 8;    // decoder rows per step handled by the persistent kernel
constexpr int kSelfChunk = 256;  // self-attention keys per work item
constexpr int kMaxChunk = 256;   // longest key chunk an attention work item may take
constexpr int kResItems = 4;     // d-row items (8 rows each) one workgroup may own in a phase
constexpr int kSampEpt = 4;  // row entries per thread of the in-launch sampler (V <= grid * kThreads * kSampEpt)
constexpr int kRep = 1;          // replicas of every exchange buffer (consumers poll blockIdx % kRep)
constexpr int kPartWords = 2 + kHeadDim;            // (m, l, acc[64]) per attention partial
constexpr int kMergeChunks = 8;                     // attention partials merged from registers
constexpr int kSelWords = 6 + 2 * W4H_TOPK_MAX;     // per-workgroup selection partial

// Device pointers of one decoder layer.  Matrices are [out][in] row-major; f16 matrices hold
// halves, q8_0 matrices hold int8 with f16 scales [out][in/32] in the s_* pointer.
struct LayerDev {
  const void *w_qkv, *w_o, *w_cq, *w_co, *w_1, *w_2, *w_ck, *w_cv;
  const uint16_t *s_qkv, *s_o, *s_cq, *s_co, *s_1, *s_2, *s_ck, *s_cv;
  const float *b_qkv, *b_o, *b_cq, *b_co, *b_1, *b_2, *b_cv;
  const float *ln1_g, *ln1_b, *ln2_g, *ln2_b, *ln3_g, *ln3_b;
};

typedef unsigned long long u64;

struct StepParams {
  // model
  const LayerDev* layers;
  int L, d, H, V, C, A;
  int wq8;
  const void* emb;
  const uint16_t* emb_s;
  const float* pos;
  const float *lnf_g, *lnf_b;
  // session
  int S, X, max_ctx;
  uint16_t *kv_k, *kv_v;        // [L][S][H][max_ctx][64]
  const uint16_t *xk, *xv;      // [X][L][H][A][64]
  const int32_t* slots;         // [S][max_ctx] or null (row r reads its own slot)
  u64 *qkv, *sp, *x1, *cq, *cp, *x2, *hm, *x3, *lp, *lpa;  // tagged exchange buffers
  int ncs_max, ncc, chc;        // self partial slots (cached chunks + current key), cross chunks, cross chunk length
  // control
  int nsteps, kv_len0;
  uint32_t tag0;
  const int32_t* tokens0;       // [S]
  const int32_t* forced;        // [nsteps-1][S] or null (greedy feedback)
  const uint32_t* mask;         // [S][mw] static suppress bitmask or null
  const uint32_t* mask2;        // [S][mw] per-step extra bitmask or null
  int mw, probe, topk;
  w4h_step_out* out;            // [nsteps][S] or null
  float* logits_out;            // [nsteps][S][V] or null
  unsigned* err;                // error word; the cancel word is the 4 bytes before it (8-byte aligned)
  int rows_per_wg;              // vocab rows one workgroup keeps in LDS in the logits phase
  int ngroups;                  // phase groups: 1, 2 (halves) or 4 (quarters); see phase_group
  size_t rep_stride;            // words between replicas of the exchange buffers
  int nres;                     // vocabulary items (8 rows) a workgroup keeps resident in LDS (S = 1)
  size_t res_off;               // byte offset of the resident vocabulary rows in dynamic LDS
  unsigned long long* trace;    // [nsteps][6L+2][grid] phase-end timestamps (wall clock) or null
  // Decode rules on the device (one-row greedy runs): every workgroup keeps the generated tokens in
  // LDS, masks the n-gram repeats and timestamp rules of the greedy driver on its own vocabulary
  // rows, and the run ends after the step that selects the end token.
  int rules;                    // 1: on (needs S = 1 and greedy feedback)
  int eot, tsb;                 // end token; first timestamp token (<= 0: no timestamp rules)
  const int32_t* hist0;         // [nhist0] tokens generated before the run
  int nhist0, hist_cap;         // history length before the run; LDS history capacity (>= nhist0 + nsteps)
  size_t rules_off;             // byte offset of the rules region in dynamic LDS
  const float* bias;            // [V] fixed logit bias added before selection, or null
  const int* stop;              // device word: the launch does nothing when it is non-zero (chained
                                // sampled decodes), or null
  // Temperature sampling inside the launch (one row, decode rules on): after the logits the
  // workgroups draw the step's token together instead of taking the argmax.
  float samp_t;                 // temperature; 0: off
  uint64_t samp_rng;            // generator state; the run's step i takes draw i + 1 after it
  u64* samp_x;                  // exchange words: [grid][6] sums (three doubles as halves), then 2
  int samp_lds;                 // 1: the phase region holds the grid's sums (8 grid + 56 floats)
  float* samp_row;              // [V] the step's masked logits (device-coherent stores and loads)
  int32_t* samp_tok;            // [nsteps] drawn tokens
  double* samp_lp;              // [nsteps] their log-probabilities
};

// Device temperature sampling of one decode row (WhisperDecoder.sample and the log-probability the
// decode loop takes of the sampled token, main/nn/WhisperDecoder.java:186-187, 576-598, 614-626).
// A masking kernel applies the rules to the raw row in place and records the maximum of each
// block's part of it; the sampling kernel runs kSampleBlocks workgroups, block b owning the vocabulary range
// [b * kSampleSpan, (b + 1) * kSampleSpan) and thread t of it the kSamplePer entries from t * that,
// so per-block sums in block order and a block scan inside the chosen block give the cumulative
// weights in vocabulary order.  The last block to finish draws the token.
constexpr int kSampleBlocks = 64;
constexpr int kSamplePer = 4;
constexpr int kSampleSpan = kSamplePer * kThreads;          // 1024 entries per block
constexpr int kSampleMaxV = kSampleBlocks * kSampleSpan;   // 65536
constexpr int kSampleHist = 1024;  // generated tokens a sampled run keeps (the decode limit)
struct SampleDev {
  int n;                         // generated tokens in hist
  int steps;                     // steps sampled by this run
  int stop;                      // set after the end token or the last step of the run
  unsigned done;                 // blocks of the current sampling launch that have finished
  int32_t tok[kMaxRows];         // input token of the next step, every row
  u64 parts[kSampleBlocks];      // per-block maxima of the masked row (low 32 bits)
  double bsum[kSampleBlocks][3]; // per-block sums: double weights, float weights, exp(weight - 1)
  int32_t hist[kSampleHist];     // generated tokens (the end token is never appended)
  int32_t out_tok[kSampleHist];  // token sampled at each step of the run (the end token included)
  double lp[kSampleHist];        // its log-probability, as the decode loop accumulates it
};
struct SampleParams {
  float* logits;        // [V] masked logits of the row (bias included); overwritten with the weights
  const u64* parts;     // maxima of parts of the row: low 32 bits of parts[k * part_stride], k < nparts
  int nparts, part_stride;
  int V, eot, rows, max_steps;
  float temperature;
  uint64_t rng;         // SplitMix64 state before the run's first draw; step k of the run draws k + 1
  SampleDev* st;
  // the masking kernel (rules from st->hist)
  const uint32_t* sup;  // [ceil(V / 32)] static suppress bitmask, or null
  int tsb;              // first timestamp token (<= 0: no timestamp rules)
  u64* parts_out;       // [kSampleBlocks] per-block maxima it writes
};
hipError_t launch_sample_mask(const SampleParams& p, hipStream_t st);
hipError_t launch_sample(const SampleParams& p, hipStream_t st);

// Attention partial chunks the one-row out phases keep room for in LDS: every chunk either
// attention phase produces, and with q8_0 weights at least kMergeChunks (their attn_merge reads that
// many slots; the f16 kernels re-read the last chunk instead and keep the LDS for resident rows).
__host__ __device__ inline int merge_chunks_1(const StepParams& p) {
  const int nc = p.ncs_max > p.ncc ? p.ncs_max : p.ncc;
  return p.wq8 && nc < kMergeChunks ? kMergeChunks : nc;
}

// Ints of the rules region in LDS: history, then a bitmap over the workgroup's logits rows, then
// the timestamp ranges (count + 4 [lo, hi) pairs); rounded to 16 bytes.
inline size_t rules_lds_bytes(int hist_cap, int rows_per_wg) {
  const size_t ints = (size_t)hist_cap + (size_t)(rows_per_wg + 31) / 32 + 9;
  return (ints * 4 + 15) & ~(size_t)15;
}

// 16-byte weight chunks per lane and weight row kept in registers by the step kernel's GEMVs over
// d (32 lanes cover a row, so a row of d halves needs d / 256 rounds, of d int8 values d / 512):
// 2 rounds for d <= 512 (f16) / d <= 1024 (q8_0), 3 for wider f16 rows; anything past the prefetched
// rounds is streamed inside the GEMV.
inline int step_rounds(int d, int wq8) { return wq8 ? 2 : (d <= 512 ? 2 : 3); }

// Batched ("wide") step engine: rows that decode in lockstep (beams or independent streams, up to
// kWideMaxRows) run as a sequence of ordinary kernels per token step, with every projection an MFMA
// GEMM over all rows.  Row counts are padded to Rp = 16 or 32 (one or two 16-row MFMA tiles).
constexpr int kWideMaxRows = 32;
constexpr int kWideKeysPerPass = 128;  // keys one pass of the batched cross-attention key loop covers
constexpr int kXattnKeys = 128;        // keys per chunk of the matrix-core cross-attention (4 waves x 32)
constexpr int kWideCols = 64;        // output columns per GEMM workgroup (16 per wave)
constexpr int kWideKBlock = 128;     // k per block: four 16x16x32 MFMA steps
constexpr int kWideSelChunk = 512;   // vocabulary entries per selection partial (one wave)
constexpr int kWideMaxSlices = 16;   // k slices per GEMM at most (consumers add every slice)

// One GEMM of the wide engine: out[ks][Rp][N] = act[:, ks-th k slice] . W[N][K]^T.
struct WideGemm {
  const void* w;         // [N][K] f16, or int8 with f16 scales [N][K/32] in ws
  const uint16_t* ws;
  int N, K;
  int nw;                // column groups of 16 per workgroup (4: one per wave); with fewer, the
                         // 4 / nw waves of a column group split the workgroup's k range
  int kb;                // 128-blocks per wave; a workgroup covers (4 / nw) * kb blocks
  int ks;                // number of k slices (workgroups per column block)
};

// Per-run values of the batched engine that its kernels read from device memory, so one captured
// step can be replayed for every step of a run.
struct WideCtl {
  int i;           // step index within the run (advanced by the last selection-merge workgroup)
  int kv_len0;     // KV length before the run
  int forced_on, out_on, logits_on, mask_on, mask2_on, slots_on, bias_on, topk, probe;
  unsigned done;   // selection-merge arrivals in the current step
  int tok_dev;     // the run's first tokens come from next_tok (a continued device beam search)
  int stop;        // set by the device beam step when the search has ended: later kernels return
};

// Device beam search state (rows are beams; beam <= kBeamMax): token histories double-buffered
// by step parity, cumulative log-probabilities in double as the reference keeps them, and the
// finished list (tokens without the end token).
constexpr int kBeamMax = W4H_TOPK_MAX - 1;
constexpr int kBeamTokMax = 1024;
struct BeamDev {
  double lps[kBeamMax];
  double fin_lp[kBeamMax];
  int len[2][kBeamMax];
  int fin_len[kBeamMax];
  int nfin, cur, done;
  int toks[2][kBeamMax][kBeamTokMax];
  int fin_toks[kBeamMax][kBeamTokMax];
};

// Captured step of a session (HIP graph exec) and the buffer addresses it was captured with.
struct WideGraph {
  void* exec = nullptr;
  const void* key[8] = {};
  uintptr_t bkey[6] = {};
};

struct WideParams {
  // model
  const LayerDev* layers;  // host array
  int L, d, H, V, C, A, wq8;
  const void* emb;
  const uint16_t* emb_s;
  const float* pos;
  const float *lnf_g, *lnf_b;
  // session
  int S, X, max_ctx, Rp;
  uint16_t *kv_k, *kv_v;    // [L][S][H][max_ctx][64]
  const uint16_t *xk, *xv;  // [X][L][H][A][64]
  const uint16_t* xvt;      // [L][H][64][Ap] V transposed (one shared encoder, at most 16 rows) or null
  int Ap;
  const int32_t* slots;     // [S][max_ctx] or null
  float* x;                 // [S][d] residual stream
  float* act;               // [Rp][4d] GEMM input rows: LN outputs, attention outputs
  float* hid;               // [Rp][4d] MLP hidden rows (GELU output, MLP2 input)
  float* part;              // GEMM split-K partial sums [slices][Rp][N] (largest GEMM)
  float* cpart;             // [S][H][nch][kPartWords] cross-attention chunk partials
  float* selp;              // [S][nsel][kSelWords] selection partials
  int32_t* next_tok;        // [S] argmax of the last step (greedy feedback)
  int nch, chlen, nsel;
  WideCtl* ctl;             // device control block
  // device beam search (beam_dev != null): one k_w_beam per step after the selection
  BeamDev* beam_dev;
  const int32_t* beam_sup;  // suppressed token ids [beam_nsup]
  int beam_nsup, beam_eot, beam_tsb, tok_dev;
  WideGraph* graph;         // host cache of the captured step, or null to launch every kernel
  WideGemm g_qkv, g_o, g_cq, g_co, g_1, g_2, g_v;  // per-layer shapes and slicing; g_v = logits
  // control
  int nsteps, kv_len0;
  const int32_t* tokens0;   // [S]
  const int32_t* forced;    // [nsteps-1][S] or null
  const uint32_t* mask;
  const uint32_t* mask2;
  int mw, probe, topk;
  w4h_step_out* out;        // [nsteps][S] or null
  float* logits_out;        // [nsteps][S][V] or null
  const float* bias;        // [V] fixed logit bias (session buffer, always present)
  int bias_on;
  int no_fuse;              // split-K GEMMs even where the whole-K step applies
};

// Enqueue p.nsteps wide steps on st.
hipError_t launch_wide(const WideParams& p, hipStream_t st);
// Set the GEMM kernels' LDS limits (before any capture) and release a captured step.
hipError_t wide_prepare(int Rp, int wq8);
void wide_graph_release(WideGraph* g);
// Slicing of one wide GEMM for a device with n_cu compute units.
WideGemm wide_plan(const void* w, const uint16_t* ws, int N, int K, int n_cu);
// Whether a step of Rp padded rows at width d runs whole-K GEMMs (residual, LayerNorm and GELU
// inside them) rather than split-K GEMMs and separate kernels.
bool wide_fused_ok(int d, int Rp);

// Launchers (return the HIP error of the launch).
hipError_t launch_step(const StepParams& p, int grid, size_t lds_bytes, hipStream_t st);
size_t step_lds_bytes(const StepParams& p, int grid);
int step_max_grid(size_t lds_bytes);
// xvt (or null): V also transposed per (layer, head), [L][H][64][Ap], frames past A zero.
// scratch (or null): cross_kv_scratch_bytes(A, d) bytes of device memory for the f16 (hi, lo)
// planes of xa; with it (and d a multiple of 128) all layers run as one GEMM.
hipError_t launch_cross_kv(const LayerDev* layers_host, int L, int d, int H, int A, int wq8, const float* xa,
                           uint16_t* xk, uint16_t* xv, uint16_t* xvt, int Ap, void* scratch, hipStream_t st);
size_t cross_kv_scratch_bytes(int A, int d);
hipError_t launch_fill_u64(u64* p, size_t n, hipStream_t st);

// Standalone op launchers (device pointers).
hipError_t launch_op_linear(const void* w, const uint16_t* ws, int wq8, int n, int k, const float* bias,
                            const float* x, int m, float* y, hipStream_t st);
hipError_t launch_op_layernorm(const float* x, int rows, int n, const float* g, const float* b, float* y,
                               hipStream_t st);
hipError_t launch_op_gelu(const float* x, int n, float* y, hipStream_t st);
hipError_t launch_op_attention(const float* q, const uint16_t* k, const uint16_t* v, int nh, int kv_len, float scale,
                               float* out, hipStream_t st);
hipError_t launch_op_select(const float* logits, int rows, int n, const uint32_t* mask, int k, w4h_step_out* out,
                            hipStream_t st);
// Allocation-free selection: the partials go to the library's fixed device array (W4H_SELECT_MAX_ROWS
// rows), whose address on `device` select_scratch resolves once per device.
constexpr int kSelectMaxLds = 160 * 1024;  // LDS bytes the partial kernel may take (long rows)
hipError_t select_scratch(int device, float** ptr);
size_t select_lds_bytes(int n);
hipError_t launch_op_select_noalloc(const float* logits, int rows, int n, const uint32_t* mask, int k, w4h_step_out* out,
                                    float* scratch_ptr, hipStream_t st);

}  // namespace w4h
